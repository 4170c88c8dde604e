"""The oracle's Qwen3.5-9B hybrid step (oracle/chpe_oracle.c forward_hybrid; no reference code)
against the library that defines the model: tests/golden/hybrid_fixtures.npz holds the hidden
state after the first four layers (three gated-DeltaNet layers and one gated full-attention
layer with q/k norms and partial rotary embedding) at positions 0, 1, 2, computed by
transformers 5.15.0's Qwen3_5DecoderLayer over the seeded 9B archive's weights
(tests/golden/make_hybrid_fixtures.py).  The library runs the prompt as one sequence (chunked
delta rule, causal mask) and the oracle as three decode steps; both in f32, in different orders
of summation: within 2e-5 of the largest hidden value (measured: 5e-6).

A mistake in the composition -- the full rotary dimension instead of 64, the gate taken from
the wrong half of a q_proj head, the norm gains used as 1 + g, q and k swapped in the DeltaNet
split, another layer pattern -- moves the hidden state by orders of magnitude more."""
import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

FX = ca.PKG_DIR.parent / "tests" / "golden" / "hybrid_fixtures.npz"


@pytest.fixture(scope="module")
def archive9b():
    return ca.ensure_archive(ca.PACK_9B_W4, 0)


def test_hybrid_layers_match_library(archive9b):
    fx = np.load(FX)
    assert str(fx["archive"]) == archive9b.name, "the fixture was written from another generator: rerun " \
                                                 "tests/golden/make_hybrid_fixtures.py"
    o = orc.Oracle(archive9b, arch=1, max_seq_len=8)
    try:
        o.set_hybrid(True)
        for pos, t in enumerate(fx["tokens"]):
            o.forward_layers(int(t), pos, int(fx["n_layers"]))
            ref = fx["hidden"][pos].astype(np.float64)
            err = float(np.abs(o.hidden() - ref).max())
            assert err <= 2e-5 * float(np.abs(ref).max()), (pos, err)
    finally:
        o.close()


def test_hybrid_state_restarts_at_position_zero(archive9b):
    # the recurrent states start from zero at position 0: a prompt run twice gives the same
    # logits, and a step at position 1 depends on the state position 0 left
    o = orc.Oracle(archive9b, arch=1, max_seq_len=8)
    try:
        o.set_hybrid(True)
        runs = []
        for _ in range(2):
            for pos, t in enumerate([17, 23, 5]):
                r = o.forward_layers(t, pos, 4)
            runs.append(o.hidden())
        assert np.array_equal(runs[0], runs[1])
        o.forward_layers(99, 0, 4)
        o.forward_layers(5, 1, 4)
        h_a = o.hidden()
        o.forward_layers(17, 0, 4)
        o.forward_layers(5, 1, 4)
        assert not np.array_equal(h_a, o.hidden())
        # the compat decode (the reference's GQA aliasing) of the same archive differs
        o.set_hybrid(False)
        o.forward_layers(17, 0, 4)
        o.forward_layers(5, 1, 4)
        assert not np.allclose(h_a, o.hidden())
    finally:
        o.close()
