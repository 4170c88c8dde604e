"""The Qwen3.5-9B hybrid decode on the GPU (chpe_init_ex arch 3: 24 gated-DeltaNet layers and 8
gated full-attention layers with q / k norms and partial rotary embedding; no reference code,
the model as transformers' Qwen3_5DecoderLayer defines it) against the oracle's hybrid step
(oracle/chpe_oracle.c forward_hybrid, itself pinned against that library by
tests/test_oracle_hybrid.py) on the seeded 9B 4-bit archive.

Bars as for the other whole-model tests: single-step logits within 2e-4 * max|logit| and cosine
>= 0.9999 with the f32 KV cache, 1.5e-3 with the fp16 cache; greedy streams identical, a
difference allowed only after an oracle step whose top-2 gap is below 1e-3.  Then the state
machinery: the recurrent states restart at position 0 (a prompt run twice gives the same
logits bit for bit); the block step (speculative verify of 4 and 8 drafts, the chunked
prefill: every weight read once, the DeltaNet states rolled over the tokens in order) against
the decode steps and against the oracle; the hybrid decode is not the reference's decode of the
same archive (arch 1); the command line's --hybrid writes chpe_forward_tokens' logits of arch
3, bit for bit."""
import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc
from test_gpu_cli import receipt, run_cli
from test_gpu_models import archive, check_stream, compare_logits, say, threads

pytestmark = pytest.mark.gpu

VOCAB = 248320


@pytest.fixture(scope="module")
def a9h():
    p = archive(ca.PACK_9B_W4)
    yield p
    p.unlink(missing_ok=True)


def prompt_of(seed, n):
    return np.random.default_rng(seed).integers(0, VOCAB, n).astype(np.uint32)


@pytest.mark.timeout(900)
def test_hybrid_steps_and_stream_match_oracle(a9h):
    prompt = prompt_of(7, 8)
    e = ca.Engine(a9h, arch=3, max_seq_len=64, kv_f16=False)
    o = orc.Oracle(a9h, arch=1, max_seq_len=64, kv_f16=False, threads=threads())
    o.set_hybrid(True)
    try:
        steps = []
        for pos in range(4):
            say(f"hybrid f32 KV step pos={pos} token={int(prompt[pos])}")
            am, lg = e.decode_step(int(prompt[pos]), pos)
            r = o.forward(int(prompt[pos]), pos)
            ol = o.logits()
            compare_logits(lg, ol, f"pos {pos}", 2e-4)
            assert am == r.argmax_token and r.all_finite
            assert e.last()["hidden_norm"] == pytest.approx(r.hidden_norm, rel=1e-4)
            steps.append((lg.astype(np.float64), ol.astype(np.float64)))
        # the steps depend on their token and on the recurrent state: the change of the logits
        # from one step to the next is at least 20 times the two steps' measured deviations
        for (g0, o0), (g1, o1) in zip(steps, steps[1:]):
            err = float(np.abs(g0 - o0).max() + np.abs(g1 - o1).max())
            dd, dref = float(np.abs((g1 - g0) - (o1 - o0)).max()), float(np.abs(o1 - o0).max())
            say(f"  logit change: max {dref:.4g}, gpu vs oracle {dd:.2e}, step deviations {err:.2e}")
            assert dd <= err + 1e-12 and dref >= 20 * err
        say("hybrid stream (f32 KV): 8 prompt + 6 generated")
        g = e.generate(prompt, 6)
        ref, gaps = o.generate(prompt, 6)
        say(f"  gpu {list(map(int, g))} oracle {list(map(int, ref))} top-2 gaps {[round(float(x), 4) for x in gaps]}")
        assert check_stream(g, ref, gaps, "hybrid") == 6
        assert np.all(np.isfinite(gaps))
    finally:
        e.close()
        o.close()
    e = ca.Engine(a9h, arch=3, max_seq_len=64, kv_f16=True)
    o = orc.Oracle(a9h, arch=1, max_seq_len=64, kv_f16=True, threads=threads())
    o.set_hybrid(True)
    try:
        for pos in range(3):
            say(f"hybrid fp16 KV step pos={pos}")
            am, lg = e.decode_step(int(prompt[pos]), pos)
            r = o.forward(int(prompt[pos]), pos)
            compare_logits(lg, o.logits(), f"kv-f16 pos {pos}", 1.5e-3)
            assert am == r.argmax_token
    finally:
        e.close()
        o.close()


def top2_gap(lg):
    t = np.sort(lg.astype(np.float64))
    return float(t[-1] - t[-2])


@pytest.mark.timeout(600)
def test_hybrid_restart_and_block_step(a9h):
    """Position 0 restarts the recurrent states; the block step (every weight read once for the
    m tokens, the DeltaNet states rolled over them in order inside one launch per kernel)
    against the decode steps on the same engine, with the block-step bars of the other models
    (2e-4 * max|logit| with the f32 cache, 3e-3 with the fp16 cache; an argmax may differ only
    where the decode step's top-2 gap is below twice the bar)."""
    prompt, drafts = prompt_of(11, 6), prompt_of(12, 8)
    n = len(prompt)
    for kv16, rel in ((True, 3e-3), (False, 2e-4)):
        e = ca.Engine(a9h, arch=3, max_seq_len=64, kv_f16=kv16)
        try:
            assert e.block_ready()
            say(f"hybrid kv_f16={kv16}: the prompt twice from position 0")
            _, l1 = e.forward_tokens(prompt, want_logits=True)
            seq = [e.decode_step(int(d), n + i) for i, d in enumerate(drafts)]
            _, l2 = e.forward_tokens(prompt, want_logits=True)
            assert np.array_equal(l1.view(np.uint32), l2.view(np.uint32))
            for m in (4, 8):
                say(f"hybrid: verify {m} drafts vs {m} decode steps")
                e.forward_tokens(prompt)
                got = e.verify(drafts[:m], n)
                for i in range(m):
                    if int(got[i]) != int(seq[i][0]):
                        assert top2_gap(seq[i][1]) < 2 * rel * float(np.abs(seq[i][1]).max()), (m, i)
                compare_logits(e.logits(), seq[m - 1][1], f"verify {m}: last draft", rel)
                if m == 4:  # the decode state continues after the block: the next draft's step
                    am, lg = e.decode_step(int(drafts[4]), n + 4)
                    compare_logits(lg, seq[4][1], "decode step after verify 4", rel)
            say("hybrid: prefill (a block step of 6) vs forward_tokens")
            _, lp = e.prefill(prompt, want_logits=True)
            compare_logits(lp, l1, "prefill vs forward_tokens", rel)
            am, lg = e.decode_step(int(drafts[0]), n)
            compare_logits(lg, seq[0][1], "decode step after prefill", rel)
            say("hybrid: prefill of 40 positions (blocks of 32 + 8) vs forward_tokens")
            long = prompt_of(13, 40)
            _, ls = e.forward_tokens(long, want_logits=True)
            _, lb = e.prefill(long, want_logits=True)
            compare_logits(lb, ls, "prefill 40 vs forward_tokens", rel)
            if kv16:
                # a step at position 1 continues from the state position 0 left
                a = e.decode_step(int(prompt[0]), 0)[1]
                b = e.decode_step(int(prompt[1]), 1)[1]
                e.decode_step(int(prompt[2]), 0)
                c = e.decode_step(int(prompt[1]), 1)[1]
                assert not np.array_equal(b, c) and not np.array_equal(a, b)
        finally:
            e.close()
    # the reference's decode of the 9B map (arch 1) is another computation
    e = ca.Engine(a9h, arch=1, max_seq_len=64, kv_f16=True)
    try:
        _, lc = e.forward_tokens(prompt, want_logits=True)
        assert not np.allclose(lc, l1, rtol=1e-2, atol=1e-2)
    finally:
        e.close()


@pytest.mark.timeout(900)
def test_hybrid_block_step_matches_oracle(a9h):
    """The speculative verify of the hybrid (4 and 8 drafts over an 11-token context, the
    block step) and the block prefill against the oracle's sequential hybrid steps (f32 cache):
    every argmax (up to a near-tie) and the last draft's logits within 2e-4 * max|logit|."""
    prompt, drafts = prompt_of(21, 11), prompt_of(22, 8)
    n = len(prompt)
    e = ca.Engine(a9h, arch=3, max_seq_len=64, kv_f16=False)
    o = orc.Oracle(a9h, arch=1, max_seq_len=64, kv_f16=False, threads=threads())
    o.set_hybrid(True)
    try:
        say("hybrid: prefill of 11 positions (one block) vs the oracle")
        _, lp = e.prefill(prompt, want_logits=True)
        for pos, t in enumerate(prompt):
            o.forward(int(t), pos)
        compare_logits(lp, o.logits(), "prefill vs oracle", 2e-4)
        for m in (4, 8):
            say(f"hybrid: verify {m} drafts vs the oracle")
            e.prefill(prompt)
            got = e.verify(drafts[:m], n)
            lv = e.logits()
            for pos, t in enumerate(prompt):  # the oracle's context again (its states restart at 0)
                o.forward(int(t), pos)
            for i in range(m):
                r = o.forward(int(drafts[i]), n + i)
                if int(got[i]) != r.argmax_token:
                    ol = o.logits()
                    assert top2_gap(ol) < 4e-4 * float(np.abs(ol).max()), (m, i, int(got[i]), r.argmax_token)
            compare_logits(lv, o.logits(), f"verify {m}: last draft vs oracle", 2e-4)
    finally:
        e.close()
        o.close()


def test_hybrid_needs_the_9b_archive(w4_archive):
    with pytest.raises(ca.EngineError):  # (a 3B archive under the 9B map)
        ca.Engine(w4_archive, arch=3, max_seq_len=16)


def test_cli_hybrid_flag(a9h, tmp_path):
    toks = prompt_of(13, 5)
    tf = tmp_path / "prompt.bin"
    tf.write_bytes(toks.astype("<u4").tobytes())
    lf = tmp_path / "logits.bin"
    rc, err = run_cli([a9h, "--hybrid", "--tokens-file", tf, "--out-logits", lf, "--max-seq-len", 16], tmp_path)
    assert rc == 0, err
    assert "Model Arch     : Qwen3.5-9B (hybrid) (32 layers, D=4096, vocab=248320)" in err
    r = receipt(err)
    logits = np.fromfile(lf, dtype="<f4")
    e = ca.Engine(a9h, arch=3, max_seq_len=16)
    try:
        am, lg = e.forward_tokens(toks, want_logits=True)
    finally:
        e.close()
    assert np.array_equal(logits.view(np.uint32), lg.view(np.uint32)) and r["argmax"] == am
