"""Gated-DeltaNet decode-step kernels (chpe-qwen-engine_amd/csrc/deltanet.hip) against the
oracle (oracle/deltanet_oracle.c, itself pinned by tests/test_oracle_deltanet.py) at the
Qwen3.5-9B linear-attention shapes: 32 value heads, 16 key heads, head dim 128, conv over
2*2048 + 4096 = 8192 channels with 4 taps; the state is carried over several steps."""
import sys

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def test_conv1d_update_matches_oracle():
    rng = np.random.default_rng(11)
    ch, taps = 8192, 4
    w = (rng.standard_normal((ch, taps)) * 0.5).astype(np.float32)
    st_g = st_o = rng.standard_normal((ch, taps - 1)).astype(np.float32)
    for t in range(4):
        say(f"deltanet conv step {t}")
        x = rng.standard_normal(ch).astype(np.float32)
        og, st_g = ca.gpu_deltanet_conv(x, w, st_g)
        oo, st_o = orc.conv1d_update(x, w, st_o)
        np.testing.assert_array_equal(st_g, st_o)  # the state is a pure shift
        # same products and order; SiLU's expf may differ in the last bit between libraries
        np.testing.assert_allclose(og, oo, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("hd,nv,nk", [(128, 32, 16), (64, 8, 8)])
@pytest.mark.parametrize("gated", [False, True])
def test_gated_delta_steps_match_oracle(hd, nv, nk, gated):
    """Tolerance 2e-5 relative to the largest output: the GPU's column sums run over row blocks
    (ungated: a workgroup per head and 16-column block, 16 row blocks; gated at head dim 128:
    k_dn_step_head, a workgroup per head, 8 row blocks, the norm in the same workgroup) against
    one sequential sum (oracle)."""
    rng = np.random.default_rng(hd + nv + int(gated))
    A_log = np.log(rng.uniform(0.1, 16, nv)).astype(np.float32)
    dt_bias = rng.standard_normal(nv).astype(np.float32)
    norm_w = (rng.standard_normal(hd) * 0.3 + 1.0).astype(np.float32) if gated else None
    S_g = S_o = (rng.standard_normal((nv, hd, hd)) * 0.2).astype(np.float32)
    for t in range(4):
        say(f"deltanet step hd={hd} nv={nv} nk={nk} gated={gated} t={t}")
        q, k = (rng.standard_normal((nk, hd)).astype(np.float32) for _ in range(2))
        v = rng.standard_normal((nv, hd)).astype(np.float32)
        a, b = (rng.standard_normal(nv).astype(np.float32) for _ in range(2))
        z = rng.standard_normal((nv, hd)).astype(np.float32) if gated else None
        og, S_g = ca.gpu_deltanet_step(q, k, v, a, b, A_log, dt_bias, S_g, z=z, norm_w=norm_w, eps=1e-6)
        oo, S_o = orc.gated_delta_step(q, k, v, a, b, A_log, dt_bias, S_o)
        if gated:
            oo = orc.gated_rmsnorm(oo, z, norm_w, 1e-6)
        scale = float(np.max(np.abs(oo)))
        assert float(np.max(np.abs(og - oo))) <= 2e-5 * scale, t
        assert float(np.max(np.abs(S_g - S_o))) <= 2e-5 * float(np.max(np.abs(S_o))), t
