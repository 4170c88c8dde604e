"""The oracle's gated-DeltaNet decode step (oracle/deltanet_oracle.c; no reference code exists
for these layers) pinned against: fixtures written by the third-party library's own torch
routines (tests/golden/make_deltanet_fixtures.py, transformers 5.15.0), the invariants of the
gated delta rule, and a float64 evaluation on random inputs."""
from pathlib import Path

import numpy as np
import pytest

import oracle as orc

FIX = Path(__file__).parent / "golden" / "deltanet_fixtures.npz"


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def test_conv1d_update_matches_library_fixture(fx):
    state = fx["conv_state0"]
    for t in range(fx["conv_x"].shape[0]):
        out, state = orc.conv1d_update(fx["conv_x"][t], fx["conv_w"], state)
        np.testing.assert_allclose(out, fx["conv_out"][t], rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(state, fx["conv_state3"])  # the state is a pure shift


def test_gated_delta_steps_match_library_fixture(fx):
    S = fx["S0"]
    for t in range(fx["q"].shape[0]):
        o, S = orc.gated_delta_step(fx["q"][t], fx["k"][t], fx["v"][t], fx["a"][t], fx["b"][t], fx["A_log"],
                                    fx["dt_bias"], S)
        np.testing.assert_allclose(o, fx["o"][t], rtol=2e-5, atol=2e-6)
    np.testing.assert_allclose(S, fx["S3"], rtol=2e-5, atol=2e-6)


def test_gated_rmsnorm_matches_library_fixture(fx):
    out = orc.gated_rmsnorm(fx["gn_x"], fx["gn_z"], fx["gn_w"], 1e-6)
    np.testing.assert_allclose(out, fx["gn_out"], rtol=1e-5, atol=1e-6)


def _f64_step(q, k, v, a, b, A_log, dt_bias, S):
    q, k, v, a, b, A_log, dt_bias, S = (np.asarray(t, np.float64) for t in (q, k, v, a, b, A_log, dt_bias, S))
    nv, nk, dk = v.shape[0], q.shape[0], q.shape[1]
    rep = nv // nk
    qn = q / np.sqrt((q * q).sum(1, keepdims=True) + 1e-6) / np.sqrt(dk)
    kn = k / np.sqrt((k * k).sum(1, keepdims=True) + 1e-6)
    qn, kn = np.repeat(qn, rep, 0), np.repeat(kn, rep, 0)
    beta = 1 / (1 + np.exp(-b))
    decay = np.exp(-np.exp(A_log) * np.logaddexp(0, a + dt_bias))
    S = S * decay[:, None, None]
    kv = np.einsum("hij,hi->hj", S, kn)
    S = S + np.einsum("hi,hj->hij", kn, (v - kv) * beta[:, None])
    return np.einsum("hij,hi->hj", S, qn), S


def test_gated_delta_step_float64():
    rng = np.random.default_rng(3)
    nv, nk, d = 8, 4, 32
    S = rng.standard_normal((nv, d, d)).astype(np.float32) * 0.3
    A_log, dt_bias = np.log(rng.uniform(0.1, 16, nv)).astype(np.float32), rng.standard_normal(nv).astype(np.float32)
    for _ in range(4):
        q, k = rng.standard_normal((nk, d)).astype(np.float32), rng.standard_normal((nk, d)).astype(np.float32)
        v = rng.standard_normal((nv, d)).astype(np.float32)
        a, b = rng.standard_normal(nv).astype(np.float32), rng.standard_normal(nv).astype(np.float32)
        o, S32 = orc.gated_delta_step(q, k, v, a, b, A_log, dt_bias, S)
        o64, S64 = _f64_step(q, k, v, a, b, A_log, dt_bias, S)
        np.testing.assert_allclose(o, o64, rtol=1e-5, atol=1e-5)
        np.testing.assert_allclose(S32, S64, rtol=1e-5, atol=1e-5)
        S = S32


def test_gated_delta_invariants():
    rng = np.random.default_rng(4)
    nv, nk, d = 2, 1, 16
    q, k = rng.standard_normal((nk, d)).astype(np.float32), rng.standard_normal((nk, d)).astype(np.float32)
    v = rng.standard_normal((nv, d)).astype(np.float32)
    S0 = rng.standard_normal((nv, d, d)).astype(np.float32)
    A_log, dt_bias, a = np.zeros(nv, np.float32), np.zeros(nv, np.float32), np.zeros(nv, np.float32)
    qn = q[0] / np.sqrt((q[0] ** 2).sum() + 1e-6) / np.sqrt(d)
    kn = k[0] / np.sqrt((k[0] ** 2).sum() + 1e-6)
    # beta = 0: the state only decays, exp(g) with g = -exp(0) * softplus(0) = -ln 2
    o, S = orc.gated_delta_step(q, k, v, a, np.full(nv, -200.0, np.float32), A_log, dt_bias, S0)
    np.testing.assert_allclose(S, S0 * 0.5, rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(o, np.einsum("hij,i->hj", S0 * 0.5, qn), rtol=1e-5, atol=1e-6)
    # decay 0 (g -> -inf) and beta = 1: the state becomes k v^T, o = (q.k) v
    o, S = orc.gated_delta_step(q, k, v, np.full(nv, 60.0, np.float32), np.full(nv, 200.0, np.float32),
                                np.full(nv, 5.0, np.float32), dt_bias, S0)
    np.testing.assert_allclose(S, np.einsum("i,hj->hij", kn, v), rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(o, float(qn @ kn) * v, rtol=1e-5, atol=1e-6)
    # zero state: o = (q.k) beta v
    b = np.array([0.3, -1.2], np.float32)
    o, _ = orc.gated_delta_step(q, k, v, a, b, A_log, dt_bias, np.zeros_like(S0))
    np.testing.assert_allclose(o, float(qn @ kn) * (1 / (1 + np.exp(-b)))[:, None] * v, rtol=1e-5, atol=1e-6)
