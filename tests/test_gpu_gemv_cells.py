"""16-row-cell GEMVs at 2048 columns (gemvTileW4, src/chpe_engine.zig:326-418, outliers added)
through the decode step's matrix-core kernels (chpe_debug_gemv_cells), against the oracle
(oracle/chpe_oracle.c: oref_gemv_tile_polymorphic per cell, oref_rmsnorm before it).  Row
counts are ragged on purpose (the 3B projections are all multiples of 16): a last cell that is
half used, a last SwiGLU unit whose gate and up cells are partly past the end, and an LM head
of 300 rows over a persistent grid.  The outliers are the cells' own (added), as in every
projection and in an untied cell LM head.

Tolerance: the kernel's products are exact integers over the input in four signed-byte limbs
per 128-column group (every element within 2^7 of its group's largest exact, the others within
2^-31 of it); the sums run in another order than the oracle's, so each output is compared within
2e-6 * sum_c |w_rc x_c| (computed from the pre-quantisation weights, with a factor 1.5 for the
quantisation)."""
import sys

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu

C = 2048
TOL = 2e-6


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_cells(rng, rows):
    n_cells = (rows + 15) // 16
    w = (rng.standard_normal((n_cells * 16, C)) * 0.02).astype(np.float32)
    w[rows:] = 0.0
    cells = np.stack([ca.pack_cell16(w[16 * t:16 * t + 16], bits=4, n_outlier_cols=8) for t in range(n_cells)])
    return cells, w[:rows]


def oracle_matvec(cells, rows, x):
    y = np.zeros(cells.shape[0] * 16, np.float32)
    for t in range(cells.shape[0]):
        y = orc.gemv_tile(cells[t], x, y.size, row_base=16 * t, accumulate=True, y=y)
    return y[:rows]


def within(got, want, tol):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= tol), f"max excess {float(np.max(err - tol)):.3e} at row {int(np.argmax(err - tol))}"


CASES = [("store", 40), ("accum", 24), ("swiglu", 56), ("logits", 300), ("store", 16)]


@pytest.mark.parametrize("mode,rows", CASES)
def test_cell_gemv_matches_oracle(mode, rows):
    rng = np.random.default_rng(rows + len(mode))
    say(f"cell gemv mode={mode} rows={rows}")
    cells, w = make_cells(rng, rows)
    x = rng.standard_normal(C).astype(np.float32)
    if mode in ("store", "accum"):
        y0 = rng.standard_normal(rows).astype(np.float32) if mode == "accum" else None
        got = ca.gpu_gemv_cells(mode, rows, cells, x, y=y0)
        want = oracle_matvec(cells, rows, x)
        mag = 1.5 * (np.abs(w).astype(np.float64) @ np.abs(x).astype(np.float64))
        if y0 is not None:
            want = want + y0
            mag = mag + np.abs(y0)
        within(got, want, TOL * mag + 1e-30)
        return
    gamma = (rng.standard_normal(C) * 0.2 + 1.0).astype(np.float32)
    xn = orc.rmsnorm(x, gamma, 1e-6)
    mag_of = lambda ww: 1.5 * (np.abs(ww).astype(np.float64) @ np.abs(xn).astype(np.float64))
    if mode == "swiglu":
        up, wu = make_cells(rng, rows)
        got = ca.gpu_gemv_cells(mode, rows, cells, x, cells_up=up, gamma=gamma, eps=1e-6)
        g = oracle_matvec(cells, rows, xn)
        u = oracle_matvec(up, rows, xn)
        sg = np.array([orc.silu(float(v)) for v in g], np.float32)
        want = sg * u
        gmag, umag = mag_of(w), mag_of(wu)
        tol = 1.1 * TOL * gmag * np.abs(u) + np.abs(sg) * TOL * umag + 1e-6 * np.abs(want) + 1e-30
        within(got, want, tol)
        return
    got, am, hn = ca.gpu_gemv_cells(mode, rows, cells, x, gamma=gamma, eps=1e-6)
    want = oracle_matvec(cells, rows, xn)
    mag = mag_of(w)
    within(got, want, TOL * mag + 1e-30)
    assert am == int(np.argmax(got))  # first index of the maximum of the GPU's own logits
    assert want[am] >= want.max() - 2 * TOL * mag.max()
    assert abs(hn - float(np.linalg.norm(x.astype(np.float64)))) <= 1e-5 * hn


def test_cell_gemv_hook_rejects_bad_arguments():
    """Argument checks run on the host before any device work: a missing gamma for a normed
    mode, a missing up tensor for SwiGLU, fewer cells than the rows need."""
    cells = np.zeros((1, 17408), np.uint8)
    x = np.zeros(C, np.float32)
    with pytest.raises(ca.EngineError):
        ca.gpu_gemv_cells("logits", 16, cells, x)
    with pytest.raises(ca.EngineError):
        ca.gpu_gemv_cells("swiglu", 16, cells, x, gamma=np.ones(C, np.float32))
    with pytest.raises(ca.EngineError):
        ca.gpu_gemv_cells("store", 17, cells, x)
