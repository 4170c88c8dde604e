"""Flat-tile GEMV launches (gemvCellFlat, src/chpe_engine.zig:584-729, driven by gemvLinear
:1396-1489 for tensors wider than 2048 columns) at the widths of the larger models, through
chpe_debug_gemv_flat, against the oracle (oracle/chpe_oracle.c: oref_gemv_cell_flat over every
tile, oref_rmsnorm before it).  The widths pick the kernel variants: 4096 / 8192 / 12288 columns
split the panels over 2 / 4 / 6 waves; launches of 4096 units or more at those widths, every
LM head and every wider input (the 72B down projection at 29568 columns) run the persistent
input-stationary kernels: 4-bit tiles on the matrix cores (k_gemv_xm: exact integer products
of the codes with the input split into four signed-byte limbs per 128-column group, which is
exact for every element within 2^7 of its group's largest and within 2^-31 of that largest
otherwise).  2-bit tiles take that kernel at every size (code ^ 2 as the operand, the 2-bit
field order in the limb tables).  The SwiGLU and LM head launches of
that kernel at 4096 and 8192 columns read their codes from the permuted copy the engine builds
for them (k_xm_layout: the same bytes in the kernel's load order).  Row counts are ragged (not
multiples of the unit).

Tolerance: the GPU sums in another order than the oracle's sequential loop (and as
sum (q x) - 8 sum x per group, which cancels), so each output is compared within
2e-6 * sum_c |w_rc x_c|; the oracle itself stays within 5e-8 of that sum against float64 on
these inputs.  The outlier replacements are exact in both."""
import sys

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu

TILE = 32768
TOL = 2e-6


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_tiles(rng, rows, cols, bits):
    """rows x cols weights (a few large ones, so that every tile has outliers) as flat cells."""
    n = rows * cols
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    hot = rng.choice(n, size=max(1, n // 2000), replace=False)
    w[hot] = (rng.standard_normal(hot.size) * 0.5).astype(np.float32)
    n_tiles = (n + TILE - 1) // TILE
    w = np.concatenate([w, np.zeros(n_tiles * TILE - n, np.float32)])
    cells = np.stack([ca.pack_flat(w[t * TILE:(t + 1) * TILE], bits=bits, n_outliers=64) for t in range(n_tiles)])
    return cells


def oracle_matvec(cells, rows, cols, x):
    y = np.zeros(rows, np.float32)
    for t in range(cells.shape[0]):
        orc.gemv_cell_flat(cells[t], t, rows, cols, x, y)
    wabs = np.abs(np.concatenate([orc.flat_tile_weights(c) for c in cells])[:rows * cols].reshape(rows, cols))
    return y, wabs.astype(np.float64) @ np.abs(x).astype(np.float64)


def within(got, want, tol):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= tol), f"max excess {float(np.max(err - tol)):.3e} at row {int(np.argmax(err - tol))}"


CASES = [  # (mode, bits, rows, cols)
    ("accum", 4, 60, 8192),
    ("store", 4, 36, 12288),
    ("swiglu", 4, 44, 8192),
    ("logits", 4, 300, 8192),
    ("logits", 4, 90, 4096),
    ("accum", 4, 20, 29568),
    ("swiglu", 4, 12, 29568),
    ("swiglu", 4, 8192, 8192),   # 4096 units: the persistent input-stationary kernel
    ("accum", 4, 16388, 8192),   # (4097 units, the last one partly past the rows)
    ("accum", 2, 40, 8192),
    ("swiglu", 2, 28, 4096),
    ("logits", 2, 70, 4096),
]


@pytest.mark.parametrize("mode,bits,rows,cols", CASES)
def test_flat_gemv_matches_oracle(mode, bits, rows, cols):
    rng = np.random.default_rng(rows * 7 + cols + bits)
    say(f"flat gemv mode={mode} bits={bits} rows={rows} cols={cols}")
    cells = make_tiles(rng, rows, cols, bits)
    x = rng.standard_normal(cols).astype(np.float32)
    if mode in ("store", "accum"):
        y0 = rng.standard_normal(rows).astype(np.float32) if mode == "accum" else None
        got = ca.gpu_gemv_flat(mode, rows, cols, cells, x, y=y0)
        want, mag = oracle_matvec(cells, rows, cols, x)
        if y0 is not None:
            want = want + y0
            mag = mag + np.abs(y0)
        within(got, want, TOL * mag + 1e-30)
        return
    gamma = (rng.standard_normal(cols) * 0.2 + 1.0).astype(np.float32)
    xn = orc.rmsnorm(x, gamma, 1e-6)
    if mode == "swiglu":
        up = make_tiles(rng, rows, cols, bits)
        got = ca.gpu_gemv_flat(mode, rows, cols, cells, x, tiles_up=up, gamma=gamma, eps=1e-6)
        g, gmag = oracle_matvec(cells, rows, cols, xn)
        u, umag = oracle_matvec(up, rows, cols, xn)
        sg = np.array([orc.silu(float(v)) for v in g], np.float32)
        want = sg * u
        # |d silu| <= 1.1 |dg|, plus the rounding of the product
        tol = 1.1 * TOL * gmag * np.abs(u) + np.abs(sg) * TOL * umag + 1e-6 * np.abs(want) + 1e-30
        within(got, want, tol)
        return
    got, am, hn = ca.gpu_gemv_flat(mode, rows, cols, cells, x, gamma=gamma, eps=1e-6)
    want, mag = oracle_matvec(cells, rows, cols, xn)
    within(got, want, TOL * mag + 1e-30)
    assert am == int(np.argmax(got))  # first index of the maximum of the GPU's own logits
    assert want[am] >= want.max() - 2 * TOL * mag.max()
    assert abs(hn - float(np.linalg.norm(x.astype(np.float64)))) <= 1e-5 * hn

