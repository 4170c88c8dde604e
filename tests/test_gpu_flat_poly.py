"""Flat-tile tensors the uniform kernels do not take, through the engine's tile-by-tile path
(FlatPoly: k_flat_poly + k_flat_poly_rows + the mode's epilogue), against the oracle's
gemvCellFlat (src/chpe_engine.zig:584-729) as gemvLinear walks the available tiles (:1423-1429):

  * tiles without GROUP128: every weight value * dims.scale + dims.bias (:619-630, :666-677),
    4- and 2-bit, outliers replacing;
  * a mix of forms in one tensor, including a width the flat path does not decode (zero weights,
    :694-696);
  * short tensors: fewer tiles than the shape needs, the last one ending inside a row (that row
    gets the dot of the weights it has, the rows past it none), 4- and 2-bit;
  * rows whose width is not a multiple of 128;
  * and a whole 3B 4-bit archive whose down-projection tiles are rewritten into the scale + bias
    form: decode steps against the oracle.

Tolerance as for the uniform flat kernels: 2e-6 * sum_c |w_rc x_c| per output (another order of
the float sums); a row with no weights is exactly 0 (Store) or its old value (Accum)."""
import os
import sys
import tempfile

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu

TILE = 32768
P = 64 + 16384  # the payload's offset in a cell
TOL = 2e-6


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def tiles_of(rng, n_tiles, form):
    """n_tiles flat cells; form per tile: 'g4', 'g2' (the writer's group-128 tiles), 'n4', 'n2'
    (no GROUP128: random dims.scale / dims.bias), 'w3' (an unsupported width)."""
    forms = form if isinstance(form, list) else [form] * n_tiles
    out = []
    for t, f in enumerate(forms):
        w = (rng.standard_normal(TILE) * 0.02).astype(np.float32)
        cell = ca.pack_flat(w, bits=2 if f in ("g2", "n2") else 4, n_outliers=int(rng.integers(0, 65)))
        if f in ("n4", "n2"):
            cell[P + 24:P + 32] = 0  # custom_flags: no GROUP128
            sb = np.array([rng.uniform(0.002, 0.006), rng.uniform(-0.002, 0.002)], np.float32)
            cell[P + 32:P + 40] = np.frombuffer(sb.tobytes(), np.uint8)
        elif f == "w3":
            cell[P + 20] = 3
        out.append(cell)
    return np.stack(out)


def oracle_matvec(cells, rows, cols, x, y0=None):
    y = np.zeros(rows, np.float32) if y0 is None else y0.copy()
    for t in range(cells.shape[0]):
        orc.gemv_cell_flat(cells[t], t, rows, cols, x, y)
    w = np.concatenate([orc.flat_tile_weights(c) for c in cells])
    n = min(w.size, rows * cols)
    wabs = np.zeros(rows * cols, np.float64)
    wabs[:n] = np.abs(w[:n])
    return y, wabs.reshape(rows, cols) @ np.abs(x).astype(np.float64)


def within(got, want, tol):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= tol), f"max excess {float(np.max(err - tol)):.3e} at row {int(np.argmax(err - tol))}"


CASES = [  # (mode, rows, cols, n_tiles or None = the shape's, form)
    ("store", 40, 8192, None, "n4"),
    ("accum", 36, 12288, None, "n2"),
    ("swiglu", 24, 8192, None, "n4"),
    ("logits", 300, 4096, None, "n4"),
    ("store", 64, 8192, None, ["g4", "n4", "g2", "w3", "n2", "g4", "g4", "g4", "g4", "g4", "g4", "g4", "g4", "g4",
                              "g4", "g4"]),
    ("store", 50, 12288, 7, "g4"),     # short: 7 tiles = 18.67 rows of 12288
    ("accum", 50, 12288, 7, "g2"),     # short 2-bit
    ("logits", 33, 3000, None, "g4"),  # a width that is not a multiple of 128
    ("accum", 20, 29568, 5, "n4"),
]


@pytest.mark.parametrize("mode,rows,cols,n_tiles,form", CASES)
def test_flat_poly_gemv_matches_oracle(mode, rows, cols, n_tiles, form):
    rng = np.random.default_rng(rows * 31 + cols + (n_tiles or 0))
    need = (rows * cols + TILE - 1) // TILE
    nt = n_tiles or need
    say(f"flat-poly gemv mode={mode} rows={rows} cols={cols} tiles={nt}/{need} form={form if isinstance(form, str) else 'mixed'}")
    cells = tiles_of(rng, nt, form)
    x = rng.standard_normal(cols).astype(np.float32)
    if mode in ("store", "accum"):
        y0 = rng.standard_normal(rows).astype(np.float32) if mode == "accum" else None
        got = ca.gpu_gemv_flat(mode, rows, cols, cells, x, y=y0)
        want, mag = oracle_matvec(cells, rows, cols, x, y0)
        if y0 is not None:
            mag = mag + np.abs(y0)
        within(got, want, TOL * mag + 1e-30)
        covered = nt * TILE // cols  # rows with every weight present
        if nt < need:  # rows past the tiles: no weights
            tail = want[covered + 1:]
            assert np.array_equal(got[covered + 1:], tail)
        return
    gamma = (rng.standard_normal(cols) * 0.2 + 1.0).astype(np.float32)
    xn = orc.rmsnorm(x, gamma, 1e-6)
    if mode == "swiglu":
        up = tiles_of(rng, nt, form)
        got = ca.gpu_gemv_flat(mode, rows, cols, cells, x, tiles_up=up, gamma=gamma, eps=1e-6)
        g, gmag = oracle_matvec(cells, rows, cols, xn)
        u, umag = oracle_matvec(up, rows, cols, xn)
        sg = np.array([orc.silu(float(v)) for v in g], np.float32)
        want = sg * u
        tol = 1.1 * TOL * gmag * np.abs(u) + np.abs(sg) * TOL * umag + 1e-6 * np.abs(want) + 1e-30
        within(got, want, tol)
        return
    got, am, hn = ca.gpu_gemv_flat(mode, rows, cols, cells, x, gamma=gamma, eps=1e-6)
    want, mag = oracle_matvec(cells, rows, cols, xn)
    within(got, want, TOL * mag + 1e-30)
    assert am == int(np.argmax(got))
    assert abs(hn - float(np.linalg.norm(x.astype(np.float64)))) <= 1e-5 * hn


def test_scale_bias_down_tiles_in_a_3b_archive(w4_archive):
    """Every down-projection tile of the 3B 4-bit archive rewritten into the no-GROUP128 form
    (dims.scale 0.004, dims.bias -0.0005: weights (q - 8) * 0.004 - 0.0005, outliers kept): the
    engine plans those tensors tile by tile; decode steps and a greedy stream against the oracle."""
    data = np.fromfile(w4_archive, dtype=np.uint8)
    sb = np.frombuffer(np.array([0.004, -0.0005], np.float32).tobytes(), np.uint8)
    for l in range(36):
        li = orc.layer_info(1, l)
        for t in range(li["down_tiles"]):
            base = 4096 + (li["down_proj"] + t) * 17408 + P
            data[base + 24] &= 0xFE
            data[base + 32:base + 40] = sb
    fd, path = tempfile.mkstemp(suffix=".chpe", prefix="qwen2.5-3b-nogroup-", dir=os.path.dirname(str(w4_archive)))
    os.close(fd)
    data.tofile(path)
    try:
        e = ca.Engine(path, arch=0, max_seq_len=64, kv_f16=False)
        o = orc.Oracle(data=data, arch=0, max_seq_len=64, threads=16)
        try:
            for pos, tok in enumerate([151643, 9707, 11, 1879]):
                say(f"no-group down tiles: step pos={pos}")
                am, lg = e.decode_step(tok, pos)
                r = o.forward(tok, pos)
                ol = o.logits()
                d = np.abs(lg.astype(np.float64) - ol)
                cos = float(lg.astype(np.float64) @ ol / np.linalg.norm(lg) / np.linalg.norm(ol))
                assert d.max() <= 2e-3 * max(1.0, float(np.abs(ol).max())) and cos >= 0.9999, (pos, float(d.max()), cos)
                assert am == r.argmax_token
            prompt = np.random.default_rng(5).integers(0, 151936, 12).astype(np.uint32)
            g = e.generate(prompt, 8)
            ref, gaps = o.generate(prompt, 8)
            for i, (a, b) in enumerate(zip(g, ref)):
                if a != b:
                    assert gaps[i] < 1e-3, (i, int(a), int(b), float(gaps[i]))
                    break
        finally:
            e.close()
            o.close()
    finally:
        os.unlink(path)
