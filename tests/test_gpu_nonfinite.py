"""Non-finite values through the engine, against the oracle.

1. GEMV inputs with a NaN or an infinite element, through the matrix-core kernels (flat tiles:
   k_gemv_xm, 4- and 2-bit; 16-row cells: k_gemv_mma), in the norm modes (the LM head, SwiGLU),
   where one NaN makes the whole normalised input NaN, and in the residual mode.  The reference
   propagates every non-finite input into every output it touches (w * NaN = NaN, including
   w = 0), so the LM head's logits are all NaN: all_finite false, argmax 0, max logit -1e30.
   The limb kernels turn a group holding a NaN or an infinity into NaN for the whole group;
   where the reference gives +-inf (an infinite input times a non-zero weight), they give NaN:
   both are non-finite, and the tests compare finiteness element by element.

2. forwardDecode's non-finite break (src/chpe_engine.zig:1753-1764): after layer l the reference
   leaves the layer loop when the hidden state's sum of squares is not finite (tested after
   layers 0-2 and 8-16, and after any layer whose hidden[0] is not finite); the final norm and
   the LM head then see the hidden state of the break, and the later layers write no KV rows.
   * Infinite weight: one outlier weight of layer 1's down projection set to +inf (flat-tile
     outliers replace the dequantised weight, :632-646) makes one hidden row infinite at every
     step.  With the break, the hidden state keeps that infinity and hidden_norm is +inf;
     without it the next layer's norm turns it into NaN everywhere.  (An infinite group scale
     would not do: the reference multiplies every code value by it, and a zero code gives
     0 * inf = NaN, where the GPU scales the group's integer sum and gets +-inf.)
   * Overflow without a non-finite element: one token's bf16 embedding row set to 1e20 (a
     bf16 archive) gives a finite hidden state whose sum of squares overflows, so the step
     breaks after layer 0; its logits are 0 and layers 1-35 keep zero KV rows at its position,
     which the next steps read.  Without the break those rows hold the q/k/v biases.
   The oracle with the break removed (Oracle.set_break(False), a planted deviation on the CPU)
   shows that each comparison tells the two apart.
"""
import os
import sys
import tempfile

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu

TILE = 32768


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def flat_tiles(rng, rows, cols, bits):
    n = rows * cols
    w = (rng.standard_normal(n) * 0.02).astype(np.float32)
    n_tiles = (n + TILE - 1) // TILE
    w = np.concatenate([w, np.zeros(n_tiles * TILE - n, np.float32)])
    return np.stack([ca.pack_flat(w[t * TILE:(t + 1) * TILE], bits=bits, n_outliers=64) for t in range(n_tiles)])


def oracle_flat(cells, rows, cols, x, y0=None):
    y = np.zeros(rows, np.float32) if y0 is None else y0.copy()
    for t in range(cells.shape[0]):
        orc.gemv_cell_flat(cells[t], t, rows, cols, x, y)
    return y


FLAT_CASES = [  # (mode, bits, rows, cols, column, value); all on the matrix-core kernel
    ("logits", 4, 300, 8192, 5, np.nan),
    ("logits", 4, 300, 8192, 4000, np.inf),
    ("logits", 2, 70, 4096, 130, np.nan),
    ("swiglu", 4, 8192, 8192, 77, np.nan),
    ("swiglu", 2, 28, 4096, 0, -np.inf),
    ("accum", 4, 16388, 8192, 100, np.nan),
    ("accum", 4, 16388, 8192, 8191, np.inf),
    ("accum", 2, 40, 8192, 3000, -np.inf),
]


@pytest.mark.parametrize("mode,bits,rows,cols,col,val", FLAT_CASES)
def test_flat_gemv_nonfinite_input(mode, bits, rows, cols, col, val):
    rng = np.random.default_rng(rows + cols + col)
    say(f"flat gemv non-finite input mode={mode} bits={bits} rows={rows} cols={cols} x[{col}]={val}")
    cells = flat_tiles(rng, rows, cols, bits)
    x = rng.standard_normal(cols).astype(np.float32)
    x[col] = val
    if mode == "accum":
        y0 = rng.standard_normal(rows).astype(np.float32)
        got = ca.gpu_gemv_flat(mode, rows, cols, cells, x, y=y0)
        want = oracle_flat(cells, rows, cols, x, y0)
        assert not np.isfinite(want).any()
        assert np.array_equal(np.isfinite(got), np.isfinite(want))
        return
    gamma = (rng.standard_normal(cols) * 0.2 + 1.0).astype(np.float32)
    xn = orc.rmsnorm(x, gamma, 1e-6)
    if mode == "swiglu":
        up = flat_tiles(rng, rows, cols, bits)
        got = ca.gpu_gemv_flat(mode, rows, cols, cells, x, tiles_up=up, gamma=gamma, eps=1e-6)
        g, u = oracle_flat(cells, rows, cols, xn), oracle_flat(up, rows, cols, xn)
        want = np.array([orc.silu(float(v)) for v in g], np.float32) * u
        assert np.isnan(want).all() and np.isnan(got).all()
        return
    got, am, hn = ca.gpu_gemv_flat(mode, rows, cols, cells, x, gamma=gamma, eps=1e-6)
    want = oracle_flat(cells, rows, cols, xn)
    # every logit NaN: all_finite false, the argmax stays at index 0 (NaN never wins)
    assert np.isnan(want).all() and np.isnan(got).all()
    assert am == 0
    assert not np.isfinite(hn)


@pytest.mark.parametrize("mode,col,val", [("logits", 9, np.nan), ("swiglu", 2047, np.inf), ("accum", 640, np.nan)])
def test_cell_gemv_nonfinite_input(mode, col, val):
    rng = np.random.default_rng(col)
    rows = 300 if mode == "logits" else 48
    say(f"cell gemv non-finite input mode={mode} x[{col}]={val}")
    n_cells = (rows + 15) // 16
    w = (rng.standard_normal((n_cells * 16, 2048)) * 0.02).astype(np.float32)
    cells = np.stack([ca.pack_cell16(w[16 * t:16 * t + 16], bits=4, n_outlier_cols=8) for t in range(n_cells)])
    x = rng.standard_normal(2048).astype(np.float32)
    x[col] = val
    if mode == "accum":
        got = ca.gpu_gemv_cells(mode, rows, cells, x, y=np.zeros(rows, np.float32))
        assert not np.isfinite(got).any()
        return
    gamma = np.ones(2048, np.float32)
    if mode == "swiglu":
        up = np.stack([ca.pack_cell16(w[16 * t:16 * t + 16], bits=4, n_outlier_cols=8) for t in range(n_cells)])
        got = ca.gpu_gemv_cells(mode, rows, cells, x, cells_up=up, gamma=gamma, eps=1e-6)
        assert np.isnan(got).all()
        return
    got, am, hn = ca.gpu_gemv_cells(mode, rows, cells, x, gamma=gamma, eps=1e-6)
    assert np.isnan(got).all() and am == 0 and not np.isfinite(hn)


# ---------------------------------------------------------------- the layer loop's break
def _modified_copy(src, edits):
    """A temporary copy of archive `src` with edits = [(offset, bytes)] applied."""
    data = np.fromfile(src, dtype=np.uint8)
    for off, b in edits:
        data[off:off + len(b)] = np.frombuffer(b, np.uint8)
    fd, path = tempfile.mkstemp(suffix=".chpe", prefix="qwen2.5-3b-mod-", dir=os.path.dirname(str(src)))
    os.close(fd)
    data.tofile(path)
    return path, data


def inf_outlier_edit(path, rec0, n_tiles):
    """(file offset, bytes) that set one outlier weight of the first flat tile from record rec0
    on that has outliers to +inf: an entry whose offset no later entry overrides."""
    P = 64 + 16384
    with open(path, "rb") as f:
        for t in range(n_tiles):
            base = 4096 + (rec0 + t) * 17408
            f.seek(base + P + 560)
            pay = f.read(272)
            n = int(np.frombuffer(pay[:2], np.uint16)[0])
            if not 0 < n <= 64:
                continue
            offs = np.frombuffer(pay[130:130 + 2 * n], np.uint16)
            for m in range(n - 1, -1, -1):
                if offs[m] not in offs[m + 1:]:
                    return base + P + 562 + 2 * m, np.uint16(0x7c00).tobytes()
    raise AssertionError("no flat tile with outliers")


def _step_result(e, tok, pos):
    am, lg = e.decode_step(tok, pos)
    return am, lg, e.last()


def _same_result(am, lg, last, r, ol, tag, apart=()):
    # apart: logits compared on their own scale (a token whose embedding row is huge)
    say(f"{tag}: gpu argmax {am} max {last['max_logit']:.6g} hidden_norm {last['hidden_norm']:.6g} "
        f"finite {bool(np.isfinite(lg).all())} | oracle argmax {r.argmax_token} max {r.max_logit:.6g} "
        f"hidden_norm {r.hidden_norm:.6g} finite {bool(r.all_finite)}")
    assert am == r.argmax_token
    assert bool(np.isfinite(lg).all()) == bool(r.all_finite)
    hn, ohn = last["hidden_norm"], r.hidden_norm
    assert (np.isnan(hn) and np.isnan(ohn)) or (np.isinf(hn) and np.isinf(ohn)) or abs(hn - ohn) <= 1e-4 * abs(ohn)
    if np.isfinite(r.max_logit):
        assert abs(last["max_logit"] - r.max_logit) <= 2e-3 * max(1.0, abs(r.max_logit))
    fin = np.isfinite(ol)
    assert np.array_equal(np.isfinite(lg), fin)
    rest = fin.copy()
    for t in apart:
        rest[t] = False
        if fin[t]:
            assert abs(lg[t] - ol[t]) <= 2e-3 * max(1.0, abs(ol[t]))
    if rest.any():
        scale = max(1.0, float(np.abs(ol[rest]).max()))
        assert float(np.abs(lg[rest] - ol[rest]).max()) <= 2e-3 * scale


def test_break_on_infinite_weight(w4_archive):
    # layer 1's down projection: one outlier weight = +inf, so a hidden row is infinite after
    # layer 1 at every step (map 1: the 3B cell map)
    li = orc.layer_info(1, 1)
    path, data = _modified_copy(w4_archive, [inf_outlier_edit(w4_archive, li["down_proj"], li["down_tiles"])])
    try:
        e = ca.Engine(path, arch=0, max_seq_len=16, kv_f16=False)
        o = orc.Oracle(data=data, arch=0, max_seq_len=16, threads=16)
        nb = orc.Oracle(data=data, arch=0, max_seq_len=16, threads=16)
        nb.set_break(False)
        try:
            for pos, tok in enumerate([151643, 17, 9001]):
                am, lg, last = _step_result(e, tok, pos)
                r = o.forward(tok, pos)
                _same_result(am, lg, last, r, o.logits(), f"inf weight pos {pos}")
                assert np.isinf(last["hidden_norm"])
                # the planted deviation: without the break the hidden state turns NaN
                assert np.isnan(nb.forward(tok, pos).hidden_norm)
        finally:
            e.close()
            o.close()
            nb.close()
    finally:
        os.unlink(path)


def test_break_on_overflowing_hidden_state(bf16_archive):
    # token 1000's embedding row (3B raw map: tile 250, row 0) = 1e20 in every column: the step
    # with it breaks after layer 0 with a finite hidden state; the steps after it read the zero
    # KV rows of layers 1-35 at its position
    T = 1000
    off = 4096 + (T // 4) * 16384 + (T % 4) * 4096
    big = np.uint16(np.float32(1e20).view(np.uint32) >> 16)
    path, data = _modified_copy(bf16_archive, [(off, np.full(2048, big, np.uint16).tobytes())])
    try:
        e = ca.Engine(path, arch=0, max_seq_len=16, kv_f16=False)
        o = orc.Oracle(data=data, arch=0, max_seq_len=16, threads=16)
        nb = orc.Oracle(data=data, arch=0, max_seq_len=16, threads=16)
        nb.set_break(False)
        try:
            for pos, tok in enumerate([5, T, 7, 9]):
                am, lg, last = _step_result(e, tok, pos)
                r = o.forward(tok, pos)
                ol = o.logits()
                _same_result(am, lg, last, r, ol, f"overflow pos {pos}", apart=(T,))
                if pos == 1:
                    assert np.isinf(last["hidden_norm"]) and not lg.any()
                nb.forward(tok, pos)
                if pos >= 2:  # the planted deviation: the later steps see other KV rows
                    rest = np.ones(ol.size, bool)
                    rest[T] = False
                    scale = max(1.0, float(np.abs(ol[rest]).max()))
                    d_nb = float(np.abs(nb.logits()[rest] - lg[rest]).max())
                    say(f"  without the break the other logits differ by {d_nb:.3g} (bar {2e-3 * scale:.3g})")
                    assert d_nb > 5 * 2e-3 * scale
        finally:
            e.close()
            o.close()
            nb.close()
    finally:
        os.unlink(path)
