"""Polymorphic 16-row cells of every width (gemvTilePolymorphic, src/chpe_engine.zig:732-751)
through the engine's polymorphic kernel (chpe_debug_gemv_poly), against the oracle
(oracle/chpe_oracle.c: oref_gemv_tile_polymorphic per cell at the prefix-sum row bases of
gemvLinear's walk, :1430-1442).

Cells: 2-bit codebook and 4-bit, each with group-128 scales (+ added outliers for 16-row cells)
and with the tile's scale and bias; int8 with the tile's scale and bias (:421-472); fp16, bf16
(:475-541); f32 (:544-581); an unknown width, which the reference reads as 2-bit (:746-749);
cells narrower than x; cells of 8, 4, 2 rows.  Tensors mix the kinds, stop at a cell with
rows == 0, clip the last cell at r_total and leave rows past the last cell zero.

One-hot inputs (x = e_j) give bit-identical outputs (each row sum has one non-zero term on both
sides).  Dense inputs are compared within 1e-5 * sum_c |w_rc x_c| (+ the int8 tile's |bias|):
the kernel sums lane-strided partials in a butterfly, the oracle sums sequentially or in the
reference's 8-wide vectors."""
import sys

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu

CELL, CODES, PL = 17408, 64, 16448
C = 2048
TOL = 1e-5
W2 = np.array([0.0, 1.0, -2.0, -1.0], np.float64)


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def header(cell, bits, rows, cols, flags, scale=0.0, bias=0.0):
    pl = cell[PL:]
    pl[20] = bits
    pl[24:32] = np.frombuffer(np.uint64(flags).tobytes(), np.uint8)
    pl[32:40] = np.frombuffer(np.array([scale, bias], np.float32).tobytes(), np.uint8)
    pl[40:48] = np.frombuffer(np.array([rows, cols], np.uint32).tobytes(), np.uint8)


def make_cell(rng, kind, rows, cols):
    """(cell bytes, |W| as float64 [rows][cols] for the tolerance, per-row additive magnitude
    terms as a function of |x|)."""
    cell = np.zeros(CELL, np.uint8)
    g128 = kind.endswith("g")
    base = kind.rstrip("g")
    bits = {"w2": 2, "w3": 3, "w4": 4, "w8": 8, "f16": 16, "bf16": 16, "f32": 32}[base]
    scale = float(rng.uniform(0.002, 0.02))
    bias = float(rng.uniform(-0.01, 0.01))
    header(cell, bits, rows, cols, (1 if g128 else 0) | (4 if base == "f16" else 0), scale, bias)
    extra = lambda ax: np.zeros(rows)
    if base in ("w2", "w3", "w4"):
        per = 2 if base == "w4" else 4
        codes = rng.integers(0, 256, rows * cols // per, dtype=np.uint8)
        cell[CODES:CODES + codes.size] = codes
        b = codes.reshape(rows, cols // per)
        if per == 2:
            q = np.stack([b & 15, b >> 4], -1).reshape(rows, cols).astype(np.float64) - 8.0
        else:
            q = W2[np.stack([(b >> s) & 3 for s in (0, 2, 4, 6)], -1).reshape(rows, cols)]
        if g128:
            g = cols // 128
            sc = rng.uniform(0.001, 0.01, rows * g).astype(np.float16)
            cell[PL + 48:PL + 48 + sc.nbytes] = sc.view(np.uint8)
            if rows == 16:  # added outliers: 8 distinct columns, one past x
                ocol = rng.choice(cols, 8, replace=False).astype(np.uint16)
                ocol[5] = 4000
                ow = (rng.standard_normal(128) * 0.05).astype(np.float16)
                cell[PL + 816:PL + 832] = ocol.view(np.uint8)
                cell[PL + 560:PL + 816] = ow.view(np.uint8)
                owa = np.abs(ow.astype(np.float64)).reshape(16, 8)

                def extra(ax, owa=owa, ocol=ocol):
                    xo = np.array([ax[c] if c < ax.size else 0.0 for c in ocol])
                    return owa @ xo
            sc = cell[PL + 48:PL + 48 + 2 * rows * g].view(np.float16)  # as written (within the cell)
            w = np.abs(q) * np.repeat(np.abs(sc.astype(np.float64)).reshape(rows, g), 128, axis=1)
        else:
            w = np.abs(q * scale + bias)
    elif base == "w8":
        codes = rng.integers(-128, 128, rows * cols).astype(np.int8)
        cell[CODES:CODES + codes.size] = codes.view(np.uint8)
        w = np.abs(codes.astype(np.float64).reshape(rows, cols)) * scale
        extra = lambda ax: np.full(rows, abs(bias))
    else:
        w32 = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
        if base == "f16":
            raw = w32.astype(np.float16).view(np.uint8).reshape(-1)
        elif base == "bf16":
            raw = (w32.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1)
        else:
            raw = w32.view(np.uint8).reshape(-1)
        cell[CODES:CODES + raw.size] = raw
        w = np.abs(w32.astype(np.float64)) * 1.01
    return cell, w, extra


# (kind, rows, cols) per cell
MIX = [("w4g", 16, 2048), ("w2g", 16, 2048), ("w4", 16, 2048), ("w2", 16, 2048), ("w8", 8, 2048),
       ("f16", 4, 2048), ("bf16", 4, 2048), ("f32", 2, 2048), ("w3", 16, 2048), ("w4g", 8, 2048),
       ("w4g", 16, 1024), ("w8", 16, 1000), ("f16", 8, 1000)]


def build(rng, spec, stop_after=None):
    cells, mats, extras, bases = [], [], [], []
    rb = 0
    for kind, rows, cols in spec:
        c, w, e = make_cell(rng, kind, rows, cols)
        cells.append(c)
        mats.append(w)
        extras.append(e)
        bases.append(rb)
        rb += rows
    if stop_after is not None:  # a cell with rows == 0 ends the walk
        cells.insert(stop_after, np.zeros(CELL, np.uint8))
        cells.append(make_cell(rng, "w4g", 16, 2048)[0])
    return np.stack(cells), mats, extras, bases


def oracle_gemv(cells, r_total, x):
    """gemvLinear's walk (:1430-1442) over the oracle's per-cell kernel."""
    y = np.zeros(r_total, np.float32)
    rb = 0
    for t in range(cells.shape[0]):
        if rb >= r_total:
            break
        rows = int(cells[t, PL + 40:PL + 44].view(np.uint32)[0])
        if rows == 0:
            break
        y = orc.gemv_tile(cells[t], x, r_total, row_base=rb, accumulate=False, y=y)
        rb += rows
    return y


def magnitude(mats, extras, bases, r_total, ax):
    m = np.zeros(r_total)
    for w, e, rb in zip(mats, extras, bases):
        if rb >= r_total:
            break
        rows, cols = w.shape
        n = min(cols, ax.size)
        part = w[:, :n] @ ax[:n] + e(ax)
        k = min(rows, r_total - rb)
        m[rb:rb + k] = part[:k]
    return m


def within(got, want, tol):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= tol), f"max excess {float(np.max(err - tol)):.3e} at row {int(np.argmax(err - tol))}"


def covered(spec):
    return sum(r for _, r, _ in spec)


@pytest.mark.parametrize("r_extra", [-5, 0, 7])  # last cell clipped / exact / rows past the cells
def test_poly_one_hot_bit_exact(r_extra):
    rng = np.random.default_rng(100 + r_extra)
    cells, _, _, _ = build(rng, MIX)
    r_total = covered(MIX) + r_extra
    for j in (0, 5, 127, 128, 999, 1000, 1023, 1024, 2047) + tuple(int(c) for c in cells[0, PL + 816:PL + 832].view(np.uint16)[:3]):
        say(f"poly one-hot r_total={r_total} j={j}")
        x = np.zeros(C, np.float32)
        x[j] = 1.0
        want = oracle_gemv(cells, r_total, x)
        got = ca.gpu_gemv_poly("store", r_total, C, cells, x)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), j
        y0 = rng.standard_normal(r_total).astype(np.float32)
        got = ca.gpu_gemv_poly("accum", r_total, C, cells, x, y=y0)
        assert np.array_equal(got.view(np.uint32), (y0 + want).view(np.uint32)), j


@pytest.mark.parametrize("mode", ["store", "accum", "swiglu", "logits"])
def test_poly_dense_matches_oracle(mode):
    rng = np.random.default_rng(7 + len(mode))
    spec = MIX * 2
    cells, mats, extras, bases = build(rng, spec)
    r_total = covered(spec) - 3
    x = rng.standard_normal(C).astype(np.float32)
    say(f"poly dense mode={mode} r_total={r_total}")
    if mode in ("store", "accum"):
        y0 = rng.standard_normal(r_total).astype(np.float32) if mode == "accum" else None
        got = ca.gpu_gemv_poly(mode, r_total, C, cells, x, y=y0)
        want = oracle_gemv(cells, r_total, x)
        mag = magnitude(mats, extras, bases, r_total, np.abs(x).astype(np.float64))
        if y0 is not None:
            want = want + y0
            mag = mag + np.abs(y0)
        within(got, want, TOL * mag + 1e-30)
        return
    gamma = (rng.standard_normal(C) * 0.2 + 1.0).astype(np.float32)
    xn = orc.rmsnorm(x, gamma, 1e-6)
    axn = np.abs(xn).astype(np.float64)
    if mode == "swiglu":
        up, umats, uextras, ubases = build(rng, spec)
        got = ca.gpu_gemv_poly(mode, r_total, C, cells, x, cells_up=up, gamma=gamma, eps=1e-6)
        g = oracle_gemv(cells, r_total, xn)
        u = oracle_gemv(up, r_total, xn)
        sg = np.array([orc.silu(float(v)) for v in g], np.float32)
        want = sg * u
        gmag = magnitude(mats, extras, bases, r_total, axn)
        umag = magnitude(umats, uextras, ubases, r_total, axn)
        tol = 1.1 * TOL * gmag * np.abs(u) + np.abs(sg) * TOL * umag + 1e-6 * np.abs(want) + 1e-30
        within(got, want, tol)
        return
    got, am, hn = ca.gpu_gemv_poly(mode, r_total, C, cells, x, gamma=gamma, eps=1e-6)
    want = oracle_gemv(cells, r_total, xn)
    mag = magnitude(mats, extras, bases, r_total, axn)
    within(got, want, TOL * mag + 1e-30)
    assert am == int(np.argmax(got))
    assert abs(hn - float(np.linalg.norm(x.astype(np.float64)))) <= 1e-5 * hn


def test_poly_walk_stops_at_zero_rows():
    """A cell with rows == 0 ends gemvLinear's walk (:1437): the rows after it stay zero even
    though later cells exist."""
    rng = np.random.default_rng(3)
    spec = MIX[:6]
    cells, _, _, _ = build(rng, spec, stop_after=4)
    r_total = covered(spec) + 16
    x = rng.standard_normal(C).astype(np.float32)
    want = oracle_gemv(cells, r_total, x)
    got = ca.gpu_gemv_poly("store", r_total, C, cells, x)
    n4 = covered(spec[:4])
    assert not want[n4:].any() and not got[n4:].any()
    assert np.allclose(got[:n4], want[:n4], rtol=1e-4, atol=1e-4)


def test_poly_hook_rejects_reads_past_the_cells():
    """A cell whose dims would make the kernel read past the given cells (and the padding after
    them) is refused on the host before any device work."""
    cell = np.zeros((1, CELL), np.uint8)
    header(cell[0], 32, 100000, 2048, 0)
    with pytest.raises(ca.EngineError):
        ca.gpu_gemv_poly("store", 100000, C, cell, np.zeros(C, np.float32))
