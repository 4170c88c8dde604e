"""Raw-tile GEMVs (gemvLinear's raw path, src/chpe_engine.zig:1455-1488, dotSegment :1194-1251)
through the engine's raw kernels (chpe_debug_gemv_raw), against the oracle's raw gemvLinear on an
archive of the same tiles (oracle/chpe_oracle.c, opened from bytes): IEEE fp16 and bf16 tiles of
8192 weights, and int8 tiles of 16384 weights whose every segment dot is scaled by the fixed
0.00373708 (:1219-1237; the 9B int8 archive).  Rows of 11008 and 12288 columns straddle the
tiles.

One-hot inputs (x = e_j) give bit-identical outputs.  Dense inputs are compared within
TOL * sum_c |w_rc x_c|: 2e-6 for fp16 / bf16 (the sums run in another order), 8e-6 for int8,
whose kernel adds the codes as unsigned bytes (w + 128) and subtracts 128 * sum(x) per 16-column
chunk, which carries about twice the magnitude through the f32 sums."""
import sys

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu

TOL = {"fp16": 2e-6, "bf16": 2e-6, "int8": 8e-6}
WPT = {"fp16": 8192, "bf16": 8192, "int8": 16384}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make_tiles(rng, kind, rows, cols):
    """(tiles [n][16384] bytes, decoded weights [rows][cols] as float64)"""
    n = rows * cols
    n_tiles = (n + WPT[kind] - 1) // WPT[kind]
    if kind == "int8":
        w = rng.integers(-128, 128, n_tiles * WPT[kind]).astype(np.int8)
        dec = w[:n].astype(np.float64).reshape(rows, cols) * float(np.float32(0.00373708))
        raw = w.view(np.uint8)
    else:
        w32 = (rng.standard_normal(n_tiles * WPT[kind]) * 0.05).astype(np.float32)
        if kind == "fp16":
            h = w32.astype(np.float16)
            raw = h.view(np.uint8)
            dec = h[:n].astype(np.float64).reshape(rows, cols)
        else:
            b = (w32.view(np.uint32) >> 16).astype(np.uint16)
            raw = b.view(np.uint8)
            dec = (b[:n].astype(np.uint32) << 16).view(np.float32).astype(np.float64).reshape(rows, cols)
    return raw.reshape(n_tiles, 16384), dec


def oracle_archive(kind, tiles):
    n = tiles.shape[0]
    hdr = np.zeros(4096, np.uint8)
    hdr[:4] = np.frombuffer(np.uint32(0x45504843).tobytes(), np.uint8)
    hdr[4:8] = np.frombuffer(np.uint32(1).tobytes(), np.uint8)
    flags = {"fp16": 0x04, "bf16": 0x00, "int8": 0x08}[kind]
    hdr[8:64] = np.frombuffer(np.array([4096, n, n, 16384, 16384, 0, flags], np.uint64).tobytes(), np.uint8)
    arch = 1 if kind == "int8" else 0  # the int8 reading is the 9B archive's (:886)
    return orc.Oracle(data=np.concatenate([hdr, tiles.reshape(-1)]), arch=arch, max_seq_len=4, threads=8)


def within(got, want, tol):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert np.all(err <= tol), f"max excess {float(np.max(err - tol)):.3e} at row {int(np.argmax(err - tol))}"


@pytest.mark.parametrize("kind", ["fp16", "bf16", "int8"])
def test_raw_one_hot_bit_exact(kind):
    rng = np.random.default_rng(5 + len(kind))
    rows, cols = 21, 11008
    tiles, _ = make_tiles(rng, kind, rows, cols)
    o = oracle_archive(kind, tiles)
    try:
        for j in (0, 1, 15, 16, 5000, 8191, 8192, 11007):
            say(f"raw one-hot kind={kind} j={j}")
            x = np.zeros(cols, np.float32)
            x[j] = 1.0
            want = o.gemv_linear(0, tiles.shape[0], x, rows, cols)
            got = ca.gpu_gemv_raw("store", rows, cols, kind, tiles, x)
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), j
    finally:
        o.close()


CASES = [  # (mode, kind, rows, cols)
    ("store", "fp16", 40, 2048), ("accum", "bf16", 33, 11008), ("swiglu", "fp16", 26, 2048),
    ("logits", "bf16", 300, 2048), ("store", "int8", 37, 4096), ("accum", "int8", 19, 12288),
    ("swiglu", "int8", 22, 4096), ("logits", "int8", 130, 4096),
]


@pytest.mark.parametrize("mode,kind,rows,cols", CASES)
def test_raw_gemv_matches_oracle(mode, kind, rows, cols):
    rng = np.random.default_rng(rows * 3 + cols)
    say(f"raw gemv mode={mode} kind={kind} rows={rows} cols={cols}")
    tiles, dec = make_tiles(rng, kind, rows, cols)
    x = rng.standard_normal(cols).astype(np.float32)
    tol = TOL[kind]
    o = oracle_archive(kind, tiles)
    try:
        if mode in ("store", "accum"):
            y0 = rng.standard_normal(rows).astype(np.float32) if mode == "accum" else None
            got = ca.gpu_gemv_raw(mode, rows, cols, kind, tiles, x, y=y0)
            want = o.gemv_linear(0, tiles.shape[0], x, rows, cols)
            mag = np.abs(dec) @ np.abs(x.astype(np.float64))
            if y0 is not None:
                want = want + y0
                mag = mag + np.abs(y0)
            within(got, want, tol * mag + 1e-30)
            return
        gamma = (rng.standard_normal(cols) * 0.2 + 1.0).astype(np.float32)
        xn = orc.rmsnorm(x, gamma, 1e-6)
        axn = np.abs(xn).astype(np.float64)
        if mode == "swiglu":
            up, dec_up = make_tiles(rng, kind, rows, cols)
            ou = oracle_archive(kind, up)
            try:
                u = ou.gemv_linear(0, up.shape[0], xn, rows, cols)
            finally:
                ou.close()
            got = ca.gpu_gemv_raw(mode, rows, cols, kind, tiles, x, tiles_up=up, gamma=gamma, eps=1e-6)
            g = o.gemv_linear(0, tiles.shape[0], xn, rows, cols)
            sg = np.array([orc.silu(float(v)) for v in g], np.float32)
            want = sg * u
            gmag, umag = np.abs(dec) @ axn, np.abs(dec_up) @ axn
            within(got, want, 1.1 * tol * gmag * np.abs(u) + np.abs(sg) * tol * umag + 1e-6 * np.abs(want) + 1e-30)
            return
        got, am, hn = ca.gpu_gemv_raw(mode, rows, cols, kind, tiles, x, gamma=gamma, eps=1e-6)
        want = o.gemv_linear(0, tiles.shape[0], xn, rows, cols)
        mag = np.abs(dec) @ axn
        within(got, want, tol * mag + 1e-30)
        assert am == int(np.argmax(got))
        assert abs(hn - float(np.linalg.norm(x.astype(np.float64)))) <= 1e-5 * hn
    finally:
        o.close()


def test_raw_hook_rejects_short_tiles():
    with pytest.raises(ca.EngineError):
        ca.gpu_gemv_raw("store", 3, 8192, "int8", np.zeros((1, 16384), np.uint8), np.zeros(8192, np.float32))
