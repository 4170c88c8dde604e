"""The oracle's primitives against the reference's own known-answer tests and closed forms.

Each case names the reference test or the mathematical fact that fixes the expected value;
none of them recomputes the oracle's formula.
"""
import math

import numpy as np
import pytest

import oracle as orc

PAYLOAD = 64 + 16384  # cell = 64-byte bytecode header + 16384 code bytes + 960-byte payload


def synthetic_cell(bits, scale, rows=4, cols=128):
    """The reference's synthetic test cell (chpe_engine.zig:1813-1891): zeroed, no GROUP128."""
    cell = np.zeros(17408, dtype=np.uint8)
    cell[PAYLOAD + 20] = bits                                   # TileMetadata.quant_bits
    cell[PAYLOAD + 32:PAYLOAD + 36] = np.frombuffer(np.float32(scale).tobytes(), np.uint8)  # TileDims.scale
    cell[PAYLOAD + 40:PAYLOAD + 44] = np.frombuffer(np.uint32(rows).tobytes(), np.uint8)
    cell[PAYLOAD + 44:PAYLOAD + 48] = np.frombuffer(np.uint32(cols).tobytes(), np.uint8)
    return cell


# ---------------------------------------------------------------- GEMV closed forms
def test_gemv_2bit_synthetic_cell():
    # chpe_engine.zig:1813-1839: words[0] = 0x5555... -> the first 32 codes are 1 (+1 in the
    # codebook), everything else code 0 (0); scale 0.5, x = 1 -> row 0 = 32 * 0.5
    cell = synthetic_cell(2, 0.5)
    cell[64:72] = 0x55
    y = orc.gemv_tile(cell, np.ones(128, np.float32), 4)
    assert y.tolist() == [16.0, 0.0, 0.0, 0.0]


def test_gemv_4bit_synthetic_cell():
    # chpe_engine.zig:1841-1865: bytes 0..63 = 0x99 -> row 0 all nibbles 9 (+1), rows 1..3
    # nibble 0 (-8); scale 0.25 -> [128 * 0.25, 128 * -8 * 0.25, ...]
    cell = synthetic_cell(4, 0.25)
    cell[64:128] = 0x99
    y = orc.gemv_tile(cell, np.ones(128, np.float32), 4)
    assert y.tolist() == [32.0, -256.0, -256.0, -256.0]


def test_gemv_8bit_synthetic_cell():
    # chpe_engine.zig:1867-1891: bytes 0..127 = 10 (i8), scale 0.1 -> row 0 = 128 * 10 * 0.1
    cell = synthetic_cell(8, 0.1)
    cell[64:192] = 10
    y = orc.gemv_tile(cell, np.ones(128, np.float32), 4)
    assert y[0] == pytest.approx(128.0, abs=1e-4)
    assert y[1:].tolist() == [0.0, 0.0, 0.0]


def test_gemv_accumulate_adds_to_y():
    cell = synthetic_cell(4, 0.25)
    cell[64:128] = 0x99
    y0 = np.array([1.0, 2.0, 3.0, 4.0], np.float32)
    y = orc.gemv_tile(cell, np.ones(128, np.float32), 4, accumulate=True, y=y0)
    assert y.tolist() == [33.0, -254.0, -253.0, -252.0]


def test_flat_tile_group128_and_replace_outliers():
    # GROUP128 flat tile: nibble 9 (+1) everywhere, group g scale = g/64 (exact in fp16);
    # outliers REPLACE the dequantised weight (chpe_engine.zig:632-646); an offset past the
    # tile (>= 32768 is impossible in u16, so use n > 64) is ignored as a whole.
    cell = np.zeros(17408, dtype=np.uint8)
    cell[PAYLOAD + 20] = 4
    cell[PAYLOAD + 24] = 0x01  # GROUP128
    cell[64:64 + 16384] = 0x99
    scales = (np.arange(256) / 64.0).astype(np.float16)
    cell[PAYLOAD + 48:PAYLOAD + 48 + 512] = np.frombuffer(scales.tobytes(), np.uint8)
    offs = np.array([5, 1000, 32767], np.uint16)
    vals = np.array([3.0, -2.0, 0.5], np.float16)
    cell[PAYLOAD + 560:PAYLOAD + 562] = np.frombuffer(np.uint16(3).tobytes(), np.uint8)
    cell[PAYLOAD + 562:PAYLOAD + 568] = np.frombuffer(vals.tobytes(), np.uint8)
    cell[PAYLOAD + 690:PAYLOAD + 696] = np.frombuffer(offs.tobytes(), np.uint8)
    w = orc.flat_tile_weights(cell)
    expect = np.repeat(np.arange(256) / 64.0, 128).astype(np.float32)
    expect[offs] = vals.astype(np.float32)
    assert np.array_equal(w, expect)
    # more than 64 outliers: the whole list is ignored
    cell[PAYLOAD + 560:PAYLOAD + 562] = np.frombuffer(np.uint16(65).tobytes(), np.uint8)
    assert np.array_equal(orc.flat_tile_weights(cell), np.repeat(np.arange(256) / 64.0, 128).astype(np.float32))


def test_flat_tile_2bit_codebook():
    # 2-bit codebook {0: 0, 1: +1, 2: -2, 3: -1} (chpe_engine.zig:220); byte 0b11100100 holds
    # codes 0,1,2,3 for weights 0..3 (low bits first)
    cell = np.zeros(17408, dtype=np.uint8)
    cell[PAYLOAD + 20] = 2
    cell[PAYLOAD + 24] = 0x01
    cell[64:64 + 8192] = 0b11100100
    cell[PAYLOAD + 48:PAYLOAD + 48 + 512] = np.frombuffer(np.full(256, 0.5, np.float16).tobytes(), np.uint8)
    w = orc.flat_tile_weights(cell)
    assert np.array_equal(w, np.tile(np.array([0.0, 0.5, -1.0, -0.5], np.float32), 8192))


def _no_group_tile(bits, scale, bias):
    cell = np.zeros(17408, dtype=np.uint8)
    cell[PAYLOAD + 20] = bits                   # quant_bits, custom_flags 0: no GROUP128
    cell[PAYLOAD + 32:PAYLOAD + 36] = np.frombuffer(np.float32(scale).tobytes(), np.uint8)
    cell[PAYLOAD + 36:PAYLOAD + 40] = np.frombuffer(np.float32(bias).tobytes(), np.uint8)
    n = 16384 if bits == 4 else 8192
    cell[64:64 + n] = (np.arange(n) * 37 + 11).astype(np.uint8)   # every code value occurs
    return cell


@pytest.mark.parametrize("bits", [4, 2])
def test_flat_tile_no_group_scale_bias(bits):
    # gemvCellFlat without GROUP128 (chpe_engine.zig:619-630 for 4 bits, :666-677 for 2): every
    # weight is value * dims.scale + dims.bias over the tile's wpt weights, the product and the
    # sum rounded separately.  Exact case: scale 0.5, bias 0.25 (every result representable).
    # Rounding case: scale 0.1, bias 0.3 -- the expected value is two float32 roundings (numpy's
    # float32 multiply, then add); for 4-bit codes a fused multiply-add differs from it on some
    # codes, which the assert below also checks, so a contracted restatement fails.
    n = 16384 if bits == 4 else 8192
    codes = (np.arange(n) * 37 + 11).astype(np.uint8)
    if bits == 4:
        val = np.stack([(codes & 15).astype(np.float32) - 8, (codes >> 4).astype(np.float32) - 8], 1).reshape(-1)
    else:
        book = np.array([0.0, 1.0, -2.0, -1.0], np.float32)   # CODEBOOK_W2 (:220)
        val = np.stack([book[(codes >> (2 * s)) & 3] for s in range(4)], 1).reshape(-1)
    w = orc.flat_tile_weights(_no_group_tile(bits, 0.5, 0.25))
    assert np.array_equal(w, val * np.float32(0.5) + np.float32(0.25))
    s, b = np.float32(0.1), np.float32(0.3)
    w = orc.flat_tile_weights(_no_group_tile(bits, s, b))
    expect = (val * s).astype(np.float32) + b
    assert np.array_equal(w, expect)
    if bits == 4:  # (the 2-bit values +-1, -2 make every product exact: nothing to contract)
        fused = (val.astype(np.float64) * np.float64(s) + np.float64(b)).astype(np.float32)
        assert not np.array_equal(expect, fused)
    # outliers still replace (:632-646), the last entry of an offset counting
    cell = _no_group_tile(bits, 0.5, 0.25)
    offs = np.array([7, 7, 30000], np.uint16)
    vals = np.array([1.5, -3.0, 2.0], np.float16)
    cell[PAYLOAD + 560:PAYLOAD + 562] = np.frombuffer(np.uint16(3).tobytes(), np.uint8)
    cell[PAYLOAD + 562:PAYLOAD + 568] = np.frombuffer(vals.tobytes(), np.uint8)
    cell[PAYLOAD + 690:PAYLOAD + 696] = np.frombuffer(offs.tobytes(), np.uint8)
    w = orc.flat_tile_weights(cell)
    expect = val * np.float32(0.5) + np.float32(0.25)
    expect[7], expect[30000] = -3.0, 2.0
    assert np.array_equal(w, expect)
    # and the tile's dot onto rows: a 256 x 128 tensor (one tile) against x = e_c picks column c
    for c in (0, 77, 127):
        x = np.zeros(128, np.float32)
        x[c] = 1.0
        y = orc.gemv_cell_flat(cell, 0, 256, 128, x, np.zeros(256, np.float32))
        assert np.array_equal(y, expect.reshape(256, 128)[:, c])


# ---------------------------------------------------------------- RoPE / SiLU / RMSNorm
def test_rope_known_answer():
    # src/qwen_rope.zig:149-162: x[i] = (i+1)*0.1, pos 1, theta 1e6, head_dim 128
    x = (np.arange(128) + 1) * 0.1
    out = orc.rope(x, 1, 1, 128)
    assert out[0] == pytest.approx(-5.415531, abs=1e-4)
    assert out[1] == pytest.approx(-4.622832, abs=1e-4)
    assert out[64] == pytest.approx(3.596112, abs=1e-4)
    assert out[65] == pytest.approx(4.714808, abs=1e-4)


def test_rope_pos0_identity_and_closed_form():
    rng = np.random.default_rng(0)
    x = rng.standard_normal(4 * 128).astype(np.float32)
    assert np.array_equal(orc.rope(x, 0, 4, 128), x)  # qwen_rope.zig:90-102
    pos, hd, theta = 37, 128, 1e6
    out = orc.rope(x, pos, 4, hd).astype(np.float64)
    xx = x.astype(np.float64).reshape(4, hd)
    i = np.arange(hd // 2)
    ang = pos * theta ** (-2.0 * i / hd)  # rotate-half pairs (i, i + hd/2)
    ref = np.concatenate([xx[:, :64] * np.cos(ang) - xx[:, 64:] * np.sin(ang),
                          xx[:, 64:] * np.cos(ang) + xx[:, :64] * np.sin(ang)], axis=1).reshape(-1)
    assert np.abs(out - ref).max() < 1e-4
    # a rotation keeps every pair's norm (qwen_rope.zig:104-124)
    n0 = np.hypot(xx[:, :64], xx[:, 64:])
    n1 = np.hypot(out.reshape(4, hd)[:, :64], out.reshape(4, hd)[:, 64:])
    assert np.abs(n0 - n1).max() < 1e-5


def test_silu_and_swiglu_known_answers():
    # src/qwen_mlp.zig:92-111
    assert orc.silu(0.0) == 0.0
    assert orc.silu(1.0) == pytest.approx(0.7310586, abs=1e-5)
    g, u = [0.0, 1.0, -1.0, 2.0], [5.0, 2.0, 3.0, 0.5]
    assert orc.silu(g[1]) * u[1] == pytest.approx(1.462117, abs=1e-5)
    assert orc.silu(-30.0) == pytest.approx(-30.0 / (1.0 + math.exp(30.0)), rel=1e-5)


def test_rmsnorm_known_answer_and_float64():
    # src/qwen_rmsnorm.zig:73-90: x = 1, gamma = 2 -> 2.0
    y = orc.rmsnorm(np.ones(64, np.float32), np.full(64, 2.0, np.float32))
    assert np.abs(y - 2.0).max() < 1e-4
    rng = np.random.default_rng(1)
    for n in (8, 128, 2048):
        x = rng.standard_normal(n).astype(np.float32) * 3
        g = rng.standard_normal(n).astype(np.float32)
        ref = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6) * g
        assert np.abs(orc.rmsnorm(x, g) - ref).max() < 1e-5 * max(1.0, np.abs(ref).max())


# ---------------------------------------------------------------- attention
def test_attention_single_position_returns_v():
    # src/qwen_attention.zig:144-169: one position -> softmax weight exp(0)/exp(0) = 1 exactly
    rng = np.random.default_rng(2)
    H, KV, hd = 16, 2, 128
    q = rng.standard_normal(H * hd).astype(np.float32)
    k = rng.standard_normal((1, KV * hd)).astype(np.float32)
    v = rng.standard_normal((1, KV * hd)).astype(np.float32)
    out = orc.attention(q, k, v, 0, H, KV, hd).reshape(H, hd)
    for h in range(H):
        assert np.array_equal(out[h], v[0].reshape(KV, hd)[h // (H // KV)])


@pytest.mark.parametrize("pos", [1, 7, 63])
def test_attention_float64_brute_force(pos):
    rng = np.random.default_rng(pos)
    H, KV, hd = 16, 2, 128
    q = rng.standard_normal(H * hd).astype(np.float32)
    k = rng.standard_normal((pos + 1, KV * hd)).astype(np.float32)
    v = rng.standard_normal((pos + 1, KV * hd)).astype(np.float32)
    out = orc.attention(q, k, v, pos, H, KV, hd).reshape(H, hd)
    for h in range(H):
        g = h // (H // KV)
        kk = k.reshape(pos + 1, KV, hd)[:, g].astype(np.float64)
        vv = v.reshape(pos + 1, KV, hd)[:, g].astype(np.float64)
        s = kk @ q.reshape(H, hd)[h].astype(np.float64) / math.sqrt(hd)
        p = np.exp(s - s.max())
        ref = (p / p.sum()) @ vv
        assert np.abs(out[h] - ref).max() < 1e-5
        # the output is a convex combination of the V rows (qwen_attention.zig:171-189)
        assert (out[h] <= vv.max(axis=0) + 1e-5).all() and (out[h] >= vv.min(axis=0) - 1e-5).all()


# ---------------------------------------------------------------- fp16 widening and rounding
def test_f16_widening_exhaustive():
    # every one of the 65536 codes against numpy's float16 -> float32 (exact by definition):
    # finite values and infinities bit for bit, NaN codes as NaN
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = h.view(np.float16).astype(np.float32)
    got = orc.f16_to_f32_array(h)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))
    # the scalar entry point agrees with the array one
    for v in range(0, 65536, 251):
        g = orc.f16_to_f32(v)
        assert g == got[v] or (np.isnan(g) and np.isnan(got[v]))


def test_f32_to_f16_matches_numpy():
    # The fp16 KV cache's rounding (round to nearest, ties to even) against numpy's float16
    # conversion, an independent implementation of IEEE 754 binary16 rounding.  Every f32 bit
    # pattern whose exponent lies in [2^-26, 2^16] -- both signs, all 2^23 mantissas of each
    # exponent -- which holds every rounding boundary that matters: the subnormal range and its
    # edge at 2^-25 (half the smallest subnormal), the ties between subnormals, the normal/
    # subnormal switch at 2^-14, ties to even across every binade, and overflow to infinity at
    # 65520 (the tie between 65504 and 2^16).  Below that range everything rounds to signed
    # zero and above it to infinity (random samples of both), plus infinities and NaN.
    mant = np.arange(1 << 23, dtype=np.uint32)
    for e in range(127 - 26, 127 + 16 + 1):
        for sign in (0, 1):
            bits = (np.uint32(sign << 31) | np.uint32(e << 23) | mant).view(np.float32)
            got = orc.f32_to_f16_array(bits)
            ref = bits.astype(np.float16).view(np.uint16)
            assert np.array_equal(got, ref), (e, sign, int(np.argmax(got != ref)))
    rng = np.random.default_rng(0)
    low = (rng.integers(0, 127 - 26, 100000).astype(np.uint32) << 23) | rng.integers(0, 1 << 23, 100000).astype(np.uint32)
    high = (rng.integers(127 + 17, 255, 100000).astype(np.uint32) << 23) | rng.integers(0, 1 << 23, 100000).astype(np.uint32)
    for bits in (low, high, low | np.uint32(1 << 31), high | np.uint32(1 << 31)):
        x = bits.view(np.float32)
        assert np.array_equal(orc.f32_to_f16_array(x), x.astype(np.float16).view(np.uint16))
    special = np.array([np.inf, -np.inf, 0.0, -0.0, 65504.0, 65519.996, 65520.0, 2.0 ** -24, 2.0 ** -25,
                        2.0 ** -25 * (1 + 2.0 ** -23), 2.0 ** -26], np.float32)
    assert np.array_equal(orc.f32_to_f16_array(special), special.astype(np.float16).view(np.uint16))
    nan = orc.f32_to_f16_array(np.array([np.nan, -np.nan], np.float32)).view(np.float16)
    assert np.isnan(nan).all()
