"""CPU emulation of one set of the matrix-core flat GEMV's operands (k_gemv_xm in
chpe-qwen-engine_amd/csrc/gemv.hip; gemvCellFlat, src/chpe_engine.zig:584-729): the limb
tables the waves build (including the 2-bit kernel's exchange between neighbouring lanes), the
B operands read from them, the A operands unpacked from the codes, and the products.

A v_mfma_i32_16x16x64_i8 sums, for output (m, n'), the products of byte i of A lane (m, kb) with
byte i of B lane (n', kb) over kb = 0..3 and i = 0..15; which k each (kb, i) stands for inside
the hardware does not change that sum, so the emulation needs no more than the pairing.  The
kernel keeps D(4 r + g, g + 4 L): unit row r, group g, limb L.  Each must equal the direct sum
over the group's 128 columns of (the code's operand value) x (limb L of the column's input),
4-bit operand = code, 2-bit operand = code ^ 2 (the value offsets are added separately)."""
import numpy as np
import pytest


def balanced_limbs(X):
    """Four signed bytes L0..L3 with X = L0 + 2^8 L1 + 2^16 L2 + 2^24 L3, as the kernel forms
    them: (uint32(X) + 0x808080) ^ 0x808080, byte by byte."""
    z = ((X.astype(np.int64) & 0xFFFFFFFF) + 0x808080) & 0xFFFFFFFF
    z ^= 0x808080
    b = np.stack([(z >> (8 * k)) & 0xFF for k in range(4)], axis=-1).astype(np.int64)
    return np.where(b >= 128, b - 256, b)  # [..., 4]


def limb_words(a, b, c, d):
    """w[L] = limb L of columns (a, b, c, d), the kernel's 4 x 4 byte transpose."""
    return [np.array([a[L], b[L], c[L], d[L]]) for L in range(4)]


def build_tables(limbs, bits):
    """limbs: [512 columns][4] for one set.  Returns entry[(g, q, h, L)] = 16 signed bytes
    (dwords lo_even, hi_even, lo_odd, hi_odd of the lane pair), as the prologue stores them."""
    entry = {}
    z = {lane: [limbs[8 * lane + i] for i in range(8)] for lane in range(64)}
    for lane in range(64):
        gs, gq, gh, odd = lane >> 4, (lane >> 2) & 3, (lane >> 1) & 1, lane & 1
        zl = z[lane]
        if bits == 2:
            zp = z[lane ^ 1]  # the neighbour's own columns
            # the neighbour sends odd ? its (z0, z1, z4, z5) : its (z2, z3, z6, z7)
            r = [zp[0], zp[1], zp[4], zp[5]] if not odd else [zp[2], zp[3], zp[6], zp[7]]
            if odd:
                lo = limb_words(r[0], r[2], zl[2], zl[6])
                hi = limb_words(r[1], r[3], zl[3], zl[7])
            else:
                lo = limb_words(zl[0], zl[4], r[0], r[2])
                hi = limb_words(zl[1], zl[5], r[1], r[3])
        else:
            lo = limb_words(zl[0], zl[2], zl[4], zl[6])
            hi = limb_words(zl[1], zl[3], zl[5], zl[7])
        for L in range(4):
            e = entry.setdefault((gs, gq, gh, L), [None] * 4)
            e[2 * odd] = lo[L]
            e[2 * odd + 1] = hi[L]
    return {k: np.concatenate(v) for k, v in entry.items()}


def a_operand(codes_row_group, q, h, bits):
    """16 unsigned bytes of A lane (m = 4 r + g, kb = q) for product h: the lane's code bytes of
    row r, group g, quarter q, unpacked as the kernel does."""
    c = codes_row_group  # 128 codes of the group (0..15 or 0..3)
    if bits == 4:
        # 16 bytes: byte b holds columns 32 q + 2 b (low nibble) and + 2 b + 1 (high)
        cols = 32 * q + np.arange(32)
        byts = c[cols[0::2]] | (c[cols[1::2]] << 4)
        w0, w1 = byts[8 * h:8 * h + 4], byts[8 * h + 4:8 * h + 8]
        return np.concatenate([w0 & 15, w0 >> 4, w1 & 15, w1 >> 4])
    # 2-bit, 8 bytes: byte b holds columns 32 q + 4 b + k in field k; product h uses bytes 4h..4h+3
    cols = 32 * q + np.arange(32)
    byts = c[cols[0::4]] | (c[cols[1::4]] << 2) | (c[cols[2::4]] << 4) | (c[cols[3::4]] << 6)
    w = byts[4 * h:4 * h + 4] ^ 0xAA
    return np.concatenate([(w >> (2 * k)) & 3 for k in range(4)])


@pytest.mark.parametrize("bits", [4, 2])
def test_operand_pairing_gives_group_dots(bits):
    rng = np.random.default_rng(41 + bits)
    x = (rng.standard_normal(512) * rng.choice([1e-3, 1.0, 40.0], 512)).astype(np.float32)
    codes = rng.integers(0, 16 if bits == 4 else 4, size=(4, 512))  # 4 unit rows, one set
    # the input as exact integers per group: X = trunc(x * 2^(30 - e)), max |x| < 2^e
    X = np.empty(512, np.int64)
    for g in range(4):
        xs = x[128 * g:128 * (g + 1)]
        e = int(np.frexp(np.float32(np.max(np.abs(xs))))[1])
        X[128 * g:128 * (g + 1)] = np.trunc(xs.astype(np.float64) * 2.0 ** (30 - e)).astype(np.int64)
    limbs = balanced_limbs(X)
    assert np.array_equal(limbs @ (np.int64(1) << (8 * np.arange(4))), X)
    table = build_tables(limbs, bits)
    for h in range(2):
        # B lane (n', kb): entry (g' = n' % 4, q = kb, h, L = n' // 4)
        B = {(n, kb): table[(n & 3, kb, h, n >> 2)] for n in range(16) for kb in range(4)}
        A = {(4 * r + g, kb): a_operand(codes[r, 128 * g:128 * (g + 1)], kb, h, bits)
             for r in range(4) for g in range(4) for kb in range(4)}
        for r in range(4):
            for g in range(4):
                for L in range(4):
                    d = sum(int(np.dot(A[(4 * r + g, kb)].astype(np.int64), B[(g + 4 * L, kb)])) for kb in range(4))
                    # the columns product h covers: 32 q + 16 h + 0..15 of the group, q = 0..3
                    cols = np.concatenate([32 * q + 16 * h + np.arange(16) for q in range(4)])
                    c = codes[r, 128 * g + cols]
                    val = c if bits == 4 else (c ^ 2)
                    want = int(np.dot(val.astype(np.int64), limbs[128 * g + cols, L]))
                    assert d == want, (bits, h, r, g, L)


def test_two_bit_operand_value():
    """(code ^ 2) - 2 is the codebook {0, +1, -2, -1} (gemvCellFlat's 2-bit decode)."""
    assert [(c ^ 2) - 2 for c in range(4)] == [0, 1, -2, -1]
