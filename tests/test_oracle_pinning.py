"""Pins the oracle's functions that the whole-archive quantization tests leave open (CPU only).

Each check is independent of the oracle's own code: float64 arithmetic on the generator's
weights (include/chpe_pack.h), numpy decoders written from the reference's byte layout
(src/chpe_engine.zig), or the reference's own known-answer test.  A transposed operand, a
dropped or misplaced norm, residual or bias, a wrong head mapping or a wrong outlier rule
moves the results by orders of magnitude more than the bounds allow.

  raw fp16 / bf16 gemvLinear + dotSegment (:1194-1286, :1455-1488), rows straddling tiles
      -> float64 W x from the generator (exact widening), bounded by the f32 summation error
  raw unpackEmbedRow (:1500-1530) -> the generator's weights, bit for bit
  raw tied computeLmHead (:1613-1659) -> float64 E x, f32 summation bound
  gemvTileF16 / gemvTileF32 (:475-581) -> float64 brute force, f32 summation bound
  unpackEmbedRowCell q8 / q2 / q4 / per-tile scale forms (:1288-1394) -> numpy decode, exact
  forwardDecode on the all-zero mock archive -> the reference's KAT (:1893-1933) and the
      closed forms its synthetic fallbacks give (:1493-1498, :1558-1563)
  forwardDecode composition on the Qwen2.5-3B 4-bit archive -> a float64 restatement of two
      decode steps from the reference's forwardDecode, on weights decoded by numpy
"""
import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

CELL, PL, CODES = 17408, 16448, 64
U = 2.0 ** -24


def f32_dot_bound(w, x):
    """Bound of an f32 dot product of length C accumulated in 8 lanes then reduced in order
    (the reference's @Vector(8, f32) + @reduce): (C/8 + 8) u sum|w x|."""
    C = w.shape[-1]
    return (C / 8 + 8) * U * (np.abs(w) @ np.abs(x))


def tid(layer, which):
    return 1000 * (layer + 1) + which


def bf16_round(w):
    b = np.ascontiguousarray(w, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def raw_weights(kind, t, first, n):
    w = ca.normals(0, t, first, n)
    return (w.astype(np.float16).astype(np.float64) if kind == ca.PACK_3B_FP16_RAW
            else bf16_round(w).astype(np.float64))


# ------------------------------------------------------------------ raw archives (C0's path)
@pytest.fixture(scope="module", params=[ca.PACK_3B_FP16_RAW, ca.PACK_3B_BF16_RAW], ids=["fp16", "bf16"])
def raw_prefix(request):
    """The embedding and layer 0 of the raw 3B archive (records 0 .. 47396), header count
    set to match, opened by the oracle from memory."""
    kind = request.param
    n = 37984 + 9413
    hdr = ca.pack_header(kind)
    hdr[16:24] = np.frombuffer(np.uint64(n).tobytes(), np.uint8)
    data = np.concatenate([hdr, ca.pack_records(kind, 0, n).reshape(-1)])
    o = orc.Oracle(data=data, arch=0, max_seq_len=8, threads=8)
    yield kind, o
    o.close()


@pytest.mark.parametrize("name,which,rows,cols,bias", [
    ("q", 1, 2048, 2048, 11), ("k", 2, 256, 2048, 12), ("down", 7, 2048, 11008, None)])
def test_raw_gemv_linear_is_float64_product(raw_prefix, name, which, rows, cols, bias):
    kind, o = raw_prefix
    li = orc.layer_info(0, 0)
    x = np.random.default_rng(which).standard_normal(cols).astype(np.float32)
    y = o.gemv_linear(li[f"{name}_proj"], li[f"{name}_tiles"], x, rows, cols,
                      bias_tile=li.get(f"{name}_bias", -1)).astype(np.float64)
    w = raw_weights(kind, tid(0, which), 0, rows * cols).reshape(rows, cols)
    ref = w @ x.astype(np.float64)
    bound = f32_dot_bound(w, x.astype(np.float64))
    if bias is not None:
        b = ca.normals(0, tid(0, bias), 0, rows).astype(np.float64)
        ref += b
        bound += U * (np.abs(ref) + np.abs(b))
    assert (np.abs(y - ref) <= bound).all(), float(np.abs(y - ref).max())
    # the transposed product is nowhere near: the bound has resolving power
    if rows == cols:
        assert np.abs(y - (w.T @ x.astype(np.float64) + (ref - w @ x.astype(np.float64)))).max() > 100 * bound.max()


def test_raw_gemv_accumulate_adds(raw_prefix):
    kind, o = raw_prefix
    li = orc.layer_info(0, 0)
    x = np.random.default_rng(9).standard_normal(2048).astype(np.float32)
    y0 = np.random.default_rng(10).standard_normal(2048).astype(np.float32)
    y = o.gemv_linear(li["o_proj"], li["o_tiles"], x, 2048, 2048, accumulate=True, y=y0.copy()).astype(np.float64)
    w = raw_weights(kind, tid(0, 4), 0, 2048 * 2048).reshape(2048, 2048)
    ref = y0 + w @ x.astype(np.float64)
    assert (np.abs(y - ref) <= f32_dot_bound(w, x.astype(np.float64)) + U * np.abs(ref) * 2).all()


def test_raw_embedding_rows_are_the_weights(raw_prefix):
    kind, o = raw_prefix
    for tok in (0, 3, 4, 77777, 151935):  # 4 rows per 16 KB tile
        want = raw_weights(kind, 1, tok * 2048, 2048).astype(np.float32)
        assert np.array_equal(o.embed_row(tok), want), tok


def test_raw_tied_lm_head_is_float64_product(raw_prefix):
    kind, o = raw_prefix
    xn = np.random.default_rng(3).standard_normal(2048).astype(np.float32)
    logits = o.lm_head(xn).astype(np.float64)
    rows = np.r_[0:9, 40000:40013, 151920:151936]
    E = np.stack([raw_weights(kind, 1, int(r) * 2048, 2048) for r in rows])
    ref = E @ xn.astype(np.float64)
    assert (np.abs(logits[rows] - ref) <= f32_dot_bound(E, xn.astype(np.float64))).all()


def test_raw_int8_dot_segment_and_embedding():
    """Raw int8 tiles (the 9B int8 archive: flags 0x08, dotSegment :1219-1237): each segment's
    dot of int8 weights is scaled by the fixed 0.00373708 (the per-tensor scales of the map are
    never read); embedding rows are int8 * 0.00373708 (:1511-1522).  Rows of 12288 columns
    straddle the 16384-element tiles."""
    rng = np.random.default_rng(88)
    n_tiles, C = 12, 12288
    tiles = rng.integers(-128, 128, n_tiles * 16384, dtype=np.int8)
    hdr = np.zeros(4096, np.uint8)
    hdr[:4] = np.frombuffer(np.uint32(0x45504843).tobytes(), np.uint8)
    fields = np.array([1, 0], np.uint32)  # version
    hdr[4:8] = np.frombuffer(fields[:1].tobytes(), np.uint8)
    hdr[8:64] = np.frombuffer(np.array([4096, n_tiles, n_tiles, 16384, 16384, 0, 0x08], np.uint64).tobytes(), np.uint8)
    o = orc.Oracle(data=np.concatenate([hdr, tiles.view(np.uint8)]), arch=1, max_seq_len=4, threads=4)
    try:
        assert o.info()["is_raw"] == 1 and o.info()["quant_bits"] == 8
        rows = n_tiles * 16384 // C
        x = rng.standard_normal(C).astype(np.float32)
        y = o.gemv_linear(0, n_tiles, x, rows, C).astype(np.float64)
        w = tiles[:rows * C].astype(np.float64).reshape(rows, C)
        s = float(np.float32(0.00373708))
        ref = (w @ x.astype(np.float64)) * s
        bound = (f32_dot_bound(w, x.astype(np.float64)) + 2 * U * np.abs(w) @ np.abs(x.astype(np.float64))) * s
        assert (np.abs(y - ref) <= bound + 2 * U * np.abs(ref)).all()
        for tok in (0, 1, 5, 47):  # 16384 / 4096 = 4 rows per tile
            want = tiles[tok * 4096:(tok + 1) * 4096].astype(np.float32) * np.float32(0.00373708)
            assert np.array_equal(o.embed_row(tok), want)
    finally:
        o.close()


# ------------------------------------------------------------------ 16- and 32-bit cells
def cell_with(bits, rows, cols, flags, codes):
    cell = np.zeros(CELL, np.uint8)
    cell[CODES:CODES + codes.size] = codes
    pl = cell[PL:]
    pl[20] = bits
    pl[24:32] = np.frombuffer(np.uint64(flags).tobytes(), np.uint8)
    pl[40:48] = np.frombuffer(np.array([rows, cols], np.uint32).tobytes(), np.uint8)
    return cell


@pytest.mark.parametrize("form,rows,cols,x_len", [
    ("fp16", 4, 2048, 2048), ("bf16", 4, 2048, 2048), ("f32", 2, 2048, 2048),
    ("fp16", 7, 1000, 1000), ("bf16", 3, 2000, 1003), ("f32", 5, 800, 613)])
def test_f16_bf16_f32_cells_are_float64_products(form, rows, cols, x_len):
    rng = np.random.default_rng(rows * cols + x_len)
    w32 = (rng.standard_normal((rows, cols)) * 0.05).astype(np.float32)
    if form == "fp16":
        w = w32.astype(np.float16)
        cell = cell_with(16, rows, cols, 0x04, w.view(np.uint8).reshape(-1))
    elif form == "bf16":
        w = bf16_round(w32)
        cell = cell_with(16, rows, cols, 0x00, (w.view(np.uint32) >> 16).astype(np.uint16).view(np.uint8).reshape(-1))
    else:
        w = w32
        cell = cell_with(32, rows, cols, 0x00, w.view(np.uint8).reshape(-1))
    w = w.astype(np.float64)
    x = rng.standard_normal(x_len).astype(np.float32)
    n = min(cols, x_len)  # max_cols = min(cols, x.len)
    ref = w[:, :n] @ x[:n].astype(np.float64)
    bound = f32_dot_bound(w[:, :n], np.abs(x[:n]).astype(np.float64))
    y = orc.gemv_tile(cell, x, rows + 3, row_base=1).astype(np.float64)
    assert y[0] == 0 and (y[rows + 1:] == 0).all()  # rows outside [row_base, row_base + rows)
    assert (np.abs(y[1:rows + 1] - ref) <= bound).all()
    y0 = rng.standard_normal(rows).astype(np.float32)
    ya = orc.gemv_tile(cell, x, rows, row_base=0, accumulate=True, y=y0.copy()).astype(np.float64)
    assert (np.abs(ya - (y0 + ref)) <= bound + 2 * U * np.abs(y0 + ref)).all()
    yc = orc.gemv_tile(cell, x, rows - 1, row_base=0)  # y shorter than the cell: max_rows clips
    assert yc.size == rows - 1


# ------------------------------------------------------------------ embedding rows of cells
def f16(b):
    return np.frombuffer(np.asarray(b, np.uint8).tobytes(), np.float16).astype(np.float32)


def decode_embed_row(region, row, D, init):
    """unpackEmbedRowCell (:1288-1394) restated over the bytes of `region` (cell at 0)."""
    out = init.copy()
    pl = region[PL:]
    bits, flags = int(pl[20]), int(np.frombuffer(pl[24:32].tobytes(), np.uint64)[0])
    ng, codes = D // 128, region[CODES:]
    g128 = flags & 1 != 0

    def scales(r):
        return f16(pl[48 + 2 * r * ng:48 + 2 * (r + 1) * ng])

    if bits == 8:
        if row >= 8:
            return out
        q = codes[row * D:(row + 1) * D].view(np.int8).astype(np.float32)
        return q * np.repeat(scales(row), 128)
    if bits == 2 or g128 or bits == 4:
        if row >= 16:
            return out
        if bits == 2:
            b = codes[row * (D // 4):(row + 1) * (D // 4)]
            q = np.stack([(b >> (2 * k)) & 3 for k in range(4)], 1).reshape(-1)
            val = np.array([0.0, 1.0, -2.0, -1.0], np.float32)[q]
        else:
            b = codes[row * (D // 2):(row + 1) * (D // 2)]
            val = np.stack([b & 15, b >> 4], 1).reshape(-1).astype(np.float32) - np.float32(8.0)
        out = (val * np.repeat(scales(row), 128)).astype(np.float32)
        if g128:
            cols = np.frombuffer(pl[816:832].tobytes(), np.uint16)
            ow = f16(pl[560:816])
            for k in range(8):
                if cols[k] < D:
                    out[cols[k]] = ow[row * 8 + k]
        return out
    scale, bias = np.frombuffer(pl[32:40].tobytes(), np.float32)
    b = codes[row * (D // 2):(row + 1) * (D // 2)]
    q = np.stack([b & 15, b >> 4], 1).reshape(-1).astype(np.float32)
    return ((q - np.float32(8.0)) * scale + bias).astype(np.float32)


@pytest.mark.parametrize("bits,flags,D", [
    (8, 0, 2048), (8, 1, 4096), (2, 1, 2048), (2, 0, 4096), (4, 1, 2048), (4, 0, 8192), (0, 0, 4096), (3, 0, 8192)])
def test_embed_row_cell_forms_match_numpy_decode(bits, flags, D):
    rng = np.random.default_rng(bits * 10 + flags + D)
    region = rng.integers(0, 256, CELL * 5, dtype=np.uint8)  # wide rows read into the next cells
    pl = region[PL:PL + 960]
    pl[20] = bits
    pl[24:32] = np.frombuffer(np.uint64(flags).tobytes(), np.uint8)
    # finite scales and outlier weights: f16 values in [-0.1, 0.1]
    pl[48:816] = np.frombuffer((rng.standard_normal(384) * 0.03).astype(np.float16).tobytes(), np.uint8)
    pl[32:40] = np.frombuffer(np.array([0.0123, -0.004], np.float32).tobytes(), np.uint8)
    cols = rng.integers(0, D, 8).astype(np.uint16)
    cols[3] = cols[5]          # a repeated column: the later entry wins
    cols[6] = D + 7            # out of range: skipped
    pl[816:832] = np.frombuffer(cols.tobytes(), np.uint8)
    for row in (0, 3, 7, 8, 15, 16):
        init = np.full(D, 5.0, np.float32)
        _, got = orc.embed_row_cell(region, row, D, init)
        want = decode_embed_row(region, row, D, init)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (bits, flags, D, row)


# ------------------------------------------------------------------ forwardDecode
@pytest.mark.parametrize("arch", [0, 1, 2])
def test_mock_zero_archive_known_answer(arch):
    """The reference's test "unified CHPEEngine forwardDecode on ... architecture"
    (chpe_engine.zig:1893-1933): an all-zero 8 KiB archive, token 151644 at position 0 gives a
    finite result with hidden_norm > 0.  With the invalid archive every fallback is a closed
    form: the embedding 0.05 ((i + token) % 17 - 8), q/k/v 0.01 ((r % 13) - 6), the o and down
    accumulations leave the residual untouched, and the logits are 0.001 ((v % 13) - 6)."""
    o = orc.Oracle(data=np.zeros(8192, np.uint8), arch=arch, max_seq_len=16, threads=4)
    try:
        r = o.forward(151644, 0)
        D = o.info()["hidden_dim"] if "hidden_dim" in o.info() else o.L.oref_hidden_dim(o.e)
        i = np.arange(D)
        emb = np.float32(0.05) * (((i + 151644) % 17) - 8).astype(np.float32)
        assert r.all_finite and r.hidden_norm > 0.0
        assert np.array_equal(o.hidden(), emb)
        sq = np.float32(0.0)
        for v in emb:  # the reference's sequential f32 sum of squares (:1789-1792)
            sq = np.float32(sq + np.float32(v * v))
        assert r.hidden_norm == np.sqrt(sq)
        assert r.argmax_token == 12 and r.max_logit == np.float32(0.006) and r.token0_logit == np.float32(-0.006)
    finally:
        o.close()


def _cells(mm, first, n):
    off = 4096 + first * CELL
    return np.asarray(mm[off:off + n * CELL]).reshape(n, CELL)


def _w4_cells(c):
    """16-row W4 cells (gemvTileW4, :326-418): weights [n][16][2048] without outliers, and the
    added outliers as (cols [n][8], weights [n][16][8])."""
    n = c.shape[0]
    b = c[:, CODES:CODES + 16384].reshape(n, 16, 1024)
    q = np.stack([b & 15, b >> 4], 3).reshape(n, 16, 2048).astype(np.float64) - 8.0
    s = f16(c[:, PL + 48:PL + 560]).reshape(n, 16, 16).astype(np.float64)
    w = q * np.repeat(s, 128, axis=2)
    cols = np.frombuffer(c[:, PL + 816:PL + 832].tobytes(), np.uint16).reshape(n, 8)
    ow = f16(c[:, PL + 560:PL + 816]).reshape(n, 16, 8).astype(np.float64)
    return w, cols, ow


def _matrix_cells(mm, first, n_cells, rows):
    """W (rows x 2048) of a 16-row-cell tensor with its outliers added (:404-410)."""
    w, cols, ow = _w4_cells(_cells(mm, first, n_cells))
    for t in range(n_cells):
        for k in range(8):
            if cols[t, k] < 2048:
                w[t, :, cols[t, k]] += ow[t, :, k]
    return w.reshape(-1, 2048)[:rows]


def _matrix_flat(mm, first, rows, cols):
    """W (rows x cols) of a flat-tile tensor (gemvCellFlat, :584-729): outliers replace."""
    n = (rows * cols + 32767) // 32768
    c = _cells(mm, first, n)
    b = c[:, CODES:CODES + 16384]
    q = np.stack([b & 15, b >> 4], 2).reshape(n, 32768).astype(np.float64) - 8.0
    s = f16(c[:, PL + 48:PL + 560]).reshape(n, 256).astype(np.float64)
    w = q * np.repeat(s, 128, axis=1)
    for t in range(n):
        k = int(np.frombuffer(c[t, PL + 560:PL + 562].tobytes(), np.uint16)[0])
        if 0 < k <= 64:
            offs = np.frombuffer(c[t, PL + 690:PL + 690 + 2 * k].tobytes(), np.uint16)
            ws = f16(c[t, PL + 562:PL + 562 + 2 * k]).astype(np.float64)
            for m in range(k):
                w[t, offs[m]] = ws[m]
    return w.reshape(-1)[:rows * cols].reshape(rows, cols)


def _vector(mm, rec, n):
    off = 4096 + rec * CELL + CODES
    return np.frombuffer(np.asarray(mm[off:off + 4 * n]).tobytes(), np.float32).astype(np.float64)


def _embed_rows(mm, tokens):
    """unpackEmbedRowCell rows (4-bit, outliers replace in entry order, :1348-1378)."""
    out = []
    for tok in tokens:
        w, cols, ow = _w4_cells(_cells(mm, int(tok) // 16, 1))
        row = w[0, int(tok) % 16].copy()
        for k in range(8):
            if cols[0, k] < 2048:
                row[cols[0, k]] = ow[0, int(tok) % 16, k]
        out.append(row)
    return np.stack(out)


def test_forward_decode_composition_float64(w4_archive):
    """Two decode steps of Qwen2.5-3B on the 4-bit cell archive, restated in float64 from the
    reference's forwardDecode (:1663-1803): embedding, per layer input RMSNorm, q/k/v with
    bias, NeoX RoPE at the position, KV append, GQA softmax attention (query head h reads kv
    head h / 8), o projection added to the residual, post-attention RMSNorm, silu(gate) * up,
    down projection added to the residual; final RMSNorm and the tied LM head.  Weights are
    decoded by numpy from the cell bytes.  The oracle (f32) must agree to f32 rounding."""
    mm = np.memmap(w4_archive, dtype=np.uint8, mode="r")
    D, H, KV, hd, eps, theta = 2048, 16, 2, 128, 1e-6, 1e6
    toks = [151643, 9707]

    def rms(x, g):
        return x / np.sqrt(np.mean(x * x) + eps) * g

    def rope(v, pos, heads):
        v = v.reshape(heads, hd).copy()
        i = np.arange(hd // 2)
        ang = pos * (1.0 / theta ** (2.0 * i / hd))
        c, s = np.cos(ang), np.sin(ang)
        a, b = v[:, :hd // 2].copy(), v[:, hd // 2:].copy()
        v[:, :hd // 2], v[:, hd // 2:] = a * c - b * s, a * s + b * c
        return v.reshape(-1)

    h = _embed_rows(mm, toks)  # [pos][D]
    kc = np.zeros((36, 2, KV * hd))
    vc = np.zeros((36, 2, KV * hd))
    for l in range(36):
        li = orc.layer_info(1, l)
        g_in, g_post = _vector(mm, li["input_norm"], D), _vector(mm, li["post_norm"], D)
        Wq = _matrix_cells(mm, li["q_proj"], 128, 2048)
        Wk = _matrix_cells(mm, li["k_proj"], 16, 256)
        Wv = _matrix_cells(mm, li["v_proj"], 16, 256)
        Wo = _matrix_cells(mm, li["o_proj"], 128, 2048)
        Wg = _matrix_cells(mm, li["gate_proj"], 688, 11008)
        Wu = _matrix_cells(mm, li["up_proj"], 688, 11008)
        Wd = _matrix_flat(mm, li["down_proj"], 2048, 11008)
        bq, bk, bv = (_vector(mm, li[f"{n}_bias"], r) for n, r in (("q", 2048), ("k", 256), ("v", 256)))
        for pos in range(2):
            xn = rms(h[pos], g_in)
            q = rope(Wq @ xn + bq, pos, H)
            kc[l, pos] = rope(Wk @ xn + bk, pos, KV)
            vc[l, pos] = Wv @ xn + bv
            att = np.zeros(H * hd)
            for head in range(H):
                kvh = head // (H // KV)
                K = kc[l, :pos + 1, kvh * hd:(kvh + 1) * hd]
                Vv = vc[l, :pos + 1, kvh * hd:(kvh + 1) * hd]
                sc = K @ q[head * hd:(head + 1) * hd] / np.sqrt(hd)
                p = np.exp(sc - sc.max())
                att[head * hd:(head + 1) * hd] = (p / p.sum()) @ Vv
            h[pos] = h[pos] + Wo @ att
            xn = rms(h[pos], g_post)
            gate = Wg @ xn
            h[pos] = h[pos] + Wd @ (gate / (1.0 + np.exp(-gate)) * (Wu @ xn))
    fin = _vector(mm, 94348, D)
    o = orc.Oracle(w4_archive, arch=0, max_seq_len=8, threads=8)
    try:
        for pos in range(2):
            r = o.forward(toks[pos], pos)
            xn = rms(h[pos], fin)
            got = o.logits().astype(np.float64)
            rows = np.r_[0:2000, 70000:71000, 150936:151936, r.argmax_token]
            ref = _embed_rows(mm, rows) @ xn
            d = np.abs(got[rows] - ref)
            assert d.max() <= 1e-3 * np.abs(ref).max(), (pos, float(d.max()))
            assert float(np.linalg.norm(o.hidden())) == pytest.approx(float(np.linalg.norm(h[pos])), rel=1e-4)
            # the oracle's argmax row is the float64 maximum over the rows checked
            assert np.argmax(ref) == rows.size - 1 or ref[-1] >= ref.max() - 1e-3
    finally:
        o.close()


@pytest.mark.parametrize("bits", [4, 2])
def test_flat_code_value_identities(bits):
    """The matrix-core flat GEMV takes each code as an unsigned operand and a constant offset:
    4-bit value = code - 8 (low nibble = even column), 2-bit value = (code ^ 2) - 2 (the
    codebook {0, +1, -2, -1} of gemvCellFlat, src/chpe_engine.zig:584-729, is the 2-bit two's
    complement; field k of byte b = column 4 b + k).  Checked bit for bit against the oracle's
    own decode of a packed tile (oref_flat_tile_weights), every weight of the tile."""
    rng = np.random.default_rng(17 + bits)
    w = (rng.standard_normal(32768) * 0.02).astype(np.float32)
    cell = ca.pack_flat(w, bits=bits, n_outliers=0)
    got = orc.flat_tile_weights(cell)
    scale = cell[16448 + 48:16448 + 48 + 512].view(np.float16).astype(np.float32)
    o = np.arange(32768)
    if bits == 4:
        b = cell[64 + o // 2]
        code = (b >> (4 * (o & 1))) & 15
        val = code.astype(np.float32) - 8.0
    else:
        b = cell[64 + o // 4]
        code = (b >> (2 * (o & 3))) & 3
        val = (code ^ 2).astype(np.float32) - 2.0
    want = (val * scale[o // 128]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
