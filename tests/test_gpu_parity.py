"""The HIP engine against the oracle, through the C ABI (libchpe.so).

Bars:
  * integer work (dequantisation / unpacking of weight tiles and embedding rows): bit-exact.
    For the production GEMV kernels this is observed with one-hot inputs: y = W e_c is the
    dequantised column c itself (every lane sum has one non-zero term, and the archive writer
    stores outlier codes as the zero code), so kernel and oracle must agree bit for bit;
  * floating point: a projection |y_gpu - y_oracle| <= 1e-5 * (|y| + rms(y)) + 1e-6 per output;
    a step's logits max-abs <= 2e-3 and cosine >= 0.9999;
  * greedy token streams: identical.
"""
import os
import sys

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

pytestmark = pytest.mark.gpu

D, I, V = 2048, 11008, 151936
PROJ = {0: ("q", 2048, D), 1: ("k", 256, D), 2: ("v", 256, D), 3: ("o", D, D), 4: ("gate", I, D),
        5: ("up", I, D), 6: ("down", D, I)}


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def w4(w4_archive):
    say(f"engine+oracle on {w4_archive.name}")
    e = ca.Engine(w4_archive, arch=0, max_seq_len=128, kv_f16=False)
    o = orc.Oracle(w4_archive, arch=0, max_seq_len=128, threads=16)
    yield e, o
    e.close()
    o.close()


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ---------------------------------------------------------------- integer work: bit-exact
@pytest.mark.parametrize("bits_,n_out", [(4, 64), (4, 0), (2, 64), (2, 17)])
def test_flat_tile_dequant_bit_exact(bits_, n_out):
    rng = np.random.default_rng(bits_ * 100 + n_out)
    w = (rng.standard_normal(32768) * 0.02).astype(np.float32)
    cell = ca.pack_flat(w, bits=bits_, n_outliers=n_out)
    say(f"flat tile dequant bits={bits_} outliers={n_out}")
    assert np.array_equal(bits(ca.gpu_flat_tile_weights(cell)), bits(orc.flat_tile_weights(cell)))


def test_flat_tile_dequant_edge_cases():
    rng = np.random.default_rng(7)
    cell = ca.pack_flat((rng.standard_normal(32768) * 0.02).astype(np.float32), bits=4, n_outliers=64)
    P = 64 + 16384
    cases = []
    c1 = cell.copy()  # duplicate offsets: the later entry wins
    c1[P + 690:P + 694] = np.frombuffer(np.array([100, 100], np.uint16).tobytes(), np.uint8)
    cases.append(c1)
    c2 = cell.copy()  # n > 64: no outlier is applied
    c2[P + 560:P + 562] = np.frombuffer(np.uint16(65).tobytes(), np.uint8)
    cases.append(c2)
    c3 = cell.copy()  # no GROUP128: q * scale + bias with the tile's scale and bias
    c3[P + 24] = 0
    c3[P + 32:P + 40] = np.frombuffer(np.array([0.01, -0.003], np.float32).tobytes(), np.uint8)
    cases.append(c3)
    c4 = cell.copy()  # an unsupported width: all zero
    c4[P + 20] = 3
    cases.append(c4)
    for i, c in enumerate(cases):
        say(f"flat tile edge case {i}")
        assert np.array_equal(bits(ca.gpu_flat_tile_weights(c)), bits(orc.flat_tile_weights(c))), i


@pytest.mark.parametrize("D_", [2048, 4096, 8192])
def test_embed_row_unpack_bit_exact(w4_archive, D_):
    m = np.memmap(w4_archive, dtype=np.uint8, mode="r")
    start = 4096 + 17408 * 100
    region = np.array(m[start:start + 17408 * 8])  # wide rows read past their cell
    for row in (0, 5, 15, 16):
        say(f"embed row cell D={D_} row={row}")
        init = np.full(D_, 7.0, np.float32)
        rg, g = ca.gpu_embed_row_cell(region, row, D_, init)
        ro, o = orc.embed_row_cell(region, row, D_, init)
        assert rg == ro
        assert np.array_equal(bits(g), bits(o))
    # outlier entries 1 and 5 on one column (the later one wins), entry 3 past the row
    cols = region[16448 + 816:16448 + 832].view(np.uint16)
    cols[1] = cols[5] = 10
    cols[3] = 65535
    for row in (0, 9):
        say(f"embed row cell D={D_} row={row} (repeated / out-of-range outlier columns)")
        init = np.full(D_, 7.0, np.float32)
        rg, g = ca.gpu_embed_row_cell(region, row, D_, init)
        ro, o = orc.embed_row_cell(region, row, D_, init)
        assert rg == ro
        assert np.array_equal(bits(g), bits(o))


@pytest.mark.parametrize("layer", [0, 21, 35])
def test_production_gemv_columns_bit_exact(w4, layer):
    e, o = w4
    li = orc.layer_info(1, layer)
    rng = np.random.default_rng(layer)
    for which, (name, rows, cols) in PROJ.items():
        for c in rng.choice(cols, 6, replace=False):
            x = np.zeros(cols, np.float32)
            x[c] = 1.0
            say(f"one-hot column layer={layer} {name} col={c}")
            yg = e.debug_gemv(layer, which, x, rows)
            bias = li.get(f"{name}_bias", -1)
            yo = o.gemv_linear(li[f"{name}_proj"], li[f"{name}_tiles"], x, rows, cols, bias_tile=bias)
            assert np.array_equal(bits(yg), bits(yo)), (name, c)


def test_lm_head_columns_bit_exact(w4):
    """Tied LM head (computeLmHead's cell path): column c of the logits matrix is the
    embedding's column c with outliers replaced, i.e. unpackEmbedRowCell of every token."""
    e, o = w4
    toks = np.r_[0:40, 151900:151936, 75000:75016]
    rows = np.stack([o.embed_row(int(t)) for t in toks])
    for c in (0, 1, 777, 2047):
        x = np.zeros(D, np.float32)
        x[c] = 1.0
        say(f"one-hot LM head col={c}")
        y = e.debug_gemv(0, 7, x, V)
        assert np.array_equal(bits(y[toks]), bits(rows[:, c]))


# ---------------------------------------------------------------- floating point
@pytest.mark.parametrize("layer", [0, 21, 35])
def test_projection_parity(w4, layer):
    e, o = w4
    li = orc.layer_info(1, layer)
    rng = np.random.default_rng(100 + layer)
    for which, (name, rows, cols) in PROJ.items():
        x = rng.standard_normal(cols).astype(np.float32)
        say(f"projection layer={layer} {name}")
        yg = e.debug_gemv(layer, which, x, rows).astype(np.float64)
        yo = o.gemv_linear(li[f"{name}_proj"], li[f"{name}_tiles"], x, rows, cols,
                           bias_tile=li.get(f"{name}_bias", -1)).astype(np.float64)
        # f32 sums of `cols` terms in different orders: a relative bound on the output's scale
        tol = 1e-5 * (np.abs(yo) + np.sqrt(np.mean(yo * yo))) + 1e-6
        assert (np.abs(yg - yo) <= tol).all(), (name, float(np.abs(yg - yo).max()))


# (head_dim, query heads, kv heads): the 3B, 9B and 72B attention shapes
ATTN_SHAPES = [(128, 16, 2), (256, 16, 4), (128, 64, 8)]


@pytest.mark.parametrize("kv_f16", [1, 0])
@pytest.mark.parametrize("hd,H,KV", ATTN_SHAPES)
def test_attention_kernels_match_oracle(hd, H, KV, kv_f16):
    """The chunk + merge kernels against the oracle's attention (chpe_engine.zig:1700-1734) on
    the same rows (fp16-rounded for the fp16 cache): first position, partial and full 16-row
    tiles, chunk boundaries and a long context.  Tolerance: 2e-5 * max|v| (the matrix-core
    path keeps ~22 bits of the f32 queries and weights; sums run in another order)."""
    rng = np.random.default_rng(hd * 1000 + H + kv_f16)
    chunk = 16384 // hd
    # the contexts the configs decode at: 3B 4096 + 256 and 72B 8192 + 128 (head dim 128),
    # 9B 2048 + 256 (head dim 256)
    far = (8191, 8192, 8320) if hd == 128 else (2304, 2312)
    for pos in (0, 1, 3, 15, 16, 17, chunk - 1, chunk, chunk + 1, 3 * chunk + 5, 1000, 4351) + far:
        say(f"attention hd={hd} H={H} KV={KV} kv_f16={kv_f16} pos={pos}")
        q = (rng.standard_normal(H * hd) * 2.0).astype(np.float32)
        k = rng.standard_normal((pos + 1, KV * hd)).astype(np.float32)
        v = rng.standard_normal((pos + 1, KV * hd)).astype(np.float32)
        kr, vr = (k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)) \
            if kv_f16 else (k, v)
        ref = orc.attention(q, kr, vr, pos, H, KV, hd)
        got = ca.gpu_attention(q, k, v, pos, H, KV, hd, kv_f16)
        err = float(np.max(np.abs(got - ref)))
        assert err <= 2e-5 * float(np.max(np.abs(vr))), (pos, err)


@pytest.mark.parametrize("kv_f16", [1, 0])
@pytest.mark.parametrize("hd,H,KV", ATTN_SHAPES)
def test_block_attention_matches_oracle(hd, H, KV, kv_f16):
    """The block step's attention (nq queries at consecutive positions, query z over the rows up
    to its own position; the fp16 cache with more than 4 queries runs the multi-query launch,
    8 queries per workgroup over one load of its K / V rows) against the oracle's attention of
    each query alone, at the bar of the single-query test: block starts at 0, inside a chunk,
    a block crossing a chunk boundary (queries whose first chunks differ), a ragged last
    workgroup (11, 13 queries) and a long context."""
    rng = np.random.default_rng(hd * 7 + H + kv_f16)
    chunk = 16384 // hd
    for pos, nq in ((0, 32), (5, 11), (chunk - 6, 13), (chunk - 1, 8), (3 * chunk + 2, 32), (4000, 6), (8160, 32)):
        say(f"block attention hd={hd} H={H} KV={KV} kv_f16={kv_f16} pos={pos} nq={nq}")
        q = (rng.standard_normal((nq, H * hd)) * 2.0).astype(np.float32)
        k = rng.standard_normal((pos + nq, KV * hd)).astype(np.float32)
        v = rng.standard_normal((pos + nq, KV * hd)).astype(np.float32)
        kr, vr = (k.astype(np.float16).astype(np.float32), v.astype(np.float16).astype(np.float32)) \
            if kv_f16 else (k, v)
        got = ca.gpu_attention_block(q, k, v, pos, H, KV, hd, kv_f16)
        for z in range(nq):
            ref = orc.attention(q[z], kr[:pos + z + 1], vr[:pos + z + 1], pos + z, H, KV, hd)
            err = float(np.max(np.abs(got[z] - ref)))
            assert err <= 2e-5 * float(np.max(np.abs(vr[:pos + z + 1]))), (pos, nq, z, err)


def compare_step(e_logits, o_logits, tag):
    d = np.abs(e_logits.astype(np.float64) - o_logits)
    cos = float(e_logits.astype(np.float64) @ o_logits / np.linalg.norm(e_logits) / np.linalg.norm(o_logits))
    assert d.max() <= 2e-3 and cos >= 0.9999, (tag, float(d.max()), cos)


def test_decode_steps_match_oracle(w4):
    e, o = w4
    toks = [151643, 9707, 11, 1879, 0, 151935, 42, 42]
    for pos, tok in enumerate(toks):
        say(f"decode step pos={pos} tok={tok}")
        am, lg = e.decode_step(tok, pos)
        r = o.forward(tok, pos)
        ol = o.logits()
        compare_step(lg, ol, pos)
        assert am == r.argmax_token
        last = e.last()
        assert last["hidden_norm"] == pytest.approx(r.hidden_norm, rel=1e-5)
        assert last["max_logit"] == pytest.approx(r.max_logit, abs=2e-3)
        assert last["token0_logit"] == pytest.approx(r.token0_logit, abs=2e-3)
        assert np.abs(e.hidden() - o.hidden()).max() <= 1e-3 * max(1.0, np.abs(o.hidden()).max())


def check_stream(gpu, ref, gaps, tag):
    """Identical greedy streams; a difference is allowed only after a step whose top-2 logit
    gap in the oracle is below the float tolerance (a tie in the reference's own precision)."""
    for i, (a, b) in enumerate(zip(gpu, ref)):
        if a != b:
            assert gaps[i] < 1e-3, (tag, i, int(a), int(b), float(gaps[i]))
            return i
    return len(ref)


def test_token_stream_w4(w4):
    e, o = w4
    prompt = np.random.default_rng(1).integers(0, V, 64).astype(np.uint32)
    say("token stream 3B W4: 64 prompt + 32 generated")
    g = e.generate(prompt, 32)
    r, gaps = o.generate(prompt, 32)
    assert check_stream(g, r, gaps, "w4") == 32


@pytest.fixture(scope="module")
def w4_replay(w4_archive):
    """An engine without the block step (CHPE_BLOCK=0, read at init): verify and prefill replay
    the decode step."""
    os.environ["CHPE_BLOCK"] = "0"
    try:
        e = ca.Engine(w4_archive, arch=0, max_seq_len=128, kv_f16=False)
    finally:
        del os.environ["CHPE_BLOCK"]
    yield e
    e.close()


@pytest.mark.parametrize("m", [1, 4, 8])
def test_verify_equals_sequential_steps(w4_replay, w4, m):
    """chpe_verify (batch-M verify, no reference code) is defined as m sequential
    forwardDecode(draft_i, pos + i); without the block step it replays them: same argmaxes and,
    for the last draft, the same logits bit for bit; for m = 4 the argmaxes also match the
    oracle's sequential steps.  (The block step: test_cell_block_step_matches_decode_steps.)"""
    e, o = w4_replay, w4[1]
    assert not e.block_ready()
    rng = np.random.default_rng(100 + m)
    prompt = rng.integers(0, V, 6).astype(np.uint32)
    drafts = rng.integers(0, V, m).astype(np.uint32)
    p = int(prompt.size)
    say(f"verify m={m} at pos {p}")
    e.forward_tokens(prompt)
    got = e.verify(drafts, p)
    last = e.logits()
    e.forward_tokens(prompt)
    seq = [e.decode_step(int(d), p + i) for i, d in enumerate(drafts)]
    assert [int(x) for x in got] == [am for am, _ in seq]
    assert np.array_equal(bits(last), bits(seq[-1][1]))
    if m == 4:
        for pos, tok in enumerate(prompt):
            o.forward(int(tok), pos)
        for i, d in enumerate(drafts):
            r = o.forward(int(d), p + i)
            compare_step(seq[i][1], o.logits(), f"verify {i}")
            assert int(got[i]) == r.argmax_token


@pytest.mark.timeout(900)
def test_cell_block_step_matches_decode_steps(w4_archive):
    """The block step on 16-row 4-bit cells (the 3B archive: q/k/v/o/gate/up and the tied LM
    head read as 2048-column flat tiles, their outliers as per-row corrections -- added, or the
    LM head's replace deltas -- and the flat down projection): prefill and verify-8 against the
    decode steps on the same engine, verify-4 and the prefill against the oracle, with the f32
    and fp16 caches (run_block's bars)."""
    from test_gpu_models import run_block
    run_block(w4_archive, 0, V, seed=7, oracle_check=True)


def test_c_abi_semantics(w4_archive):
    """chpe_forward_tokens restarts at position 0 (chpe_c_api.zig:61-63); chpe_init fixes
    max_seq_len 2048 and guesses the 3B architecture from a path without "9B"/"72B"."""
    say("C ABI semantics")
    e = ca.Engine(w4_archive, reference_init=True)
    try:
        assert (e.vocab, e.hidden_dim, e.num_layers, e.max_seq_len) == (V, D, 36, 2048)
        toks = np.array([5, 6, 7], np.uint32)
        a1, l1 = e.forward_tokens(toks, want_logits=True)
        a2, l2 = e.forward_tokens(toks, want_logits=True)
        assert a1 == a2 and np.array_equal(l1, l2)
        assert np.array_equal(e.logits(), l2)
        assert e.last()["argmax"] == a2 and e.last()["elapsed_ns"] > 0
    finally:
        e.close()
    e = ca.Engine(w4_archive, arch=0, max_seq_len=4)
    try:
        with pytest.raises(ca.EngineError):
            e.forward_tokens(np.arange(5, dtype=np.uint32))
        with pytest.raises(ca.EngineError):
            e.decode_step(1, 4)
        e.forward_tokens(np.arange(4, dtype=np.uint32))
    finally:
        e.close()


def test_stage_kernel_lookup_launches_nothing(w4_archive):
    """chpe_stage_kernel names each stage's kernel without launching it: decode steps with the
    lookups between them give the logits of the same steps without, bit for bit."""
    toks = [151643, 9707, 11]
    runs = []
    for lookups in (False, True):
        e = ca.Engine(w4_archive, arch=0, max_seq_len=16)
        try:
            out = []
            for pos, t in enumerate(toks):
                if lookups:
                    names = [e.stage_kernel(st) for st in range(7)]
                    assert all(names), names
                out.append(e.decode_step(t, pos)[1])
            runs.append(np.stack(out))
        finally:
            e.close()
    assert np.array_equal(runs[0].view(np.uint32), runs[1].view(np.uint32))


def test_kv_f16_matches_oracle_kv_f16(w4_archive):
    """fp16 KV cache against the oracle's fp16-cache mode.  Every k / v element is rounded to
    fp16, and an element whose f32 value differs from the oracle's in the last bits (another
    summation order) can round to the neighbouring fp16 value: a 2^-11 relative step that the
    following layers carry to the logits.  With the f32 cache the same steps agree to ~2e-5
    (test_decode_steps_match_oracle); with the fp16 cache the rounding flips leave ~1-3e-3 on
    logits of magnitude ~4 (measured at these positions: 1.3e-3 for the vector-ALU cell kernel,
    2.5e-3 for the matrix-core one).  Bounds: max 5e-3, rms 1e-3, cos 0.9999, same argmax."""
    e = ca.Engine(w4_archive, arch=0, max_seq_len=16, kv_f16=True)
    o = orc.Oracle(w4_archive, arch=0, max_seq_len=16, kv_f16=True, threads=16)
    try:
        for pos, tok in enumerate([3, 1000, 20000, 151000, 8]):
            say(f"kv f16 pos={pos}")
            am, lg = e.decode_step(tok, pos)
            r = o.forward(tok, pos)
            ol = o.logits()
            d = np.abs(lg.astype(np.float64) - ol)
            cos = float(lg.astype(np.float64) @ ol / np.linalg.norm(lg) / np.linalg.norm(ol))
            assert d.max() <= 5e-3 and np.sqrt(np.mean(d * d)) <= 1e-3 and cos >= 0.9999, (pos, float(d.max()), cos)
            assert am == r.argmax_token
    finally:
        e.close()
        o.close()


def test_token_stream_w4_kv_f16(w4_archive):
    """C1's own configuration: the 4-bit cell archive with the fp16 KV cache, a greedy stream
    against the oracle's kv-f16 mode (256-token prompt + 32 generated).  The fp16 cache's
    rounding flips leave ~1-3e-3 on the logits (test_kv_f16_matches_oracle_kv_f16), so the
    streams may part only after a step whose top-2 gap in the oracle is below 5e-3."""
    e = ca.Engine(w4_archive, arch=0, max_seq_len=320, kv_f16=True)
    o = orc.Oracle(w4_archive, arch=0, max_seq_len=320, kv_f16=True, threads=16)
    try:
        prompt = np.random.default_rng(11).integers(0, V, 256).astype(np.uint32)
        say("token stream 3B W4, fp16 KV: 256 prompt + 32 generated")
        g = e.generate(prompt, 32)
        r, gaps = o.generate(prompt, 32)
        for i, (a, b) in enumerate(zip(g, r)):
            if a != b:
                assert gaps[i] < 5e-3, (i, int(a), int(b), float(gaps[i]))
                break
        else:
            i = 32
        say(f"  identical for {i} of 32 tokens")
    finally:
        e.close()
        o.close()


def test_token_stream_fp16_raw(fp16_archive):
    """The reference's CPU configuration: 3B FP16 raw tiles, 32-token prompt + 64 greedy."""
    say("token stream 3B FP16 raw: 32 prompt + 64 generated")
    e = ca.Engine(fp16_archive, arch=0, max_seq_len=128)
    o = orc.Oracle(fp16_archive, arch=0, max_seq_len=128, threads=16)
    try:
        prompt = np.random.default_rng(0).integers(0, V, 32).astype(np.uint32)
        g = e.generate(prompt, 64)
        r, gaps = o.generate(prompt, 64)
        assert check_stream(g, r, gaps, "fp16") == 64
        am, lg = e.decode_step(int(prompt[0]), 0)
        o.forward(int(prompt[0]), 0)
        compare_step(lg, o.logits(), "fp16 pos 0")
    finally:
        e.close()
        o.close()


def test_token_stream_bf16_raw(bf16_archive):
    """3B bf16 raw tiles (dotSegment's bf16 branch :1238-1251, the bf16 embedding rows and tied
    LM head :1626-1641): 16-token prompt + 32 greedy against the oracle."""
    say("token stream 3B BF16 raw: 16 prompt + 32 generated")
    e = ca.Engine(bf16_archive, arch=0, max_seq_len=64)
    o = orc.Oracle(bf16_archive, arch=0, max_seq_len=64, threads=16)
    try:
        prompt = np.random.default_rng(3).integers(0, V, 16).astype(np.uint32)
        g = e.generate(prompt, 32)
        r, gaps = o.generate(prompt, 32)
        assert check_stream(g, r, gaps, "bf16") == 32
        am, lg = e.decode_step(int(prompt[0]), 0)
        o.forward(int(prompt[0]), 0)
        compare_step(lg, o.logits(), "bf16 pos 0")
    finally:
        e.close()
        o.close()
