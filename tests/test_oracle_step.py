"""The oracle on a whole seeded Qwen2.5-3B 4-bit cell archive.

The quantized archive is the quantization of known fp16 weights (the generator in
include/chpe_pack.h), so every dequantising path of the oracle (16-row cells with added
outliers, flat tiles with replaced outliers, the embedding row, the tied LM head) is pinned
against those weights in float64 by the quantizer's error bound: |w - w_q| <= s/2 per weight,
s = group absmax / 7 (outliers exact).  A transposed operand, a wrong nibble order, a wrong
group-scale index or a wrong outlier rule breaks the bound by orders of magnitude.
"""
import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc

SEED = 0
D, I, V = 2048, 11008, 151936
TID_EMBED = 1


def tid(layer, which):  # generator tensor ids: q 1, k 2, v 3, o 4, gate 5, up 6, down 7
    return 1000 * (layer + 1) + which


def fp16_weights(t, first, n):
    return ca.normals(SEED, t, first, n).astype(np.float16).astype(np.float64)


def quant_bound(w, x):
    """Per-row bound of |W_q x - W x| for 4-bit GROUP128 rows (w: [R][C], groups along C)."""
    R, C = w.shape
    s = np.abs(w.reshape(R, C // 128, 128)).max(axis=2) / 7.0 * 0.51 * (1 + 2.0 ** -10)
    return (s * np.abs(x.astype(np.float64)).reshape(C // 128, 128).sum(axis=1)).sum(axis=1)


@pytest.fixture(scope="module")
def oracle(w4_archive):
    return orc.Oracle(w4_archive, arch=0, max_seq_len=64, threads=8)


@pytest.mark.parametrize("layer,which,name,rows,cols", [
    (0, 1, "q", 2048, 2048), (21, 2, "k", 256, 2048), (35, 3, "v", 256, 2048), (3, 4, "o", 2048, 2048),
    (21, 5, "gate", 11008, 2048), (9, 6, "up", 11008, 2048), (21, 7, "down", 2048, 11008),
    (0, 7, "down", 2048, 11008)])
def test_projection_within_quantization_bound(oracle, layer, which, name, rows, cols):
    li = orc.layer_info(1, layer)
    start, tiles = li[f"{name}_proj"], li[f"{name}_tiles"]
    x = np.random.default_rng(layer * 10 + which).standard_normal(cols).astype(np.float32)
    y = oracle.gemv_linear(start, tiles, x, rows, cols).astype(np.float64)
    w = fp16_weights(tid(layer, which), 0, rows * cols).reshape(rows, cols)
    err = np.abs(y - w @ x.astype(np.float64))
    bound = quant_bound(w, x) + 1e-5 * (np.abs(w) @ np.abs(x.astype(np.float64)))
    assert (err <= bound).all(), (name, float((err / bound).max()))
    assert np.median(err) > 0  # the weights really are quantized


def test_bias_tile_is_added(oracle):
    li = orc.layer_info(1, 4)
    x = np.random.default_rng(5).standard_normal(D).astype(np.float32)
    y0 = oracle.gemv_linear(li["k_proj"], 16, x, 256, D)
    y1 = oracle.gemv_linear(li["k_proj"], 16, x, 256, D, bias_tile=li["k_bias"])
    bias = ca.normals(SEED, tid(4, 12), 0, 256)  # q/k/v biases are f32 generator values
    assert np.array_equal(y1, y0 + bias)


def test_embedding_row_within_quantization_bound(oracle):
    for tok in (0, 17, 151935):
        row = oracle.embed_row(tok).astype(np.float64)
        w = fp16_weights(TID_EMBED, tok * D, D)
        s = np.repeat(np.abs(w.reshape(16, 128)).max(axis=1) / 7.0, 128)
        assert (np.abs(row - w) <= 0.51 * s * (1 + 2.0 ** -10)).all()
        # outlier columns are replaced by the exact fp16 weight, so some entries are exact
        assert (row == w).sum() >= 8


def test_step_logits_are_tied_lm_head_of_final_norm(oracle):
    r = oracle.forward(151643, 0)
    h = oracle.hidden().astype(np.float64)
    hn = h / np.sqrt(np.mean(h * h) + 1e-6)  # final RMSNorm, gains 1.0
    logits = oracle.logits()
    assert r.hidden_norm == pytest.approx(float(np.linalg.norm(h)), rel=1e-5)
    assert r.argmax_token == int(np.argmax(logits)) and r.max_logit == logits.max()
    assert r.token0_logit == logits[0] and r.all_finite
    rows = np.r_[0:64, 70000:70016, V - 64:V]
    w = np.stack([fp16_weights(TID_EMBED, int(t) * D, D) for t in rows])
    err = np.abs(logits[rows] - w @ hn)
    assert (err <= quant_bound(w, hn) + 1e-4).all()


def test_threads_do_not_change_results(w4_archive):
    a = orc.Oracle(w4_archive, arch=0, max_seq_len=8, threads=1)
    b = orc.Oracle(w4_archive, arch=0, max_seq_len=8, threads=8)
    for pos, tok in enumerate((9, 151935)):
        ra, rb = a.forward(tok, pos), b.forward(tok, pos)
        assert np.array_equal(a.logits(), b.logits())
        assert ra.argmax_token == rb.argmax_token


def test_kv_f16_and_position_limit(w4_archive):
    a = orc.Oracle(w4_archive, arch=0, max_seq_len=3, kv_f16=False, threads=8)
    b = orc.Oracle(w4_archive, arch=0, max_seq_len=3, kv_f16=True, threads=8)
    for pos, tok in enumerate((5, 6, 7)):
        a.forward(tok, pos), b.forward(tok, pos)
        la, lb = a.logits(), b.logits()
        cos = float(la.astype(np.float64) @ lb / np.linalg.norm(la) / np.linalg.norm(lb))
        assert cos > 0.9999
    with pytest.raises(RuntimeError):
        a.forward(8, 3)  # pos >= max_seq_len
