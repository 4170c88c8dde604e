"""Archive format: tensor maps, header validation, the seeded archive writer.

Golden data: tests/golden/tensor_maps.json (extracted from the reference's tensor-map sources
by tests/golden/make_tensor_maps.py) and the archive size in the reference's
models/manifest.json:8.
"""
import json
from pathlib import Path

import numpy as np
import pytest

import chpe_amd as ca
import oracle as orc
from conftest import archive_path

GOLDEN = json.loads((Path(__file__).parent / "golden" / "tensor_maps.json").read_text())
PAYLOAD = 64 + 16384


# ---------------------------------------------------------------- tensor maps
def test_3b_cell_map_matches_reference_table():
    g = GOLDEN["qwen3b_cell"]
    for l, ref in enumerate(g["layers"]):
        li = orc.layer_info(1, l)
        for k in ("input_norm", "q_proj", "k_proj", "v_proj", "o_proj", "post_norm", "gate_proj",
                  "up_proj", "down_proj", "q_bias", "k_bias", "v_bias"):
            assert li[k] == ref[k], (l, k)
        assert (li["q_tiles"], li["k_tiles"], li["v_tiles"], li["o_tiles"]) == (128, 16, 16, 128)
        assert (li["gate_tiles"], li["up_tiles"], li["down_tiles"]) == (688, 688, 688)
    assert orc.lib().oref_final_norm_for(1) == g["final_norm"] == 94348
    assert g["total"] == g["final_norm"] + 1


def test_3b_raw_map_matches_reference_offsets():
    g = GOLDEN["qwen3b_raw"]
    off = g["offsets"]
    names = {"inNorm": "input_norm", "qProj": "q_proj", "qBias": "q_bias", "kProj": "k_proj",
             "kBias": "k_bias", "vProj": "v_proj", "vBias": "v_bias", "oProj": "o_proj",
             "postNorm": "post_norm", "gateProj": "gate_proj", "upProj": "up_proj", "downProj": "down_proj"}
    for l in (0, 1, 17, 35):
        li = orc.layer_info(0, l)
        base = g["EMBED_TOKENS_RECORDS"] + l * g["RECORDS_PER_LAYER"]
        for zig, mine in names.items():
            assert li[mine] == base + off[zig], (l, zig)
        assert li["q_tiles"] == g["Q_PROJ_TILES"] and li["k_tiles"] == g["K_PROJ_TILES"]
        assert li["v_tiles"] == g["V_PROJ_TILES"] and li["o_tiles"] == g["O_PROJ_TILES"]
        assert li["gate_tiles"] == g["GATE_PROJ_TILES"] and li["down_tiles"] == g["DOWN_PROJ_TILES"]
    assert orc.lib().oref_final_norm_for(0) == g["FINAL_NORM_RECORD"]


def test_9b_map_with_gqa_aliasing():
    g = GOLDEN["qwen35_9b"]
    for l, ref in enumerate(g["layers"]):
        li = orc.layer_info(2, l)
        assert li["input_norm"] == ref["input_norm_tile"]
        assert li["post_norm"] == ref["post_norm_tile"]
        assert li["gate_proj"] == ref["gate_proj_tile"] and li["up_proj"] == ref["up_proj_tile"]
        assert li["down_proj"] == ref["down_proj_tile"]
        if ref["is_full_attn"]:
            assert (li["q_proj"], li["k_proj"], li["v_proj"], li["o_proj"]) == (
                ref["q_proj_tile"], ref["k_proj_tile"], ref["v_proj_tile"], ref["o_proj_tile"])
            assert (li["q_tiles"], li["k_tiles"], li["v_tiles"]) == (
                ref["q_proj_tiles"], ref["k_proj_tiles"], ref["v_proj_tiles"])
        else:  # chpe_engine.zig:1107-1131: q <- in_proj_qkv, k <- in_proj_z, v <- in_proj_a
            assert (li["q_proj"], li["k_proj"], li["v_proj"], li["o_proj"]) == (
                ref["in_proj_qkv_tile"], ref["in_proj_z_tile"], ref["in_proj_a_tile"], ref["out_proj_tile"])
    assert orc.lib().oref_final_norm_for(2) == g["final_norm"]


def test_72b_map_reference_asserts():
    # the values of qwen72b_tensor_map.zig:89-112 in the order that test asserts them
    a = GOLDEN["qwen72b"]["asserts"]
    per_layer, embed = a[0], a[1]
    l0, l1 = orc.layer_info(3, 0), orc.layer_info(3, 1)
    assert per_layer == 26789 and embed == 38016
    assert [l0["input_norm"], l0["q_proj"], l0["q_bias"], l0["k_proj"], l0["k_bias"], l0["v_proj"],
            l0["v_bias"], l0["o_proj"], l0["post_norm"], l0["gate_proj"], l0["up_proj"],
            l0["down_proj"], l1["input_norm"]] == a[2:15]
    assert orc.lib().oref_final_norm_for(3) == a[15]
    l79 = orc.layer_info(3, 79)
    assert l79["down_proj"] + l79["down_tiles"] == a[15]


# ---------------------------------------------------------------- header validation
def header(magic=0x57415243, version=1, header_bytes=4096, count=0, record=20480, cell=17408,
           prefetch=3072, flags=0):
    b = np.zeros(4096, np.uint8)
    for off, v, t in ((0, magic, np.uint32), (4, version, np.uint32), (8, header_bytes, np.uint64),
                      (16, count, np.uint64), (24, count, np.uint64), (32, record, np.uint64),
                      (40, cell, np.uint64), (48, prefetch, np.uint64), (56, flags, np.uint64)):
        raw = np.frombuffer(t(v).tobytes(), np.uint8)
        b[off:off + raw.size] = raw
    return b


def test_validate_reference_error_cases():
    # weight_archive.zig:1048-1078: too small, bad magic, bad geometry, truncated
    assert orc.validate(np.zeros(100, np.uint8)) == 1
    assert orc.validate(header(magic=0xDEADBEEF)) == 2
    assert orc.validate(header(record=20480 + 64)) == 5
    assert orc.validate(header(count=1)) == 6
    assert orc.validate(header()) == 0
    assert orc.validate(header(version=2)) == 3
    assert orc.validate(header(magic=0x45504843, record=17408, prefetch=0)) == 0  # dense CHPE
    assert orc.validate(header(record=16384, cell=16384, prefetch=0)) == 0        # raw
    assert orc.validate(header(record=16384, cell=17408, prefetch=0)) == 5


# ---------------------------------------------------------------- archive writer
def test_archive_sizes():
    # models/manifest.json:8: the raw 3B archive is 6,174,363,648 bytes = 4096 + 376853 * 16384
    assert ca.archive_size(ca.PACK_3B_FP16_RAW) == 6174363648
    assert ca.archive_size(ca.PACK_3B_W4) == 4096 + 94349 * 17408
    assert ca.archive_size(ca.PACK_3B_W4_STD) == 4096 + 94349 * 20480
    assert ca.archive_size(ca.PACK_72B_W4) == 4096 + 2219153 * 17408


def test_generator_is_deterministic_and_normal():
    a = ca.normals(0, 1001, 0, 200000)
    assert np.array_equal(a, ca.normals(0, 1001, 0, 200000))
    assert np.array_equal(a[12345:12400], ca.normals(0, 1001, 12345, 55))  # random access
    assert not np.array_equal(a, ca.normals(1, 1001, 0, 200000))
    assert not np.array_equal(a, ca.normals(0, 1002, 0, 200000))
    assert abs(a.mean()) < 2e-4 and abs(a.std() - 0.02) < 2e-4


def test_cell16_quantizer_error_bound():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((16, 2048)) * 0.02).astype(np.float16).astype(np.float32)
    w[3, 77] = 0.5  # an outlier column
    cell = ca.pack_cell16(w, bits=4)
    x = np.eye(2048, dtype=np.float32)
    wq = np.stack([orc.gemv_tile(cell, x[c], 16) for c in range(0, 2048, 97)], axis=1)
    cols = np.arange(0, 2048, 97)
    amax = np.abs(w.reshape(16, 16, 128)).max(axis=2)                      # per (row, group)
    bound = 0.51 * (amax / 7.0)[:, cols // 128] * (1 + 2.0 ** -10)
    assert (np.abs(wq - w[:, cols]) <= bound).all()
    assert orc.gemv_tile(cell, x[77], 16)[3] == np.float32(0.5)  # outliers are exact


def test_flat_quantizer_error_bound_and_outliers():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal(32768) * 0.02).astype(np.float16).astype(np.float32)
    for bits, qmax in ((4, 7.0), (2, 2.0)):
        cell = ca.pack_flat(w, bits=bits)
        wq = orc.flat_tile_weights(cell)
        top = np.argsort(-np.abs(w), kind="stable")[:64]
        assert np.array_equal(wq[top], w[top])  # the 64 largest |w| are stored exactly
        amax = np.abs(w.reshape(256, 128)).max(axis=1)
        tol = (1.01 if bits == 2 else 0.51) * np.repeat(amax / qmax, 128) * (1 + 2.0 ** -10)
        assert (np.abs(wq - w) <= tol).all()


def test_w4_archive_layout(w4_archive):
    """Every tensor of the 3B cell archive sits at the record the reference's map names."""
    m = np.memmap(w4_archive, dtype=np.uint8, mode="r")
    assert orc.validate(m[:4096 + 17408]) in (0, 6)
    stride = 17408

    def rec(i):
        return m[4096 + i * stride: 4096 + (i + 1) * stride]

    g = GOLDEN["qwen3b_cell"]
    for l in (0, 5, 35):
        ref = g["layers"][l]
        for k in ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj"):
            c = rec(ref[k])
            assert c[PAYLOAD + 20] == 4
            assert np.frombuffer(c[PAYLOAD + 40:PAYLOAD + 48].tobytes(), np.uint32).tolist() == [16, 2048]
            assert np.frombuffer(c[PAYLOAD:PAYLOAD + 4].tobytes(), np.uint32)[0] == l
        c = rec(ref["down_proj"])
        assert c[PAYLOAD + 20] == 4 and np.frombuffer(c[PAYLOAD + 560:PAYLOAD + 562].tobytes(), np.uint16)[0] == 64
        for k in ("input_norm", "post_norm"):
            gains = np.frombuffer(rec(ref[k])[64:64 + 8192].tobytes(), np.float32)
            assert (gains == 1.0).all()
    gains = np.frombuffer(rec(g["final_norm"])[64:64 + 8192].tobytes(), np.float32)
    assert (gains == 1.0).all()
