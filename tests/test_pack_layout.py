"""The seeded archive writer's layout where the reference reads past a record (CPU only).

The reference reads a 1-D tensor as `len` floats from its record's code area
(unpackNorm / unpackBias, src/chpe_engine.zig:1144-1192) and an embedding row of a cell
archive as row `token % 16` of cell `token / 16` with a row stride of D * bits / 8
(:1540-1546, :1288-1394), with no bound at the record.  These tests read the writer's records
exactly that way, with numpy, and check that every value those reads reach is the tensor's
own: gains of 1.0, the generator's biases, finite embedding rows whose values decode from the
bytes the reference decodes.  Records are produced with chpe_pack_records, so no archive file
is written.
"""
import numpy as np
import pytest

import chpe_amd as ca

CELL, CODES, PAYLOAD = 17408, 64, 16448


def floats_from_code_area(records, rel, n):
    """n f32 from the code area of record `rel` of a contiguous record block, running on
    into the following records as the reference's read does."""
    flat = records.reshape(-1)
    off = rel * CELL + CODES
    assert off + 4 * n <= flat.size
    return flat[off:off + 4 * n].view(np.float32)


def unpack_norm(vals):
    """unpackNorm's rules (:1161-1169): any non-finite value -> all 1.0; all zero -> 1.0."""
    if not np.all(np.isfinite(vals)) or not np.any(vals):
        return np.ones_like(vals)
    return vals


def tid(layer, which):
    return 1000 * (layer + 1) + which


@pytest.mark.parametrize("kind", [ca.PACK_72B_W4, ca.PACK_72B_W2])
def test_72b_long_vectors_read_back(kind):
    base = 38016  # layer 0: input_norm, q_proj (2048), q_bias, k_proj (256), k_bias, v_proj, ...
    recs = ca.pack_records(kind, base, 2052)
    assert np.all(unpack_norm(floats_from_code_area(recs, 0, 8192)) == 1.0)  # input_norm, 8192 wide
    assert np.isnan(floats_from_code_area(recs, 0, 8192)[4096])         # (through the NaN rule)
    qb = floats_from_code_area(recs, 2049, 8192)                        # q_proj bias, 8192 wide
    assert np.array_equal(qb, ca.normals(0, tid(0, 11), 0, 8192))
    # the tile the bias runs into keeps valid metadata and, for 4-bit, its outliers lie after
    # the bytes the vector owns; the tile after the norm keeps all of its own codes
    n_q = int(recs[1, PAYLOAD + 560:PAYLOAD + 562].view(np.uint16)[0])
    assert n_q == 64 and np.any(recs[1, PAYLOAD + 690:PAYLOAD + 818].view(np.uint16) < 2 * 15360)
    for rel in (2050,):
        pl = recs[rel, PAYLOAD:]
        assert pl[20] == (4 if kind == ca.PACK_72B_W4 else 2) and pl[24] & 1
        n = int(pl[560:562].view(np.uint16)[0])
        offs = pl[690:690 + 2 * n].view(np.uint16)
        if kind == ca.PACK_72B_W4:
            assert n == 64 and np.all(offs >= 2 * 15360) and np.all(np.diff(offs.astype(int)) > 0)
        else:
            assert n == 0  # every 2-bit code of the tile is a vector byte
    k = ca.pack_records(kind, base + 2306, 1)                           # k_bias, 1024 wide: fits
    assert np.array_equal(floats_from_code_area(k, 0, 1024), ca.normals(0, tid(0, 12), 0, 1024))
    post = ca.pack_records(kind, base + 4612, 2)                        # post_attention_layernorm
    assert np.all(unpack_norm(floats_from_code_area(post, 0, 8192)) == 1.0)
    fin = ca.pack_records(kind, 2181136, 2)                             # final norm -> lm_head tile 0
    assert np.all(unpack_norm(floats_from_code_area(fin, 0, 8192)) == 1.0)


def embed_row_dims(records, token, D):
    """unpackEmbedRowCell's per-tile-scale branch (:1384-1394) on a record block starting at
    record 0: (nibble - 8) * scale + bias over D / 2 bytes from row token % 16."""
    flat = records.reshape(-1)
    c, r = token // 16, token % 16
    pl = c * CELL + PAYLOAD
    meta_bits, flags = flat[pl + 20], flat[pl + 24]
    assert meta_bits not in (2, 4, 8) and flags & 1 == 0   # the branch the writer chose
    scale = flat[pl + 32:pl + 36].view(np.float32)[0]
    bias = flat[pl + 36:pl + 40].view(np.float32)[0]
    b = flat[c * CELL + CODES + r * (D // 2): c * CELL + CODES + (r + 1) * (D // 2)]
    q = np.stack([b & 15, b >> 4], 1).reshape(-1).astype(np.float32)
    return ((q - np.float32(8.0)) * scale + bias).astype(np.float32), scale


@pytest.mark.parametrize("kind,D", [(ca.PACK_72B_W4, 8192), (ca.PACK_9B_W4, 4096)])
def test_wide_embedding_rows_are_finite_codes(kind, D):
    recs = ca.pack_records(kind, 0, 40)
    norms = []
    for token in range(0, 16 * 36, 5):
        row, scale = embed_row_dims(recs, token, D)
        assert np.all(np.isfinite(row))
        assert 0.0 < scale < 0.02  # absmax / 7 of N(0, 0.02) weights
        norms.append(float(np.linalg.norm(row)))
    # N(0, 0.02) weights give |row| ~ 0.02 sqrt(D); rows read past the cell decode the codes of
    # the header / payload / next records, quantized the same way
    assert 0.5 * 0.02 * np.sqrt(D) < min(norms) and max(norms) < 2.0 * 0.02 * np.sqrt(D)
    # rows inside the cell are rows of the flat embedding matrix: token 16c + r reads matrix row
    # (32768 / D) c + r for r < 32768 / D
    per = 32768 // D
    w = ca.normals(0, 1, 0, D * per)  # tile 0 of the embedding (tensor id 1)
    row, scale = embed_row_dims(recs, 1, D)
    fp16w = w[D:2 * D].astype(np.float16).astype(np.float32)
    assert np.abs(row - fp16w).max() <= scale / 2 * 1.0001


def test_9b_layout():
    assert ca.archive_size(ca.PACK_9B_W4) == 4096 + 546681 * CELL
    hdr = ca.pack_header(ca.PACK_9B_W4)
    assert hdr[:4].view(np.uint32)[0] == 0x45504843 and hdr[16:24].view(np.uint64)[0] == 546681
    # layer 0 (linear attention): in_proj_a is 32 x 4096 -> 4 flat tiles of its 8-record span
    a0 = 62080 + 3073
    recs = ca.pack_records(ca.PACK_9B_W4, a0, 24)
    for i in range(4):
        assert recs[i, PAYLOAD + 20] == 4 and recs[i, PAYLOAD + 24] & 1
    assert not recs[4:8].any()                       # the rest of the span
    conv = recs[16:20, CODES:CODES + 16384].reshape(-1).view(np.uint16)  # conv1d bf16 [8192][4]
    want = ca.normals(0, tid(0, 25), 0, 32768)
    got = (conv.astype(np.uint32) << 16).view(np.float32)
    assert np.abs(got - want).max() <= np.abs(want).max() * 2.0 ** -8
    # full-attention layer 3: q_proj (query + gate rows, 8192 x 4096) fills 1024 of 2048 records
    r3 = 62080 + 3 * 13337
    q = ca.pack_records(ca.PACK_9B_W4, r3 + 1 + 1023, 2)
    assert q[0, PAYLOAD + 20] == 4 and not q[1].any()


def test_archive_needs_room(tmp_path, monkeypatch):
    # the writer fills a memory-mapped file: without room it would die of SIGBUS mid-write, so
    # ensure_archive checks the free space first and writes nothing
    class Usage:
        free = ca.archive_size(ca.PACK_72B_W4) - 1

    monkeypatch.setattr(ca.shutil, "disk_usage", lambda d: Usage)
    (tmp_path / "stale.tmp").write_bytes(b"x")
    with pytest.raises(OSError, match="GB free"):
        ca.ensure_archive(ca.PACK_72B_W4, 0, directory=tmp_path)
    assert [p.name for p in tmp_path.iterdir()] == ["stale.tmp"]
