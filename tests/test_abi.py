"""The C ABI without a GPU: both libraries load, export exactly what include/*.h declares, and
the reference's sentinel behaviour on NULL / invalid input (src/chpe_c_api.zig:25-143) holds.
Nothing here reaches the HIP runtime's device code."""
import ctypes
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest

import chpe_amd as ca

ROOT = Path(__file__).resolve().parents[1]


def declared(header):
    text = re.sub(r"/\*.*?\*/", "", (ROOT / "include" / header).read_text(), flags=re.S)
    return set(re.findall(r"\b(chpe_\w+)\s*\(", text))


def exported(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True,
                         check=True).stdout
    return {ln.split()[-1] for ln in out.splitlines() if re.search(r" T chpe_\w+$", ln)}


@pytest.mark.parametrize("header,lib", [("chpe.h", ca.ENGINE_LIB), ("chpe_pack.h", ca.PACK_LIB)])
def test_exports_match_header(header, lib):
    decl = declared(header)
    assert decl, header
    assert exported(lib) == decl
    handle = ctypes.CDLL(str(lib))
    for name in decl:
        assert getattr(handle, name)


def test_python_binding_covers_header():
    assert set(ca.ENGINE_SYMBOLS) == declared("chpe.h")
    ca.load_engine_lib()


def test_null_context_sentinels():
    L = ca.load_engine_lib()
    # chpe_c_api.zig:89-105: NULL -> the 3B defaults; :107-135: NULL -> 0
    assert L.chpe_get_vocab_size(None) == 151936
    assert L.chpe_get_hidden_dim(None) == 2048
    assert L.chpe_get_num_layers(None) == 36
    assert L.chpe_get_last_elapsed_ns(None) == 0
    assert L.chpe_get_last_argmax(None) == 0
    assert L.chpe_get_last_max_logit(None) == 0.0
    assert L.chpe_get_last_token0_logit(None) == 0.0
    assert L.chpe_get_last_hidden_norm(None) == 0.0
    toks = np.array([1, 2], np.uint32)
    assert L.chpe_forward_tokens(None, toks.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), 2, None) == -1
    out = np.zeros(4, np.float32)
    assert L.chpe_get_last_logits(None, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), 4) == 0
    L.chpe_free(None)  # no-op


def test_init_rejects_missing_and_malformed_archives(tmp_path):
    L = ca.load_engine_lib()
    assert not L.chpe_init(str(tmp_path / "absent.chpe").encode())
    assert b"cannot open" in L.chpe_last_error()
    small = tmp_path / "small.chpe"
    small.write_bytes(b"\0" * 100)
    assert not L.chpe_init(str(small).encode())
    assert L.chpe_last_error() == b"FileTooSmall"
    bad = tmp_path / "bad.chpe"
    bad.write_bytes(np.frombuffer(np.uint32(0xDEADBEEF).tobytes(), np.uint8).tobytes() + b"\0" * 4092)
    assert not L.chpe_init(str(bad).encode())
    assert L.chpe_last_error() == b"InvalidMagic"
    trunc = bytearray(4096)
    for off, v, n in ((0, 0x45504843, 4), (4, 1, 4), (8, 4096, 8), (16, 5, 8), (32, 17408, 8), (40, 17408, 8)):
        trunc[off:off + n] = int(v).to_bytes(n, "little")
    (tmp_path / "trunc.chpe").write_bytes(bytes(trunc))
    assert not L.chpe_init(str(tmp_path / "trunc.chpe").encode())
    assert L.chpe_last_error() == b"Truncated"
    assert not L.chpe_init_ex(str(small).encode(), 7, 16, 0)
    assert L.chpe_last_error() == b"unknown architecture"


def test_flat_gemv_hook_rejects_bad_arguments_before_the_device():
    """chpe_debug_gemv_flat checks its arguments on the host first.  (Tiles of any form, a mix of
    forms, fewer tiles than the shape needs and widths that are not a multiple of 128 are legal:
    the engine runs them tile by tile, tests/test_gpu_flat_poly.py.)"""
    w = (np.random.default_rng(1).standard_normal(32768) * 0.02).astype(np.float32)
    cells = np.stack([ca.pack_flat(w, bits=4), ca.pack_flat(w, bits=4)])
    x, g = np.ones(4096, np.float32), np.ones(4096, np.float32)
    bad = [
        dict(mode="swiglu", rows=16, cols=4096, tiles=cells, x=x, gamma=g),       # no up tiles
        dict(mode="store", rows=16, cols=4096, tiles=cells, x=x, gamma=g),        # gamma outside 2/3
        dict(mode="logits", rows=16, cols=4096, tiles=cells, x=x),                # no gamma
        dict(mode="store", rows=16, cols=2048, tiles=cells, x=x),                 # not a flat width
        dict(mode="store", rows=0, cols=4096, tiles=cells, x=x),                  # no rows
        dict(mode="store", rows=16, cols=4096, tiles=cells[:0], x=x),             # no tiles
    ]
    for kw in bad:
        with pytest.raises(ca.EngineError):
            ca.gpu_gemv_flat(**kw)
