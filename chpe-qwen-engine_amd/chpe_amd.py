"""ctypes bindings of the MI355X decode engine (libchpe.so) and the archive writer
(libchpe_pack.so), both built in this directory by its Makefile.

The engine API mirrors the reference's C ABI (src/chpe_c_api.zig) plus the additions
declared in include/chpe.h.  Nothing here computes on the CPU: a missing or unloadable
libchpe.so raises, it is never replaced by a fallback.
"""
import ctypes
import os
import shutil
from pathlib import Path

import numpy as np

PKG_DIR = Path(__file__).resolve().parent
ENGINE_LIB = PKG_DIR / "libchpe.so"
PACK_LIB = PKG_DIR / "libchpe_pack.so"

ARCH_3B, ARCH_9B, ARCH_72B = 0, 1, 2
# archive kinds of chpe_pack_write (include/chpe_pack.h)
(PACK_3B_FP16_RAW, PACK_3B_BF16_RAW, PACK_3B_W4, PACK_3B_W2, PACK_3B_W4_STD, PACK_72B_W4, PACK_72B_W2,
 PACK_9B_W4) = range(8)

# every symbol include/chpe.h declares, in order
ENGINE_SYMBOLS = [
    "chpe_init", "chpe_forward_tokens", "chpe_get_last_logits", "chpe_get_vocab_size",
    "chpe_get_hidden_dim", "chpe_get_num_layers", "chpe_get_last_elapsed_ns",
    "chpe_get_last_argmax", "chpe_get_last_max_logit", "chpe_get_last_token0_logit",
    "chpe_get_last_hidden_norm", "chpe_free", "chpe_init_ex", "chpe_decode_step",
    "chpe_generate", "chpe_verify", "chpe_prefill", "chpe_block_ready", "chpe_last_error", "chpe_build_id", "chpe_get_max_seq_len", "chpe_get_hidden",
    "chpe_time_steps", "chpe_time_stage", "chpe_time_stage_live", "chpe_stage_bytes", "chpe_step_bytes", "chpe_stage_kernel",
    "chpe_debug_gemv", "chpe_debug_flat_tile_weights", "chpe_debug_gemv_flat", "chpe_debug_gemv_cells", "chpe_debug_gemv_poly", "chpe_debug_gemv_raw", "chpe_debug_embed_row_cell",
    "chpe_debug_attention", "chpe_debug_attention_block", "chpe_attention_noalloc", "chpe_debug_deltanet_conv", "chpe_debug_deltanet_step",
]

_c_float_p = ctypes.POINTER(ctypes.c_float)
_c_u32_p = ctypes.POINTER(ctypes.c_uint32)
_c_u8_p = ctypes.POINTER(ctypes.c_uint8)
_engine_lib = None
_pack_lib = None


def _fp(a):
    return a.ctypes.data_as(_c_float_p)


def source_hash():
    """The hash libchpe.so carries of the sources it was built from (chpe_build_id): the
    Makefile's LIBSRC list, in its order, through SHA-256, first 16 hex digits."""
    import hashlib
    src = PKG_DIR / "csrc"
    files = sorted(list(src.glob("*.hip")) + list(src.glob("*.hpp")), key=lambda p: f"csrc/{p.name}")
    files += [src / "engine.cpp", src / "c_api.cpp", PKG_DIR.parent / "include" / "chpe.h", PKG_DIR / "Makefile"]
    h = hashlib.sha256()
    for f in files:
        h.update(f.read_bytes())
    return h.hexdigest()[:16]


def load_engine_lib():
    """Load libchpe.so (raises OSError when it is not built, or was built from other sources
    than the ones beside it)."""
    global _engine_lib
    if _engine_lib is None:
        if not ENGINE_LIB.exists():
            raise OSError(f"{ENGINE_LIB} is not built (run `make -C {PKG_DIR}`)")
        lib = ctypes.CDLL(str(ENGINE_LIB))
        lib.chpe_build_id.restype = ctypes.c_char_p
        built, here = lib.chpe_build_id().decode(), source_hash()
        if built != here:
            raise OSError(f"{ENGINE_LIB} was built from other sources (build id {built}, sources {here}): "
                          f"run `make -C {PKG_DIR}`")
        V, S, I, U64, F, D = (ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64,
                              ctypes.c_float, ctypes.c_double)
        sig = {
            "chpe_init": (V, [ctypes.c_char_p]),
            "chpe_forward_tokens": (I, [V, _c_u32_p, S, _c_float_p]),
            "chpe_get_last_logits": (S, [V, _c_float_p, S]),
            "chpe_get_vocab_size": (S, [V]),
            "chpe_get_hidden_dim": (S, [V]),
            "chpe_get_num_layers": (S, [V]),
            "chpe_get_last_elapsed_ns": (U64, [V]),
            "chpe_get_last_argmax": (ctypes.c_uint32, [V]),
            "chpe_get_last_max_logit": (F, [V]),
            "chpe_get_last_token0_logit": (F, [V]),
            "chpe_get_last_hidden_norm": (F, [V]),
            "chpe_free": (None, [V]),
            "chpe_init_ex": (V, [ctypes.c_char_p, I, S, I]),
            "chpe_decode_step": (I, [V, ctypes.c_uint32, S, _c_float_p]),
            "chpe_generate": (I, [V, _c_u32_p, S, S, _c_u32_p]),
            "chpe_prefill": (I, [V, _c_u32_p, S, _c_float_p]),
            "chpe_block_ready": (I, [V]),
            "chpe_verify": (I, [V, _c_u32_p, S, S, _c_u32_p]),
            "chpe_last_error": (ctypes.c_char_p, []),
            "chpe_build_id": (ctypes.c_char_p, []),
            "chpe_get_max_seq_len": (S, [V]),
            "chpe_get_hidden": (I, [V, _c_float_p]),
            "chpe_time_steps": (I, [V, S, _c_float_p]),
            "chpe_time_stage": (I, [V, I, S, S, S, _c_float_p]),
            "chpe_time_stage_live": (I, [V, I, S, _c_float_p]),
            "chpe_stage_bytes": (D, [V, I, S]),
            "chpe_step_bytes": (D, [V, S]),
            "chpe_stage_kernel": (ctypes.c_char_p, [V, I]),
            "chpe_debug_gemv": (I, [V, S, I, _c_float_p, _c_float_p]),
            "chpe_debug_flat_tile_weights": (I, [_c_u8_p, _c_float_p]),
            "chpe_debug_gemv_flat": (I, [I, ctypes.c_uint32, ctypes.c_uint32, _c_u8_p, _c_u8_p, S, _c_float_p,
                                         _c_float_p, F, _c_float_p, _c_u32_p, _c_float_p]),
            "chpe_debug_gemv_cells": (I, [I, ctypes.c_uint32, _c_u8_p, _c_u8_p, S, _c_float_p, _c_float_p, F,
                                          _c_float_p, _c_u32_p, _c_float_p]),
            "chpe_debug_gemv_poly": (I, [I, ctypes.c_uint32, ctypes.c_uint32, _c_u8_p, _c_u8_p, S, _c_float_p,
                                         _c_float_p, F, _c_float_p, _c_u32_p, _c_float_p]),
            "chpe_debug_gemv_raw": (I, [I, ctypes.c_uint32, ctypes.c_uint32, I, _c_u8_p, _c_u8_p, S, _c_float_p,
                                        _c_float_p, F, _c_float_p, _c_u32_p, _c_float_p]),
            "chpe_debug_embed_row_cell": (I, [_c_u8_p, S, ctypes.c_uint32, ctypes.c_uint32, _c_float_p]),
            "chpe_debug_attention": (I, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, I, ctypes.c_uint32,
                                         _c_float_p, _c_float_p, _c_float_p, _c_float_p]),
            "chpe_debug_attention_block": (I, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, I, ctypes.c_uint32,
                                               ctypes.c_uint32, _c_float_p, _c_float_p, _c_float_p, _c_float_p]),
            "chpe_attention_noalloc": (I, [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, I, ctypes.c_uint32,
                                           ctypes.c_uint32, V, V, V, V, V]),
            "chpe_debug_deltanet_conv": (I, [ctypes.c_uint32, ctypes.c_uint32, _c_float_p, _c_float_p, _c_float_p,
                                             _c_float_p]),
            "chpe_debug_deltanet_step": (I, [ctypes.c_uint32] * 3 + [_c_float_p] * 9 + [F, _c_float_p, _c_float_p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _engine_lib = lib
    return _engine_lib


def load_pack_lib():
    global _pack_lib
    if _pack_lib is None:
        if not PACK_LIB.exists():
            raise OSError(f"{PACK_LIB} is not built (run `make -C {PKG_DIR}`)")
        lib = ctypes.CDLL(str(PACK_LIB))
        lib.chpe_pack_size.restype = ctypes.c_uint64
        lib.chpe_pack_size.argtypes = [ctypes.c_int]
        lib.chpe_pack_write.restype = ctypes.c_int
        lib.chpe_pack_write.argtypes = [ctypes.c_char_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_int]
        lib.chpe_pack_records.restype = ctypes.c_int
        lib.chpe_pack_records.argtypes = [ctypes.c_int, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                          ctypes.c_int, _c_u8_p]
        lib.chpe_pack_header.restype = ctypes.c_int
        lib.chpe_pack_header.argtypes = [ctypes.c_int, _c_u8_p]
        lib.chpe_pack_normals.restype = None
        lib.chpe_pack_normals.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                          ctypes.c_uint64, ctypes.c_float, _c_float_p]
        lib.chpe_pack_cell16.restype = ctypes.c_int
        lib.chpe_pack_cell16.argtypes = [_c_float_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                         ctypes.c_int, ctypes.c_uint32, _c_u8_p]
        lib.chpe_pack_flat.restype = ctypes.c_int
        lib.chpe_pack_flat.argtypes = [_c_float_p, ctypes.c_int, ctypes.c_int, ctypes.c_uint32, _c_u8_p]
        _pack_lib = lib
    return _pack_lib


# ------------------------------------------------------------------ archive writer
def archive_size(kind):
    return int(load_pack_lib().chpe_pack_size(kind))


def write_archive(path, kind, seed=0, threads=0):
    rc = load_pack_lib().chpe_pack_write(str(path).encode(), kind, seed, threads)
    if rc != 0:
        raise RuntimeError(f"chpe_pack_write({path}, kind={kind}) failed: {rc}")
    return path


def pack_records(kind, first, count, seed=0, threads=0):
    """Records [first, first + count) of archive `kind`, as they lie in the file, as a
    (count, record_bytes) uint8 array."""
    rb = 16384 if kind in (PACK_3B_FP16_RAW, PACK_3B_BF16_RAW) else (20480 if kind == PACK_3B_W4_STD else 17408)
    out = np.zeros((count, rb), dtype=np.uint8)
    if load_pack_lib().chpe_pack_records(kind, seed, first, count, threads, out.ctypes.data_as(_c_u8_p)) != 0:
        raise ValueError("chpe_pack_records rejected the arguments")
    return out


def pack_header(kind):
    out = np.zeros(4096, dtype=np.uint8)
    if load_pack_lib().chpe_pack_header(kind, out.ctypes.data_as(_c_u8_p)) != 0:
        raise ValueError("chpe_pack_header rejected the kind")
    return out


def normals(seed, tid, first, n, std=0.02):
    out = np.empty(n, dtype=np.float32)
    load_pack_lib().chpe_pack_normals(seed, tid, first, n, std, _fp(out))
    return out


def pack_cell16(w, bits=4, n_outlier_cols=8, layer=0):
    w = np.ascontiguousarray(w, dtype=np.float32)
    cell = np.zeros(17408, dtype=np.uint8)
    rc = load_pack_lib().chpe_pack_cell16(_fp(w), w.shape[0], w.shape[1], bits, n_outlier_cols,
                                          layer, cell.ctypes.data_as(_c_u8_p))
    if rc:
        raise ValueError("chpe_pack_cell16 rejected the shape")
    return cell


def pack_flat(w, bits=4, n_outliers=64, layer=0):
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(32768)
    cell = np.zeros(17408, dtype=np.uint8)
    rc = load_pack_lib().chpe_pack_flat(_fp(w), bits, n_outliers, layer, cell.ctypes.data_as(_c_u8_p))
    if rc:
        raise ValueError("chpe_pack_flat rejected the arguments")
    return cell


# ------------------------------------------------------------------ engine
class EngineError(RuntimeError):
    pass


class Engine:
    """One engine context (chpe_init / chpe_init_ex)."""

    def __init__(self, path, arch=-1, max_seq_len=2048, kv_f16=False, reference_init=False):
        self.lib = load_engine_lib()
        if reference_init:
            self.ctx = self.lib.chpe_init(str(path).encode())
        else:
            self.ctx = self.lib.chpe_init_ex(str(path).encode(), arch, max_seq_len, 1 if kv_f16 else 0)
        if not self.ctx:
            raise EngineError(self.lib.chpe_last_error().decode())
        self.vocab = self.lib.chpe_get_vocab_size(self.ctx)
        self.hidden_dim = self.lib.chpe_get_hidden_dim(self.ctx)
        self.num_layers = self.lib.chpe_get_num_layers(self.ctx)
        self.max_seq_len = self.lib.chpe_get_max_seq_len(self.ctx)

    def close(self):
        if self.ctx:
            self.lib.chpe_free(self.ctx)
            self.ctx = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc < 0:
            raise EngineError(f"{what} failed: {rc}")
        return rc

    def forward_tokens(self, tokens, want_logits=False):
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.vocab, dtype=np.float32) if want_logits else None
        rc = self.lib.chpe_forward_tokens(self.ctx, toks.ctypes.data_as(_c_u32_p), toks.size,
                                          _fp(logits) if want_logits else None)
        self._check(rc, "chpe_forward_tokens")
        return (rc, logits) if want_logits else rc

    def decode_step(self, token, pos, want_logits=True):
        logits = np.empty(self.vocab, dtype=np.float32) if want_logits else None
        rc = self.lib.chpe_decode_step(self.ctx, token, pos, _fp(logits) if want_logits else None)
        self._check(rc, "chpe_decode_step")
        return (rc, logits) if want_logits else rc

    def generate(self, prompt, n_gen):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        out = np.empty(n_gen, dtype=np.uint32)
        rc = self.lib.chpe_generate(self.ctx, p.ctypes.data_as(_c_u32_p), p.size, n_gen,
                                    out.ctypes.data_as(_c_u32_p))
        self._check(rc, "chpe_generate")
        return out

    def prefill(self, tokens, want_logits=False):
        toks = np.ascontiguousarray(tokens, dtype=np.uint32)
        logits = np.empty(self.vocab, dtype=np.float32) if want_logits else None
        rc = self.lib.chpe_prefill(self.ctx, toks.ctypes.data_as(_c_u32_p), toks.size,
                                   _fp(logits) if want_logits else None)
        self._check(rc, "chpe_prefill")
        return (rc, logits) if want_logits else rc

    def block_ready(self):
        return bool(self.lib.chpe_block_ready(self.ctx))

    def verify(self, drafts, pos):
        d = np.ascontiguousarray(drafts, dtype=np.uint32)
        out = np.empty(d.size, dtype=np.uint32)
        rc = self.lib.chpe_verify(self.ctx, d.ctypes.data_as(_c_u32_p), d.size, pos, out.ctypes.data_as(_c_u32_p))
        self._check(rc, "chpe_verify")
        return out

    def logits(self):
        out = np.empty(self.vocab, dtype=np.float32)
        if self.lib.chpe_get_last_logits(self.ctx, _fp(out), self.vocab) != self.vocab:
            raise EngineError("chpe_get_last_logits failed")
        return out

    def hidden(self):
        out = np.empty(self.hidden_dim, dtype=np.float32)
        self._check(self.lib.chpe_get_hidden(self.ctx, _fp(out)), "chpe_get_hidden")
        return out

    def last(self):
        L = self.lib
        return dict(argmax=L.chpe_get_last_argmax(self.ctx), max_logit=L.chpe_get_last_max_logit(self.ctx),
                    token0_logit=L.chpe_get_last_token0_logit(self.ctx),
                    hidden_norm=L.chpe_get_last_hidden_norm(self.ctx),
                    elapsed_ns=L.chpe_get_last_elapsed_ns(self.ctx))

    def debug_gemv(self, layer, which, x, rows):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y = np.empty(rows, dtype=np.float32)
        self._check(self.lib.chpe_debug_gemv(self.ctx, layer, which, _fp(x), _fp(y)), "chpe_debug_gemv")
        return y

    def time_steps(self, n):
        ms = ctypes.c_float()
        self._check(self.lib.chpe_time_steps(self.ctx, n, ctypes.byref(ms)), "chpe_time_steps")
        return ms.value

    def time_stage(self, stage, layer0, layer1, iters):
        ms = ctypes.c_float()
        self._check(self.lib.chpe_time_stage(self.ctx, stage, layer0, layer1, iters, ctypes.byref(ms)),
                    "chpe_time_stage")
        return ms.value

    def time_stage_live(self, stage, n_steps):
        ms = ctypes.c_float()
        self._check(self.lib.chpe_time_stage_live(self.ctx, stage, n_steps, ctypes.byref(ms)),
                    "chpe_time_stage_live")
        return ms.value

    def stage_bytes(self, stage, layer):
        return self.lib.chpe_stage_bytes(self.ctx, stage, layer)

    def step_bytes(self, pos):
        return self.lib.chpe_step_bytes(self.ctx, pos)

    def stage_kernel(self, stage):
        """The kernel that runs `stage`, demangled when c++filt is available."""
        name = self.lib.chpe_stage_kernel(self.ctx, stage).decode()
        try:
            import subprocess
            out = subprocess.run(["c++filt", name], capture_output=True, text=True, timeout=10)
            return out.stdout.strip() or name
        except (OSError, subprocess.SubprocessError):
            return name


def gpu_flat_tile_weights(cell):
    cell = np.ascontiguousarray(cell, dtype=np.uint8)
    out = np.empty(32768, dtype=np.float32)
    rc = load_engine_lib().chpe_debug_flat_tile_weights(cell.ctypes.data_as(_c_u8_p), _fp(out))
    if rc:
        raise EngineError(f"chpe_debug_flat_tile_weights failed: {rc}")
    return out


GEMV_MODES = {"store": 0, "accum": 1, "swiglu": 2, "logits": 3}


def gpu_gemv_flat(mode, rows, cols, tiles, x, tiles_up=None, gamma=None, eps=1e-6, y=None):
    """One flat-tile GEMV through the decode step's kernels (chpe_debug_gemv_flat).  `tiles`
    (and `tiles_up` for "swiglu") are consecutive 17408-byte cells; returns y, or for "logits"
    (y, argmax, hidden_norm)."""
    m = GEMV_MODES[mode]
    tiles = np.ascontiguousarray(tiles, dtype=np.uint8).reshape(-1)
    n_tiles = tiles.size // 17408
    up = None if tiles_up is None else np.ascontiguousarray(tiles_up, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
    out = np.zeros(rows, np.float32) if y is None else np.array(y, dtype=np.float32)
    am, hn = ctypes.c_uint32(0), ctypes.c_float(0.0)
    rc = load_engine_lib().chpe_debug_gemv_flat(
        m, rows, cols, tiles.ctypes.data_as(_c_u8_p), None if up is None else up.ctypes.data_as(_c_u8_p),
        n_tiles, _fp(x), None if g is None else _fp(g), eps, _fp(out), ctypes.byref(am), ctypes.byref(hn))
    if rc:
        raise EngineError(f"chpe_debug_gemv_flat failed: {rc} {load_engine_lib().chpe_last_error().decode()}")
    return (out, am.value, hn.value) if mode == "logits" else out


def gpu_gemv_cells(mode, rows, cells, x, cells_up=None, gamma=None, eps=1e-6, y=None):
    """One 16-row-cell GEMV at 2048 columns through the decode step's kernels
    (chpe_debug_gemv_cells); returns y, or for "logits" (y, argmax, hidden_norm)."""
    m = GEMV_MODES[mode]
    cells = np.ascontiguousarray(cells, dtype=np.uint8).reshape(-1)
    up = None if cells_up is None else np.ascontiguousarray(cells_up, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
    out = np.zeros(rows, np.float32) if y is None else np.array(y, dtype=np.float32)
    am, hn = ctypes.c_uint32(0), ctypes.c_float(0.0)
    rc = load_engine_lib().chpe_debug_gemv_cells(
        m, rows, cells.ctypes.data_as(_c_u8_p), None if up is None else up.ctypes.data_as(_c_u8_p),
        cells.size // 17408, _fp(x), None if g is None else _fp(g), eps, _fp(out), ctypes.byref(am), ctypes.byref(hn))
    if rc:
        raise EngineError(f"chpe_debug_gemv_cells failed: {rc} {load_engine_lib().chpe_last_error().decode()}")
    return (out, am.value, hn.value) if mode == "logits" else out


def gpu_gemv_poly(mode, rows, cols, cells, x, cells_up=None, gamma=None, eps=1e-6, y=None):
    """One GEMV over polymorphic 16-row cells of any width through the engine's polymorphic
    path (chpe_debug_gemv_poly); returns y, or for "logits" (y, argmax, hidden_norm)."""
    m = GEMV_MODES[mode]
    cells = np.ascontiguousarray(cells, dtype=np.uint8).reshape(-1)
    up = None if cells_up is None else np.ascontiguousarray(cells_up, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
    out = np.zeros(rows, np.float32) if y is None else np.array(y, dtype=np.float32)
    am, hn = ctypes.c_uint32(0), ctypes.c_float(0.0)
    rc = load_engine_lib().chpe_debug_gemv_poly(
        m, rows, cols, cells.ctypes.data_as(_c_u8_p), None if up is None else up.ctypes.data_as(_c_u8_p),
        cells.size // 17408, _fp(x), None if g is None else _fp(g), eps, _fp(out), ctypes.byref(am), ctypes.byref(hn))
    if rc:
        raise EngineError(f"chpe_debug_gemv_poly failed: {rc} {load_engine_lib().chpe_last_error().decode()}")
    return (out, am.value, hn.value) if mode == "logits" else out


RAW_KINDS = {"fp16": 0, "bf16": 1, "int8": 2}


def gpu_gemv_raw(mode, rows, cols, kind, tiles, x, tiles_up=None, gamma=None, eps=1e-6, y=None):
    """One GEMV over raw 16384-byte tiles (one row-major matrix) through the engine's raw
    kernels (chpe_debug_gemv_raw); returns y, or for "logits" (y, argmax, hidden_norm)."""
    m = GEMV_MODES[mode]
    t = np.ascontiguousarray(tiles, dtype=np.uint8).reshape(-1)
    up = None if tiles_up is None else np.ascontiguousarray(tiles_up, dtype=np.uint8).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = None if gamma is None else np.ascontiguousarray(gamma, dtype=np.float32)
    out = np.zeros(rows, np.float32) if y is None else np.array(y, dtype=np.float32)
    am, hn = ctypes.c_uint32(0), ctypes.c_float(0.0)
    rc = load_engine_lib().chpe_debug_gemv_raw(
        m, rows, cols, RAW_KINDS[kind], t.ctypes.data_as(_c_u8_p), None if up is None else up.ctypes.data_as(_c_u8_p),
        t.size // 16384, _fp(x), None if g is None else _fp(g), eps, _fp(out), ctypes.byref(am), ctypes.byref(hn))
    if rc:
        raise EngineError(f"chpe_debug_gemv_raw failed: {rc} {load_engine_lib().chpe_last_error().decode()}")
    return (out, am.value, hn.value) if mode == "logits" else out


def gpu_embed_row_cell(region, row, D, init=None):
    region = np.ascontiguousarray(region, dtype=np.uint8)
    out = np.array(init, dtype=np.float32) if init is not None else np.zeros(D, dtype=np.float32)
    rc = load_engine_lib().chpe_debug_embed_row_cell(region.ctypes.data_as(_c_u8_p), region.size, row, D, _fp(out))
    if rc < 0:
        raise EngineError(f"chpe_debug_embed_row_cell failed: {rc}")
    return rc, out


def gpu_attention(q, k_rows, v_rows, pos, heads, kv_heads, head_dim, kv_f16):
    """The decode step's attention kernels on caller rows (k_rows / v_rows: [pos+1][kv*hd] f32)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k_rows, dtype=np.float32)
    v = np.ascontiguousarray(v_rows, dtype=np.float32)
    if q.size != heads * head_dim or k.size != (pos + 1) * kv_heads * head_dim or v.size != k.size:
        raise ValueError("attention operand sizes do not match the shape")
    out = np.empty(heads * head_dim, dtype=np.float32)
    rc = load_engine_lib().chpe_debug_attention(head_dim, heads, kv_heads, int(kv_f16), pos, _fp(q), _fp(k),
                                                _fp(v), _fp(out))
    if rc:
        raise EngineError(f"chpe_debug_attention failed: {rc}")
    return out


def gpu_attention_block(q, k_rows, v_rows, pos, heads, kv_heads, head_dim, kv_f16):
    """The block step's attention kernels on caller rows: q [nq][heads*hd] at positions pos ..
    pos+nq-1, k_rows / v_rows [pos+nq][kv*hd] f32; returns [nq][heads*hd]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k_rows, dtype=np.float32)
    v = np.ascontiguousarray(v_rows, dtype=np.float32)
    nq = q.shape[0]
    if q.ndim != 2 or q.shape[1] != heads * head_dim or k.size != (pos + nq) * kv_heads * head_dim or v.size != k.size:
        raise ValueError("attention operand sizes do not match the shape")
    out = np.empty_like(q)
    rc = load_engine_lib().chpe_debug_attention_block(head_dim, heads, kv_heads, int(kv_f16), pos, nq, _fp(q),
                                                      _fp(k), _fp(v), _fp(out))
    if rc:
        raise EngineError(f"chpe_debug_attention_block failed: {rc}")
    return out


def _f32c(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def gpu_deltanet_conv(x, w, state):
    """k_dn_conv on caller data; returns (out, new_state)."""
    x, w, st = _f32c(x), _f32c(w), _f32c(state).copy()
    ch, taps = w.shape
    out = np.empty(ch, dtype=np.float32)
    rc = load_engine_lib().chpe_debug_deltanet_conv(ch, taps, _fp(x), _fp(w), _fp(st), _fp(out))
    if rc:
        raise EngineError(f"chpe_debug_deltanet_conv failed: {rc}")
    return out, st


def gpu_deltanet_step(q, k, v, a, b, A_log, dt_bias, state, z=None, norm_w=None, eps=1e-6):
    """k_dn_step on caller data; returns (out, new_state)."""
    q, k, v, a, b, A_log, dt_bias = (_f32c(t) for t in (q, k, v, a, b, A_log, dt_bias))
    st = _f32c(state).copy()
    nk, hd = q.shape
    nv = v.shape[0]
    out = np.empty((nv, hd), dtype=np.float32)
    zz = _f32c(z) if z is not None else None
    ww = _f32c(norm_w) if norm_w is not None else None
    rc = load_engine_lib().chpe_debug_deltanet_step(nv, nk, hd, _fp(q), _fp(k), _fp(v), _fp(a), _fp(b), _fp(A_log),
                                                    _fp(dt_bias), _fp(zz) if zz is not None else None,
                                                    _fp(ww) if ww is not None else None, eps, _fp(st), _fp(out))
    if rc:
        raise EngineError(f"chpe_debug_deltanet_step failed: {rc}")
    return out, st


def build(jobs=8):
    """Compile libchpe.so, libchpe_pack.so and the CLIs in place (make)."""
    import subprocess
    subprocess.run(["make", "-C", str(PKG_DIR), f"-j{jobs}"], check=True)


def default_archive_dir():
    d = Path(os.environ.get("CHPE_ARCHIVE_DIR", "/tmp/chpe_archives"))
    d.mkdir(parents=True, exist_ok=True)
    return d


ARCHIVE_NAMES = {
    PACK_3B_FP16_RAW: "qwen2.5-3b-fp16raw", PACK_3B_BF16_RAW: "qwen2.5-3b-bf16raw",
    PACK_3B_W4: "qwen2.5-3b-w4", PACK_3B_W2: "qwen2.5-3b-w2", PACK_3B_W4_STD: "qwen2.5-3b-w4std",
    PACK_72B_W4: "qwen2.5-72b-w4", PACK_72B_W2: "qwen2.5-72b-w2", PACK_9B_W4: "qwen3.5-9b-w4",
}


def _generator_tag():
    import hashlib
    h = hashlib.sha1()
    for f in ("csrc/pack.cpp", "csrc/format.hpp", "csrc/tensor_maps.hpp"):
        h.update((PKG_DIR / f).read_bytes())
    # letters only: chpe_init guesses the architecture from "9b" / "72b" in the path
    return "".join(chr(ord("a") + int(c, 16)) for c in h.hexdigest()[:10])


def ensure_archive(kind, seed=0, directory=None, threads=0):
    """Path of the seeded archive `kind` under `directory` (default $CHPE_ARCHIVE_DIR or
    /tmp/chpe_archives), written on first use and reused while the generator is unchanged."""
    d = Path(directory) if directory else default_archive_dir()
    path = d / f"{ARCHIVE_NAMES[kind]}-s{seed}-{_generator_tag()}.chpe"
    if not path.exists() or path.stat().st_size != archive_size(kind):
        tmp = path.with_suffix(".tmp")
        # the writer fills a memory-mapped file: on a file system without room for it the
        # process would die of SIGBUS mid-write, so the room is checked first
        d.mkdir(parents=True, exist_ok=True)
        tmp.unlink(missing_ok=True)  # (a write that did not finish)
        have = shutil.disk_usage(d).free
        if have < archive_size(kind):
            raise OSError(f"{d}: {have / 1e9:.1f} GB free, {ARCHIVE_NAMES[kind]} needs {archive_size(kind) / 1e9:.1f} GB "
                          "(remove older archives there or set CHPE_ARCHIVE_DIR)")
        write_archive(tmp, kind, seed, threads)
        os.replace(tmp, path)
    return path
