"""ctypes wrapper of the CPU oracle (oracle/liboracle.so).  TEST INFRASTRUCTURE.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg: it is the
checker and the timed CPU baseline, never part of the engine.
"""
import ctypes
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB = ORACLE_DIR / "liboracle.so"
_lib = None
_fp = ctypes.POINTER(ctypes.c_float)
_u8p = ctypes.POINTER(ctypes.c_uint8)
_u32p = ctypes.POINTER(ctypes.c_uint32)


class Result(ctypes.Structure):
    _fields_ = [("argmax_token", ctypes.c_uint32), ("max_logit", ctypes.c_float),
                ("token0_logit", ctypes.c_float), ("elapsed_ns", ctypes.c_uint64),
                ("hidden_norm", ctypes.c_float), ("all_finite", ctypes.c_int)]


class LayerInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in (
        "input_norm", "q_proj", "q_tiles", "k_proj", "k_tiles", "v_proj", "v_tiles", "o_proj",
        "o_tiles", "post_norm", "gate_proj", "gate_tiles", "up_proj", "up_tiles", "down_proj",
        "down_tiles")] + [("q_bias", ctypes.c_int64), ("k_bias", ctypes.c_int64), ("v_bias", ctypes.c_int64)]


def build():
    subprocess.run(["make", "-C", str(ORACLE_DIR)], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        V, S = ctypes.c_void_p, ctypes.c_size_t
        L.oref_open.restype = V
        L.oref_open.argtypes = [ctypes.c_char_p, ctypes.c_int, S, ctypes.c_int, ctypes.c_int,
                                ctypes.POINTER(ctypes.c_int)]
        L.oref_open_bytes.restype = V
        L.oref_open_bytes.argtypes = [_u8p, S, ctypes.c_int, S, ctypes.c_int, ctypes.c_int]
        L.oref_close.argtypes = [V]
        L.oref_forward.restype = ctypes.c_int
        L.oref_forward.argtypes = [V, ctypes.c_uint32, S, ctypes.POINTER(Result)]
        L.oref_forward_layers.restype = ctypes.c_int
        L.oref_forward_layers.argtypes = [V, ctypes.c_uint32, S, S, ctypes.POINTER(Result)]
        L.oref_set_threads.argtypes = [V, ctypes.c_int]
        L.oref_set_break.argtypes = [V, ctypes.c_int]
        L.oref_set_hybrid.restype = ctypes.c_int
        L.oref_set_hybrid.argtypes = [V, ctypes.c_int]
        L.oref_logits.restype = _fp
        L.oref_logits.argtypes = [V]
        L.oref_hidden.restype = _fp
        L.oref_hidden.argtypes = [V]
        L.oref_vocab.restype = S
        L.oref_vocab.argtypes = [V]
        L.oref_hidden_dim.restype = S
        L.oref_hidden_dim.argtypes = [V]
        L.oref_engine_info.argtypes = [V, ctypes.POINTER(ctypes.c_int64)]
        L.oref_gemv_linear.argtypes = [V, S, S, _fp, S, _fp, S, S, S, ctypes.c_int, ctypes.c_int64]
        L.oref_unpack_norm.argtypes = [V, S, _fp, S]
        L.oref_unpack_bias.argtypes = [V, S, _fp, S]
        L.oref_unpack_embed_row.argtypes = [V, ctypes.c_uint32, _fp]
        L.oref_compute_lm_head.argtypes = [V, _fp, _fp]
        L.oref_prefill_synthetic.restype = ctypes.c_int
        L.oref_prefill_synthetic.argtypes = [V, S, ctypes.c_uint64]
        L.oref_generate.restype = ctypes.c_int
        L.oref_generate.argtypes = [V, _u32p, S, S, _u32p, _fp]
        L.oref_validate.restype = ctypes.c_int
        L.oref_validate.argtypes = [_u8p, S]
        L.oref_silu.restype = ctypes.c_float
        L.oref_silu.argtypes = [ctypes.c_float]
        L.oref_rmsnorm.argtypes = [_fp, _fp, _fp, S, ctypes.c_float]
        L.oref_apply_rope.argtypes = [_fp, S, S, S, ctypes.c_float]
        L.oref_f16_to_f32.restype = ctypes.c_float
        L.oref_f16_to_f32.argtypes = [ctypes.c_uint16]
        _u16p = ctypes.POINTER(ctypes.c_uint16)
        L.oref_f32_to_f16_n.argtypes = [_fp, _u16p, S]
        L.oref_f16_to_f32_n.argtypes = [_u16p, _fp, S]
        L.oref_gemv_tile_polymorphic.argtypes = [_u8p, _fp, S, _fp, S, S, ctypes.c_int]
        L.oref_flat_tile_weights.argtypes = [_u8p, S, _fp]
        L.oref_gemv_cell_flat.argtypes = [_u8p, S, S, S, S, _fp, _fp]
        L.oref_unpack_embed_row_cell.restype = ctypes.c_int
        L.oref_unpack_embed_row_cell.argtypes = [_u8p, S, _fp, S]
        L.oref_attention.argtypes = [_fp, _fp, _fp, S, S, S, S, _fp, _fp]
        L.oref_conv1d_update.argtypes = [S, S, _fp, _fp, _fp, _fp]
        L.oref_gated_delta_step.argtypes = [S, S, S, S, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp, _fp]
        L.oref_gated_rmsnorm.argtypes = [S, S, _fp, _fp, _fp, ctypes.c_float, _fp]
        L.oref_layer_info_for.restype = ctypes.c_int
        L.oref_layer_info_for.argtypes = [ctypes.c_int, S, ctypes.POINTER(LayerInfo)]
        L.oref_final_norm_for.restype = S
        L.oref_final_norm_for.argtypes = [ctypes.c_int]
        L.oref_arch_from_path.restype = ctypes.c_int
        L.oref_arch_from_path.argtypes = [ctypes.c_char_p]
        _lib = L
    return _lib


def f(a):
    return np.ascontiguousarray(a, dtype=np.float32).ctypes.data_as(_fp)


def u8(a):
    return a.ctypes.data_as(_u8p)


class Oracle:
    """CHPEEngine restated on the CPU (oref_open)."""

    def __init__(self, path=None, arch=-1, max_seq_len=2048, kv_f16=False, threads=0, data=None):
        self.L = lib()
        self._keep = None
        if data is not None:
            self._keep = np.ascontiguousarray(data, dtype=np.uint8)
            self.e = self.L.oref_open_bytes(u8(self._keep), self._keep.size, arch, max_seq_len,
                                            1 if kv_f16 else 0, threads)
        else:
            err = ctypes.c_int()
            self.e = self.L.oref_open(str(path).encode(), arch, max_seq_len, 1 if kv_f16 else 0,
                                      threads, ctypes.byref(err))
            self.open_error = err.value
        if not self.e:
            raise RuntimeError("oracle open failed")
        self.vocab = self.L.oref_vocab(self.e)
        self.hidden_dim = self.L.oref_hidden_dim(self.e)

    def close(self):
        if self.e:
            self.L.oref_close(self.e)
            self.e = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward(self, token, pos):
        r = Result()
        rc = self.L.oref_forward(self.e, token, pos, ctypes.byref(r))
        if rc:
            raise RuntimeError(f"oref_forward rc={rc}")
        return r

    def forward_layers(self, token, pos, n_layers):
        """The decode step over the first n_layers layers only (a timing sample)."""
        r = Result()
        rc = self.L.oref_forward_layers(self.e, token, pos, n_layers, ctypes.byref(r))
        if rc:
            raise RuntimeError(f"oref_forward_layers rc={rc}")
        return r

    def set_threads(self, n):
        self.L.oref_set_threads(self.e, n)

    def set_hybrid(self, on=True):
        """The true Qwen3.5-9B hybrid layers (DeltaNet + gated attention) on a 9B archive."""
        if self.L.oref_set_hybrid(self.e, 1 if on else 0):
            raise RuntimeError("oref_set_hybrid: not a 9B cell archive")

    def set_break(self, on):
        """Test only: set_break(False) removes forwardDecode's non-finite break (:1763), a
        planted deviation that shows a comparison can tell the break from its absence."""
        self.L.oref_set_break(self.e, 1 if on else 0)

    def prefill_synthetic(self, n_pos, seed=0):
        if self.L.oref_prefill_synthetic(self.e, n_pos, seed):
            raise RuntimeError("oref_prefill_synthetic: n_pos > max_seq_len")

    def logits(self):
        return np.ctypeslib.as_array(self.L.oref_logits(self.e), shape=(self.vocab,)).copy()

    def hidden(self):
        return np.ctypeslib.as_array(self.L.oref_hidden(self.e), shape=(self.hidden_dim,)).copy()

    def info(self):
        out = (ctypes.c_int64 * 8)()
        self.L.oref_engine_info(self.e, out)
        keys = ("is_raw", "is_raw_fp16", "is_dense", "quant_bits", "wpt", "record_count", "valid", "map")
        return dict(zip(keys, list(out)))

    def gemv_linear(self, tile_start, num_tiles, x, r_total, c_total, y_len=None, accumulate=False,
                    bias_tile=-1, y=None):
        x = np.ascontiguousarray(x, dtype=np.float32)
        y_len = y_len or r_total
        y = np.zeros(y_len, dtype=np.float32) if y is None else np.ascontiguousarray(y, dtype=np.float32)
        self.L.oref_gemv_linear(self.e, tile_start, num_tiles, x.ctypes.data_as(_fp), x.size,
                                y.ctypes.data_as(_fp), y_len, r_total, c_total, 1 if accumulate else 0,
                                bias_tile)
        return y

    def unpack_norm(self, tile, n):
        out = np.empty(n, dtype=np.float32)
        self.L.oref_unpack_norm(self.e, tile, out.ctypes.data_as(_fp), n)
        return out

    def embed_row(self, token):
        out = np.zeros(self.hidden_dim, dtype=np.float32)
        self.L.oref_unpack_embed_row(self.e, token, out.ctypes.data_as(_fp))
        return out

    def lm_head(self, xn):
        """computeLmHead on a normed hidden state: the vocab_size logits."""
        x = np.ascontiguousarray(xn, dtype=np.float32)
        out = np.empty(self.L.oref_vocab(self.e), dtype=np.float32)
        self.L.oref_compute_lm_head(self.e, x.ctypes.data_as(_fp), out.ctypes.data_as(_fp))
        return out

    def generate(self, prompt, n_gen):
        p = np.ascontiguousarray(prompt, dtype=np.uint32)
        toks = np.empty(n_gen, dtype=np.uint32)
        gaps = np.empty(n_gen, dtype=np.float32)
        rc = self.L.oref_generate(self.e, p.ctypes.data_as(_u32p), p.size, n_gen,
                                  toks.ctypes.data_as(_u32p), gaps.ctypes.data_as(_fp))
        if rc:
            raise RuntimeError(f"oref_generate rc={rc}")
        return toks, gaps


def layer_info(map_id, layer):
    li = LayerInfo()
    lib().oref_layer_info_for(map_id, layer, ctypes.byref(li))
    return {k: getattr(li, k) for k, _ in LayerInfo._fields_}


def gemv_tile(cell, x, y_len, row_base=0, accumulate=False, y=None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(y_len, dtype=np.float32) if y is None else np.ascontiguousarray(y, dtype=np.float32)
    lib().oref_gemv_tile_polymorphic(u8(cell), x.ctypes.data_as(_fp), x.size, y.ctypes.data_as(_fp),
                                     y.size, row_base, 1 if accumulate else 0)
    return y


def flat_tile_weights(cell, wpt=32768):
    out = np.empty(32768, dtype=np.float32)
    lib().oref_flat_tile_weights(u8(cell), wpt, out.ctypes.data_as(_fp))
    return out


def gemv_cell_flat(cell, t, r_total, c_total, x, y, wpt=32768):
    x = np.ascontiguousarray(x, dtype=np.float32)
    lib().oref_gemv_cell_flat(u8(cell), t, wpt, r_total, c_total, x.ctypes.data_as(_fp), y.ctypes.data_as(_fp))
    return y


def embed_row_cell(region, row, D, init=None):
    out = np.array(init, dtype=np.float32) if init is not None else np.zeros(D, dtype=np.float32)
    w = lib().oref_unpack_embed_row_cell(u8(region), row, out.ctypes.data_as(_fp), D)
    return w, out


def rmsnorm(x, g, eps=1e-6):
    x = np.ascontiguousarray(x, dtype=np.float32)
    g = np.ascontiguousarray(g, dtype=np.float32)
    y = np.empty_like(x)
    lib().oref_rmsnorm(x.ctypes.data_as(_fp), g.ctypes.data_as(_fp), y.ctypes.data_as(_fp), x.size, eps)
    return y


def rope(vec, pos, num_heads, head_dim, theta=1000000.0):
    v = np.array(vec, dtype=np.float32)
    lib().oref_apply_rope(v.ctypes.data_as(_fp), pos, num_heads, head_dim, theta)
    return v


def silu(z):
    return lib().oref_silu(z)


def attention(q, k_cache, v_cache, pos, heads, kv_heads, head_dim):
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(k_cache, dtype=np.float32)
    vc = np.ascontiguousarray(v_cache, dtype=np.float32)
    scores = np.empty(heads * (pos + 1), dtype=np.float32)
    out = np.empty(heads * head_dim, dtype=np.float32)
    lib().oref_attention(q.ctypes.data_as(_fp), kc.ctypes.data_as(_fp), vc.ctypes.data_as(_fp), pos,
                         heads, kv_heads, head_dim, scores.ctypes.data_as(_fp), out.ctypes.data_as(_fp))
    return out


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def conv1d_update(x, w, state):
    """One causal depthwise conv step + SiLU; returns (out, new_state)."""
    x, w, st = _f32(x), _f32(w), _f32(state).copy()
    ch, taps = w.shape
    out = np.empty(ch, dtype=np.float32)
    lib().oref_conv1d_update(ch, taps, x.ctypes.data_as(_fp), w.ctypes.data_as(_fp), st.ctypes.data_as(_fp),
                             out.ctypes.data_as(_fp))
    return out, st


def gated_delta_step(q, k, v, a, b, A_log, dt_bias, state):
    """One gated-delta-rule step over all value heads; returns (out, new_state)."""
    q, k, v, a, b, A_log, dt_bias = (_f32(t) for t in (q, k, v, a, b, A_log, dt_bias))
    st = _f32(state).copy()
    nk, dk = q.shape
    nv, dv = v.shape
    out = np.empty((nv, dv), dtype=np.float32)
    lib().oref_gated_delta_step(nv, nk, dk, dv, *(t.ctypes.data_as(_fp) for t in (q, k, v, a, b, A_log, dt_bias)),
                                st.ctypes.data_as(_fp), out.ctypes.data_as(_fp))
    return out, st


def gated_rmsnorm(x, z, w, eps):
    x, z, w = _f32(x), _f32(z), _f32(w)
    n, dv = x.shape
    out = np.empty_like(x)
    lib().oref_gated_rmsnorm(n, dv, x.ctypes.data_as(_fp), z.ctypes.data_as(_fp), w.ctypes.data_as(_fp), eps,
                             out.ctypes.data_as(_fp))
    return out


def validate(data):
    d = np.ascontiguousarray(data, dtype=np.uint8)
    return lib().oref_validate(u8(d), d.size)


def f16_to_f32(h):
    return lib().oref_f16_to_f32(h)


def f16_to_f32_array(h):
    """The oracle's f16 -> f32 widening of every element of a uint16 array."""
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.size, dtype=np.float32)
    lib().oref_f16_to_f32_n(h.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), out.ctypes.data_as(_fp), h.size)
    return out


def f32_to_f16_array(x):
    """The oracle's f32 -> f16 rounding (its fp16 KV cache) of every element, as uint16 codes."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.uint16)
    lib().oref_f32_to_f16_n(x.ctypes.data_as(_fp), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), x.size)
    return out
