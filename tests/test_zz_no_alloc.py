"""chpe_attention_noalloc (the decode attention on caller device buffers with no allocation)
against chpe_debug_attention (the same chunk + merge kernels behind an entry point that
allocates): bit-identical outputs on two calls in a row, the second with a shorter context,
and a size past the scratch refused.  The test's device buffers come from the HIP runtime
libchpe.so itself links (through ctypes); the entry point allocates nothing."""
import ctypes

import numpy as np
import pytest

import chpe_amd as ca

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


def hip_runtime():
    ca.load_engine_lib()  # the runtime is already mapped by libchpe.so; this finds the same one
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
    hip.hipFree.argtypes = [ctypes.c_void_p]
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    return hip


class DeviceArray:
    def __init__(self, hip, host):
        self.hip, self.nbytes = hip, host.nbytes
        self.ptr = ctypes.c_void_p()
        assert hip.hipMalloc(ctypes.byref(self.ptr), self.nbytes) == 0
        assert hip.hipMemcpy(self.ptr, host.ctypes.data, self.nbytes, H2D) == 0

    def get(self, dtype, n):
        out = np.empty(n, dtype)
        assert self.hip.hipMemcpy(out.ctypes.data, self.ptr, self.nbytes, D2H) == 0
        return out

    def free(self):
        self.hip.hipFree(self.ptr)


def engine_cache(k_rows, v_rows, kv_heads, hd, max_seq, kv_f16):
    """Rows [ctx][kv_heads * hd] in the engine's cache layout: k [kv][max_seq][hd]; v as k for
    the f32 cache and [kv][max_seq / 4][hd][4] for the fp16 cache."""
    ctx = k_rows.shape[0]
    kk = k_rows.reshape(ctx, kv_heads, hd).transpose(1, 0, 2)
    vv = v_rows.reshape(ctx, kv_heads, hd).transpose(1, 0, 2)
    dt = np.float16 if kv_f16 else np.float32
    k = np.zeros((kv_heads, max_seq, hd), dt)
    k[:, :ctx] = kk.astype(dt)
    if kv_f16:
        v = np.zeros((kv_heads, max_seq // 4, hd, 4), dt)
        for t in range(ctx):
            v[:, t // 4, :, t % 4] = vv[:, t].astype(dt)
    else:
        v = np.zeros((kv_heads, max_seq, hd), dt)
        v[:, :ctx] = vv.astype(dt)
    return k, v


@pytest.mark.parametrize("hd,H,KV,kv_f16", [(128, 64, 8, 1), (256, 16, 4, 0), (128, 16, 2, 1), (256, 16, 4, 1)])
def test_noalloc_attention_matches_allocating_entry(hd, H, KV, kv_f16):
    lib, hip = ca.load_engine_lib(), hip_runtime()
    max_seq = 4352
    rng = np.random.default_rng(hd + H + kv_f16)
    for pos in (1000, 37):  # the second call is smaller and reuses the scratch
        print(f"noalloc attention hd={hd} H={H} KV={KV} kv_f16={kv_f16} pos={pos}", flush=True)
        q = (rng.standard_normal(H * hd) * 2.0).astype(np.float32)
        k = rng.standard_normal((pos + 1, KV * hd)).astype(np.float32)
        v = rng.standard_normal((pos + 1, KV * hd)).astype(np.float32)
        ref = ca.gpu_attention(q, k, v, pos, H, KV, hd, kv_f16)
        kc, vc = engine_cache(k, v, KV, hd, max_seq, kv_f16)
        bufs = [DeviceArray(hip, a) for a in (q, kc, vc, np.full(H * hd, np.nan, np.float32))]
        try:
            dq, dk, dv, dout = (b.ptr for b in bufs)
            rc = lib.chpe_attention_noalloc(hd, H, KV, kv_f16, pos, max_seq, dq, dk, dv, dout, None)
            assert rc == 0
            got = bufs[3].get(np.float32, H * hd)  # hipMemcpy waits for the default stream
            assert np.array_equal(got.view(np.uint32), ref.view(np.uint32)), float(np.abs(got - ref).max())
            # partials past the 8 MiB scratch (64 heads x 320 chunks of 128 positions x 130 floats):
            # refused, nothing launched
            assert lib.chpe_attention_noalloc(128, 64, 8, 1, 40959, 40960, dq, dk, dv, dout, None) == -2
            # bad arguments: a position past the cache, a null pointer
            assert lib.chpe_attention_noalloc(hd, H, KV, kv_f16, max_seq, max_seq, dq, dk, dv, dout, None) == -1
            assert lib.chpe_attention_noalloc(hd, H, KV, kv_f16, pos, max_seq, None, dk, dv, dout, None) == -1
        finally:
            for b in bufs:
                b.free()
