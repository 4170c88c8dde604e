// hybrid.hip -- the gated full-attention layer of the Qwen3.5-9B hybrid around the decode
// attention kernels.  No reference code (README.md:17,62 only name the model); the arithmetic
// follows the library that defines the layer, transformers 5.15.0
// models/qwen3_5/modeling_qwen3_5.py Qwen3_5Attention (:629-701): q_proj rows per head are the
// query then the output gate (:672-675); RMSNorm of each query and key head (:677-678, the
// gains as stored: the engine's norm tiles hold the effective gain); the rotary embedding of
// the first rot dims, rotate_half pairs (i, i + rot/2) (:546-591), angles from the engine's
// tables (the reference's applyRope formula over rot dims, chpe_engine.zig:195-216).  The
// attention output times sigmoid(gate) (:696) is applied by the attention merge
// (AttnArgs::gate).
#include "device_common.hpp"
#include "kernels.hpp"

namespace chpe {
namespace {
using namespace dev;

// one workgroup per head and token (blockIdx.y: token t at position pos + t of a block step, 0
// in the decode step): blocks 0..H-1 the query heads, H..H+KV-1 the key heads, then the value
// heads; thread d holds dimension d
template <int HD>
__global__ void __launch_bounds__(HD) k_hyb_qk(HybQkArgs a) {
#pragma clang fp contract(off)
  const uint32_t b = blockIdx.x, d = threadIdx.x, tk = blockIdx.y;
  const bool is_q = b < a.H, is_k = !is_q && b < a.H + a.KV;
  const uint32_t h = is_q ? b : (is_k ? b - a.H : b - a.H - a.KV);
  StepState st = *a.state;
  st.pos += tk;
  if (a.brk) st.broken = a.brk[tk];
  const float* qg = a.qg + size_t(tk) * a.qg_stride;
  const float* kk = a.k + size_t(tk) * a.kv_stride;
  const float* vv = a.v + size_t(tk) * a.kv_stride;
  __shared__ float s_x[HD];
  __shared__ float s_red[HD / 64];
  float x = is_q ? qg[size_t(h) * 2 * HD + d] : (is_k ? kk[size_t(h) * HD + d] : vv[size_t(h) * HD + d]);
  if (is_q || is_k) {  // (uniform per workgroup)
    const float g = is_q ? a.q_norm[d] : a.k_norm[d];
    const float s2 = wave_sum(x * x);
    if ((d & 63) == 0) s_red[d >> 6] = s2;
    __syncthreads();
    float tot = 0.0f;
#pragma unroll
    for (int w = 0; w < HD / 64; ++w) tot += s_red[w];
    const float inv = 1.0f / sqrtf(tot / float(HD) + a.eps);
    x = x * inv * g;
    s_x[d] = x;
    __syncthreads();
    const uint32_t half = a.rot / 2;
    if (d < a.rot && st.pos < a.rope_rows) {
      const uint32_t i = d < half ? d : d - half;
      const float c = a.rope_cos[size_t(st.pos) * half + i], sn = a.rope_sin[size_t(st.pos) * half + i];
      const float x0 = s_x[i], x1 = s_x[i + half];
      x = d < half ? x0 * c - x1 * sn : x0 * sn + x1 * c;
    }
  }
  if (is_q) {
    a.q_out[size_t(tk) * a.q_stride + size_t(h) * HD + d] = x;
    return;
  }
  if (st.broken) return;  // forwardDecode's break: no KV append
  const uint32_t pos = st.pos;
  void* cache = is_k ? a.k_cache : a.v_cache;
  if (a.kv_f16 && !is_k) {  // 4-position blocks: [pos/4][dim][pos%4]
    const size_t blk = (size_t(h) * a.max_seq + (pos & ~3u)) * HD + (pos & 3u);
    reinterpret_cast<__half*>(cache)[blk + size_t(d) * 4] = __float2half_rn(x);
  } else if (a.kv_f16) {
    reinterpret_cast<__half*>(cache)[(size_t(h) * a.max_seq + pos) * HD + d] = __float2half_rn(x);
  } else {
    reinterpret_cast<float*>(cache)[(size_t(h) * a.max_seq + pos) * HD + d] = x;
  }
}

}  // namespace

void launch_hyb_qk(const HybQkArgs& a, hipStream_t st) {
  if (a.hd != 256) return;  // (the 9B head dim; the engine checks the shape at init)
  launch_kernel(&k_hyb_qk<256>, dim3(a.H + 2 * a.KV, a.m ? a.m : 1), dim3(256), st, a);
}

}  // namespace chpe
