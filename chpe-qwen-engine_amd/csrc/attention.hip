// attention.hip -- RoPE + KV append + GQA decode attention over the HBM KV cache.
//
// Semantics: applyRope (chpe_engine.zig:195-216), KV write at `pos` (:1693-1697) and the
// per-head attention loop (:1700-1734): scores (q.k_t)*scale, softmax over t <= pos, output
// sum_t softmax_t * v_t.  The context is split into chunks of 8192/hd positions (flash
// decoding): k_attn_partial computes, per chunk and query head, the chunk max m, the sum of
// exp(s - m) and the exp-weighted sum of V; k_attn_combine rescales and merges the chunks.
// Workgroup (chunk c, kv head g) serves the H/KV query heads that share kv head g, so every
// K/V row is read from HBM once per step.  The workgroup holding `pos` rotates the new K row,
// rounds K/V to the cache type, stores them and uses the stored values.
#include "device_common.hpp"
#include "kernels.hpp"

namespace chpe {
namespace {
using namespace dev;

// x0*cos - x1*sin / x0*sin + x1*cos without contraction, as applyRope (:212-213)
__device__ __forceinline__ float rope_rot(float x0, float x1, float c, float s, bool first) {
#pragma clang fp contract(off)
  return first ? x0 * c - x1 * s : x0 * s + x1 * c;
}

template <int HD>
__global__ void __launch_bounds__(256) k_attn_partial(AttnArgs a) {
  constexpr int CH = 8192 / HD;  // 64 positions at hd 128, 32 at hd 256
  constexpr int HALF = HD / 2;
  constexpr int VEC = 8;         // elements per 16-byte fp16 cache access
  const uint32_t pos = a.state->pos, ctx = pos + 1;
  const uint32_t c = blockIdx.x, kvh = blockIdx.y;
  if (c * CH >= ctx) return;
  const uint32_t t0 = c * CH, nv = min(uint32_t(CH), ctx - t0);
  const uint32_t G = a.H / a.KV;
  const int tid = threadIdx.x, nt = blockDim.x;

  __shared__ float qs[8][HD];
  __shared__ float ks[CH][HD + 1];
  __shared__ float vs[CH][HD];
  __shared__ float ps[8][CH];
  __shared__ float s_m[8], s_l[8];

  const float* cs = a.rope_cos + size_t(pos) * HALF;
  const float* sn = a.rope_sin + size_t(pos) * HALF;
  for (uint32_t i = tid; i < G * HD; i += nt) {  // rotated queries of the group
    const uint32_t g = i / HD, d = i % HD, j = d % HALF;
    const float* q = a.q_raw + size_t(kvh * G + g) * HD;
    qs[g][d] = rope_rot(q[j], q[j + HALF], cs[j], sn[j], d < HALF);
  }
  const size_t head_base = size_t(kvh) * a.max_seq * HD;
  for (uint32_t i = tid; i < nv * (HD / VEC); i += nt) {
    const uint32_t t = i / (HD / VEC), d0 = (i % (HD / VEC)) * VEC, tp = t0 + t;
    const size_t off = head_base + size_t(tp) * HD + d0;
    float kv[VEC], vv[VEC];
    if (tp == pos) {  // the new row
      const float* k = a.k_raw + size_t(kvh) * HD;
      const float* v = a.v_raw + size_t(kvh) * HD;
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        const uint32_t d = d0 + e, j = d % HALF;
        kv[e] = rope_rot(k[j], k[j + HALF], cs[j], sn[j], d < HALF);
        vv[e] = v[d];
      }
      if (a.kv_f16) {
        __half kh[VEC], vh[VEC];
#pragma unroll
        for (int e = 0; e < VEC; ++e) {
          kh[e] = __float2half_rn(kv[e]);
          vh[e] = __float2half_rn(vv[e]);
          kv[e] = __half2float(kh[e]);
          vv[e] = __half2float(vh[e]);
        }
        *reinterpret_cast<uint4*>(reinterpret_cast<__half*>(a.k_cache) + off) = *reinterpret_cast<uint4*>(kh);
        *reinterpret_cast<uint4*>(reinterpret_cast<__half*>(a.v_cache) + off) = *reinterpret_cast<uint4*>(vh);
      } else {
        float4* kc = reinterpret_cast<float4*>(reinterpret_cast<float*>(a.k_cache) + off);
        float4* vc = reinterpret_cast<float4*>(reinterpret_cast<float*>(a.v_cache) + off);
        kc[0] = make_float4(kv[0], kv[1], kv[2], kv[3]);
        kc[1] = make_float4(kv[4], kv[5], kv[6], kv[7]);
        vc[0] = make_float4(vv[0], vv[1], vv[2], vv[3]);
        vc[1] = make_float4(vv[4], vv[5], vv[6], vv[7]);
      }
    } else if (a.kv_f16) {
      const uint4 kq = *reinterpret_cast<const uint4*>(reinterpret_cast<const __half*>(a.k_cache) + off);
      const uint4 vq = *reinterpret_cast<const uint4*>(reinterpret_cast<const __half*>(a.v_cache) + off);
      const uint32_t kw[4] = {kq.x, kq.y, kq.z, kq.w}, vw[4] = {vq.x, vq.y, vq.z, vq.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        kv[2 * e] = h2f(uint16_t(kw[e] & 0xffffu));
        kv[2 * e + 1] = h2f(uint16_t(kw[e] >> 16));
        vv[2 * e] = h2f(uint16_t(vw[e] & 0xffffu));
        vv[2 * e + 1] = h2f(uint16_t(vw[e] >> 16));
      }
    } else {
      const float4* kc = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.k_cache) + off);
      const float4* vc = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(a.v_cache) + off);
      const float4 k0 = kc[0], k1 = kc[1], v0 = vc[0], v1 = vc[1];
      kv[0] = k0.x; kv[1] = k0.y; kv[2] = k0.z; kv[3] = k0.w; kv[4] = k1.x; kv[5] = k1.y; kv[6] = k1.z; kv[7] = k1.w;
      vv[0] = v0.x; vv[1] = v0.y; vv[2] = v0.z; vv[3] = v0.w; vv[4] = v1.x; vv[5] = v1.y; vv[6] = v1.z; vv[7] = v1.w;
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      ks[t][d0 + e] = kv[e];
      vs[t][d0 + e] = vv[e];
    }
  }
  __syncthreads();
  for (uint32_t i = tid; i < G * CH; i += nt) {  // scores: one (head, position) per thread
    const uint32_t g = i / CH, t = i % CH;
    float s = -INFINITY;
    if (t < nv) {
      float dot = 0.0f;
#pragma unroll 8
      for (int d = 0; d < HD; ++d) dot += qs[g][d] * ks[t][d];
      s = dot * a.scale;
    }
    ps[g][t] = s;
  }
  __syncthreads();
  const int wave = tid >> 6, lane = tid & 63, nw = nt / kWave;
  for (uint32_t g = wave; g < G; g += nw) {  // chunk-local softmax statistics
    float m = -INFINITY;
    for (int t = lane; t < CH; t += kWave) m = fmaxf(m, ps[g][t]);
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    float l = 0.0f;
    for (int t = lane; t < CH; t += kWave) {
      const float e = t < int(nv) ? expf(ps[g][t] - m) : 0.0f;
      ps[g][t] = e;
      l += e;
    }
    l = wave_sum(l);
    if (lane == 0) { s_m[g] = m; s_l[g] = l; }
  }
  __syncthreads();
  const uint32_t nch = a.n_chunks;
  for (uint32_t i = tid; i < G * HD; i += nt) {
    const uint32_t g = i / HD, d = i % HD, h = kvh * G + g;
    float acc = 0.0f;
    for (uint32_t t = 0; t < nv; ++t) acc += ps[g][t] * vs[t][d];
    a.part_acc[(size_t(h) * nch + c) * HD + d] = acc;
    if (d == 0) {
      a.part_ml[(size_t(h) * nch + c) * 2] = s_m[g];
      a.part_ml[(size_t(h) * nch + c) * 2 + 1] = s_l[g];
    }
  }
}

// out[h][d] = sum_c acc_c[d] * exp(m_c - M) / sum_c l_c * exp(m_c - M)
__global__ void __launch_bounds__(256) k_attn_combine(AttnArgs a) {
  const uint32_t h = blockIdx.x, d = threadIdx.x;
  if (d >= a.hd) return;
  const uint32_t ch = 8192u / a.hd, n_act = (a.state->pos + 1 + ch - 1) / ch, nch = a.n_chunks;
  const float* ml = a.part_ml + size_t(h) * nch * 2;
  float M = -INFINITY;
  for (uint32_t j = 0; j < n_act; ++j) M = fmaxf(M, ml[2 * j]);
  float L = 0.0f, o = 0.0f;
  for (uint32_t j = 0; j < n_act; ++j) {
    const float w = expf(ml[2 * j] - M);
    L += ml[2 * j + 1] * w;
    o += a.part_acc[(size_t(h) * nch + j) * a.hd + d] * w;
  }
  a.out[size_t(h) * a.hd + d] = o / L;
}

}  // namespace

void launch_attention_partial(const AttnArgs& a, hipStream_t st) {
  const dim3 grid(a.n_chunks, a.KV);
  if (a.hd == 128) launch_kernel(&k_attn_partial<128>, grid, dim3(256), st, a);
  else launch_kernel(&k_attn_partial<256>, grid, dim3(256), st, a);
}

void launch_attention_combine(const AttnArgs& a, hipStream_t st) {
  launch_kernel(k_attn_combine, dim3(a.H), dim3(a.hd), st, a);
}

void launch_attention(const AttnArgs& a, hipStream_t st) {
  launch_attention_partial(a, st);
  launch_attention_combine(a, st);
}

}  // namespace chpe
