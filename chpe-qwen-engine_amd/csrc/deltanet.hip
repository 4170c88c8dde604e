// deltanet.hip -- one decode step of a gated-DeltaNet (linear-attention) layer of Qwen3.5.
//
// The reference engine has no code for these layers (its README only claims them); the
// arithmetic follows the published gated delta rule (Yang, Kautz, Hatamizadeh, ICLR 2025)
// in the form of the library that defines the Qwen3.5 layer (transformers 5.15.0,
// models/qwen3_5/modeling_qwen3_5.py: causal_conv1d_update :200-217, l2norm :242-245,
// torch_recurrent_gated_delta_rule :331-380, beta/g :497-499, head repetition :500-502,
// RMSNormGated :168-184).
//
// k_dn_conv: the depthwise causal conv over [state, x] + SiLU, one thread per channel, the
// state shifted in place (the decode step applies it in its in-projection's epilogue instead).
// k_dn_step_head: the gated delta rule and the gated RMSNorm of one value head per workgroup
// (the decode step's form); k_dn_step: a workgroup per (value head, 16-column block), its slab
// of the head's 128x128 f32 state read once and written once (the columns of the update are
// independent), with k_dn_gnorm for the gated RMSNorm of each head's output.  2 x 64 KiB of
// state per head and step.
//
// The block step (m <= kMaxBlock tokens in order, the speculative verify and the prefill):
// k_dn_conv_block, k_dn_step_block and k_dn_gnorm_block run the same arithmetic token after
// token inside one launch, each state read once and written once for the m tokens (the conv
// state in registers per channel, a head's state slab in registers per workgroup).
#include <cstdio>

#include "device_common.hpp"
#include "kernels.hpp"

namespace chpe {
namespace {
using namespace dev;

__device__ __forceinline__ float silu_f(float x) { return x / (1.0f + expf(-x)); }
__device__ __forceinline__ float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

__global__ void __launch_bounds__(256) k_dn_conv(DnConvArgs a) {
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.channels) return;
  const uint32_t T = a.taps;
  const float* w = a.w + size_t(c) * T;
  float* st = a.state + size_t(c) * (T - 1);
  float wv[kDnMaxTaps], sv[kDnMaxTaps];
#pragma unroll
  for (uint32_t k = 0; k < kDnMaxTaps; ++k) {
    wv[k] = k + 1 < T ? w[k] : 0.0f;
    sv[k] = k + 1 < T ? st[k] : 0.0f;
  }
  const float x = a.x[c], wl = w[T - 1];
  const bool keep = a.step && a.step->broken;  // (after the step's break: the state stays)
  float acc = 0.0f;  // oldest tap first, the new input last
#pragma unroll
  for (uint32_t k = 0; k < kDnMaxTaps; ++k)
    if (k + 1 < T) acc += wv[k] * sv[k];
  acc += wl * x;
  a.out[c] = silu_f(acc);
  if (keep) return;
#pragma unroll
  for (uint32_t k = 0; k + 1 < kDnMaxTaps; ++k)
    if (k + 2 < T) st[k] = sv[k + 1];
  st[T - 2] = x;
}

// grid (value head, column block of CW columns): the block's D x CW slab of the head's state
// (rows i, columns c0 + j) is read once and written once; every column of the update is
// independent (kv_mem[j], delta_j, S[:, j], o[j]), so the head's columns spread over D / CW
// workgroups.  Thread (row block rb, column j) holds rows rb * RPB .. of column c0 + j; the
// two column sums (S^T k before the update, S^T q after) meet over the row blocks of a wave
// (lanes 16 and 32 apart) and over the waves in LDS, in a fixed order.  q and k are
// l2-normalised by every workgroup of the head (D values each).  Writes o[j] = (S^T q)_j; the
// gated norm, a reduction over the whole head, is k_dn_gnorm.
template <int D, int CW>
__global__ void __launch_bounds__(256) k_dn_step(DnStepArgs a) {
  constexpr int NT = 256, RB = NT / CW, RPB = D / RB, NWV = NT / 64;
  static_assert(CW == 16 && NT % CW == 0 && D % RB == 0 && D % 64 == 0, "lanes 16 / 32 apart share a column");
  const uint32_t h = blockIdx.x, c0 = blockIdx.y * CW, kh = h / (a.n_v_heads / a.n_k_heads);
  const int t = threadIdx.x, j = t % CW, rb = t / CW, lane = t & 63, wave = t >> 6;
  __shared__ float s_qn[D], s_kn[D];
  __shared__ float s_part[NWV][CW];

  // 1. loads: the thread's state rows, then the head's inputs (all before any use)
  float* S = a.state + size_t(h) * D * D + c0 + j;
  float sr[RPB];
#pragma unroll
  for (int r = 0; r < RPB; ++r) sr[r] = S[size_t(rb * RPB + r) * D];
  constexpr int PL = D / 64;  // q/k values per lane (every wave normalises both vectors)
  float qv[PL], kv[PL];
#pragma unroll
  for (int m = 0; m < PL; ++m) {
    qv[m] = a.q[size_t(kh) * D + lane + 64 * m];
    kv[m] = a.k[size_t(kh) * D + lane + 64 * m];
  }
  const float vj = a.v[size_t(h) * D + c0 + j];
  const bool keep = a.step && a.step->broken;  // (after the step's break: the state stays)
  const float beta = 1.0f / (1.0f + expf(-a.b[h]));
  const float decay = expf(-expf(a.A_log[h]) * softplus_f(a.a[h] + a.dt_bias[h]));

  // 2. l2-normalised q (scaled by 1/sqrt(D)) and k, into LDS
  float q2 = 0.0f, k2 = 0.0f;
#pragma unroll
  for (int m = 0; m < PL; ++m) {
    q2 += qv[m] * qv[m];
    k2 += kv[m] * kv[m];
  }
  q2 = wave_sum(q2);
  k2 = wave_sum(k2);
  const float qi = 1.0f / sqrtf(q2 + 1e-6f), ki = 1.0f / sqrtf(k2 + 1e-6f), scale = 1.0f / sqrtf(float(D));
  if (wave == 0) {
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      s_qn[lane + 64 * m] = qv[m] * qi * scale;
      s_kn[lane + 64 * m] = kv[m] * ki;
    }
  }
  __syncthreads();

  // the column sum of a per-thread partial: over the wave's 4 row blocks, then the waves
  auto column_sum = [&](float p) {
    p = pair_sum(p, 16);
    p = pair_sum(p, 32);
    if (lane < CW) s_part[wave][lane] = p;
    __syncthreads();
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) v += s_part[w][j];
    __syncthreads();  // s_part is reused by the next sum
    return v;
  };

  // 3. decayed state; kv_mem[j] = sum_i S[i][j] k[i]
  float p = 0.0f;
#pragma unroll
  for (int r = 0; r < RPB; ++r) {
    sr[r] *= decay;
    p += sr[r] * s_kn[rb * RPB + r];
  }
  const float kvm = column_sum(p);
  const float delta = (vj - kvm) * beta;

  // 4. S += k delta^T, written back; o[j] = sum_i S[i][j] q[i]
  float o = 0.0f;
#pragma unroll
  for (int r = 0; r < RPB; ++r) {
    sr[r] += s_kn[rb * RPB + r] * delta;
    if (!keep) S[size_t(rb * RPB + r) * D] = sr[r];
    o += sr[r] * s_qn[rb * RPB + r];
  }
  o = column_sum(o);
  if (t < CW) a.out[size_t(h) * D + c0 + j] = o;
}

// The gated delta rule and the gated RMSNorm of one value head in one workgroup of kDnRb * D
// threads (thread (row block rb, column j): rows rb * D / kDnRb .. of column j; the column sums
// meet in LDS over the row blocks in order), so that the norm, a reduction over the head's D
// outputs, needs no second launch.  The same arithmetic as k_dn_step + k_dn_gnorm up to the
// order of the float sums.
constexpr int kDnRb = 8;
template <int D>
__global__ void __launch_bounds__(kDnRb * D) k_dn_step_head(DnStepArgs a) {
  constexpr int NT = kDnRb * D, RPB = D / kDnRb, NWV = NT / 64;
  static_assert(D % 64 == 0 && D % kDnRb == 0, "");
  const uint32_t h = blockIdx.x, kh = h / (a.n_v_heads / a.n_k_heads);
  const int t = threadIdx.x, j = t % D, rb = t / D, lane = t & 63, wave = t >> 6;
  __shared__ float s_qn[D], s_kn[D];
  __shared__ float s_part[kDnRb][D];
  __shared__ float s_red[NWV];

  // 1. loads: the thread's state rows, then the head's inputs (all before any use)
  float* S = a.state + size_t(h) * D * D + j;
  float sr[RPB];
#pragma unroll
  for (int r = 0; r < RPB; ++r) sr[r] = S[size_t(rb * RPB + r) * D];
  constexpr int PL = D / 64;
  float qv[PL], kv[PL];
#pragma unroll
  for (int m = 0; m < PL; ++m) {
    qv[m] = a.q[size_t(kh) * D + lane + 64 * m];
    kv[m] = a.k[size_t(kh) * D + lane + 64 * m];
  }
  const float vj = a.v[size_t(h) * D + j], zj = a.z[size_t(h) * D + j], wj = a.norm_w[j];
  const bool keep = a.step && a.step->broken;  // (after the step's break: the state stays)
  const float beta = 1.0f / (1.0f + expf(-a.b[h]));
  const float decay = expf(-expf(a.A_log[h]) * softplus_f(a.a[h] + a.dt_bias[h]));

  // 2. l2-normalised q (scaled by 1/sqrt(D)) and k, into LDS
  float q2 = 0.0f, k2 = 0.0f;
#pragma unroll
  for (int m = 0; m < PL; ++m) {
    q2 += qv[m] * qv[m];
    k2 += kv[m] * kv[m];
  }
  q2 = wave_sum(q2);
  k2 = wave_sum(k2);
  const float qi = 1.0f / sqrtf(q2 + 1e-6f), ki = 1.0f / sqrtf(k2 + 1e-6f), scale = 1.0f / sqrtf(float(D));
  if (wave == 0) {
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      s_qn[lane + 64 * m] = qv[m] * qi * scale;
      s_kn[lane + 64 * m] = kv[m] * ki;
    }
  }
  __syncthreads();

  // the column sum of a per-thread partial over the row blocks, in order (every thread gets it)
  auto column_sum = [&](float p) {
    s_part[rb][j] = p;
    __syncthreads();
    float v = 0.0f;
#pragma unroll
    for (int b = 0; b < kDnRb; ++b) v += s_part[b][j];
    __syncthreads();  // s_part is reused by the next sum
    return v;
  };

  // 3. decayed state; kv_mem[j] = sum_i S[i][j] k[i]
  float p = 0.0f;
#pragma unroll
  for (int r = 0; r < RPB; ++r) {
    sr[r] *= decay;
    p += sr[r] * s_kn[rb * RPB + r];
  }
  const float kvm = column_sum(p);
  const float delta = (vj - kvm) * beta;

  // 4. S += k delta^T, written back; o[j] = sum_i S[i][j] q[i]
  float o = 0.0f;
#pragma unroll
  for (int r = 0; r < RPB; ++r) {
    sr[r] += s_kn[rb * RPB + r] * delta;
    if (!keep) S[size_t(rb * RPB + r) * D] = sr[r];
    o += sr[r] * s_qn[rb * RPB + r];
  }
  o = column_sum(o);

  // 5. the gated RMSNorm over the head's D outputs (row block 0's threads): w * (o * rr) * silu(z)
  if (rb == 0) {
    const float s2 = wave_sum(o * o);
    if (lane == 0) s_red[wave] = s2;
  }
  __syncthreads();
  if (rb != 0) return;
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < D / 64; ++w) tot += s_red[w];
  const float rr = 1.0f / sqrtf(tot / float(D) + a.eps);
  a.out[size_t(h) * D + j] = wj * (o * rr) * silu_f(zj);
}

// the gated RMSNorm of each value head's output (one workgroup of D threads per head):
// w * (o * rsqrt(mean o^2 + eps)) * silu(z)
template <int D>
__global__ void __launch_bounds__(D) k_dn_gnorm(DnStepArgs a) {
  const uint32_t h = blockIdx.x;
  const int j = threadIdx.x, lane = j & 63, wave = j >> 6;
  __shared__ float s_red[D / 64];
  const float o = a.out[size_t(h) * D + j], z = a.z[size_t(h) * D + j], w = a.norm_w[j];
  const float s2 = wave_sum(o * o);
  if (lane == 0) s_red[wave] = s2;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int k = 0; k < D / 64; ++k) tot += s_red[k];
  const float rr = 1.0f / sqrtf(tot / float(D) + a.eps);
  a.out[size_t(h) * D + j] = w * (o * rr) * silu_f(z);
}

// ---- the block step: m tokens in order, each state read and written once ----------------------
// (the conv's taps fixed at compile time: the token loop unrolls, the inputs stay in registers)
__global__ void __launch_bounds__(256) k_dn_conv_block(DnBlockArgs a) {
  const uint32_t c = blockIdx.x * 256 + threadIdx.x;
  if (c >= a.channels) return;
  constexpr uint32_t T = kDnConvTaps;
  const float* w = a.w + size_t(c) * T;
  float* st = a.conv_state + size_t(c) * (T - 1);
  float wv[kDnMaxTaps], sv[kDnMaxTaps];
#pragma unroll
  for (uint32_t k = 0; k < kDnMaxTaps; ++k) {
    wv[k] = k + 1 < T ? w[k] : 0.0f;
    sv[k] = k + 1 < T ? st[k] : 0.0f;
  }
  const float wl = w[T - 1];
  // every token's input and break flag requested before the first is used (the tokens' chain
  // through the state is short; their loads are not)
  float xs[kMaxBlock];
  uint32_t bm = 0;
#pragma unroll
  for (uint32_t t = 0; t < kMaxBlock; ++t) {
    xs[t] = t < a.m ? a.x[size_t(t) * a.x_stride + c] : 0.0f;
    bm |= (t < a.m && a.brk[t] != 0u ? 1u : 0u) << t;
  }
#pragma unroll
  for (uint32_t t = 0; t < kMaxBlock; ++t) {
    if (t >= a.m) break;
    const float x = xs[t];
    float acc = 0.0f;  // oldest tap first, the new input last (k_dn_conv)
#pragma unroll
    for (uint32_t k = 0; k < kDnMaxTaps; ++k)
      if (k + 1 < T) acc += wv[k] * sv[k];
    acc += wl * x;
    a.conv_out[size_t(t) * a.channels + c] = silu_f(acc);
    if ((bm >> t) & 1u) continue;  // (token t broke before this layer: its shift is skipped)
#pragma unroll
    for (uint32_t k = 0; k + 1 < kDnMaxTaps; ++k)
      if (k + 2 < T) sv[k] = sv[k + 1];
    sv[T - 2] = x;
  }
#pragma unroll
  for (uint32_t k = 0; k + 1 < kDnMaxTaps; ++k)
    if (k + 1 < T) st[k] = sv[k];
}

// k_dn_step's workgroup (value head, 16-column block) over the m tokens: the slab stays in
// registers from the first token's read to the last token's write; per token the same steps as
// k_dn_step (l2-normalised q and k, decay, kv_mem, delta, the update, o), a token that broke
// before this layer leaving the slab as it is.
template <int D, int CW>
__global__ void __launch_bounds__(256) k_dn_step_block(DnBlockArgs a) {
  constexpr int NT = 256, RB = NT / CW, RPB = D / RB, NWV = NT / 64;
  static_assert(CW == 16 && NT % CW == 0 && D % RB == 0 && D % 64 == 0, "lanes 16 / 32 apart share a column");
  const uint32_t h = blockIdx.x, c0 = blockIdx.y * CW, kh = h / (a.n_v_heads / a.n_k_heads);
  const int t = threadIdx.x, j = t % CW, rb = t / CW, lane = t & 63, wave = t >> 6;
  __shared__ float s_qn[D], s_kn[D];
  __shared__ float s_part[NWV][CW];
  float* S = a.state + size_t(h) * D * D + c0 + j;
  float sr[RPB];
#pragma unroll
  for (int r = 0; r < RPB; ++r) sr[r] = S[size_t(rb * RPB + r) * D];
  constexpr int PL = D / 64;
  const float scale = 1.0f / sqrtf(float(D));
  const uint32_t nk = a.n_k_heads * D;  // q: [0, nk), k: [nk, 2 nk), v: [2 nk, ..) of a token's channels
  const float A = expf(a.A_log[h]), dtb = a.dt_bias[h];

  auto column_sum = [&](float p) {
    p = pair_sum(p, 16);
    p = pair_sum(p, 32);
    if (lane < CW) s_part[wave][lane] = p;
    __syncthreads();
    float v = 0.0f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) v += s_part[w][j];
    __syncthreads();
    return v;
  };
  uint32_t bm = 0;  // the tokens' break flags, read once (not one dependent load per token)
#pragma unroll
  for (uint32_t u = 0; u < kMaxBlock; ++u) bm |= (u < a.m && a.brk[u] != 0u ? 1u : 0u) << u;

  for (uint32_t tk = 0; tk < a.m; ++tk) {
    const float* xc = a.conv_out + size_t(tk) * a.channels;
    float qv[PL], kv[PL];
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      qv[m] = xc[size_t(kh) * D + lane + 64 * m];
      kv[m] = xc[nk + size_t(kh) * D + lane + 64 * m];
    }
    const float vj = xc[2 * nk + size_t(h) * D + c0 + j];
    const float bt = a.b[size_t(tk) * a.ab_stride + h], at = a.a[size_t(tk) * a.ab_stride + h];
    const float beta = 1.0f / (1.0f + expf(-bt));
    const float decay = expf(-A * softplus_f(at + dtb));
    float q2 = 0.0f, k2 = 0.0f;
#pragma unroll
    for (int m = 0; m < PL; ++m) {
      q2 += qv[m] * qv[m];
      k2 += kv[m] * kv[m];
    }
    q2 = wave_sum(q2);
    k2 = wave_sum(k2);
    const float qi = 1.0f / sqrtf(q2 + 1e-6f), ki = 1.0f / sqrtf(k2 + 1e-6f);
    __syncthreads();  // the previous token's reads of s_qn / s_kn are done
    if (wave == 0) {
#pragma unroll
      for (int m = 0; m < PL; ++m) {
        s_qn[lane + 64 * m] = qv[m] * qi * scale;
        s_kn[lane + 64 * m] = kv[m] * ki;
      }
    }
    __syncthreads();
    if ((bm >> tk) & 1u) {  // (uniform: the token's slab update is skipped, its output is not used)
      if (t < CW) a.out[size_t(tk) * a.out_stride + size_t(h) * D + c0 + j] = 0.0f;
      continue;
    }
    float p = 0.0f;
#pragma unroll
    for (int r = 0; r < RPB; ++r) {
      sr[r] *= decay;
      p += sr[r] * s_kn[rb * RPB + r];
    }
    const float kvm = column_sum(p);
    const float delta = (vj - kvm) * beta;
    float o = 0.0f;
#pragma unroll
    for (int r = 0; r < RPB; ++r) {
      sr[r] += s_kn[rb * RPB + r] * delta;
      o += sr[r] * s_qn[rb * RPB + r];
    }
    o = column_sum(o);
    if (t < CW) a.out[size_t(tk) * a.out_stride + size_t(h) * D + c0 + j] = o;
  }
#pragma unroll
  for (int r = 0; r < RPB; ++r) S[size_t(rb * RPB + r) * D] = sr[r];
}

// k_dn_gnorm for token blockIdx.y
template <int D>
__global__ void __launch_bounds__(D) k_dn_gnorm_block(DnBlockArgs a) {
  const uint32_t h = blockIdx.x, tk = blockIdx.y;
  const int j = threadIdx.x, lane = j & 63, wave = j >> 6;
  __shared__ float s_red[D / 64];
  float* out = a.out + size_t(tk) * a.out_stride;
  const float* zt = a.z + size_t(tk) * a.z_stride;
  const float o = out[size_t(h) * D + j], z = zt[size_t(h) * D + j], w = a.norm_w[j];
  const float s2 = wave_sum(o * o);
  if (lane == 0) s_red[wave] = s2;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int k = 0; k < D / 64; ++k) tot += s_red[k];
  const float rr = 1.0f / sqrtf(tot / float(D) + a.eps);
  out[size_t(h) * D + j] = w * (o * rr) * silu_f(z);
}

}  // namespace

void launch_dn_block(const DnBlockArgs& a, hipStream_t st) {
  constexpr uint32_t CW = 16;
  if (a.taps != kDnConvTaps) {  // (the engine plans the 9B layers: 4 taps)
    std::fprintf(stderr, "chpe: the block step's conv is built for %u taps\n", kDnConvTaps);
    return;
  }
  launch_kernel(&k_dn_conv_block, dim3((a.channels + 255) / 256), dim3(256), st, a);
  if (a.head_dim == 128) {
    launch_kernel(&k_dn_step_block<128, CW>, dim3(a.n_v_heads, 128 / CW), dim3(256), st, a);
    launch_kernel(&k_dn_gnorm_block<128>, dim3(a.n_v_heads, a.m), dim3(128), st, a);
  } else {
    launch_kernel(&k_dn_step_block<64, CW>, dim3(a.n_v_heads, 64 / CW), dim3(256), st, a);
    launch_kernel(&k_dn_gnorm_block<64>, dim3(a.n_v_heads, a.m), dim3(64), st, a);
  }
}

bool deltanet_supported(uint32_t n_v_heads, uint32_t n_k_heads, uint32_t head_dim, uint32_t taps) {
  return n_k_heads > 0 && n_v_heads % n_k_heads == 0 && (head_dim == 64 || head_dim == 128) && taps >= 2 &&
         taps <= kDnMaxTaps;
}

void launch_dn_conv(const DnConvArgs& a, hipStream_t st) {
  launch_kernel(&k_dn_conv, dim3((a.channels + 255) / 256), dim3(256), st, a);
}

void launch_dn_step(const DnStepArgs& a, uint32_t head_dim, hipStream_t st) {
  constexpr uint32_t CW = 16;
  if (a.norm_w && head_dim == 128) {  // the gated form: a workgroup per head, the norm included
    launch_kernel(&k_dn_step_head<128>, dim3(a.n_v_heads), dim3(kDnRb * 128), st, a);
    return;
  }
  if (head_dim == 128) {
    launch_kernel(&k_dn_step<128, CW>, dim3(a.n_v_heads, 128 / CW), dim3(256), st, a);
    if (a.norm_w) launch_kernel(&k_dn_gnorm<128>, dim3(a.n_v_heads), dim3(128), st, a);
  } else {
    launch_kernel(&k_dn_step<64, CW>, dim3(a.n_v_heads, 64 / CW), dim3(256), st, a);
    if (a.norm_w) launch_kernel(&k_dn_gnorm<64>, dim3(a.n_v_heads), dim3(64), st, a);
  }
}

}  // namespace chpe
