// attention.hip -- GQA decode attention over the HBM KV cache.
//
// Semantics: the per-head attention loop of forwardDecode (chpe_engine.zig:1700-1734): scores
// (q.k_t)*scale, softmax over t <= pos, output sum_t softmax_t * v_t.  RoPE and the KV append
// at `pos` (:1688-1697) are done by the q/k/v projection's epilogue (GemvMode::QkvRope), so
// the queries arrive rotated and cache rows 0..pos are complete.  The context is split into
// chunks of attn_chunk(hd, kv) positions (64 or 128 at hd 128, 32 at hd 256): the chunk kernel computes, per
// chunk and query head, the chunk max, the sum of exp(s - max) and the exp-weighted sum of the
// V rows (k_attn_mfma on the matrix cores for the fp16 cache, k_attn_chunk on the vector ALUs
// for the f32 cache); k_attn_merge rescales and merges the chunks.  Workgroup (chunk, kv head)
// serves the query heads that share the kv head, so every K/V row is read from HBM once per step.
#include <cmath>
#include <mutex>

#include "device_common.hpp"
#include "kernels.hpp"

namespace chpe {
namespace {
using namespace dev;

// Cache element access of k_attn_chunk (the f32 KV cache).
template <typename T> struct KvElem;
template <> struct KvElem<float> {
  static constexpr int kBytes = 4;
  __device__ static float get(const uint32_t* w, int i) { return __uint_as_float(w[i]); }
};

// One workgroup = NW waves = one chunk of CH = NW * PW positions of one kv head, for the GQ
// query heads that share it.  In a wave, LPP lanes hold one position's K row (DK = HD/LPP dims
// each) for the q.k dots, and every lane holds HD/64 dims of every V row of the wave's
// PW = 64/LPP positions for the weighted sum; all K/V loads of a wave are issued before any
// arithmetic.  The softmax statistics are per wave, merged over the NW waves in LDS; one
// partial (max, sum, weighted V sum) per chunk and query head goes to HBM for k_attn_merge.
// query z of a block step (blockIdx.z; 0 in the batch-1 step): its query and output rows, its
// chunk partials, position pos + z
__device__ __forceinline__ AttnArgs attn_query(AttnArgs a) {
  const uint32_t z = blockIdx.z;
  a.q += size_t(z) * a.H * a.hd;
  a.out += size_t(z) * a.H * a.hd;
  a.part_ml += size_t(z) * a.H * a.n_chunks * 2;
  a.part_acc += size_t(z) * a.H * a.n_chunks * a.hd;
  return a;
}

template <int HD, int GQ, typename KT, int LPP, int NW>
__global__ void __launch_bounds__(NW * 64) k_attn_chunk(AttnArgs a0) {
  const AttnArgs a = attn_query(a0);
  using E = KvElem<KT>;
  constexpr int PW = 64 / LPP, CH = NW * PW, NT = NW * 64;
  constexpr int DK = HD / LPP;               // K dims per lane
  static_assert(DK % 4 == 0, "");
  constexpr int KW = DK * E::kBytes / 4;    // 32-bit words of a lane's K dims
  constexpr int DPL = HD / 64;              // V dims per lane
  constexpr int VW = DPL * E::kBytes / 4;   // 32-bit words of a lane's V dims (1, 2 or 4)
  static_assert(KW % 4 == 0 && VW >= 1, "");
  const uint32_t pos = a.state->pos + blockIdx.z, ctx = pos + 1;
  const uint32_t c = blockIdx.x, kvh = blockIdx.y;
  if (c * CH >= ctx) return;  // the whole workgroup
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;

  __shared__ __align__(16) float qs[GQ][LPP][DK + 4];  // rotated queries; padding spreads banks
  __shared__ __align__(16) float ps[NW][PW][GQ];   // exp(s - m) per wave
  __shared__ __align__(16) float s_acc[NW][GQ][HD];
  __shared__ float s_ml[NW][GQ][2];

  // 1. the rotated queries of the group, then the wave's K and V rows (row `pos` was appended by
  // the q/k/v projection); all loads are issued before any value is used, and rows past the
  // context read row 0 and are masked at use
  constexpr int QPT = GQ * HD / NT;  // query elements per thread
  float qv[QPT];
#pragma unroll
  for (int k = 0; k < QPT; ++k) qv[k] = a.q[size_t(kvh * GQ) * HD + tid + NT * k];
  const uint32_t tw0 = c * CH + wave * PW;
  const uint32_t t = tw0 + lane / LPP;
  const int grp = lane % LPP;
  const size_t head = size_t(kvh) * a.max_seq * HD;
  const uint8_t* kc = reinterpret_cast<const uint8_t*>(a.k_cache) + head * E::kBytes;
  const uint8_t* vc = reinterpret_cast<const uint8_t*>(a.v_cache) + head * E::kBytes;
  uint32_t kw[KW];
  {
    const uint32_t tk = t < ctx ? t : 0u;
    const uint8_t* src = kc + (size_t(tk) * HD + grp * DK) * E::kBytes;
#pragma unroll
    for (int i = 0; i < KW / 4; ++i) {
      const uint4 v = ld_u128(src + 16 * i);
      kw[4 * i] = v.x; kw[4 * i + 1] = v.y; kw[4 * i + 2] = v.z; kw[4 * i + 3] = v.w;
    }
  }
  uint32_t vw[PW][VW];
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    const uint32_t tj = tw0 + j < ctx ? tw0 + j : 0u;
    const uint8_t* src = vc + (size_t(tj) * HD + lane * DPL) * E::kBytes;
    if constexpr (VW == 1) {
      vw[j][0] = *reinterpret_cast<const uint32_t*>(src);
    } else if constexpr (VW == 2) {
      const uint2 v = *reinterpret_cast<const uint2*>(src);
      vw[j][0] = v.x; vw[j][1] = v.y;
    } else {
      const uint4 v = ld_u128(src);
      vw[j][0] = v.x; vw[j][1] = v.y; vw[j][2] = v.z; vw[j][3] = v.w;
    }
  }
#pragma unroll
  for (int k = 0; k < QPT; ++k) {
    const int i = tid + NT * k, g = i / HD, d = i % HD;
    qs[g][d / DK][d % DK] = qv[k];
  }
  __syncthreads();

  // 3. scores s = (q . k) * scale over the lane's DK dims, summed over the LPP lanes
  float s[GQ];
#pragma unroll
  for (int g = 0; g < GQ; ++g) s[g] = 0.0f;
#pragma unroll
  for (int r4 = 0; r4 < DK / 4; ++r4) {
    float kf[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) kf[e] = E::get(kw, 4 * r4 + e);
#pragma unroll
    for (int g = 0; g < GQ; ++g) {
      const float4 q4 = *reinterpret_cast<const float4*>(&qs[g][grp][4 * r4]);
      s[g] = fmaf(q4.x, kf[0], s[g]);
      s[g] = fmaf(q4.y, kf[1], s[g]);
      s[g] = fmaf(q4.z, kf[2], s[g]);
      s[g] = fmaf(q4.w, kf[3], s[g]);
    }
  }
  const bool valid = t < ctx;
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
#pragma unroll
    for (int o = 1; o < LPP; o <<= 1) s[g] = pair_sum(s[g], o);
    s[g] = valid ? s[g] * a.scale : -INFINITY;
  }

  // 4. per-wave softmax statistics over the PW positions
  float m_w[GQ], l_w[GQ];
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
    const float m = wave_max(s[g]);
    const float e = valid ? expf(s[g] - m) : 0.0f;
    float l = grp == 0 ? e : 0.0f;
    l = wave_sum(l);
    if (grp == 0) ps[wave][lane / LPP][g] = e;
    m_w[g] = m;
    l_w[g] = l;
  }
  __syncthreads();

  // 5. exp-weighted sum of the V rows over the lane's dims
  float acc[GQ][DPL];
#pragma unroll
  for (int g = 0; g < GQ; ++g)
#pragma unroll
    for (int dd = 0; dd < DPL; ++dd) acc[g][dd] = 0.0f;
#pragma unroll
  for (int j = 0; j < PW; ++j) {
    float p[GQ];
#pragma unroll
    for (int g4 = 0; g4 < GQ / 4; ++g4) {
      const float4 v = *reinterpret_cast<const float4*>(&ps[wave][j][4 * g4]);
      p[4 * g4] = v.x; p[4 * g4 + 1] = v.y; p[4 * g4 + 2] = v.z; p[4 * g4 + 3] = v.w;
    }
    const bool vj = tw0 + j < ctx;
#pragma unroll
    for (int dd = 0; dd < DPL; ++dd) {
      const float v = vj ? E::get(vw[j], dd) : 0.0f;
#pragma unroll
      for (int g = 0; g < GQ; ++g) acc[g][dd] = fmaf(p[g], v, acc[g][dd]);
    }
  }
#pragma unroll
  for (int g = 0; g < GQ; ++g) {
#pragma unroll
    for (int dd = 0; dd < DPL; ++dd) s_acc[wave][g][lane * DPL + dd] = acc[g][dd];
    if (lane == 0) { s_ml[wave][g][0] = m_w[g]; s_ml[wave][g][1] = l_w[g]; }
  }
  __syncthreads();

  // 6. merge the waves; one partial per (query head, chunk)
  const uint32_t nch = a.n_chunks;
  for (int i = tid; i < GQ * HD; i += NT) {
    const int g = i / HD, d = i % HD;
    float M = s_ml[0][g][0];
#pragma unroll
    for (int w = 1; w < NW; ++w) M = fmaxf(M, s_ml[w][g][0]);
    float A = 0.0f, L = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = s_ml[w][g][1] > 0.0f ? expf(s_ml[w][g][0] - M) : 0.0f;
      A = fmaf(s_acc[w][g][d], f, A);
      L = fmaf(s_ml[w][g][1], f, L);
    }
    const size_t hc = size_t(kvh * GQ + g) * nch + c;
    a.part_acc[hc * HD + d] = A;
    if (d == 0) {
      a.part_ml[hc * 2] = M;
      a.part_ml[hc * 2 + 1] = L;
    }
  }
}

// fp16 cache: the same chunk partials computed on the matrix cores.  Per tile of 16 positions a
// wave forms S^T = K . Q^T with v_mfma_f32_16x16x16_f16: A = the 16 K rows, B = 16 query
// columns, of which column h < 8 holds query head h rounded to f16 and column h + 8 the f16
// remainder q - f16(q); adding the two halves of the result (lanes n and n ^ 8) gives the score
// with ~22 bits of the f32 query.  O = P . V likewise: A rows h and h + 8 hold the exp-weights
// of head h as f16 and f16 remainder, B = 16 V columns; rows h and h + 8 of the result are added
// when the waves are merged.  The accumulator layout of the first product (lane n + 16 G holds
// positions 4G..4G+3 of column n) is the operand layout P needs in the second, so the weights
// stay in registers.  Dimension order inside an MFMA is free as long as both operands agree:
// lane group G takes dims [G*HD/4, (G+1)*HD/4) of a K row (one contiguous read), and output
// column n of N-tile j is dim n*HD/16 + j, so a lane's V operand over all N-tiles is one
// contiguous read of the 4-position-blocked V cache.  Exact fp16 products, f32 accumulation.
// QZ > 1 (a block step): the workgroup serves queries QZ blockIdx.z .. + QZ - 1 in turn over the
// K and V rows it loaded once (each query's arithmetic as alone), the next query's rows loaded
// while one is processed.
constexpr int kAttnQz = 8;    // queries per workgroup of a block step's attention (k_attn_mfma)
constexpr int kAttnMqQz = 8;  // the same for k_attn_mq
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ h4_t as_h4(uint32_t lo, uint32_t hi) {
  const u2_t w = {lo, hi};
  return __builtin_bit_cast(h4_t, w);
}
// f16(v) (rem false) or the f16 of the remainder v - f16(v) (rem true), for 4 values
__device__ __forceinline__ h4_t f16_part(float a, float b, float c, float d, bool rem) {
  const h4_t h = {(_Float16)a, (_Float16)b, (_Float16)c, (_Float16)d};
  const h4_t r = {(_Float16)(a - float(h[0])), (_Float16)(b - float(h[1])), (_Float16)(c - float(h[2])),
                  (_Float16)(d - float(h[3]))};
  return rem ? r : h;
}

template <int HD, int GQ, int NW, int T, int QZ>
__global__ void __launch_bounds__(NW * 64) k_attn_mfma(AttnArgs a) {
  constexpr int KD = HD / 4;   // K dims per lane
  constexpr int KS = HD / 16;  // k-steps of the score product
  constexpr int VD = HD / 16;  // V dims per lane = N-tiles of the output product
  constexpr int CH = NW * T * 16, NT = NW * 64;
  static_assert(GQ <= 8 && NW * GQ <= 64 && (NW & (NW - 1)) == 0, "");
  const uint32_t c = blockIdx.x, kvh = blockIdx.y;
  // the queries z0 .. z1 - 1 (positions pos + z); the position is requested first and waited
  // for only after the loads below are issued
  const uint32_t nz = a.nq > 1 ? a.nq : 1u, z0 = blockIdx.z * QZ;
  const uint32_t z1 = QZ == 1 ? z0 + 1 : (z0 + QZ < nz ? z0 + QZ : nz);  // (QZ = 1: grid.z = nz)
  const uint32_t pos0 = a.state->pos;
  const size_t qrows = size_t(a.H) * HD;  // one query's rows of q / out
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = lane >> 4, n = lane & 15, h = n & 7;  // h: the query head of column / row n
  const bool rem = n >= 8;

  __shared__ __align__(16) float s_acc[NW][16][HD + 4];
  __shared__ float s_ml[NW][GQ][2];
  __shared__ float s_f[GQ][NW];

  // 1. loads, all issued before any use and before the position is known: the lane's query
  // dims (head h), K rows (position n of each tile, dims of group G) and V blocks (positions
  // 4G..4G+3 of each tile, dims n*VD..); rows past the context are masked at use
  const uint32_t p0 = c * CH + uint32_t(wave) * T * 16;
  const bool qok = h < GQ;
  // the group's queries are read once per workgroup (QF4 float4 per thread) and shared through
  // LDS: every lane needs 32 of them, and 4 waves reading all their own would quadruple the
  // workgroup's request traffic
  constexpr int QN4 = GQ * HD / 4, QF4 = (QN4 + NT - 1) / NT;
  __shared__ __align__(16) float s_q[GQ * HD];
  float4 qld[QF4];
  auto load_q = [&](uint32_t z) {
#pragma unroll
    for (int k = 0; k < QF4; ++k) qld[k] = ld_f4(a.q + z * qrows + size_t(kvh * GQ) * HD + min(tid + NT * k, QN4 - 1) * 4);
  };
  load_q(z0);
  const uint8_t* kc = reinterpret_cast<const uint8_t*>(a.k_cache) + size_t(kvh) * a.max_seq * HD * 2;
  const uint8_t* vc = reinterpret_cast<const uint8_t*>(a.v_cache) + size_t(kvh) * a.max_seq * HD * 2;
  uint4 kf[T][KD / 8], vf[T][VD / 2];
#pragma unroll
  for (int t = 0; t < T; ++t) {
    const uint32_t pk = p0 + t * 16 + n;
    const uint8_t* ks = kc + (size_t(min(pk, a.max_seq - 1)) * HD + G * KD) * 2;
#pragma unroll
    for (int i = 0; i < KD / 8; ++i) kf[t][i] = ld_u128(ks + 16 * i);
    const uint32_t pb = p0 + t * 16 + 4 * G;  // first position of the lane's V block
    const uint8_t* vs = vc + (size_t(min(pb, a.max_seq - 4)) * HD + n * VD * 4) * 2;
#pragma unroll
    for (int i = 0; i < VD / 2; ++i) vf[t][i] = ld_u128(vs + 16 * i);
  }
  // keep every load above this point: the scheduler would otherwise sink the V loads next to
  // the P.V products, after the softmax
  __builtin_amdgcn_sched_barrier(0);
  for (uint32_t z = z0; z < z1; ++z) {
  const uint32_t pos = pos0 + z, ctx = pos + 1;
  if (z != z0) __syncthreads();  // (the previous query's LDS reads are done)
#pragma unroll
  for (int k = 0; k < QF4; ++k)
    if (tid + NT * k < QN4) *reinterpret_cast<float4*>(&s_q[(tid + NT * k) * 4]) = qld[k];
  __syncthreads();
  if (c * CH >= ctx) {  // the whole workgroup (a later query may reach the chunk)
    if (QZ > 1 && z + 1 < z1) load_q(z + 1);
    continue;
  }
  float* const part_ml = a.part_ml + size_t(z) * a.H * a.n_chunks * 2;
  float* const part_acc = a.part_acc + size_t(z) * a.H * a.n_chunks * HD;

  // 2. the query operand (zero for heads past the group); the next query's rows are loaded
  const float* qsrc = s_q + (qok ? h : 0) * HD + G * KD;
  float4 qv[KD / 4];
#pragma unroll
  for (int i = 0; i < KD / 4; ++i) qv[i] = *reinterpret_cast<const float4*>(qsrc + 4 * i);
  if (QZ > 1 && z + 1 < z1) load_q(z + 1);
  h4_t qb[KS];
#pragma unroll
  for (int st = 0; st < KS; ++st) {
    const float4 v = qok ? qv[st] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    qb[st] = f16_part(v.x, v.y, v.z, v.w, rem);
  }

  // 3. scores: lane (G, n) gets head h at positions 4G + i of each tile (lanes n and n ^ 8 alike)
  float sc[T][4];
  float m = -INFINITY;
#pragma unroll
  for (int t = 0; t < T; ++t) {
    f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int st = 0; st < KS; ++st) {
      const uint4 w = kf[t][st / 2];
      const h4_t kk = (st & 1) ? as_h4(w.z, w.w) : as_h4(w.x, w.y);
      acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kk, qb[st], acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float s = pair_sum(acc[i], 8);
      const bool ok = p0 + t * 16 + 4 * G + i < ctx;
      sc[t][i] = ok ? s * a.scale : -INFINITY;
      m = fmaxf(m, sc[t][i]);
    }
  }
  m = pair_max(pair_max(m, 16), 32);

  // 4. exp-weights and their sum per head; O = P . V
  float l = 0.0f;
  f4_t o[VD];
#pragma unroll
  for (int j = 0; j < VD; ++j) o[j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int t = 0; t < T; ++t) {
    float e[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      e[i] = sc[t][i] > -INFINITY ? expf(sc[t][i] - m) : 0.0f;
      l += e[i];
    }
    const h4_t pa = f16_part(e[0], e[1], e[2], e[3], rem);
    // V rows past the context hold stale or zero rows: zeroed, so that 0 * (non-finite) cannot
    // reach the sums (e = 0 there already)
    const uint32_t pb = p0 + t * 16 + 4 * G;
    const uint32_t mlo = (pb < ctx ? 0xffffu : 0u) | (pb + 1 < ctx ? 0xffff0000u : 0u);
    const uint32_t mhi = (pb + 2 < ctx ? 0xffffu : 0u) | (pb + 3 < ctx ? 0xffff0000u : 0u);
#pragma unroll
    for (int j = 0; j < VD; ++j) {
      const uint4 w0 = vf[t][j / 2];
      const uint4 w = make_uint4(w0.x & mlo, w0.y & mhi, w0.z & mlo, w0.w & mhi);
      const h4_t vv = (j & 1) ? as_h4(w.z, w.w) : as_h4(w.x, w.y);
      o[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, vv, o[j], 0, 0, 0);
    }
  }
  l = pair_sum(pair_sum(l, 16), 32);

  // 5. the wave's statistics and sums to LDS (lane (G, n) holds rows 4G + i, dims n*VD + j)
  if (G == 0 && n < GQ) {
    s_ml[wave][n][0] = m;
    s_ml[wave][n][1] = l;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < VD; j += 4)
      *reinterpret_cast<float4*>(&s_acc[wave][4 * G + i][n * VD + j]) =
          make_float4(o[j][i], o[j + 1][i], o[j + 2][i], o[j + 3][i]);
  __syncthreads();

  // 6. the waves' rescale factors exp(m_w - M) and the chunk statistics (M, L), per head: thread
  // g*NW + w of the first wave
  const uint32_t nch = a.n_chunks;
  if (tid < NW * GQ) {
    const int g = tid / NW, w = tid % NW;
    const float mw = s_ml[w][g][0], lw = s_ml[w][g][1];
    float M = mw;
#pragma unroll
    for (int o2 = 1; o2 < NW; o2 <<= 1) M = pair_max(M, o2);
    const float f = lw > 0.0f ? expf(mw - M) : 0.0f;
    float L = lw * f;
#pragma unroll
    for (int o2 = 1; o2 < NW; o2 <<= 1) L = pair_sum(L, o2);
    s_f[g][w] = f;
    if (w == 0) {
      const size_t hc = size_t(kvh * GQ + g) * nch + c;
      part_ml[hc * 2] = M;
      part_ml[hc * 2 + 1] = L;
    }
  }
  __syncthreads();

  // 7. merge the waves (rows h and h + 8 of each wave); one partial per (query head, chunk)
  for (int i = tid; i < GQ * HD; i += NT) {
    const int g = i / HD, d = i % HD;
    float A = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) A = fmaf(s_acc[w][g][d] + s_acc[w][g + 8][d], s_f[g][w], A);
    part_acc[(size_t(kvh * GQ + g) * nch + c) * HD + d] = A;
  }
  }  // (query z)
}

// A block step of more than 8 queries (the prefill), fp16 cache, head dim 128, 8 query heads per
// kv head: workgroup (chunk c of 128 positions, kv head, QZ queries).  The chunk's K rows and V
// blocks are staged in LDS once; wave w then takes queries w, w + 4, ... of the QZ, each over all
// 128 positions with k_attn_mfma's arithmetic and operand layouts (the operands read from LDS:
// eight 16-position tiles per wave), and writes that query's chunk partial (max, sum, weighted V
// sum) itself: the wave covers the chunk, so there is no merge over waves and no barrier per
// query.  Rows h and h + 8 of the output product (the f16 weights and their remainders of head h)
// sit in lanes G and G + 2: one lane exchange adds them.
template <int QZ>
__global__ void __launch_bounds__(256) k_attn_mq(AttnArgs a) {
  constexpr int HD = 128, GQ = 8, CH = 128, NT = CH / 16;
  constexpr int KD = HD / 4, KS = HD / 16, VD = HD / 16;
  constexpr int KROW = HD * 2 + 16;  // LDS bytes per K row (16 B of padding: a read's 16 rows on distinct banks)
  static_assert(QZ % 4 == 0, "");
  __shared__ __align__(16) uint8_t s_k[CH * KROW];
  __shared__ __align__(16) uint8_t s_v[CH * HD * 2];  // [CH/4][HD][4] f16, as the cache holds it
  const uint32_t c = blockIdx.x, kvh = blockIdx.y, p0 = c * CH;
  const uint32_t nz = a.nq > 1 ? a.nq : 1u, z0 = blockIdx.z * QZ;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int G = lane >> 4, n = lane & 15, h = n & 7;
  const bool rem = n >= 8;
  const uint8_t* kc = reinterpret_cast<const uint8_t*>(a.k_cache) + size_t(kvh) * a.max_seq * HD * 2;
  const uint8_t* vc = reinterpret_cast<const uint8_t*>(a.v_cache) + size_t(kvh) * a.max_seq * HD * 2;
  // 1. the chunk: K rows (16 threads per 256-byte row) and V blocks (64 threads per 1 KB block of
  // 4 positions); rows past the cache repeat its last row / block and are masked at use
  {
    uint4 kv[8], vv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t e = uint32_t(tid) + 256u * uint32_t(i), row = e / 16, col = e % 16;
      const uint32_t pk = p0 + row < a.max_seq ? p0 + row : a.max_seq - 1;
      kv[i] = ld_u128(kc + size_t(pk) * HD * 2 + col * 16);
      const uint32_t blk = e / 64, piece = e % 64;
      const uint32_t pb = p0 + 4 * blk < a.max_seq - 3 ? p0 + 4 * blk : a.max_seq - 4;
      vv[i] = ld_u128(vc + size_t(pb) * HD * 2 + piece * 16);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      const uint32_t e = uint32_t(tid) + 256u * uint32_t(i);
      *reinterpret_cast<uint4*>(s_k + (e / 16) * KROW + (e % 16) * 16) = kv[i];
      *reinterpret_cast<uint4*>(s_v + e * 16) = vv[i];
    }
  }
  const uint32_t pos0 = a.state->pos;
  __syncthreads();
  // 2. the wave's queries (no barrier below: a wave leaves on its own)
  for (int k = 0; k < QZ / 4; ++k) {
    const uint32_t z = z0 + uint32_t(wave) + 4u * uint32_t(k);
    if (z >= nz) break;
    const uint32_t ctx = pos0 + z + 1;
    if (p0 >= ctx) continue;  // (a later query may reach the chunk)
    const float* qsrc = a.q + size_t(z) * a.H * HD + size_t(kvh * GQ + h) * HD + G * KD;
    float4 qv[KD / 4];
#pragma unroll
    for (int i = 0; i < KD / 4; ++i) qv[i] = ld_f4(qsrc + 4 * i);
    h4_t qb[KS];
#pragma unroll
    for (int st = 0; st < KS; ++st) qb[st] = f16_part(qv[st].x, qv[st].y, qv[st].z, qv[st].w, rem);
    // scores: lane (G, n) gets head h at positions 4G + i of each tile
    float sc[NT][4];
    float m = -INFINITY;
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      f4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
      const uint8_t* kr = s_k + (t * 16 + n) * KROW + G * KD * 2;
#pragma unroll
      for (int st = 0; st < KS; ++st) {
        const uint4 w = *reinterpret_cast<const uint4*>(kr + 16 * (st / 2));
        const h4_t kk = (st & 1) ? as_h4(w.z, w.w) : as_h4(w.x, w.y);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(kk, qb[st], acc, 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float sv = pair_sum(acc[i], 8);
        const bool ok = p0 + t * 16 + 4 * G + i < ctx;
        sc[t][i] = ok ? sv * a.scale : -INFINITY;
        m = fmaxf(m, sc[t][i]);
      }
    }
    m = pair_max(pair_max(m, 16), 32);
    // exp-weights, their sum per head; O = P . V
    float l = 0.0f;
    f4_t o[VD];
#pragma unroll
    for (int j = 0; j < VD; ++j) o[j] = f4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < NT; ++t) {
      float e[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        e[i] = sc[t][i] > -INFINITY ? expf(sc[t][i] - m) : 0.0f;
        l += e[i];
      }
      const h4_t pa = f16_part(e[0], e[1], e[2], e[3], rem);
      // V rows past the context hold stale or zero rows: zeroed, so that 0 * (non-finite) cannot
      // reach the sums (e = 0 there already)
      const uint32_t pb = p0 + t * 16 + 4 * G;
      const uint32_t mlo = (pb < ctx ? 0xffffu : 0u) | (pb + 1 < ctx ? 0xffff0000u : 0u);
      const uint32_t mhi = (pb + 2 < ctx ? 0xffffu : 0u) | (pb + 3 < ctx ? 0xffff0000u : 0u);
      const uint8_t* vr = s_v + size_t(t * 4 + G) * HD * 8 + n * VD * 8;
#pragma unroll
      for (int j = 0; j < VD; ++j) {
        const uint4 w0 = *reinterpret_cast<const uint4*>(vr + 16 * (j / 2));
        const uint4 w = make_uint4(w0.x & mlo, w0.y & mhi, w0.z & mlo, w0.w & mhi);
        const h4_t vv = (j & 1) ? as_h4(w.z, w.w) : as_h4(w.x, w.y);
        o[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(pa, vv, o[j], 0, 0, 0);
      }
    }
    l = pair_sum(pair_sum(l, 16), 32);
    // 3. the chunk partial of query z: (max, sum) per head, and the weighted V sums of rows h and
    // h + 8 added (lanes G and G + 2: lanes G < 2 hold heads 4 G + i, dims n VD + j)
    const uint32_t nch = a.n_chunks;
    float* const part_ml = a.part_ml + size_t(z) * a.H * nch * 2;
    float* const part_acc = a.part_acc + size_t(z) * a.H * nch * HD;
    if (G == 0 && n < GQ) {
      const size_t hc = size_t(kvh * GQ + n) * nch + c;
      part_ml[hc * 2] = m;
      part_ml[hc * 2 + 1] = l;
    }
#pragma unroll
    for (int j = 0; j < VD; ++j)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[j][i] = pair_sum(o[j][i], 32);
    if (G < 2) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float* dst = part_acc + (size_t(kvh * GQ + 4 * G + i) * nch + c) * HD + n * VD;
        *reinterpret_cast<float4*>(dst) = make_float4(o[0][i], o[1][i], o[2][i], o[3][i]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(o[4][i], o[5][i], o[6][i], o[7][i]);
      }
    }
  }
}

// out[h][d] = sum_c A_c[d] w_c / sum_c L_c w_c, w_c = exp(M_c - M), over the active chunks.  One
// wave per (head, 64 dims): lane d of dims block y.  The chunk statistics are spread over the
// lanes (chunk lane + 64 k), the weights go through LDS (w_c = 0 past the active chunks, whose
// sums are read at chunk 0 and so contribute exactly 0), and every load of a batch of 32
// chunks is issued before its use.
// The merge: one workgroup of kMergeWaves waves per (query head, 64 output dims).  Wave w sums
// the chunks w, w + 4, ... (every load issued before the position is known; chunks past the
// context are masked), the waves' sums meet in LDS in wave order.  Every wave forms the chunk
// weights exp(m_c - M) itself from the chunk statistics (no barrier before the sums).
constexpr uint32_t kMergeWaves = 4;
template <int HD>
__global__ void __launch_bounds__(64 * kMergeWaves) k_attn_merge(AttnArgs a0) {
  const AttnArgs a = attn_query(a0);
  constexpr uint32_t KC = (kAttnMaxChunks + 63) / 64, B = 32;
  const uint32_t CH = a0.chunk;
  static_assert(kAttnMaxChunks % 4 == 0, "");
  __shared__ __align__(16) float s_w[KC * 64];
  __shared__ float s_o[kMergeWaves][64];
  const uint32_t h = blockIdx.x, lane = threadIdx.x & 63, d = blockIdx.y * 64 + lane;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t pos = a.state->pos + blockIdx.z, nch = a.n_chunks;
  const float* ml = a.part_ml + size_t(h) * nch * 2;
  const float* acc = a.part_acc + size_t(h) * nch * HD + d;
  float mv[KC], lv[KC], av[B];
#pragma unroll
  for (uint32_t k = 0; k < KC; ++k) {
    const uint32_t cc = lane + 64 * k, cl = cc < nch ? cc : 0u;
    mv[k] = ml[2 * cl];
    lv[k] = ml[2 * cl + 1];
  }
#pragma unroll
  for (uint32_t k = 0; k < B; ++k) {
    const uint32_t cc = wave + kMergeWaves * k;
    av[k] = acc[size_t(cc < nch ? cc : 0u) * HD];
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t n_act = (pos + CH) / CH;
  float M = -INFINITY;
#pragma unroll
  for (uint32_t k = 0; k < KC; ++k) M = fmaxf(M, lane + 64 * k < n_act ? mv[k] : -INFINITY);
  M = wave_max(M);
  float L = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k < KC; ++k) {
    const bool ok = lane + 64 * k < n_act;
    const float w = ok ? expf(mv[k] - M) : 0.0f;
    s_w[lane + 64 * k] = w;  // every wave writes the same values
    L = fmaf(ok ? lv[k] : 0.0f, w, L);
  }
  L = wave_sum(L);
  __syncthreads();
  float o = 0.0f;
  for (uint32_t c0 = 0; c0 * kMergeWaves < n_act; c0 += B) {
    if (c0 > 0) {  // longer contexts: further batches
#pragma unroll
      for (uint32_t k = 0; k < B; ++k) {
        const uint32_t cc = wave + kMergeWaves * (c0 + k);
        av[k] = acc[size_t(cc < n_act ? cc : 0u) * HD];
      }
    }
#pragma unroll
    for (uint32_t k = 0; k < B; ++k) {  // branch-free: every weight is read, the unused ones masked
      const uint32_t cc = wave + kMergeWaves * (c0 + k);
      const bool ok = cc < n_act;
      const float wv = s_w[ok ? cc : 0u];
      o = fmaf(ok ? av[k] : 0.0f, ok ? wv : 0.0f, o);
    }
  }
  s_o[wave][lane] = o;
  __syncthreads();
  if (wave == 0) {
#pragma clang fp contract(off)
    float v = ((s_o[0][lane] + s_o[1][lane]) + (s_o[2][lane] + s_o[3][lane])) / L;
    if (a.gate) {  // the hybrid's output gate: the merged value times sigmoid(g)
      const float g = a.gate[size_t(blockIdx.z) * 2 * a.H * HD + size_t(h) * 2 * HD + HD + d];
      v = v * (1.0f / (1.0f + expf(-g)));
    }
    a.out[size_t(h) * HD + d] = v;
  }
}

}  // namespace

void launch_attention_partial(const AttnArgs& a, hipStream_t st) {
  const uint32_t nq = a.nq > 1 ? a.nq : 1;
  const dim3 grid(a.n_chunks, a.KV, nq);
  // fp16 cache, a block of more than 8 queries (the prefill): kAttnQz queries per workgroup over
  // one load of its K / V rows (the verify's few queries run in parallel workgroups)
  const bool mq = a.kv_f16 && nq > kSmallBlock;
  const dim3 grid_mq(a.n_chunks, a.KV, (nq + kAttnQz - 1) / kAttnQz);
  const uint32_t gq = a.H / a.KV;
  // (the chunk size a.chunk = attn_chunk(hd, KV) picks the instance: CH = waves x positions)
  if (a.hd == 128 && gq == 8 && a.chunk == 128) {  // fp16: 4 waves x 2 tiles; f32: 8 waves x 16 positions
    if (mq) launch_kernel(&k_attn_mq<kAttnMqQz>, dim3(a.n_chunks, a.KV, (nq + kAttnMqQz - 1) / kAttnMqQz), dim3(256), st, a);
    else if (a.kv_f16) launch_kernel(&k_attn_mfma<128, 8, 4, 2, 1>, grid, dim3(256), st, a);
    else launch_kernel(&k_attn_chunk<128, 8, float, 4, 8>, grid, dim3(512), st, a);
  } else if (a.hd == 128 && gq == 8) {  // 64: fp16 4 waves x 1 tile; f32 4 waves x 16 positions, 4 lanes per K row
    if (mq) launch_kernel(&k_attn_mfma<128, 8, 4, 1, kAttnQz>, grid_mq, dim3(256), st, a);
    else if (a.kv_f16) launch_kernel(&k_attn_mfma<128, 8, 4, 1, 1>, grid, dim3(256), st, a);
    else launch_kernel(&k_attn_chunk<128, 8, float, 4, 4>, grid, dim3(256), st, a);
  } else if (a.hd == 256 && gq == 4) {  // fp16: 2 waves x 1 tile; f32: 2 waves x 16 positions
    if (mq) launch_kernel(&k_attn_mfma<256, 4, 2, 1, kAttnQz>, grid_mq, dim3(128), st, a);
    else if (a.kv_f16) launch_kernel(&k_attn_mfma<256, 4, 2, 1, 1>, grid, dim3(128), st, a);
    else launch_kernel(&k_attn_chunk<256, 4, float, 4, 2>, grid, dim3(128), st, a);
  }
}

void launch_attention_combine(const AttnArgs& a, hipStream_t st) {
  const uint32_t nq = a.nq > 1 ? a.nq : 1;
  if (a.hd == 128) launch_kernel(&k_attn_merge<128>, dim3(a.H, 2, nq), dim3(64 * kMergeWaves), st, a);
  else launch_kernel(&k_attn_merge<256>, dim3(a.H, 4, nq), dim3(64 * kMergeWaves), st, a);
}

bool attention_supported(uint32_t H, uint32_t KV, uint32_t hd) {
  return KV > 0 && H % KV == 0 && ((hd == 128 && H / KV == 8) || (hd == 256 && H / KV == 4));
}

void launch_attention(const AttnArgs& a, hipStream_t st) {
  launch_attention_partial(a, st);
  launch_attention_combine(a, st);
}

// ---- the decode attention on caller buffers with no allocation ------------------------------
// The chunk kernels' partials (max and sum per chunk and query head, and the weighted V rows)
// and the position they read live in `scratch`, a file-scope device array: each GPU holds its
// own copy.  Host code never passes the array's name to a kernel (on the host it is a stand-in,
// not a device address): the device address of each GPU's copy is looked up once, with that
// device current, and kept in g_scratch_ptr.
namespace {

__device__ __align__(256) uint8_t scratch[kAttnScratchBytes];

constexpr int kMaxDevices = 64;
void* g_scratch_ptr[kMaxDevices] = {};
std::once_flag g_scratch_once[kMaxDevices];
hipError_t g_scratch_err[kMaxDevices] = {};

__global__ void k_set_position(StepState* st, uint32_t pos) {
  StepState s{};
  s.pos = pos;
  *st = s;
}

}  // namespace

// device address of this GPU's scratch array (null when the lookup failed)
static void* scratch_on_current_device() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  std::call_once(g_scratch_once[dev], [dev] {
    void* p = nullptr;
    g_scratch_err[dev] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (g_scratch_err[dev] == hipSuccess) g_scratch_ptr[dev] = p;
  });
  return g_scratch_ptr[dev];
}

}  // namespace chpe

using namespace chpe;

extern "C" int chpe_attention_noalloc(uint32_t head_dim, uint32_t heads, uint32_t kv_heads, int kv_f16,
                                      uint32_t pos, uint32_t max_seq, const float* q, const void* k_cache,
                                      const void* v_cache, float* out, void* stream) {
  if (!q || !k_cache || !v_cache || !out || !attention_supported(heads, kv_heads, head_dim)) return -1;
  if (max_seq == 0 || max_seq % 16 != 0 || pos >= max_seq) return -1;
  const uint32_t chunk = attn_chunk(head_dim, kv_heads), n_chunks = (pos + chunk) / chunk;
  const size_t ml = size_t(heads) * n_chunks * 2 * 4, acc = size_t(heads) * n_chunks * head_dim * 4;
  // the position, then the two partial arrays, each at a 256-byte boundary
  const size_t off_ml = 256, off_acc = off_ml + (ml + 255) / 256 * 256;
  if (n_chunks > kAttnMaxChunks || off_acc + acc > kAttnScratchBytes) return -2;
  uint8_t* base = static_cast<uint8_t*>(scratch_on_current_device());
  if (!base) return -3;
  hipStream_t st = static_cast<hipStream_t>(stream);
  StepState* state = reinterpret_cast<StepState*>(base);
  hipLaunchKernelGGL(k_set_position, dim3(1), dim3(1), 0, st, state, pos);
  AttnArgs a{};
  a.state = state;
  a.q = q;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.out = out;
  a.part_ml = reinterpret_cast<float*>(base + off_ml);
  a.part_acc = reinterpret_cast<float*>(base + off_acc);
  a.H = heads;
  a.KV = kv_heads;
  a.hd = head_dim;
  a.max_seq = max_seq;
  a.n_chunks = n_chunks;
  a.chunk = chunk;
  a.kv_f16 = kv_f16 ? 1 : 0;
  a.scale = 1.0f / std::sqrt(float(head_dim));
  launch_attention(a, st);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}
