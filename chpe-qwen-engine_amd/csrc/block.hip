// block.hip -- the block step's GEMV: m <= kMaxBlock tokens at consecutive positions through
// flat 4-bit tiles (gemvCellFlat, chpe_engine.zig:584-729), every weight read once for all of
// them.  Used by the batch-M verify and by the chunked prefill; each token's arithmetic is the
// batch-1 step's (forwardDecode :1663-1803).
//
// 1. k_block_limbs: per token the GEMV input (RMS-normalised, (x * inv) * gamma, rmsNorm
//    :187-191, when gamma is set) as exact integers per 128-column group, X = x * 2^(30-e) with
//    max |x| < 2^e, in four signed-byte limbs -- the operand tables of the matrix cores.
// 2. k_gemv_mt: a workgroup owns one range of 2048 input columns (its tables staged in LDS) and
//    strides over units of 16 weight rows.  Per group a wave runs, for each quad of tokens, two
//    v_mfma_i32_16x16x64_i8 with
//      A (16 x 64): row 4 t + L = limb L of token t of the quad (one half of the group),
//      B (64 x 16): column n = weight row n of the unit (the same half, codes as bytes),
//    so lane (n, q) holds D(4 q + j, n): token q, limb j, row n -- the exact integer sum of
//    code * limb over the group, starting at -8 * (the limb's sum) for the codes' offset.  The
//    lane combines its 4 limbs (2^(8 j)), scales by 2^(e - 30) and by the row's group scale,
//    and accumulates row n of token q over the range's groups; the raw row sums of each range
//    go to a partial-sum buffer.  Lane (n, q) loads 16 bytes of row n per group (quarter q), the
//    next item's loads are issued before the current item's products.
// 3. k_block_epi: per output row the ranges' sums in a fixed order, the flat-tile outlier
//    corrections ((w_out - dequantised code) * x[col], outliers replace weights :632-646) over
//    16 lanes, and the batch-1 step's epilogue per token: bias, residual, SwiGLU, RoPE at the
//    token's position with the K/V append, or logits with per-token argmax partials.
#include <cstdio>

#include "device_common.hpp"
#include "kernels.hpp"

namespace chpe {
namespace {
using namespace dev;

template <bool kNorm>
__global__ void __launch_bounds__(1024) k_block_limbs(const float* X, const float* gamma, float eps, uint32_t C,
                                                       uint32_t m, BlockTables t) {
  const uint32_t tok = blockIdx.x, T = tok >> 2, tl = tok & 3u, ng = C >> 7;
  const bool live = tok < m;
  const float* x = X + size_t(live ? tok : 0u) * C;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ float s_red[16];
  float ss = 0.0f;
  for (uint32_t c = uint32_t(tid); c < C; c += 1024) {
    const float v = x[c];
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if (lane == 0) s_red[wave] = ss;
  __syncthreads();
  float tot = 0.0f;
#pragma unroll
  for (int w = 0; w < 16; ++w) tot += s_red[w];
  if (tid == 0) t.ss[tok] = live ? tot : 0.0f;
  const float inv = kNorm ? 1.0f / sqrtf(tot / float(C) + eps) : 1.0f;
  uint2* tb2 = reinterpret_cast<uint2*>(t.tb);
  const uint32_t passes = (ng * 128 + 8 * 1024 - 1) / (8 * 1024);
  for (uint32_t ps = 0; ps < passes; ++ps) {  // the same trip count on every lane (DPP below)
    const uint32_t c0 = 8 * (uint32_t(tid) + 1024 * ps);
    const bool in = c0 < ng * 128;
    const uint32_t cc = in ? c0 : 0u;
    const float4 xa = ld_f4(x + cc), xb = ld_f4(x + cc + 4);
    float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
    if constexpr (kNorm) {
      const float4 ga = ld_f4(gamma + cc), gb = ld_f4(gamma + cc + 4);
      const float gv[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
      for (int i = 0; i < 8; ++i) xv[i] = (xv[i] * inv) * gv[i];
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xv[i] = (live && in) ? xv[i] : 0.0f;
      mx = fmaxf(mx, fabsf(xv[i]));
    }
    mx = pair_max(mx, 1);
    mx = pair_max(mx, 2);
    mx = pair_max(mx, 4);
    mx = pair_max(mx, 8);
    int e = 0;
    (void)frexpf(mx, &e);  // mx < 2^e (mx = 0: e = 0)
    const float up = ldexpf(1.0f, 30 - e);
    uint32_t z[8];  // bytes: the balanced limbs of X
#pragma unroll
    for (int i = 0; i < 8; ++i) z[i] = (uint32_t(int(xv[i] * up)) + 0x808080u) ^ 0x808080u;
    uint32_t lo[4], hi[4];
    limb_words(z[0], z[2], z[4], z[6], lo);
    limb_words(z[1], z[3], z[5], z[7], hi);
    const uint32_t g = cc >> 7, c = cc & 127u, kq = c >> 5, h = (c >> 4) & 1u, p = (c >> 3) & 1u;
    int sums[4];
#pragma unroll
    for (int L = 0; L < 4; ++L) {
      if (in)
        tb2[((((size_t(T) * ng + g) * 4 + kq) * 2 + h) * 16 + (4 * tl + uint32_t(L))) * 2 + p] = make_uint2(lo[L], hi[L]);
      int sl = __builtin_amdgcn_sdot4(int(lo[L]), 0x01010101, __builtin_amdgcn_sdot4(int(hi[L]), 0x01010101, 0, false), false);
      sl += int(pair_u(uint32_t(sl), 1));
      sl += int(pair_u(uint32_t(sl), 2));
      sl += int(pair_u(uint32_t(sl), 4));
      sl += int(pair_u(uint32_t(sl), 8));
      sums[L] = sl;
    }
    if (in && c == 0) {
      t.ci[(size_t(T) * ng + g) * 4 + tl] = make_int4(-8 * sums[0], -8 * sums[1], -8 * sums[2], -8 * sums[3]);
      t.ew[(size_t(T) * ng + g) * 4 + tl] = isfinite(mx) ? ldexpf(1.0f, e - 30) : __int_as_float(0x7fc00000);
    }
    if (in) {
#pragma unroll
      for (int i = 0; i < 8; ++i) t.xt[size_t(cc + uint32_t(i)) * kMaxBlock + tok] = xv[i];
    }
  }
}

struct MtItem {
  uint4 q[4];      // codes of row n, groups 4 S .. 4 S + 3 of the range, quarter q
  uint32_t s[4];   // their group scales
};

template <int NQ, int NW>
__global__ void __launch_bounds__(kWave * NW) k_gemv_mt(BlockGemvArgs a) {
  __shared__ __align__(16) uint4 s_tb[NQ][16][128];
  __shared__ __align__(16) int4 s_ci[NQ][16][4];
  __shared__ float s_ew[NQ][16][4];
  const int lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t C = a.g.C, ng = C >> 7, range = blockIdx.x, g0 = range * 16;
  const uint32_t ngr = ng - g0 < 16u ? ng - g0 : 16u;
  // the range's operands (zero past the input)
  for (uint32_t i = threadIdx.x; i < uint32_t(NQ) * 16 * 128; i += kWave * NW) {
    const uint32_t T = i >> 11, gl = (i >> 7) & 15u, e = i & 127u;
    s_tb[T][gl][e] = gl < ngr ? a.t.tb[(size_t(T) * ng + g0 + gl) * 128 + e] : make_uint4(0, 0, 0, 0);
  }
  for (uint32_t i = threadIdx.x; i < uint32_t(NQ) * 16 * 4; i += kWave * NW) {
    const uint32_t T = i >> 6, gl = (i >> 2) & 15u, k = i & 3u;
    const bool ok = gl < ngr;
    s_ci[T][gl][k] = ok ? a.t.ci[(size_t(T) * ng + g0 + gl) * 4 + k] : make_int4(0, 0, 0, 0);
    s_ew[T][gl][k] = ok ? a.t.ew[(size_t(T) * ng + g0 + gl) * 4 + k] : 0.0f;
  }
  __syncthreads();

  const uint32_t n_units = a.n_units, waves_total = gridDim.y * NW;
  const uint32_t wid = blockIdx.y * NW + wave;
  if (wid >= n_units) return;  // (no barrier follows)
  // the unit's part: parts hold consecutive unit ranges from part[p].unit_begin
  auto part_index = [&](uint32_t u) {
    int p = 0;
#pragma unroll
    for (int k = 1; k < kMaxParts; ++k) p += (k < a.g.n_parts && u >= a.g.part[k].unit_begin) ? 1 : 0;
    return p;
  };
  auto issue = [&](uint32_t u, uint32_t S, MtItem* it) {
    const int p = int(__builtin_amdgcn_readfirstlane(part_index(u)));
    const GemvPart& P = a.g.part[p];
    const uint8_t* base = P.base;
    const uint32_t stride = P.stride, wr = P.wrows;
    const uint32_t r = (u - P.unit_begin) * 16 + uint32_t(n), rr = r < wr ? r : 0u;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t k = 4 * S + uint32_t(s);
      const uint32_t G = rr * ng + g0 + (k < ngr ? k : 0u);
      const uint32_t off = (G >> 8) * stride;
      it->q[s] = ld_u128(base + (off + 64 + (G & 255u) * 64 + 16 * uint32_t(q)));
      it->s[s] = ld_u16(base + (off + 16448 + 48 + 2 * (G & 255u)));
    }
  };
  float acc[NQ];
#pragma unroll
  for (int T = 0; T < NQ; ++T) acc[T] = 0.0f;
  auto compute = [&](uint32_t u, uint32_t S, const MtItem& it) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      const uint32_t k = 4 * S + uint32_t(s);
      const bool gv = k < ngr;
      const uint32_t kk = gv ? k : 0u;
      const uint32_t w4[4] = {it.q[s].x, it.q[s].y, it.q[s].z, it.q[s].w};
      const float sc = h2f(uint16_t(it.s[s]));
#pragma unroll
      for (int T = 0; T < NQ; ++T) {
        const int4 c4 = s_ci[T][kk][q];
        i32x4_t D = {c4.x, c4.y, c4.z, c4.w};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint4 t = s_tb[T][kk][(uint32_t(q) * 2 + uint32_t(h)) * 16 + uint32_t(n)];
          const i32x4_t A = {int(t.x), int(t.y), int(t.z), int(t.w)};
          const uint32_t w0 = w4[2 * h], w1 = w4[2 * h + 1];
          const i32x4_t B = {int(w0 & 0x0f0f0f0fu), int((w0 >> 4) & 0x0f0f0f0fu), int(w1 & 0x0f0f0f0fu),
                             int((w1 >> 4) & 0x0f0f0f0fu)};
          D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, D, 0, 0, 0);
        }
        const float f = ((float(D[0]) + float(D[1]) * 256.0f) + float(D[2]) * 65536.0f) + float(D[3]) * 16777216.0f;
        const float v = f * s_ew[T][kk][q] * sc;
        acc[T] += gv ? v : 0.0f;
      }
    }
    if (S == 3) {  // the unit's last set: row n of tokens 4 T + q
      const int p = int(__builtin_amdgcn_readfirstlane(part_index(u)));
      const GemvPart& P = a.g.part[p];
      const uint32_t r = (u - P.unit_begin) * 16 + uint32_t(n);
      const uint32_t at = P.unit_begin * 16 + (u - P.unit_begin) * 16 + uint32_t(n);
#pragma unroll
      for (int T = 0; T < NQ; ++T) {
        const uint32_t tk = 4 * uint32_t(T) + uint32_t(q);
        if (tk < a.m) a.partial[(size_t(range) * kMaxBlock + tk) * a.rows_all + at] = r < P.wrows ? acc[T] : 0.0f;
        acc[T] = 0.0f;
      }
    }
  };
  // items (unit, set of 4 groups); the next item's loads before the current item's products (a
  // repeat of the last item past the end: its lines are cached)
  uint32_t u0 = wid, S0 = 0;
  MtItem IA, IB;
  issue(u0, S0, &IA);
  while (true) {
    const uint32_t u1 = S0 < 3 ? u0 : u0 + waves_total, S1 = S0 < 3 ? S0 + 1 : 0u;
    const bool v1 = u1 < n_units;
    issue(v1 ? u1 : u0, v1 ? S1 : S0, &IB);
    compute(u0, S0, IA);
    if (!v1) break;
    const uint32_t u2 = S1 < 3 ? u1 : u1 + waves_total, S2 = S1 < 3 ? S1 + 1 : 0u;
    const bool v2 = u2 < n_units;
    issue(v2 ? u2 : u1, v2 ? S2 : S1, &IA);
    compute(u1, S1, IB);
    if (!v2) break;
    u0 = u2;
    S0 = S2;
  }
}

// Epilogue: a wave serves 4 outputs (16 lanes each: lane (i, e) = output i, correction entries
// e, e + 16, ..; after the 16-lane reduction lane (i, t) finishes token t of output i).
// Outputs: rows of part 0 (Store / Accum / Logits), gate row = up row (SwiGlu), RoPE pairs of
// every part (QkvRope).
template <int MODE>
__global__ void __launch_bounds__(256) k_block_epi(BlockGemvArgs a) {
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr int NR = (kSwi || kRope) ? 2 : 1;  // rows per output
  const int lane = threadIdx.x & 63, e0 = lane & 15, i = lane >> 4, wave = threadIdx.x >> 6;
  const uint32_t m = a.m, ranges = (a.g.C + kBlockRange - 1) / kBlockRange;
  const uint32_t half = a.g.rope.head_dim / 2;
  uint32_t total = 0;
  if constexpr (kRope) {
    for (int p = 0; p < a.g.n_parts; ++p) total += a.g.part[p].rows / 2;
  } else {
    total = a.g.part[0].rows;
  }
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  const uint32_t pos0 = kRope ? a.state->pos : 0u;
  for (uint32_t q4 = blockIdx.x * 4 + uint32_t(wave); q4 * 4 < total; q4 += gridDim.x * 4) {
    const uint32_t o = q4 * 4 + uint32_t(i);
    const bool ok = o < total;
    // the output's part and rows
    int p = 0;
    uint32_t rows_k[NR];
    if constexpr (kRope) {
      uint32_t oo = ok ? o : 0u;
      while (p + 1 < a.g.n_parts && oo >= a.g.part[p].rows / 2) {
        oo -= a.g.part[p].rows / 2;
        ++p;
      }
      const uint32_t lo = (oo / half) * (2 * half) + oo % half;
      rows_k[0] = lo;
      rows_k[1] = lo + half;
    } else {
      rows_k[0] = ok ? o : 0u;
      if constexpr (kSwi) rows_k[1] = rows_k[0];
    }
    // corrections of each row, all tokens
    float cor[NR][kMaxBlock];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const GemvPart& P = a.g.part[kSwi ? k : p];
      const uint32_t r = rows_k[k];
      const float2* corr = P.corr;
      const uint32_t kmax = P.corr_kmax;
#pragma unroll
      for (int t = 0; t < int(kMaxBlock); ++t) cor[k][t] = 0.0f;
      if (corr != nullptr && ok && r < P.wrows) {
        for (uint32_t e = uint32_t(e0); e < kmax; e += 16) {
          const float2 ce = corr[size_t(r) * kmax + e];
          if (ce.y == 0.0f) continue;
          const float4* xr = reinterpret_cast<const float4*>(a.t.xt + size_t(__float_as_uint(ce.x)) * kMaxBlock);
          const float4 xa = xr[0], xb = xr[1];
          cor[k][0] = fmaf(ce.y, xa.x, cor[k][0]);
          cor[k][1] = fmaf(ce.y, xa.y, cor[k][1]);
          cor[k][2] = fmaf(ce.y, xa.z, cor[k][2]);
          cor[k][3] = fmaf(ce.y, xa.w, cor[k][3]);
          cor[k][4] = fmaf(ce.y, xb.x, cor[k][4]);
          cor[k][5] = fmaf(ce.y, xb.y, cor[k][5]);
          cor[k][6] = fmaf(ce.y, xb.z, cor[k][6]);
          cor[k][7] = fmaf(ce.y, xb.w, cor[k][7]);
        }
      }
#pragma unroll
      for (int t = 0; t < int(kMaxBlock); ++t) {
        float v = cor[k][t];
        v = pair_sum(v, 1);
        v = pair_sum(v, 2);
        v = pair_sum(v, 4);
        v = pair_sum(v, 8);
        cor[k][t] = v;
      }
    }
    // lane (i, t): token t of the output
    const uint32_t t = uint32_t(e0);
    if (!ok || t >= m) continue;
    float v[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const GemvPart& P = a.g.part[kSwi ? k : p];
      const uint32_t at = P.unit_begin * 16 + rows_k[k];
      float s = 0.0f;
      for (uint32_t rg = 0; rg < ranges; ++rg) s += a.partial[(size_t(rg) * kMaxBlock + t) * a.rows_all + at];
      float c = cor[k][0];
#pragma unroll
      for (int tt = 1; tt < int(kMaxBlock); ++tt) c = t == uint32_t(tt) ? cor[k][tt] : c;
      v[k] = s + c;
    }
    const GemvPart& P0 = a.g.part[kSwi ? 0 : p];
    const uint32_t r = rows_k[0];
    float* y = P0.y + size_t(t) * P0.rows;
    if constexpr (MODE == int(GemvMode::Store)) {
      y[r] = v[0] + (P0.bias ? P0.bias[r] : 0.0f);
    } else if constexpr (MODE == int(GemvMode::Accum)) {
      if (r < P0.wrows) y[r] = y[r] + v[0];  // rows past the tiles stay
    } else if constexpr (kSwi) {
      y[r] = v[0] / (1.0f + expf(-v[0])) * v[1];  // silu(g)*u: :159-161, :1746-1748
    } else if constexpr (kRope) {
#pragma clang fp contract(off)
      const float lo = v[0] + (P0.bias ? P0.bias[r] : 0.0f);
      const float hi = v[1] + (P0.bias ? P0.bias[r + half] : 0.0f);
      const uint32_t pos = pos0 + t, d = r % (2 * half);
      float o0 = lo, o1 = hi;
      if (P0.rope_role != kRoleV && pos < a.rope_rows) {  // applyRope :195-216
        const float c = a.rope_cos[size_t(pos) * half + d], sn = a.rope_sin[size_t(pos) * half + d];
        o0 = lo * c - hi * sn;
        o1 = lo * sn + hi * c;
      }
      if (P0.rope_role == kRoleQ) {
        y[r] = o0;
        y[r + half] = o1;
      } else {
        const uint32_t hd = a.g.rope.head_dim, head = r / hd;
        void* cache = P0.rope_role == kRoleK ? a.g.rope.k_cache : a.g.rope.v_cache;
        if (a.g.rope.kv_f16 && P0.rope_role == kRoleV) {  // 4-position blocks: [pos/4][dim][pos%4]
          const size_t blk = (size_t(head) * a.g.rope.max_seq + (pos & ~3u)) * hd + (pos & 3u);
          reinterpret_cast<__half*>(cache)[blk + size_t(d) * 4] = __float2half_rn(o0);
          reinterpret_cast<__half*>(cache)[blk + size_t(d + half) * 4] = __float2half_rn(o1);
        } else {
          const size_t at = (size_t(head) * a.g.rope.max_seq + pos) * hd + d;
          if (a.g.rope.kv_f16) {
            reinterpret_cast<__half*>(cache)[at] = __float2half_rn(o0);
            reinterpret_cast<__half*>(cache)[at + half] = __float2half_rn(o1);
          } else {
            reinterpret_cast<float*>(cache)[at] = o0;
            reinterpret_cast<float*>(cache)[at + half] = o1;
          }
        }
      }
    } else {
      y[r] = v[0];
      if (!isfinite(v[0])) nf = 1;
      if (v[0] > -1e30f && better(v[0], r, bv, bi)) {
        bv = v[0];
        bi = r;
      }
    }
  }
  if constexpr (kLogits) {
    // per token (lanes e0 = t of the 4 outputs), then over the waves
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
      const float ov = pair_val(bv, o);
      const uint32_t oi = pair_u(bi, o);
      nf |= pair_u(nf, o);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    __shared__ float s_bv[4][16];
    __shared__ uint32_t s_bi[4][16], s_nf[4][16];
    if (lane < 16) {
      s_bv[wave][lane] = bv;
      s_bi[wave][lane] = bi;
      s_nf[wave][lane] = nf;
    }
    __syncthreads();
    if (threadIdx.x < m) {
      const uint32_t tk = threadIdx.x;
      float b = s_bv[0][tk];
      uint32_t bx = s_bi[0][tk], f = s_nf[0][tk];
      for (int w = 1; w < 4; ++w) {
        f |= s_nf[w][tk];
        if (better(s_bv[w][tk], s_bi[w][tk], b, bx)) {
          b = s_bv[w][tk];
          bx = s_bi[w][tk];
        }
      }
      a.partials[size_t(tk) * a.epi_blocks + blockIdx.x] = ArgmaxPartial{b, bx, f, 0u};
    }
  }
}

__global__ void __launch_bounds__(256) k_block_finish(BlockFinishArgs a) {
  const uint32_t t = blockIdx.x;
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  for (uint32_t i = threadIdx.x; i < a.n_partials; i += blockDim.x) {
    const ArgmaxPartial p = a.partials[size_t(t) * a.n_partials + i];
    nf |= p.nonfinite;
    if (better(p.value, p.index, bv, bi)) {
      bv = p.value;
      bi = p.index;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = pair_val(bv, o);
    const uint32_t oi = pair_u(bi, o);
    nf |= pair_u(nf, o);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
  __shared__ float s_v[4];
  __shared__ uint32_t s_i[4], s_nf[4];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) {
    s_v[w] = bv;
    s_i[w] = bi;
    s_nf[w] = nf;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 1; k < int(blockDim.x >> 6); ++k) {
      nf |= s_nf[k];
      if (better(s_v[k], s_i[k], bv, bi)) {
        bv = s_v[k];
        bi = s_i[k];
      }
    }
    const uint32_t arg = bi == 0xffffffffu ? 0u : bi;
    a.out_argmax[t] = arg;
    if (t + 1 == a.m) {
      StepResult* r = a.result;
      r->argmax = arg;
      r->max_logit = bv;
      r->token0_logit = a.logits[size_t(t) * a.V];
      r->hidden_norm = sqrtf(a.ss[t]);
      r->all_finite = nf ? 0u : 1u;
    }
  }
}

}  // namespace

void launch_block_limbs(const float* x, const float* gamma, float eps, uint32_t C, uint32_t m, const BlockTables& t,
                        hipStream_t st) {
  const uint32_t nq = (m + 3) / 4;
  if (gamma) launch_kernel(&k_block_limbs<true>, dim3(4 * nq), dim3(1024), st, x, gamma, eps, C, m, t);
  else launch_kernel(&k_block_limbs<false>, dim3(4 * nq), dim3(1024), st, x, gamma, eps, C, m, t);
}

uint32_t launch_block_gemv(BlockGemvArgs& a, hipStream_t st) {
  const uint32_t ranges = (a.g.C + kBlockRange - 1) / kBlockRange;
  // workgroups per range: about 512 workgroups of 8 waves in all (two per CU: the LDS tables)
  uint32_t per = (512 + ranges - 1) / ranges;
  const uint32_t need = (a.n_units + 7) / 8;
  if (per > need) per = need;
  if (per == 0) per = 1;
  const dim3 grid(ranges, per);
  if (a.nq <= 1) launch_kernel(&k_gemv_mt<1, 8>, grid, dim3(512), st, a);
  else launch_kernel(&k_gemv_mt<2, 8>, grid, dim3(512), st, a);
  uint32_t outs = 0;
  if (GemvMode(a.g.mode) == GemvMode::QkvRope) {
    for (int p = 0; p < a.g.n_parts; ++p) outs += a.g.part[p].rows / 2;
  } else {
    outs = a.g.part[0].rows;
  }
  uint32_t eb = (outs + 15) / 16;
  if (eb > 1024) eb = 1024;
  if (GemvMode(a.g.mode) == GemvMode::Logits && eb > 512) eb = 512;
  a.epi_blocks = eb;
  switch (GemvMode(a.g.mode)) {
    case GemvMode::Store: launch_kernel(&k_block_epi<int(GemvMode::Store)>, dim3(eb), dim3(256), st, a); break;
    case GemvMode::Accum: launch_kernel(&k_block_epi<int(GemvMode::Accum)>, dim3(eb), dim3(256), st, a); break;
    case GemvMode::SwiGlu: launch_kernel(&k_block_epi<int(GemvMode::SwiGlu)>, dim3(eb), dim3(256), st, a); break;
    case GemvMode::Logits: launch_kernel(&k_block_epi<int(GemvMode::Logits)>, dim3(eb), dim3(256), st, a); break;
    case GemvMode::QkvRope: launch_kernel(&k_block_epi<int(GemvMode::QkvRope)>, dim3(eb), dim3(256), st, a); break;
  }
  return eb;
}

void launch_block_finish(const BlockFinishArgs& a, hipStream_t st) {
  launch_kernel(&k_block_finish, dim3(a.m), dim3(256), st, a);
}

}  // namespace chpe
