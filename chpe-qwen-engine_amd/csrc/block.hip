// block.hip -- the block step's GEMV: m <= kMaxBlock tokens at consecutive positions through
// flat 4- or 2-bit tiles (gemvCellFlat, chpe_engine.zig:584-729), every weight read once for all
// of them.  Used by the batch-M verify and by the chunked prefill; each token's arithmetic is the
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
//    code * limb over the group, starting at -8 * (the limb's sum) for the codes' offset.  2-bit
//    tiles: the codebook {0, +1, -2, -1} (:220) is the 2-bit two's complement, so the operand
//    is code ^ 2 (0..3) and the sum starts at -2 * (the limb's sum); the tables then hold the
//    columns in the 2-bit fields' order.  The
//    lane combines its 4 limbs (2^(8 j)), scales by 2^(e - 30) and by the row's group scale,
//    and accumulates row n of token q over the range's groups; the raw row sums of each range
//    go to a partial-sum buffer.  The B layout reads only 64 bytes of each of 16 rows per load
//    instruction, which the memory system serves at about half the rate of long runs, so the
//    codes are loaded 512 contiguous bytes of a row at a time (a stage of 16 rows x 8 groups;
//    2-bit: x 16 groups, the whole range),
//    passed through a wave-private LDS slot and read back in the B layout; the next stage's
//    loads are in flight meanwhile.
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

// grid (column chunks of 1024, token slots 4 nq): a workgroup of 128 threads converts 1024
// columns of one token (8 per thread, 16 threads per 128-column group) into the operand tables:
// the input, RMS-normalised ((x * inv) * gamma, rmsNorm :187-191) when gamma is set, as
// X = x * 2^(30-e) with max |x| < 2^e (exact in int32) per 128-column group, in four balanced
// signed-byte limbs (BlockTables).  The norm's sum of squares comes as the producer's partial
// sums (ssp), read together with the columns; chunk 0 keeps it (the LM head's hidden norm).
// Token slots >= m get zero tables.  A q/k/v launch (chk, as RopeArgs::brk_check) also makes
// forwardDecode's break test (StepState::broken) on each token's input and records it in brk[token].
// BITS: the tiles' code width, which fixes the tables' column order and the codes' offset.
template <bool kNorm, int BITS>
__global__ void __launch_bounds__(128) k_block_limbs(const float* X, const float* gamma, float eps, uint32_t C,
                                                      uint32_t m, const float* ssp, uint32_t n_ssp, BlockTables t,
                                                      uint32_t* brk, uint32_t chk, uint32_t ts) {
  const uint32_t tok = blockIdx.y, T = tok >> 2, tl = tok & 3u, ng = C >> 7;
  const bool live = tok < m;
  const float* x = X + size_t(live ? tok : 0u) * C;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const uint32_t c0 = blockIdx.x * 1024 + 8 * uint32_t(tid);
  const bool in = c0 < ng * 128;
  const uint32_t cc = in ? c0 : 0u;
  // every load first
  const float4 xa = ld_f4(x + cc), xb = ld_f4(x + cc + 4);
  float4 ga = make_float4(1.f, 1.f, 1.f, 1.f), gb = ga;
  float ss = 0.0f;
  if constexpr (kNorm) {
    ga = ld_f4(gamma + cc);
    gb = ld_f4(gamma + cc + 4);
    if (live) {
#pragma unroll 4
      for (uint32_t i = uint32_t(tid); i < n_ssp; i += 128) ss += ssp[size_t(i) * kMaxBlock + tok];
    }
  }
  float inv = 1.0f;
  if constexpr (kNorm) {
    __shared__ float s_red[2];
    ss = wave_sum(ss);
    if (lane == 0) s_red[wave] = ss;
    __syncthreads();
    const float tot = s_red[0] + s_red[1];
    if (blockIdx.x == 0 && tid == 0) {
      t.ss[tok] = live ? tot : 0.0f;
      if (live && ((chk == 1u && !isfinite(tot)) || (chk == 2u && !isfinite(x[0])))) brk[tok] = 1u;
    }
    inv = 1.0f / sqrtf(tot / float(C) + eps);
  }
  float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  if constexpr (kNorm) {
    const float gv[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) xv[i] = (xv[i] * inv) * gv[i];
  }
  float mx = 0.0f;  // (a NaN counts as infinite: the group's scale becomes NaN, as its sum would)
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xv[i] = (live && in) ? xv[i] : 0.0f;
    const float ax = fabsf(xv[i]);
    mx = ax != ax ? __int_as_float(0x7f800000) : fmaxf(mx, ax);
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
  if constexpr (BITS == 2) {
    // threads 2k, 2k + 1 hold columns 0..7 and 8..15 of a 16-column block; the 2-bit fields'
    // order wants {0,4,8,12}, {1,5,9,13} in the even thread and {2,6,10,14}, {3,7,11,15} in the
    // odd one: each sends the four its neighbour needs
    const bool odd = (lane & 1) != 0;
    const uint32_t r0 = pair_u(odd ? z[0] : z[2], 1), r1 = pair_u(odd ? z[1] : z[3], 1);
    const uint32_t r2 = pair_u(odd ? z[4] : z[6], 1), r3 = pair_u(odd ? z[5] : z[7], 1);
    if (odd) {
      limb_words(r0, r2, z[2], z[6], lo);
      limb_words(r1, r3, z[3], z[7], hi);
    } else {
      limb_words(z[0], z[4], r0, r2, lo);
      limb_words(z[1], z[5], r1, r3, hi);
    }
  } else {  // the nibbles' order {0,2,4,6}, {1,3,5,7}, {8,10,12,14}, {9,11,13,15}
    limb_words(z[0], z[2], z[4], z[6], lo);
    limb_words(z[1], z[3], z[5], z[7], hi);
  }
  const uint32_t g = cc >> 7, c = cc & 127u, kq = c >> 5, h = (c >> 4) & 1u, p = (c >> 3) & 1u;
  uint2* tb2 = reinterpret_cast<uint2*>(t.tb);
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
    constexpr int kOff = BITS == 2 ? -2 : -8;
    t.ci[(size_t(T) * ng + g) * 4 + tl] = make_int4(kOff * sums[0], kOff * sums[1], kOff * sums[2], kOff * sums[3]);
    t.ew[(size_t(T) * ng + g) * 4 + tl] = isfinite(mx) ? ldexpf(1.0f, e - 30) : __int_as_float(0x7fc00000);
  }
  if (in && live) {
#pragma unroll
    for (int i = 0; i < 8; ++i) t.xt[size_t(cc + uint32_t(i)) * ts + tok] = xv[i];
  }
}

// A stage: 16 weight rows x 512 bytes of codes of the range (8 KB): 8 groups of 4-bit codes
// (64 B each) or 16 groups of 2-bit codes (32 B each, the whole 2048-column range), loaded 512
// contiguous bytes of two rows per instruction (lane l: row 2 i + (l >> 5), bytes 16 (l & 31)
// of the row's 512), then written to the wave's LDS slot so that the matrix-core layout (lane
// (n, q): row n, quarter q of a group) reads it back; rows at kStageRow bytes (16 B of padding:
// the 16 rows of one read fall on distinct banks).
constexpr uint32_t kStageRow = 528, kStageBytes = 16 * kStageRow;
// The stage geometry of a range of RG groups: GPS groups per stage (at most 512 bytes of a row),
// SPU stages per unit, RB bytes of a row per stage, LPR lanes per row and RPI rows per load
// instruction, NLD 16-byte loads per lane and stage.
template <int BITS, int RG>
struct MtGeom {
  static constexpr uint32_t GB = BITS == 2 ? 32 : 64;  // code bytes per group and row
  static constexpr uint32_t GPS = RG * GB <= 512 ? RG : 512 / GB;
  static constexpr uint32_t SPU = RG / GPS;
  static constexpr uint32_t RB = GPS * GB, LPR = RB / 16, RPI = 64 / LPR, NLD = 16 / RPI;
  static constexpr uint32_t kScales = 16 * GPS / 64, kRowsPer = 64 / GPS;  // scales per lane; rows per scale load
  static_assert(RG % GPS == 0 && LPR * RPI == 64 && NLD * RPI == 16 && kScales >= 1, "");
};
template <int BITS, int RG>
struct MtStage {
  using G = MtGeom<BITS, RG>;
  uint4 v[G::NLD];           // codes: lane l, row RPI i + l / LPR, bytes 16 (l % LPR) of the row's RB
  uint32_t sc[G::kScales];   // group scales: lane l, row kRowsPer i + l / GPS, group l % GPS
};

// NQ token quads (tables in LDS: NQ x RG groups x 2 KB), RG groups of 128 columns per range
template <int NQ, int NW, int BITS, int RG>
__global__ void __launch_bounds__(kWave * NW) k_gemv_mt(BlockGemvArgs a) {
  using G = MtGeom<BITS, RG>;
  constexpr uint32_t GPS = G::GPS, SPU = G::SPU, GB = G::GB;
  __shared__ __align__(16) uint4 s_tb[NQ][RG][128];
  __shared__ __align__(16) int4 s_ci[NQ][RG][4];
  __shared__ float s_ew[NQ][RG][4];
  __shared__ __align__(16) uint8_t s_w[NW][kStageBytes];
  __shared__ uint16_t s_sc[NW][16][GPS];
  const int lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t C = a.g.C, ng = C >> 7, range = blockIdx.x, g0 = range * RG;
  const uint32_t ngr = ng - g0 < uint32_t(RG) ? ng - g0 : uint32_t(RG);
  const uint32_t nq = a.nq;  // (quads past it hold no tokens: skipped)
  const uint32_t n_units = a.n_units, waves_total = gridDim.y * NW;
  const uint32_t wid = blockIdx.y * NW + wave;
  const bool active = wid < n_units;
  const uint32_t n_stages = active ? SPU * ((n_units - wid + waves_total - 1) / waves_total) : 0u;
  uint8_t* slot = s_w[wave];
  // the unit's part: parts hold consecutive unit ranges from part[p].unit_begin
  auto part_index = [&](uint32_t u) {
    int p = 0;
#pragma unroll
    for (int k = 1; k < kMaxParts; ++k) p += (k < a.g.n_parts && u >= a.g.part[k].unit_begin) ? 1 : 0;
    return p;
  };
  // stage j of this wave: unit wid + (j / SPU) * waves_total, groups GPS (j % SPU) .. + GPS - 1
  // of the range (a stage past the last repeats the last: its lines are cached)
  auto issue = [&](uint32_t j, MtStage<BITS, RG>* st) {
    j = j < n_stages ? j : n_stages - 1;
    const uint32_t u = wid + (j / SPU) * waves_total, h = j % SPU;
    const int p = int(__builtin_amdgcn_readfirstlane(part_index(u)));
    const GemvPart& P = a.g.part[p];
    const uint8_t* base = P.base;
    const uint32_t stride = P.stride, wr = P.wrows, r0 = (u - P.unit_begin) * kBlockUnit;
    const uint32_t lb = 16 * (uint32_t(lane) % G::LPR);  // the lane's bytes in the row's RB
    const uint32_t gl = GPS * h + lb / GB, gc = gl < ngr ? gl : 0u;
#pragma unroll
    for (int i = 0; i < int(G::NLD); ++i) {
      const uint32_t r = r0 + G::RPI * uint32_t(i) + uint32_t(lane) / G::LPR, rr = r < wr ? r : 0u;
      const uint32_t Gi = rr * ng + g0 + gc;
      st->v[i] = ld_u128(base + ((Gi >> 8) * stride + 64 + (Gi & 255u) * GB + lb % GB));
    }
#pragma unroll
    for (int i = 0; i < int(G::kScales); ++i) {
      const uint32_t r = r0 + G::kRowsPer * uint32_t(i) + uint32_t(lane) / GPS, rr = r < wr ? r : 0u;
      const uint32_t g = GPS * h + (uint32_t(lane) % GPS), Gi = rr * ng + g0 + (g < ngr ? g : 0u);
      st->sc[i] = ld_u16(base + ((Gi >> 8) * stride + 16448 + 48 + 2 * (Gi & 255u)));
    }
  };
  // into the wave's slot (LDS operations of one wave complete in order: the previous stage's
  // reads are done before these writes land)
  auto stage = [&](const MtStage<BITS, RG>& st) {
#pragma unroll
    for (int i = 0; i < int(G::NLD); ++i)
      *reinterpret_cast<uint4*>(slot + (G::RPI * i + lane / G::LPR) * kStageRow + 16 * (lane % G::LPR)) = st.v[i];
#pragma unroll
    for (int i = 0; i < int(G::kScales); ++i)
      s_sc[wave][G::kRowsPer * i + lane / int(GPS)][lane % int(GPS)] = uint16_t(st.sc[i]);
  };
  float acc[NQ];
#pragma unroll
  for (int T = 0; T < NQ; ++T) acc[T] = 0.0f;
  auto compute = [&](uint32_t j) {
    const uint32_t h = j % SPU;
#pragma unroll 4
    for (int k = 0; k < int(GPS); ++k) {
      const uint32_t gl = GPS * h + uint32_t(k);
      const bool gv = gl < ngr;
      const uint32_t gk = gv ? gl : 0u;
      const float sc = gv ? h2f(s_sc[wave][n][k]) : 0.0f;
      i32x4_t B0, B1;
      if constexpr (BITS == 2) {  // 16 codes in 4 bytes: field f of each byte, code ^ 2
        const uint2 w2 = *reinterpret_cast<const uint2*>(slot + n * kStageRow + 32 * k + 8 * q);
        const uint32_t x = w2.x ^ 0xAAAAAAAAu, y = w2.y ^ 0xAAAAAAAAu;
        B0 = i32x4_t{int(x & 0x03030303u), int((x >> 2) & 0x03030303u), int((x >> 4) & 0x03030303u),
                     int((x >> 6) & 0x03030303u)};
        B1 = i32x4_t{int(y & 0x03030303u), int((y >> 2) & 0x03030303u), int((y >> 4) & 0x03030303u),
                     int((y >> 6) & 0x03030303u)};
      } else {
        const uint4 w = *reinterpret_cast<const uint4*>(slot + n * kStageRow + 64 * k + 16 * q);
        B0 = i32x4_t{int(w.x & 0x0f0f0f0fu), int((w.x >> 4) & 0x0f0f0f0fu), int(w.y & 0x0f0f0f0fu),
                     int((w.y >> 4) & 0x0f0f0f0fu)};
        B1 = i32x4_t{int(w.z & 0x0f0f0f0fu), int((w.z >> 4) & 0x0f0f0f0fu), int(w.w & 0x0f0f0f0fu),
                     int((w.w >> 4) & 0x0f0f0f0fu)};
      }
#pragma unroll
      for (int T = 0; T < NQ; ++T) {
        if (NQ > 2 && uint32_t(T) >= nq) break;  // (uniform)
        const uint4 t0 = s_tb[T][gk][(uint32_t(q) * 2) * 16 + uint32_t(n)];
        const uint4 t1 = s_tb[T][gk][(uint32_t(q) * 2 + 1) * 16 + uint32_t(n)];
        const i32x4_t A0 = {int(t0.x), int(t0.y), int(t0.z), int(t0.w)};
        const i32x4_t A1 = {int(t1.x), int(t1.y), int(t1.z), int(t1.w)};
        const int4 c4 = s_ci[T][gk][q];
        i32x4_t D = {c4.x, c4.y, c4.z, c4.w};
        D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0, D, 0, 0, 0);
        D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1, D, 0, 0, 0);
        const float f = ((float(D[0]) + float(D[1]) * 256.0f) + float(D[2]) * 65536.0f) + float(D[3]) * 16777216.0f;
        acc[T] += gv ? f * s_ew[T][gk][q] * sc : 0.0f;
      }
    }
    if (h == SPU - 1) {  // the unit's last stage: row n of tokens 4 T + q
      const uint32_t u = wid + (j / SPU) * waves_total;
      const int p = int(__builtin_amdgcn_readfirstlane(part_index(u)));
      const GemvPart& P = a.g.part[p];
      const uint32_t r = (u - P.unit_begin) * kBlockUnit + uint32_t(n), at = P.unit_begin * kBlockUnit + r;
#pragma unroll
      for (int T = 0; T < NQ; ++T) {
        const uint32_t tk = 4 * uint32_t(T) + uint32_t(q);
        if (tk < a.m) a.partial[(size_t(range) * a.rows_all + at) * a.ts + tk] = r < P.wrows ? acc[T] : 0.0f;
        acc[T] = 0.0f;
      }
    }
  };
  // the first stage's loads are in flight while the range's operand tables are staged, the next
  // stage's while the current stage is staged and multiplied
  MtStage<BITS, RG> SA, SB;
  if (active) issue(0, &SA);
  const uint32_t nqt = NQ > 2 ? (nq < uint32_t(NQ) ? nq : uint32_t(NQ)) : uint32_t(NQ);  // quads with tables
  for (uint32_t i = threadIdx.x; i < nqt * RG * 128; i += kWave * NW) {
    const uint32_t T = i / (RG * 128), gl = (i / 128) % RG, e = i % 128;
    s_tb[T][gl][e] = gl < ngr ? a.t.tb[(size_t(T) * ng + g0 + gl) * 128 + e] : make_uint4(0, 0, 0, 0);
  }
  for (uint32_t i = threadIdx.x; i < nqt * RG * 4; i += kWave * NW) {
    const uint32_t T = i / (RG * 4), gl = (i / 4) % RG, k = i % 4;
    const bool ok = gl < ngr;
    s_ci[T][gl][k] = ok ? a.t.ci[(size_t(T) * ng + g0 + gl) * 4 + k] : make_int4(0, 0, 0, 0);
    s_ew[T][gl][k] = ok ? a.t.ew[(size_t(T) * ng + g0 + gl) * 4 + k] : 0.0f;
  }
  __syncthreads();
  if (!active) return;  // (no barrier follows)
  for (uint32_t j = 0;; j += 2) {
    stage(SA);
    issue(j + 1, &SB);
    compute(j);
    if (j + 1 >= n_stages) break;
    stage(SB);
    issue(j + 2, &SA);
    compute(j + 1);
    if (j + 2 >= n_stages) break;
  }
}

// Blocks of 9 .. kMaxBlock tokens (the prefill): output-stationary.  A workgroup of kGmWaves
// waves owns a row block of kGmWaves * U units (wave w: units U w .. U w + U - 1 of the block)
// and one range of column chunks (GC groups each: 128 code bytes of a row for 4-bit GC = 2).
// Per chunk:
//   * the token quads' operand tables of the chunk are in one of two LDS buffers; the workgroup
//     loads the next chunk's tables into registers meanwhile and writes them to the other
//     buffer after its multiplies (one barrier per chunk);
//   * each wave loads the chunk's codes of its 16 U rows (RPI whole rows of RB bytes per
//     instruction), passes them through its LDS slot into the B layout, with the next chunk's
//     loads in flight;
//   * per group and token quad the wave reads the quad's operand once and runs it against its
//     U units (k_gemv_mt reads it once per unit: U times the LDS reads per weight byte, the
//     bound of that loop at 32 tokens).
// The codes enter the matrix cores as signed bytes, code - 8 (4-bit) or the 2-bit two's
// complement value, so no offset term is needed.  A range's raw row sums go to the partial-sum
// buffer as k_gemv_mt's; the ranges are few (block_gemv_ranges: enough workgroups to fill the
// CUs).
constexpr int kGmWaves = 16;
constexpr uint32_t kGmUnits = 2, kGmChunk = 2;  // U, GC of the launches
template <int BITS, int U, int GC>
struct GmGeom {
  static constexpr uint32_t GB = BITS == 2 ? 32 : 64;      // code bytes per group and row
  static constexpr uint32_t RB = GC * GB;                    // code bytes per row and chunk
  static constexpr uint32_t LPR = RB / 16, RPI = 64 / LPR;   // lanes per row; rows per load
  static constexpr uint32_t ROWS = 16 * U, NLD = ROWS / RPI;  // the wave's rows; loads per lane
  static constexpr uint32_t SROW = RB + 16, SLOT = ROWS * SROW;  // slot rows (16 B of padding)
  static_assert(LPR * RPI == 64 && 16 % RPI == 0 && 16 * GC <= 64, "a load within one unit");
};
template <int BITS, int U, int GC>
struct GmStage {
  uint4 v[GmGeom<BITS, U, GC>::NLD];  // codes: lane l, row RPI i + l / LPR, bytes 16 (l % LPR)
  uint32_t sc[U];                     // scales of unit u: lane l < 16 GC, row l / GC, group l % GC
};
// bytes b (0..15 each) as signed bytes b - 8, and (0..3 each) as b - 2: + (128 - off), then the
// sign bit flipped (no carry leaves a byte)
__device__ __forceinline__ int sbytes4(uint32_t b) { return int((b + 0x78787878u) ^ 0x80808080u); }
__device__ __forceinline__ int sbytes2(uint32_t b) { return int((b + 0x7e7e7e7eu) ^ 0x80808080u); }

template <int BITS, int U, int GC>
__global__ void __launch_bounds__(kWave * kGmWaves) k_block_gemm(BlockGemvArgs a) {
  using G = GmGeom<BITS, U, GC>;
  constexpr int NQ = int(kMaxBlock / 4);
  constexpr int kThreads = kWave * kGmWaves;
  // (the two table buffers are separate objects, so that the compiler sees the loads into one
  // and the reads of the other as independent)
  __shared__ __align__(16) uint4 s_tb0[NQ][GC][128], s_tb1[NQ][GC][128];
  __shared__ float s_ew0[NQ][GC][4], s_ew1[NQ][GC][4];
  __shared__ __align__(16) uint8_t s_w[kGmWaves][G::SLOT];
  __shared__ uint16_t s_sc[kGmWaves][G::ROWS][GC];
  const int tid = threadIdx.x, lane = tid & 63, n = lane & 15, q = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(uint32_t(tid) >> 6);
  const uint32_t ng = a.g.C >> 7, nch = (ng + GC - 1) / GC, range = blockIdx.x;
  const uint32_t c_begin = uint32_t(uint64_t(range) * nch / gridDim.x);
  const uint32_t c_end = uint32_t(uint64_t(range + 1) * nch / gridDim.x);
  const uint32_t u0 = (blockIdx.y * kGmWaves + wave) * U;  // the wave's first unit
  uint8_t* slot = s_w[wave];
  // each unit's part (parts hold consecutive unit ranges from part[p].unit_begin); a unit past
  // the last reads unit 0's rows and writes nothing
  const uint8_t* ubase[U];
  uint32_t ustride[U], uwr[U], ur0[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t uu = u0 + uint32_t(u) < a.n_units ? u0 + uint32_t(u) : 0u;
    int p = 0;
#pragma unroll
    for (int k = 1; k < kMaxParts; ++k) p += (k < a.g.n_parts && uu >= a.g.part[k].unit_begin) ? 1 : 0;
    p = int(__builtin_amdgcn_readfirstlane(p));
    ubase[u] = a.g.part[p].base;
    ustride[u] = a.g.part[p].stride;
    uwr[u] = a.g.part[p].wrows;
    ur0[u] = (uu - a.g.part[p].unit_begin) * kBlockUnit;
  }
  const bool active = u0 < a.n_units;
  // the chunk's codes and scales of the wave's rows (groups past the last repeat the chunk's first)
  auto issue = [&](uint32_t c, GmStage<BITS, U, GC>* st) {
    const uint32_t cg = c * GC;
    const uint32_t lb = 16 * (uint32_t(lane) % G::LPR), gk = cg + lb / G::GB, gg = gk < ng ? gk : cg;
#pragma unroll
    for (int i = 0; i < int(G::NLD); ++i) {
      const int u = int(G::RPI) * i / 16;
      const uint32_t r = ur0[u] + (G::RPI * uint32_t(i)) % 16 + uint32_t(lane) / G::LPR, rr = r < uwr[u] ? r : 0u;
      const uint32_t Gi = rr * ng + gg;
      st->v[i] = ld_u128(ubase[u] + ((Gi >> 8) * ustride[u] + 64 + (Gi & 255u) * G::GB + lb % G::GB));
    }
    // (every lane loads; lanes past 16 GC read a row of the part or row 0 and are not staged)
    const uint32_t sk = uint32_t(lane) % GC, sg = cg + sk < ng ? cg + sk : cg;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const uint32_t r = ur0[u] + uint32_t(lane) / GC, rr = r < uwr[u] ? r : 0u;
      const uint32_t Gi = rr * ng + sg;
      st->sc[u] = ld_u16(ubase[u] + ((Gi >> 8) * ustride[u] + 16448 + 48 + 2 * (Gi & 255u)));
    }
  };
  // into the wave's slot (LDS operations of one wave complete in order: the previous chunk's
  // reads are done before these writes land)
  // (the scale of a group past the last, chunk c's, is staged as 0)
  auto stage = [&](const GmStage<BITS, U, GC>& st, uint32_t c, uint8_t* sl, uint16_t* sc) {
#pragma unroll
    for (int i = 0; i < int(G::NLD); ++i)
      *reinterpret_cast<uint4*>(sl + (G::RPI * i + lane / G::LPR) * G::SROW + 16 * (lane % G::LPR)) = st.v[i];
    const bool gv = c * GC + uint32_t(lane) % GC < ng;
    if (lane < 16 * GC) {
#pragma unroll
      for (int u = 0; u < U; ++u) sc[(16 * u + lane / GC) * GC + lane % GC] = gv ? uint16_t(st.sc[u]) : uint16_t(0);
    }
  };
  // the operand tables of chunk c straight into LDS buffer b (global_load_lds: 64 lanes x 16 B
  // to consecutive LDS per instruction, no registers), each wave kTabInst instructions, wave 0
  // also the 64 group exponents.  Nothing is zeroed: the tables of quads past nq -- allocated
  // for kMaxBlock tokens, stale -- feed only results that are not stored, and a group past the
  // last reads the last group's and is skipped in compute.
  constexpr int kTabInst = NQ * GC * 128 / kThreads;
  auto fetch_tables = [&](uint32_t c, uint4* tdst, float* edst) {
    const uint32_t cg = c * GC;
#pragma unroll
    for (int j = 0; j < kTabInst; ++j) {
      const uint32_t i0 = (wave * kTabInst + uint32_t(j)) * kWave, i = i0 + uint32_t(lane);
      const uint32_t T = i / (GC * 128), k = (i / 128) % GC, e = i % 128, g = cg + k < ng ? cg + k : ng - 1;
      __builtin_amdgcn_global_load_lds(a.t.tb + (size_t(T) * ng + g) * 128 + e, tdst + i0, 16, 0, 0);
    }
    if (wave == 0) {
      const uint32_t T = uint32_t(lane) / (GC * 4) % NQ, k = (uint32_t(lane) / 4) % GC, qq = uint32_t(lane) % 4;
      const uint32_t g = cg + k < ng ? cg + k : ng - 1;
      __builtin_amdgcn_global_load_lds(a.t.ew + (size_t(T) * ng + g) * 4 + qq, edst, 4, 0, 0);
    }
  };
  static_assert(NQ * GC * 128 % kThreads == 0 && NQ * GC * 4 == kWave, "table loads: whole instructions");
  float acc[U][NQ];
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int T = 0; T < NQ; ++T) acc[u][T] = 0.0f;
  // per group the U units' operands (a group past the last -- only in the last chunk of an odd
  // group count -- runs on the clamped, finite data with the scale 0 stage() gave it: no
  // branch); per token quad
  // the 2 U matrix-core products first, then the conversions: lane (n, q) holds token q's limb
  // sums D0..D3 of row n, combined exactly in pairs (|D| < 2^18: D0 + 2^8 D1 fits), then
  // lo + 2^16 hi in float, scaled by 2^(e - 30) * the row's group scale
  auto compute = [&](const uint4* tsrc, const float* esrc, const uint8_t* sl, const uint16_t* scs) {
#pragma unroll
    for (int k = 0; k < GC; ++k) {
      i32x4_t B0[U], B1[U];
      float scv[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint8_t* row = sl + (16 * u + n) * G::SROW + G::GB * k;
        if constexpr (BITS == 2) {  // 16 codes in 4 bytes: field f of each byte, as (code ^ 2) - 2
          const uint2 w2 = *reinterpret_cast<const uint2*>(row + 8 * q);
          const uint32_t x = w2.x ^ 0xAAAAAAAAu, y = w2.y ^ 0xAAAAAAAAu;
          B0[u] = i32x4_t{sbytes2(x & 0x03030303u), sbytes2((x >> 2) & 0x03030303u), sbytes2((x >> 4) & 0x03030303u),
                          sbytes2((x >> 6) & 0x03030303u)};
          B1[u] = i32x4_t{sbytes2(y & 0x03030303u), sbytes2((y >> 2) & 0x03030303u), sbytes2((y >> 4) & 0x03030303u),
                          sbytes2((y >> 6) & 0x03030303u)};
        } else {
          const uint4 w = *reinterpret_cast<const uint4*>(row + 16 * q);
          B0[u] = i32x4_t{sbytes4(w.x & 0x0f0f0f0fu), sbytes4((w.x >> 4) & 0x0f0f0f0fu), sbytes4(w.y & 0x0f0f0f0fu),
                          sbytes4((w.y >> 4) & 0x0f0f0f0fu)};
          B1[u] = i32x4_t{sbytes4(w.z & 0x0f0f0f0fu), sbytes4((w.z >> 4) & 0x0f0f0f0fu), sbytes4(w.w & 0x0f0f0f0fu),
                          sbytes4((w.w >> 4) & 0x0f0f0f0fu)};
        }
        scv[u] = h2f(scs[(16 * u + n) * GC + k]);
      }
#pragma unroll
      for (int T = 0; T < NQ; ++T) {  // (quads past nq: zero tables, no stores)
        const uint4* tb = tsrc + (T * GC + k) * 128;
        const uint4 t0 = tb[(uint32_t(q) * 2) * 16 + uint32_t(n)];
        const uint4 t1 = tb[(uint32_t(q) * 2 + 1) * 16 + uint32_t(n)];
        const i32x4_t A0 = {int(t0.x), int(t0.y), int(t0.z), int(t0.w)};
        const i32x4_t A1 = {int(t1.x), int(t1.y), int(t1.z), int(t1.w)};
        const float ew = esrc[(T * GC + k) * 4 + q];
        i32x4_t D[U];
#pragma unroll
        for (int u = 0; u < U; ++u) D[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A0, B0[u], i32x4_t{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
        for (int u = 0; u < U; ++u) D[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A1, B1[u], D[u], 0, 0, 0);
#pragma unroll
        for (int u = 0; u < U; ++u) {
          const int lo = D[u][0] + int(uint32_t(D[u][1]) << 8), hi = D[u][2] + int(uint32_t(D[u][3]) << 8);
          const float f = fmaf(float(hi), 65536.0f, float(lo));
          acc[u][T] = fmaf(f, ew * scv[u], acc[u][T]);
        }
      }
    }
  };
  GmStage<BITS, U, GC> SA, SB;
  fetch_tables(c_begin, &s_tb0[0][0][0], &s_ew0[0][0][0]);
  issue(c_begin, &SA);
  __builtin_amdgcn_s_waitcnt(0);  // (the first tables; vmcnt, expcnt and lgkmcnt all 0)
  __syncthreads();
  // chunk c (tables in buffer b): its codes in `cur`, staged first (the wait is for them alone);
  // then the next chunk's tables into registers and its codes into `nxt` while c is
  // multiplied, then the tables into buffer b ^ 1 (last read by chunk c - 1, before the
  // previous barrier); the barrier is uniform (c_end is the workgroup's)
  // (s_waitcnt immediates: vmcnt in bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8; expcnt and
  // lgkmcnt left at their maxima)
  constexpr int kCodeLoads = int(G::NLD) + U;  // the loads of one issue()
  static_assert(kCodeLoads < 16, "");
  // The body has no branch (a branch around loads makes the compiler wait for every load in
  // flight where the paths join): a wave past the last unit works on unit 0's rows and stores
  // nothing, and the last chunk's "next" chunk is itself again (loads of data that exist, not
  // used).  The buffers come in as restrict pointers: the compiler then knows that the reads of
  // one do not wait for the loads into the other.  The barrier is a bare s_barrier: the only LDS
  // data other waves read are the tables, whose loads each wave has waited for (a fenced
  // __syncthreads would also wait for the code loads in flight); no table load is in flight
  // when the workgroup ends.
  auto body = [&](uint32_t c, const uint4* __restrict__ tcur, const float* __restrict__ ecur, uint4* __restrict__ tnxt,
                  float* __restrict__ enxt, uint8_t* __restrict__ sl, uint16_t* __restrict__ scs,
                  GmStage<BITS, U, GC>& cur, GmStage<BITS, U, GC>& nxt) {
    const uint32_t cn = c + 1 < c_end ? c + 1 : c;
    stage(cur, c, sl, scs);
    fetch_tables(cn, tnxt, enxt);
    __builtin_amdgcn_sched_barrier(0);  // (the table loads are issued before the code loads)
    issue(cn, &nxt);
    compute(tcur, ecur, sl, scs);
    __builtin_amdgcn_s_waitcnt(0x0F70 | kCodeLoads);  // the next tables have landed
    __builtin_amdgcn_s_barrier();
  };
  uint4* const tb0 = &s_tb0[0][0][0];
  uint4* const tb1 = &s_tb1[0][0][0];
  float* const ew0 = &s_ew0[0][0][0];
  float* const ew1 = &s_ew1[0][0][0];
  uint16_t* const scw = &s_sc[wave][0][0];
  for (uint32_t c = c_begin;; c += 2) {
    body(c, tb0, ew0, tb1, ew1, slot, scw, SA, SB);
    if (c + 1 >= c_end) break;
    body(c + 1, tb1, ew1, tb0, ew0, slot, scw, SB, SA);
    if (c + 2 >= c_end) break;
  }
  if (!active) return;
  // row n of unit u, tokens 4 T + q
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t uu = u0 + uint32_t(u);
    if (uu >= a.n_units) break;
    const bool row_ok = ur0[u] + uint32_t(n) < uwr[u];
    float* dst = a.partial + (size_t(range) * a.rows_all + uu * kBlockUnit + uint32_t(n)) * kMaxBlock;
#pragma unroll
    for (int T = 0; T < NQ; ++T) {
      const uint32_t tk = 4 * uint32_t(T) + uint32_t(q);
      if (tk < a.m) dst[tk] = row_ok ? acc[u][T] : 0.0f;
    }
  }
}

// Epilogue of blocks of up to kSmallBlock tokens (the partial sums and the input token-minor
// with stride kSmallBlock): a wave serves 4 outputs (16 lanes each: lane (i, e) = output i, correction entries
// e, e + 16, ..; after the 16-lane reduction lane (i, t) finishes token t of output i).
// Outputs: rows of part 0 (Store / Accum / Logits), gate row = up row (SwiGlu), RoPE pairs of
// every part (QkvRope).
template <int MODE>
__global__ void __launch_bounds__(256) k_block_epi8(BlockGemvArgs a) {
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr int NR = (kSwi || kRope) ? 2 : 1;  // rows per output
  const int lane = threadIdx.x & 63, e0 = lane & 15, i = lane >> 4, wave = threadIdx.x >> 6;
  const uint32_t m = a.m, ranges = a.ranges;
  const uint32_t half = a.g.rope.head_dim / 2;
  uint32_t total = 0;
  if constexpr (kRope) {
    for (int p = 0; p < a.g.n_parts; ++p) total += a.g.part[p].rows / 2;
  } else {
    total = a.g.part[0].rows;
  }
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  float sq = 0.0f;  // Accum: this lane's sum of y^2 over its token's updated rows
  const uint32_t pos0 = kRope ? a.state->pos : 0u;
  // token e0's break (k_block_limbs): no KV append, the residual stays
  const bool brk = (kRope || MODE == int(GemvMode::Accum)) && uint32_t(e0) < m && a.brk[e0] != 0u;
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
    // the ranges' raw sums of token t = e0 of each row (requested before the corrections)
    const uint32_t t = uint32_t(e0);
    float sum_k[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const GemvPart& P = a.g.part[kSwi ? k : p];
      const uint32_t at = P.unit_begin * kBlockUnit + rows_k[k];
      float acc_s = 0.0f;
      if (ok && t < m)
        for (uint32_t rg = 0; rg < ranges; ++rg) acc_s += a.partial[(size_t(rg) * a.rows_all + at) * kSmallBlock + t];
      sum_k[k] = acc_s;
    }
    // corrections of each row, all tokens
    float cor[NR][kSmallBlock];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const GemvPart& P = a.g.part[kSwi ? k : p];
      const uint32_t r = rows_k[k];
      const float2* corr = P.corr;
      const uint32_t kmax = P.corr_kmax;
#pragma unroll
      for (int t = 0; t < int(kSmallBlock); ++t) cor[k][t] = 0.0f;
      if (corr != nullptr && ok && r < P.wrows) {
        // two entries per trip, their loads together (unused slots read entry 0, masked)
        for (uint32_t e = uint32_t(e0); e < kmax; e += 32) {
          const bool u1 = e + 16 < kmax;
          const float2 c0 = corr[size_t(r) * kmax + e];
          const float2 c1 = corr[size_t(r) * kmax + (u1 ? e + 16 : e)];
          const float w0 = c0.y, w1 = u1 ? c1.y : 0.0f;
          const float4* x0 = reinterpret_cast<const float4*>(a.t.xt + size_t(__float_as_uint(c0.x)) * kSmallBlock);
          const float4* x1 = reinterpret_cast<const float4*>(a.t.xt + size_t(__float_as_uint(c1.x)) * kSmallBlock);
          const float4 xa = x0[0], xb = x0[1], ya = x1[0], yb = x1[1];
          const float xs0[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
          const float xs1[8] = {ya.x, ya.y, ya.z, ya.w, yb.x, yb.y, yb.z, yb.w};
#pragma unroll
          for (int tt = 0; tt < int(kSmallBlock); ++tt) {  // padding entries (w = 0) are skipped
            float c = cor[k][tt];
            c = w0 != 0.0f ? fmaf(w0, xs0[tt], c) : c;
            c = w1 != 0.0f ? fmaf(w1, xs1[tt], c) : c;
            cor[k][tt] = c;
          }
        }
      }
#pragma unroll
      for (int t = 0; t < int(kSmallBlock); ++t) {
        float v = cor[k][t];
        v = pair_sum(v, 1);
        v = pair_sum(v, 2);
        v = pair_sum(v, 4);
        v = pair_sum(v, 8);
        cor[k][t] = v;
      }
    }
    // lane (i, t): token t of the output
    if (!ok || t >= m) continue;
    float v[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      float c = cor[k][0];
#pragma unroll
      for (int tt = 1; tt < int(kSmallBlock); ++tt) c = t == uint32_t(tt) ? cor[k][tt] : c;
      v[k] = sum_k[k] + c;
    }
    const GemvPart& P0 = a.g.part[kSwi ? 0 : p];
    const uint32_t r = rows_k[0];
    float* y = P0.y + size_t(t) * P0.rows;
    if constexpr (MODE == int(GemvMode::Store)) {
      y[r] = v[0] + (P0.bias ? P0.bias[r] : 0.0f);
    } else if constexpr (MODE == int(GemvMode::Accum)) {
      const bool upd = r < P0.wrows && !brk;  // rows past the tiles stay
      const float yo = y[r], yn = upd ? yo + v[0] : yo;
      if (upd) y[r] = yn;
      sq = fmaf(yn, yn, sq);
    } else if constexpr (kSwi) {
      y[r] = v[0] / (1.0f + expf(-v[0])) * v[1];  // silu(g)*u: :159-161, :1746-1748
    } else if constexpr (kRope) {
#pragma clang fp contract(off)
      const float lo = v[0] + (P0.bias ? P0.bias[r] : 0.0f);
      const float hi = v[1] + (P0.bias ? P0.bias[r + half] : 0.0f);
      const uint32_t pos = pos0 + t, d = r % (2 * half);
      float o0 = lo, o1 = hi;
      if (P0.rope_role < kRoleV && pos < a.rope_rows) {  // applyRope :195-216
        const float c = a.rope_cos[size_t(pos) * half + d], sn = a.rope_sin[size_t(pos) * half + d];
        o0 = lo * c - hi * sn;
        o1 = lo * sn + hi * c;
      }
      if (P0.rope_role == kRoleQ || P0.rope_role == kRoleStore) {  // (Store: as computed)
        y[r] = o0;
        y[r + half] = o1;
      } else if (!brk) {
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
  if constexpr (MODE == int(GemvMode::Accum)) {
    // the workgroup's sums of y^2 per token for the next GEMV's RMS norm (lanes e0 = t of the 4
    // outputs, then over the waves, in a fixed order)
    if (a.ssp_out) {
      float v = pair_sum(sq, 16);
      v = pair_sum(v, 32);
      __shared__ float s_sq[4][16];
      if (lane < 16) s_sq[wave][lane] = v;
      __syncthreads();
      if (threadIdx.x < kSmallBlock) {
        const uint32_t tk = threadIdx.x;
        a.ssp_out[size_t(blockIdx.x) * kMaxBlock + tk] = (s_sq[0][tk] + s_sq[1][tk]) + (s_sq[2][tk] + s_sq[3][tk]);
      }
    }
  }
}

// Epilogue of blocks of more than kSmallBlock tokens (token stride kMaxBlock): a wave serves
// 64 / TW outputs, TW lanes each (TW >= m): lane (i, t) = output i, token t.  Per token: the
// ranges' raw sums in range order, the outlier corrections of the row in entry order (w * x[col]
// of the token: the flat tiles' replace deltas, the cells' added outliers; the row's non-zero
// entries only, BlockGemvArgs::cpack), then the batch-1 step's epilogue.  Outputs: rows of part 0 (Store / Accum /
// Logits), gate row = up row (SwiGlu), RoPE pairs of every part (QkvRope).
template <int MODE, int TW>
__global__ void __launch_bounds__(256) k_block_epi(BlockGemvArgs a) {
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr bool kAcc = MODE == int(GemvMode::Accum);
  constexpr int NR = (kSwi || kRope) ? 2 : 1;  // rows per output
  constexpr int OPW = 64 / TW;                 // outputs per wave
  static_assert(TW <= int(kMaxBlock) && TW > int(kSmallBlock) && 64 % TW == 0, "");
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const uint32_t t = uint32_t(lane % TW), i = uint32_t(lane / TW);
  const uint32_t m = a.m, ranges = a.ranges;
  const bool live = t < m;
  const uint32_t half = a.g.rope.head_dim / 2;
  const size_t rstride = size_t(a.rows_all) * kMaxBlock;  // one range of the partial sums
  uint32_t total = 0;
  if constexpr (kRope) {
    for (int p = 0; p < a.g.n_parts; ++p) total += a.g.part[p].rows / 2;
  } else {
    total = a.g.part[0].rows;
  }
  float bv = -1e30f, sq = 0.0f;  // Logits: the lane's best value / index; Accum: Σy² of the token
  uint32_t bi = 0xffffffffu, nf = 0;
  const bool brk = (kRope || kAcc) && live && a.brk[t] != 0u;  // (k_block_limbs): no KV append, the residual stays
  const uint32_t pos0 = kRope ? a.state->pos : 0u;
  for (uint32_t ob = (blockIdx.x * 4 + uint32_t(wave)) * OPW; ob < total; ob += gridDim.x * 4 * OPW) {
    const uint32_t o = ob + i;
    // (every lane of an output's TW runs the sums: the correction entries are loaded one per
    // lane; lanes of tokens past m read stale partial sums and inputs and store nothing)
    if (o >= total) continue;
    // the output's part and rows
    int p = 0;
    uint32_t rows_k[NR];
    if constexpr (kRope) {
      uint32_t oo = o;
      while (p + 1 < a.g.n_parts && oo >= a.g.part[p].rows / 2) {
        oo -= a.g.part[p].rows / 2;
        ++p;
      }
      const uint32_t lo = (oo / half) * (2 * half) + oo % half;
      rows_k[0] = lo;
      rows_k[1] = lo + half;
    } else {
      rows_k[0] = o;
      if constexpr (kSwi) rows_k[1] = o;
    }
    // the rows' correction ranges, requested before the partial sums
    uint32_t e0[NR], e1[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const uint32_t* coff = a.coff[kSwi ? k : p];
      const bool has = coff != nullptr && rows_k[k] < a.g.part[kSwi ? k : p].wrows;
      e0[k] = has ? coff[rows_k[k]] : 0u;
      e1[k] = has ? coff[rows_k[k] + 1] : 0u;
    }
    float v[NR];
#pragma unroll
    for (int k = 0; k < NR; ++k) {
      const GemvPart& P = a.g.part[kSwi ? k : p];
      const uint32_t r = rows_k[k];
      const float* ps = a.partial + size_t(P.unit_begin * kBlockUnit + r) * kMaxBlock + t;
      float acc_s = 0.0f;  // (four loads in flight, added in range order)
      uint32_t rg = 0;
      for (; rg + 4 <= ranges; rg += 4) {
        const float p0 = ps[rg * rstride], p1 = ps[(rg + 1) * rstride];
        const float p2 = ps[(rg + 2) * rstride], p3 = ps[(rg + 3) * rstride];
        acc_s += p0;
        acc_s += p1;
        acc_s += p2;
        acc_s += p3;
      }
      for (; rg < ranges; ++rg) acc_s += ps[rg * rstride];
      float c = 0.0f;
      {
        // the row's non-zero entries (the padded table's terms in its order): TW entries in one
        // load, one per lane of the output, then each entry's column and weight from its lane
        // and 16 columns' loads in flight together (entries past the row's last repeat it and
        // add nothing)
        const float2* ce = a.cpack[kSwi ? k : p];
        const uint32_t ee = e1[k];
        const int g0 = lane & ~(TW - 1);  // the output's first lane
        for (uint32_t e = e0[k]; e < ee; e += TW) {
          const float2 mine = ce[e + t < ee ? e + t : ee - 1];
          const uint32_t n = ee - e < uint32_t(TW) ? ee - e : uint32_t(TW);
          for (uint32_t j = 0; j < n; j += 16) {  // (j + 15 < TW)
            float xc[16];
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
              const uint32_t col = __shfl(__float_as_uint(mine.x), g0 + int(j) + jj);
              xc[jj] = a.t.xt[size_t(col) * kMaxBlock + t];
            }
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
              const float w = __shfl(mine.y, g0 + int(j) + jj);
              c = j + uint32_t(jj) < n ? fmaf(w, xc[jj], c) : c;
            }
          }
        }
      }
      v[k] = acc_s + c;
    }
    if (!live) continue;
    const GemvPart& P0 = a.g.part[kSwi ? 0 : p];
    const uint32_t r = rows_k[0];
    float* y = P0.y + size_t(t) * P0.rows;
    if constexpr (MODE == int(GemvMode::Store)) {
      y[r] = v[0] + (P0.bias ? P0.bias[r] : 0.0f);
    } else if constexpr (kAcc) {
      const bool upd = r < P0.wrows && !brk;  // rows past the tiles stay
      const float yo = y[r], yn = upd ? yo + v[0] : yo;
      if (upd) y[r] = yn;
      sq = fmaf(yn, yn, sq);
    } else if constexpr (kSwi) {
      y[r] = v[0] / (1.0f + expf(-v[0])) * v[1];  // silu(g)*u: :159-161, :1746-1748
    } else if constexpr (kRope) {
#pragma clang fp contract(off)
      const float lo = v[0] + (P0.bias ? P0.bias[r] : 0.0f);
      const float hi = v[1] + (P0.bias ? P0.bias[r + half] : 0.0f);
      const uint32_t pos = pos0 + t, d = r % (2 * half);
      float o0 = lo, o1 = hi;
      if (P0.rope_role < kRoleV && pos < a.rope_rows) {  // applyRope :195-216
        const float cc = a.rope_cos[size_t(pos) * half + d], sn = a.rope_sin[size_t(pos) * half + d];
        o0 = lo * cc - hi * sn;
        o1 = lo * sn + hi * cc;
      }
      if (P0.rope_role == kRoleQ || P0.rope_role == kRoleStore) {  // (Store: as computed)
        y[r] = o0;
        y[r + half] = o1;
      } else if (!brk) {
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
    // per token over the wave's outputs (lanes t + TW i), then over the waves
    __shared__ float s_bv[4][TW];
    __shared__ uint32_t s_bi[4][TW], s_nf[4][TW];
#pragma unroll
    for (int off = TW; off < 64; off <<= 1) {
      const float ov = pair_val(bv, off);
      const uint32_t oi = pair_u(bi, off);
      nf |= pair_u(nf, off);
      if (better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
      }
    }
    if (lane < TW) {
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
  if constexpr (kAcc) {
    // the workgroup's sums of y^2 per token for the next GEMV's RMS norm (over the wave's
    // outputs, then over the waves, in a fixed order)
    if (a.ssp_out) {
      __shared__ float s_sq[4][TW];
#pragma unroll
      for (int off = TW; off < 64; off <<= 1) sq = pair_sum(sq, off);
      if (lane < TW) s_sq[wave][lane] = sq;
      __syncthreads();
      if (threadIdx.x < m) {
        const uint32_t tk = threadIdx.x;
        a.ssp_out[size_t(blockIdx.x) * kMaxBlock + tk] = (s_sq[0][tk] + s_sq[1][tk]) + (s_sq[2][tk] + s_sq[3][tk]);
      }
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

void launch_block_limbs(const BlockGemvArgs& a, hipStream_t st) {
  const dim3 grid((a.g.C + 1023) / 1024, 4 * a.nq);
  const uint32_t chk = GemvMode(a.g.mode) == GemvMode::QkvRope ? a.g.rope.brk_check : 0u;
  auto go = [&](auto kern, uint32_t c) {
    launch_kernel(kern, grid, dim3(128), st, a.g.x, a.g.gamma, a.g.eps, a.g.C, a.m, a.ssp, a.n_ssp, a.t, a.brk, c, a.ts);
  };
  if (a.bits == 2) a.g.gamma ? go(&k_block_limbs<true, 2>, chk) : go(&k_block_limbs<false, 2>, 0u);
  else a.g.gamma ? go(&k_block_limbs<true, 4>, chk) : go(&k_block_limbs<false, 4>, 0u);
}

uint32_t block_gemv_ranges(uint32_t n_units, uint32_t C, uint32_t m) {
  if (m <= kSmallBlock) return (C + kBlockRange - 1) / kBlockRange;
  // k_block_gemm: the fewest ranges for the least time in rounds of one workgroup per CU, a
  // range costing about two chunks more (its partial sums written and read back)
  const uint32_t rb = (n_units + kGmWaves * kGmUnits - 1) / (kGmWaves * kGmUnits);
  const uint32_t nch = (C / 128 + kGmChunk - 1) / kGmChunk;
  constexpr uint32_t kSlots = 256;
  uint32_t best = 1, best_cost = 0xffffffffu;
  for (uint32_t R = 1; R <= nch; ++R) {
    const uint32_t rounds = (rb * R + kSlots - 1) / kSlots, cost = rounds * ((nch + R - 1) / R + 2);
    if (cost < best_cost) {
      best_cost = cost;
      best = R;
    }
  }
  return best;
}

uint32_t launch_block_gemv(BlockGemvArgs& a, hipStream_t st) {
  const uint32_t ranges = block_gemv_ranges(a.n_units, a.g.C, a.m);
  a.ranges = ranges;
  if (a.m > kSmallBlock) {  // output-stationary: row blocks of kGmWaves waves x kGmUnits units, few ranges
    const dim3 grid(ranges, (a.n_units + kGmWaves * kGmUnits - 1) / (kGmWaves * kGmUnits));
    if (a.bits == 2) launch_kernel(&k_block_gemm<2, kGmUnits, kGmChunk>, grid, dim3(kWave * kGmWaves), st, a);
    else launch_kernel(&k_block_gemm<4, kGmUnits, kGmChunk>, grid, dim3(kWave * kGmWaves), st, a);
  } else {
    // up to 8 tokens: ranges of 2048 columns (the tables of 2 quads in LDS), workgroups per
    // range: at most 256 workgroups of 8 waves in all, one round on the 256 CUs (one workgroup
    // per CU: the LDS tables and stage slots; a 257th workgroup would double the launch)
    uint32_t per = 256 / ranges;
    if (per == 0) per = 1;
    const uint32_t need = (a.n_units + 7) / 8;  // (a wave per unit at least)
    if (per > need) per = need;
    const dim3 grid(ranges, per);
    if (a.bits == 2) {
      if (a.nq <= 1) launch_kernel(&k_gemv_mt<1, 8, 2, 16>, grid, dim3(512), st, a);
      else launch_kernel(&k_gemv_mt<2, 8, 2, 16>, grid, dim3(512), st, a);
    } else {
      if (a.nq <= 1) launch_kernel(&k_gemv_mt<1, 8, 4, 16>, grid, dim3(512), st, a);
      else launch_kernel(&k_gemv_mt<2, 8, 4, 16>, grid, dim3(512), st, a);
    }
  }
  uint32_t outs = 0;
  if (GemvMode(a.g.mode) == GemvMode::QkvRope) {
    for (int p = 0; p < a.g.n_parts; ++p) outs += a.g.part[p].rows / 2;
  } else {
    outs = a.g.part[0].rows;
  }
  // up to kSmallBlock tokens: 16 outputs per workgroup (4 per wave, the correction entries over
  // 16 lanes); more: lanes per output = the token count rounded up to 16 or 32, one pass of 4 waves
  const bool small = a.m <= kSmallBlock;
  const uint32_t tw = a.m <= 16 ? 16u : 32u, per_wg = small ? 16u : 4 * (64 / tw);
  uint32_t eb = (outs + per_wg - 1) / per_wg;  // (one pass: the most latency chains in flight)
  if (GemvMode(a.g.mode) == GemvMode::Accum && eb > 1024) eb = 1024;  // (a Σy² partial per workgroup)
  if (GemvMode(a.g.mode) == GemvMode::Logits && eb > 512) eb = 512;   // (an argmax partial per workgroup)
  a.epi_blocks = eb;
  auto epi = [&](auto k8, auto k16, auto k32) {
    if (small) launch_kernel(k8, dim3(eb), dim3(256), st, a);
    else if (tw == 16) launch_kernel(k16, dim3(eb), dim3(256), st, a);
    else launch_kernel(k32, dim3(eb), dim3(256), st, a);
  };
#define CHPE_EPI(M) epi(&k_block_epi8<int(M)>, &k_block_epi<int(M), 16>, &k_block_epi<int(M), 32>)
  switch (GemvMode(a.g.mode)) {
    case GemvMode::Store: CHPE_EPI(GemvMode::Store); break;
    case GemvMode::Accum: CHPE_EPI(GemvMode::Accum); break;
    case GemvMode::SwiGlu: CHPE_EPI(GemvMode::SwiGlu); break;
    case GemvMode::Logits: CHPE_EPI(GemvMode::Logits); break;
    case GemvMode::QkvRope: CHPE_EPI(GemvMode::QkvRope); break;
  }
#undef CHPE_EPI
  return eb;
}

void launch_block_finish(const BlockFinishArgs& a, hipStream_t st) {
  launch_kernel(&k_block_finish, dim3(a.m), dim3(256), st, a);
}

}  // namespace chpe
