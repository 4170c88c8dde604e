// gemv.hip -- batch-1 GEMV over the archive's weight layouts, dequantised in registers.
//
// Work decomposition (wave64): a work unit is RU output rows.  Each lane owns a fixed chunk
// of columns per "panel" (the columns one 16-byte-per-lane load covers for one row: 2048 for
// 4-bit, 4096 for 2-bit, 512 for fp16).  For a panel a lane loads the RU rows' 16-byte code
// chunks first (RU loads in flight), then its x chunk (RMSNorm applied on the fly), so x is
// read once per RU rows.  Wide matrices split their panels over up to 8 waves of one
// workgroup, combined in LDS in a fixed order (deterministic); otherwise every wave owns its
// own units and the grid is persistent (grid-stride over units).
//
// Arithmetic per group of 128 weights: sum(q*x) - off*sum(x), times the fp16 group scale
// (the 4-bit weight is q-8, the 2-bit weight (c^2)-2), equal to the reference's
// sum((q-8)*x)*scale up to float rounding.  Outliers: added for 16-row cells (gemvTileW4
// :404-410), replacing for the tied LM head (unpackEmbedRowCell :1369-1378) and for flat tiles
// (gemvCellFlat :632-646, applied as per-row corrections prepared at load time).
#include <type_traits>

#include "device_common.hpp"
#include "kernels.hpp"

namespace chpe {
namespace {
using namespace dev;

// ---- layouts -------------------------------------------------------------------------
struct Cell16W4 {  // gemvTileW4 over 16x2048 group-128 cells (chpe_engine.zig:326-418)
  static constexpr int kCols = 32, kPanelCols = 2048, kPPW = 1;
  static constexpr float kOff = 8.0f;
  __device__ static bool lane_cols(uint32_t, int lane, uint32_t, uint32_t* c0) {
    *c0 = uint32_t(lane) * 32;
    return true;
  }
  __device__ static void locate(const GemvPart& P, uint32_t r, uint32_t, int lane, uint32_t, uint4* q,
                                float* s) {
    const uint8_t* cell = P.base + size_t(r >> 4) * P.stride;
    const uint32_t n = r & 15;
    *q = ld_u128(cell + 64 + n * 1024 + lane * 16);
    *s = h2f(ld_u16(cell + 16448 + 48 + 2 * (n * 16 + (lane >> 2))));
  }
  __device__ static float dot(uint4 q, const float* x, bool) { return dot32_w4(q, x); }
};

struct FlatW4 {  // gemvCellFlat, 4-bit group-128 (chpe_engine.zig:584-729)
  static constexpr int kCols = 32, kPanelCols = 2048, kPPW = 1;
  static constexpr float kOff = 8.0f;
  __device__ static bool lane_cols(uint32_t p, int lane, uint32_t C, uint32_t* c0) {
    const uint32_t g = p * 16 + (lane >> 2);
    *c0 = g * 128 + (lane & 3) * 32;
    return g < (C >> 7);
  }
  __device__ static void locate(const GemvPart& P, uint32_t r, uint32_t p, int lane, uint32_t C, uint4* q,
                                float* s) {
    const uint64_t G = uint64_t(r) * (C >> 7) + p * 16 + (lane >> 2);
    const uint8_t* cp = P.base + (G >> 8) * P.stride;
    const uint32_t gi = uint32_t(G & 255u);
    *q = ld_u128(cp + 64 + gi * 64 + (lane & 3) * 16);
    *s = h2f(ld_u16(cp + 16448 + 48 + 2 * gi));
  }
  __device__ static float dot(uint4 q, const float* x, bool) { return dot32_w4(q, x); }
};

struct FlatW2 {  // gemvCellFlat, 2-bit group-128
  static constexpr int kCols = 64, kPanelCols = 4096, kPPW = 1;
  static constexpr float kOff = 2.0f;
  __device__ static bool lane_cols(uint32_t p, int lane, uint32_t C, uint32_t* c0) {
    const uint32_t g = p * 32 + (lane >> 1);
    *c0 = g * 128 + (lane & 1) * 64;
    return g < (C >> 7);
  }
  __device__ static void locate(const GemvPart& P, uint32_t r, uint32_t p, int lane, uint32_t C, uint4* q,
                                float* s) {
    const uint64_t G = uint64_t(r) * (C >> 7) + p * 32 + (lane >> 1);
    const uint8_t* cp = P.base + (G >> 8) * P.stride;
    const uint32_t gi = uint32_t(G & 255u);
    *q = ld_u128(cp + 64 + gi * 32 + (lane & 1) * 16);
    *s = h2f(ld_u16(cp + 16448 + 48 + 2 * gi));
  }
  __device__ static float dot(uint4 q, const float* x, bool) { return dot64_w2(q, x); }
};

struct Raw16 {  // raw fp16 / bf16 tiles read as one row-major matrix (dotSegment :1194-1251)
  static constexpr int kCols = 8, kPanelCols = 512, kPPW = 4;
  static constexpr float kOff = 0.0f;
  __device__ static bool lane_cols(uint32_t p, int lane, uint32_t C, uint32_t* c0) {
    *c0 = p * 512 + uint32_t(lane) * 8;
    return *c0 < C;
  }
  __device__ static void locate(const GemvPart& P, uint32_t r, uint32_t p, int lane, uint32_t C, uint4* q,
                                float* s) {
    *q = ld_u128(P.base + (uint64_t(r) * C + p * 512 + lane * 8) * 2);
    *s = 1.0f;
  }
  __device__ static float dot(uint4 q, const float* x, bool bf16) { return dot8_f16(q, x, bf16); }
};

__device__ __forceinline__ int part_of(const GemvArgs& a, uint32_t unit) {
  int p = 0;
  while (p + 1 < a.n_parts && unit >= a.part[p + 1].unit_begin) ++p;
  return p;
}

// input element with RMSNorm applied on load: (x * inv) * gamma (rmsNorm :187-191)
__device__ __forceinline__ float xin(const GemvArgs& a, uint32_t c, float inv) {
  return a.gamma ? a.x[c] * inv * a.gamma[c] : a.x[c];
}

// Per-row terms outside the dense codes, added once per row (by the wave holding panel 0).
// P0 holds rows i < RU/2 of a SwiGlu unit (gate), P1 the rest (up); otherwise P0 == P1.
// For 16-row cells the outlier weights/columns load with the codes; x comes from LDS.
template <class F, int RU, bool kSwi, bool kReplace, bool kCellX>
__device__ __forceinline__ void apply_extras(const GemvArgs& a, const GemvPart& P0, const GemvPart& P1,
                                             uint32_t row_base, float (&acc)[RU], int lane, float inv,
                                             const float* s_x) {
  if constexpr (std::is_same_v<F, Cell16W4>) {
    // the unit's rows lie in one cell (two for SwiGlu: the gate cell and the up cell)
    const int k = lane & 7;  // outlier entry of this lane (lanes 8.. mirror lanes 0..7)
    uint32_t colA, colB;
    float w[RU];
    if constexpr (kReplace) {  // tied LM head: prepared (column, w_out - code) per cell
      const CellReplace& R = P0.repl[row_base >> 4];
      colA = colB = R.col[k];
#pragma unroll
      for (int i = 0; i < RU; ++i) w[i] = R.delta[(row_base + uint32_t(i)) & 15][k];
    } else {  // gemvTileW4: the payload's fp16 outlier weights are added (:309-315)
      const uint8_t* cA = P0.base + size_t(row_base >> 4) * P0.stride;
      const uint8_t* cB = P1.base + size_t(row_base >> 4) * P1.stride;
      colA = ld_u16(cA + 16448 + 816 + 2 * k);
      colB = kSwi ? ld_u16(cB + 16448 + 816 + 2 * k) : colA;
#pragma unroll
      for (int i = 0; i < RU; ++i) {
        const uint8_t* c = (kSwi && i >= RU / 2) ? cB : cA;
        const uint32_t n = (row_base + uint32_t(kSwi ? i % (RU / 2) : i)) & 15;
        w[i] = h2f(ld_u16(c + 16448 + 560 + 2 * (n * 8 + k)));
      }
    }
    // normalised x at the outlier columns: from the LDS mirror of the x chunk when present
    const float xoA = colA < a.C ? (kCellX ? s_x[colA] : xin(a, colA, inv)) : 0.0f;
    const float xoB = kSwi ? (colB < a.C ? (kCellX ? s_x[colB] : xin(a, colB, inv)) : 0.0f) : xoA;
    if (lane < 8) {
#pragma unroll
      for (int i = 0; i < RU; ++i) {
        const GemvPart& P = (kSwi && i >= RU / 2) ? P1 : P0;
        if (row_base + uint32_t(kSwi ? i % (RU / 2) : i) < P.rows)
          acc[i] += w[i] * ((kSwi && i >= RU / 2) ? xoB : xoA);
      }
    }
  } else if constexpr (std::is_same_v<F, FlatW4> || std::is_same_v<F, FlatW2>) {
#pragma unroll
    for (int i = 0; i < RU; ++i) {
      const GemvPart& P = (kSwi && i >= RU / 2) ? P1 : P0;
      const uint32_t r = row_base + uint32_t(kSwi ? i % (RU / 2) : i);
      if (!P.corr_ptr || r >= P.rows) continue;
      for (uint32_t j = P.corr_ptr[r] + lane; j < P.corr_ptr[r + 1]; j += kWave) {
        const float2 c = P.corr[j];
        acc[i] += c.y * xin(a, __float_as_uint(c.x), inv);
      }
    }
  }
}

template <int MODE>
__device__ __forceinline__ void store_row(const GemvPart& P, uint32_t r, float v, float* bv, uint32_t* bi,
                                          uint32_t* nf) {
  if (r >= P.rows) return;
  if constexpr (MODE == int(GemvMode::Store)) {
    P.y[r] = v + (P.bias ? P.bias[r] : 0.0f);
  } else if constexpr (MODE == int(GemvMode::Accum)) {
    P.y[r] = P.y[r] + v;
  } else if constexpr (MODE == int(GemvMode::Logits)) {
    P.y[r] = v;
    if (!isfinite(v)) *nf = 1;
    if (v > -1e30f && better(v, r, *bv, *bi)) { *bv = v; *bi = r; }
  }
}

// x chunk of panel p for this lane: raw values, normalised when `gamma` is set.  Returns
// sum of squares of the raw values (for the single-panel RMSNorm) in *sq.
template <class F>
__device__ __forceinline__ bool load_x(const GemvArgs& a, uint32_t p, int lane, float inv, bool normalise,
                                       float (&xr)[F::kCols], float* sx, float* sq) {
  uint32_t c0;
  const bool v = F::lane_cols(p, lane, a.C, &c0);
  float s = 0.0f, q2 = 0.0f;
  if (v) {
    const float4* x4 = reinterpret_cast<const float4*>(a.x + c0);
#pragma unroll
    for (int k = 0; k < F::kCols / 4; ++k) {
      const float4 t = x4[k];
      xr[4 * k] = t.x; xr[4 * k + 1] = t.y; xr[4 * k + 2] = t.z; xr[4 * k + 3] = t.w;
    }
#pragma unroll
    for (int k = 0; k < F::kCols; ++k) q2 = fmaf(xr[k], xr[k], q2);
    if (normalise) {
      const float4* g4 = reinterpret_cast<const float4*>(a.gamma + c0);
#pragma unroll
      for (int k = 0; k < F::kCols / 4; ++k) {
        const float4 g = g4[k];
        xr[4 * k] = xr[4 * k] * inv * g.x;
        xr[4 * k + 1] = xr[4 * k + 1] * inv * g.y;
        xr[4 * k + 2] = xr[4 * k + 2] * inv * g.z;
        xr[4 * k + 3] = xr[4 * k + 3] * inv * g.w;
      }
    }
#pragma unroll
    for (int k = 0; k < F::kCols; ++k) s += xr[k];
  } else {
#pragma unroll
    for (int k = 0; k < F::kCols; ++k) xr[k] = 0.0f;
  }
  *sx = s;
  *sq = q2;
  return v;
}

// occupancy floor per layout: the 16-row-cell kernels need more registers (outlier columns)
template <class F>
constexpr int kMinWavesPerSimd = 3;
template <>
constexpr int kMinWavesPerSimd<Cell16W4> = 2;

template <class F, int MODE, int RU, bool SINGLE>
__global__ void __launch_bounds__(512, kMinWavesPerSimd<F>) k_gemv(GemvArgs a) {
  constexpr int S = kWave / RU;  // lanes per row after the reduce-scatter
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr bool kPre = MODE == int(GemvMode::Store) || MODE == int(GemvMode::Accum);
  constexpr bool kCellX = std::is_same_v<F, Cell16W4> && SINGLE;  // outlier x from the LDS copy
  __shared__ float s_part[kMaxWavesPerUnit][RU];
  __shared__ float s_bv[8];
  __shared__ uint32_t s_bi[8], s_nf[8];
  __shared__ float s_x[SINGLE ? F::kPanelCols : 1];  // normalised input (single panel)
  __shared__ float s_red[kMaxWavesPerUnit];
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t NW = a.waves_per_unit, C = a.C;
  const uint32_t upb = NW == 1 ? blockDim.x / kWave : 1u;  // units per pass of the workgroup

  // RMSNorm statistics (sum of x^2 over the input) and, for a single panel, the lane's x
  // chunk, normalised once and reused for every unit of the wave.  Run after the first
  // unit's weight loads are issued so that their latency overlaps.
  float ss = 0.0f, inv = 1.0f, sx0 = 0.0f;
  float x0[SINGLE ? F::kCols : 1];
  bool pending = true;
  auto prologue = [&]() {
    if constexpr (SINGLE) {
      // the whole input (C <= one panel) is staged in LDS by the workgroup, normalised once,
      // then each lane keeps its chunk in registers; the LDS copy also serves the outlier
      // column lookups
      const int tid = threadIdx.x, nt = blockDim.x;
      float q2 = 0.0f;
      for (uint32_t i = uint32_t(tid) * 4; i < C; i += uint32_t(nt) * 4) {
        const float4 t = *reinterpret_cast<const float4*>(a.x + i);
        *reinterpret_cast<float4*>(s_x + i) = t;
        q2 = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, fmaf(t.w, t.w, q2))));
      }
      if (a.gamma || kLogits) {
        q2 = wave_sum(q2);
        if (lane == 0) s_red[wave] = q2;
        __syncthreads();
        for (int w = 0; w < nt / kWave; ++w) ss += s_red[w];
        if (a.gamma) {
          inv = 1.0f / sqrtf(ss / float(C) + a.eps);
          for (uint32_t i = uint32_t(tid) * 4; i < C; i += uint32_t(nt) * 4) {
            const float4 g = *reinterpret_cast<const float4*>(a.gamma + i);
            float4 t = *reinterpret_cast<float4*>(s_x + i);
            t.x = t.x * inv * g.x;
            t.y = t.y * inv * g.y;
            t.z = t.z * inv * g.z;
            t.w = t.w * inv * g.w;
            *reinterpret_cast<float4*>(s_x + i) = t;
          }
        }
      }
      __syncthreads();
      uint32_t c0;
      sx0 = 0.0f;
      if (F::lane_cols(0, lane, C, &c0)) {
#pragma unroll
        for (int k = 0; k < F::kCols / 4; ++k) {
          const float4 t = *reinterpret_cast<const float4*>(s_x + c0 + 4 * k);
          x0[4 * k] = t.x; x0[4 * k + 1] = t.y; x0[4 * k + 2] = t.z; x0[4 * k + 3] = t.w;
        }
      } else {
#pragma unroll
        for (int k = 0; k < F::kCols; ++k) x0[k] = 0.0f;
      }
#pragma unroll
      for (int k = 0; k < F::kCols; ++k) sx0 += x0[k];
    } else if (a.gamma || kLogits) {
      for (uint32_t b = uint32_t(lane) * 4; b < C; b += 256 * 8) {  // 8 x 16-byte loads per pass
        float4 t[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
          const uint32_t i = b + uint32_t(k) * 256;
          t[k] = i < C ? *reinterpret_cast<const float4*>(a.x + i) : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int k = 0; k < 8; ++k)
          ss = fmaf(t[k].x, t[k].x, fmaf(t[k].y, t[k].y, fmaf(t[k].z, t[k].z, fmaf(t[k].w, t[k].w, ss))));
      }
      ss = wave_sum(ss);
      if (a.gamma) inv = 1.0f / sqrtf(ss / float(C) + a.eps);
    }
    pending = false;
  };
  const uint32_t ppw = (a.n_panels + NW - 1) / NW;
  const uint32_t p0 = NW == 1 ? 0u : wave * ppw;
  const uint32_t p1 = NW == 1 ? a.n_panels : min(a.n_panels, p0 + ppw);

  float bv = -1e30f;  // Logits: running (max, first index) of the rows this thread owns
  uint32_t bi = 0xffffffffu, nf = 0;

  for (uint32_t u0 = blockIdx.x * upb; u0 < a.n_units; u0 += gridDim.x * upb) {
    const uint32_t unit = __builtin_amdgcn_readfirstlane(u0 + (NW == 1 ? wave : 0u));
    const bool active = unit < a.n_units;
    const int pu = kSwi ? 0 : __builtin_amdgcn_readfirstlane(part_of(a, active ? unit : 0u));
    const GemvPart P0 = a.part[pu];
    const GemvPart P1 = a.part[kSwi ? 1 : pu];
    // unit-local row i: SwiGlu = RU/2 rows of part 0 (gate), then the same rows of part 1 (up)
    const uint32_t row_base = kSwi ? unit * (RU / 2) : (unit - P0.unit_begin) * RU;
    // the epilogue's other operand (residual or bias), fetched with the weights
    float pre = 0.0f;
    const uint32_t own = row_base + uint32_t(lane / S);
    if constexpr (kPre) {
      if (NW == 1 && active && (lane % S) == 0 && own < P0.rows)
        pre = MODE == int(GemvMode::Accum) ? P0.y[own] : (P0.bias ? P0.bias[own] : 0.0f);
    }
    float acc[RU];
#pragma unroll
    for (int i = 0; i < RU; ++i) acc[i] = 0.0f;
    for (uint32_t p = p0; p < p1; ++p) {
      uint32_t c0;
      const bool v = active && F::lane_cols(p, lane, C, &c0);
      uint4 q[RU];
      float s[RU];
#pragma unroll
      for (int i = 0; i < RU; ++i) {  // all row loads first: RU 16-byte loads in flight
        const GemvPart& P = (kSwi && i >= RU / 2) ? P1 : P0;
        const uint32_t r = row_base + uint32_t(kSwi ? i % (RU / 2) : i);
        if (v && r < P.rows) {
          F::locate(P, r, p, lane, C, &q[i], &s[i]);
        } else {
          q[i] = make_uint4(0, 0, 0, 0);
          s[i] = 0.0f;
        }
      }
      if (pending) prologue();
      if (!active) continue;
      if constexpr (SINGLE) {
#pragma unroll
        for (int i = 0; i < RU; ++i) {
          const GemvPart& P = (kSwi && i >= RU / 2) ? P1 : P0;
          acc[i] += (F::dot(q[i], x0, P.bf16 != 0) - F::kOff * sx0) * s[i];
        }
      } else {
        float xr[F::kCols], sx, q2;
        load_x<F>(a, p, lane, inv, a.gamma != nullptr, xr, &sx, &q2);
#pragma unroll
        for (int i = 0; i < RU; ++i) {
          const GemvPart& P = (kSwi && i >= RU / 2) ? P1 : P0;
          acc[i] += (F::dot(q[i], xr, P.bf16 != 0) - F::kOff * sx) * s[i];
        }
      }
    }
    if (pending) prologue();
    if (active && p0 == 0) apply_extras<F, RU, kSwi, kLogits, kCellX>(a, P0, P1, row_base, acc, lane, inv, s_x);
    const float tot = wave_reduce_rows<RU>(acc, lane);
    if (NW == 1) {
      const int i = lane / S;
      const bool owner = active && (lane % S) == 0;
      if constexpr (kSwi) {
        const float u = __shfl(tot, (lane + 32) & 63);  // up row i sits 32 lanes above gate row i
        if (owner && i < RU / 2 && own < P0.rows)
          P0.y[own] = tot / (1.0f + expf(-tot)) * u;  // silu(g)*u: :159-161, :1746-1748
      } else if constexpr (kPre) {
        if (owner && own < P0.rows) P0.y[own] = MODE == int(GemvMode::Accum) ? pre + tot : tot + pre;
      } else if (owner) {
        store_row<MODE>(P0, own, tot, &bv, &bi, &nf);
      }
    } else {
      if (lane % S == 0) s_part[wave][lane / S] = tot;
      __syncthreads();
      const int t = threadIdx.x;
      if (t < RU) {
        float v = 0.0f;
        for (uint32_t w = 0; w < NW; ++w) v += s_part[w][t];
        if constexpr (kSwi) {
          if (t < RU / 2) {
            float u = 0.0f;
            for (uint32_t w = 0; w < NW; ++w) u += s_part[w][t + RU / 2];
            const uint32_t r = row_base + uint32_t(t);
            if (r < P0.rows) P0.y[r] = v / (1.0f + expf(-v)) * u;
          }
        } else {
          store_row<MODE>(P0, row_base + uint32_t(t), v, &bv, &bi, &nf);
        }
      }
      __syncthreads();
    }
  }
  if (pending) prologue();

  if constexpr (kLogits) {  // this workgroup's partial of the argmax scan
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      const float ov = __shfl_xor(bv, o);
      const uint32_t oi = __shfl_xor(bi, o);
      nf |= __shfl_xor(nf, o);
      if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { s_bv[wave] = bv; s_bi[wave] = bi; s_nf[wave] = nf; }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int w = 1; w < int(blockDim.x / kWave); ++w) {
        nf |= s_nf[w];
        if (better(s_bv[w], s_bi[w], bv, bi)) { bv = s_bv[w]; bi = s_bi[w]; }
      }
      a.partials[blockIdx.x] = ArgmaxPartial{bv, bi, nf, 0u};
      if (blockIdx.x == 0) a.result->hidden_norm = sqrtf(ss);
    }
  }
}

template <class F, int MODE, int RU>
void launch_one(const GemvArgs& a, const GemvLaunch& g, hipStream_t st) {
  if (a.n_panels == 1)
    launch_kernel(&k_gemv<F, MODE, RU, true>, dim3(g.blocks), dim3(g.threads), st, a);
  else
    launch_kernel(&k_gemv<F, MODE, RU, false>, dim3(g.blocks), dim3(g.threads), st, a);
}

template <class F>
void launch_layout(const GemvArgs& a, const GemvLaunch& g, hipStream_t st) {
  switch (GemvMode(a.mode)) {
    case GemvMode::Store: launch_one<F, int(GemvMode::Store), 8>(a, g, st); break;
    case GemvMode::Accum: launch_one<F, int(GemvMode::Accum), 8>(a, g, st); break;
    case GemvMode::SwiGlu: launch_one<F, int(GemvMode::SwiGlu), 8>(a, g, st); break;
    case GemvMode::Logits: launch_one<F, int(GemvMode::Logits), 8>(a, g, st); break;
  }
}

}  // namespace

GemvLaunch gemv_geometry(WeightKind kind, GemvMode mode, uint32_t C, const uint32_t* rows, int n_parts,
                         uint32_t* n_units, uint32_t* n_panels, uint32_t* waves_per_unit,
                         uint32_t* unit_begin) {
  const uint32_t ru = 8;
  uint32_t panel_cols = 2048, ppw = 1;
  switch (kind) {
    case WeightKind::Cell16W4: panel_cols = Cell16W4::kPanelCols; ppw = Cell16W4::kPPW; break;
    case WeightKind::FlatW4: panel_cols = FlatW4::kPanelCols; ppw = FlatW4::kPPW; break;
    case WeightKind::FlatW2: panel_cols = FlatW2::kPanelCols; ppw = FlatW2::kPPW; break;
    case WeightKind::Raw16: panel_cols = Raw16::kPanelCols; ppw = Raw16::kPPW; break;
  }
  *n_panels = (C + panel_cols - 1) / panel_cols;
  uint32_t nw = (*n_panels + ppw - 1) / ppw;
  if (nw > kMaxWavesPerUnit) nw = kMaxWavesPerUnit;
  *waves_per_unit = nw;
  uint32_t units = 0;
  if (mode == GemvMode::SwiGlu) {
    units = (rows[0] + ru / 2 - 1) / (ru / 2);
    unit_begin[0] = unit_begin[1] = 0;
  } else {
    for (int p = 0; p < n_parts; ++p) {
      unit_begin[p] = units;
      units += (rows[p] + ru - 1) / ru;
    }
  }
  *n_units = units;
  GemvLaunch g{};
  g.ru = ru;
  const uint32_t upb = nw == 1 ? 4 : 1;
  g.threads = nw == 1 ? 256 : nw * 64;
  g.blocks = (units + upb - 1) / upb;
  const uint32_t cap = mode == GemvMode::Logits ? kMaxLogitsBlocks : 8192u;
  if (g.blocks > cap) g.blocks = cap;
  return g;
}

void launch_gemv(WeightKind kind, const GemvArgs& a, const GemvLaunch& g, hipStream_t st) {
  switch (kind) {
    case WeightKind::Cell16W4: launch_layout<Cell16W4>(a, g, st); break;
    case WeightKind::FlatW4: launch_layout<FlatW4>(a, g, st); break;
    case WeightKind::FlatW2: launch_layout<FlatW2>(a, g, st); break;
    case WeightKind::Raw16: launch_layout<Raw16>(a, g, st); break;
  }
}

}  // namespace chpe
