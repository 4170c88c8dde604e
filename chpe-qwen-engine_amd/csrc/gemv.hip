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
#include <cstdio>
#include <cstdlib>
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
                                uint32_t* s) {
    const uint8_t* cell = P.base + size_t(r >> 4) * P.stride;
    const uint32_t n = r & 15;
    *q = ld_u128(cell + 64 + n * 1024 + lane * 16);
    *s = ld_u16(cell + 16448 + 48 + 2 * (n * 16 + (lane >> 2)));
  }
  __device__ static float scale(uint32_t s) { return h2f(uint16_t(s)); }
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
                                uint32_t* s) {
    const uint64_t G = uint64_t(r) * (C >> 7) + p * 16 + (lane >> 2);
    const uint8_t* cp = P.base + (G >> 8) * P.stride;
    const uint32_t gi = uint32_t(G & 255u);
    *q = ld_u128(cp + 64 + gi * 64 + (lane & 3) * 16);
    *s = ld_u16(cp + 16448 + 48 + 2 * gi);
  }
  __device__ static float scale(uint32_t s) { return h2f(uint16_t(s)); }
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
                                uint32_t* s) {
    const uint64_t G = uint64_t(r) * (C >> 7) + p * 32 + (lane >> 1);
    const uint8_t* cp = P.base + (G >> 8) * P.stride;
    const uint32_t gi = uint32_t(G & 255u);
    *q = ld_u128(cp + 64 + gi * 32 + (lane & 1) * 16);
    *s = ld_u16(cp + 16448 + 48 + 2 * gi);
  }
  __device__ static float scale(uint32_t s) { return h2f(uint16_t(s)); }
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
                                uint32_t* s) {
    *q = ld_u128(P.base + (uint64_t(r) * C + p * 512 + lane * 8) * 2);
    *s = 0;
  }
  __device__ static float scale(uint32_t) { return 1.0f; }
  __device__ static float dot(uint4 q, const float* x, bool bf16) { return dot8_f16(q, x, bf16); }
};

struct Raw8 {  // raw int8 tiles read as one row-major matrix, each dot times 0.00373708 (:1219-1237)
  static constexpr int kCols = 16, kPanelCols = 1024, kPPW = 4;
  static constexpr float kOff = 128.0f;  // the codes enter the dot as unsigned bytes (w + 128)
  __device__ static bool lane_cols(uint32_t p, int lane, uint32_t C, uint32_t* c0) {
    *c0 = p * 1024 + uint32_t(lane) * 16;
    return *c0 < C;
  }
  __device__ static void locate(const GemvPart& P, uint32_t r, uint32_t p, int lane, uint32_t C, uint4* q,
                                uint32_t* s) {
    *q = ld_u128(P.base + (uint64_t(r) * C + p * 1024 + lane * 16));
    *s = 0;
  }
  __device__ static float scale(uint32_t) { return 0.00373708f; }
  __device__ static float dot(uint4 q, const float* x, bool) { return dot16_i8p(q, x); }
};

__device__ __forceinline__ int part_of(const GemvArgs& a, uint32_t unit) {
  int p = 0;  // unrolled over the fixed part count: a loop here would precede the weight loads
#pragma unroll
  for (int k = 1; k < kMaxParts; ++k) p += (k < int(a.n_parts) && unit >= a.part[k].unit_begin) ? 1 : 0;
  return p;
}

template <int RU, bool kSwi>
__device__ __forceinline__ const GemvPart& row_part(const GemvPart& P0, const GemvPart& P1, int i) {
  return (kSwi && i >= RU / 2) ? P1 : P0;
}
// Row of unit-local row i.  SwiGlu: rows i and i + RU/2 are the same row of gate and up.
// QkvRope: rows i and i + RU/2 are the RoPE pair (j, j + head_dim/2) of one head.
template <int RU, int MODE>
__device__ __forceinline__ uint32_t row_of(uint32_t row_base, int i, uint32_t half) {
  if constexpr (MODE == int(GemvMode::SwiGlu)) return row_base + uint32_t(i % (RU / 2));
  else if constexpr (MODE == int(GemvMode::QkvRope))
    return row_base + (i < RU / 2 ? uint32_t(i) : half + uint32_t(i - RU / 2));
  else return row_base + uint32_t(i);
}

// A kernel-argument field as a uniform (scalar) value: selecting between two parts' fields per
// lane must not become a per-lane load from the argument block.
__device__ __forceinline__ uint32_t uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
// (pointers: global memory, kept visible to the compiler through the address-space casts)
template <class T>
__device__ __forceinline__ T* uni(T* p) {
  const uint64_t v = reinterpret_cast<uint64_t>(p);
  using G = __attribute__((address_space(1))) T*;
  const G g = reinterpret_cast<G>(uint64_t(uni(uint32_t(v))) | (uint64_t(uni(uint32_t(v >> 32))) << 32));
  return (T*)(g);
}

// v if ok, else +0 -- by bit masking, so that no branch separates a load from its use (a branch
// there makes the compiler wait for every outstanding load)
__device__ __forceinline__ float keep_if(bool ok, float v) {
  return __uint_as_float(__float_as_uint(v) & (ok ? 0xffffffffu : 0u));
}
__device__ __forceinline__ float4 keep_if(bool ok, float4 v) {
  return make_float4(keep_if(ok, v.x), keep_if(ok, v.y), keep_if(ok, v.z), keep_if(ok, v.w));
}

// The kernel-argument fields a GEMV reads before its first weight load, requested together:
// the empty asm consumes them all in scalar registers, so their loads are issued as one batch
// and waited for once (left to itself the scheduler interleaves them with the address
// arithmetic, and each later batch costs another round trip before the weights can be
// addressed).
template <int MODE>
__device__ __forceinline__ void args_batch(const GemvArgs& a) {
  const GemvPart& p0 = a.part[0];
  if constexpr (MODE == int(GemvMode::QkvRope)) {
    const GemvPart& p1 = a.part[1];
    const GemvPart& p2 = a.part[2];
    asm volatile("" ::"s"(p0.base), "s"(p0.stride), "s"(p0.rows), "s"(p0.unit_begin), "s"(p0.bias), "s"(p0.rope_role),
                 "s"(p1.base), "s"(p1.stride), "s"(p1.rows), "s"(p1.unit_begin), "s"(p1.bias), "s"(p1.rope_role),
                 "s"(p2.base), "s"(p2.stride), "s"(p2.rows), "s"(p2.unit_begin), "s"(p2.bias), "s"(p2.rope_role),
                 "s"(a.x), "s"(a.gamma), "s"(a.C), "s"(a.n_units), "s"(a.n_parts), "s"(a.rope.head_dim));
    asm volatile("" ::"s"(p0.corr), "s"(p0.corr_kmax), "s"(p0.wrows), "s"(p1.corr), "s"(p1.corr_kmax), "s"(p1.wrows),
                 "s"(p2.corr), "s"(p2.corr_kmax), "s"(p2.wrows));
  } else if constexpr (MODE == int(GemvMode::SwiGlu)) {
    const GemvPart& p1 = a.part[1];
    asm volatile("" ::"s"(p0.base), "s"(p0.stride), "s"(p0.rows), "s"(p0.y), "s"(p0.corr), "s"(p0.corr_kmax),
                 "s"(p1.base), "s"(p1.stride), "s"(p1.rows), "s"(p1.corr), "s"(p1.corr_kmax), "s"(a.x), "s"(a.gamma),
                 "s"(a.C), "s"(a.n_units), "s"(a.n_panels));
  } else if constexpr (MODE == int(GemvMode::Logits)) {
    asm volatile("" ::"s"(p0.base), "s"(p0.stride), "s"(p0.rows), "s"(p0.y), "s"(p0.corr), "s"(p0.corr_kmax),
                 "s"(p0.repl), "s"(a.x), "s"(a.gamma), "s"(a.C), "s"(a.n_units), "s"(a.n_panels));
  } else {
    asm volatile("" ::"s"(p0.base), "s"(p0.stride), "s"(p0.rows), "s"(p0.unit_begin), "s"(p0.y), "s"(p0.bias),
                 "s"(p0.corr), "s"(p0.corr_kmax), "s"(a.x), "s"(a.C), "s"(a.n_units), "s"(a.n_panels));
  }
}

// The q/k/v launch's part of a unit as a value: every field selected from the three parts'
// fields (loaded in the one batch above), not loaded again at an address that depends on the
// unit.  Other modes use part 0 (and part 1 for SwiGlu) at fixed offsets.
__device__ __forceinline__ GemvPart pick_part(const GemvArgs& a, int pu) {
  GemvPart p = a.part[0];
  const GemvPart& b = a.part[1];
  const GemvPart& c = a.part[2];
  p.base = pu == 0 ? p.base : (pu == 1 ? b.base : c.base);
  p.stride = pu == 0 ? p.stride : (pu == 1 ? b.stride : c.stride);
  p.rows = pu == 0 ? p.rows : (pu == 1 ? b.rows : c.rows);
  p.unit_begin = pu == 0 ? p.unit_begin : (pu == 1 ? b.unit_begin : c.unit_begin);
  p.y = pu == 0 ? p.y : (pu == 1 ? b.y : c.y);
  p.bias = pu == 0 ? p.bias : (pu == 1 ? b.bias : c.bias);
  p.rope_role = pu == 0 ? p.rope_role : (pu == 1 ? b.rope_role : c.rope_role);
  p.corr = pu == 0 ? p.corr : (pu == 1 ? b.corr : c.corr);
  p.corr_kmax = pu == 0 ? p.corr_kmax : (pu == 1 ? b.corr_kmax : c.corr_kmax);
  p.xcodes = pu == 0 ? p.xcodes : (pu == 1 ? b.xcodes : c.xcodes);
  p.wrows = pu == 0 ? p.wrows : (pu == 1 ? b.wrows : c.wrows);
  return p;
}

// Position of input column c in the workgroup's LDS copy: 16 bytes of padding after every 32
// columns, so that lanes reading consecutive 32-column chunks (128 bytes apart) start on
// different banks and a 16-byte-per-lane read is conflict-free.
__device__ __forceinline__ uint32_t xs_at(uint32_t c) { return c + ((c >> 5) << 2); }
// (+4 floats: a slot that absorbs the writes of threads past the input)
__host__ __device__ constexpr uint32_t xs_floats(uint32_t C) { return C + ((C + 31) >> 5) * 4 + 4; }
__device__ __forceinline__ uint32_t xs_spare(uint32_t C) { return xs_floats(C) - 4; }

// ---- per-unit terms outside the dense codes, loaded together with the weights -----------
// 16-row cells: lane i < RU serves unit row i: the 8 outlier columns of the row's cell and the
// row's 8 outlier weights (added, gemvTileW4 :404-410), or for the tied LM head the prepared
// (column, w_out - dequantised code) that makes the outlier replace the weight
// (unpackEmbedRowCell :1369-1378).  Two 16-byte loads (three for the replace table) per lane.
template <int RU>
struct CellExtras {
  uint4 cols;     // 8 u16 columns
  uint4 w0, w1;   // 8 fp16 weights (w0), or 8 f32 replace corrections (w0, w1)
  bool valid;
};

template <class F, int RU, int MODE>
__device__ __forceinline__ void load_cell_extras(const GemvPart& P0, const GemvPart& P1, uint32_t row_base,
                                                 uint32_t half, int lane, bool active, CellExtras<RU>* e) {
  // every lane loads (lanes >= RU and rows past the end read row 0 of the part); the values
  // are decoded where they are used, so the loads stay in flight together with the codes
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kReplace = MODE == int(GemvMode::Logits);
  const int i = lane;
  // the part's fields are read as uniform values and selected per lane (a per-lane choice of
  // the part itself would turn them into vector loads that stall the loads issued before)
  const bool second = kSwi && i >= RU / 2;
  const uint32_t rows = second ? uni(P1.rows) : uni(P0.rows);
  const uint32_t r = row_of<RU, MODE>(row_base, i < RU ? i : 0, half);
  e->valid = active && i < RU && r < rows;
  const uint32_t rr = e->valid ? r : 0u;
  if constexpr (kReplace) {
    const CellReplace* R = P0.repl + (rr >> 4);
    e->cols = *reinterpret_cast<const uint4*>(R->col);
    const uint4* d = reinterpret_cast<const uint4*>(R->delta[rr & 15]);
    e->w0 = d[0];
    e->w1 = d[1];
  } else {
    const uint8_t* base = second ? uni(P1.base) : uni(P0.base);
    const uint32_t stride = second ? uni(P1.stride) : uni(P0.stride);
    const uint8_t* cell = base + size_t(rr >> 4) * stride;
    e->cols = ld_u128(cell + 16448 + 816);
    e->w0 = ld_u128(cell + 16448 + 560 + (rr & 15) * 16);
    e->w1 = e->w0;
  }
}

// sum_k w[k] * x[col_k] of the lane's row (0 on lanes >= RU)
template <bool kReplace>
__device__ __forceinline__ float cell_outlier_sum(const CellExtras<8>& e, const float* s_x, uint32_t C) {
  const uint32_t cw[4] = {e.cols.x, e.cols.y, e.cols.z, e.cols.w};
  const uint32_t w0[4] = {e.w0.x, e.w0.y, e.w0.z, e.w0.w}, w1[4] = {e.w1.x, e.w1.y, e.w1.z, e.w1.w};
  float o = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t c = (k & 1) ? (cw[k >> 1] >> 16) : (cw[k >> 1] & 0xffffu);
    float w;
    if constexpr (kReplace) w = __uint_as_float(k < 4 ? w0[k] : w1[k - 4]);
    else w = (k & 1) ? half_hi(w0[k >> 1]) : half_lo(w0[k >> 1]);
    // branch-free: every entry reads LDS (at column 0 when absent), so the reads issue together
    const float t = fmaf(w, s_x[xs_at(c < C ? c : 0u)], o);
    o = c < C ? t : o;
  }
  return e.valid ? o : 0.0f;
}

// Flat tiles: outliers replace weights (gemvCellFlat :632-646), applied as per-row corrections
// (w_out - dequantised code) * x[col] prepared at load time.  Lane l serves unit row l >> 3 --
// the row it owns after the reduce-scatter -- and entries (l & 7) + 8 j of that row's list.
constexpr int kCorrSlots = int(kMaxCorrPerRow) / 8;
struct FlatExtras {
  float2 e[kCorrSlots];  // (column bits, correction) as loaded
  uint32_t use;          // bit j: slot j is an entry of the row (applied at use, not at load)
};
struct NoExtras {};

template <int RU, int MODE>
__device__ __forceinline__ void load_flat_extras(const GemvPart& P0, const GemvPart& P1, uint32_t row_base,
                                                 uint32_t half, int lane, bool enable, const float* x_any,
                                                 FlatExtras* f) {
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  const int i = lane >> 3;
  const bool second = kSwi && i >= RU / 2;  // uniform fields selected per lane (see load_cell_extras)
  const float2* corr = second ? uni(P1.corr) : uni(P0.corr);
  const uint32_t kmax = second ? uni(P1.corr_kmax) : uni(P0.corr_kmax);
  const uint32_t rows = second ? uni(P1.rows) : uni(P0.rows);
  const uint32_t r = row_of<RU, MODE>(row_base, i, half);
  const bool ok = enable && corr != nullptr && r < rows;
  // every slot loads (absent ones: the first entry of a valid table, or of the input vector
  // when there is no table) and is masked afterwards
  const float2* src = corr ? corr : reinterpret_cast<const float2*>(x_any);
  uint32_t m = 0;
#pragma unroll
  for (int j = 0; j < kCorrSlots; ++j) {
    const uint32_t k = uint32_t(lane & 7) + 8u * uint32_t(j);
    const bool use = ok && k < kmax;
    f->e[j] = src[use ? size_t(r) * kmax + k : 0];
    m |= uint32_t(use) << j;
  }
  f->use = m;
}

// sum over the lane's entries (x from the workgroup's normalised copy), then over the 8 lanes
// of its row
__device__ __forceinline__ float flat_correction(const FlatExtras& f, const float* s_x) {
  float cs = 0.0f;
#pragma unroll
  for (int j = 0; j < kCorrSlots; ++j) {
    // branch-free: every slot reads LDS (at column 0 when unused), so the reads issue together
    const bool on = ((f.use >> j) & 1u) && f.e[j].y != 0.0f;
    const float t = fmaf(f.e[j].y, s_x[xs_at(on ? __float_as_uint(f.e[j].x) : 0u)], cs);
    cs = on ? t : cs;
  }
  cs = pair_sum(cs, 1);
  cs = pair_sum(cs, 2);
  cs = pair_sum(cs, 4);
  return cs;
}

// The workgroup's copy of the input in LDS, normalised (x * inv) * gamma when `gamma` is set
// (rmsNorm :187-191); *ss = sum of x^2 over the input (also the LM head's hidden norm).
// Split in two so that the input's loads are issued before the weights' and the staging (its
// barriers included) overlaps the weights' latency: stage_x_issue loads up to 32 floats per
// thread into registers, stage_x_finish completes the staging (wider inputs take a two-pass
// path over LDS in stage_x_finish).
template <int SL>  // float4 slots per thread
struct StageRegs {
  float4 xs[SL], gs[SL];
};

// branch-free: every slot loads (past the input: its first float4) and is masked when used, so
// that the wait for these loads does not also wait for the weights issued after them
// NT: the workgroup size when fixed at compile time (0: blockDim.x, an argument load)
template <bool kNorm, int SL, int NT = 0, uint32_t CFIX = 0>
__device__ __forceinline__ void stage_x_issue(const GemvArgs& a, StageRegs<SL>* r) {
  const uint32_t C = CFIX ? CFIX : a.C, tid = threadIdx.x, nt = NT ? uint32_t(NT) : blockDim.x;
#pragma unroll
  for (int k = 0; k < SL; ++k) {
    const uint32_t i = (tid + uint32_t(k) * nt) * 4, ic = i < C ? i : 0u;
    r->xs[k] = *reinterpret_cast<const float4*>(a.x + ic);
    if constexpr (kNorm) r->gs[k] = *reinterpret_cast<const float4*>(a.gamma + ic);
  }
}

// kNorm: RMSNorm with the gains `gamma` (and the sum of squares, also the LM head's hidden norm);
// kWide: the input may exceed the register slots (then two passes over LDS).  Both are
// compile-time so that no runtime branch sits between the loads and their use.
// (NT, CFIX: the workgroup size and the input length when fixed at compile time)
template <bool kNorm, bool kWide, int SL, int NT = 0, uint32_t CFIX = 0>
__device__ __forceinline__ void stage_x_finish(const GemvArgs& a, const StageRegs<SL>& r, float* s_x, float* s_red,
                                               float* ss, float* inv) {
  const uint32_t C = CFIX ? CFIX : a.C, tid = threadIdx.x, nt = NT ? uint32_t(NT) : blockDim.x;
  const int lane = tid & 63, wave = tid >> 6;
  if constexpr (kWide) {  // two passes over LDS
    float q2 = 0.0f;
    for (uint32_t i = tid * 4; i < C; i += nt * 4) {
      const float4 t = *reinterpret_cast<const float4*>(a.x + i);
      *reinterpret_cast<float4*>(s_x + xs_at(i)) = t;
      q2 = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, fmaf(t.w, t.w, q2))));
    }
    if constexpr (kNorm) {
      q2 = wave_sum(q2);
      if (lane == 0) s_red[wave] = q2;
      __syncthreads();
      float t = 0.0f;
      for (uint32_t w = 0; w < nt / kWave; ++w) t += s_red[w];
      *ss = t;
      const float iv = 1.0f / sqrtf(t / float(C) + a.eps);
      *inv = iv;
      for (uint32_t i = tid * 4; i < C; i += nt * 4) {
        const float4 g = *reinterpret_cast<const float4*>(a.gamma + i);
        float4 v = *reinterpret_cast<float4*>(s_x + xs_at(i));
        v.x = v.x * iv * g.x;
        v.y = v.y * iv * g.y;
        v.z = v.z * iv * g.z;
        v.w = v.w * iv * g.w;
        *reinterpret_cast<float4*>(s_x + xs_at(i)) = v;
      }
    }
    __syncthreads();
    return;
  } else {
    float iv = 1.0f;
    if constexpr (kNorm) {
      float q2 = 0.0f;
#pragma unroll
      for (int k = 0; k < SL; ++k) {
        const float4 t = keep_if((tid + uint32_t(k) * nt) * 4 < C, r.xs[k]);
        q2 = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, fmaf(t.w, t.w, q2))));
      }
      q2 = wave_sum(q2);
      if (lane == 0) s_red[wave] = q2;
      __syncthreads();
      float t = 0.0f;
      for (uint32_t w = 0; w < nt / kWave; ++w) t += s_red[w];
      *ss = t;
      iv = 1.0f / sqrtf(t / float(C) + a.eps);
    }
    *inv = iv;
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      const uint32_t i = (tid + uint32_t(k) * nt) * 4;
      float4 v = r.xs[k];
      if constexpr (kNorm) {
        v.x = v.x * iv * r.gs[k].x;
        v.y = v.y * iv * r.gs[k].y;
        v.z = v.z * iv * r.gs[k].z;
        v.w = v.w * iv * r.gs[k].w;
      }
      *reinterpret_cast<float4*>(s_x + (i < C ? xs_at(i) : xs_spare(C))) = v;
    }
    __syncthreads();
  }
}

template <bool kNorm, int SL = 2>
__device__ __forceinline__ void stage_x(const GemvArgs& a, float* s_x, float* s_red, float* ss, float* inv) {
  StageRegs<SL> r;
  stage_x_issue<kNorm>(a, &r);
  stage_x_finish<kNorm, false>(a, r, s_x, s_red, ss, inv);
}

// the lane's input chunk of panel p from LDS, and its sum
template <class F>
__device__ __forceinline__ float lds_chunk(const float* s_x, uint32_t C, uint32_t p, int lane, float (&xr)[F::kCols]) {
  uint32_t c0;
  float s = 0.0f;
  if (F::lane_cols(p, lane, C, &c0)) {
#pragma unroll
    for (int k = 0; k < F::kCols / 4; ++k) {
      const float4 t = *reinterpret_cast<const float4*>(s_x + xs_at(c0 + 4 * k));
      xr[4 * k] = t.x; xr[4 * k + 1] = t.y; xr[4 * k + 2] = t.z; xr[4 * k + 3] = t.w;
    }
#pragma unroll
    for (int k = 0; k < F::kCols; ++k) s += xr[k];
  } else {
#pragma unroll
    for (int k = 0; k < F::kCols; ++k) xr[k] = 0.0f;
  }
  return s;
}

// Everything one work unit loads: dense codes + group scales of one panel, outlier terms, and
// the epilogue operand (residual or bias).  Issued before any arithmetic that needs them.
template <class F, int MODE>
struct UnitLoads {
  static constexpr int RU = 8;
  static constexpr bool kCell = std::is_same_v<F, Cell16W4>;
  static constexpr bool kFlat = std::is_same_v<F, FlatW4> || std::is_same_v<F, FlatW2>;
  uint32_t unit, row_base;
  int pu;
  uint4 q[RU];
  uint32_t s[RU];  // raw scale bits
  uint32_t vm;     // bit i: row i of the unit is present
  float rc, rs;    // QkvRope: cos / sin of the lane's RoPE pair (used when rope_ok)
  bool rope_ok;
  std::conditional_t<kCell, CellExtras<RU>, NoExtras> ce;
  std::conditional_t<kFlat, FlatExtras, NoExtras> fe;
  float pre;  // the epilogue operand of the lane's row (used when pre_ok)
  bool pre_ok;
};

template <class F, int MODE>
__device__ __forceinline__ void issue_panel(const GemvArgs& a, const GemvPart& P0, const GemvPart& P1, bool active,
                                            uint32_t row_base, uint32_t p, int lane, uint4 (&q)[8], uint32_t (&s)[8],
                                            uint32_t* vm) {
  // branch-free: absent rows / lanes read row 0 / panel 0 and are masked out in the sum
  constexpr int RU = 8;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  uint32_t c0;
  const bool lv = active && F::lane_cols(p, lane, a.C, &c0);
  const uint32_t half = a.rope.head_dim / 2;
  uint32_t m = 0;
#pragma unroll
  for (int i = 0; i < RU; ++i) {
    const GemvPart& P = row_part<RU, kSwi>(P0, P1, i);
    const uint32_t r = row_of<RU, MODE>(row_base, i, half);
    const bool ok = lv && r < P.rows;
    F::locate(P, ok ? r : 0u, ok ? p : 0u, lane, a.C, &q[i], &s[i]);
    m |= uint32_t(ok) << i;
  }
  *vm = m;
}

// sum of the panel's dense terms into acc
template <class F, int MODE>
__device__ __forceinline__ void panel_math(const GemvPart& P0, const GemvPart& P1, const uint4 (&q)[8],
                                           const uint32_t (&s)[8], uint32_t vm, const float* x, float sx,
                                           float (&acc)[8]) {
  constexpr int RU = 8;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  // row by row in load order, so that row i's arithmetic waits only for row i's loads and runs
  // while the later rows are still arriving (the scheduler would otherwise wait for all of them)
#pragma unroll
  for (int i = 0; i < RU; ++i) {
    const GemvPart& P = row_part<RU, kSwi>(P0, P1, i);
    const float t = (F::dot(q[i], x, P.bf16 != 0) - F::kOff * sx) * F::scale(s[i]);
    acc[i] += ((vm >> i) & 1u) ? t : 0.0f;
    __builtin_amdgcn_sched_barrier(0);
  }
}

// extras: the unit's outlier terms (cells), its correction entries (flat: only the wave
// `with_corr`), and for NW == 1 the epilogue operand of the lane's row
template <class F, int MODE>
__device__ __forceinline__ void issue_unit(const GemvArgs& a, uint32_t unit, uint32_t p, int lane, bool with_corr,
                                           bool with_pre, UnitLoads<F, MODE>* u) {
  constexpr int RU = 8, S = kWave / RU;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kPre = MODE == int(GemvMode::Store) || MODE == int(GemvMode::Accum) || kRope;
  const bool active = unit < a.n_units;
  const uint32_t half = a.rope.head_dim / 2;
  u->unit = unit;
  // only the q/k/v launch has several parts with units of their own; elsewhere the part is 0 at
  // compile time, so its fields are kernel-argument loads at fixed offsets, issued together
  // (a part chosen at run time costs a second dependent round of argument loads before the
  // first weight load can be addressed)
  u->pu = kRope ? __builtin_amdgcn_readfirstlane(part_of(a, active ? unit : 0u)) : 0;
  const GemvPart& P0 = a.part[u->pu];
  const GemvPart& P1 = a.part[kSwi ? 1 : u->pu];
  if constexpr (kSwi) {
    u->row_base = unit * (RU / 2);
  } else if constexpr (kRope) {  // RU/2 pairs per unit, half/(RU/2) units per head
    const uint32_t ul = unit - P0.unit_begin, per_head = half / (RU / 2);
    u->row_base = (ul / per_head) * (2 * half) + (ul % per_head) * (RU / 2);
  } else {
    u->row_base = (unit - P0.unit_begin) * RU;
  }
  // no branch before the loads: a branch would need its condition's argument loads first
  if constexpr (UnitLoads<F, MODE>::kCell) load_cell_extras<F, RU, MODE>(P0, P1, u->row_base, half, lane, active, &u->ce);
  if constexpr (UnitLoads<F, MODE>::kFlat) {  // (with_corr is wave-uniform and needs no argument load)
    u->fe.use = 0;
    if (with_corr) load_flat_extras<RU, MODE>(P0, P1, u->row_base, half, lane, active, a.x, &u->fe);
  }
  // Branch-free like the panel loads: each lane loads at a valid (clamped) address and the
  // flags say which values count; they are applied where the values are used, after the sums.
  const uint32_t own = row_of<RU, MODE>(u->row_base, lane / S, half);
  u->pre = 0.0f;
  u->pre_ok = false;
  if constexpr (kPre) {
    const float* src = MODE == int(GemvMode::Accum) ? P0.y : P0.bias;
    const bool ok = with_pre && active && (lane % S) == 0 && own < P0.rows && src != nullptr;
    u->pre = (src ? src : a.x)[ok ? own : 0u];
    u->pre_ok = ok;
  }
  if constexpr (kRope) {  // cos / sin of the pair (j, j + half) served by lane S * i, i < RU/2
    const bool ok = with_pre && active && (lane % S) == 0 && lane < 32 && P0.rope_role < kRoleV;
    const size_t at = ok ? (own % (2 * half)) : 0u;  // (the step's cos / sin row, staged)
    u->rc = a.rope.cos[at];
    u->rs = a.rope.sin[at];
    u->rope_ok = ok;
  }
  issue_panel<F, MODE>(a, P0, P1, active, u->row_base, p, lane, u->q, u->s, &u->vm);
}

// forwardDecode's non-finite break (StepState::broken), as the q/k/v and residual launches see
// it: loaded at the launch's start, whether an earlier launch of the step broke and (q/k/v) the
// input's first element.
struct BreakIn {
  uint32_t was;
  float x0;
};
template <int MODE>
__device__ __forceinline__ BreakIn break_in(const GemvArgs& a) {
  BreakIn b{0u, 0.0f};
  if constexpr (MODE == int(GemvMode::QkvRope) || MODE == int(GemvMode::Accum)) {
    // (global-address-space loads of uniform addresses, issued before any store of the kernel:
    // scalar loads, kept out of the vector registers)
    if (a.rope.state) b.was = gld(&a.rope.state->broken);
    if constexpr (MODE == int(GemvMode::QkvRope)) b.x0 = gld(a.x);
  }
  return b;
}
// Whether the launch leaves the KV cache (q/k/v) or the residual stream (o, down) alone.  The
// q/k/v launch tests its input (ss_bad: the input's sum of squares is not finite; the first
// element, RopeArgs::brk_check) and records a new break.  Every workgroup reaches the same
// answer from the same input; thread 0 of workgroup 0 stores it, so every thread of a q/k/v
// launch calls this outside lane-dependent branches.
template <int MODE>
__device__ __forceinline__ bool break_now(const GemvArgs& a, const BreakIn& b, bool ss_bad) {
  if constexpr (MODE == int(GemvMode::QkvRope)) {
    const uint32_t chk = a.rope.brk_check;
    // (uniform: kept in scalar registers)
    const bool now = __builtin_amdgcn_readfirstlane(((chk == 1u && ss_bad) || (chk == 2u && !isfinite(b.x0))) ? 1 : 0) != 0;
    if (now && b.was == 0u && blockIdx.x == 0 && threadIdx.x == 0) a.rope.state->broken = 1u;
    return now || b.was != 0u;
  } else {
    return b.was != 0u;
  }
}

// kRoleConv: channel c of the hybrid's depthwise causal conv with input x (k_dn_conv's
// arithmetic: the oldest tap first, the new input last, then SiLU); the state is shifted unless
// the step broke
__device__ __forceinline__ void conv_store(const RopeArgs& ra, const GemvPart& P, uint32_t c, float x, bool brk) {
#pragma clang fp contract(off)
  constexpr uint32_t T = kDnConvTaps;
  const float* w = ra.conv_w + size_t(c) * T;
  float* st = ra.conv_state + size_t(c) * (T - 1);
  float sv[T - 1];
#pragma unroll
  for (uint32_t k = 0; k + 1 < T; ++k) sv[k] = st[k];
  float acc = 0.0f;
#pragma unroll
  for (uint32_t k = 0; k + 1 < T; ++k) acc += w[k] * sv[k];
  acc += w[T - 1] * x;
  P.y[c] = acc / (1.0f + expf(-acc));
  if (brk) return;
#pragma unroll
  for (uint32_t k = 0; k + 2 < T; ++k) st[k] = sv[k + 1];
  st[T - 2] = x;
}

// QkvRope epilogue for the pair (r, r + half) of part P: bias added, then RoPE (q, k) with the
// reference's arithmetic (x0*cos - x1*sin, x0*sin + x1*cos, :212-213); q into y, k and v into
// the KV cache at `pos`, rounded to the cache type (not after a break: brk).  kRoleConv: both
// rows through the hybrid's conv (conv_store).
__device__ __forceinline__ void rope_store(const GemvArgs& a, const GemvPart& P, uint32_t r, float lo, float hi,
                                           float c, float sn, bool brk) {
#pragma clang fp contract(off)
  const uint32_t half = a.rope.head_dim / 2;
  if (P.rope_role == kRoleConv) {
    conv_store(a.rope, P, r, lo, brk);
    conv_store(a.rope, P, r + half, hi, brk);
    return;
  }
  float o0 = lo, o1 = hi;
  if (P.rope_role < kRoleV) {
    o0 = lo * c - hi * sn;
    o1 = lo * sn + hi * c;
  }
  if (P.rope_role == kRoleQ || P.rope_role == kRoleStore) {
    P.y[r] = o0;
    P.y[r + half] = o1;
    return;
  }
  if (brk) return;
  const uint32_t hd = a.rope.head_dim, head = r / hd, d = r % hd, pos = a.rope.state->pos;
  const size_t at = (size_t(head) * a.rope.max_seq + pos) * hd + d;
  void* cache = P.rope_role == kRoleK ? a.rope.k_cache : a.rope.v_cache;
  if (a.rope.kv_f16 && P.rope_role == kRoleV) {  // 4-position blocks: [pos/4][dim][pos%4]
    const size_t blk = (size_t(head) * a.rope.max_seq + (pos & ~3u)) * hd + (pos & 3u);
    reinterpret_cast<__half*>(cache)[blk + size_t(d) * 4] = __float2half_rn(o0);
    reinterpret_cast<__half*>(cache)[blk + size_t(d + half) * 4] = __float2half_rn(o1);
  } else if (a.rope.kv_f16) {
    reinterpret_cast<__half*>(cache)[at] = __float2half_rn(o0);
    reinterpret_cast<__half*>(cache)[at + half] = __float2half_rn(o1);
  } else {
    reinterpret_cast<float*>(cache)[at] = o0;
    reinterpret_cast<float*>(cache)[at + half] = o1;
  }
}

// final value v of unit row i (lane-owned): SwiGlu pairs gate row i with up row i + RU/2; the
// residual (Accum) stays as it is after a break (brk)
template <int MODE>
__device__ __forceinline__ void epilogue(const GemvPart& P0, uint32_t r, float v, float u, float pre, float* bv,
                                         uint32_t* bi, uint32_t* nf, bool brk = false) {
  if (r >= P0.rows) return;
  if constexpr (MODE == int(GemvMode::SwiGlu)) {
    P0.y[r] = v / (1.0f + expf(-v)) * u;  // silu(g)*u: :159-161, :1746-1748
  } else if constexpr (MODE == int(GemvMode::Accum)) {
    if (!brk) P0.y[r] = pre + v;
  } else if constexpr (MODE == int(GemvMode::Store)) {
    P0.y[r] = v + pre;
  } else {
    P0.y[r] = v;
    if (!isfinite(v)) *nf = 1;
    if (v > -1e30f && better(v, r, *bv, *bi)) { *bv = v; *bi = r; }
  }
}

template <int MODE>
__device__ __forceinline__ void argmax_partial(const GemvArgs& a, float bv, uint32_t bi, uint32_t nf,
                                               float* s_bv, uint32_t* s_bi, uint32_t* s_nf) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = pair_val(bv, o);
    const uint32_t oi = pair_u(bi, o);
    nf |= pair_u(nf, o);
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
  }
}

// The arithmetic and the epilogue of one unit of k_gemv_rows (row-by-row, see panel_math).
template <class F, int MODE>
__device__ __forceinline__ void rows_unit(const GemvArgs& a, const UnitLoads<F, MODE>& cur, const float* s_x,
                                          const float (&x0)[F::kCols], float sx0, int lane, float* bv,
                                          uint32_t* bi, uint32_t* nf, bool brk) {
  constexpr int RU = 8, S = kWave / RU;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  using U = UnitLoads<F, MODE>;
  const GemvPart& P0 = a.part[cur.pu];
  const GemvPart& P1 = a.part[kSwi ? 1 : cur.pu];
  float acc[RU];
#pragma unroll
  for (int i = 0; i < RU; ++i) acc[i] = 0.0f;
  panel_math<F, MODE>(P0, P1, cur.q, cur.s, cur.vm, x0, sx0, acc);
  if constexpr (F::kPPW > 1) {  // further panels (raw tiles)
    uint4 qn[RU];
    uint32_t sn[RU], vn;
    for (uint32_t p = 1; p < a.n_panels; ++p) {
      issue_panel<F, MODE>(a, P0, P1, cur.unit < a.n_units, cur.row_base, p, lane, qn, sn, &vn);
      float xr[F::kCols];
      const float sx = lds_chunk<F>(s_x, a.C, p, lane, xr);
      panel_math<F, MODE>(P0, P1, qn, sn, vn, xr, sx, acc);
    }
  }
  float tot = wave_reduce_rows<RU>(acc, lane);  // lane l: row l / S of the unit
  if constexpr (U::kCell) tot += __shfl(cell_outlier_sum<kLogits>(cur.ce, s_x, a.C), lane / S);
  if constexpr (U::kFlat) tot += flat_correction(cur.fe, s_x);
  const int i = lane / S;
  // SwiGlu / QkvRope: the partner of row i < RU/2 sits 32 lanes above it
  const float up = (kSwi || kRope) ? pair_val(tot, 32) : 0.0f;
  const float pre = cur.pre_ok ? cur.pre : 0.0f;
  const float up_pre = kRope ? pair_val(pre, 32) : 0.0f;
  if constexpr (kRope) {
    const uint32_t r = row_of<RU, MODE>(cur.row_base, i, a.rope.head_dim / 2);
    if ((lane % S) == 0 && i < RU / 2 && cur.unit < a.n_units && r < P0.rows)
      rope_store(a, P0, r, tot + pre, up + up_pre, cur.rope_ok ? cur.rc : 1.0f, cur.rope_ok ? cur.rs : 0.0f, brk);
  } else if ((lane % S) == 0 && (!kSwi || i < RU / 2) && cur.unit < a.n_units) {
    epilogue<MODE>(P0, row_of<RU, MODE>(cur.row_base, i, 0), tot, up, pre, bv, bi, nf, brk);
  }
}

// Modes whose input is the raw hidden state and which apply the layer's RMS norm while staging.
template <int MODE>
constexpr bool kNormOf = MODE == int(GemvMode::SwiGlu) || MODE == int(GemvMode::QkvRope) ||
                         MODE == int(GemvMode::Logits);

// The staging wave of k_gemv_rows: the whole input (C <= CMAX floats) into the workgroup's LDS
// copy, RMS-normalised (x * inv) * gamma when kNorm (rmsNorm :187-191); every load is issued
// before any use and this wave issues no other loads.  Returns the sum of squares (on every
// lane; also the LM head's hidden norm).
template <bool kNorm, uint32_t CMAX>
__device__ __forceinline__ float stage_wave(const GemvArgs& a, float* s_x, int lane) {
  constexpr int SL = int((CMAX + 255) / 256);  // float4 per lane
  const uint32_t C = a.C;
  float4 xs[SL], gs[SL];
#pragma unroll
  for (int k = 0; k < SL; ++k) {
    const uint32_t i = (uint32_t(lane) + 64u * uint32_t(k)) * 4, ic = i < C ? i : 0u;
    xs[k] = *reinterpret_cast<const float4*>(a.x + ic);
    if constexpr (kNorm) gs[k] = *reinterpret_cast<const float4*>(a.gamma + ic);
  }
  float ss = 0.0f, iv = 1.0f;
  if constexpr (kNorm) {
#pragma unroll
    for (int k = 0; k < SL; ++k) {
      const float4 t = keep_if((uint32_t(lane) + 64u * uint32_t(k)) * 4 < C, xs[k]);
      ss = fmaf(t.x, t.x, fmaf(t.y, t.y, fmaf(t.z, t.z, fmaf(t.w, t.w, ss))));
    }
    ss = wave_sum(ss);
    iv = 1.0f / sqrtf(ss / float(C) + a.eps);
  }
#pragma unroll
  for (int k = 0; k < SL; ++k) {
    const uint32_t i = (uint32_t(lane) + 64u * uint32_t(k)) * 4;
    float4 v = xs[k];
    if constexpr (kNorm) {
      v.x = v.x * iv * gs[k].x;
      v.y = v.y * iv * gs[k].y;
      v.z = v.z * iv * gs[k].z;
      v.w = v.w * iv * gs[k].w;
    }
    *reinterpret_cast<float4*>(s_x + (i < C ? xs_at(i) : xs_spare(C))) = v;
  }
  return ss;
}

// One wave = one unit of RU rows over all columns (NW == 1); the workgroup is kRowWaves such
// waves plus one staging wave that puts the (normalised) input into LDS, so the unit waves'
// loads are only weights and their arithmetic runs row by row as the rows arrive.  A wave
// whose grid is capped (the LM head) strides over further units.
constexpr int kRowWaves = 3;
template <class F, int MODE>
__global__ void __launch_bounds__(kWave * (kRowWaves + 1), 2) k_gemv_rows(GemvArgs a) {
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr bool kNorm = kNormOf<MODE>;
  using U = UnitLoads<F, MODE>;
  __shared__ __align__(16) float s_x[xs_floats(F::kPanelCols * F::kPPW)];
  __shared__ float s_bv[kRowWaves + 1];
  __shared__ uint32_t s_bi[kRowWaves + 1], s_nf[kRowWaves + 1];
  __shared__ uint32_t s_bad;  // QkvRope: the input's sum of squares is not finite
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t stride = gridDim.x * kRowWaves;
  const bool stager = wave == kRowWaves;
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  const BreakIn bin = break_in<MODE>(a);  // (before any store or asm: scalar loads)
  args_batch<MODE>(a);

  // The two roles are wave-uniform branches that each pass the same barriers (one after the
  // staging, one more in the LM head's argmax).  Keeping them apart means no value of a unit
  // wave's loads meets the staging wave's control flow, so nothing that uses those values can be
  // placed before the barrier (where it would wait for every weight load at once).
  if (stager) {
    const float ss = stage_wave<kNorm, F::kPanelCols * F::kPPW>(a, s_x, lane);
    if (kLogits && blockIdx.x == 0 && lane == 0) a.result->hidden_norm = sqrtf(ss);
    if (kRope && lane == 0) s_bad = isfinite(ss) ? 0u : 1u;
    __syncthreads();
    if constexpr (kLogits) argmax_partial<MODE>(a, -1e30f, 0xffffffffu, 0u, s_bv, s_bi, s_nf);
  } else {
    const uint32_t unit0 = blockIdx.x * kRowWaves + wave;
    U cur;
    issue_unit<F, MODE>(a, unit0, 0, lane, true, true, &cur);
    __syncthreads();
    const bool brk = break_now<MODE>(a, bin, kRope && s_bad != 0u);
    float x0[F::kCols];
    const float sx0 = lds_chunk<F>(s_x, a.C, 0, lane, x0);
    float bv = -1e30f;
    uint32_t bi = 0xffffffffu, nf = 0;
    if (unit0 < a.n_units) rows_unit<F, MODE>(a, cur, s_x, x0, sx0, lane, &bv, &bi, &nf, brk);
    for (uint32_t unit = unit0 + stride; unit < a.n_units; unit += stride) {
      U u;
      issue_unit<F, MODE>(a, unit, 0, lane, true, true, &u);
      rows_unit<F, MODE>(a, u, s_x, x0, sx0, lane, &bv, &bi, &nf, brk);
    }
    if constexpr (kLogits) argmax_partial<MODE>(a, bv, bi, nf, s_bv, s_bi, s_nf);
  }
}

// One workgroup = one unit, its panels split over NW waves (K-split); partial sums meet in LDS
// in a fixed order.  The input sits in LDS (dynamic, C floats) so that the flat-tile outlier
// corrections read any column; wave 0 adds them and writes the unit's rows.
template <class F, int MODE, bool kWide>
__global__ void __launch_bounds__(512, 2) k_gemv_split(GemvArgs a) {
  constexpr bool kNorm = kNormOf<MODE>;
  constexpr int RU = 8, S = kWave / RU;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  using U = UnitLoads<F, MODE>;
  extern __shared__ __align__(16) float s_x[];  // xs_floats(C) floats
  __shared__ float s_part[kMaxWavesPerUnit][RU];
  __shared__ float s_red[8], s_bv[8];
  __shared__ uint32_t s_bi[8], s_nf[8];
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const uint32_t NW = blockDim.x / kWave;
  const uint32_t ppw = (a.n_panels + NW - 1) / NW;
  const uint32_t p0 = wave * ppw, p1 = min(a.n_panels, p0 + ppw);

  const BreakIn bin = break_in<MODE>(a);  // (before any store or asm: scalar loads)
  args_batch<MODE>(a);
  U cur;
  uint32_t unit = blockIdx.x;
  StageRegs<8> xr0;
  if constexpr (!kWide) stage_x_issue<kNorm>(a, &xr0);  // the input first (see k_gemv_rows)
  issue_unit<F, MODE>(a, unit, p0, lane, wave == 0, false, &cur);
  float ss = 0.0f, inv = 1.0f;
  stage_x_finish<kNorm, kWide>(a, xr0, s_x, s_red, &ss, &inv);
  const bool brk = break_now<MODE>(a, bin, !isfinite(ss));

  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  for (; unit < a.n_units; unit += gridDim.x) {
    const GemvPart& P0 = a.part[cur.pu];
    const GemvPart& P1 = a.part[kSwi ? 1 : cur.pu];
    // epilogue operands of wave 0's rows, requested now so they overlap the arithmetic
    const uint32_t half = a.rope.head_dim / 2;
    float pre = 0.0f, rc = 1.0f, rs = 0.0f;
    if constexpr (MODE == int(GemvMode::Store) || MODE == int(GemvMode::Accum) || kRope) {
      const uint32_t own = row_of<RU, MODE>(cur.row_base, lane / S, half);
      if (wave == 0 && (lane % S) == 0 && own < P0.rows) {
        pre = MODE == int(GemvMode::Accum) ? P0.y[own] : (P0.bias ? P0.bias[own] : 0.0f);
        if constexpr (kRope) {
          if (lane < 32 && P0.rope_role < kRoleV) {
            const size_t at = own % (2 * half);
            rc = a.rope.cos[at];
            rs = a.rope.sin[at];
          }
        }
      }
    }
    float acc[RU];
#pragma unroll
    for (int i = 0; i < RU; ++i) acc[i] = 0.0f;
    for (uint32_t p = p0; p < p1; ++p) {
      if (p != p0) issue_panel<F, MODE>(a, P0, P1, unit < a.n_units, cur.row_base, p, lane, cur.q, cur.s, &cur.vm);
      float xr[F::kCols];
      const float sx = lds_chunk<F>(s_x, a.C, p, lane, xr);
      panel_math<F, MODE>(P0, P1, cur.q, cur.s, cur.vm, xr, sx, acc);
    }
    const float tot = wave_reduce_rows<RU>(acc, lane);
    if (lane % S == 0) s_part[wave][lane / S] = tot;
    __syncthreads();
    if (wave == 0) {
      const int i = lane / S;
      float v = 0.0f;
      for (uint32_t w = 0; w < NW; ++w) v += s_part[w][i];
      if constexpr (U::kFlat) v += flat_correction(cur.fe, s_x);
      const float up = (kSwi || kRope) ? pair_val(v, 32) : 0.0f;
      const float up_pre = kRope ? pair_val(pre, 32) : 0.0f;
      if constexpr (kRope) {
        const uint32_t r = row_of<RU, MODE>(cur.row_base, i, half);
        if (unit < a.n_units && (lane % S) == 0 && i < RU / 2 && r < P0.rows)
          rope_store(a, P0, r, v + pre, up + up_pre, rc, rs, brk);
      } else if (unit < a.n_units && (lane % S) == 0 && (!kSwi || i < RU / 2)) {
        epilogue<MODE>(P0, row_of<RU, MODE>(cur.row_base, i, 0), v, up, pre, &bv, &bi, &nf, brk);
      }
    }
    __syncthreads();
    if (unit + gridDim.x < a.n_units) issue_unit<F, MODE>(a, unit + gridDim.x, p0, lane, wave == 0, false, &cur);
  }
  if constexpr (kLogits) {
    if (blockIdx.x == 0 && threadIdx.x == 0) a.result->hidden_norm = sqrtf(ss);
    argmax_partial<MODE>(a, bv, bi, nf, s_bv, s_bi, s_nf);
  }
}

// 16-row cells at 2048 columns (the q/k/v, o and gate/up projections), K-split: one workgroup
// = UPW units of RU = 8 rows, kCellWaves = 4 waves x 512 columns.  Lane (j, c) = (lane / 16,
// lane % 16) of wave w holds rows j and j + 4 of every unit of the workgroup at columns
// 512 w + 32 c .. + 31 (one 16-byte code load and one group scale per row), so a unit's dot
// products run on four SIMDs at once instead of one; UPW > 1 shares one staging of the input
// between units (the gate/up projection has thousands).  Row sums meet over the 16 lanes of a
// row (DPP) and over the waves (LDS, in wave order); wave u then holds row i of unit u on lanes
// 8 i .. 8 i + 7, adds the outlier terms and runs the epilogue of the one-unit-per-wave kernel.
// Every load is issued before the input staging waits, with no branch in front of them.
constexpr int kCellWaves = 4;

// where unit u's rows start (the unit's part already chosen)
template <int MODE>
__device__ __forceinline__ uint32_t cells_row_base(const GemvPart& P0, uint32_t unit, uint32_t half) {
  constexpr int RU = 8;
  if constexpr (MODE == int(GemvMode::SwiGlu)) {
    return unit * (RU / 2);
  } else if constexpr (MODE == int(GemvMode::QkvRope)) {  // RU/2 pairs per unit, half/(RU/2) units per head
    const uint32_t ul = unit - P0.unit_begin, per_head = half / (RU / 2);
    return (ul / per_head) * (2 * half) + (ul % per_head) * (RU / 2);
  } else {
    return (unit - P0.unit_begin) * RU;
  }
}

template <int MODE, int UPW>
__global__ void __launch_bounds__(kWave * kCellWaves) k_gemv_cells(GemvArgs a) {
  constexpr int RU = 8, S = kWave / RU;
  constexpr bool kNorm = kNormOf<MODE>;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kPre = MODE == int(GemvMode::Store) || MODE == int(GemvMode::Accum) || kRope;
  static_assert(MODE != int(GemvMode::Logits), "the LM head stays on k_gemv_rows");
  static_assert(UPW >= 1 && UPW <= kCellWaves, "one epilogue wave per unit");
  __shared__ __align__(16) float s_x[xs_floats(2048)];
  __shared__ float s_part[kCellWaves][UPW * RU];
  __shared__ float s_red[kCellWaves];
  const int lane = threadIdx.x & 63, j = lane >> 4, c = lane & 15, i8 = lane >> 3;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const BreakIn bin = break_in<MODE>(a);  // (before any store or asm: scalar loads)
  args_batch<MODE>(a);
  const uint32_t half = a.rope.head_dim / 2, unit0 = blockIdx.x * UPW;

  // 1. the input first (its wait then leaves the later loads in flight), then per unit the codes
  // and scales of the lane's rows j and j + 4 (rows past the part read a row of it that exists
  // and count zero): unit rows 0..3 and 4..7 each lie in one cell (their first row is a
  // multiple of 4)
  StageRegs<2> xr;
  stage_x_issue<kNorm, 2, kWave * kCellWaves, 2048>(a, &xr);
  const uint32_t boff = wave * 256 + uint32_t(c) * 16, grp = wave * 4 + uint32_t(c >> 2);
  uint4 qA[UPW], qB[UPW];
  uint32_t sA[UPW], sB[UPW];
  bool okA[UPW], okB[UPW];
  // per unit, uniform: the two cells, their first rows and row counts, the row base, the part's
  // epilogue fields (kept for the epilogue wave of the unit)
  const uint8_t* cellA_[UPW];
  const uint8_t* cellB_[UPW];
  uint32_t rowA_[UPW], rowB_[UPW], rowsA_[UPW], rowsB_[UPW], rbase_[UPW];
  const float* src_[UPW];
  uint32_t role_[UPW];
#pragma unroll
  for (int u = 0; u < UPW; ++u) {
    const uint32_t unit = min(unit0 + u, a.n_units - 1);  // a unit past the end repeats the last, counting zero
    const bool live = unit0 + u < a.n_units;
    const GemvPart P0 = kRope ? pick_part(a, int(__builtin_amdgcn_readfirstlane(part_of(a, unit)))) : a.part[0];
    const GemvPart& P1 = kSwi ? a.part[1] : P0;
    const uint32_t row_base = cells_row_base<MODE>(P0, unit, half);
    const uint32_t rowA = row_of<RU, MODE>(row_base, 0, half), rowB = row_of<RU, MODE>(row_base, RU / 2, half);
    okA[u] = live && rowA + j < P0.rows;
    okB[u] = live && rowB + j < P1.rows;
    const uint32_t cA = rowA < P0.rows ? rowA : 0u, cB = rowB < P1.rows ? rowB : 0u;
    const uint8_t* cellA = P0.base + size_t(cA >> 4) * P0.stride;
    const uint8_t* cellB = P1.base + size_t(cB >> 4) * P1.stride;
    const uint32_t nA = (cA & 15u) + (rowA + j < P0.rows ? uint32_t(j) : 0u);
    const uint32_t nB = (cB & 15u) + (rowB + j < P1.rows ? uint32_t(j) : 0u);
    // (a scalar base plus one 32-bit vector offset per load; uni() keeps the constant in the
    // scalar base, where the compiler would otherwise fold it into a 64-bit vector address)
    const uint8_t* scA = uni(cellA + 16448 + 48);
    const uint8_t* scB = uni(cellB + 16448 + 48);
    qA[u] = ld_u128(cellA + (64 + nA * 1024 + boff));
    qB[u] = ld_u128(cellB + (64 + nB * 1024 + boff));
    sA[u] = ld_u16(scA + 2 * (nA * 16 + grp));
    sB[u] = ld_u16(scB + 2 * (nB * 16 + grp));
    cellA_[u] = cellA;
    cellB_[u] = cellB;
    rowA_[u] = live ? rowA : 0xffffffffu;  // (a unit past the end has no rows)
    rowB_[u] = live ? rowB : 0xffffffffu;
    rowsA_[u] = P0.rows;
    rowsB_[u] = P1.rows;
    rbase_[u] = row_base;
    src_[u] = MODE == int(GemvMode::Accum) ? P0.y : P0.bias;
    role_[u] = P0.rope_role;
  }
  // the epilogue operands of unit `wave` (when wave < UPW), its uniform values selected above:
  // outlier k = lane % 8 of unit row i8 (gemvTileW4 :404-410: the cell's 8 columns, the row's 8
  // weights); lane 8 i's residual or bias and RoPE factors
  const uint32_t ew = wave < uint32_t(UPW) ? wave : 0u;
  const uint8_t* eA = cellA_[0];
  const uint8_t* eB = cellB_[0];
  uint32_t erA = rowA_[0], erB = rowB_[0], ersA = rowsA_[0], ersB = rowsB_[0], erow_base = rbase_[0], erole = role_[0];
  const float* esrc = src_[0];
#pragma unroll
  for (int u = 1; u < UPW; ++u)
    if (ew == uint32_t(u)) {
      eA = cellA_[u]; eB = cellB_[u]; erA = rowA_[u]; erB = rowB_[u]; ersA = rowsA_[u]; ersB = rowsB_[u];
      erow_base = rbase_[u]; esrc = src_[u]; erole = role_[u];
    }
  const bool elive = wave < uint32_t(UPW) && unit0 + wave < a.n_units;
  const bool ohalf = i8 >= RU / 2;  // unit rows 4..7: the second cell
  const uint32_t orow = row_of<RU, MODE>(erow_base, i8, half);
  const uint32_t ofirst = ohalf ? erB : erA, oi = uint32_t(i8 & 3), k8 = uint32_t(lane & 7);
  const bool ovalid = elive && ofirst != 0xffffffffu && ofirst + oi < (ohalf ? ersB : ersA);
  // every lane reads its outlier from both cells through scalar bases and keeps one
  const uint8_t* oA = uni(eA + 16448);
  const uint8_t* oB = uni(eB + 16448);
  const uint32_t onA = erA != 0xffffffffu && erA + oi < ersA ? (erA & 15u) + oi : 0u;
  const uint32_t onB = erB != 0xffffffffu && erB + oi < ersB ? (erB & 15u) + oi : 0u;
  const uint32_t colA = ld_u16(oA + (816 + 2 * k8)), colB = ld_u16(oB + (816 + 2 * k8));
  const uint32_t wA = ld_u16(oA + (560 + 2 * (onA * 8 + k8))), wB = ld_u16(oB + (560 + 2 * (onB * 8 + k8)));
  const uint32_t ocol = ohalf ? colB : colA, ow = ohalf ? wB : wA;
  float pre = 0.0f, rc = 1.0f, rs = 0.0f;
  bool pre_ok = false, rope_ok = false;
  if constexpr (kPre) {
    pre_ok = elive && (lane % S) == 0 && orow < ersA && esrc != nullptr;
    pre = (esrc ? esrc : a.x)[pre_ok ? orow : 0u];
  }
  if constexpr (kRope) {
    rope_ok = elive && (lane % S) == 0 && lane < 32 && erole < kRoleV;
    const size_t at = rope_ok ? (orow % (2 * half)) : 0u;
    rc = a.rope.cos[at];
    rs = a.rope.sin[at];
  }

  // 2. the (normalised) input into LDS
  float ss = 0.0f, inv = 1.0f;
  stage_x_finish<kNorm, false, 2, kWave * kCellWaves, 2048>(a, xr, s_x, s_red, &ss, &inv);
  const bool brk = break_now<MODE>(a, bin, !isfinite(ss));

  // 3. per unit the lane's two 32-column dots, summed over the 16 lanes of each row, then over
  // the waves
  float xv[32];
  const uint32_t col0 = wave * 512 + uint32_t(c) * 32;
  float sx = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const float4 t = *reinterpret_cast<const float4*>(s_x + xs_at(col0 + 4 * k));
    xv[4 * k] = t.x; xv[4 * k + 1] = t.y; xv[4 * k + 2] = t.z; xv[4 * k + 3] = t.w;
  }
#pragma unroll
  for (int k = 0; k < 32; ++k) sx += xv[k];
#pragma unroll
  for (int u = 0; u < UPW; ++u) {
    float tA = (dot32_w4(qA[u], xv) - Cell16W4::kOff * sx) * Cell16W4::scale(sA[u]);
    float tB = (dot32_w4(qB[u], xv) - Cell16W4::kOff * sx) * Cell16W4::scale(sB[u]);
    tA = okA[u] ? tA : 0.0f;
    tB = okB[u] ? tB : 0.0f;
#pragma unroll
    for (int m = 1; m < 16; m <<= 1) {
      tA = pair_sum(tA, m);
      tB = pair_sum(tB, m);
    }
    if (c == 0) {
      s_part[wave][u * RU + j] = tA;
      s_part[wave][u * RU + j + RU / 2] = tB;
    }
  }
  __syncthreads();
  if (wave >= uint32_t(UPW)) return;

  // 4. wave u: row i8 of unit u with its outlier terms on the row's 8 lanes, then the epilogue
  float v = 0.0f;
#pragma unroll
  for (int w = 0; w < kCellWaves; ++w) v += s_part[w][wave * RU + i8];
  const float ox = s_x[xs_at(ocol < 2048u ? ocol : 0u)];
  float o = (ovalid && ocol < 2048u) ? half_lo(ow) * ox : 0.0f;
  o = pair_sum(o, 1);
  o = pair_sum(o, 2);
  o = pair_sum(o, 4);
  v += o;
  const float up = (kSwi || kRope) ? pair_val(v, 32) : 0.0f;
  const float prev = pre_ok ? pre : 0.0f;
  const float up_pre = kRope ? pair_val(prev, 32) : 0.0f;
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  if (!elive) return;
  // the epilogue's view of the unit's part (rows, output, KV role; base and stride unused)
  GemvPart E0 = a.part[0];
  E0.rows = ersA;
  if constexpr (kRope) {
    E0.rope_role = erole;
    E0.y = pick_part(a, int(__builtin_amdgcn_readfirstlane(part_of(a, min(unit0 + ew, a.n_units - 1))))).y;
    if ((lane % S) == 0 && i8 < RU / 2 && orow < E0.rows)
      rope_store(a, E0, orow, v + prev, up + up_pre, rope_ok ? rc : 1.0f, rope_ok ? rs : 0.0f, brk);
  } else if ((lane % S) == 0 && (!kSwi || i8 < RU / 2)) {
    epilogue<MODE>(E0, row_of<RU, MODE>(erow_base, i8, 0), v, up, prev, &bv, &bi, &nf, brk);
  }
}

// ---- 16-row cells on the matrix cores --------------------------------------------------------
// k_gemv_mma: the dense 4-bit products of the cell GEMVs at 2048 columns as exact integer matrix
// products (v_mfma_i32_16x16x64_i8).  A tile is 16 rows in two halves of 8 (QkvRope: 8 RoPE
// pairs (r, r + head_dim/2); otherwise one cell, rows 0..7 and 8..15) and a workgroup runs UPW
// tiles on 4 waves of 512 columns (4 groups of 128) each; a SwiGlu workgroup takes the gate cell
// and the up cell of the same 16 rows as its two tiles.
//
// Input: lane l of wave w holds columns 512 w + 8 l .. + 7 of x' (x * gamma in the modes that
// normalise: their 1/rms multiplies the row sums instead).  Per group (16 lanes) a power of two
// 2^(30-e) with max |x'| < 2^e scales x' to integers X (|X| <= 2^30: exact for every element
// within 2^7 of the group's largest, 2^(e-31) off otherwise), split into four signed bytes
// (limbs: X = L0 + 2^8 L1 + 2^16 L2 + 2^24 L3), written to the wave's LDS table in the byte
// order of the A operand.  A (lane (m, kq) = (lane % 16, lane / 16)): the 16 codes of row m at
// 16 columns of each quarter kq of a group, the nibbles as bytes (two masks and a shift per 8
// codes).  B column n = s + 4 limb holds limb `limb` of group slot s (zero in the products of the
// other slots), so one accumulator collects the wave's 4 groups x 4 limbs; it starts at -8 * (the
// limb summed over the group), the codes' offset, and stays exact: |sum (q - 8) L| <= 128 * 8 *
// 128.  Row sums: the limbs weighted 2^(8 limb) and by 2^(e-30) and added on DPP (row_shr 4, 8,
// 12), times the group scale, added over the 4 groups on DPP and over the waves in LDS (fixed
// order).  Then wave e < 2 UPW takes half e % 2 of tile e / 2 (rows 4h..4h+3 of each part,
// row i on lanes 8i..8i+7), adds the cell's outlier terms and runs the epilogue of the other
// cell kernels.  The only workgroup barrier is the one before the epilogue.
constexpr int kMmaWaves = 4;
constexpr int kMmaTable = 4 * 4 * 2 * 4;  // B table entries per wave: groups x quarters x halves x limbs

// first rows of the two 8-row halves of a tile (the tile's part already chosen; SwiGlu tiles are
// whole cells of the gate and the up projection, see k_gemv_mma)
template <int MODE>
__device__ __forceinline__ void mma_tile_rows(const GemvPart& P, uint32_t tile, uint32_t half, uint32_t* rA,
                                              uint32_t* rB) {
  if constexpr (MODE == int(GemvMode::QkvRope)) {  // half / 8 tiles per head
    const uint32_t tl = tile - P.unit_begin, per_head = half / 8;
    *rA = (tl / per_head) * (2 * half) + (tl % per_head) * 8;
    *rB = *rA + half;
  } else {
    *rA = (tile - P.unit_begin) * 16;
    *rB = *rA + 8;
  }
}


// The wave's 512 input columns (lane l: c0 .. c0 + 7; x' = x * gamma when kNorm) as the B
// operands of k_gemv_mma's products, through the wave's LDS table: the group exponent (max over
// the group's 16 lanes), the four signed-byte limbs per column in the A operand's byte order,
// the limb sums (the accumulators' start, -8 * sum) and 2^(e-30); x' also into s_x (for the
// outliers) and, when kNorm, the wave's sum of x^2 into s_red[wave].  Lane (n, kq) =
// (lane % 16, lane / 16) gets B[s][h] = limb n / 4 of group slot s = n % 4 (zero for the other
// slots) for quarter kq and half h, its accumulator start and its readout factor.
template <bool kNorm>
__device__ __forceinline__ void mma_stage(const float4& xa, const float4& xb, const float4& ga, const float4& gb,
                                          uint32_t wave, int lane, uint32_t c0, float* s_x, uint4* s_bw, int* s_sxw,
                                          float* s_ew, float* s_red, i32x4_t (&B)[4][2], int* cinit, float* lpf) {
  const int m = lane & 15, kq = lane >> 4;
  const float xv[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
  const float gv[8] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w};
  float xp[8], q2 = 0.0f, mx = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    xp[i] = kNorm ? xv[i] * gv[i] : xv[i];
    q2 = fmaf(xv[i], xv[i], q2);
    const float ax = fabsf(xp[i]);  // (a NaN counts as infinite: the group's factor becomes NaN)
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
  for (int i = 0; i < 8; ++i) z[i] = (uint32_t(int(xp[i] * up)) + 0x808080u) ^ 0x808080u;  // (toward zero)
  uint32_t lo[4], hi[4];
  limb_words(z[0], z[2], z[4], z[6], lo);
  limb_words(z[1], z[3], z[5], z[7], hi);
  const uint32_t gs = uint32_t(lane) >> 4, gkq = (uint32_t(lane) >> 2) & 3u, gh = (uint32_t(lane) >> 1) & 1u;
  uint2* tb = reinterpret_cast<uint2*>(s_bw);
#pragma unroll
  for (int L = 0; L < 4; ++L) tb[(((gs * 4 + gkq) * 2 + gh) * 4 + L) * 2 + (lane & 1)] = make_uint2(lo[L], hi[L]);
  // limb sums over the group: per lane 8 signed bytes (+1024, so that two 16-bit sums share a
  // word: 16 lanes x 2040 < 2^15), over the 16 lanes on DPP
  uint32_t lp[2];
#pragma unroll
  for (int P = 0; P < 2; ++P) {
    const int s0 = __builtin_amdgcn_sdot4(int(lo[2 * P]), 0x01010101, __builtin_amdgcn_sdot4(int(hi[2 * P]), 0x01010101, 1024, false), false);
    const int s1 = __builtin_amdgcn_sdot4(int(lo[2 * P + 1]), 0x01010101, __builtin_amdgcn_sdot4(int(hi[2 * P + 1]), 0x01010101, 1024, false), false);
    uint32_t w = uint32_t(s0) | (uint32_t(s1) << 16);
    w += pair_u(w, 1);
    w += pair_u(w, 2);
    w += pair_u(w, 4);
    w += pair_u(w, 8);
    lp[P] = w;
  }
  if ((lane & 15) == 0) {
#pragma unroll
    for (int L = 0; L < 4; ++L) s_sxw[gs * 4 + L] = -8 * (int((lp[L >> 1] >> (16 * (L & 1))) & 0xffffu) - 16 * 1024);
    s_ew[gs] = isfinite(mx) ? ldexpf(1.0f, e - 30) : __int_as_float(0x7fc00000);  // NaN / inf propagate
  }
  if (lane == 0) s_bw[kMmaTable] = make_uint4(0, 0, 0, 0);
  *reinterpret_cast<float4*>(s_x + xs_at(c0)) = make_float4(xp[0], xp[1], xp[2], xp[3]);
  *reinterpret_cast<float4*>(s_x + xs_at(c0) + 4) = make_float4(xp[4], xp[5], xp[6], xp[7]);
  if constexpr (kNorm) {
    q2 = wave_sum(q2);
    if (lane == 0) s_red[wave] = q2;
  }
  __builtin_amdgcn_wave_barrier();  // (one wave's LDS accesses execute in order)
  const uint32_t bs = uint32_t(m & 3), bl = uint32_t(m >> 2);
#pragma unroll
  for (int s = 0; s < 4; ++s)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t ent = bs == uint32_t(s) ? ((uint32_t(s) * 4 + uint32_t(kq)) * 2 + uint32_t(h)) * 4 + bl
                                             : uint32_t(kMmaTable);
      const uint4 t = s_bw[ent];
      B[s][h] = i32x4_t{int(t.x), int(t.y), int(t.z), int(t.w)};
    }
  *cinit = s_sxw[bs * 4 + bl];
  *lpf = s_ew[bs] * __int_as_float(int(127 + 8 * bl) << 23);  // * 2^(8 limb)
}

// One tile's 8 products (4 groups x 2 halves of 64 columns) and the wave's row sums: the limbs
// combined on DPP (row_shr 4, 8, 12: lanes 12..15 of each row), times the group scale, summed
// over the 4 groups (DPP); lane 12 of row kq writes tile rows 4 kq .. 4 kq + 3 to part[].
__device__ __forceinline__ void mma_tile(const uint4 (&q)[4], const uint32_t (&sc)[4], const i32x4_t (&B)[4][2],
                                         int cinit, float lpf, int lane, float* part) {
  i32x4_t D = {cinit, cinit, cinit, cinit};
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const uint32_t w[4] = {q[g].x, q[g].y, q[g].z, q[g].w};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t w0 = w[2 * h], w1 = w[2 * h + 1];
      const i32x4_t A = {int(w0 & 0x0f0f0f0fu), int((w0 >> 4) & 0x0f0f0f0fu), int(w1 & 0x0f0f0f0fu),
                         int((w1 >> 4) & 0x0f0f0f0fu)};
      D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B[g][h], D, 0, 0, 0);
    }
  }
  float t[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const float f = float(D[j]) * lpf;
    const float v = ((f + dpp_f<0x114>(f)) + dpp_f<0x118>(f)) + dpp_f<0x11c>(f);
    t[j] = v * h2f(uint16_t(sc[j]));
    t[j] = pair_sum(t[j], 1);
    t[j] = pair_sum(t[j], 2);
  }
  if ((lane & 15) == 12) *reinterpret_cast<float4*>(part + 4 * (lane >> 4)) = make_float4(t[0], t[1], t[2], t[3]);
}

template <int MODE, int UPW>
__global__ void __launch_bounds__(kWave * kMmaWaves) k_gemv_mma(GemvArgs a) {
  constexpr bool kNorm = kNormOf<MODE>;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kPre = MODE == int(GemvMode::Store) || MODE == int(GemvMode::Accum) || kRope;
  constexpr int S = 8;  // lanes per epilogue row
  static_assert(MODE != int(GemvMode::Logits), "the LM head stays on k_gemv_rows");
  static_assert(UPW == 1 || UPW == 2, "two epilogue waves per tile");
  static_assert(!kSwi || UPW == 2, "a SwiGlu workgroup holds the gate and the up cell");
  __shared__ __align__(16) float s_x[xs_floats(2048)];          // x' for the outlier terms
  __shared__ __align__(16) uint4 s_b[kMmaWaves][kMmaTable + 1];  // B table per wave (+ a zero entry)
  __shared__ int s_sx[kMmaWaves][4][4];                            // -8 * limb sums per group
  __shared__ float s_e[kMmaWaves][4];                              // 2^(e - 30) per group
  __shared__ __align__(16) float s_part[UPW][kMmaWaves][16];
  __shared__ float s_red[kMmaWaves];
  const int lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4, i8 = lane >> 3;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const BreakIn bin = break_in<MODE>(a);  // (before any store or asm: scalar loads)
  args_batch<MODE>(a);
  const uint32_t half = a.rope.head_dim / 2, tile0 = blockIdx.x * UPW;

  // 1. loads: the input (columns c0 .. c0 + 7 of x and gamma), then the weights
  const uint32_t c0 = wave * 512 + uint32_t(lane) * 8;
  const float4 xa = ld_f4(a.x + c0), xb = ld_f4(a.x + c0 + 4);
  float4 ga = make_float4(1.f, 1.f, 1.f, 1.f), gb = ga;
  if constexpr (kNorm) {
    ga = ld_f4(a.gamma + c0);
    gb = ld_f4(a.gamma + c0 + 4);
  }
  __builtin_amdgcn_sched_barrier(0);
  // per tile: where its two 8-row halves sit -- part A's cell (a uniform base), the halves'
  // rows in their cells and the byte distance to the second half's cell -- then lane m's codes
  // (A half: m < 8) in the wave's 4 groups and the group scales of rows 4 kq .. 4 kq + 3 in the
  // lane's readout slot (lane % 4).  Every address is that base plus one 32-bit lane offset.
  // Rows past a part read bytes of its last cell and are dropped in the epilogue.
  uint4 q[UPW][4];
  uint32_t sc[UPW][4];
  const uint8_t* cA_[UPW];
  uint32_t dB_[UPW], nA_[UPW], nB_[UPW], rA_[UPW], rB_[UPW], rows_[UPW], role_[UPW];
  const float* src_[UPW];
  float* y_[UPW];
#pragma unroll
  for (int u = 0; u < UPW; ++u) {
    uint32_t tile, rA, rB;
    bool live;
    GemvPart PA;
    if constexpr (kSwi) {  // workgroup = one unit: the gate cell (u = 0) and the up cell (u = 1)
      tile = blockIdx.x;
      live = true;
      PA = a.part[u];
      rA = tile * 16;
      rB = rA + 8;
    } else {
      tile = min(tile0 + u, a.n_units - 1);
      live = tile0 + u < a.n_units;
      PA = kRope ? pick_part(a, int(__builtin_amdgcn_readfirstlane(part_of(a, tile)))) : a.part[0];
      mma_tile_rows<MODE>(PA, tile, half, &rA, &rB);
    }
    const uint32_t rows = PA.rows, ca = rA >> 4, cb = rB < rows ? rB >> 4 : ca;  // (rA < rows)
    const uint8_t* cellA = PA.base + size_t(ca) * PA.stride;
    const uint32_t dB = (cb - ca) * PA.stride, nA0 = rA & 15u, nB0 = rB & 15u;
    const uint32_t vrow = m < 8 ? (nA0 + uint32_t(m)) * 1024u : dB + (nB0 + uint32_t(m - 8)) * 1024u;
    const uint8_t* cbase = uni(cellA + 64 + wave * 256);
    const uint32_t vo = vrow + uint32_t(kq) * 16;
#pragma unroll
    for (int g = 0; g < 4; ++g) q[u][g] = ld_u128(cbase + (vo + uint32_t(g) * 64));
    const uint32_t vs = (kq >= 2 ? dB + (nB0 + 4 * uint32_t(kq - 2)) * 32u : (nA0 + 4 * uint32_t(kq)) * 32u) +
                        2 * (wave * 4 + uint32_t(lane & 3));
    const uint8_t* sbase = uni(cellA + 16448 + 48);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) sc[u][jj] = ld_u16(sbase + (vs + uint32_t(jj) * 32));
    cA_[u] = cellA;
    dB_[u] = dB;
    nA_[u] = nA0;
    nB_[u] = nB0;
    rA_[u] = live ? rA : 0xffffffffu;
    rB_[u] = live ? rB : 0xffffffffu;
    rows_[u] = rows;
    role_[u] = PA.rope_role;
    src_[u] = MODE == int(GemvMode::Accum) ? PA.y : PA.bias;
    y_[u] = PA.y;
  }
  // the epilogue operands of wave e < 2 UPW, lane 8 i + k: outlier k of row i's cell
  // (gemvTileW4 :404-410: the cell's 8 columns, the row's 8 weights), lane 8 i's residual or bias
  // and RoPE factors.  SwiGlu: wave e < 2 takes rows 8 e + i of the gate and the up cell;
  // otherwise half eh = e % 2 of tile eu = e / 2 (i < 4: part A row 4 eh + i; i >= 4: part B row
  // 4 eh + i - 4).
  const uint32_t ew = wave < uint32_t(kSwi ? 2 : 2 * UPW) ? wave : 0u, eu = kSwi ? 0u : ew >> 1, eh = ew & 1u;
  const uint8_t* eA = cA_[0];
  uint32_t edB = dB_[0], enA = nA_[0], enB = nB_[0], erA = rA_[0], erB = rB_[0], erows = rows_[0], erole = role_[0];
  const float* esrc = src_[0];
  float* ey = y_[0];
  if constexpr (UPW == 2 && !kSwi) {
    if (eu == 1u) {
      eA = cA_[1]; edB = dB_[1]; enA = nA_[1]; enB = nB_[1]; erA = rA_[1]; erB = rB_[1]; erows = rows_[1];
      erole = role_[1]; esrc = src_[1]; ey = y_[1];
    }
  }
  const bool elive = wave < uint32_t(kSwi ? 2 : 2 * UPW) && (kSwi || tile0 + eu < a.n_units);
  const bool oB = !kSwi && i8 >= 4;
  const uint32_t oi = kSwi ? 8 * eh + uint32_t(i8) : 4 * eh + uint32_t(i8 & 3);
  const uint32_t orow = (oB ? erB : erA) + oi;
  const bool ovalid = elive && erA != 0xffffffffu && orow < erows;
  const uint32_t on = (oB ? enB : enA) + oi, ovo = oB ? edB : 0u, k8 = uint32_t(lane & 7);
  const uint8_t* obase = uni(eA + 16448);
  const uint32_t ocol = ld_u16(obase + (ovo + 816 + 2 * k8));
  const uint32_t ow = ld_u16(obase + (ovo + 560 + 2 * (on * 8 + k8)));
  uint32_t ocol2 = 0, ow2 = 0;  // SwiGlu: the up cell's outlier of the same row
  if constexpr (kSwi) {
    const uint8_t* obase2 = uni(cA_[UPW - 1] + 16448);
    ocol2 = ld_u16(obase2 + (816 + 2 * k8));
    ow2 = ld_u16(obase2 + (560 + 2 * (on * 8 + k8)));
  }
  float pre = 0.0f, rc = 1.0f, rs = 0.0f;
  bool pre_ok = false, rope_ok = false;
  if constexpr (kPre) {
    pre_ok = ovalid && (lane % S) == 0 && esrc != nullptr;
    pre = (esrc ? esrc : a.x)[pre_ok ? orow : 0u];
  }
  if constexpr (kRope) {  // the pair's dimension: (first row of part A mod head_dim) + 4 eh + i < half
    rope_ok = ovalid && (lane % S) == 0 && !oB && erole < kRoleV;
    const uint32_t fa = erA != 0xffffffffu ? erA : 0u, dA = fa - (fa / (2 * half)) * (2 * half);
    const size_t at = dA + 4 * eh + uint32_t(i8 & 3);
    rc = a.rope.cos[at];
    rs = a.rope.sin[at];
  }

  __builtin_amdgcn_sched_barrier(0);  // every load above is issued before the input is used

  // 2. the wave's B operands (wave-local LDS table), 3. the products of each tile
  i32x4_t B[4][2];
  int cinit;
  float lpf;
  mma_stage<kNorm>(xa, xb, ga, gb, wave, lane, c0, s_x, &s_b[wave][0], &s_sx[wave][0][0], &s_e[wave][0], s_red, B,
                   &cinit, &lpf);
#pragma unroll
  for (int u = 0; u < UPW; ++u) mma_tile(q[u], sc[u], B, cinit, lpf, lane, &s_part[u][wave][0]);
  __syncthreads();
  if (wave >= uint32_t(kSwi ? 2 : 2 * UPW)) return;

  // 4. wave e: rows of its tile half (SwiGlu: of both cells), the outlier terms, 1/rms, the epilogue
  const uint32_t tr = kSwi ? oi : (oB ? 8 + 4 * eh + uint32_t(i8 - 4) : 4 * eh + uint32_t(i8));
  float v = 0.0f, v2 = 0.0f;
#pragma unroll
  for (int w = 0; w < kMmaWaves; ++w) {
    v += s_part[eu][w][tr];
    if constexpr (kSwi) v2 += s_part[UPW - 1][w][tr];
  }
  float o = (ovalid && ocol < 2048u) ? half_lo(ow) * s_x[xs_at(ocol < 2048u ? ocol : 0u)] : 0.0f;
  o = pair_sum(o, 1);
  o = pair_sum(o, 2);
  o = pair_sum(o, 4);
  v += o;
  if constexpr (kSwi) {
    float o2 = (ovalid && ocol2 < 2048u) ? half_lo(ow2) * s_x[xs_at(ocol2 < 2048u ? ocol2 : 0u)] : 0.0f;
    o2 = pair_sum(o2, 1);
    o2 = pair_sum(o2, 2);
    o2 = pair_sum(o2, 4);
    v2 += o2;
  }
  float ss = 0.0f;
  if constexpr (kNorm) {
#pragma unroll
    for (int w = 0; w < kMmaWaves; ++w) ss += s_red[w];
    const float inv = 1.0f / sqrtf(ss / 2048.0f + a.eps);
    v *= inv;
    v2 *= inv;
  }
  const bool brk = break_now<MODE>(a, bin, !isfinite(ss));
  const float upv = kSwi ? v2 : (kRope ? pair_val(v, 32) : 0.0f);
  const float prev = pre_ok ? pre : 0.0f;
  const float up_pre = kRope ? pair_val(prev, 32) : 0.0f;
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  if (!elive) return;
  GemvPart E0 = a.part[0];
  E0.rows = erows;
  E0.y = ey;
  if constexpr (kRope) {
    E0.rope_role = erole;
    if ((lane % S) == 0 && !oB && ovalid)
      rope_store(a, E0, orow, v + prev, upv + up_pre, rope_ok ? rc : 1.0f, rope_ok ? rs : 0.0f, brk);
  } else if constexpr (kSwi) {
    if ((lane % S) == 0 && ovalid) epilogue<MODE>(E0, orow, v, upv, prev, &bv, &bi, &nf);
  } else {
    if ((lane % S) == 0 && ovalid) epilogue<MODE>(E0, orow, v, upv, prev, &bv, &bi, &nf, brk);
  }
}

// The LM head on the matrix cores: a persistent grid whose workgroups stage the final-normed
// input once (x * gamma; 1/rms multiplies the row sums) and stride over the 16-row cells, one
// cell per iteration on the 4 waves (the products of k_gemv_mma), the next cell's loads issued
// before the current cell's products; waves 0 and 1 finish rows 8 w .. 8 w + 7: the outliers
// replace weights through the prepared table of the tied head (unpackEmbedRowCell :1369-1378)
// or are added from the cell (untied cells, gemvTileW4 :404-410), then the logit and the
// workgroup's argmax partial (computeLmHead :1554-1660, argmax :1775-1803).
struct MmaCellLoads {
  uint4 q[4];
  uint32_t sc[4];
  uint32_t ocol, ow;  // outlier column and fp16 weight (added), or
  float od;           // the replace table's correction
};

__global__ void __launch_bounds__(kWave * kMmaWaves) k_gemv_mma_logits(GemvArgs a) {
  constexpr int MODE = int(GemvMode::Logits);
  __shared__ __align__(16) float s_x[xs_floats(2048)];
  __shared__ __align__(16) uint4 s_b[kMmaWaves][kMmaTable + 1];
  __shared__ int s_sx[kMmaWaves][4][4];
  __shared__ float s_e[kMmaWaves][4];
  __shared__ __align__(16) float s_part[2][kMmaWaves][16];
  __shared__ float s_red[kMmaWaves], s_bv[kMmaWaves];
  __shared__ uint32_t s_bi[kMmaWaves], s_nf[kMmaWaves];
  const int lane = threadIdx.x & 63, m = lane & 15, kq = lane >> 4, i8 = lane >> 3;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  args_batch<MODE>(a);
  const GemvPart& P = a.part[0];
  const uint32_t n_tiles = a.n_units, step = gridDim.x;
  const bool repl = P.repl != nullptr;
  const uint32_t c0 = wave * 512 + uint32_t(lane) * 8;
  const float4 xa = ld_f4(a.x + c0), xb = ld_f4(a.x + c0 + 4);
  const float4 ga = ld_f4(a.gamma + c0), gb = ld_f4(a.gamma + c0 + 4);
  __builtin_amdgcn_sched_barrier(0);
  if (a.hidden_out && blockIdx.x == 0) {  // the step's final hidden state, kept for the host
    *reinterpret_cast<float4*>(a.hidden_out + c0) = xa;
    *reinterpret_cast<float4*>(a.hidden_out + c0 + 4) = xb;
  }
  const uint32_t tr = 8 * (wave & 1u) + uint32_t(i8), k8 = uint32_t(lane & 7);
  const uint32_t vo = uint32_t(m) * 1024u + uint32_t(kq) * 16, vs = uint32_t(kq) * 128u + 2 * (wave * 4 + uint32_t(lane & 3));
  auto issue = [&](uint32_t tile, MmaCellLoads* t) {
    const uint8_t* cell = P.base + size_t(tile) * P.stride;
    const uint8_t* cbase = uni(cell + 64 + wave * 256);
#pragma unroll
    for (int g = 0; g < 4; ++g) t->q[g] = ld_u128(cbase + (vo + uint32_t(g) * 64));
    const uint8_t* sbase = uni(cell + 16448 + 48);
#pragma unroll
    for (int j = 0; j < 4; ++j) t->sc[j] = ld_u16(sbase + (vs + uint32_t(j) * 32));
    // branch-free: both kinds are loaded (the replace table's from the cell when there is none)
    const uint8_t* obase = uni(cell + 16448);
    const CellReplace* R = uni(P.repl + tile);
    const uint8_t* cp = repl ? reinterpret_cast<const uint8_t*>(R->col) : obase + 816;
    const uint8_t* dp = repl ? reinterpret_cast<const uint8_t*>(R->delta[0]) : obase + 560;
    t->ocol = ld_u16(cp + 2 * k8);
    t->od = gld(reinterpret_cast<const float*>(dp + 4 * (tr * 8 + k8) * (repl ? 1u : 0u)));
    t->ow = ld_u16(obase + (560 + 2 * (tr * 8 + k8)));
  };
  uint32_t tile = blockIdx.x;  // < n_tiles: the grid is at most the tile count
  MmaCellLoads L0, L1;
  issue(tile, &L0);
  __builtin_amdgcn_sched_barrier(0);
  i32x4_t B[4][2];
  int cinit;
  float lpf;
  mma_stage<true>(xa, xb, ga, gb, wave, lane, c0, s_x, &s_b[wave][0], &s_sx[wave][0][0], &s_e[wave][0], s_red, B,
                  &cinit, &lpf);
  __syncthreads();  // s_x (the outliers' inputs) and s_red complete
  float ss = 0.0f;
#pragma unroll
  for (int w = 0; w < kMmaWaves; ++w) ss += s_red[w];
  const float inv = 1.0f / sqrtf(ss / 2048.0f + a.eps);
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  // one cell: products, row sums in s_part[buf], then the two epilogue waves (two buffers: a
  // buffer is written again only after the next barrier, when its readers are done)
  auto process = [&](uint32_t t, const MmaCellLoads& c, int buf) {
    mma_tile(c.q, c.sc, B, cinit, lpf, lane, &s_part[buf][wave][0]);
    __syncthreads();
    if (wave < 2) {
      float v = 0.0f;
#pragma unroll
      for (int w = 0; w < kMmaWaves; ++w) v += s_part[buf][w][tr];
      const float xo = s_x[xs_at(c.ocol < 2048u ? c.ocol : 0u)];
      float o = c.ocol < 2048u ? (repl ? c.od : half_lo(c.ow)) * xo : 0.0f;
      o = pair_sum(o, 1);
      o = pair_sum(o, 2);
      o = pair_sum(o, 4);
      v = (v + o) * inv;
      if ((lane & 7) == 0) epilogue<MODE>(P, t * 16 + tr, v, 0.0f, 0.0f, &bv, &bi, &nf);
    }
  };
  // two cells per trip, the loads of the next cell issued before the current one's products (a
  // clamped repeat past the end); the trip count is the same for every wave of the workgroup
  while (true) {
    const uint32_t t1 = tile + step;
    issue(t1 < n_tiles ? t1 : tile, &L1);
    process(tile, L0, 0);
    if (t1 >= n_tiles) break;
    const uint32_t t2 = t1 + step;
    issue(t2 < n_tiles ? t2 : t1, &L0);
    process(t1, L1, 1);
    if (t2 >= n_tiles) break;
    tile = t2;
  }
  argmax_partial<MODE>(a, bv, bi, nf, s_bv, s_bi, s_nf);
  if (blockIdx.x == 0 && threadIdx.x == 0) a.result->hidden_norm = sqrtf(ss);
}

// Flat 4-bit tiles (gemvCellFlat: the down projection, and every projection wider than 2048
// columns), K-split: one workgroup = one unit of RU = 8 rows, kFlatWaves = 8 waves (two per
// SIMD) striding over panels of 512 columns (4 groups of 128; panel p goes to wave p % 8).
// Lane (j, c) = (lane / 16, lane % 16) holds unit rows j and j + 4 at columns 512 p + 32 c ..
// + 31 of each of its wave's panels: one 16-byte code load and one group scale per row and
// panel, all issued before the input staging waits (up to MAXP panels per wave), after one
// outlier-correction entry per row and lane.  Row sums meet over the 16 lanes (DPP) and the
// waves (LDS, in wave order); wave 0 runs the epilogue.  The input sits in LDS (dynamic, C
// floats) for the dots and for the corrections, which read any column; without the norm each
// wave stages only its own panels and the corrections read their columns from global memory.
constexpr int kFlatWaves = 8;
template <int MODE, int MAXP, bool kWide, int W = kFlatWaves>
__global__ void __launch_bounds__(kWave * W) k_gemv_flat(GemvArgs a) {
  constexpr int RU = 8, S = kWave / RU, NT = kWave * W;
  // input float4 slots per thread: C <= MAXP * W * 512 columns, so 2 * MAXP suffice
  constexpr int SL = kWide ? 1 : (2 * MAXP < 8 ? 2 * MAXP : 8);
  constexpr bool kNorm = kNormOf<MODE>;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kPre = MODE == int(GemvMode::Store) || MODE == int(GemvMode::Accum) || kRope;
  static_assert(MODE != int(GemvMode::Logits), "the flat LM head stays on k_gemv_split");
  extern __shared__ __align__(16) float s_x[];  // xs_floats(C) floats
  __shared__ float s_part[W][RU];
  __shared__ float s_red[W];
  const int lane = threadIdx.x & 63, j = lane >> 4, c = lane & 15;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const BreakIn bin = break_in<MODE>(a);  // (before any store or asm: scalar loads)
  args_batch<MODE>(a);
  const uint32_t C = a.C, ng = C >> 7, npan = (ng + 3) / 4, half = a.rope.head_dim / 2, unit = blockIdx.x;
  const GemvPart P0 = kRope ? pick_part(a, int(__builtin_amdgcn_readfirstlane(part_of(a, unit)))) : a.part[0];
  const GemvPart& P1 = kSwi ? a.part[1] : P0;
  const uint32_t row_base = cells_row_base<MODE>(P0, unit, half);

  // 1. the input first, then codes and scales of rows j and j + 4 for each of the wave's panels
  // Without the norm (kLocal), a wave stages only its own panels' columns (the only ones its
  // dots read) and no workgroup barrier precedes the dots; the corrections then read their
  // input columns from global memory.
  constexpr bool kLocal = !kNorm && !kWide;
  StageRegs<SL> xr;
  float4 xl[MAXP][2];
  if constexpr (kLocal) {
#pragma unroll
    for (int q = 0; q < MAXP; ++q) {
      const uint32_t col = 512 * (wave + W * uint32_t(q)) + 8 * uint32_t(lane), cl = col < C ? col : 0u;
      xl[q][0] = ld_f4(a.x + cl);
      xl[q][1] = ld_f4(a.x + cl + 4);
    }
  } else if constexpr (!kWide) {
    stage_x_issue<kNorm, SL, NT>(a, &xr);
  }
  __builtin_amdgcn_sched_barrier(0);  // every input load ahead of the code loads
  const uint32_t rowA = row_of<RU, MODE>(row_base, j, half), rowB = row_of<RU, MODE>(row_base, j + RU / 2, half);
  const bool okA = rowA < P0.wrows, okB = rowB < P1.wrows;
  // 32-bit group indices and byte offsets from the part's base (a uniform 64-bit pointer), so
  // that each load is a scalar base plus one vector offset (the tensors here are < 4 GiB)
  const uint32_t GA = (okA ? rowA : 0u) * ng, GB = (okB ? rowB : 0u) * ng;
  const uint8_t* baseA = P0.base;
  const uint8_t* baseB = P1.base;
  const uint32_t strA = P0.stride, strB = P1.stride, lo16 = uint32_t(c & 3) * 16;
  // the rows' outlier corrections, spread over the waves: lane (j, c) of the wave in slot
  // position s (wsl below) takes entries c + 16 (s + W t) of rows j and j + 4, and the
  // corrections join the row sums before the lane reduction (a wave skips the slots past every
  // row's entries: a uniform test on the tables' row width)
  constexpr int SPL = int(kMaxCorrPerRow + 16 * W - 1) / (16 * W);
  float2 ca[SPL], cb[SPL];
  uint32_t cuse = 0;
  const uint32_t kmU = max(uni(P0.corr_kmax), uni(P1.corr_kmax));
  // the waves' slot order starts at wave 1: wave 0, which runs the epilogue, takes the last slot
  const uint32_t wsl = wave == 0 ? uint32_t(W - 1) : wave - 1;
  {
    const float2* corrA = uni(P0.corr);
    const float2* corrB = uni(P1.corr);
    const uint32_t kmA = uni(P0.corr_kmax), kmB = uni(P1.corr_kmax);
    const float2* srcA = corrA ? corrA : reinterpret_cast<const float2*>(a.x);
    const float2* srcB = corrB ? corrB : reinterpret_cast<const float2*>(a.x);
#pragma unroll
    for (int t = 0; t < SPL; ++t) {
      ca[t] = cb[t] = make_float2(0.0f, 0.0f);
      if (16u * (wsl + uint32_t(W * t)) < kmU) {
        const uint32_t e = uint32_t(c) + 16u * (wsl + uint32_t(W * t));
        const bool ua = corrA != nullptr && okA && e < kmA, ub = corrB != nullptr && okB && e < kmB;
        ca[t] = srcA[ua ? size_t(rowA) * kmA + e : 0];
        cb[t] = srcB[ub ? size_t(rowB) * kmB + e : 0];
        cuse |= (uint32_t(ua) << (2 * t)) | (uint32_t(ub) << (2 * t + 1));
      }
    }
  }
  uint4 qa[MAXP], qb[MAXP];
  uint32_t sa[MAXP], sb[MAXP], gvm = 0;
#pragma unroll
  for (int q = 0; q < MAXP; ++q) {
    const uint32_t p = wave + W * uint32_t(q), g = 4 * p + uint32_t(c >> 2);
    const bool gv = p < npan && g < ng;
    gvm |= uint32_t(gv) << q;
    const uint32_t Ga = GA + (gv ? g : 0u), Gb = GB + (gv ? g : 0u);
    const uint32_t oa = (Ga >> 8) * strA + (Ga & 255u) * 64, ob = (Gb >> 8) * strB + (Gb & 255u) * 64;
    const uint32_t sa_off = (Ga >> 8) * strA + 16448 + 48 + 2 * (Ga & 255u);
    const uint32_t sb_off = (Gb >> 8) * strB + 16448 + 48 + 2 * (Gb & 255u);
    qa[q] = ld_u128(baseA + (oa + 64 + lo16));
    qb[q] = ld_u128(baseB + (ob + 64 + lo16));
    sa[q] = ld_u16(baseA + sa_off);
    sb[q] = ld_u16(baseB + sb_off);
  }
  // lane 8 i's residual / bias / RoPE operands
  const int i8 = lane >> 3;
  const uint32_t orow = row_of<RU, MODE>(row_base, i8, half);
  float pre = 0.0f, rc = 1.0f, rs = 0.0f;
  bool pre_ok = false, rope_ok = false;
  if constexpr (kPre) {
    const float* src = MODE == int(GemvMode::Accum) ? P0.y : P0.bias;
    pre_ok = (lane % S) == 0 && orow < P0.rows && src != nullptr;
    pre = (src ? src : a.x)[pre_ok ? orow : 0u];
  }
  if constexpr (kRope) {
    rope_ok = (lane % S) == 0 && lane < 32 && P0.rope_role < kRoleV;
    const size_t at = rope_ok ? (orow % (2 * half)) : 0u;
    rc = a.rope.cos[at];
    rs = a.rope.sin[at];
  }

  // 2. the (normalised) input into LDS, once every load above is issued
  __builtin_amdgcn_sched_barrier(0);
  float ss = 0.0f, inv = 1.0f;
  if constexpr (kLocal) {
#pragma unroll
    for (int q = 0; q < MAXP; ++q) {
      const uint32_t col = 512 * (wave + W * uint32_t(q)) + 8 * uint32_t(lane);
      if (col < C) {
        *reinterpret_cast<float4*>(s_x + xs_at(col)) = xl[q][0];
        *reinterpret_cast<float4*>(s_x + xs_at(col) + 4) = xl[q][1];
      }
    }
    __builtin_amdgcn_wave_barrier();  // (one wave's LDS accesses execute in order)
  } else {
    stage_x_finish<kNorm, kWide, SL, NT>(a, xr, s_x, s_red, &ss, &inv);
  }
  const bool brk = break_now<MODE>(a, bin, !isfinite(ss));
  // the corrections' input columns (kLocal: from global memory, requested before the dots)
  float xca[SPL], xcb[SPL];
#pragma unroll
  for (int t = 0; t < SPL; ++t) {
    xca[t] = xcb[t] = 0.0f;
    if (16u * (wsl + uint32_t(W * t)) < kmU) {
      const bool ua = ((cuse >> (2 * t)) & 1u) && ca[t].y != 0.0f;
      const bool ub = ((cuse >> (2 * t + 1)) & 1u) && cb[t].y != 0.0f;
      const uint32_t qa = ua ? __float_as_uint(ca[t].x) : 0u, qb = ub ? __float_as_uint(cb[t].x) : 0u;
      xca[t] = kLocal ? a.x[qa] : s_x[xs_at(qa)];
      xcb[t] = kLocal ? a.x[qb] : s_x[xs_at(qb)];
    }
  }

  // 3. the dots of the wave's panels, summed over the 16 lanes of each row, then over the waves
  float accA = 0.0f, accB = 0.0f;
#pragma unroll
  for (int q = 0; q < MAXP; ++q) {
    const uint32_t p = wave + W * uint32_t(q);
    const bool gv = (gvm >> q) & 1u;
    const uint32_t col0 = gv ? 512 * p + 32 * uint32_t(c) : 0u;
    float xv[32];
    float sx = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      const float4 t = *reinterpret_cast<const float4*>(s_x + xs_at(col0 + 4 * k));
      xv[4 * k] = t.x; xv[4 * k + 1] = t.y; xv[4 * k + 2] = t.z; xv[4 * k + 3] = t.w;
    }
#pragma unroll
    for (int k = 0; k < 32; ++k) sx += xv[k];
    const float tA = (dot32_w4(qa[q], xv) - FlatW4::kOff * sx) * FlatW4::scale(sa[q]);
    const float tB = (dot32_w4(qb[q], xv) - FlatW4::kOff * sx) * FlatW4::scale(sb[q]);
    accA += gv ? tA : 0.0f;
    accB += gv ? tB : 0.0f;
  }
  // corrections (w_out - dequantised code) * x[col], branch-free: unused entries read column 0
#pragma unroll
  for (int t = 0; t < SPL; ++t) {
    const bool ua = ((cuse >> (2 * t)) & 1u) && ca[t].y != 0.0f;
    const bool ub = ((cuse >> (2 * t + 1)) & 1u) && cb[t].y != 0.0f;
    accA = ua ? fmaf(ca[t].y, xca[t], accA) : accA;
    accB = ub ? fmaf(cb[t].y, xcb[t], accB) : accB;
  }
  accA = okA ? accA : 0.0f;
  accB = okB ? accB : 0.0f;
#pragma unroll
  for (int m = 1; m < 16; m <<= 1) {
    accA = pair_sum(accA, m);
    accB = pair_sum(accB, m);
  }
  if (c == 0) {
    s_part[wave][j] = accA;
    s_part[wave][j + RU / 2] = accB;
  }
  __syncthreads();
  if (wave != 0) return;

  // 4. wave 0: row i8 on lanes 8 i8 .. 8 i8 + 7, the epilogue
  float v = 0.0f;
#pragma unroll
  for (int w = 0; w < W; ++w) v += s_part[w][i8];
  const float up = (kSwi || kRope) ? pair_val(v, 32) : 0.0f;
  const float prev = pre_ok ? pre : 0.0f;
  const float up_pre = kRope ? pair_val(prev, 32) : 0.0f;
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  if constexpr (kRope) {
    if ((lane % S) == 0 && i8 < RU / 2 && orow < P0.rows)
      rope_store(a, P0, orow, v + prev, up + up_pre, rope_ok ? rc : 1.0f, rope_ok ? rs : 0.0f, brk);
  } else if ((lane % S) == 0 && (!kSwi || i8 < RU / 2) &&
             (MODE != int(GemvMode::Accum) || orow < P0.wrows)) {  // Accum: rows past the tiles stay
    epilogue<MODE>(P0, row_of<RU, MODE>(row_base, i8, 0), v, up, prev, &bv, &bi, &nf, brk);
  }
}

// ---- flat tiles, input-stationary and pipelined (k_gemv_xs) ---------------------------------
// gemvCellFlat (:584-729) for every mode, x held in registers: wave w of NW owns the columns
// w * 64 * F::kCols .. + 64 * F::kCols - 1 (lane l: F::kCols columns from F::kCols * l, one
// 16-byte code load per row), normalised once per workgroup ((x * inv) * gamma, rmsNorm
// :187-191) and kept for every unit the workgroup takes.  The grid is persistent: a workgroup
// strides over units of R rows (SwiGlu: R/2 gate + R/2 up rows; QkvRope: R/2 RoPE pairs) and
// issues the code, scale, correction and residual loads of its next unit before the arithmetic
// of the current one, so each wave keeps its own loads in flight while it computes.  Row sums
// meet over the lanes (reduce-scatter) and the waves (LDS, double-buffered, in wave order);
// wave 0 runs the epilogue.  Outliers replace weights (:632-646): per-row corrections
// (w_out - dequantised code) * x[col], spread over all lanes of all waves, with x[col] from the
// workgroup's LDS copy of the (normalised) input.
template <int R, int MODE>
__device__ __forceinline__ uint32_t xs_row_base(const GemvPart& P0, uint32_t unit, uint32_t half) {
  if constexpr (MODE == int(GemvMode::SwiGlu)) {
    return unit * (R / 2);
  } else if constexpr (MODE == int(GemvMode::QkvRope)) {  // R/2 pairs per unit, half/(R/2) units per head
    const uint32_t ul = unit - P0.unit_begin, per_head = half / (R / 2);
    return (ul / per_head) * (2 * half) + (ul % per_head) * (R / 2);
  } else {
    return (unit - P0.unit_begin) * R;
  }
}

template <int R, int SPL>
struct XsLoads {
  uint4 q[R];          // codes of row i at the lane's columns
  uint32_t s[R];       // their group scale
  float2 ce[SPL];      // correction entries (column bits, w_out - code) of the lane's row
  uint32_t cuse;       // bit t: ce[t] belongs to the row
  float pre, pre2;     // lane i: residual / bias of row i (QkvRope: pre2 = bias of the pair's row)
  float rc, rs;        // lane i < R/2 (QkvRope): cos / sin of the pair
  uint32_t row_base;   // first row of the unit in its part
  int pu;              // the unit's part (QkvRope)
};

template <class F, int MODE, int R, int NW>
__global__ void __launch_bounds__(kWave * NW) k_gemv_xs(GemvArgs a) {
  constexpr int KC = F::kCols, CH = kWave * KC;
  constexpr bool kNorm = kNormOf<MODE>;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr bool kPre = MODE == int(GemvMode::Store) || MODE == int(GemvMode::Accum) || kRope;
  constexpr int LPR = kWave / R;                                  // lanes per row (corrections)
  constexpr int SPL = int(kMaxCorrPerRow + LPR * NW - 1) / (LPR * NW);
  constexpr int NE = (kSwi || kRope) ? R / 2 : R;                 // epilogue lanes
  static_assert(R == 2 || R == 4 || R == 8, "rows per unit");
  extern __shared__ __align__(16) float s_x[];                    // C floats: the (normalised) input
  __shared__ float s_part[2][NW][R];
  __shared__ float s_red[NW];
  __shared__ float s_bv[NW];
  __shared__ uint32_t s_bi[NW], s_nf[NW];
  const int lane = threadIdx.x & 63;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const BreakIn bin = break_in<MODE>(a);  // (before any store or asm: scalar loads)
  args_batch<MODE>(a);
  const uint32_t C = a.C, ng = C >> 7, half = a.rope.head_dim / 2, n_units = a.n_units, step = gridDim.x;
  const uint32_t col = wave * CH + uint32_t(KC * lane);
  const bool okc = col < C;
  const uint32_t cc = okc ? col : 0u;

  // 1. the lane's input columns (and gains)
  float xv[KC];
  float4 gq[kNorm ? KC / 4 : 1];
#pragma unroll
  for (int j = 0; j < KC / 4; ++j) {
    const float4 t = ld_f4(a.x + cc + 4 * j);
    xv[4 * j] = t.x; xv[4 * j + 1] = t.y; xv[4 * j + 2] = t.z; xv[4 * j + 3] = t.w;
    if constexpr (kNorm) gq[j] = ld_f4(a.gamma + cc + 4 * j);
  }
  __builtin_amdgcn_sched_barrier(0);

  // loads of unit u into L: codes + scales of its R rows, correction entries, residual / bias,
  // RoPE factors -- every address a uniform base plus a 32-bit lane offset, rows past the part
  // (or past its tiles) read row 0 and are dropped
  auto issue = [&](uint32_t u, XsLoads<R, SPL>* L) {
    const int pu = kRope ? int(__builtin_amdgcn_readfirstlane(part_of(a, u))) : 0;
    const GemvPart P0 = kRope ? pick_part(a, pu) : a.part[0];
    const GemvPart& P1 = kSwi ? a.part[1] : P0;
    const uint32_t rb = xs_row_base<R, MODE>(P0, u, half);
    L->pu = pu;
    L->row_base = rb;
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const bool second = kSwi && i >= R / 2;
      const uint32_t r = row_of<R, MODE>(rb, i, half);
      const uint32_t wr = second ? uni(P1.wrows) : uni(P0.wrows);
      const uint32_t G = (r < wr ? r : 0u) * ng + (cc >> 7);
      const uint8_t* base = second ? uni(P1.base) : uni(P0.base);
      const uint32_t stride = second ? uni(P1.stride) : uni(P0.stride);
      const uint32_t tile_off = (G >> 8) * stride, gi = G & 255u;
      L->q[i] = ld_u128(base + (tile_off + 64 + gi * (KC == 32 ? 64u : 32u) + ((cc & 127u) / (KC == 32 ? 2u : 4u))));
      L->s[i] = ld_u16(base + (tile_off + 16448 + 48 + 2 * gi));
    }
    {  // corrections: lane l takes entries (l % LPR) + LPR (w + NW t) of unit row l / LPR
      const int ci = lane / LPR;
      const bool second = kSwi && ci >= R / 2;
      const float2* corr = second ? uni(P1.corr) : uni(P0.corr);
      const uint32_t kmax = second ? uni(P1.corr_kmax) : uni(P0.corr_kmax);
      const uint32_t wr = second ? uni(P1.wrows) : uni(P0.wrows);
      const uint32_t r = row_of<R, MODE>(rb, ci, half);
      const bool ok = corr != nullptr && r < wr;
      const float2* src = corr ? corr : reinterpret_cast<const float2*>(a.x);
      uint32_t m = 0;
#pragma unroll
      for (int t = 0; t < SPL; ++t) {
        const uint32_t e = uint32_t(lane % LPR) + uint32_t(LPR) * (wave + uint32_t(NW * t));
        const bool use = ok && e < kmax;
        L->ce[t] = src[use ? size_t(r) * kmax + e : 0];
        m |= uint32_t(use) << t;
      }
      L->cuse = m;
    }
    L->pre = 0.0f;
    L->pre2 = 0.0f;
    L->rc = 1.0f;
    L->rs = 0.0f;
    if constexpr (kPre) {
      const int i = lane < NE ? lane : 0;
      const float* src = MODE == int(GemvMode::Accum) ? P0.y : P0.bias;
      const uint32_t r = row_of<R, MODE>(rb, i, half);
      const bool ok = lane < NE && r < P0.rows && src != nullptr;
      L->pre = (src ? src : a.x)[ok ? r : 0u];
      L->pre = ok ? L->pre : 0.0f;
      if constexpr (kRope) {
        const uint32_t r2 = row_of<R, MODE>(rb, i + R / 2, half);
        const bool ok2 = lane < NE && r2 < P0.rows && src != nullptr;
        L->pre2 = (src ? src : a.x)[ok2 ? r2 : 0u];
        L->pre2 = ok2 ? L->pre2 : 0.0f;
        const bool rope = lane < NE && P0.rope_role < kRoleV;
        const size_t at = rope ? (r % (2 * half)) : 0u;
        L->rc = rope ? a.rope.cos[at] : 1.0f;
        L->rs = rope ? a.rope.sin[at] : 0.0f;
      }
    }
  };

  XsLoads<R, SPL> LA, LB;
  uint32_t unit = blockIdx.x;  // < n_units: the grid is at most the unit count
  issue(unit, &LA);

  // 2. the input normalised in registers ((x * inv) * gamma) and copied to LDS for the corrections
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < KC; ++j) {
    xv[j] = okc ? xv[j] : 0.0f;
    ss = fmaf(xv[j], xv[j], ss);
  }
  float tot = 0.0f;
  if constexpr (kNorm) {  // (the residual modes skip the sum of squares and its barrier)
    ss = wave_sum(ss);
    if (lane == 0) s_red[wave] = ss;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += s_red[w];
    const float inv = 1.0f / sqrtf(tot / float(C) + a.eps);
#pragma unroll
    for (int j = 0; j < KC / 4; ++j) {
      xv[4 * j] = (xv[4 * j] * inv) * gq[j].x;
      xv[4 * j + 1] = (xv[4 * j + 1] * inv) * gq[j].y;
      xv[4 * j + 2] = (xv[4 * j + 2] * inv) * gq[j].z;
      xv[4 * j + 3] = (xv[4 * j + 3] * inv) * gq[j].w;
    }
  }
  if (okc) {
#pragma unroll
    for (int j = 0; j < KC / 4; ++j)
      *reinterpret_cast<float4*>(s_x + col + 4 * j) = make_float4(xv[4 * j], xv[4 * j + 1], xv[4 * j + 2], xv[4 * j + 3]);
  }
  float sx = 0.0f;
#pragma unroll
  for (int j = 0; j < KC; ++j) sx += xv[j];
  const bool brk = break_now<MODE>(a, bin, !isfinite(tot));
  __syncthreads();  // s_x complete

  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  auto compute = [&](const XsLoads<R, SPL>& L, int buf) {
    const GemvPart P0 = kRope ? pick_part(a, L.pu) : a.part[0];
    const GemvPart& P1 = kSwi ? a.part[1] : P0;
    const uint32_t rb = L.row_base;
    float acc[R];
#pragma unroll
    for (int i = 0; i < R; ++i) {
      const bool second = kSwi && i >= R / 2;
      const uint32_t r = row_of<R, MODE>(rb, i, half);
      const uint32_t wr = second ? uni(P1.wrows) : uni(P0.wrows);
      const float t = (F::dot(L.q[i], xv, false) - F::kOff * sx) * F::scale(L.s[i]);
      acc[i] = (okc && r < wr) ? t : 0.0f;
    }
    const int ci = lane / LPR;
#pragma unroll
    for (int t = 0; t < SPL; ++t) {
      const bool on = ((L.cuse >> t) & 1u) && L.ce[t].y != 0.0f;
      const float xc = s_x[on ? __float_as_uint(L.ce[t].x) : 0u];
      const float d = on ? L.ce[t].y * xc : 0.0f;
#pragma unroll
      for (int i = 0; i < R; ++i) acc[i] += ci == i ? d : 0.0f;
    }
    const float v = wave_reduce_rows<R>(acc, lane);  // lane l: row l / LPR
    if ((lane % LPR) == 0) s_part[buf][wave][lane / LPR] = v;
    __syncthreads();
    if (wave == 0 && lane < NE) {
      float y0 = 0.0f, y1 = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        y0 += s_part[buf][w][lane];
        if constexpr (kSwi || kRope) y1 += s_part[buf][w][lane + R / 2];
      }
      const uint32_t r = row_of<R, MODE>(rb, lane, half);
      if constexpr (kRope) {
        if (r < P0.rows) rope_store(a, P0, r, y0 + L.pre, y1 + L.pre2, L.rc, L.rs, brk);
      } else if (MODE != int(GemvMode::Accum) || r < P0.wrows) {  // Accum: rows past the tiles stay
        epilogue<MODE>(P0, r, y0, y1, L.pre, &bv, &bi, &nf, brk);
      }
    }
  };

  // 3. the units: the next unit's loads, then the current unit's arithmetic (static buffers)
  bool last_b = false;
  while (unit + step < n_units) {
    issue(unit + step, &LB);
    compute(LA, 0);
    unit += step;
    if (unit + step >= n_units) {
      last_b = true;
      break;
    }
    issue(unit + step, &LA);
    compute(LB, 1);
    unit += step;
  }
  if (last_b) compute(LB, 1);
  else compute(LA, 0);
  if constexpr (kLogits) {
    argmax_partial<MODE>(a, bv, bi, nf, s_bv, s_bi, s_nf);
    if (blockIdx.x == 0 && threadIdx.x == 0) a.result->hidden_norm = sqrtf(tot);
  }
}

// ---- flat 4-bit tiles on the matrix cores, input-stationary (k_gemv_xm) ----------------------
// gemvCellFlat (:584-729) for every mode.  Wave w of NW owns the columns 2048 w .. 2048 w + 2047
// (four sets of 4 groups of 128) for the whole launch: its input (normalised, (x * inv) * gamma,
// rmsNorm :187-191) is split into exact integers per group (X = x * 2^(30-e), max |x| < 2^e,
// truncated; four signed-byte limbs, X = L0 + 2^8 L1 + 2^16 L2 + 2^24 L3) held in a per-wave LDS
// table in the byte order of the matrix-core operands.  A unit is 4 rows (SwiGlu: 2 gate + 2 up
// rows; QkvRope: 2 RoPE pairs); per set the wave runs two v_mfma_i32_16x16x64_i8 with
//   A (16 x 64): row m = 4 r + g -> unit row r, group g of the set, 64 of its codes (one half),
//   B (64 x 16): column n = g' + 4 L -> limb L of the input in group g' (the same half),
// so D(r, g; g', L) is the exact integer sum over the half of code * limb where g == g', starting
// at -8 * (the limb's sum over the group) for the codes' offset.  Lane (n, q) holds D(q, j; n % 4,
// n / 4) for j = 0..3 and keeps j = n % 4, times 2^(8 L) 2^(e - 30) and the group scale; it adds
// these over the four sets (and its share of row q's corrections), and row q's sum over its 16
// lanes (the limbs, then the groups; DPP) is taken once per unit.  Each lane loads 16 bytes of unit row n / 4, group n % 4, quarter q per set: the unit's rows as
// 256-byte runs in the records, or 1 KB contiguous per load from the launch's permuted copy
// (xm_code_at).  The grid is persistent; the next unit's loads are issued before the current
// unit's products.  Row sums meet over the waves in LDS (double-buffered, in wave order); wave 0
// runs the epilogue.  Outliers replace weights (:632-646): per-row corrections
// (w_out - dequantised code) * x[col] on the 16 lanes of each row, with x[col] rebuilt from the
// limb tables (the same integers the products use).  The residual modes skip the input's sum of
// squares.
constexpr uint32_t kXmTableBytes = 4 * 128 * 16;  // per wave: 4 sets x (group, quarter, half, limb) x 16 bytes

template <int R, int SPL>
struct XmLoads {
  uint4 q[4];          // codes: unit row n / 4, group n % 4 of set S, quarter q
  uint32_t s[4];       // group scale: unit row q, group n % 4 of set S
  float2 ce[SPL];      // correction entries (column bits, w_out - code) of unit row q
  uint32_t cuse;
  float pre, pre2, rc, rs;
  uint32_t row_base;
  int pu;
};

// x'[col] from the limb tables: the integer X of the column times 2^(e - 30) of its group.
// Within a 16-column block's 16 bytes per limb, 4-bit tables hold the columns in the order
// {0,2,4,6}, {1,3,5,7}, {8,10,12,14}, {9,11,13,15} (the nibbles of the codes), 2-bit tables in
// the order {0,4,8,12}, {1,5,9,13}, {2,6,10,14}, {3,7,11,15} (the 2-bit fields).
template <int BITS = 4>
__device__ __forceinline__ float xm_input(const uint8_t* tb, const float* s_e, uint32_t col) {
  const uint32_t w = col >> 11, S = (col >> 9) & 3u, g = (col >> 7) & 3u, c = col & 127u;
  const uint32_t q = c >> 5, h = (c >> 4) & 1u, p = (c >> 3) & 1u, i = c & 7u, c16 = c & 15u;
  const uint32_t in16 = BITS == 2 ? 4 * (c16 & 3u) + (c16 >> 2) : 4 * (2 * p + (i & 1u)) + (i >> 1);
  const uint32_t at = (w * 4 + S) * 128 * 16 + (((g * 4 + q) * 2 + h) * 4) * 16 + in16;
  const int X = int(int8_t(tb[at])) + (int(int8_t(tb[at + 16])) << 8) + (int(int8_t(tb[at + 32])) << 16) +
                (int(int8_t(tb[at + 48])) << 24);
  return float(X) * s_e[(w * 4 + S) * 4 + g];
}

// The 16 code bytes lane (n, q) of wave w reads for set S of the unit at row base rb: unit row
// n / 4 (SwiGlu: rows 2 and 3 from the up part), group 16 w + 4 S + n % 4, quarter q, in the
// records (rows past the tiles and groups past the input read row 0 / group 0; their products
// are not used).  The launch's permuted copy (GemvPart::xcodes) holds the same bytes at
// u * NW * 4096 + ((w * 4 + S) * 64 + lane) * 16: each load instruction of a wave then reads
// 1 KB of contiguous memory instead of four 256-byte runs.
template <int R, int MODE, int BITS = 4>
__device__ __forceinline__ const uint8_t* xm_code_at(const GemvPart& P0, const GemvPart& P1, uint32_t rb,
                                                     uint32_t half, uint32_t ng, uint32_t gw, int S, int n, int q) {
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  const uint32_t ia = uint32_t(n >> 2);
  const bool sa = kSwi && ia >= R / 2;
  const uint32_t ra = row_of<R, MODE>(rb, int(ia), half);
  const uint32_t wa = sa ? uni(P1.wrows) : uni(P0.wrows);
  const uint8_t* ba = sa ? uni(P1.base) : uni(P0.base);
  const uint32_t sta = sa ? uni(P1.stride) : uni(P0.stride);
  const uint32_t g = gw + 4 * uint32_t(S) + uint32_t(n & 3), gc = g < ng ? g : 0u;
  const uint32_t Ga = (ra < wa ? ra : 0u) * ng + gc;
  if constexpr (BITS == 2)  // 32 bytes per group: quarter q is 8 bytes (the same 32 columns)
    return ba + ((Ga >> 8) * sta + 64 + (Ga & 255u) * 32 + 8 * uint32_t(q));
  return ba + ((Ga >> 8) * sta + 64 + (Ga & 255u) * 64 + 16 * uint32_t(q));
}

// BITS = 2: 2-bit flat tiles.  Their codebook {0, +1, -2, -1} is the 2-bit two's complement, so
// (code ^ 2) - 2 is the weight: the products take code ^ 2 (0..3) as the A operand and start at
// -2 * (the limb's sum over the group).  A lane reads 8 bytes per set (the same 32 columns of its
// group quarter); the B tables hold the 2-bit field order (xm_input).
// kXc (2-bit): the codes come from the launch's permuted copy, two sets per 16-byte load (a
// compile-time choice: the two forms issue different numbers of loads, and a runtime branch
// between them would leave every later wait counting the larger number)
template <int MODE, int NW, int BITS = 4, bool kXc = false>
__global__ void __launch_bounds__(kWave * NW) k_gemv_xm(GemvArgs a) {
  constexpr int R = 4;
  static_assert(BITS == 4 || BITS == 2, "4- or 2-bit flat tiles");
  static_assert(!kXc || BITS == 2, "the 4-bit copy is read through the same loads as the records");
  constexpr bool kNorm = kNormOf<MODE>;
  constexpr bool kSwi = MODE == int(GemvMode::SwiGlu);
  constexpr bool kRope = MODE == int(GemvMode::QkvRope);
  constexpr bool kLogits = MODE == int(GemvMode::Logits);
  constexpr bool kPre = MODE == int(GemvMode::Store) || MODE == int(GemvMode::Accum) || kRope;
  constexpr int SPL = int(kMaxCorrPerRow + 16 * NW - 1) / (16 * NW);
  constexpr int NE = (kSwi || kRope) ? R / 2 : R;
  extern __shared__ __align__(16) uint8_t s_dyn[];  // NW limb tables, then 2^(e-30) per group
  uint4* s_tb = reinterpret_cast<uint4*>(s_dyn);
  float* s_e = reinterpret_cast<float*>(s_dyn + NW * kXmTableBytes);
  __shared__ int s_ci[NW][4][16];
  __shared__ float s_part[2][NW][R];
  __shared__ float s_red[NW];
  __shared__ float s_bv[NW];
  __shared__ uint32_t s_bi[NW], s_nf[NW];
  const int lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const BreakIn bin = break_in<MODE>(a);  // (before any store or asm: scalar loads)
  args_batch<MODE>(a);
  const uint32_t C = a.C, ng = C >> 7, half = a.rope.head_dim / 2, n_units = a.n_units, step = gridDim.x;
  const uint32_t gw = wave * 16;  // the wave's first group
  // correction slots in wave order from wave 1: wave 0, which runs the epilogue, takes the last
  const uint32_t wsl = wave == 0 ? uint32_t(NW - 1) : wave - 1;

  // 1. the wave's input: 8 columns per lane and set (lane l: set S, columns 2048 w + 512 S + 8 l)
  float4 xr[4][2], gr[kNorm ? 4 : 1][2];
#pragma unroll
  for (int S = 0; S < 4; ++S) {
    const uint32_t c0 = (gw + 4 * S) * 128 + 8 * uint32_t(lane), cc = c0 < C ? c0 : 0u;
    xr[S][0] = ld_f4(a.x + cc);
    xr[S][1] = ld_f4(a.x + cc + 4);
    if constexpr (kNorm) {
      gr[S][0] = ld_f4(a.gamma + cc);
      gr[S][1] = ld_f4(a.gamma + cc + 4);
    }
  }
  __builtin_amdgcn_sched_barrier(0);

  auto issue = [&](uint32_t u, XmLoads<R, SPL>* L) {
    const int pu = kRope ? int(__builtin_amdgcn_readfirstlane(part_of(a, u))) : 0;
    const GemvPart P0 = kRope ? pick_part(a, pu) : a.part[0];
    const GemvPart& P1 = kSwi ? a.part[1] : P0;
    const uint32_t rb = xs_row_base<R, MODE>(P0, u, half);
    L->pu = pu;
    L->row_base = rb;
    {  // codes (xm_code_at, or the permuted copy); scales: unit row q (each in its part, rows
       // past the tiles read row 0)
      const uint32_t is = uint32_t(q);
      const bool ss = kSwi && is >= R / 2;
      const uint32_t rs = row_of<R, MODE>(rb, int(is), half);
      const uint32_t ws = ss ? uni(P1.wrows) : uni(P0.wrows);
      const uint8_t* bs = ss ? uni(P1.base) : uni(P0.base);
      const uint32_t sts = ss ? uni(P1.stride) : uni(P0.stride);
      const uint32_t Gs0 = (rs < ws ? rs : 0u) * ng;
      const uint8_t* xc = uni(P0.xcodes);
#pragma unroll
      for (int S = 0; S < 4; ++S) {
        const uint32_t g = gw + 4 * uint32_t(S) + uint32_t(n & 3), gc = g < ng ? g : 0u;
        const uint32_t Gs = Gs0 + gc;
        if constexpr (BITS == 2 && kXc) {  // sets S and S + 1 in one 16-byte load (the permuted copy)
          if ((S & 1) == 0) {
            const uint4 v = ld_u128(uni(a.part[0].xcodes) +
                                    (u * (NW * 2048u) + ((wave * 2 + uint32_t(S / 2)) * 64 + uint32_t(lane)) * 16));
            L->q[S] = make_uint4(v.x, v.y, 0u, 0u);
            L->q[S + 1] = make_uint4(v.z, v.w, 0u, 0u);
          }
        } else if constexpr (BITS == 2) {
          const uint2 v = ld_u64(xm_code_at<R, MODE, 2>(P0, P1, rb, half, ng, gw, S, n, q));
          L->q[S] = make_uint4(v.x, v.y, 0u, 0u);
        } else {
          const uint8_t* src = xc ? xc + (u * (NW * 4096u) + ((wave * 4 + uint32_t(S)) * 64 + uint32_t(lane)) * 16)
                                  : xm_code_at<R, MODE>(P0, P1, rb, half, ng, gw, S, n, q);
          L->q[S] = ld_u128(src);
        }
        L->s[S] = ld_u16(bs + ((Gs >> 8) * sts + 16448 + 48 + 2 * (Gs & 255u)));
      }
    }
    {  // corrections: lane (n, q) takes entries n + 16 (s + NW t) of unit row q (s = wsl)
      const bool second = kSwi && q >= R / 2;
      const float2* corr = second ? uni(P1.corr) : uni(P0.corr);
      const uint32_t kmax = second ? uni(P1.corr_kmax) : uni(P0.corr_kmax);
      const uint32_t wr = second ? uni(P1.wrows) : uni(P0.wrows);
      const uint32_t r = row_of<R, MODE>(rb, q, half);
      const bool ok = corr != nullptr && r < wr;
      const float2* src = corr ? corr : reinterpret_cast<const float2*>(a.x);
      uint32_t m = 0;
#pragma unroll
      for (int t = 0; t < SPL; ++t) {
        const uint32_t e = uint32_t(n) + 16u * (wsl + uint32_t(NW * t));
        const bool use = ok && e < kmax;
        L->ce[t] = src[use ? size_t(r) * kmax + e : 0];
        m |= uint32_t(use) << t;
      }
      L->cuse = m;
    }
    L->pre = 0.0f;
    L->pre2 = 0.0f;
    L->rc = 1.0f;
    L->rs = 0.0f;
    if constexpr (kPre) {
      const int i = lane < NE ? lane : 0;
      const float* src = MODE == int(GemvMode::Accum) ? P0.y : P0.bias;
      const uint32_t r = row_of<R, MODE>(rb, i, half);
      const bool ok = lane < NE && r < P0.rows && src != nullptr;
      L->pre = (src ? src : a.x)[ok ? r : 0u];
      L->pre = ok ? L->pre : 0.0f;
      if constexpr (kRope) {
        const uint32_t r2 = row_of<R, MODE>(rb, i + R / 2, half);
        const bool ok2 = lane < NE && r2 < P0.rows && src != nullptr;
        L->pre2 = (src ? src : a.x)[ok2 ? r2 : 0u];
        L->pre2 = ok2 ? L->pre2 : 0.0f;
        const bool rope = lane < NE && P0.rope_role < kRoleV;
        const size_t at = rope ? (r % (2 * half)) : 0u;
        L->rc = rope ? a.rope.cos[at] : 1.0f;
        L->rs = rope ? a.rope.sin[at] : 0.0f;
      }
    }
  };

  XmLoads<R, SPL> LA, LB;
  uint32_t unit = blockIdx.x;  // < n_units: the grid is at most the unit count
  issue(unit, &LA);

  // 2. normalise (the norm modes only: the sum of squares and its workgroup barrier cost the
  // residual launches about 1.4 us), then the limb tables, limb sums and group exponents
  float tot = 0.0f;
  if constexpr (kNorm) {
    float ss = 0.0f;
#pragma unroll
    for (int S = 0; S < 4; ++S) {
      const bool live = (gw + 4 * S) * 128 + 8 * uint32_t(lane) < C;
      const float v[8] = {xr[S][0].x, xr[S][0].y, xr[S][0].z, xr[S][0].w, xr[S][1].x, xr[S][1].y, xr[S][1].z, xr[S][1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) ss = live ? fmaf(v[i], v[i], ss) : ss;
    }
    ss = wave_sum(ss);
    if (lane == 0) s_red[wave] = ss;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < NW; ++w) tot += s_red[w];
  }
  const float inv = kNorm ? 1.0f / sqrtf(tot / float(C) + a.eps) : 1.0f;
  uint2* tb2 = reinterpret_cast<uint2*>(s_tb + wave * (kXmTableBytes / 16));
#pragma unroll
  for (int S = 0; S < 4; ++S) {
    const bool live = (gw + 4 * S) * 128 + 8 * uint32_t(lane) < C;
    float xp[8] = {xr[S][0].x, xr[S][0].y, xr[S][0].z, xr[S][0].w, xr[S][1].x, xr[S][1].y, xr[S][1].z, xr[S][1].w};
    if constexpr (kNorm) {
      const float gv[8] = {gr[S][0].x, gr[S][0].y, gr[S][0].z, gr[S][0].w, gr[S][1].x, gr[S][1].y, gr[S][1].z, gr[S][1].w};
#pragma unroll
      for (int i = 0; i < 8; ++i) xp[i] = (xp[i] * inv) * gv[i];
    }
    float mx = 0.0f;  // (a NaN counts as infinite: the group's factor becomes NaN, as its sum would)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      xp[i] = live ? xp[i] : 0.0f;
      const float ax = fabsf(xp[i]);
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
    for (int i = 0; i < 8; ++i) z[i] = (uint32_t(int(xp[i] * up)) + 0x808080u) ^ 0x808080u;
    uint32_t lo[4], hi[4];
    if constexpr (BITS == 2) {
      // lanes 2k, 2k + 1 hold columns 0..7 and 8..15 of a 16-column block; the 2-bit order wants
      // {0,4,8,12}, {1,5,9,13} in the even lane and {2,6,10,14}, {3,7,11,15} in the odd one:
      // each sends the four its neighbour needs
      const bool odd = (lane & 1) != 0;
      const uint32_t r0 = pair_u(odd ? z[0] : z[2], 1), r1 = pair_u(odd ? z[1] : z[3], 1);
      const uint32_t r2 = pair_u(odd ? z[4] : z[6], 1), r3 = pair_u(odd ? z[5] : z[7], 1);
      if (odd) {  // columns 2, 6, 10, 14 and 3, 7, 11, 15
        limb_words(r0, r2, z[2], z[6], lo);
        limb_words(r1, r3, z[3], z[7], hi);
      } else {    // columns 0, 4, 8, 12 and 1, 5, 9, 13
        limb_words(z[0], z[4], r0, r2, lo);
        limb_words(z[1], z[5], r1, r3, hi);
      }
    } else {
      limb_words(z[0], z[2], z[4], z[6], lo);
      limb_words(z[1], z[3], z[5], z[7], hi);
    }
    const uint32_t gs = uint32_t(lane) >> 4, gq = (uint32_t(lane) >> 2) & 3u, gh = (uint32_t(lane) >> 1) & 1u;
#pragma unroll
    for (int L = 0; L < 4; ++L) {
      tb2[((uint32_t(S) * 128 + ((gs * 4 + gq) * 2 + gh) * 4 + uint32_t(L))) * 2 + uint32_t(lane & 1)] =
          make_uint2(lo[L], hi[L]);
      int sl = __builtin_amdgcn_sdot4(int(lo[L]), 0x01010101, __builtin_amdgcn_sdot4(int(hi[L]), 0x01010101, 0, false), false);
      sl += int(pair_u(uint32_t(sl), 1));
      sl += int(pair_u(uint32_t(sl), 2));
      sl += int(pair_u(uint32_t(sl), 4));
      sl += int(pair_u(uint32_t(sl), 8));
      if ((lane & 15) == 0) s_ci[wave][S][gs + 4 * uint32_t(L)] = (BITS == 2 ? -2 : -8) * sl;
    }
    if ((lane & 15) == 0)
      s_e[(wave * 4 + uint32_t(S)) * 4 + gs] = isfinite(mx) ? ldexpf(1.0f, e - 30) : __int_as_float(0x7fc00000);
  }
  const bool brk = break_now<MODE>(a, bin, !isfinite(tot));
  __syncthreads();  // every wave's table (the corrections read any column)
  int cinit[4];
  float lpf[4];
#pragma unroll
  for (int S = 0; S < 4; ++S) {
    cinit[S] = s_ci[wave][S][n];
    lpf[S] = s_e[(wave * 4 + uint32_t(S)) * 4 + uint32_t(n & 3)] * __int_as_float(int(127 + 8 * (n >> 2)) << 23);
  }
  const uint4* tbw = s_tb + wave * (kXmTableBytes / 16);
  const uint8_t* tbytes = reinterpret_cast<const uint8_t*>(s_tb);

  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  auto compute = [&](const XmLoads<R, SPL>& L, int buf) {
    const GemvPart P0 = kRope ? pick_part(a, L.pu) : a.part[0];
    const GemvPart& P1 = kSwi ? a.part[1] : P0;
    const uint32_t rb = L.row_base;
    // corrections of row q, spread over its 16 lanes (first: their LDS reads overlap the
    // products).  Slot t of the wave holds entries 16 (wsl + NW t) .. + 15 of each row: the
    // wave skips the slots past every row's entries (a uniform test on the tables' row width)
    const uint32_t km = kSwi ? max(uni(P0.corr_kmax), uni(P1.corr_kmax)) : uni(P0.corr_kmax);
    float acc = 0.0f;
    if (16u * wsl < km) {
#pragma unroll
      for (int t = 0; t < SPL; ++t) {
        if (16u * (wsl + uint32_t(NW * t)) < km) {
          const bool on = ((L.cuse >> t) & 1u) && L.ce[t].y != 0.0f;
          const float xc = xm_input<BITS>(tbytes, s_e, on ? __float_as_uint(L.ce[t].x) : 0u);
          acc = on ? fmaf(L.ce[t].y, xc, acc) : acc;
        }
      }
    }
    // the products: lane (n, q) adds its limb's share of group n % 4 of each set, times the
    // group scale; the row's sum over the 16 lanes (limbs, then groups) is taken once at the end
#pragma unroll
    for (int S = 0; S < 4; ++S) {
      i32x4_t D = {cinit[S], cinit[S], cinit[S], cinit[S]};
      const uint32_t w4[4] = {L.q[S].x, L.q[S].y, L.q[S].z, L.q[S].w};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 t = tbw[uint32_t(S) * 128 + (((uint32_t(n & 3) * 4 + uint32_t(q)) * 2 + uint32_t(h)) * 4) + uint32_t(n >> 2)];
        const i32x4_t B = {int(t.x), int(t.y), int(t.z), int(t.w)};
        i32x4_t A;
        if constexpr (BITS == 2) {  // 16 codes in 4 bytes: field k of each byte, code ^ 2
          const uint32_t w = w4[h] ^ 0xAAAAAAAAu;
          A = i32x4_t{int(w & 0x03030303u), int((w >> 2) & 0x03030303u), int((w >> 4) & 0x03030303u),
                      int((w >> 6) & 0x03030303u)};
        } else {
          const uint32_t w0 = w4[2 * h], w1 = w4[2 * h + 1];
          A = i32x4_t{int(w0 & 0x0f0f0f0fu), int((w0 >> 4) & 0x0f0f0f0fu), int(w1 & 0x0f0f0f0fu),
                      int((w1 >> 4) & 0x0f0f0f0fu)};
        }
        D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, D, 0, 0, 0);
      }
      const int j = n & 3;
      const int v = j == 0 ? D[0] : j == 1 ? D[1] : j == 2 ? D[2] : D[3];
      // (a group past the input: its products are zero; its scale, read from group 0, is not used)
      const bool gv = gw + 4 * uint32_t(S) + uint32_t(n & 3) < ng;
      acc = gv ? fmaf(float(v) * lpf[S], h2f(uint16_t(L.s[S])), acc) : acc;
    }
    acc = ((acc + dpp_f<0x114>(acc)) + dpp_f<0x118>(acc)) + dpp_f<0x11c>(acc);
    acc = pair_sum(acc, 1);
    acc = pair_sum(acc, 2);
    {
      const bool second = kSwi && q >= R / 2;
      const uint32_t r = row_of<R, MODE>(rb, q, half);
      const uint32_t wr = second ? uni(P1.wrows) : uni(P0.wrows);
      if (n == 12) s_part[buf][wave][q] = r < wr ? acc : 0.0f;
    }
    __syncthreads();
    if (wave == 0 && lane < NE) {
      float y0 = 0.0f, y1 = 0.0f;
#pragma unroll
      for (int w = 0; w < NW; ++w) {
        y0 += s_part[buf][w][lane];
        if constexpr (kSwi || kRope) y1 += s_part[buf][w][lane + R / 2];
      }
      const uint32_t r = row_of<R, MODE>(rb, lane, half);
      if constexpr (kRope) {
        if (r < P0.rows) rope_store(a, P0, r, y0 + L.pre, y1 + L.pre2, L.rc, L.rs, brk);
      } else if (MODE != int(GemvMode::Accum) || r < P0.wrows) {  // Accum: rows past the tiles stay
        epilogue<MODE>(P0, r, y0, y1, L.pre, &bv, &bi, &nf, brk);
      }
    }
  };

  // 3. the units: the next unit's loads, then the current unit's products (static buffers)
  bool last_b = false;
  while (unit + step < n_units) {
    issue(unit + step, &LB);
    compute(LA, 0);
    unit += step;
    if (unit + step >= n_units) {
      last_b = true;
      break;
    }
    issue(unit + step, &LA);
    compute(LB, 1);
    unit += step;
  }
  if (last_b) compute(LB, 1);
  else compute(LA, 0);
  if constexpr (kLogits) {
    argmax_partial<MODE>(a, bv, bi, nf, s_bv, s_bi, s_nf);
    if (blockIdx.x == 0 && threadIdx.x == 0) a.result->hidden_norm = sqrtf(tot);
  }
}

template <int MODE, int BITS = 4, bool kXc = false>
bool launch_xm(const GemvArgs& a, const GemvLaunch& g, hipStream_t st) {
  if constexpr (BITS == 2 && !kXc)
    if (a.part[0].xcodes) return launch_xm<MODE, 2, true>(a, g, st);
  const uint32_t nw = g.threads / kWave;
  const size_t lds = size_t(nw) * kXmTableBytes + size_t(nw) * 16 * 4;
  const dim3 gr(g.blocks), bl(g.threads);
  switch (nw) {
    case 1: launch_kernel_lds(&k_gemv_xm<MODE, 1, BITS, kXc>, gr, bl, lds, st, a); return true;
    case 2: launch_kernel_lds(&k_gemv_xm<MODE, 2, BITS, kXc>, gr, bl, lds, st, a); return true;
    case 4: launch_kernel_lds(&k_gemv_xm<MODE, 4, BITS, kXc>, gr, bl, lds, st, a); return true;
    case 8: launch_kernel_lds(&k_gemv_xm<MODE, 8, BITS, kXc>, gr, bl, lds, st, a); return true;
    case 15: launch_kernel_lds(&k_gemv_xm<MODE, 15, BITS, kXc>, gr, bl, lds, st, a); return true;
    case 16: launch_kernel_lds(&k_gemv_xm<MODE, 16, BITS, kXc>, gr, bl, lds, st, a); return true;
    default: return false;
  }
}

// The permuted copy of a launch's codes for k_gemv_xm: thread (w, lane) of workgroup u copies
// what the kernel's lane reads for unit u (xm_code_at).  4-bit: the 16 bytes of set S to
// dst + u * NW * 4096 + ((w * 4 + S) * 64 + lane) * 16.  2-bit: the 8 bytes of sets 2 p and
// 2 p + 1 side by side to dst + u * NW * 2048 + ((w * 2 + p) * 64 + lane) * 16.
template <int MODE, int NW, int BITS = 4>
__global__ void __launch_bounds__(kWave * NW) k_xm_layout(GemvArgs a, uint8_t* dst) {
  constexpr int R = 4;
  const int lane = threadIdx.x & 63, n = lane & 15, q = lane >> 4;
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), u = blockIdx.x;
  const uint32_t ng = a.C >> 7, half = a.rope.head_dim / 2, gw = wave * 16;
  args_batch<MODE>(a);
  const GemvPart P0 = MODE == int(GemvMode::QkvRope) ? pick_part(a, int(__builtin_amdgcn_readfirstlane(part_of(a, u))))
                                                      : a.part[0];
  const GemvPart& P1 = MODE == int(GemvMode::SwiGlu) ? a.part[1] : P0;
  const uint32_t rb = xs_row_base<R, MODE>(P0, u, half);
  if constexpr (BITS == 2) {
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      const uint2 v0 = ld_u64(xm_code_at<R, MODE, 2>(P0, P1, rb, half, ng, gw, 2 * p, n, q));
      const uint2 v1 = ld_u64(xm_code_at<R, MODE, 2>(P0, P1, rb, half, ng, gw, 2 * p + 1, n, q));
      *reinterpret_cast<uint4*>(dst + (size_t(u) * (NW * 2048u) + ((wave * 2 + uint32_t(p)) * 64 + uint32_t(lane)) * 16)) =
          make_uint4(v0.x, v0.y, v1.x, v1.y);
    }
  } else {
#pragma unroll
    for (int S = 0; S < 4; ++S) {
      const uint4 v = ld_u128(xm_code_at<R, MODE>(P0, P1, rb, half, ng, gw, S, n, q));
      *reinterpret_cast<uint4*>(dst + (size_t(u) * (NW * 4096u) + ((wave * 4 + uint32_t(S)) * 64 + uint32_t(lane)) * 16)) = v;
    }
  }
}

template <int MODE, int BITS>
bool launch_xm_layout(const GemvArgs& a, const GemvLaunch& g, uint8_t* dst, hipStream_t st) {
  const dim3 gr(a.n_units), bl(g.threads);
  switch (g.threads / kWave) {
    case 1: launch_kernel(&k_xm_layout<MODE, 1, BITS>, gr, bl, st, a, dst); return true;
    case 2: launch_kernel(&k_xm_layout<MODE, 2, BITS>, gr, bl, st, a, dst); return true;
    case 4: launch_kernel(&k_xm_layout<MODE, 4, BITS>, gr, bl, st, a, dst); return true;
    case 8: launch_kernel(&k_xm_layout<MODE, 8, BITS>, gr, bl, st, a, dst); return true;
    case 15: launch_kernel(&k_xm_layout<MODE, 15, BITS>, gr, bl, st, a, dst); return true;
    case 16: launch_kernel(&k_xm_layout<MODE, 16, BITS>, gr, bl, st, a, dst); return true;
    default: return false;
  }
}

// the x-stationary kernel's variant for a launch: NW waves of 64 * F::kCols columns
template <class F, int MODE>
bool launch_xs(const GemvArgs& a, const GemvLaunch& g, hipStream_t st) {
  const size_t lds = size_t(a.C) * 4;
  const dim3 gr(g.blocks), bl(g.threads);
  const uint32_t nw = g.threads / kWave;
#define CHPE_XS(Rv, NWv)                                                                         \
  if (g.xs == Rv && nw == NWv) {                                                                 \
    launch_kernel_lds(&k_gemv_xs<F, MODE, Rv, NWv>, gr, bl, lds, st, a);                         \
    return true;                                                                                 \
  }
  CHPE_XS(4, 1) CHPE_XS(4, 2) CHPE_XS(4, 4) CHPE_XS(2, 4) CHPE_XS(2, 8) CHPE_XS(4, 8) CHPE_XS(2, 16) CHPE_XS(4, 16)
#undef CHPE_XS
  return false;
}

template <class F, int MODE>
void launch_one(const GemvArgs& a, const GemvLaunch& g, hipStream_t st) {
  const size_t lds = size_t(xs_floats(a.C)) * 4;
  if constexpr (std::is_same_v<F, Cell16W4> && MODE == int(GemvMode::Logits)) {
    if (g.mma) {
      launch_kernel(&k_gemv_mma_logits, dim3(g.blocks), dim3(g.threads), st, a);
      return;
    }
  }
  if constexpr (std::is_same_v<F, Cell16W4> && MODE != int(GemvMode::Logits)) {
    if (g.mma) {
      if constexpr (MODE == int(GemvMode::SwiGlu)) {
        launch_kernel(&k_gemv_mma<MODE, 2>, dim3(g.blocks), dim3(g.threads), st, a);
      } else if (g.mma == 2) {
        launch_kernel(&k_gemv_mma<MODE, 2>, dim3(g.blocks), dim3(g.threads), st, a);
      } else {
        launch_kernel(&k_gemv_mma<MODE, 1>, dim3(g.blocks), dim3(g.threads), st, a);
      }
      return;
    }
    if (g.cells == 1) { launch_kernel(&k_gemv_cells<MODE, 1>, dim3(g.blocks), dim3(g.threads), st, a); return; }
    if (g.cells == 2) { launch_kernel(&k_gemv_cells<MODE, 2>, dim3(g.blocks), dim3(g.threads), st, a); return; }
    if (g.cells == 4) { launch_kernel(&k_gemv_cells<MODE, 4>, dim3(g.blocks), dim3(g.threads), st, a); return; }
  }
  if constexpr (std::is_same_v<F, FlatW4> || std::is_same_v<F, FlatW2>) {
    if (g.xm) {
      if (launch_xm<MODE, std::is_same_v<F, FlatW2> ? 2 : 4>(a, g, st)) return;
      std::fprintf(stderr, "chpe: no matrix-core flat kernel for %u waves\n", g.threads / kWave);
      return;
    }
  }
  if constexpr (std::is_same_v<F, FlatW4> || std::is_same_v<F, FlatW2>) {
    if (g.xs) {
      if (launch_xs<F, MODE>(a, g, st)) return;
      std::fprintf(stderr, "chpe: no input-stationary kernel for %u rows x %u waves\n", g.xs, g.threads / kWave);
      return;
    }
  }
  if constexpr (std::is_same_v<F, FlatW4> && MODE != int(GemvMode::Logits)) {
    if (g.flat) {
      const dim3 gr(g.blocks), bl(g.threads);
      const bool wide = a.C > 8u * 4u * uint32_t(kWave * kFlatWaves);
      switch (g.flat) {
        case 1: launch_kernel_lds(&k_gemv_flat<MODE, 1, false>, gr, bl, lds, st, a); return;
        case 2: launch_kernel_lds(&k_gemv_flat<MODE, 2, false>, gr, bl, lds, st, a); return;
        case 3: launch_kernel_lds(&k_gemv_flat<MODE, 3, false>, gr, bl, lds, st, a); return;
        case 4: launch_kernel_lds(&k_gemv_flat<MODE, 4, false>, gr, bl, lds, st, a); return;
        default:
          if (wide) launch_kernel_lds(&k_gemv_flat<MODE, 8, true>, gr, bl, lds, st, a);
          else launch_kernel_lds(&k_gemv_flat<MODE, 8, false>, gr, bl, lds, st, a);
          return;
      }
    }
  }
  if (a.waves_per_unit == 1)
    launch_kernel(&k_gemv_rows<F, MODE>, dim3(g.blocks), dim3(g.threads), st, a);
  else if (a.C > 4 * 8 * g.threads)  // more than 8 float4 per thread: staged in two passes
    launch_kernel_lds(&k_gemv_split<F, MODE, true>, dim3(g.blocks), dim3(g.threads), lds, st, a);
  else
    launch_kernel_lds(&k_gemv_split<F, MODE, false>, dim3(g.blocks), dim3(g.threads), lds, st, a);
}

template <class F>
void launch_layout(const GemvArgs& a, const GemvLaunch& g, hipStream_t st) {
  switch (GemvMode(a.mode)) {
    case GemvMode::Store: launch_one<F, int(GemvMode::Store)>(a, g, st); break;
    case GemvMode::Accum: launch_one<F, int(GemvMode::Accum)>(a, g, st); break;
    case GemvMode::SwiGlu: launch_one<F, int(GemvMode::SwiGlu)>(a, g, st); break;
    case GemvMode::Logits: launch_one<F, int(GemvMode::Logits)>(a, g, st); break;
    case GemvMode::QkvRope: launch_one<F, int(GemvMode::QkvRope)>(a, g, st); break;
  }
}

// ---- polymorphic 16-row cells of any width (gemvTilePolymorphic, chpe_engine.zig:732-751) ----
// Tensors whose cells are not all 16 x 2048 group-128 4-bit cells: each cell is dequantised by
// its own metadata -- 2-bit codebook (:223-323), 4-bit (:326-418), int8 with one scale and
// bias per row (:421-472), fp16 / bf16 (:475-541), f32 (:544-581), unknown widths as 2-bit
// (:746-749), group-128 scales or the tile's scale / bias, outliers added for group-128 cells
// of 16 rows -- into raw row sums; a second launch applies the mode's epilogue.  Rows are the
// prefix sums of dims.rows the host computed by gemvLinear's walk (:1430-1442).

// x (RMSNorm'ed with gamma when gamma is set: (x * inv_rms) * gamma, rmsNorm :163-193) into out
// and its sum of squares into out[n] (and |x|, the hidden norm of the LM head's input, into
// *result when set)
__global__ void __launch_bounds__(1024) k_rmsnorm(const float* x, const float* gamma, float eps, uint32_t n,
                                                  float* out, StepResult* result) {
#pragma clang fp contract(off)
  __shared__ float s_red[16];
  float ss = 0.0f;
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) ss += x[i] * x[i];
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) ss = pair_sum(ss, m);
  if ((threadIdx.x & 63) == 0) s_red[threadIdx.x >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
  for (int w = 0; w < int(blockDim.x / kWave); ++w) tot += s_red[w];
  const float inv = 1.0f / sqrtf(tot / float(n) + eps);
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) out[i] = (x[i] * inv) * gamma[i];
  if (threadIdx.x == 0) out[n] = tot;
  if (result && threadIdx.x == 0) result->hidden_norm = sqrtf(tot);
}

__device__ __forceinline__ float poly_w2(uint32_t code) {  // CODEBOOK_W2 (:220)
  return code == 0 ? 0.0f : (code == 1 ? 1.0f : (code == 2 ? -2.0f : -1.0f));
}

// one workgroup per cell (4 waves, wave w takes rows w, w + 4, ...); block n_cells zeroes the
// rows past the last cell
__global__ void __launch_bounds__(256) k_gemv_poly(const uint8_t* base, uint32_t stride, const uint32_t* row_base,
                                                    uint32_t n_cells, const float* x, uint32_t x_len, float* raw,
                                                    uint32_t y_len) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (blockIdx.x == n_cells) {
    for (uint32_t r = row_base[n_cells] + threadIdx.x; r < y_len; r += blockDim.x) raw[r] = 0.0f;
    return;
  }
  const uint8_t* cell = base + size_t(blockIdx.x) * stride;
  const uint8_t* codes = cell + 64;
  const uint8_t* pl = cell + 16448;
  const uint32_t qb = pl[20];
  const bool g128 = (*reinterpret_cast<const uint32_t*>(pl + 24) & 1u) != 0;
  const float scale = *reinterpret_cast<const float*>(pl + 32), bias = *reinterpret_cast<const float*>(pl + 36);
  const uint32_t rows = *reinterpret_cast<const uint32_t*>(pl + 40), cols = *reinterpret_cast<const uint32_t*>(pl + 44);
  const uint32_t rb = row_base[blockIdx.x];
  if (rb >= y_len) return;
  const uint32_t max_rows = rows < y_len - rb ? rows : y_len - rb;
  const uint32_t kind = (qb == 4 || qb == 8 || qb == 16 || qb == 32) ? qb : 2u;
  const bool outl = g128 && rows == 16 && (kind == 2 || kind == 4);
  const uint32_t total_g = cols / 128, ng = total_g < x_len / 128 ? total_g : x_len / 128;
  const uint32_t max_cols = cols < x_len ? cols : x_len;
  for (uint32_t r = wave; r < max_rows; r += 4) {
    float acc = 0.0f;
    if (kind == 4) {
      const uint8_t* rowb = codes + size_t(r) * (cols / 2);
      if (g128) {
        for (uint32_t c = lane; c < ng * 128; c += 64) {
          const float q = float((rowb[c / 2] >> (4 * (c & 1))) & 15u) - 8.0f;
          acc += (q * x[c]) * h2f(*reinterpret_cast<const uint16_t*>(pl + 48 + 2 * (r * total_g + c / 128)));
        }
      } else {
        const uint32_t pairs = cols / 2 < x_len / 2 ? cols / 2 : x_len / 2;
        for (uint32_t c = lane; c < 2 * pairs; c += 64) {
          const float q = float((rowb[c / 2] >> (4 * (c & 1))) & 15u) - 8.0f;
          acc += (q * scale + bias) * x[c];
        }
      }
    } else if (kind == 2) {
      const uint8_t* rowb = codes + size_t(r) * (cols / 4);
      if (g128) {
        for (uint32_t c = lane; c < ng * 128; c += 64) {
          const float q = poly_w2((rowb[c / 4] >> (2 * (c & 3))) & 3u);
          acc += (q * x[c]) * h2f(*reinterpret_cast<const uint16_t*>(pl + 48 + 2 * (r * total_g + c / 128)));
        }
      } else {
        const uint32_t quads = cols / 4 < x_len / 4 ? cols / 4 : x_len / 4;
        for (uint32_t c = lane; c < 4 * quads; c += 64) {
          const float q = poly_w2((rowb[c / 4] >> (2 * (c & 3))) & 3u);
          acc += (q * scale + bias) * x[c];
        }
      }
    } else if (kind == 8) {
      const int8_t* rowb = reinterpret_cast<const int8_t*>(codes) + size_t(r) * cols;
      for (uint32_t c = lane; c < max_cols; c += 64) acc += float(rowb[c]) * x[c];
    } else if (kind == 16) {
      const uint16_t* rowb = reinterpret_cast<const uint16_t*>(codes) + size_t(r) * cols;
      const bool fp16 = (*reinterpret_cast<const uint32_t*>(pl + 24) & 4u) != 0;
      for (uint32_t c = lane; c < max_cols; c += 64) acc += (fp16 ? h2f(rowb[c]) : bf2f(rowb[c])) * x[c];
    } else {
      const float* rowb = reinterpret_cast<const float*>(codes) + size_t(r) * cols;
      for (uint32_t c = lane; c < max_cols; c += 64) acc += rowb[c] * x[c];
    }
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) acc = pair_sum(acc, m);
    if (outl) {  // outliers added (:309-315): lane k < 8 takes entry k; their sum joins on lane 0
      const uint32_t k = uint32_t(lane) & 7u;
      const uint32_t col = *reinterpret_cast<const uint16_t*>(pl + 816 + 2 * k);
      float o = (lane < 8 && col < x_len) ? h2f(*reinterpret_cast<const uint16_t*>(pl + 560 + 2 * (r * 8 + k))) * x[col]
                                          : 0.0f;
#pragma unroll
      for (int m = 1; m < 8; m <<= 1) o = pair_sum(o, m);
      acc += o;
    }
    if (kind == 8) acc = acc * scale + bias;  // (:461)
    if (lane == 0) raw[rb + r] = acc;
  }
}

// ---- flat tiles of any form gemvCellFlat decodes (src/chpe_engine.zig:584-729) ---------------
// Tensors the uniform flat kernels do not take -- tiles without GROUP128 (each weight
// value * dims.scale + dims.bias), widths other than 2 and 4 bits (all weights zero), a mix of
// forms, tiles that end inside a row of a short tensor, rows whose width is not a multiple of
// 128, more outliers per row than the correction table holds -- run here.  One workgroup per
// tile materialises its 32768 weights in LDS as the reference does (the product and the sum
// rounded separately, outliers replacing in entry order), then dots each row segment of the tile
// with x into part[tile][segment]; k_flat_poly_rows adds each row's segments in tile order.
constexpr uint32_t kFlatPolyThreads = 512;
__host__ __device__ constexpr uint32_t flat_poly_segments(uint32_t C) { return 32768u / C + 2u; }

__global__ void __launch_bounds__(kFlatPolyThreads) k_flat_poly(const uint8_t* base, uint32_t stride, uint32_t R,
                                                                uint32_t C, const float* x, float* part) {
#pragma clang fp contract(off)
  extern __shared__ __align__(16) float s_w[];  // the tile's 32768 weights
  const uint32_t t = blockIdx.x, tid = threadIdx.x, lane = tid & 63u, wave = tid >> 6;
  const uint8_t* cell = base + size_t(t) * stride;
  const uint8_t* codes = cell + 64;
  const uint8_t* pl = cell + 16448;
  const uint32_t qb = pl[20];
  const bool g128 = (*reinterpret_cast<const uint32_t*>(pl + 24) & 1u) != 0;
  const float scale = *reinterpret_cast<const float*>(pl + 32), bias = *reinterpret_cast<const float*>(pl + 36);
  const uint16_t* gs = reinterpret_cast<const uint16_t*>(pl + 48);
  for (uint32_t k = tid; k < 32768u; k += blockDim.x) {
    float w = 0.0f;  // (other widths: zero, :694-696)
    if (qb == 4 || qb == 2) {
      const float q = qb == 4 ? float((codes[k / 2] >> (4 * (k & 1))) & 15u) - 8.0f
                              : poly_w2((codes[k / 4] >> (2 * (k & 3))) & 3u);
      w = g128 ? q * h2f(gs[k / 128]) : q * scale + bias;  // :607-630, :654-677
    }
    s_w[k] = w;
  }
  __syncthreads();
  if (tid == 0 && (qb == 4 || qb == 2)) {  // outliers replace, in entry order (:632-646, :680-693)
    const uint32_t n = *reinterpret_cast<const uint16_t*>(pl + 560);
    if (n > 0 && n <= 64)
      for (uint32_t m = 0; m < n; ++m) {
        const uint32_t off = *reinterpret_cast<const uint16_t*>(pl + 690 + 2 * m);
        if (off < 32768u) s_w[off] = h2f(*reinterpret_cast<const uint16_t*>(pl + 562 + 2 * m));
      }
  }
  __syncthreads();
  // the segments (:698-727): row r_first + s of the tile, wave w takes segments w, w + 8, ..
  const uint64_t f0 = uint64_t(t) * 32768u;
  const uint64_t r_first = f0 / C;
  if (r_first >= R) return;
  const uint64_t r_last = min(uint64_t(R) - 1, (f0 + 32767u) / C);
  const uint32_t n_seg = uint32_t(r_last - r_first + 1), ps = flat_poly_segments(C);
  for (uint32_t sg = wave; sg < n_seg; sg += blockDim.x / 64) {
    const uint64_t r = r_first + sg, rs = r * C;
    const uint32_t j0 = uint32_t((rs > f0 ? rs : f0) - f0), j1 = uint32_t(min(f0 + 32768u, rs + C) - f0);
    const float* xs = x + (f0 + j0 - rs);
    float acc = 0.0f;
    for (uint32_t j = j0 + lane; j < j1; j += 64) acc = fmaf(s_w[j], xs[j - j0], acc);
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) acc = pair_sum(acc, m);
    if (lane == 0) part[size_t(t) * ps + sg] = acc;
  }
}

// raw[r] = the row's segments in tile order (y[r] += dot, :719); rows past the tiles: 0
__global__ void __launch_bounds__(256) k_flat_poly_rows(const float* part, uint32_t n_tiles, uint32_t R, uint32_t C,
                                                        float* raw) {
#pragma clang fp contract(off)
  const uint32_t ps = flat_poly_segments(C);
  for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < R; r += gridDim.x * blockDim.x) {
    const uint64_t a = uint64_t(r) * C, b = a + C - 1;
    float v = 0.0f;
    for (uint64_t t = a / 32768u; t <= b / 32768u && t < n_tiles; ++t) v += part[t * ps + (r - (t * 32768u) / C)];
    raw[r] = v;
  }
}

// the mode's epilogue on the raw row sums: grid-stride over rows (QkvRope: over RoPE pairs);
// ss: the normalised input's sum of squares (k_rmsnorm), or null
template <int MODE>
__global__ void __launch_bounds__(256) k_poly_epilogue(GemvArgs a, PolyRaw raw, const float* ss) {
#pragma clang fp contract(off)
  __shared__ float s_bv[4];
  __shared__ uint32_t s_bi[4], s_nf[4];
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  const uint32_t stride = gridDim.x * blockDim.x;
  const bool brk = break_now<MODE>(a, break_in<MODE>(a), ss != nullptr && !isfinite(*ss));
  if constexpr (MODE == int(GemvMode::QkvRope)) {
    const uint32_t half = a.rope.head_dim / 2;
    for (int p = 0; p < a.n_parts; ++p) {
      const GemvPart& P = a.part[p];
      for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < P.rows / 2; i += stride) {
        const uint32_t r = (i / half) * (2 * half) + i % half, d = i % half;
        const float lo = raw.y[p][r] + (P.bias ? P.bias[r] : 0.0f);
        const float hi = raw.y[p][r + half] + (P.bias ? P.bias[r + half] : 0.0f);
        rope_store(a, P, r, lo, hi, a.rope.cos[d], a.rope.sin[d], brk);
      }
    }
  } else {
    const GemvPart& P = a.part[0];
    for (uint32_t r = blockIdx.x * blockDim.x + threadIdx.x; r < P.rows; r += stride) {
      const float v = raw.y[0][r];
      const float u = MODE == int(GemvMode::SwiGlu) ? raw.y[1][r] : 0.0f;
      const float pre = MODE == int(GemvMode::Accum) ? P.y[r] : (P.bias ? P.bias[r] : 0.0f);
      epilogue<MODE>(P, r, v, u, pre, &bv, &bi, &nf, brk);
    }
  }
  if constexpr (MODE == int(GemvMode::Logits)) argmax_partial<MODE>(a, bv, bi, nf, s_bv, s_bi, s_nf);
}

}  // namespace

const GemvTuning& gemv_tuning() {
  static const GemvTuning t = [] {
    GemvTuning v;
    if (const char* e = std::getenv("CHPE_GEMV_ROWS_BLOCKS")) v.rows_blocks = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_LOGITS_BLOCKS")) v.logits_blocks = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_CELLS")) v.cells = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_FLAT")) v.flat = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_MMA")) v.mma = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_MMA_LOGITS_BLOCKS")) v.mma_logits_blocks = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_XS")) v.xs = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_XM")) v.xm = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_XM_WPC")) {
      unsigned w[4] = {v.xm_wpc_small, v.xm_wpc_large, v.xm_wpc_logits, v.xm_wpc_wide};
      if (std::sscanf(e, "%u,%u,%u,%u", &w[0], &w[1], &w[2], &w[3]) == 4 && w[0] && w[1] && w[2] && w[3]) {
        v.xm_wpc_small = w[0];
        v.xm_wpc_large = w[1];
        v.xm_wpc_logits = w[2];
        v.xm_wpc_wide = w[3];
      }
    }
    if (const char* e = std::getenv("CHPE_XM_LAYOUT")) v.xm_layout = e[0] == '0' ? 0u : 1u;
    if (const char* e = std::getenv("CHPE_GEMV_XM2")) v.xm2 = e[0] == '0' ? 0u : 1u;
    if (const char* e = std::getenv("CHPE_GEMV_XM_WPC_GATEUP")) v.xm_wpc_gateup = uint32_t(std::strtoul(e, nullptr, 10));
    if (v.xm_wpc_gateup == 0) v.xm_wpc_gateup = 1;
    if (const char* e = std::getenv("CHPE_GEMV_XS_MIN_UNITS")) v.xs_min_units = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_XM_MIN_MB")) v.xm_min_mb = uint32_t(std::strtoul(e, nullptr, 10));
    if (const char* e = std::getenv("CHPE_GEMV_XS_WPC")) {
      unsigned w[4] = {v.xs_wpc_small, v.xs_wpc_large, v.xs_wpc_logits, v.xs_wpc_wide};
      if (std::sscanf(e, "%u,%u,%u,%u", &w[0], &w[1], &w[2], &w[3]) == 4 && w[0] && w[1] && w[2] && w[3]) {
        v.xs_wpc_small = w[0];
        v.xs_wpc_large = w[1];
        v.xs_wpc_logits = w[2];
        v.xs_wpc_wide = w[3];
      }
    }
    if (v.mma_logits_blocks == 0 || v.mma_logits_blocks > kMaxLogitsBlocks) v.mma_logits_blocks = kMaxLogitsBlocks;
    if (v.logits_blocks == 0 || v.logits_blocks > kMaxLogitsBlocks) v.logits_blocks = kMaxLogitsBlocks;
    return v;
  }();
  return t;
}

// the 4-bit codes of the launch reach the persistent kernels' size threshold (CHPE_GEMV_XM_MIN_MB)
static bool persistent_pays(const uint32_t* rows, int n_parts, GemvMode mode, uint32_t C) {
  uint64_t r = 0;
  for (int p = 0; p < n_parts; ++p) r += rows[p];
  if (mode == GemvMode::SwiGlu && n_parts == 1) r *= 2;
  return r * C / 2 >= uint64_t(gemv_tuning().xm_min_mb) << 20;
}

GemvLaunch gemv_geometry(WeightKind kind, GemvMode mode, uint32_t C, const uint32_t* rows, int n_parts,
                         uint32_t* n_units, uint32_t* n_panels, uint32_t* waves_per_unit,
                         uint32_t* unit_begin) {
  const uint32_t ru = 8;
  if (((kind == WeightKind::FlatW4 && gemv_tuning().xm) || (kind == WeightKind::FlatW2 && gemv_tuning().xm2)) &&
      C % 128 == 0 && C <= 32768) {
    // the matrix-core input-stationary kernel: waves of 2048 columns, units of 4 rows
    const uint32_t need = (C + 2047) / 2048;
    // (15 columns of waves exactly: the 72B down projection's 29568 columns; a 16th wave would
    // hold no group and still join every unit's barrier)
    const uint32_t nw = need <= 1 ? 1u : need <= 2 ? 2u : need <= 4 ? 4u : need <= 8 ? 8u : need == 15 ? 15u : 16u;
    constexpr uint32_t R = 4;
    bool ok = true;
    if (mode == GemvMode::QkvRope)  // whole units per part (head dims are 128 or 256: whole pairs per unit)
      for (int p = 0; p < n_parts; ++p) ok = ok && rows[p] % R == 0;
    // (launches of fewer units -- the 72B q/k/v and o projections, the 3B and 9B down
    // projections -- run faster on the one-unit-per-workgroup kernels: the persistent grid's
    // start-up, the input's limb tables included, is not amortised over enough units; a launch
    // reading many codes in few wide units, the 72B down projection, amortises it all the same)
    // (2-bit tiles take the matrix-core kernel at every size: the vector-ALU kernels are
    // bound by their arithmetic there)
    if (kind == WeightKind::FlatW4 && mode != GemvMode::Logits && !persistent_pays(rows, n_parts, mode, C)) {
      uint32_t u = 0;
      for (int p = 0; p < (mode == GemvMode::SwiGlu ? 1 : n_parts); ++p)
        u += mode == GemvMode::SwiGlu ? (rows[p] + R / 2 - 1) / (R / 2) : (rows[p] + R - 1) / R;
      ok = ok && u >= gemv_tuning().xs_min_units;
    }
    if (ok) {
      uint32_t units = 0;
      if (mode == GemvMode::SwiGlu) {
        units = (rows[0] + R / 2 - 1) / (R / 2);
        unit_begin[0] = unit_begin[1] = 0;
      } else {
        for (int p = 0; p < n_parts; ++p) {
          unit_begin[p] = units;
          units += (rows[p] + R - 1) / R;
        }
      }
      *n_units = units;
      *n_panels = need;
      *waves_per_unit = nw;
      const GemvTuning& t = gemv_tuning();
      uint32_t wpc = nw >= 8 ? t.xm_wpc_wide
                     : mode == GemvMode::Logits ? t.xm_wpc_logits
                     : units >= 4096 ? (mode == GemvMode::SwiGlu && nw == 4 && t.xm_layout && kind == WeightKind::FlatW4
                                            ? t.xm_wpc_gateup  // (2-bit gate/up: 3 per CU measured faster)
                                            : t.xm_wpc_large)
                     : t.xm_wpc_small;
      if (nw < 4) wpc *= 4 / nw;  // narrower inputs: as many waves per CU as at 8192 columns
      GemvLaunch g{};
      g.ru = R;
      g.xm = R;
      g.threads = kWave * nw;
      g.blocks = std::min<uint32_t>(units, 256u * wpc);
      if (mode == GemvMode::Logits && g.blocks > kMaxLogitsBlocks) g.blocks = kMaxLogitsBlocks;
      return g;
    }
  }
  if ((kind == WeightKind::FlatW4 || kind == WeightKind::FlatW2) && gemv_tuning().xs && C % 128 == 0 &&
      size_t(C) * 4 <= size_t(150) << 10) {
    // the input-stationary persistent kernel: waves of 64 * 32 (4-bit) / 64 * 64 (2-bit) columns
    const uint32_t chunk = kind == WeightKind::FlatW4 ? 2048u : 4096u, need = (C + chunk - 1) / chunk;
    const uint32_t nw = need <= 1 ? 1u : need <= 2 ? 2u : need <= 4 ? 4u : need <= 8 ? 8u : 16u;
    const uint32_t R = nw >= 8 ? 2u : 4u;
    bool ok = need <= 16;
    // (launches of fewer units run faster on the one-unit-per-workgroup kernels, as above)
    if (mode != GemvMode::Logits && !persistent_pays(rows, n_parts, mode, C)) {
      uint32_t u = 0;
      for (int p = 0; p < (mode == GemvMode::SwiGlu ? 1 : n_parts); ++p)
        u += mode == GemvMode::SwiGlu ? (rows[p] + R / 2 - 1) / (R / 2) : (rows[p] + R - 1) / R;
      ok = ok && u >= gemv_tuning().xs_min_units;
    }
    if (mode == GemvMode::QkvRope)  // whole units per part (head dims are 128 or 256: whole pairs per unit)
      for (int p = 0; p < n_parts; ++p) ok = ok && rows[p] % R == 0;
    if (ok) {
      uint32_t units = 0;
      if (mode == GemvMode::SwiGlu) {
        units = (rows[0] + R / 2 - 1) / (R / 2);
        unit_begin[0] = unit_begin[1] = 0;
      } else {
        for (int p = 0; p < n_parts; ++p) {
          unit_begin[p] = units;
          units += (rows[p] + R - 1) / R;
        }
      }
      *n_units = units;
      *n_panels = need;
      *waves_per_unit = nw;
      const GemvTuning& t = gemv_tuning();
      const uint32_t wpc = nw >= 8 ? t.xs_wpc_wide
                           : mode == GemvMode::Logits ? t.xs_wpc_logits
                           : units >= 4096 ? t.xs_wpc_large : t.xs_wpc_small;
      GemvLaunch g{};
      g.ru = R;
      g.xs = R;
      g.threads = kWave * nw;
      g.blocks = std::min<uint32_t>(units, 256u * wpc);
      if (mode == GemvMode::Logits && g.blocks > kMaxLogitsBlocks) g.blocks = kMaxLogitsBlocks;
      return g;
    }
  }
  uint32_t panel_cols = 2048, ppw = 1;
  switch (kind) {
    case WeightKind::Cell16W4: panel_cols = Cell16W4::kPanelCols; ppw = Cell16W4::kPPW; break;
    case WeightKind::FlatW4: panel_cols = FlatW4::kPanelCols; ppw = FlatW4::kPPW; break;
    case WeightKind::FlatW2: panel_cols = FlatW2::kPanelCols; ppw = FlatW2::kPPW; break;
    case WeightKind::Raw16: panel_cols = Raw16::kPanelCols; ppw = Raw16::kPPW; break;
    case WeightKind::Raw8: panel_cols = Raw8::kPanelCols; ppw = Raw8::kPPW; break;
    case WeightKind::Cell16Poly: break;  // launched by launch_gemv_poly
    case WeightKind::FlatPoly: break;    // launched by launch_gemv_flat_poly
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
  bool rope_tiles = true;  // QkvRope tiles pair rows r, r + head_dim/2 in 8s: parts of whole 16-row heads
  for (int p = 0; p < n_parts; ++p) rope_tiles = rope_tiles && rows[p] % 16 == 0;
  if (kind == WeightKind::Cell16W4 && mode == GemvMode::Logits && C == 2048 && gemv_tuning().mma && n_parts == 1) {
    // the LM head on the matrix cores: a persistent grid striding over the 16-row cells
    const uint32_t tiles = (rows[0] + 15) / 16;
    unit_begin[0] = 0;
    *n_units = tiles;
    g.mma = 1;
    g.threads = kWave * kMmaWaves;
    const uint32_t cap = gemv_tuning().mma_logits_blocks;
    g.blocks = tiles < cap ? tiles : cap;
  } else if (kind == WeightKind::Cell16W4 && mode != GemvMode::Logits && C == 2048 && gemv_tuning().mma &&
      (mode != GemvMode::QkvRope || rope_tiles)) {
    // matrix-core kernel: tiles of 16 rows (SwiGlu: 8 gate + 8 up rows), UPW tiles per workgroup
    uint32_t tiles = 0;
    if (mode == GemvMode::SwiGlu) {  // units of 16 rows: the gate and the up cell in one workgroup
      tiles = (rows[0] + 15) / 16;
      unit_begin[0] = unit_begin[1] = 0;
    } else {
      for (int p = 0; p < n_parts; ++p) {
        unit_begin[p] = tiles;
        tiles += (rows[p] + 15) / 16;
      }
    }
    *n_units = tiles;
    const uint32_t upw = mode == GemvMode::SwiGlu || (tiles >= 1024 && gemv_tuning().mma == 2) ? 2u : 1u;
    g.mma = upw;
    g.threads = kWave * kMmaWaves;
    g.blocks = mode == GemvMode::SwiGlu ? tiles : (tiles + upw - 1) / upw;
  } else if (kind == WeightKind::Cell16W4 && mode != GemvMode::Logits && C == 2048 && gemv_tuning().cells) {
    // K-split over kCellWaves waves; units per workgroup: 1 for the small projections (more
    // workgroups, more parallel dot work), up to the tuning cap when there are thousands
    uint32_t upw = units >= 2048 ? gemv_tuning().cells : 1u;
    if (upw != 1 && upw != 2 && upw != 4) upw = 1;
    g.cells = upw;
    g.threads = kWave * kCellWaves;
    g.blocks = (units + upw - 1) / upw;
  } else if (kind == WeightKind::FlatW4 && mode != GemvMode::Logits && C <= 32768 && gemv_tuning().flat &&
             uint64_t(rows[0]) * C / 2 < (uint64_t(1) << 31) && uint64_t(rows[n_parts - 1]) * C / 2 < (uint64_t(1) << 31)) {
    // K-split over kFlatWaves waves striding over 512-column panels, one unit per workgroup
    const uint32_t panels = (C / 128 + 3) / 4, per_wave = (panels + kFlatWaves - 1) / kFlatWaves;
    g.flat = per_wave <= 4 ? per_wave : 8;
    g.threads = kWave * kFlatWaves;
    g.blocks = units;
  } else if (nw == 1) {
    g.threads = kWave * (kRowWaves + 1);
    g.blocks = (units + kRowWaves - 1) / kRowWaves;
    const uint32_t cap = mode == GemvMode::Logits ? gemv_tuning().logits_blocks : gemv_tuning().rows_blocks;
    if (cap && g.blocks > cap) g.blocks = cap;  // persistent: the waves stride over the units
  } else {
    g.threads = nw * 64;
    g.blocks = units;
    if (mode == GemvMode::Logits && g.blocks > kMaxLogitsBlocks) g.blocks = kMaxLogitsBlocks;
  }
  return g;
}

size_t flat_poly_part_floats(uint32_t n_tiles, uint32_t C) { return size_t(n_tiles) * flat_poly_segments(C); }

uint32_t launch_gemv_flat_poly(const GemvArgs& a, const uint32_t* n_tiles, float* xn, const PolyRaw& raw,
                               float* part, hipStream_t st) {
  const float* x = a.x;
  const float* ss = nullptr;
  if (a.gamma) {
    StepResult* res = GemvMode(a.mode) == GemvMode::Logits ? a.result : nullptr;
    launch_kernel(&k_rmsnorm, dim3(1), dim3(1024), st, a.x, a.gamma, a.eps, a.C, xn, res);
    x = xn;
    ss = xn + a.C;
  }
  for (int p = 0; p < a.n_parts; ++p) {
    if (n_tiles[p])
      launch_kernel_lds(&k_flat_poly, dim3(n_tiles[p]), dim3(kFlatPolyThreads), size_t(32768) * 4, st, a.part[p].base,
                        a.part[p].stride, a.part[p].rows, a.C, x, part);
    launch_kernel(&k_flat_poly_rows, dim3((a.part[p].rows + 255) / 256), dim3(256), st, part, n_tiles[p],
                  a.part[p].rows, a.C, raw.y[p]);
  }
  const uint32_t blocks = kPolyEpilogueBlocks;
  switch (GemvMode(a.mode)) {
    case GemvMode::Store: launch_kernel(&k_poly_epilogue<int(GemvMode::Store)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
    case GemvMode::Accum: launch_kernel(&k_poly_epilogue<int(GemvMode::Accum)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
    case GemvMode::SwiGlu: launch_kernel(&k_poly_epilogue<int(GemvMode::SwiGlu)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
    case GemvMode::Logits: launch_kernel(&k_poly_epilogue<int(GemvMode::Logits)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
    case GemvMode::QkvRope: launch_kernel(&k_poly_epilogue<int(GemvMode::QkvRope)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
  }
  return blocks;
}

uint32_t launch_gemv_poly(const GemvArgs& a, const PolyPlan* const* plans, float* xn, const PolyRaw& raw,
                          hipStream_t st) {
  const float* x = a.x;
  const float* ss = nullptr;
  if (a.gamma) {
    StepResult* res = GemvMode(a.mode) == GemvMode::Logits ? a.result : nullptr;
    launch_kernel(&k_rmsnorm, dim3(1), dim3(1024), st, a.x, a.gamma, a.eps, a.C, xn, res);
    x = xn;
    ss = xn + a.C;
  }
  for (int p = 0; p < a.n_parts; ++p)
    launch_kernel(&k_gemv_poly, dim3(plans[p]->n_cells + 1), dim3(256), st, a.part[p].base, a.part[p].stride,
                  plans[p]->row_base, plans[p]->n_cells, x, a.C, raw.y[p], a.part[p].rows);
  const uint32_t blocks = kPolyEpilogueBlocks;
  switch (GemvMode(a.mode)) {
    case GemvMode::Store: launch_kernel(&k_poly_epilogue<int(GemvMode::Store)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
    case GemvMode::Accum: launch_kernel(&k_poly_epilogue<int(GemvMode::Accum)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
    case GemvMode::SwiGlu: launch_kernel(&k_poly_epilogue<int(GemvMode::SwiGlu)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
    case GemvMode::Logits: launch_kernel(&k_poly_epilogue<int(GemvMode::Logits)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
    case GemvMode::QkvRope: launch_kernel(&k_poly_epilogue<int(GemvMode::QkvRope)>, dim3(blocks), dim3(256), st, a, raw, ss); break;
  }
  return blocks;
}

size_t xm_layout_bytes(WeightKind kind, const GemvArgs& a, const GemvLaunch& g) {
  const GemvMode m = GemvMode(a.mode);
  const uint32_t nw = g.threads / kWave;
  if (!gemv_tuning().xm_layout || (kind != WeightKind::FlatW4 && kind != WeightKind::FlatW2) || !g.xm) return 0;
  if (kind == WeightKind::FlatW4 && ((m != GemvMode::SwiGlu && m != GemvMode::Logits) || a.C != nw * 2048u)) return 0;
  // 2-bit: every mode of the decode step; the last wave's columns may be partly empty (the copy
  // then holds group 0 there, as the records path reads)
  if (kind == WeightKind::FlatW2 && (m == GemvMode::Store || a.C > nw * 2048u || a.C <= (nw - 1) * 2048u)) return 0;
  const size_t bytes = size_t(a.n_units) * nw * (kind == WeightKind::FlatW2 ? 2048u : 4096u);
  return bytes < (size_t(1) << 32) ? bytes : 0;
}

bool build_xm_layout(WeightKind kind, const GemvArgs& a, const GemvLaunch& g, uint8_t* dst, hipStream_t st) {
  const bool w2 = kind == WeightKind::FlatW2;
  switch (GemvMode(a.mode)) {
    case GemvMode::SwiGlu:
      return w2 ? launch_xm_layout<int(GemvMode::SwiGlu), 2>(a, g, dst, st)
                : launch_xm_layout<int(GemvMode::SwiGlu), 4>(a, g, dst, st);
    case GemvMode::Logits:
      return w2 ? launch_xm_layout<int(GemvMode::Logits), 2>(a, g, dst, st)
                : launch_xm_layout<int(GemvMode::Logits), 4>(a, g, dst, st);
    case GemvMode::Accum: return w2 && launch_xm_layout<int(GemvMode::Accum), 2>(a, g, dst, st);
    case GemvMode::QkvRope: return w2 && launch_xm_layout<int(GemvMode::QkvRope), 2>(a, g, dst, st);
    default: return false;
  }
}

void launch_gemv(WeightKind kind, const GemvArgs& a, const GemvLaunch& g, hipStream_t st) {
  const GemvMode m = GemvMode(a.mode);
  if (a.n_parts < 1 || a.n_parts > (m == GemvMode::QkvRope ? kMaxParts : m == GemvMode::SwiGlu ? 2 : 1)) {
    std::fprintf(stderr, "chpe: GEMV launch with %d parts in mode %d is not built\n", a.n_parts, a.mode);
    return;
  }
  switch (kind) {
    case WeightKind::Cell16W4: launch_layout<Cell16W4>(a, g, st); break;
    case WeightKind::FlatW4: launch_layout<FlatW4>(a, g, st); break;
    case WeightKind::FlatW2: launch_layout<FlatW2>(a, g, st); break;
    case WeightKind::Raw16: launch_layout<Raw16>(a, g, st); break;
    case WeightKind::Raw8: launch_layout<Raw8>(a, g, st); break;
    case WeightKind::Cell16Poly:
    case WeightKind::FlatPoly:
      std::fprintf(stderr, "chpe: polymorphic cells and tiles go through launch_gemv_poly / launch_gemv_flat_poly\n");
      break;
  }
}

}  // namespace chpe
