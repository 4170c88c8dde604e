// kernels.hip -- gfx950 (CDNA4) kernels of the decode step.
//
// Layout in HBM: the archive image is uploaded verbatim (cells keep their 17408/20480-byte
// stride) at a 64-byte shift so that every cell's 16384-byte code area starts on a 128-byte
// boundary.  Weights are read straight from the image with 16-byte loads and dequantised in
// registers; nothing is repacked, so every quirk of the reference's byte addressing is kept.
//
// GEMV mapping (wave64): a wave owns RW output rows; each lane owns a fixed 32-column chunk of
// x (4-bit: 16 bytes of codes per row, 2-bit: 64 columns, fp16: 8 columns per panel) held in
// registers and reused for every row the wave computes, so x is read from LDS once per wave
// while weights stream from HBM once.  The group-128 offset of the 4-bit code (q-8) is hoisted:
// sum((q-8) x) = sum(q x) - 8 sum(x).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "kernels.hpp"

namespace chpe {
namespace {

constexpr int kWave = 64;

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }
__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) {
  return *reinterpret_cast<const uint16_t*>(p);
}
__device__ __forceinline__ uint4 ld_u128(const uint8_t* p) {
  return *reinterpret_cast<const uint4*>(p);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// Reduce 4 per-lane partials (one per row) over the wave.  Lane 16*k ends with row k's sum.
__device__ __forceinline__ float wave_reduce4(const float acc[4], int lane) {
  const bool hi32 = lane & 32;
  float k0 = hi32 ? acc[2] : acc[0], k1 = hi32 ? acc[3] : acc[1];
  float s0 = hi32 ? acc[0] : acc[2], s1 = hi32 ? acc[1] : acc[3];
  k0 += __shfl_xor(s0, 32);
  k1 += __shfl_xor(s1, 32);
  const bool hi16 = lane & 16;
  float k = hi16 ? k1 : k0, s = hi16 ? k0 : k1;
  k += __shfl_xor(s, 16);
  k += __shfl_xor(k, 8);
  k += __shfl_xor(k, 4);
  k += __shfl_xor(k, 2);
  k += __shfl_xor(k, 1);
  return k;
}

// sum over 32 4-bit codes (byte k: low nibble = column 2k, high nibble = column 2k+1) times x
__device__ __forceinline__ float dot32_w4(uint4 q, const float* x) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t lo = w[i] & 0x0F0F0F0Fu, hi = (w[i] >> 4) & 0x0F0F0F0Fu;
    a0 = fmaf(float(lo & 0xffu), x[8 * i + 0], a0);
    a1 = fmaf(float(hi & 0xffu), x[8 * i + 1], a1);
    a0 = fmaf(float((lo >> 8) & 0xffu), x[8 * i + 2], a0);
    a1 = fmaf(float((hi >> 8) & 0xffu), x[8 * i + 3], a1);
    a0 = fmaf(float((lo >> 16) & 0xffu), x[8 * i + 4], a0);
    a1 = fmaf(float((hi >> 16) & 0xffu), x[8 * i + 5], a1);
    a0 = fmaf(float(lo >> 24), x[8 * i + 6], a0);
    a1 = fmaf(float(hi >> 24), x[8 * i + 7], a1);
  }
  return a0 + a1;
}

// sum over 64 2-bit codes of (code ^ 2) * x; the codebook value {0,+1,-2,-1}[c] equals
// (c ^ 2) - 2, so the -2 is hoisted like the 4-bit offset.
__device__ __forceinline__ float dot64_w2(uint4 q, const float* x) {
  const uint32_t w[4] = {q.x ^ 0xAAAAAAAAu, q.y ^ 0xAAAAAAAAu, q.z ^ 0xAAAAAAAAu, q.w ^ 0xAAAAAAAAu};
  float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {  // code k of each byte: column 4*byte + k
      const uint32_t c = (w[i] >> (2 * k)) & 0x03030303u;
      a0 = fmaf(float(c & 0xffu), x[16 * i + 0 + k], a0);
      a1 = fmaf(float((c >> 8) & 0xffu), x[16 * i + 4 + k], a1);
      a0 = fmaf(float((c >> 16) & 0xffu), x[16 * i + 8 + k], a0);
      a1 = fmaf(float(c >> 24), x[16 * i + 12 + k], a1);
    }
  }
  return a0 + a1;
}

__device__ __forceinline__ float dot8_f16(uint4 q, const float* x, bool bf16) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = uint16_t(w[i] & 0xffffu), hi = uint16_t(w[i] >> 16);
    a = fmaf(bf16 ? bf2f(lo) : h2f(lo), x[2 * i], a);
    a = fmaf(bf16 ? bf2f(hi) : h2f(hi), x[2 * i + 1], a);
  }
  return a;
}

// Block prologue: x -> LDS, normalised by RMSNorm when gamma is set (rmsNorm,
// chpe_engine.zig:163-193: inv = 1/sqrt(sum(x^2)/n + eps), y = (x*inv)*gamma).
// Returns sum(x^2) of the raw input (all threads).
__device__ float stage_x(const GemvArgs& a, float* xs, float* red) {
  const int tid = threadIdx.x, nt = blockDim.x;
  float ss = 0.0f;
  for (uint32_t i = tid; i < a.C; i += nt) {
    const float v = a.x[i];
    xs[i] = v;
    ss = fmaf(v, v, ss);
  }
  ss = wave_sum(ss);
  if ((tid & 63) == 0) red[tid >> 6] = ss;
  __syncthreads();
  float tot = 0.0f;
  for (int w = 0; w < nt / kWave; ++w) tot += red[w];
  if (a.gamma) {
    const float inv = 1.0f / sqrtf(tot / float(a.C) + a.eps);
    for (uint32_t i = tid; i < a.C; i += nt) xs[i] = xs[i] * inv * a.gamma[i];
  }
  __syncthreads();
  return tot;
}

__device__ __forceinline__ int part_of(const GemvArgs& a, uint32_t b) {
  int p = 0;
  while (p + 1 < a.n_parts && b >= a.part[p + 1].block_begin) ++p;
  return p;
}

__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return bi == 0xffffffffu || v > bv || (v == bv && i < bi);
}

// Epilogue shared by every GEMV kind.  `rowsum` is valid in lanes 16*k for k < 4 (row
// sub*4 + k of the block's row range); `row0` is the block's first row of the part.
template <int MODE>
__device__ void epilogue(const GemvArgs& a, const GemvPart& P, int which, uint32_t row0, int sub,
                         int lane, float rowsum, float* red, float hidden_ss) {
  const int k = lane >> 4;
  const bool owner = (lane & 15) == 0;
  const uint32_t r = row0 + uint32_t(sub * 4 + k);
  if constexpr (MODE == int(GemvMode::Store)) {
    if (owner && r < P.rows) P.y[r] = rowsum + (P.bias ? P.bias[r] : 0.0f);
  } else if constexpr (MODE == int(GemvMode::Accum)) {
    if (owner && r < P.rows) P.y[r] = P.y[r] + rowsum;
  } else if constexpr (MODE == int(GemvMode::SwiGlu)) {
    float* sw = red + 64;  // [2][rows_per_block]
    if (owner) sw[which * a.rows_per_block + sub * 4 + k] = rowsum;
    __syncthreads();
    const uint32_t t = threadIdx.x;
    if (t < a.rows_per_block && row0 + t < P.rows) {
      const float g = sw[t], u = sw[a.rows_per_block + t];
      P.y[row0 + t] = g / (1.0f + expf(-g)) * u;  // silu(g) * up: chpe_engine.zig:159-161, :1746-1748
    }
  } else {  // Logits: store, then the block's (max, first index) over its rows
    float* lg = red + 64;
    if (owner) {
      if (r < P.rows) P.y[r] = rowsum;
      lg[sub * 4 + k] = rowsum;
    }
    __syncthreads();
    __shared__ uint32_t s_last;
    if (threadIdx.x == 0) {
      float bv = -1e30f;
      uint32_t bi = 0xffffffffu, nonfinite = 0;
      for (uint32_t i = 0; i < a.rows_per_block && row0 + i < P.rows; ++i) {
        const float v = lg[i];
        if (!isfinite(v)) nonfinite = 1;
        if (v > -1e30f && better(v, row0 + i, bv, bi)) { bv = v; bi = row0 + i; }
      }
      a.partials[blockIdx.x] = ArgmaxPartial{bv, bi, nonfinite, 0u};
      if (blockIdx.x == 0) a.result->hidden_norm = sqrtf(hidden_ss);
      __threadfence();
      s_last = atomicAdd(a.counter, 1u) == gridDim.x - 1;
    }
    __syncthreads();
    if (s_last) {  // the last block reduces every block's partial: chpe_engine.zig:1775-1787
      __threadfence();
      float bv = -1e30f;
      uint32_t bi = 0xffffffffu, nf = 0;
      for (uint32_t i = threadIdx.x; i < gridDim.x; i += blockDim.x) {
        const ArgmaxPartial p = a.partials[i];
        nf |= p.nonfinite;
        if (p.index != 0xffffffffu && better(p.value, p.index, bv, bi)) { bv = p.value; bi = p.index; }
      }
      __shared__ float s_v[16];
      __shared__ uint32_t s_i[16], s_nf[16];
      for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o);
        const uint32_t oi = __shfl_xor(bi, o);
        if (oi != 0xffffffffu && better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
        nf |= __shfl_xor(nf, o);
      }
      const int w = threadIdx.x >> 6;
      if ((threadIdx.x & 63) == 0) { s_v[w] = bv; s_i[w] = bi; s_nf[w] = nf; }
      __syncthreads();
      if (threadIdx.x == 0) {
        for (int i = 1; i < int(blockDim.x / kWave); ++i) {
          nf |= s_nf[i];
          if (s_i[i] != 0xffffffffu && better(s_v[i], s_i[i], bv, bi)) { bv = s_v[i]; bi = s_i[i]; }
        }
        StepResult* res = a.result;
        res->argmax = bi == 0xffffffffu ? 0u : bi;
        res->max_logit = bv;
        res->token0_logit = P.y[0];
        res->all_finite = nf ? 0u : 1u;
        *a.counter = 0u;
        __threadfence();
      }
    }
  }
}

// ---------------------------------------------------------------------------------------
// 16-row 4-bit cells (gemvTileW4 + outliers: chpe_engine.zig:326-418; for the tied LM head
// the outliers replace instead: unpackEmbedRowCell :1335-1378).  Block = one cell per part
// (SwiGlu: the gate cell and the up cell); wave = 4 of the cell's 16 rows.
template <int MODE>
__global__ void __launch_bounds__(512) k_gemv_cell16_w4(GemvArgs a) {
  extern __shared__ float lds[];
  float* xs = lds;
  float* red = lds + ((a.C + 3) & ~3u);
  const float hidden_ss = stage_x(a, xs, red);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int pidx, sub;
  uint32_t cell;
  if constexpr (MODE == int(GemvMode::SwiGlu)) {
    pidx = wave >> 2; sub = wave & 3; cell = blockIdx.x;
  } else {
    pidx = part_of(a, blockIdx.x); sub = wave; cell = blockIdx.x - a.part[pidx].block_begin;
  }
  const GemvPart& P = a.part[pidx];
  const uint8_t* cp = P.base + size_t(cell) * P.stride;
  const uint8_t* codes = cp + 64;
  const uint8_t* pl = cp + 16448;

  float xr[32];
  const float4* x4 = reinterpret_cast<const float4*>(xs + lane * 32);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float4 t = x4[i];
    xr[4 * i] = t.x; xr[4 * i + 1] = t.y; xr[4 * i + 2] = t.z; xr[4 * i + 3] = t.w;
  }
  float sx = 0.0f;
#pragma unroll
  for (int i = 0; i < 32; ++i) sx += xr[i];

  uint4 q[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) q[k] = ld_u128(codes + (sub * 4 + k) * 1024 + lane * 16);
  float acc[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = sub * 4 + k;
    const float s = h2f(ld_u16(pl + 48 + 2 * (r * 16 + (lane >> 2))));
    acc[k] = (dot32_w4(q[k], xr) - 8.0f * sx) * s;
  }
  if (lane < 8) {  // 8 outlier columns shared by the cell's rows
    const uint32_t col = ld_u16(pl + 816 + 2 * lane);
    const float xo = col < a.C ? xs[col] : 0.0f;
    bool last = true;  // replace semantics: the last entry for a column wins
    for (int k2 = lane + 1; k2 < 8; ++k2) last &= ld_u16(pl + 816 + 2 * k2) != col;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int r = sub * 4 + k;
      const float w = h2f(ld_u16(pl + 560 + 2 * (r * 8 + lane)));
      if (!P.replace_outliers) {
        acc[k] += w * xo;
      } else if (last && col < a.C) {
        const uint32_t byte = codes[r * 1024 + (col >> 1)];
        const float qv = float((byte >> (4 * (col & 1))) & 15u) - 8.0f;
        const float qs = h2f(ld_u16(pl + 48 + 2 * (r * 16 + (col >> 7))));
        acc[k] += (w - qv * qs) * xo;
      }
    }
  }
  const float rs = wave_reduce4(acc, lane);
  epilogue<MODE>(a, P, pidx, cell * 16u, sub, lane, rs, red, hidden_ss);
}

// ---------------------------------------------------------------------------------------
// Flat 32768-weight tiles (gemvCellFlat: chpe_engine.zig:584-729).  Row r of an R x C tensor
// is the run of 128-weight groups [r*C/128, (r+1)*C/128); group G lives in tile G/256 at
// slot G%256 (64 code bytes at 4 bits, 32 at 2 bits; one fp16 scale).  Outliers, which
// replace weights, are applied as per-row corrections (w_out - dequantised code) * x.
template <int MODE, int BITS>
__global__ void __launch_bounds__(512) k_gemv_flat(GemvArgs a) {
  extern __shared__ float lds[];
  float* xs = lds;
  float* red = lds + ((a.C + 3) & ~3u);
  const float hidden_ss = stage_x(a, xs, red);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int pidx, sub;
  uint32_t blk;
  if constexpr (MODE == int(GemvMode::SwiGlu)) {
    pidx = wave >> 2; sub = wave & 3; blk = blockIdx.x;
  } else {
    pidx = part_of(a, blockIdx.x); sub = wave; blk = blockIdx.x - a.part[pidx].block_begin;
  }
  const GemvPart& P = a.part[pidx];
  const uint32_t row0 = blk * a.rows_per_block;
  const uint32_t gpr = a.C >> 7;
  constexpr int kLanesPerGroup = BITS == 4 ? 4 : 2;   // 16 bytes per lane
  constexpr int kGroupsPerPanel = kWave / kLanesPerGroup;
  constexpr int kCols = 128 / kLanesPerGroup;          // columns per lane
  constexpr int kGroupBytes = 16 * BITS;               // 64 or 32 code bytes per group
  const uint32_t n_panels = (gpr + kGroupsPerPanel - 1) / kGroupsPerPanel;
  const int qtr = lane % kLanesPerGroup;

  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t p = 0; p < n_panels; ++p) {
    const uint32_t gl = p * kGroupsPerPanel + lane / kLanesPerGroup;
    if (gl < gpr) {
      float xr[kCols];
      const float4* x4 = reinterpret_cast<const float4*>(xs + gl * 128 + qtr * kCols);
#pragma unroll
      for (int i = 0; i < kCols / 4; ++i) {
        const float4 t = x4[i];
        xr[4 * i] = t.x; xr[4 * i + 1] = t.y; xr[4 * i + 2] = t.z; xr[4 * i + 3] = t.w;
      }
      float sx = 0.0f;
#pragma unroll
      for (int i = 0; i < kCols; ++i) sx += xr[i];
      uint4 q[4];
      float sc[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t r = row0 + sub * 4 + k;
        if (r < P.rows) {
          const uint64_t G = uint64_t(r) * gpr + gl;
          const uint8_t* cp = P.base + (G >> 8) * P.stride;
          const uint32_t gi = uint32_t(G & 255u);
          q[k] = ld_u128(cp + 64 + gi * kGroupBytes + qtr * 16);
          sc[k] = h2f(ld_u16(cp + 16448 + 48 + 2 * gi));
        } else {
          q[k] = make_uint4(0, 0, 0, 0);
          sc[k] = 0.0f;
        }
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if constexpr (BITS == 4) acc[k] += (dot32_w4(q[k], xr) - 8.0f * sx) * sc[k];
        else acc[k] += (dot64_w2(q[k], xr) - 2.0f * sx) * sc[k];
      }
    }
  }
  if (P.corr_ptr) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t r = row0 + sub * 4 + k;
      if (r < P.rows)
        for (uint32_t j = P.corr_ptr[r] + lane; j < P.corr_ptr[r + 1]; j += kWave) {
          const float2 c = P.corr[j];
          acc[k] += c.y * xs[__float_as_uint(c.x)];
        }
    }
  }
  const float rs = wave_reduce4(acc, lane);
  epilogue<MODE>(a, P, pidx, row0, sub, lane, rs, red, hidden_ss);
}

// ---------------------------------------------------------------------------------------
// Raw fp16 / bf16 tiles (dotSegment: chpe_engine.zig:1194-1251).  Consecutive raw tiles are
// one contiguous row-major matrix, so row r is C contiguous 16-bit weights.
template <int MODE>
__global__ void __launch_bounds__(512) k_gemv_raw16(GemvArgs a) {
  extern __shared__ float lds[];
  float* xs = lds;
  float* red = lds + ((a.C + 3) & ~3u);
  const float hidden_ss = stage_x(a, xs, red);
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  int pidx, sub;
  uint32_t blk;
  if constexpr (MODE == int(GemvMode::SwiGlu)) {
    pidx = wave >> 2; sub = wave & 3; blk = blockIdx.x;
  } else {
    pidx = part_of(a, blockIdx.x); sub = wave; blk = blockIdx.x - a.part[pidx].block_begin;
  }
  const GemvPart& P = a.part[pidx];
  const uint32_t row0 = blk * a.rows_per_block;
  const bool bf16 = P.bf16 != 0;
  const uint32_t n_panels = (a.C + 511) / 512;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (uint32_t p = 0; p < n_panels; ++p) {
    const uint32_t c0 = p * 512 + lane * 8;
    if (c0 < a.C) {
      float xr[8];
      const float4 t0 = *reinterpret_cast<const float4*>(xs + c0);
      const float4 t1 = *reinterpret_cast<const float4*>(xs + c0 + 4);
      xr[0] = t0.x; xr[1] = t0.y; xr[2] = t0.z; xr[3] = t0.w;
      xr[4] = t1.x; xr[5] = t1.y; xr[6] = t1.z; xr[7] = t1.w;
      uint4 q[4];
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t r = row0 + sub * 4 + k;
        q[k] = r < P.rows ? ld_u128(P.base + (uint64_t(r) * a.C + c0) * 2) : make_uint4(0, 0, 0, 0);
      }
#pragma unroll
      for (int k = 0; k < 4; ++k) acc[k] += dot8_f16(q[k], xr, bf16);
    }
  }
  const float rs = wave_reduce4(acc, lane);
  epilogue<MODE>(a, P, pidx, row0, sub, lane, rs, red, hidden_ss);
}

// ---------------------------------------------------------------------------------------
// Byte reads of the archive image, bounded by its length: the reference reads some tensors
// past the end of their cell (see the embedding lookup below); those reads land on the
// following records exactly as on the CPU, and reads past the archive end return zero.
struct Image {
  const uint8_t* p;
  uint64_t len;
  __device__ uint8_t u8(uint64_t off) const { return off < len ? p[off] : 0; }
  __device__ uint16_t u16(uint64_t off) const { return uint16_t(u8(off) | (u8(off + 1) << 8)); }
  __device__ uint32_t u32(uint64_t off) const { return u16(off) | (uint32_t(u16(off + 2)) << 16); }
  __device__ uint64_t u64(uint64_t off) const { return u32(off) | (uint64_t(u32(off + 4)) << 32); }
  __device__ float f32(uint64_t off) const { return __uint_as_float(u32(off)); }
};

// x0*cos - x1*sin / x0*sin + x1*cos without contraction, as applyRope (chpe_engine.zig:212-213)
__device__ __forceinline__ float rope_rot(float x0, float x1, float c, float s, bool first) {
#pragma clang fp contract(off)
  return first ? x0 * c - x1 * s : x0 * s + x1 * c;
}

__device__ __forceinline__ float codebook_w2(uint32_t c) {  // chpe_engine.zig:220
  return c == 0 ? 0.0f : (c == 1 ? 1.0f : (c == 2 ? -2.0f : -1.0f));
}

// unpackEmbedRowCell (chpe_engine.zig:1288-1394) for one row of the cell at byte offset
// `cell` of the image, block-parallel over columns.  Returns false when the row is out of the
// cell's range and `out` must stay untouched.
__device__ bool unpack_embed_row_cell(const Image& im, uint64_t cell, uint32_t row, uint32_t D,
                                      float* out) {
  const uint64_t codes = cell + 64, pl = cell + 16448;
  const uint8_t qb = im.u8(pl + 20);
  const uint64_t flags = im.u64(pl + 24);
  const uint32_t ng = D / 128;
  const int tid = threadIdx.x, nt = blockDim.x;
  bool g128 = (flags & 1u) != 0;
  if (qb == 8) {
    if (row >= 8) return false;
    for (uint32_t i = tid; i < ng * 128; i += nt) {
      const float s = h2f(im.u16(pl + 48 + 2 * (row * ng + i / 128)));
      out[i] = float(int8_t(im.u8(codes + uint64_t(row) * D + i))) * s;
    }
    return true;
  }
  if (qb == 2) {
    if (row >= 16) return false;
    for (uint32_t i = tid; i < ng * 128; i += nt) {
      const float s = h2f(im.u16(pl + 48 + 2 * (row * ng + i / 128)));
      const uint32_t b = im.u8(codes + uint64_t(row) * (D / 4) + i / 4);
      out[i] = codebook_w2((b >> (2 * (i & 3))) & 3u) * s;
    }
  } else if (g128 || qb == 4) {
    if (row >= 16) return false;
    for (uint32_t i = tid; i < ng * 128; i += nt) {
      const float s = h2f(im.u16(pl + 48 + 2 * (row * ng + i / 128)));
      const uint32_t b = im.u8(codes + uint64_t(row) * (D / 2) + i / 2);
      out[i] = (float((b >> (4 * (i & 1))) & 15u) - 8.0f) * s;
    }
  } else {
    const float scale = im.f32(pl + 32), bias = im.f32(pl + 36);
    for (uint32_t i = tid; i < (D / 2) * 2; i += nt) {
      const uint32_t b = im.u8(codes + uint64_t(row) * (D / 2) + i / 2);
      const float q = float((b >> (4 * (i & 1))) & 15u);
      out[i] = __fadd_rn(__fmul_rn(q - 8.0f, scale), bias);
    }
    return true;
  }
  if (g128) {  // outliers replace, in entry order (the last entry for a column wins)
    __syncthreads();
    if (tid == 0)
      for (int k = 0; k < 8; ++k) {
        const uint32_t col = im.u16(pl + 816 + 2 * k);
        if (col < D) out[col] = h2f(im.u16(pl + 560 + 2 * (row * 8 + k)));
      }
  }
  return true;
}

// unpackEmbedRow: chpe_engine.zig:1491-1552
__global__ void __launch_bounds__(256) k_embed(EmbedArgs a) {
  const uint32_t tok = a.state->token, D = a.D;
  const Image im{a.image, a.image_len};
  const int tid = threadIdx.x, nt = blockDim.x;
  bool done = false;
  if (a.kind == 1 || a.kind == 2 || a.kind == 3) {
    const uint32_t rpt = (a.kind == 3 ? 16384u : 8192u) / D;
    if (rpt > 0 && tok / rpt < a.record_count) {
      const uint64_t base = 4096 + uint64_t(tok / rpt) * 16384;
      const uint32_t row = tok % rpt;
      for (uint32_t i = tid; i < D; i += nt) {
        const uint64_t e = uint64_t(row) * D + i;
        float v;
        if (a.kind == 1) v = h2f(im.u16(base + 2 * e));
        else if (a.kind == 2) v = bf2f(im.u16(base + 2 * e));
        else v = float(int8_t(im.u8(base + e))) * 0.00373708f;
        a.hidden[i] = v;
      }
      done = true;
    }
  } else if (a.kind == 4) {
    const uint32_t tile = tok / 16, row = tok % 16;
    if (tile < a.record_count) {
      unpack_embed_row_cell(im, 4096 + uint64_t(tile) * a.stride + a.cell_off, row, D, a.hidden);
      done = true;  // an out-of-range row leaves the previous hidden state, as on the CPU
    }
  }
  if (!done)
    for (uint32_t i = tid; i < D; i += nt) a.hidden[i] = 0.05f * float(int((i + tok) % 17u) - 8);
}

// ---------------------------------------------------------------------------------------
// RoPE + KV append + GQA attention, split over the context (flash-decoding).
// Block (c, kvh) handles positions [c*CH, c*CH+CH) for the H/KV query heads sharing kv head
// kvh; the block holding `pos` rotates and stores the new K/V row.  The last block to finish
// for kvh merges the chunks.  Semantics: chpe_engine.zig:195-216, :1693-1734 (scores
// (q.k)*scale, softmax, weighted sum of V).
template <int HD>
__global__ void __launch_bounds__(256) k_attention(AttnArgs a) {
  constexpr int CH = 8192 / HD;  // 64 positions at hd 128, 32 at hd 256
  constexpr int HALF = HD / 2;
  const uint32_t pos = a.state->pos, ctx = pos + 1;
  const uint32_t c = blockIdx.x, kvh = blockIdx.y;
  if (c * CH >= ctx) return;
  const uint32_t n_act = (ctx + CH - 1) / CH;
  const uint32_t t0 = c * CH, nv = min(uint32_t(CH), ctx - t0);
  const uint32_t G = a.H / a.KV;
  const int tid = threadIdx.x, nt = blockDim.x;

  __shared__ float qs[8][HD];
  __shared__ float ks[CH][HD + 1];
  __shared__ float vs[CH][HD];
  __shared__ float ps[8][CH];
  __shared__ float wts[8 * kAttnMaxChunks];
  __shared__ float s_m[8], s_l[8];
  __shared__ uint32_t s_last;

  const float* cs = a.rope_cos + size_t(pos) * HALF;
  const float* sn = a.rope_sin + size_t(pos) * HALF;
  for (uint32_t i = tid; i < G * HD; i += nt) {  // rotated queries
    const uint32_t g = i / HD, d = i % HD;
    const float* q = a.q_raw + size_t(kvh * G + g) * HD;
    const uint32_t j = d % HALF;
    const float x0 = q[j], x1 = q[j + HALF];
    qs[g][d] = rope_rot(x0, x1, cs[j], sn[j], d < HALF);
  }
  const size_t row_elems = size_t(a.max_seq) * HD;
  for (uint32_t i = tid; i < nv * HD; i += nt) {
    const uint32_t t = i / HD, d = i % HD, tp = t0 + t;
    float kv, vv;
    const size_t off = kvh * row_elems + size_t(tp) * HD + d;
    if (tp == pos) {  // the new row: rotate K, round to the cache type, store
      const float* k = a.k_raw + size_t(kvh) * HD;
      const uint32_t j = d % HALF;
      const float x0 = k[j], x1 = k[j + HALF];
      kv = rope_rot(x0, x1, cs[j], sn[j], d < HALF);
      vv = a.v_raw[size_t(kvh) * HD + d];
      if (a.kv_f16) {
        const __half kh = __float2half_rn(kv), vh = __float2half_rn(vv);
        reinterpret_cast<__half*>(a.k_cache)[off] = kh;
        reinterpret_cast<__half*>(a.v_cache)[off] = vh;
        kv = __half2float(kh);
        vv = __half2float(vh);
      } else {
        reinterpret_cast<float*>(a.k_cache)[off] = kv;
        reinterpret_cast<float*>(a.v_cache)[off] = vv;
      }
    } else if (a.kv_f16) {
      kv = __half2float(reinterpret_cast<const __half*>(a.k_cache)[off]);
      vv = __half2float(reinterpret_cast<const __half*>(a.v_cache)[off]);
    } else {
      kv = reinterpret_cast<const float*>(a.k_cache)[off];
      vv = reinterpret_cast<const float*>(a.v_cache)[off];
    }
    ks[t][d] = kv;
    vs[t][d] = vv;
  }
  __syncthreads();
  // scores: one (position, head) pair per thread
  for (uint32_t i = tid; i < G * CH; i += nt) {
    const uint32_t g = i / CH, t = i % CH;
    float s = -INFINITY;
    if (t < nv) {
      float dot = 0.0f;
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
    const uint32_t g = i / HD, d = i % HD;
    float acc = 0.0f;
    for (uint32_t t = 0; t < nv; ++t) acc += ps[g][t] * vs[t][d];
    const uint32_t h = kvh * G + g;
    a.part_acc[(size_t(h) * nch + c) * HD + d] = acc;
    if (d == 0) {
      a.part_ml[(size_t(h) * nch + c) * 2] = s_m[g];
      a.part_ml[(size_t(h) * nch + c) * 2 + 1] = s_l[g];
    }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(a.counter + kvh, 1u) == n_act - 1;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  // merge: out = sum_c acc_c * exp(m_c - M) / sum_c l_c * exp(m_c - M)
  for (uint32_t g = wave; g < G; g += nw) {
    const uint32_t h = kvh * G + g;
    float M = -INFINITY;
    for (uint32_t j = lane; j < n_act; j += kWave) M = fmaxf(M, a.part_ml[(size_t(h) * nch + j) * 2]);
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o));
    float L = 0.0f;
    for (uint32_t j = lane; j < n_act; j += kWave)
      L += a.part_ml[(size_t(h) * nch + j) * 2 + 1] * expf(a.part_ml[(size_t(h) * nch + j) * 2] - M);
    L = wave_sum(L);
    const float inv = 1.0f / L;
    for (uint32_t j = lane; j < n_act; j += kWave)
      wts[g * n_act + j] = expf(a.part_ml[(size_t(h) * nch + j) * 2] - M) * inv;
  }
  __syncthreads();
  for (uint32_t i = tid; i < G * HD; i += nt) {
    const uint32_t g = i / HD, d = i % HD, h = kvh * G + g;
    float o = 0.0f;
    for (uint32_t j = 0; j < n_act; ++j) o += a.part_acc[(size_t(h) * nch + j) * HD + d] * wts[g * n_act + j];
    a.out[size_t(h) * HD + d] = o;
  }
  if (tid == 0) a.counter[kvh] = 0u;
}

__global__ void k_advance(AdvanceArgs a) {
  StepState s = *a.state;
  const uint32_t arg = a.result->argmax;
  if (a.out_tokens) a.out_tokens[s.pos] = arg;
  const uint32_t next = s.pos + 1;
  s.token = (a.prompt && next < s.n_prompt) ? a.prompt[next] : arg;
  s.pos = next;
  s.n_steps += 1;
  *a.state = s;
}

// test hooks ---------------------------------------------------------------------------
__global__ void k_flat_tile_weights(const uint8_t* cell, float* out) {
  // dequantisation half of gemvCellFlat (chpe_engine.zig:598-699), materialised
  const Image im{cell, 17408};
  const uint8_t qb = im.u8(16448 + 20);
  const bool g128 = (im.u64(16448 + 24) & 1u) != 0;
  const float scale = im.f32(16448 + 32), bias = im.f32(16448 + 36);
  for (uint32_t i = threadIdx.x; i < 32768; i += blockDim.x) {
    float w = 0.0f;
    if (qb == 4) {
      const float q = float((im.u8(64 + i / 2) >> (4 * (i & 1))) & 15u) - 8.0f;
      w = g128 ? q * h2f(im.u16(16448 + 48 + 2 * (i / 128))) : __fadd_rn(__fmul_rn(q, scale), bias);
    } else if (qb == 2) {
      const float q = codebook_w2((im.u8(64 + i / 4) >> (2 * (i & 3))) & 3u);
      w = g128 ? q * h2f(im.u16(16448 + 48 + 2 * (i / 128))) : __fadd_rn(__fmul_rn(q, scale), bias);
    }
    out[i] = w;
  }
  __syncthreads();
  if (threadIdx.x == 0 && (qb == 4 || qb == 2)) {
    const uint32_t n = im.u16(16448 + 560);
    if (n > 0 && n <= 64)
      for (uint32_t m = 0; m < n; ++m) {
        const uint32_t off = im.u16(16448 + 690 + 2 * m);
        if (off < 32768) out[off] = h2f(im.u16(16448 + 562 + 2 * m));
      }
  }
}

__global__ void k_embed_row_cell(const uint8_t* cell, uint64_t len, uint32_t row, uint32_t D,
                                 float* out, int* written) {
  const Image im{cell, len};
  const bool w = unpack_embed_row_cell(im, 0, row, D, out);
  if (threadIdx.x == 0) *written = w ? 1 : 0;
}

template <int MODE>
void launch_kind(WeightKind kind, const GemvArgs& a, uint32_t n_blocks, uint32_t threads,
                 size_t lds, hipStream_t st) {
  switch (kind) {
    case WeightKind::Cell16W4:
      hipLaunchKernelGGL(k_gemv_cell16_w4<MODE>, dim3(n_blocks), dim3(threads), lds, st, a);
      break;
    case WeightKind::FlatW4:
      hipLaunchKernelGGL((k_gemv_flat<MODE, 4>), dim3(n_blocks), dim3(threads), lds, st, a);
      break;
    case WeightKind::FlatW2:
      hipLaunchKernelGGL((k_gemv_flat<MODE, 2>), dim3(n_blocks), dim3(threads), lds, st, a);
      break;
    case WeightKind::Raw16:
      hipLaunchKernelGGL(k_gemv_raw16<MODE>, dim3(n_blocks), dim3(threads), lds, st, a);
      break;
  }
}

}  // namespace

uint32_t gemv_threads(WeightKind, GemvMode mode) { return mode == GemvMode::SwiGlu ? 512u : 256u; }
uint32_t gemv_rows_per_block(WeightKind) { return 16u; }

size_t gemv_lds_bytes(WeightKind, const GemvArgs& a) {
  return (size_t((a.C + 3) & ~3u) + 64 + 2 * 16 + 16) * sizeof(float);
}

void launch_gemv(WeightKind kind, const GemvArgs& a, uint32_t n_blocks, hipStream_t st) {
  const GemvMode mode = GemvMode(a.mode);
  const uint32_t threads = gemv_threads(kind, mode);
  const size_t lds = gemv_lds_bytes(kind, a);
  switch (mode) {
    case GemvMode::Store: launch_kind<int(GemvMode::Store)>(kind, a, n_blocks, threads, lds, st); break;
    case GemvMode::Accum: launch_kind<int(GemvMode::Accum)>(kind, a, n_blocks, threads, lds, st); break;
    case GemvMode::SwiGlu: launch_kind<int(GemvMode::SwiGlu)>(kind, a, n_blocks, threads, lds, st); break;
    case GemvMode::Logits: launch_kind<int(GemvMode::Logits)>(kind, a, n_blocks, threads, lds, st); break;
  }
}

void launch_embed(const EmbedArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_embed, dim3(1), dim3(256), 0, st, a);
}

void launch_attention(const AttnArgs& a, hipStream_t st) {
  const dim3 grid(a.n_chunks, a.KV);
  if (a.hd == 128) hipLaunchKernelGGL(k_attention<128>, grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL(k_attention<256>, grid, dim3(256), 0, st, a);
}

void launch_advance(const AdvanceArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(k_advance, dim3(1), dim3(1), 0, st, a);
}

void launch_flat_tile_weights(const uint8_t* cell, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_flat_tile_weights, dim3(1), dim3(256), 0, st, cell, out);
}

void launch_embed_row_cell(const uint8_t* cell, uint64_t len, uint32_t row, uint32_t D, float* out,
                           int* written, hipStream_t st) {
  hipLaunchKernelGGL(k_embed_row_cell, dim3(1), dim3(256), 0, st, cell, len, row, D, out, written);
}

}  // namespace chpe
