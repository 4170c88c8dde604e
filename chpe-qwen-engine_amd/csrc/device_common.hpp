// device_common.hpp -- device helpers shared by the gfx950 kernels.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace chpe {

// Launch through the measurement probe when one is armed (see arm_launch_probe), with
// `lds` bytes of dynamic LDS (above 64 KiB the kernel's limit is raised first).
template <class K, class... A>
inline void launch_kernel_lds(K kernel, dim3 grid, dim3 block, size_t lds, hipStream_t st, A... args) {
  if (lds > 65536)
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              int(lds));
  if (detail::g_record_names) {  // (name lookup only: nothing is launched)
    detail::g_last_kernel = hipKernelNameRefByPtr(reinterpret_cast<const void*>(kernel), st);
    return;
  }
  const LaunchProbe p = take_launch_probe();
  if (p.start)
    hipExtLaunchKernelGGL(kernel, grid, block, uint32_t(lds), st, p.start, p.stop, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, uint32_t(lds), st, args...);
}

template <class K, class... A>
inline void launch_kernel(K kernel, dim3 grid, dim3 block, hipStream_t st, A... args) {
  launch_kernel_lds(kernel, grid, block, 0, st, args...);
}

namespace dev {

constexpr int kWave = 64;

__device__ __forceinline__ float h2f(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(uint32_t(h) << 16); }
// Global-memory views.  A load through a generic pointer whose origin the compiler cannot trace
// to global memory becomes a FLAT load, which counts on both the vector-memory and the LDS
// counters; while one is outstanding every wait falls back to "all loads done", so the loads of
// a unit can no longer be consumed as they arrive.  Every device buffer here is global memory.
template <class T>
using gptr = const __attribute__((address_space(1))) T*;
template <class T>
__device__ __forceinline__ gptr<T> as_global(const T* p) {
  return (gptr<T>)(p);
}
template <class T>
__device__ __forceinline__ T gld(const T* p) {
  return *as_global(p);
}
__device__ __forceinline__ uint16_t ld_u16(const uint8_t* p) { return gld(reinterpret_cast<const uint16_t*>(p)); }
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_f4(const float* p) {
  const f32x4_t v = gld(reinterpret_cast<const f32x4_t*>(p));
  return make_float4(v.x, v.y, v.z, v.w);
}
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint2 ld_u64(const uint8_t* p) {
  const u32x2_t v = gld(reinterpret_cast<const u32x2_t*>(p));
  return make_uint2(v.x, v.y);
}
__device__ __forceinline__ uint4 ld_u128(const uint8_t* p) {
  const u32x4_t v = gld(reinterpret_cast<const u32x4_t*>(p));
  return make_uint4(v.x, v.y, v.z, v.w);
}

// ---- cross-lane exchanges on the vector ALU -------------------------------------------------
// DPP (quad_perm, row_half_mirror, row_ror) and gfx950's v_permlane16_swap / v_permlane32_swap
// move values between lanes in a few cycles; ds_bpermute (__shfl_xor) goes through the LDS
// crossbar and costs an LDS round trip per step of a reduction.  Every lane of the wave must
// be active.  pair_val(v, M) returns v of lane ^ M (M = 1, 2, 4, 8, 16, 32), so reductions
// built on it add in the same order as the __shfl_xor butterflies they replace.
template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_u(uint32_t v) {
  return uint32_t(__builtin_amdgcn_update_dpp(0, int(v), CTRL, 0xF, 0xF, false));
}
// quad_perm [1,0,3,2], [2,3,0,1], [3,2,1,0]; row_half_mirror (lane i <-> 7 - i of its 8);
// row_ror:8 (lane i <-> i ^ 8 of its 16)
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppXor3 = 0x1B, kDppHalfMirror = 0x141, kDppRor8 = 0x128;

__device__ __forceinline__ uint32_t pair_u(uint32_t v, int m) {
  switch (m) {
    case 1: return dpp_u<kDppXor1>(v);
    case 2: return dpp_u<kDppXor2>(v);
    case 4: return dpp_u<kDppHalfMirror>(dpp_u<kDppXor3>(v));  // i ^ 3, then ^ 7
    case 8: return dpp_u<kDppRor8>(v);
    case 16: {  // rows 0 <-> 1 and 2 <-> 3 of 16 lanes: [0] = even row's values, [1] = odd row's
      const auto p = __builtin_amdgcn_permlane16_swap(v, v, false, false);
      return (__lane_id() & 16) ? p[0] : p[1];
    }
    default: {  // 32: the two halves of the wave
      const auto p = __builtin_amdgcn_permlane32_swap(v, v, false, false);
      return (__lane_id() & 32) ? p[0] : p[1];
    }
  }
}
__device__ __forceinline__ float pair_val(float v, int m) { return __uint_as_float(pair_u(__float_as_uint(v), m)); }

// v + (v of the partner across bit m); for m = 16 / 32 the swap yields both halves directly
__device__ __forceinline__ float pair_sum(float v, int m) {
  if (m == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  if (m == 32) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
  }
  return v + pair_val(v, m);
}
__device__ __forceinline__ float pair_max(float v, int m) {
  if (m == 16) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
  if (m == 32) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
  }
  return fmaxf(v, pair_val(v, m));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = pair_sum(v, o);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = pair_max(v, o);
  return v;
}

// Reduce N per-lane partials (one per row) over the wave with a reduce-scatter: after the
// call, lane l holds the total of row l / (64/N) in v[0].  N in {4, 8, 16}.
// Both halves are summed with their partner lane and the lane keeps the half it serves; the
// choice is made between the two new sums, so no lane-dependent index into v[] arises.
template <int N>
__device__ __forceinline__ float wave_reduce_rows(float (&v)[N], int lane) {
  int mask = 32;
#pragma unroll
  for (int n = N; n > 1; n >>= 1) {
    const bool up = lane & mask;
#pragma unroll
    for (int j = 0; j < n / 2; ++j) {
      const float lo = pair_sum(v[j], mask);
      const float hi = pair_sum(v[n / 2 + j], mask);
      v[j] = up ? hi : lo;
    }
    mask >>= 1;
  }
  float s = v[0];
#pragma unroll
  for (; mask > 0; mask >>= 1) s = pair_sum(s, mask);
  return s;
}

// fp16 halves of a 32-bit word, widened (the widening folds into v_fma_mix_f32's op_sel)
__device__ __forceinline__ float half_lo(uint32_t w) {
  return float(__builtin_bit_cast(_Float16, static_cast<unsigned short>(w & 0xffffu)));
}
__device__ __forceinline__ float half_hi(uint32_t w) {
  return float(__builtin_bit_cast(_Float16, static_cast<unsigned short>(w >> 16)));
}

// sum over 32 4-bit codes (byte k: low nibble = column 2k, high nibble = column 2k+1) * x.
// A nibble masked in place inside a 16-bit half is an fp16 subnormal: bits 0-3 hold n*2^-24,
// bits 4-7 hold n*2^-20, both exact.  v_fma_mix_f32 widens such a half exactly and fuses the
// multiply-add with the f32 x, so 8 weights cost 4 masks + 1 shift + 8 fused ops; the two
// accumulators are rescaled by 2^24 and 2^20 (exact) at the end.
__device__ __forceinline__ float dot32_w4(uint4 q, const float* x) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t m0 = w[i] & 0x000F000Fu, m1 = w[i] & 0x00F000F0u, w8 = w[i] >> 8;
    const uint32_t m2 = w8 & 0x000F000Fu, m3 = w8 & 0x00F000F0u;
    const float* xi = x + 8 * i;  // columns 8i..8i+7: byte k holds columns 2k, 2k+1
    a = fmaf(half_lo(m0), xi[0], a);
    a = fmaf(half_hi(m0), xi[4], a);
    b = fmaf(half_lo(m1), xi[1], b);
    b = fmaf(half_hi(m1), xi[5], b);
    a = fmaf(half_lo(m2), xi[2], a);
    a = fmaf(half_hi(m2), xi[6], a);
    b = fmaf(half_lo(m3), xi[3], b);
    b = fmaf(half_hi(m3), xi[7], b);
  }
  return a * 16777216.0f + b * 1048576.0f;
}

// sum over 64 2-bit codes of (code ^ 2) * x.  The codebook {0:0, 1:+1, 2:-2, 3:-1}
// (chpe_engine.zig:220) equals (code ^ 2) - 2, so the -2 is applied once per chunk.
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

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// the 4 x 4 byte transpose: w[k] = (a.k, b.k, c.k, d.k)
__device__ __forceinline__ void limb_words(uint32_t a, uint32_t b, uint32_t c, uint32_t d, uint32_t* w) {
  const uint32_t pab = __builtin_amdgcn_perm(b, a, 0x05010400u), qab = __builtin_amdgcn_perm(b, a, 0x07030602u);
  const uint32_t pcd = __builtin_amdgcn_perm(d, c, 0x05010400u), qcd = __builtin_amdgcn_perm(d, c, 0x07030602u);
  w[0] = __builtin_amdgcn_perm(pcd, pab, 0x05040100u);
  w[1] = __builtin_amdgcn_perm(pcd, pab, 0x07060302u);
  w[2] = __builtin_amdgcn_perm(qcd, qab, 0x05040100u);
  w[3] = __builtin_amdgcn_perm(qcd, qab, 0x07060302u);
}

// sum over 16 int8 weights (+128, as unsigned bytes: the sign bit flipped) * x; the caller
// subtracts 128 * sum(x)
__device__ __forceinline__ float dot16_i8p(uint4 q, const float* x) {
  const uint32_t w[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a = fmaf(float(w[i] & 0xffu), x[4 * i], a);
    b = fmaf(float((w[i] >> 8) & 0xffu), x[4 * i + 1], b);
    a = fmaf(float((w[i] >> 16) & 0xffu), x[4 * i + 2], a);
    b = fmaf(float(w[i] >> 24), x[4 * i + 3], b);
  }
  return a + b;
}

__device__ __forceinline__ float dot8_f16(uint4 q, const float* x, bool bf16) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float a = 0.0f, b = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = uint16_t(w[i] & 0xffffu), hi = uint16_t(w[i] >> 16);
    a = fmaf(bf16 ? bf2f(lo) : h2f(lo), x[2 * i], a);
    b = fmaf(bf16 ? bf2f(hi) : h2f(hi), x[2 * i + 1], b);
  }
  return a + b;
}

__device__ __forceinline__ float codebook_w2(uint32_t c) {  // chpe_engine.zig:220
  return c == 0 ? 0.0f : (c == 1 ? 1.0f : (c == 2 ? -2.0f : -1.0f));
}

// (value, index) order of the reference's argmax scan (chpe_engine.zig:1775-1787): the
// greatest value, first index among equals; 0xffffffff marks "no candidate".
__device__ __forceinline__ bool better(float v, uint32_t i, float bv, uint32_t bi) {
  return i != 0xffffffffu && (bi == 0xffffffffu || v > bv || (v == bv && i < bi));
}

// Byte reads of the archive image bounded by its length: some reference reads run past the
// end of a cell into the following records, exactly as here; reads past the image are zero.
struct Image {
  const uint8_t* p;
  uint64_t len;
  __device__ uint8_t u8(uint64_t off) const { return off < len ? p[off] : 0; }
  __device__ uint16_t u16(uint64_t off) const { return uint16_t(u8(off) | (u8(off + 1) << 8)); }
  __device__ uint32_t u32(uint64_t off) const { return u16(off) | (uint32_t(u16(off + 2)) << 16); }
  __device__ uint64_t u64(uint64_t off) const { return u32(off) | (uint64_t(u32(off + 4)) << 32); }
  __device__ float f32(uint64_t off) const { return __uint_as_float(u32(off)); }
};

}  // namespace dev
}  // namespace chpe
