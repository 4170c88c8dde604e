// pack.cpp -- seeded synthetic .chpe archive writer (libchpe_pack.so, chpe_pack CLI).
//
// Writes archives in the reference's on-disk format (src/weight_archive.zig:53-123,
// src/geometry.zig:243-270) laid out by the reference's tensor maps, filling every record
// in parallel straight into an mmap'd file.  The generator, the quantizer and the layout
// rules are specified in include/chpe_pack.h.
//
// Layout rules that follow from how the reference reads an archive:
//  * A 1-D tensor is read as `len` floats from the start of its record's code area
//    (unpackNorm / unpackBias, src/chpe_engine.zig:1144-1192), with no bound at the record.
//    Vectors longer than the 4096 floats of a code area (the 8192-wide q_proj bias of
//    Qwen2.5-72B) therefore continue through the record's payload, the next record's 64-byte
//    header and the first bytes of the next record's code area.  The writer puts the
//    vector's floats in exactly those bytes; the next record (always a flat weight tile in
//    the maps) then has those bytes as its leading codes, and its outliers are chosen among
//    the weights after them.  Gains of 1.0 that wide (the 72B norms) are written as 1.0 in
//    the code area and a NaN first in the payload: unpackNorm resets every gain to 1.0 when
//    one is non-finite (:1161-1166), so they need none of the next record's bytes.
//  * Embedding rows of cell archives are read as 16-row cells (tile = token / 16, row =
//    token % 16, row stride D * bits / 8, src/chpe_engine.zig:1540-1546, :1288-1394).  For
//    D >= 4096 a row runs past its cell, and in the group-128 forms its group scales run past
//    the payload into code bytes of later records, which decode to non-finite scales.  The
//    embedding tiles of these archives are therefore written in the per-tile scale form the
//    reader takes when quant_bits is none of 2/4/8 and the group-128 flag is clear
//    ((nibble - 8) * scale + bias, :1384-1394): every byte a row reaches -- codes, headers and
//    payload tails -- holds 4-bit codes of generated weights.
#include <fcntl.h>
#include <immintrin.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <thread>
#include <vector>

#include "../../include/chpe_pack.h"
#include "format.hpp"
#include "tensor_maps.hpp"

namespace chpe {
namespace {

constexpr float kStd = 0.02f;
constexpr size_t kNone = ~size_t(0);
constexpr size_t kCodeFloats = kTileCodeBytes / 4;                       // 4096
constexpr size_t kSpillFloats = kCodeFloats + (kPayloadBytes + kBytecodeHeader) / 4;  // 4352
constexpr size_t kMaxVecFloats = kSpillFloats + kCodeFloats;             // 8448

inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t tensor_key(uint64_t seed, uint64_t tid) {
  return splitmix64(splitmix64(seed) ^ (tid * 0xD1B54A32D192ED03ull));
}

// ln(u) for u in (0, 1]: u = m 2^e with m in [0.75, 1.5), ln m = 2 atanh(t), t = (m-1)/(m+1)
// (|t| <= 0.2, series to t^11).  Only correctly rounded operations, no library call, so the
// value is the same on every machine and the loops below vectorize.
inline float ln_unit(float u) {
  int32_t b;
  std::memcpy(&b, &u, 4);
  int32_t e = ((b >> 23) & 0xff) - 127;
  const int32_t mb = (b & 0x7fffff) | 0x3f800000;
  float m;
  std::memcpy(&m, &mb, 4);
  const bool big = m >= 1.5f;
  m = big ? m * 0.5f : m;
  e = big ? e + 1 : e;
  const float t = (m - 1.0f) / (m + 1.0f), t2 = t * t;
  const float p = 1.0f + t2 * (1.0f / 3 + t2 * (1.0f / 5 + t2 * (1.0f / 7 + t2 * (1.0f / 9 + t2 * (1.0f / 11)))));
  return float(e) * 0.693147180559945309f + 2.0f * t * p;
}

// sin and cos of 2 pi u for u in [0, 1): the nearest quarter turn, then Taylor polynomials
// on [-pi/4, pi/4] (to x^9 and x^10).
inline void sincos_turn(float u, float* s, float* c) {
  const float turns = 4.0f * u;  // quarter turns, exact
  const float n = std::nearbyint(turns);
  const int32_t q = int32_t(n) & 3;
  const float x = (turns - n) * 1.57079632679489662f, x2 = x * x;
  const float sp = x * (1.0f + x2 * (-1.0f / 6 + x2 * (1.0f / 120 + x2 * (-1.0f / 5040 + x2 * (1.0f / 362880)))));
  const float cp = 1.0f + x2 * (-0.5f + x2 * (1.0f / 24 + x2 * (-1.0f / 720 + x2 * (1.0f / 40320 + x2 * (-1.0f / 3628800)))));
  // quarter turn q: (s, c) = (sp, cp), (cp, -sp), (-sp, -cp), (-cp, sp)
  const bool odd = (q & 1) != 0;
  const float a = odd ? cp : sp, b = odd ? sp : cp;
  *s = (q & 2) ? -a : a;
  *c = ((q + 1) & 2) ? -b : b;
}

// Box-Muller pairs p0 .. p0 + m - 1 of a tensor (m <= 64), in single precision: z[2i] is
// the cosine branch, z[2i + 1] the sine branch.  u1 = (high 24 bits + 1) / 2^24,
// u2 = (low 24 bits) / 2^24, r = sqrt(-2 ln u1).
void normal_pairs(uint64_t key, uint64_t p0, int m, float* z) {
  float u1[64], u2[64];
  for (int i = 0; i < m; ++i) {
    const uint64_t h = splitmix64(key + p0 + uint64_t(i));
    u1[i] = float(uint32_t(h >> 40) + 1u) * (1.0f / 16777216.0f);
    u2[i] = float(uint32_t(h & 0xFFFFFFu)) * (1.0f / 16777216.0f);
  }
  float zc[64], zs[64];
  for (int i = 0; i < m; ++i) {
    const float r = std::sqrt(-2.0f * ln_unit(u1[i]));
    float sn, cs;
    sincos_turn(u2[i], &sn, &cs);
    zc[i] = r * cs;
    zs[i] = r * sn;
  }
  for (int i = 0; i < m; ++i) {
    z[2 * i] = zc[i];
    z[2 * i + 1] = zs[i];
  }
}

// n values of a tensor from element `first`: element e is sd * (pair e/2, branch e%2).
void normals(uint64_t key, uint64_t first, uint64_t n, float sd, float* out) {
  float z[128];
  uint64_t e = first;
  const uint64_t end = first + n;
  while (e < end) {
    const uint64_t p0 = e >> 1, p_end = std::min<uint64_t>((end + 1) >> 1, p0 + 64);
    normal_pairs(key, p0, int(p_end - p0), z);
    const uint64_t hi = std::min(end, 2 * p_end);
    for (uint64_t k = e; k < hi; ++k) *out++ = sd * z[k - 2 * p0];
    e = hi;
  }
}

// The "FP16 weights": generator values rounded to fp16 (nearest even) and widened back.
void fp16_weights(uint64_t key, uint64_t first, uint64_t n, float* out) {
  normals(key, first, n, kStd, out);
  uint64_t i = 0;
  for (; i + 8 <= n; i += 8) {  // F16C conversions: IEEE round-to-nearest-even, exact widening
    const __m128i h = _mm256_cvtps_ph(_mm256_loadu_ps(out + i), _MM_FROUND_TO_NEAREST_INT);
    _mm256_storeu_ps(out + i, _mm256_cvtph_ps(h));
  }
  for (; i < n; ++i) out[i] = f16_to_f32(f32_to_f16(out[i]));
}

inline void put16(uint8_t* p, uint16_t v) { std::memcpy(p, &v, 2); }
inline void put32(uint8_t* p, uint32_t v) { std::memcpy(p, &v, 4); }
inline void putf(uint8_t* p, float v) { std::memcpy(p, &v, 4); }
inline void put64(uint8_t* p, uint64_t v) { std::memcpy(p, &v, 8); }

void write_meta(uint8_t* cell, uint32_t layer, uint8_t bits, uint64_t flags, uint32_t rows,
                uint32_t cols, float scale = 0.0f) {
  uint8_t* pl = cell + kPayloadOff;
  put32(pl + 0, layer);
  put32(pl + 16, bits);  // bit_budget
  pl[kMetaQuantBits] = bits;
  put64(pl + kMetaCustomFlags, flags);
  putf(pl + kDimsScale, scale);
  putf(pl + kDimsBias, 0.0f);
  put32(pl + kDimsRows, rows);
  put32(pl + kDimsCols, cols);
}

// Symmetric quantizer.  4-bit: q = clamp(rint(w/s), -8, 7), code q + 8.  2-bit: codebook
// {0:0, 1:+1, 2:-2, 3:-1} (chpe_engine.zig:220), q = clamp(rint(w/s), -2, 1).
inline uint8_t quant_code(float w, float s, int bits) {
  if (!(s > 0.0f)) return bits == 4 ? 8 : 0;
  const int q = int(std::nearbyint(w / s));
  if (bits == 4) return uint8_t(std::min(7, std::max(-8, q)) + 8);
  static const uint8_t map2[4] = {2, 3, 0, 1};  // -2,-1,0,+1 -> codes
  return map2[std::min(1, std::max(-2, q)) + 2];
}

inline uint16_t group_scale(float absmax, int bits) {
  return f32_to_f16(absmax / (bits == 4 ? 7.0f : 2.0f));
}

inline void set_code(uint8_t* codes, size_t idx, uint8_t c, int bits) {
  if (bits == 4) {
    uint8_t& b = codes[idx >> 1];
    b = (idx & 1) ? uint8_t((b & 0x0F) | (c << 4)) : uint8_t((b & 0xF0) | c);
  } else {
    uint8_t& b = codes[idx >> 2];
    const int sh = int(idx & 3) * 2;
    b = uint8_t((b & ~(3 << sh)) | (c << sh));
  }
}

// 128 weights of one group into 16 * bits code bytes with scale s (outliers take the zero
// code): the quantizer of quant_code, written so that it vectorizes.
void quantize_group(const float* w, const char* is_out, float s, int bits, uint8_t* dst) {
  int8_t q[128];
  const float lo = bits == 4 ? -8.0f : -2.0f, hi = bits == 4 ? 7.0f : 1.0f;
  if (s > 0.0f) {
    for (int j = 0; j < 128; ++j) {
      const float r = std::nearbyint(w[j] / s);
      q[j] = is_out[j] ? int8_t(0) : int8_t(int(std::min(std::max(r, lo), hi)));
    }
  } else {
    std::memset(q, 0, sizeof q);
  }
  if (bits == 4) {  // code = q + 8, low nibble first
    for (int k = 0; k < 64; ++k) dst[k] = uint8_t(((q[2 * k] + 8) & 15) | (((q[2 * k + 1] + 8) & 15) << 4));
  } else {          // code = q & 3 ({0:0, 1:+1, 2:-2, 3:-1}), LSB first
    for (int k = 0; k < 32; ++k)
      dst[k] = uint8_t((q[4 * k] & 3) | ((q[4 * k + 1] & 3) << 2) | ((q[4 * k + 2] & 3) << 4) | ((q[4 * k + 3] & 3) << 6));
  }
}

// The n largest |w[i]| for i in [lo, hi) (ties: lower index first), returned in ascending
// index order: a min-heap of 64-bit keys (|w| bits, then the complemented index).
int top_magnitudes(const float* w, size_t lo, size_t hi, int n, int* idx) {
  if (n <= 0 || hi <= lo) return 0;
  uint64_t heap[64];
  int size = 0;
  auto key = [&](size_t i) {
    uint32_t b;
    std::memcpy(&b, &w[i], 4);
    return (uint64_t(b & 0x7fffffffu) << 32) | uint64_t(0xffffffffu - uint32_t(i));
  };
  auto sift_down = [&](int i) {
    for (;;) {
      int m = i;
      const int l = 2 * i + 1, r = l + 1;
      if (l < size && heap[l] < heap[m]) m = l;
      if (r < size && heap[r] < heap[m]) m = r;
      if (m == i) return;
      std::swap(heap[i], heap[m]);
      i = m;
    }
  };
  for (size_t i = lo; i < hi; ++i) {
    const uint64_t k = key(i);
    if (size < n) {
      int j = size++;
      heap[j] = k;
      while (j > 0 && heap[(j - 1) / 2] > heap[j]) {
        std::swap(heap[j], heap[(j - 1) / 2]);
        j = (j - 1) / 2;
      }
    } else if (k > heap[0]) {
      heap[0] = k;
      sift_down(0);
    }
  }
  for (int m = 0; m < size; ++m) idx[m] = int(0xffffffffu - uint32_t(heap[m]));
  std::sort(idx, idx + size);
  return size;
}

}  // namespace

// rows x cols weights into a 16-row cell (rows <= 16, cols % 128 == 0, rows*cols*bits/8 <= 16384)
int pack_cell16(const float* w, int rows, int cols, int bits, int n_out, uint32_t layer,
                uint8_t* cell) {
  if ((bits != 4 && bits != 2) || rows <= 0 || rows > 16 || cols <= 0 || cols % 128 ||
      size_t(rows) * cols * bits / 8 > kTileCodeBytes || (n_out != 0 && n_out != 8) ||
      rows * (cols / 128) > 256)
    return -1;
  std::memset(cell, 0, kCellBytes);
  write_meta(cell, layer, uint8_t(bits), kFlagGroup128, uint32_t(rows), uint32_t(cols));
  uint8_t* codes = cell + kBytecodeHeader;
  uint8_t* pl = cell + kPayloadOff;
  thread_local std::vector<char> is_out;
  is_out.assign(size_t(cols), 0);
  uint16_t out_cols[8] = {0};
  if (n_out == 8 && rows == 16) {
    // the 8 columns with the largest max |w| over the tile's rows (ties: lower column)
    thread_local std::vector<float> colmax;
    colmax.assign(size_t(cols), 0.0f);
    for (int c = 0; c < cols; ++c) {
      float m = 0.0f;
      for (int r = 0; r < rows; ++r) m = std::max(m, std::fabs(w[size_t(r) * cols + c]));
      colmax[size_t(c)] = m;
    }
    int idx[8];
    top_magnitudes(colmax.data(), 0, size_t(cols), 8, idx);
    for (int k = 0; k < 8; ++k) {
      out_cols[k] = uint16_t(idx[k]);
      is_out[size_t(idx[k])] = 1;
    }
    for (int k = 0; k < 8; ++k) put16(pl + kRowOutlierCols + 2 * k, out_cols[k]);
    for (int r = 0; r < 16; ++r)
      for (int k = 0; k < 8; ++k)
        put16(pl + kRowOutlierW + 2 * (r * 8 + k), f32_to_f16(w[size_t(r) * cols + out_cols[k]]));
  }
  const int gpr = cols / 128;
  for (int r = 0; r < rows; ++r) {
    uint8_t* rc = codes + size_t(r) * cols * bits / 8;
    for (int g = 0; g < gpr; ++g) {
      float amax = 0.0f;
      for (int j = 0; j < 128; ++j) {
        const int c = g * 128 + j;
        if (!is_out[size_t(c)]) amax = std::max(amax, std::fabs(w[size_t(r) * cols + c]));
      }
      const uint16_t sh = group_scale(amax, bits);
      put16(pl + kGroupScales + 2 * (r * gpr + g), sh);
      const float s = f16_to_f32(sh);
      for (int j = 0; j < 128; ++j) {
        const int c = g * 128 + j;
        const uint8_t code = is_out[size_t(c)] ? uint8_t(bits == 4 ? 8 : 0) : quant_code(w[size_t(r) * cols + c], s, bits);
        set_code(rc, size_t(c), code, bits);
      }
    }
  }
  return 0;
}

// 32768 flat weights into a flat tile with up to 64 outliers (largest |w|, ties: lower offset).
// The first `n_fixed` bytes of the code area are given (`fixed`): the weights they cover keep
// those codes, and outliers are chosen among the weights after them.
int pack_flat_fixed(const float* w, int bits, int n_out, uint32_t layer, const uint8_t* fixed,
                    size_t n_fixed, uint8_t* cell) {
  if ((bits != 4 && bits != 2) || n_out < 0 || n_out > 64 || n_fixed > kTileCodeBytes) return -1;
  std::memset(cell, 0, kCellBytes);
  write_meta(cell, layer, uint8_t(bits), kFlagGroup128, 0, 0);
  uint8_t* codes = cell + kBytecodeHeader;
  uint8_t* pl = cell + kPayloadOff;
  const size_t w_fixed = std::min(kFlatWeights, n_fixed * 8 / size_t(bits));
  thread_local std::vector<char> is_out;
  is_out.assign(kFlatWeights, 0);
  int offs[64];
  const int n = top_magnitudes(w, w_fixed, kFlatWeights, n_out, offs);
  if (n > 0) {
    put16(pl + kFlatOutlierN, uint16_t(n));
    for (int m = 0; m < n; ++m) {
      is_out[size_t(offs[m])] = 1;
      put16(pl + kFlatOutlierW + 2 * m, f32_to_f16(w[offs[m]]));
      put16(pl + kFlatOutlierOff + 2 * m, uint16_t(offs[m]));
    }
  }
  for (int g = 0; g < 256; ++g) {
    const float* wg = w + size_t(g) * 128;
    const char* og = is_out.data() + size_t(g) * 128;
    float amax = 0.0f;
    for (int j = 0; j < 128; ++j) amax = std::max(amax, og[j] ? 0.0f : std::fabs(wg[j]));
    const uint16_t sh = group_scale(amax, bits);
    put16(pl + kGroupScales + 2 * g, sh);
    quantize_group(wg, og, f16_to_f32(sh), bits, codes + size_t(g) * 16 * size_t(bits));
  }
  if (n_fixed) std::memcpy(codes, fixed, n_fixed);
  return 0;
}

int pack_flat(const float* w, int bits, int n_out, uint32_t layer, uint8_t* cell) {
  return pack_flat_fixed(w, bits, n_out, layer, nullptr, 0, cell);
}

namespace {

enum class SegKind {
  RawMat,     // raw fp16 / bf16 tiles of a row-major matrix
  RawVec,     // f32 vector in a raw tile
  Cell16,     // 16-row cells of a matrix
  Flat,       // flat 32768-weight tiles of a row-major matrix
  CellVec,    // f32 vector from a cell's code area (spilling into the next record when long)
  EmbedDims,  // embedding tiles in the per-tile scale form (every byte a row reaches is a code)
  Bf16Vec,    // bf16 vector, 8192 values per record's code area
  Zero,       // records no reader reaches (the unused halves of the 9B spans)
};

struct Segment {
  size_t first, count;
  SegKind kind;
  uint64_t tid;
  size_t R, C;         // matrix shape, or vector length (vectors)
  bool ones;           // vectors: 1.0 instead of N(0, sd)
  uint32_t layer;
  float sd = kStd;     // vectors: standard deviation of the generated values
  size_t spill = kNone;  // Flat: index of the vector segment whose tail fills tile 0's first bytes
};

struct Plan {
  size_t records = 0, stride = 0, prefetch = 0;
  uint64_t flags = 0;
  int bits = 0;          // 16 = raw fp16, 17 = raw bf16, else cell quant bits
  std::vector<Segment> segs;
};

// tensor ids of the generator (shared by every archive kind of a model, so a quantized
// archive is the quantization of the fp16 archive with the same seed)
constexpr uint64_t kTidEmbed = 1, kTidLmHead = 2, kTidEmbedExtra = 3;
inline uint64_t tid_of(size_t layer, int which) { return 1000 * (layer + 1) + uint64_t(which); }
enum {
  kQ = 1, kK = 2, kV = 3, kO = 4, kGate = 5, kUp = 6, kDown = 7, kQB = 11, kKB = 12, kVB = 13,
  kQkv = 21, kZ = 22, kA = 23, kB = 24, kConv = 25, kALog = 26, kDtBias = 27, kLinNorm = 28,
  kQNorm = 29, kKNorm = 30,
};

Segment mat(size_t first, size_t count, SegKind k, uint64_t tid, size_t R, size_t C, uint32_t l) {
  return Segment{first, count, k, tid, R, C, false, l};
}
Segment vec(size_t first, SegKind k, uint64_t tid, size_t n, bool ones, uint32_t l, float sd = kStd) {
  Segment s{first, 1, k, tid, n, 0, ones, l};
  s.sd = sd;
  if (k == SegKind::Bf16Vec) s.count = (n + 8191) / 8192;
  return s;
}

// A flat tensor of R x C weights at `first`, `span` records in the map: the tiles it needs,
// then zero records for the rest of the span.
void flat_span(std::vector<Segment>* segs, size_t first, size_t span, uint64_t tid, size_t R, size_t C,
               uint32_t l) {
  const size_t need = (R * C + kFlatWeights - 1) / kFlatWeights;
  segs->push_back(mat(first, std::min(need, span), SegKind::Flat, tid, R, C, l));
  if (span > need) segs->push_back(mat(first + need, span - need, SegKind::Zero, 0, 0, 0, l));
}

bool make_plan(int kind, Plan* p) {
  const size_t D3 = 2048, I3 = 11008, V3 = 151936;
  if (kind == CHPE_PACK_3B_FP16_RAW || kind == CHPE_PACK_3B_BF16_RAW) {
    p->records = kTotalRecords3bRaw;
    p->stride = kTileCodeBytes;
    p->flags = kind == CHPE_PACK_3B_FP16_RAW ? kFlagRawFp16 : 0;
    p->bits = kind == CHPE_PACK_3B_FP16_RAW ? 16 : 17;
    p->segs.push_back(mat(0, 37984, SegKind::RawMat, kTidEmbed, V3, D3, 0));
    for (size_t l = 0; l < 36; ++l) {
      const LayerInfo li = layer_info(MapKind::Qwen3bRaw, l);
      const uint32_t L = uint32_t(l);
      p->segs.push_back(vec(li.input_norm, SegKind::RawVec, 0, D3, true, L));
      p->segs.push_back(mat(li.q_proj, li.q_tiles, SegKind::RawMat, tid_of(l, kQ), 2048, D3, L));
      p->segs.push_back(vec(size_t(li.q_bias), SegKind::RawVec, tid_of(l, kQB), 2048, false, L));
      p->segs.push_back(mat(li.k_proj, li.k_tiles, SegKind::RawMat, tid_of(l, kK), 256, D3, L));
      p->segs.push_back(vec(size_t(li.k_bias), SegKind::RawVec, tid_of(l, kKB), 256, false, L));
      p->segs.push_back(mat(li.v_proj, li.v_tiles, SegKind::RawMat, tid_of(l, kV), 256, D3, L));
      p->segs.push_back(vec(size_t(li.v_bias), SegKind::RawVec, tid_of(l, kVB), 256, false, L));
      p->segs.push_back(mat(li.o_proj, li.o_tiles, SegKind::RawMat, tid_of(l, kO), D3, D3, L));
      p->segs.push_back(vec(li.post_norm, SegKind::RawVec, 0, D3, true, L));
      p->segs.push_back(mat(li.gate_proj, li.gate_tiles, SegKind::RawMat, tid_of(l, kGate), I3, D3, L));
      p->segs.push_back(mat(li.up_proj, li.up_tiles, SegKind::RawMat, tid_of(l, kUp), I3, D3, L));
      p->segs.push_back(mat(li.down_proj, li.down_tiles, SegKind::RawMat, tid_of(l, kDown), D3, I3, L));
    }
    p->segs.push_back(vec(final_norm_record(MapKind::Qwen3bRaw), SegKind::RawVec, 0, D3, true, 36));
  } else if (kind == CHPE_PACK_3B_W4 || kind == CHPE_PACK_3B_W2 || kind == CHPE_PACK_3B_W4_STD) {
    p->records = kTotalRecords3bCell;
    p->stride = kind == CHPE_PACK_3B_W4_STD ? kRecordBytes : kCellBytes;
    p->prefetch = kind == CHPE_PACK_3B_W4_STD ? kPrefetchBytes : 0;
    p->flags = kFlagGroup128;
    p->bits = kind == CHPE_PACK_3B_W2 ? 2 : 4;
    p->segs.push_back(mat(0, 9496, SegKind::Cell16, kTidEmbed, V3, D3, 0));
    for (size_t l = 0; l < 36; ++l) {
      const LayerInfo li = layer_info(MapKind::Qwen3bCell, l);
      const uint32_t L = uint32_t(l);
      p->segs.push_back(vec(li.input_norm, SegKind::CellVec, 0, D3, true, L));
      p->segs.push_back(mat(li.down_proj, li.down_tiles, SegKind::Flat, tid_of(l, kDown), D3, I3, L));
      p->segs.push_back(mat(li.gate_proj, li.gate_tiles, SegKind::Cell16, tid_of(l, kGate), I3, D3, L));
      p->segs.push_back(mat(li.up_proj, li.up_tiles, SegKind::Cell16, tid_of(l, kUp), I3, D3, L));
      p->segs.push_back(vec(li.post_norm, SegKind::CellVec, 0, D3, true, L));
      p->segs.push_back(vec(size_t(li.k_bias), SegKind::CellVec, tid_of(l, kKB), 256, false, L));
      p->segs.push_back(mat(li.k_proj, li.k_tiles, SegKind::Cell16, tid_of(l, kK), 256, D3, L));
      p->segs.push_back(mat(li.o_proj, li.o_tiles, SegKind::Cell16, tid_of(l, kO), D3, D3, L));
      p->segs.push_back(vec(size_t(li.q_bias), SegKind::CellVec, tid_of(l, kQB), 2048, false, L));
      p->segs.push_back(mat(li.q_proj, li.q_tiles, SegKind::Cell16, tid_of(l, kQ), 2048, D3, L));
      p->segs.push_back(vec(size_t(li.v_bias), SegKind::CellVec, tid_of(l, kVB), 256, false, L));
      p->segs.push_back(mat(li.v_proj, li.v_tiles, SegKind::Cell16, tid_of(l, kV), 256, D3, L));
    }
    p->segs.push_back(vec(final_norm_record(MapKind::Qwen3bCell), SegKind::CellVec, 0, D3, true, 36));
  } else if (kind == CHPE_PACK_72B_W4 || kind == CHPE_PACK_72B_W2) {
    const size_t D = 8192, I = 29568, V = 152064, KVD = 1024;
    p->records = kTotalRecords72b;
    p->stride = kCellBytes;
    p->flags = kFlagGroup128;
    p->bits = kind == CHPE_PACK_72B_W4 ? 4 : 2;
    p->segs.push_back(mat(0, 38016, SegKind::EmbedDims, kTidEmbed, V, D, 0));
    for (size_t l = 0; l < 80; ++l) {
      const LayerInfo li = layer_info(MapKind::Qwen72b, l);
      const uint32_t L = uint32_t(l);
      p->segs.push_back(vec(li.input_norm, SegKind::CellVec, 0, D, true, L));
      p->segs.push_back(mat(li.q_proj, li.q_tiles, SegKind::Flat, tid_of(l, kQ), D, D, L));
      p->segs.push_back(vec(size_t(li.q_bias), SegKind::CellVec, tid_of(l, kQB), D, false, L));
      p->segs.push_back(mat(li.k_proj, li.k_tiles, SegKind::Flat, tid_of(l, kK), KVD, D, L));
      p->segs.push_back(vec(size_t(li.k_bias), SegKind::CellVec, tid_of(l, kKB), KVD, false, L));
      p->segs.push_back(mat(li.v_proj, li.v_tiles, SegKind::Flat, tid_of(l, kV), KVD, D, L));
      p->segs.push_back(vec(size_t(li.v_bias), SegKind::CellVec, tid_of(l, kVB), KVD, false, L));
      p->segs.push_back(mat(li.o_proj, li.o_tiles, SegKind::Flat, tid_of(l, kO), D, D, L));
      p->segs.push_back(vec(li.post_norm, SegKind::CellVec, 0, D, true, L));
      p->segs.push_back(mat(li.gate_proj, li.gate_tiles, SegKind::Flat, tid_of(l, kGate), I, D, L));
      p->segs.push_back(mat(li.up_proj, li.up_tiles, SegKind::Flat, tid_of(l, kUp), I, D, L));
      p->segs.push_back(mat(li.down_proj, li.down_tiles, SegKind::Flat, tid_of(l, kDown), D, I, L));
    }
    p->segs.push_back(vec(final_norm_record(MapKind::Qwen72b), SegKind::CellVec, 0, D, true, 80));
    size_t lm, lmt;
    lm_head_record(D, &lm, &lmt);
    p->segs.push_back(mat(lm, lmt, SegKind::Flat, kTidLmHead, V, D, 80));
  } else if (kind == CHPE_PACK_9B_W4) {
    // Qwen3.5-9B: the real tensors (qwen35_tensor_map.zig:7-50 names them) as 4-bit flat
    // tiles at the front of each INT8-map span; a span's remaining records are zero.
    const size_t D = 4096, I = 12288, V = 248320, KVD = 4 * 256, QG = 2 * 16 * 256;
    p->records = kTotalRecords9b;
    p->stride = kCellBytes;
    p->flags = kFlagGroup128;
    p->bits = 4;
    const size_t emb_tiles = V * D / kFlatWeights;  // 31040 of the 62080-record span
    p->segs.push_back(mat(0, emb_tiles, SegKind::EmbedDims, kTidEmbed, V, D, 0));
    p->segs.push_back(mat(emb_tiles, 62080 - emb_tiles, SegKind::Zero, 0, 0, 0, 0));
    for (size_t l = 0; l < 32; ++l) {
      const Qwen35Records m = qwen35_records(l);
      const uint32_t L = uint32_t(l);
      std::vector<Segment>& S = p->segs;
      S.push_back(vec(m.input_norm, SegKind::CellVec, 0, D, true, L));
      if (m.full_attn) {
        flat_span(&S, m.q_proj, 2048, tid_of(l, kQ), QG, D, L);  // query and output gate rows
        flat_span(&S, m.k_proj, 256, tid_of(l, kK), KVD, D, L);
        flat_span(&S, m.v_proj, 256, tid_of(l, kV), KVD, D, L);
        flat_span(&S, m.o_proj, 1024, tid_of(l, kO), D, 16 * 256, L);
        S.push_back(vec(m.q_norm, SegKind::Bf16Vec, tid_of(l, kQNorm), 256, true, L));
        S.push_back(vec(m.k_norm, SegKind::Bf16Vec, tid_of(l, kKNorm), 256, true, L));
      } else {
        flat_span(&S, m.in_proj_qkv, 2048, tid_of(l, kQkv), 2 * 2048 + 4096, D, L);
        flat_span(&S, m.in_proj_z, 1024, tid_of(l, kZ), 4096, D, L);
        flat_span(&S, m.in_proj_a, 8, tid_of(l, kA), 32, D, L);
        flat_span(&S, m.in_proj_b, 8, tid_of(l, kB), 32, D, L);
        S.push_back(vec(m.conv1d, SegKind::Bf16Vec, tid_of(l, kConv), 8192 * 4, false, L));
        S.push_back(vec(m.a_log, SegKind::Bf16Vec, tid_of(l, kALog), 32, false, L, 0.1f));
        S.push_back(vec(m.dt_bias, SegKind::Bf16Vec, tid_of(l, kDtBias), 32, false, L, 0.1f));
        S.push_back(vec(m.linear_norm, SegKind::Bf16Vec, tid_of(l, kLinNorm), 128, true, L));
        flat_span(&S, m.out_proj, 1024, tid_of(l, kO), D, 4096, L);
      }
      S.push_back(vec(m.post_norm, SegKind::CellVec, 0, D, true, L));
      flat_span(&S, m.gate_proj, 3072, tid_of(l, kGate), I, D, L);
      flat_span(&S, m.up_proj, 3072, tid_of(l, kUp), I, D, L);
      flat_span(&S, m.down_proj, 3072, tid_of(l, kDown), D, I, L);
    }
    p->segs.push_back(vec(final_norm_record(MapKind::Qwen35_9b), SegKind::CellVec, 0, D, true, 32));
    size_t lm, lmt;
    lm_head_record(D, &lm, &lmt);
    flat_span(&p->segs, lm, lmt, kTidLmHead, V, D, 32);
  } else {
    return false;
  }
  std::sort(p->segs.begin(), p->segs.end(),
            [](const Segment& a, const Segment& b) { return a.first < b.first; });
  size_t next = 0;
  for (size_t i = 0; i < p->segs.size(); ++i) {
    const Segment& s = p->segs[i];
    if (s.first != next) return false;  // the map must tile [0, records) exactly
    next += s.count;
    if (s.kind == SegKind::CellVec && s.R > kCodeFloats && !s.ones) {  // a long vector: its tail fills the next tile
      if (s.R > kMaxVecFloats || i + 1 >= p->segs.size() || p->segs[i + 1].kind != SegKind::Flat) return false;
      p->segs[i + 1].spill = i;
    }
  }
  return next == p->records;
}

// The generated values of a vector segment.
void vector_values(const Segment& s, uint64_t seed, std::vector<float>* v) {
  v->resize(s.R);
  if (s.ones) std::fill(v->begin(), v->end(), 1.0f);
  else normals(tensor_key(seed, s.tid), 0, s.R, s.sd, v->data());
}

// Fill record `t` of segment `s`.  `out` points at the record's code area for raw archives
// and at the cell for cell archives.
void fill_record(const Plan& p, const Segment& s, size_t t, uint64_t seed, uint8_t* out,
                 std::vector<float>& buf) {
  const uint64_t key = tensor_key(seed, s.tid);
  switch (s.kind) {
    case SegKind::Zero:
      break;
    case SegKind::RawMat: {
      const size_t per = kTileCodeBytes / 2, total = s.R * s.C;
      const size_t e0 = t * per, n = e0 < total ? std::min(per, total - e0) : 0;
      buf.resize(per);
      normals(key, e0, n, kStd, buf.data());
      for (size_t i = 0; i < n; ++i)
        put16(out + 2 * i, p.bits == 16 ? f32_to_f16(buf[i]) : f32_to_bf16(buf[i]));
      break;
    }
    case SegKind::RawVec: {
      const size_t n = std::min(s.R, kCodeFloats);
      vector_values(s, seed, &buf);
      for (size_t i = 0; i < n; ++i) putf(out + 4 * i, buf[i]);
      break;
    }
    case SegKind::CellVec: {
      vector_values(s, seed, &buf);
      if (s.R <= kCodeFloats) {
        write_meta(out, s.layer, 32, 0, 1, uint32_t(s.R));
        std::memcpy(out + kBytecodeHeader, buf.data(), 4 * s.R);
      } else if (s.ones) {
        // gains of 1.0 wider than the code area: 1.0 in the code area and a NaN first in the
        // payload, which unpackNorm's non-finite rule (:1161-1166) turns into gains of 1.0 for
        // every element, so the next record keeps its own codes
        std::memcpy(out + kBytecodeHeader, buf.data(), kTileCodeBytes);
        std::vector<float> pl(kPayloadBytes / 4, 1.0f);
        pl[0] = std::numeric_limits<float>::quiet_NaN();
        std::memcpy(out + kPayloadOff, pl.data(), kPayloadBytes);
      } else {  // the code area, then the payload (the rest goes into the next record)
        std::memcpy(out + kBytecodeHeader, buf.data(), kTileCodeBytes);
        std::memcpy(out + kPayloadOff, buf.data() + kCodeFloats, kPayloadBytes);
      }
      break;
    }
    case SegKind::Bf16Vec: {
      const size_t i0 = t * 8192, n = i0 < s.R ? std::min<size_t>(8192, s.R - i0) : 0;
      vector_values(s, seed, &buf);
      for (size_t i = 0; i < n; ++i) put16(out + kBytecodeHeader + 2 * i, f32_to_bf16(buf[i0 + i]));
      break;
    }
    case SegKind::Cell16: {
      const size_t r0 = t * 16, rows = r0 < s.R ? std::min<size_t>(16, s.R - r0) : 0;
      if (!rows) break;
      buf.resize(rows * s.C);
      fp16_weights(key, r0 * s.C, rows * s.C, buf.data());
      pack_cell16(buf.data(), int(rows), int(s.C), p.bits, 8, s.layer, out);
      break;
    }
    case SegKind::Flat: {
      const size_t total = s.R * s.C, e0 = t * kFlatWeights;
      buf.assign(kFlatWeights, 0.0f);
      if (e0 < total) fp16_weights(key, e0, std::min(kFlatWeights, total - e0), buf.data());
      if (t == 0 && s.spill != kNone) {
        const Segment& v = p.segs[s.spill];
        std::vector<float> vals;
        vector_values(v, seed, &vals);
        const uint8_t* vb = reinterpret_cast<const uint8_t*>(vals.data());
        const size_t n_fixed = 4 * (v.R - kSpillFloats);
        pack_flat_fixed(buf.data(), p.bits, 64, s.layer, vb + 4 * kSpillFloats, n_fixed, out);
        std::memcpy(out, vb + 4 * (kCodeFloats + kPayloadBytes / 4), kBytecodeHeader);  // the header
      } else {
        pack_flat(buf.data(), p.bits, 64, s.layer, out);
      }
      break;
    }
    case SegKind::EmbedDims: {
      // 32768 weights of the flat embedding matrix in the code area plus 1952 more for the
      // header (128) and the payload after its metadata and dims (1824), one f32 scale
      constexpr size_t kExtra = 2 * (kBytecodeHeader + kPayloadBytes - 48);
      const size_t total = s.R * s.C, e0 = t * kFlatWeights;
      buf.assign(kFlatWeights + kExtra, 0.0f);
      if (e0 < total) fp16_weights(key, e0, std::min(kFlatWeights, total - e0), buf.data());
      fp16_weights(tensor_key(seed, kTidEmbedExtra), t * kExtra, kExtra, buf.data() + kFlatWeights);
      float amax = 0.0f;
      for (float x : buf) amax = std::max(amax, std::fabs(x));
      const float sc = amax / 7.0f;
      std::memset(out, 0, kCellBytes);
      auto codes_at = [&](uint8_t* dst, const float* w, size_t n) {
        for (size_t i = 0; i < n; ++i) set_code(dst, i, quant_code(w[i], sc, 4), 4);
      };
      codes_at(out + kBytecodeHeader, buf.data(), kFlatWeights);
      codes_at(out, buf.data() + kFlatWeights, 2 * kBytecodeHeader);
      write_meta(out, s.layer, 0, 0, 0, 0, sc);
      put32(out + kPayloadOff + 16, 4);  // bit_budget
      codes_at(out + kPayloadOff + 48, buf.data() + kFlatWeights + 2 * kBytecodeHeader, 2 * (kPayloadBytes - 48));
      break;
    }
  }
}

void write_header(const Plan& p, uint8_t* base) {
  ArchiveHeader h{};
  h.magic = kChpeMagic;
  h.version = kArchiveVersion;
  h.header_bytes = kHeaderBytes;
  h.record_count = p.records;
  h.tile_count = p.records;
  h.record_bytes = p.stride;
  h.cell_bytes = p.stride == kTileCodeBytes ? kTileCodeBytes : kCellBytes;
  h.prefetch_bytes = p.prefetch;
  h.flags = p.flags;
  std::memset(base, 0, kHeaderBytes);
  std::memcpy(base, &h, sizeof h);
}

// Fill records [r_begin, r_end) into `dst` (record r at dst + (r - r_begin) * stride) with
// `threads` workers.
void fill_range(const Plan& p, uint64_t seed, size_t r_begin, size_t r_end, uint8_t* dst, unsigned nt,
                const char* progress_name) {
  std::vector<uint32_t> seg_of(r_end - r_begin);
  for (size_t i = 0; i < p.segs.size(); ++i) {
    const Segment& s = p.segs[i];
    const size_t a = std::max(s.first, r_begin), b = std::min(s.first + s.count, r_end);
    for (size_t r = a; r < b; ++r) seg_of[r - r_begin] = uint32_t(i);
  }
  std::atomic<size_t> next{r_begin};
  const size_t chunk = 64, n = r_end - r_begin;
  const size_t step = std::max<size_t>(chunk, n / 16 / chunk * chunk);
  auto worker = [&]() {
    std::vector<float> buf;
    for (;;) {
      const size_t r0 = next.fetch_add(chunk);
      if (r0 >= r_end) break;
      if (progress_name && (r0 - r_begin) % step == 0)
        std::fprintf(stderr, "chpe_pack: %s record %zu of %zu\n", progress_name, r0, p.records);
      for (size_t r = r0; r < std::min(r_end, r0 + chunk); ++r) {
        const Segment& s = p.segs[seg_of[r - r_begin]];
        uint8_t* rec = dst + (r - r_begin) * p.stride;
        uint8_t* out = p.stride == kTileCodeBytes ? rec : rec + p.prefetch;
        fill_record(p, s, r - s.first, seed, out, buf);
      }
    }
  };
  nt = std::max(1u, std::min<unsigned>(nt, unsigned((n + chunk - 1) / chunk)));
  std::vector<std::thread> pool;
  for (unsigned i = 0; i < nt; ++i) pool.emplace_back(worker);
  for (auto& th : pool) th.join();
}

unsigned thread_count(int threads) {
  return threads > 0 ? unsigned(threads) : std::max(1u, std::thread::hardware_concurrency());
}

}  // namespace
}  // namespace chpe

using namespace chpe;

extern "C" uint64_t chpe_pack_size(int kind) {
  Plan p;
  if (!make_plan(kind, &p)) return 0;
  return kHeaderBytes + uint64_t(p.records) * p.stride;
}

extern "C" int chpe_pack_write(const char* path, int kind, uint64_t seed, int threads) {
  Plan p;
  if (!make_plan(kind, &p)) return -1;
  const uint64_t size = kHeaderBytes + uint64_t(p.records) * p.stride;
  const int fd = ::open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) return -2;
  if (::ftruncate(fd, off_t(size)) != 0) { ::close(fd); return -2; }
  void* m = ::mmap(nullptr, size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return -2;
  uint8_t* base = static_cast<uint8_t*>(m);
  write_header(p, base);
  // CHPE_PACK_PROGRESS set: a line on stderr each time another sixteenth of the records is
  // claimed (large archives take a minute or more to write)
  fill_range(p, seed, 0, p.records, base + kHeaderBytes, thread_count(threads),
             std::getenv("CHPE_PACK_PROGRESS") ? path : nullptr);
  ::munmap(m, size);
  return 0;
}

extern "C" int chpe_pack_records(int kind, uint64_t seed, uint64_t first, uint64_t count, int threads,
                                 uint8_t* out) {
  Plan p;
  if (!make_plan(kind, &p) || !out || first > p.records || count > p.records - first) return -1;
  if (count) fill_range(p, seed, size_t(first), size_t(first + count), out, thread_count(threads), nullptr);
  return 0;
}

extern "C" int chpe_pack_header(int kind, uint8_t* out) {
  Plan p;
  if (!make_plan(kind, &p) || !out) return -1;
  write_header(p, out);
  return 0;
}

extern "C" void chpe_pack_normals(uint64_t seed, uint64_t tid, uint64_t first, uint64_t n,
                                  float std_dev, float* out) {
  normals(tensor_key(seed, tid), first, n, std_dev, out);
}

extern "C" int chpe_pack_cell16(const float* w, int rows, int cols, int bits, int n_outlier_cols,
                                uint32_t layer, uint8_t* cell) {
  return pack_cell16(w, rows, cols, bits, n_outlier_cols, layer, cell);
}

extern "C" int chpe_pack_flat(const float* w, int bits, int n_outliers, uint32_t layer,
                              uint8_t* cell) {
  return pack_flat(w, bits, n_outliers, layer, cell);
}
