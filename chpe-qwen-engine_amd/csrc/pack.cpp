// pack.cpp -- seeded synthetic .chpe archive writer (libchpe_pack.so, chpe_pack CLI).
//
// Writes archives in the reference's on-disk format (src/weight_archive.zig:53-123,
// src/geometry.zig:243-270) laid out by the reference's tensor maps, filling every record
// in parallel straight into an mmap'd file.  The generator and quantizer are specified in
// include/chpe_pack.h.
#include <fcntl.h>
#include <sys/mman.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../include/chpe_pack.h"
#include "format.hpp"
#include "tensor_maps.hpp"

namespace chpe {
namespace {

constexpr float kStd = 0.02f;

inline uint64_t splitmix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

inline uint64_t tensor_key(uint64_t seed, uint64_t tid) {
  return splitmix64(splitmix64(seed) ^ (tid * 0xD1B54A32D192ED03ull));
}

// Box-Muller pair p of a tensor: elements 2p (cos) and 2p+1 (sin).
inline void normal_pair(uint64_t key, uint64_t p, double* z0, double* z1) {
  uint64_t h = splitmix64(key + p);
  double u1 = double((h >> 40) + 1) * (1.0 / 16777216.0);  // (0, 1]
  double u2 = double(h & 0xFFFFFFu) * (1.0 / 16777216.0);  // [0, 1)
  double r = std::sqrt(-2.0 * std::log(u1)), th = 6.283185307179586 * u2;
  *z0 = r * std::cos(th);
  *z1 = r * std::sin(th);
}

void normals(uint64_t key, uint64_t first, uint64_t n, float sd, float* out) {
  uint64_t e = first, end = first + n;
  double z0, z1;
  if (e < end && (e & 1)) {
    normal_pair(key, e >> 1, &z0, &z1);
    *out++ = float(sd * z1);
    ++e;
  }
  for (; e + 1 < end; e += 2) {
    normal_pair(key, e >> 1, &z0, &z1);
    *out++ = float(sd * z0);
    *out++ = float(sd * z1);
  }
  if (e < end) {
    normal_pair(key, e >> 1, &z0, &z1);
    *out++ = float(sd * z0);
  }
}

// The "FP16 weights": generator values rounded to fp16 and widened back.
void fp16_weights(uint64_t key, uint64_t first, uint64_t n, float* out) {
  normals(key, first, n, kStd, out);
  for (uint64_t i = 0; i < n; ++i) out[i] = f16_to_f32(f32_to_f16(out[i]));
}

inline void put16(uint8_t* p, uint16_t v) { std::memcpy(p, &v, 2); }
inline void put32(uint8_t* p, uint32_t v) { std::memcpy(p, &v, 4); }
inline void putf(uint8_t* p, float v) { std::memcpy(p, &v, 4); }
inline void put64(uint8_t* p, uint64_t v) { std::memcpy(p, &v, 8); }

void write_meta(uint8_t* cell, uint32_t layer, uint8_t bits, uint64_t flags, uint32_t rows,
                uint32_t cols) {
  uint8_t* pl = cell + kPayloadOff;
  put32(pl + 0, layer);
  put32(pl + 16, bits);  // bit_budget
  pl[kMetaQuantBits] = bits;
  put64(pl + kMetaCustomFlags, flags);
  putf(pl + kDimsScale, 0.0f);
  putf(pl + kDimsBias, 0.0f);
  put32(pl + kDimsRows, rows);
  put32(pl + kDimsCols, cols);
}

// symmetric group quantizer.  4-bit: q = clamp(rint(w/s), -8, 7), code q+8, s = absmax/7.
// 2-bit: codebook {0:0, 1:+1, 2:-2, 3:-1} (chpe_engine.zig:220), s = absmax/2.
inline uint8_t quant_code(float w, float s, int bits) {
  if (!(s > 0.0f)) return bits == 4 ? 8 : 0;
  int q = int(std::lrint(w / s));
  if (bits == 4) return uint8_t(std::min(7, std::max(-8, q)) + 8);
  q = std::min(1, std::max(-2, q));
  static const uint8_t map2[4] = {2, 3, 0, 1};  // -2,-1,0,+1 -> codes
  return map2[q + 2];
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
    int sh = int(idx & 3) * 2;
    b = uint8_t((b & ~(3 << sh)) | (c << sh));
  }
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
  std::vector<char> is_out(cols, 0);
  uint16_t out_cols[8] = {0};
  if (n_out == 8 && rows == 16) {
    // the 8 columns with the largest max |w| over the tile's rows (ties: lower column)
    std::vector<std::pair<float, int>> colmax(cols);
    for (int c = 0; c < cols; ++c) {
      float m = 0.0f;
      for (int r = 0; r < rows; ++r) m = std::max(m, std::fabs(w[size_t(r) * cols + c]));
      colmax[c] = {-m, c};
    }
    std::partial_sort(colmax.begin(), colmax.begin() + 8, colmax.end());
    for (int k = 0; k < 8; ++k) {
      out_cols[k] = uint16_t(colmax[k].second);
      is_out[out_cols[k]] = 1;
    }
    std::sort(out_cols, out_cols + 8);
    for (int k = 0; k < 8; ++k) put16(pl + kRowOutlierCols + 2 * k, out_cols[k]);
    for (int r = 0; r < 16; ++r)
      for (int k = 0; k < 8; ++k)
        put16(pl + kRowOutlierW + 2 * (r * 8 + k), f32_to_f16(w[size_t(r) * cols + out_cols[k]]));
  }
  int gpr = cols / 128;
  for (int r = 0; r < rows; ++r) {
    uint8_t* rc = codes + size_t(r) * cols * bits / 8;
    for (int g = 0; g < gpr; ++g) {
      float amax = 0.0f;
      for (int j = 0; j < 128; ++j) {
        int c = g * 128 + j;
        if (!is_out[c]) amax = std::max(amax, std::fabs(w[size_t(r) * cols + c]));
      }
      uint16_t sh = group_scale(amax, bits);
      put16(pl + kGroupScales + 2 * (r * gpr + g), sh);
      float s = f16_to_f32(sh);
      for (int j = 0; j < 128; ++j) {
        int c = g * 128 + j;
        uint8_t code = is_out[c] ? uint8_t(bits == 4 ? 8 : 0) : quant_code(w[size_t(r) * cols + c], s, bits);
        set_code(rc, size_t(c), code, bits);
      }
    }
  }
  return 0;
}

// 32768 flat weights into a flat tile with up to 64 outliers (largest |w|, ties: lower offset)
int pack_flat(const float* w, int bits, int n_out, uint32_t layer, uint8_t* cell) {
  if ((bits != 4 && bits != 2) || n_out < 0 || n_out > 64) return -1;
  std::memset(cell, 0, kCellBytes);
  write_meta(cell, layer, uint8_t(bits), kFlagGroup128, 0, 0);
  uint8_t* codes = cell + kBytecodeHeader;
  uint8_t* pl = cell + kPayloadOff;
  std::vector<char> is_out(kFlatWeights, 0);
  if (n_out > 0) {
    std::vector<std::pair<float, int>> mag(kFlatWeights);
    for (size_t i = 0; i < kFlatWeights; ++i) mag[i] = {-std::fabs(w[i]), int(i)};
    std::partial_sort(mag.begin(), mag.begin() + n_out, mag.end());
    std::vector<int> offs(n_out);
    for (int m = 0; m < n_out; ++m) offs[m] = mag[m].second;
    std::sort(offs.begin(), offs.end());
    put16(pl + kFlatOutlierN, uint16_t(n_out));
    for (int m = 0; m < n_out; ++m) {
      is_out[offs[m]] = 1;
      put16(pl + kFlatOutlierW + 2 * m, f32_to_f16(w[offs[m]]));
      put16(pl + kFlatOutlierOff + 2 * m, uint16_t(offs[m]));
    }
  }
  for (int g = 0; g < 256; ++g) {
    float amax = 0.0f;
    for (int j = 0; j < 128; ++j)
      if (!is_out[g * 128 + j]) amax = std::max(amax, std::fabs(w[g * 128 + j]));
    uint16_t sh = group_scale(amax, bits);
    put16(pl + kGroupScales + 2 * g, sh);
    float s = f16_to_f32(sh);
    for (int j = 0; j < 128; ++j) {
      size_t i = size_t(g) * 128 + j;
      set_code(codes, i, is_out[i] ? uint8_t(bits == 4 ? 8 : 0) : quant_code(w[i], s, bits), bits);
    }
  }
  return 0;
}

namespace {

enum class SegKind { RawMat, RawVec, Cell16, Flat, CellVec };

struct Segment {
  size_t first, count;
  SegKind kind;
  uint64_t tid;
  size_t R, C;     // matrix shape (RawMat / Cell16 / Flat) or vector length (vectors)
  bool ones;       // vectors: gains of 1.0 instead of N(0, 0.02)
  uint32_t layer;
};

struct Plan {
  size_t records = 0, stride = 0, prefetch = 0;
  uint64_t flags = 0;
  int bits = 0;          // 16 = raw fp16, 17 = raw bf16, else cell quant bits
  std::vector<Segment> segs;
};

// tensor ids of the generator (shared by every archive kind, so a quantized archive is
// the quantization of the fp16 archive with the same seed)
constexpr uint64_t kTidEmbed = 1, kTidLmHead = 2;
inline uint64_t tid_of(size_t layer, int which) { return 1000 * (layer + 1) + uint64_t(which); }
enum { kQ = 1, kK = 2, kV = 3, kO = 4, kGate = 5, kUp = 6, kDown = 7, kQB = 11, kKB = 12, kVB = 13 };

bool make_plan(int kind, Plan* p) {
  const size_t D3 = 2048, I3 = 11008, V3 = 151936;
  auto mat = [](size_t first, size_t count, SegKind k, uint64_t tid, size_t R, size_t C, uint32_t l) {
    return Segment{first, count, k, tid, R, C, false, l};
  };
  auto vec = [](size_t first, SegKind k, uint64_t tid, size_t n, bool ones, uint32_t l) {
    return Segment{first, 1, k, tid, n, 0, ones, l};
  };
  if (kind == CHPE_PACK_3B_FP16_RAW || kind == CHPE_PACK_3B_BF16_RAW) {
    p->records = kTotalRecords3bRaw;
    p->stride = kTileCodeBytes;
    p->flags = kind == CHPE_PACK_3B_FP16_RAW ? kFlagRawFp16 : 0;
    p->bits = kind == CHPE_PACK_3B_FP16_RAW ? 16 : 17;
    p->segs.push_back(mat(0, 37984, SegKind::RawMat, kTidEmbed, V3, D3, 0));
    for (size_t l = 0; l < 36; ++l) {
      LayerInfo li = layer_info(MapKind::Qwen3bRaw, l);
      uint32_t L = uint32_t(l);
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
      LayerInfo li = layer_info(MapKind::Qwen3bCell, l);
      uint32_t L = uint32_t(l);
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
    p->segs.push_back(mat(0, 38016, SegKind::Flat, kTidEmbed, V, D, 0));
    for (size_t l = 0; l < 80; ++l) {
      LayerInfo li = layer_info(MapKind::Qwen72b, l);
      uint32_t L = uint32_t(l);
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
  } else {
    return false;
  }
  std::sort(p->segs.begin(), p->segs.end(),
            [](const Segment& a, const Segment& b) { return a.first < b.first; });
  size_t next = 0;
  for (const Segment& s : p->segs) {
    if (s.first != next) return false;  // the map must tile [0, records) exactly
    next += s.count;
  }
  return next == p->records;
}

// Fill record `rec` (tile t of segment s).  `out` points at the record's code area for raw
// archives and at the cell for cell archives.
void fill_record(const Plan& p, const Segment& s, size_t t, uint64_t seed, uint8_t* out,
                 std::vector<float>& buf) {
  const uint64_t key = tensor_key(seed, s.tid);
  switch (s.kind) {
    case SegKind::RawMat: {
      const size_t per = kTileCodeBytes / 2, total = s.R * s.C;
      size_t e0 = t * per, n = e0 < total ? std::min(per, total - e0) : 0;
      buf.resize(per);
      normals(key, e0, n, kStd, buf.data());
      for (size_t i = 0; i < n; ++i)
        put16(out + 2 * i, p.bits == 16 ? f32_to_f16(buf[i]) : f32_to_bf16(buf[i]));
      break;
    }
    case SegKind::RawVec:
    case SegKind::CellVec: {
      uint8_t* dst = out;
      if (s.kind == SegKind::CellVec) {
        write_meta(out, s.layer, 32, 0, 1, uint32_t(s.R));
        dst = out + kBytecodeHeader;
      }
      size_t n = std::min(s.R, kTileCodeBytes / 4);  // the rest of a longer vector does not fit
      buf.resize(n);
      if (s.ones) std::fill(buf.begin(), buf.end(), 1.0f);
      else normals(key, 0, n, kStd, buf.data());
      for (size_t i = 0; i < n; ++i) putf(dst + 4 * i, buf[i]);
      break;
    }
    case SegKind::Cell16: {
      size_t r0 = t * 16, rows = r0 < s.R ? std::min<size_t>(16, s.R - r0) : 0;
      if (!rows) break;
      buf.resize(rows * s.C);
      fp16_weights(key, r0 * s.C, rows * s.C, buf.data());
      pack_cell16(buf.data(), int(rows), int(s.C), p.bits, 8, s.layer, out);
      break;
    }
    case SegKind::Flat: {
      size_t total = s.R * s.C, e0 = t * kFlatWeights;
      buf.assign(kFlatWeights, 0.0f);
      if (e0 < total) fp16_weights(key, e0, std::min(kFlatWeights, total - e0), buf.data());
      pack_flat(buf.data(), p.bits, 64, s.layer, out);
      break;
    }
  }
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
  int fd = ::open(path, O_RDWR | O_CREAT | O_TRUNC, 0644);
  if (fd < 0) return -2;
  if (::ftruncate(fd, off_t(size)) != 0) { ::close(fd); return -2; }
  void* m = ::mmap(nullptr, size, PROT_READ | PROT_WRITE, MAP_SHARED, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) return -2;
  uint8_t* base = static_cast<uint8_t*>(m);
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
  std::memcpy(base, &h, sizeof h);

  // record -> segment lookup table (segments are sorted and contiguous)
  std::vector<uint32_t> seg_of(p.records);
  for (size_t i = 0; i < p.segs.size(); ++i)
    for (size_t r = 0; r < p.segs[i].count; ++r) seg_of[p.segs[i].first + r] = uint32_t(i);

  unsigned nt = threads > 0 ? unsigned(threads) : std::max(1u, std::thread::hardware_concurrency());
  std::atomic<size_t> next{0};
  const size_t chunk = 64;
  auto worker = [&]() {
    std::vector<float> buf;
    for (;;) {
      size_t r0 = next.fetch_add(chunk);
      if (r0 >= p.records) break;
      for (size_t r = r0; r < std::min(p.records, r0 + chunk); ++r) {
        const Segment& s = p.segs[seg_of[r]];
        uint8_t* rec = base + kHeaderBytes + r * p.stride;
        uint8_t* out = p.stride == kTileCodeBytes ? rec : rec + p.prefetch;
        fill_record(p, s, r - s.first, seed, out, buf);
      }
    }
  };
  std::vector<std::thread> pool;
  for (unsigned i = 0; i < nt; ++i) pool.emplace_back(worker);
  for (auto& th : pool) th.join();
  ::munmap(m, size);
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
