// format.hpp -- the .chpe archive format: header, record geometries, cell layout.
//
// Byte-compatible with the reference format:
//   header         src/weight_archive.zig:53-86 (64 B at offset 0 of a 4096 B sector)
//   TileMetadata   src/weight_archive.zig:92-105 (32 B at the start of the cell payload)
//   TileDims       src/chpe_engine.zig:150-155   (16 B at payload + 32)
//   Cell / Record  src/geometry.zig:243-270      (17408 B cell, 20480 B record)
//   flags          src/weight_archive.zig:108-112
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstring>

namespace chpe {

constexpr uint32_t kArchiveMagic = 0x57415243u;  // "WARC"
constexpr uint32_t kChpeMagic = 0x45504843u;     // "CHPE"
constexpr uint32_t kArchiveVersion = 1;
constexpr size_t kHeaderBytes = 4096;
constexpr size_t kCellBytes = 17408;       // 272 x 64 B
constexpr size_t kRecordBytes = 20480;     // 5 x 4096 B
constexpr size_t kPrefetchBytes = 3072;    // record = prefetch label + cell
constexpr size_t kBytecodeHeader = 64;     // cell: [0,64) header
constexpr size_t kTileCodeBytes = 16384;   // cell: [64,16448) codes; also the raw tile size
constexpr size_t kPayloadOff = 16448;      // cell: [16448,17408) payload (960 B)
constexpr size_t kPayloadBytes = 960;

constexpr uint64_t kFlagGroup128 = 0x01;   // group-128 f16 scales + outliers
constexpr uint64_t kFlagHybrid = 0x02;
constexpr uint64_t kFlagRawFp16 = 0x04;    // raw tiles hold IEEE fp16 (else bf16)
constexpr uint64_t kFlagInt8Hint = 0x08;   // read as "9B raw is int8" (chpe_engine.zig:886)

// payload offsets (relative to the payload start)
constexpr size_t kMetaQuantBits = 20;      // u8
constexpr size_t kMetaCustomFlags = 24;    // u64
constexpr size_t kDimsScale = 32, kDimsBias = 36, kDimsRows = 40, kDimsCols = 44;
constexpr size_t kGroupScales = 48;        // f16[256] (f16[128] for the 8-bit embed cell)
constexpr size_t kRowOutlierW = 560;       // 16-row cells: f16[16][8]
constexpr size_t kRowOutlierCols = 816;    // 16-row cells: u16[8]
constexpr size_t kFlatOutlierN = 560;      // flat cells: u16 n (applied if 0 < n <= 64)
constexpr size_t kFlatOutlierW = 562;      // flat cells: f16[n]
constexpr size_t kFlatOutlierOff = 690;    // flat cells: u16[n] flat offsets
constexpr size_t kFlatWeights = 32768;     // weights per flat tile

static_assert(kCellBytes == 272 * 64, "cell is 272 cache lines");
static_assert(kRecordBytes == 5 * 4096, "record is 5 sectors");
static_assert(kRecordBytes - kCellBytes == kPrefetchBytes, "record = label + cell");
static_assert(kBytecodeHeader + kTileCodeBytes == kPayloadOff, "codes follow the header");
static_assert(kPayloadOff + kPayloadBytes == kCellBytes, "payload closes the cell");
static_assert(kFlatOutlierW + 2 * 64 == kFlatOutlierOff, "flat outlier arrays abut");

struct ArchiveHeader {
  uint32_t magic;
  uint32_t version;
  uint64_t header_bytes;
  uint64_t record_count;
  uint64_t tile_count;
  uint64_t record_bytes;
  uint64_t cell_bytes;
  uint64_t prefetch_bytes;
  uint64_t flags;
};
static_assert(sizeof(ArchiveHeader) == 64, "64-byte header");
static_assert(offsetof(ArchiveHeader, record_count) == 16, "");
static_assert(offsetof(ArchiveHeader, record_bytes) == 32, "");
static_assert(offsetof(ArchiveHeader, flags) == 56, "");

struct TileMetadata {
  uint32_t layer_index;
  uint32_t expert_index;
  uint64_t zeck_index;
  uint32_t bit_budget;
  uint8_t quant_bits;
  uint8_t reserved[3];
  uint64_t custom_flags;
};
static_assert(sizeof(TileMetadata) == 32, "");
static_assert(offsetof(TileMetadata, quant_bits) == kMetaQuantBits, "");
static_assert(offsetof(TileMetadata, custom_flags) == kMetaCustomFlags, "");

struct TileDims {
  float scale;
  float bias;
  uint32_t rows;
  uint32_t cols;
};
static_assert(sizeof(TileDims) == 16, "");

// IEEE half <-> float.  Widening is exact; narrowing rounds to nearest even.
inline float f16_to_f32(uint16_t h) {
  uint32_t sign = uint32_t(h & 0x8000u) << 16, ex = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
  if (ex == 0) {
    float v = float(man) * 5.9604644775390625e-8f;
    return sign ? -v : v;
  }
  bits = ex == 31 ? (sign | 0x7f800000u | (man << 13)) : (sign | ((ex + 112u) << 23) | (man << 13));
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

inline uint16_t f32_to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  uint32_t sign = (x >> 16) & 0x8000u, ex = (x >> 23) & 0xffu, man = x & 0x7fffffu;
  if (ex == 0xff) return uint16_t(sign | 0x7c00u | (man ? 0x200u : 0u));
  int e = int(ex) - 127 + 15;
  if (e >= 31) return uint16_t(sign | 0x7c00u);
  if (e <= 0) {
    if (e < -10) return uint16_t(sign);
    man |= 0x800000u;
    int shift = 14 - e;
    uint32_t half = man >> shift, rem = man & ((1u << shift) - 1u), mid = 1u << (shift - 1);
    if (rem > mid || (rem == mid && (half & 1u))) half++;
    return uint16_t(sign | half);
  }
  uint32_t half = (uint32_t(e) << 10) | (man >> 13), rem = man & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
  return uint16_t(sign | half);
}

inline float bf16_to_f32(uint16_t h) {
  uint32_t bits = uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &bits, 4);
  return f;
}

inline uint16_t f32_to_bf16(float f) {  // round to nearest even
  uint32_t x;
  std::memcpy(&x, &f, 4);
  if ((x & 0x7f800000u) == 0x7f800000u) return uint16_t((x >> 16) | ((x & 0xffffu) ? 0x40u : 0u));
  uint32_t lsb = (x >> 16) & 1u;
  return uint16_t((x + 0x7fffu + lsb) >> 16);
}

}  // namespace chpe
