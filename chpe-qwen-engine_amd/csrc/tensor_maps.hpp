// tensor_maps.hpp -- record index of every tensor for the four archive layouts.
//
// The reference keeps these as static tables; here they are computed from each table's
// construction rule (the same record indices, checked against the tables by the tests):
//   3B raw   Bf16LayerOffsets            src/qwen3b_geometry.zig:48-79
//   3B cell  LAYERS (HF alphabetical)    src/qwen3b_tensor_map.zig:21-531
//   9B       LAYERS                      src/qwen35_tensor_map.zig:53-1015
//   72B      makeLayer                   src/qwen72b_tensor_map.zig:16-87
// and the engine's view of them (tile counts, 9B GQA aliasing): src/chpe_engine.zig:1017-1142.
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstring>

namespace chpe {

enum class MapKind : int { Qwen3bRaw = 0, Qwen3bCell = 1, Qwen35_9b = 2, Qwen72b = 3 };

struct LayerInfo {  // CHPEEngine.LayerInfo, src/chpe_engine.zig:1017-1033
  size_t input_norm, q_proj, q_tiles, k_proj, k_tiles, v_proj, v_tiles, o_proj, o_tiles;
  size_t post_norm, gate_proj, gate_tiles, up_proj, up_tiles, down_proj, down_tiles;
  int64_t q_bias = -1, k_bias = -1, v_bias = -1;  // -1 = no bias tensor
};

// 3B cell archives store layers in the order of their names sorted as strings.
inline size_t alpha_rank(size_t l, size_t n_layers) {
  char a[8], b[8];
  std::snprintf(a, sizeof a, "%zu", l);
  size_t rank = 0;
  for (size_t i = 0; i < n_layers; ++i) {
    std::snprintf(b, sizeof b, "%zu", i);
    if (std::strcmp(b, a) < 0) ++rank;
  }
  return rank;
}

inline bool qwen35_is_full_attn(size_t l) { return l % 4 == 3; }  // layers 3, 7, ..., 31

inline LayerInfo layer_info(MapKind m, size_t l) {
  LayerInfo o{};
  switch (m) {
    case MapKind::Qwen3bRaw: {
      size_t b = 37984 + l * 9413;
      o.input_norm = b;
      o.q_proj = b + 1; o.q_tiles = 512; o.q_bias = int64_t(b + 513);
      o.k_proj = b + 514; o.k_tiles = 64; o.k_bias = int64_t(b + 578);
      o.v_proj = b + 579; o.v_tiles = 64; o.v_bias = int64_t(b + 643);
      o.o_proj = b + 644; o.o_tiles = 512;
      o.post_norm = b + 1156;
      o.gate_proj = b + 1157; o.gate_tiles = 2752;
      o.up_proj = b + 3909; o.up_tiles = 2752;
      o.down_proj = b + 6661; o.down_tiles = 2752;
      break;
    }
    case MapKind::Qwen3bCell: {
      size_t b = 9496 + alpha_rank(l, 36) * 2357;
      o.input_norm = b;
      o.down_proj = b + 1; o.gate_proj = b + 689; o.up_proj = b + 1377;
      o.post_norm = b + 2065;
      o.k_bias = int64_t(b + 2066); o.k_proj = b + 2067;
      o.o_proj = b + 2083;
      o.q_bias = int64_t(b + 2211); o.q_proj = b + 2212;
      o.v_bias = int64_t(b + 2340); o.v_proj = b + 2341;
      o.q_tiles = 128; o.k_tiles = 16; o.v_tiles = 16; o.o_tiles = 128;
      o.gate_tiles = 688; o.up_tiles = 688; o.down_tiles = 688;
      break;
    }
    case MapKind::Qwen35_9b: {
      size_t b = 62080;
      for (size_t i = 0; i < l; ++i) b += qwen35_is_full_attn(i) ? 12804 : 13337;
      o.input_norm = b;
      o.q_proj = b + 1; o.q_tiles = 2048;
      o.k_proj = b + 2049;
      if (qwen35_is_full_attn(l)) {
        o.k_tiles = 256;
        o.v_proj = b + 2305; o.v_tiles = 256;
        o.o_proj = b + 2561; o.o_tiles = 1024;
        o.post_norm = b + 3587; o.gate_proj = b + 3588; o.up_proj = b + 6660; o.down_proj = b + 9732;
      } else {  // linear-attention layer aliased onto GQA (in_proj_qkv / z / a, out_proj)
        o.k_tiles = 1024;
        o.v_proj = b + 3073; o.v_tiles = 1;
        o.o_proj = b + 3096; o.o_tiles = 1024;
        o.post_norm = b + 4120; o.gate_proj = b + 4121; o.up_proj = b + 7193; o.down_proj = b + 10265;
      }
      o.gate_tiles = o.up_tiles = o.down_tiles = 3072;
      break;
    }
    case MapKind::Qwen72b: {
      size_t b = 38016 + l * 26789;
      o.input_norm = b;
      o.q_proj = b + 1; o.q_tiles = 2048; o.q_bias = int64_t(b + 2049);
      o.k_proj = b + 2050; o.k_tiles = 256; o.k_bias = int64_t(b + 2306);
      o.v_proj = b + 2307; o.v_tiles = 256; o.v_bias = int64_t(b + 2563);
      o.o_proj = b + 2564; o.o_tiles = 2048;
      o.post_norm = b + 4612;
      o.gate_proj = b + 4613; o.gate_tiles = 7392;
      o.up_proj = b + 12005; o.up_tiles = 7392;
      o.down_proj = b + 19397; o.down_tiles = 7392;
      break;
    }
  }
  return o;
}

inline size_t final_norm_record(MapKind m) {
  switch (m) {
    case MapKind::Qwen3bRaw: return 376852;
    case MapKind::Qwen3bCell: return 94348;
    case MapKind::Qwen35_9b: return 484600;
    default: return 2181136;
  }
}

// Untied LM head (computeLmHead, src/chpe_engine.zig:1565-1580); 3B ties it to the embedding.
inline bool lm_head_record(size_t hidden_dim, size_t* start, size_t* tiles) {
  if (hidden_dim == 8192) { *start = 2181137; *tiles = 38016; return true; }
  if (hidden_dim == 4096) { *start = 484601; *tiles = 62080; return true; }
  return false;
}

// record counts of complete archives
constexpr size_t kTotalRecords3bRaw = 376853;
constexpr size_t kTotalRecords3bCell = 94349;
constexpr size_t kTotalRecords9b = 546681;
constexpr size_t kTotalRecords72b = 2219153;

}  // namespace chpe
