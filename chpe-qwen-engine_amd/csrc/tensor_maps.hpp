// tensor_maps.hpp -- record index of every tensor for the four archive layouts.
//
// The raw 3B, 9B and 72B layouts follow a construction rule and are computed from it; the
// 3B cell layout has no rule (its layers sit in an irregular order and layer 21 keeps its
// down_proj apart from the rest of the layer), so it is carried as a table of records:
//   3B raw   Bf16LayerOffsets            src/qwen3b_geometry.zig:48-79
//   3B cell  LAYERS                      src/qwen3b_tensor_map.zig:26-531
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

// Records of the 3B cell archive, per layer: input_norm, q_proj, q_bias, k_proj, k_bias,
// v_proj, v_bias, o_proj, post_norm, gate_proj, up_proj, down_proj
// (qwen3b_tensor_map.LAYERS, src/qwen3b_tensor_map.zig:26-531).
inline constexpr uint32_t kQwen3bCellRecords[36][12] = {
    {9496, 11708, 11707, 11563, 11562, 11837, 11836, 11579, 11561, 10185, 10873, 9497},  // 0
    {11853, 14065, 14064, 13920, 13919, 14194, 14193, 13936, 13918, 12542, 13230, 11854},  // 1
    {37780, 39992, 39991, 39847, 39846, 40121, 40120, 39863, 39845, 38469, 39157, 37781},  // 2
    {44163, 46375, 46374, 46230, 46229, 46504, 46503, 46246, 46228, 44852, 45540, 44164},  // 3
    {46520, 48732, 48731, 48587, 48586, 48861, 48860, 48603, 48585, 47209, 47897, 46521},  // 4
    {48877, 51089, 51088, 50944, 50943, 51218, 51217, 50960, 50942, 49566, 50254, 48878},  // 5
    {51234, 53446, 53445, 53301, 53300, 53575, 53574, 53317, 53299, 51923, 52611, 51235},  // 6
    {53591, 55803, 55802, 55658, 55657, 55932, 55931, 55674, 55656, 54280, 54968, 53592},  // 7
    {55948, 58160, 58159, 58015, 58014, 58289, 58288, 58031, 58013, 56637, 57325, 55949},  // 8
    {58305, 60517, 60516, 60372, 60371, 60646, 60645, 60388, 60370, 58994, 59682, 58306},  // 9
    {14210, 16422, 16421, 16277, 16276, 16551, 16550, 16293, 16275, 14899, 15587, 14211},  // 10
    {16567, 18779, 18778, 18634, 18633, 18908, 18907, 18650, 18632, 17256, 17944, 16568},  // 11
    {18924, 21136, 21135, 20991, 20990, 21265, 21264, 21007, 20989, 19613, 20301, 18925},  // 12
    {21281, 23493, 23492, 23348, 23347, 23622, 23621, 23364, 23346, 21970, 22658, 21282},  // 13
    {23638, 25850, 25849, 25705, 25704, 25979, 25978, 25721, 25703, 24327, 25015, 23639},  // 14
    {25995, 28207, 28206, 28062, 28061, 28336, 28335, 28078, 28060, 26684, 27372, 25996},  // 15
    {28352, 30564, 30563, 30419, 30418, 30693, 30692, 30435, 30417, 29041, 29729, 28353},  // 16
    {30709, 32921, 32920, 32776, 32775, 33050, 33049, 32792, 32774, 31398, 32086, 30710},  // 17
    {33066, 35278, 35277, 35133, 35132, 35407, 35406, 35149, 35131, 33755, 34443, 33067},  // 18
    {35423, 37635, 37634, 37490, 37489, 37764, 37763, 37506, 37488, 36112, 36800, 35424},  // 19
    {40137, 42349, 42348, 42204, 42203, 42478, 42477, 42220, 42202, 40826, 41514, 40138},  // 20
    {42494, 44018, 44017, 43873, 43872, 44147, 44146, 43889, 43871, 42495, 43183, 60662},  // 21
    {61350, 63562, 63561, 63417, 63416, 63691, 63690, 63433, 63415, 62039, 62727, 61351},  // 22
    {63707, 65919, 65918, 65774, 65773, 66048, 66047, 65790, 65772, 64396, 65084, 63708},  // 23
    {66064, 68276, 68275, 68131, 68130, 68405, 68404, 68147, 68129, 66753, 67441, 66065},  // 24
    {68421, 70633, 70632, 70488, 70487, 70762, 70761, 70504, 70486, 69110, 69798, 68422},  // 25
    {70778, 72990, 72989, 72845, 72844, 73119, 73118, 72861, 72843, 71467, 72155, 70779},  // 26
    {73135, 75347, 75346, 75202, 75201, 75476, 75475, 75218, 75200, 73824, 74512, 73136},  // 27
    {75492, 77704, 77703, 77559, 77558, 77833, 77832, 77575, 77557, 76181, 76869, 75493},  // 28
    {77849, 80061, 80060, 79916, 79915, 80190, 80189, 79932, 79914, 78538, 79226, 77850},  // 29
    {80206, 82418, 82417, 82273, 82272, 82547, 82546, 82289, 82271, 80895, 81583, 80207},  // 30
    {82563, 84775, 84774, 84630, 84629, 84904, 84903, 84646, 84628, 83252, 83940, 82564},  // 31
    {84920, 87132, 87131, 86987, 86986, 87261, 87260, 87003, 86985, 85609, 86297, 84921},  // 32
    {87277, 89489, 89488, 89344, 89343, 89618, 89617, 89360, 89342, 87966, 88654, 87278},  // 33
    {89634, 91846, 91845, 91701, 91700, 91975, 91974, 91717, 91699, 90323, 91011, 89635},  // 34
    {91991, 94203, 94202, 94058, 94057, 94332, 94331, 94074, 94056, 92680, 93368, 91992},  // 35
};

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
      const uint32_t* t = kQwen3bCellRecords[l];
      o.input_norm = t[0];
      o.q_proj = t[1]; o.q_bias = t[2]; o.k_proj = t[3]; o.k_bias = t[4];
      o.v_proj = t[5]; o.v_bias = t[6]; o.o_proj = t[7]; o.post_norm = t[8];
      o.gate_proj = t[9]; o.up_proj = t[10]; o.down_proj = t[11];
      o.q_tiles = 128; o.k_tiles = 16; o.v_tiles = 16; o.o_tiles = 128;  // chpe_engine.zig:1061-1082
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

// Every record index of a Qwen3.5-9B layer (qwen35_tensor_map.LAYERS, the INT8 spans;
// src/qwen35_tensor_map.zig:7-50 names the fields).  Full-attention layers (3, 7, ..., 31):
// q (2048 records), k (256), v (256), o (1024), q_norm, k_norm; linear-attention layers:
// in_proj_qkv (2048), in_proj_z (1024), in_proj_a (8), in_proj_b (8), conv1d (4), a_log,
// dt_bias, linear_norm, out_proj (1024).  gate / up / down: 3072 records each.
struct Qwen35Records {
  bool full_attn;
  size_t input_norm, post_norm, gate_proj, up_proj, down_proj;
  size_t q_proj, k_proj, v_proj, o_proj, q_norm, k_norm;                      // full attention
  size_t in_proj_qkv, in_proj_z, in_proj_a, in_proj_b, conv1d, a_log, dt_bias, linear_norm,
      out_proj;                                                               // linear attention
};

inline Qwen35Records qwen35_records(size_t l) {
  Qwen35Records r{};
  size_t b = 62080;
  for (size_t i = 0; i < l; ++i) b += qwen35_is_full_attn(i) ? 12804 : 13337;
  r.full_attn = qwen35_is_full_attn(l);
  r.input_norm = b;
  if (r.full_attn) {
    r.q_proj = b + 1; r.k_proj = b + 2049; r.v_proj = b + 2305; r.o_proj = b + 2561;
    r.q_norm = b + 3585; r.k_norm = b + 3586; r.post_norm = b + 3587;
  } else {
    r.in_proj_qkv = b + 1; r.in_proj_z = b + 2049; r.in_proj_a = b + 3073; r.in_proj_b = b + 3081;
    r.conv1d = b + 3089; r.a_log = b + 3093; r.dt_bias = b + 3094; r.linear_norm = b + 3095;
    r.out_proj = b + 3096; r.post_norm = b + 4120;
  }
  r.gate_proj = r.post_norm + 1;
  r.up_proj = r.gate_proj + 3072;
  r.down_proj = r.up_proj + 3072;
  return r;
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
