/* chpe_oracle.c -- CPU restatement of the reference decode path.  TEST INFRASTRUCTURE.
 *
 * Loaded only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
 * checker and the timed CPU baseline.  The engine never links or calls it.
 *
 * Every function cites the reference function it restates (paths relative to the
 * reference tree).  Float structure follows the reference exactly: 8-lane `@Vector`
 * accumulators, ordered `@reduce(.Add)`, fmaf() only where Zig writes `@mulAdd`,
 * separate multiply/add everywhere else (compiled -ffp-contract=off).
 *
 * What pins each function (the tests named are the checks; none retypes this file's formulas):
 *   gemvTileW2/W4/W8 ........ closed forms of the reference's own synthetic cells
 *                             (chpe_engine.zig:1814-1891): test_oracle_kats.py
 *                             test_gemv_{2,4,8}bit_synthetic_cell, test_gemv_accumulate_adds_to_y;
 *                             the float64 product of the generator's weights within the
 *                             quantizer's bound on a whole archive: test_oracle_step.py
 *                             test_projection_within_quantization_bound
 *   gemvTileF16/F32 ......... float64 brute force (fp16, bf16, f32 cells; tails, clipping,
 *                             accumulate): test_oracle_pinning.py
 *                             test_f16_bf16_f32_cells_are_float64_products
 *   gemvCellFlat ............ closed-form tiles (group scales, replaced outliers, the 2-bit
 *                             codebook, the no-group scale + bias forms of both widths with
 *                             the product and the sum rounded separately): test_oracle_kats.py
 *                             test_flat_tile_*; the down projection within the quantizer's
 *                             bound (test_oracle_step.py)
 *   dotSegment / raw gemvLinear / raw unpackEmbedRow / raw tied computeLmHead (fp16, bf16,
 *   int8 x 0.00373708) ...... float64 products of the generator's weights within the f32
 *                             summation bound, rows straddling tiles, embedding rows bit for
 *                             bit: test_oracle_pinning.py test_raw_*
 *   unpackEmbedRowCell ...... a numpy decode of the q8 / q2 / q4 / per-tile-scale forms
 *                             (outliers replacing in entry order, rows past the cell):
 *                             test_oracle_pinning.py test_embed_row_cell_forms_match_numpy_decode;
 *                             the generator's weights within the quantizer's bound:
 *                             test_oracle_step.py test_embedding_row_within_quantization_bound
 *   f16 / bf16 widening, f32 -> f16 rounding (the fp16 KV cache) ...... numpy's float16 over
 *                             all 65536 codes and over every f32 of the f16 exponent range:
 *                             test_oracle_kats.py test_f16_widening_exhaustive,
 *                             test_f32_to_f16_matches_numpy
 *   rmsNorm ................. KAT qwen_rmsnorm.zig:73-90 + float64: test_oracle_kats.py
 *   applyRope ............... KAT qwen_rope.zig:149-162, pos-0 identity, closed form
 *   silu .................... KAT qwen_mlp.zig:92-111
 *   attention ............... seq-1 pass-through KAT (qwen_attention.zig:144-169), float64
 *                             softmax brute force: test_oracle_kats.py
 *   validate ................ the malformed-file cases of weight_archive.zig:1048-1078:
 *                             test_format.py test_validate_reference_error_cases
 *   layer maps .............. tests/golden/tensor_maps.json (the reference tables):
 *                             test_format.py test_*_map_*
 *   forwardDecode ........... the mock zero archive KAT (chpe_engine.zig:1893-1933) with the
 *                             closed forms of its fallbacks, and two decode steps restated in
 *                             float64 from forwardDecode on numpy-decoded weights:
 *                             test_oracle_pinning.py test_mock_zero_archive_known_answer,
 *                             test_forward_decode_composition_float64
 *   Gated DeltaNet (deltanet_oracle.c, no reference code): library fixtures, float64 and
 *                             invariants: test_oracle_deltanet.py
 *   Not pinned bit for bit: libm-level ulps of expf / powf / sinf / cosf (Zig's
 *   implementations are not available here); covered by the tolerances above.
 */
#define _GNU_SOURCE
#include "chpe_oracle.h"

#include <fcntl.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>
#ifdef _OPENMP
#include <omp.h>
#endif

/* ---- format constants: src/geometry.zig:21-62, src/weight_archive.zig:17-123 ---- */
#define HEADER_BYTES 4096u
#define CELL_BYTES 17408u
#define RECORD_BYTES 20480u
#define PREFETCH_BYTES 3072u
#define BYTECODE_HEADER 64u
#define TILE_CODE_BYTES 16384u
#define PAYLOAD_OFF 16448u
#define ARCHIVE_MAGIC 0x57415243u
#define CHPE_MAGIC 0x45504843u
#define FLAG_GROUP128 0x01u
#define FLAG_RAW_FP16 0x04u
#define MAP_PAD (1u << 20) /* zero bytes mapped after the file end */

static inline uint16_t rd16(const uint8_t *p) { uint16_t v; memcpy(&v, p, 2); return v; }
static inline uint32_t rd32(const uint8_t *p) { uint32_t v; memcpy(&v, p, 4); return v; }
static inline uint64_t rd64(const uint8_t *p) { uint64_t v; memcpy(&v, p, 8); return v; }
static inline float rdf32(const uint8_t *p) { float v; memcpy(&v, p, 4); return v; }

/* @reduce(.Add, v) on @Vector(8,f32): ordered fadd chain */
static inline float reduce8(const float a[8]) {
    float s = a[0];
    s += a[1]; s += a[2]; s += a[3]; s += a[4]; s += a[5]; s += a[6]; s += a[7];
    return s;
}

float oref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (ex == 0) {
        float v = (float)man * 5.9604644775390625e-8f; /* man * 2^-24, exact */
        return sign ? -v : v;
    } else if (ex == 31) {
        bits = sign | 0x7f800000u | (man << 13);
    } else {
        bits = sign | ((ex + 112u) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

float oref_bf16_to_f32(uint16_t h) {
    uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* f32 -> f16 round-to-nearest-even (used for the fp16-KV variant only; the reference keeps an
 * f32 cache).  Pinned against numpy's float16 conversion over every f32 whose exponent reaches
 * the f16 range, both signs (test_oracle_kats.py test_f32_to_f16_matches_numpy). */
static uint16_t f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint32_t sign = (x >> 16) & 0x8000u, ex = (x >> 23) & 0xffu, man = x & 0x7fffffu;
    if (ex == 0xff) return (uint16_t)(sign | 0x7c00u | (man ? 0x200u : 0u));
    int e = (int)ex - 127 + 15;
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        man |= 0x800000u;
        int shift = 14 - e;
        uint32_t half = man >> shift, rem = man & ((1u << shift) - 1u), mid = 1u << (shift - 1);
        if (rem > mid || (rem == mid && (half & 1u))) half++;
        return (uint16_t)(sign | half);
    }
    uint32_t half = ((uint32_t)e << 10) | (man >> 13), rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (half & 1u))) half++;
    return (uint16_t)(sign | half);
}

void oref_f32_to_f16_n(const float *x, uint16_t *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = f32_to_f16(x[i]);
}

void oref_f16_to_f32_n(const uint16_t *h, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) out[i] = oref_f16_to_f32(h[i]);
}

static uint64_t now_ns(void) { /* nowNs: src/chpe_engine.zig:812-816 */
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (uint64_t)ts.tv_sec * 1000000000ull + (uint64_t)ts.tv_nsec;
}

/* ---------------------------------------------------------------- presets */
int oref_arch_preset(int id, oref_arch *a) { /* src/chpe_engine.zig:110-145 */
    memset(a, 0, sizeof *a);
    a->id = id;
    a->rope_theta = 1000000.0f;
    a->rms_eps = 1e-6f;
    switch (id) {
    case 0: a->hidden_dim = 2048; a->intermediate_dim = 11008; a->num_layers = 36;
        a->num_attn_heads = 16; a->num_kv_heads = 2; a->head_dim = 128; a->vocab_size = 151936;
        return 0;
    case 1: a->hidden_dim = 4096; a->intermediate_dim = 12288; a->num_layers = 32;
        a->num_attn_heads = 16; a->num_kv_heads = 4; a->head_dim = 256; a->vocab_size = 248320;
        return 0;
    case 2: a->hidden_dim = 8192; a->intermediate_dim = 29568; a->num_layers = 80;
        a->num_attn_heads = 64; a->num_kv_heads = 8; a->head_dim = 128; a->vocab_size = 152064;
        return 0;
    }
    return -1;
}

int oref_arch_from_path(const char *p) { /* src/chpe_c_api.zig:29-37 */
    if (strstr(p, "9B") || strstr(p, "9b") || strstr(p, "qwen35")) return 1;
    if (strstr(p, "72B") || strstr(p, "72b")) return 2;
    return 0;
}

/* ---------------------------------------------------------------- layer maps */
/* qwen3b_tensor_map.LAYERS (src/qwen3b_tensor_map.zig:26-531), per layer: input_norm,
 * q_proj, q_bias, k_proj, k_bias, v_proj, v_bias, o_proj, post_norm, gate_proj, up_proj,
 * down_proj.  The table has no construction rule (irregular layer order; layer 21's
 * down_proj sits apart from the rest of its layer). */
static const uint32_t QWEN3B_CELL[36][12] = {
    {9496, 11708, 11707, 11563, 11562, 11837, 11836, 11579, 11561, 10185, 10873, 9497}, /* 0 */
    {11853, 14065, 14064, 13920, 13919, 14194, 14193, 13936, 13918, 12542, 13230, 11854}, /* 1 */
    {37780, 39992, 39991, 39847, 39846, 40121, 40120, 39863, 39845, 38469, 39157, 37781}, /* 2 */
    {44163, 46375, 46374, 46230, 46229, 46504, 46503, 46246, 46228, 44852, 45540, 44164}, /* 3 */
    {46520, 48732, 48731, 48587, 48586, 48861, 48860, 48603, 48585, 47209, 47897, 46521}, /* 4 */
    {48877, 51089, 51088, 50944, 50943, 51218, 51217, 50960, 50942, 49566, 50254, 48878}, /* 5 */
    {51234, 53446, 53445, 53301, 53300, 53575, 53574, 53317, 53299, 51923, 52611, 51235}, /* 6 */
    {53591, 55803, 55802, 55658, 55657, 55932, 55931, 55674, 55656, 54280, 54968, 53592}, /* 7 */
    {55948, 58160, 58159, 58015, 58014, 58289, 58288, 58031, 58013, 56637, 57325, 55949}, /* 8 */
    {58305, 60517, 60516, 60372, 60371, 60646, 60645, 60388, 60370, 58994, 59682, 58306}, /* 9 */
    {14210, 16422, 16421, 16277, 16276, 16551, 16550, 16293, 16275, 14899, 15587, 14211}, /* 10 */
    {16567, 18779, 18778, 18634, 18633, 18908, 18907, 18650, 18632, 17256, 17944, 16568}, /* 11 */
    {18924, 21136, 21135, 20991, 20990, 21265, 21264, 21007, 20989, 19613, 20301, 18925}, /* 12 */
    {21281, 23493, 23492, 23348, 23347, 23622, 23621, 23364, 23346, 21970, 22658, 21282}, /* 13 */
    {23638, 25850, 25849, 25705, 25704, 25979, 25978, 25721, 25703, 24327, 25015, 23639}, /* 14 */
    {25995, 28207, 28206, 28062, 28061, 28336, 28335, 28078, 28060, 26684, 27372, 25996}, /* 15 */
    {28352, 30564, 30563, 30419, 30418, 30693, 30692, 30435, 30417, 29041, 29729, 28353}, /* 16 */
    {30709, 32921, 32920, 32776, 32775, 33050, 33049, 32792, 32774, 31398, 32086, 30710}, /* 17 */
    {33066, 35278, 35277, 35133, 35132, 35407, 35406, 35149, 35131, 33755, 34443, 33067}, /* 18 */
    {35423, 37635, 37634, 37490, 37489, 37764, 37763, 37506, 37488, 36112, 36800, 35424}, /* 19 */
    {40137, 42349, 42348, 42204, 42203, 42478, 42477, 42220, 42202, 40826, 41514, 40138}, /* 20 */
    {42494, 44018, 44017, 43873, 43872, 44147, 44146, 43889, 43871, 42495, 43183, 60662}, /* 21 */
    {61350, 63562, 63561, 63417, 63416, 63691, 63690, 63433, 63415, 62039, 62727, 61351}, /* 22 */
    {63707, 65919, 65918, 65774, 65773, 66048, 66047, 65790, 65772, 64396, 65084, 63708}, /* 23 */
    {66064, 68276, 68275, 68131, 68130, 68405, 68404, 68147, 68129, 66753, 67441, 66065}, /* 24 */
    {68421, 70633, 70632, 70488, 70487, 70762, 70761, 70504, 70486, 69110, 69798, 68422}, /* 25 */
    {70778, 72990, 72989, 72845, 72844, 73119, 73118, 72861, 72843, 71467, 72155, 70779}, /* 26 */
    {73135, 75347, 75346, 75202, 75201, 75476, 75475, 75218, 75200, 73824, 74512, 73136}, /* 27 */
    {75492, 77704, 77703, 77559, 77558, 77833, 77832, 77575, 77557, 76181, 76869, 75493}, /* 28 */
    {77849, 80061, 80060, 79916, 79915, 80190, 80189, 79932, 79914, 78538, 79226, 77850}, /* 29 */
    {80206, 82418, 82417, 82273, 82272, 82547, 82546, 82289, 82271, 80895, 81583, 80207}, /* 30 */
    {82563, 84775, 84774, 84630, 84629, 84904, 84903, 84646, 84628, 83252, 83940, 82564}, /* 31 */
    {84920, 87132, 87131, 86987, 86986, 87261, 87260, 87003, 86985, 85609, 86297, 84921}, /* 32 */
    {87277, 89489, 89488, 89344, 89343, 89618, 89617, 89360, 89342, 87966, 88654, 87278}, /* 33 */
    {89634, 91846, 91845, 91701, 91700, 91975, 91974, 91717, 91699, 90323, 91011, 89635}, /* 34 */
    {91991, 94203, 94202, 94058, 94057, 94332, 94331, 94074, 94056, 92680, 93368, 91992}, /* 35 */
};

int oref_layer_info_for(int map, size_t l, oref_layer_info *o) {
    memset(o, 0, sizeof *o);
    o->q_bias = o->k_bias = o->v_bias = -1;
    if (map == 0) { /* Bf16LayerOffsets: src/qwen3b_geometry.zig:48-79 */
        size_t b = 37984 + l * 9413;
        o->input_norm = b; o->q_proj = b + 1; o->q_tiles = 512; o->q_bias = (int64_t)(b + 513);
        o->k_proj = b + 514; o->k_tiles = 64; o->k_bias = (int64_t)(b + 578);
        o->v_proj = b + 579; o->v_tiles = 64; o->v_bias = (int64_t)(b + 643);
        o->o_proj = b + 644; o->o_tiles = 512; o->post_norm = b + 1156;
        o->gate_proj = b + 1157; o->gate_tiles = 2752; o->up_proj = b + 3909; o->up_tiles = 2752;
        o->down_proj = b + 6661; o->down_tiles = 2752;
        return 0;
    }
    if (map == 1) { /* qwen3b_tensor_map.LAYERS + fixed counts: chpe_engine.zig:1060-1082 */
        const uint32_t *t = QWEN3B_CELL[l];
        o->input_norm = t[0]; o->q_proj = t[1]; o->q_bias = t[2]; o->k_proj = t[3]; o->k_bias = t[4];
        o->v_proj = t[5]; o->v_bias = t[6]; o->o_proj = t[7]; o->post_norm = t[8];
        o->gate_proj = t[9]; o->up_proj = t[10]; o->down_proj = t[11];
        o->q_tiles = 128; o->k_tiles = 16; o->v_tiles = 16; o->o_tiles = 128;
        o->gate_tiles = 688; o->up_tiles = 688; o->down_tiles = 688;
        return 0;
    }
    if (map == 2) { /* qwen35_tensor_map.LAYERS + GQA aliasing: chpe_engine.zig:1107-1131 */
        size_t b = 62080;
        for (size_t i = 0; i < l; i++) b += (i % 4 == 3) ? 12804 : 13337;
        if (l % 4 == 3) { /* full attention */
            o->input_norm = b; o->q_proj = b + 1; o->q_tiles = 2048; o->k_proj = b + 2049;
            o->k_tiles = 256; o->v_proj = b + 2305; o->v_tiles = 256; o->o_proj = b + 2561;
            o->o_tiles = 1024; o->post_norm = b + 3587; o->gate_proj = b + 3588;
            o->up_proj = b + 6660; o->down_proj = b + 9732;
        } else { /* linear attention, aliased: q<-in_proj_qkv, k<-in_proj_z, v<-in_proj_a */
            o->input_norm = b; o->q_proj = b + 1; o->q_tiles = 2048; o->k_proj = b + 2049;
            o->k_tiles = 1024; o->v_proj = b + 3073; o->v_tiles = 1; o->o_proj = b + 3096;
            o->o_tiles = 1024; o->post_norm = b + 4120; o->gate_proj = b + 4121;
            o->up_proj = b + 7193; o->down_proj = b + 10265;
        }
        o->gate_tiles = 3072; o->up_tiles = 3072; o->down_tiles = 3072;
        return 0;
    }
    if (map == 3) { /* qwen72b_tensor_map.makeLayer: src/qwen72b_tensor_map.zig:60-76 */
        size_t b = 38016 + l * 26789;
        o->input_norm = b; o->q_proj = b + 1; o->q_tiles = 2048; o->q_bias = (int64_t)(b + 2049);
        o->k_proj = b + 2050; o->k_tiles = 256; o->k_bias = (int64_t)(b + 2306);
        o->v_proj = b + 2307; o->v_tiles = 256; o->v_bias = (int64_t)(b + 2563);
        o->o_proj = b + 2564; o->o_tiles = 2048; o->post_norm = b + 4612;
        o->gate_proj = b + 4613; o->gate_tiles = 7392; o->up_proj = b + 12005; o->up_tiles = 7392;
        o->down_proj = b + 19397; o->down_tiles = 7392;
        return 0;
    }
    return -1;
}

size_t oref_final_norm_for(int map) { /* getFinalNormIndex: chpe_engine.zig:1134-1142 */
    switch (map) {
    case 0: return 376852;
    case 1: return 94348;
    case 2: return 484600;
    default: return 2181136;
    }
}

/* ---------------------------------------------------------------- validate */
int oref_validate(const uint8_t *b, size_t len) { /* WeightArchive.validate: weight_archive.zig:152-172 */
    if (len < HEADER_BYTES) return 1;
    uint32_t magic = rd32(b), version = rd32(b + 4);
    uint64_t header_bytes = rd64(b + 8), record_count = rd64(b + 16), record_bytes = rd64(b + 32),
             cell_bytes = rd64(b + 40), prefetch = rd64(b + 48);
    if (magic != ARCHIVE_MAGIC && magic != CHPE_MAGIC) return 2;
    if (version != 1) return 3;
    if (header_bytes != HEADER_BYTES) return 4;
    int is_standard = record_bytes == RECORD_BYTES && prefetch == PREFETCH_BYTES;
    int is_dense = record_bytes == CELL_BYTES && prefetch == 0;
    int is_raw = record_bytes == TILE_CODE_BYTES && prefetch == 0;
    if (!is_standard && !is_dense && !is_raw) return 5;
    if (!is_raw && cell_bytes != CELL_BYTES) return 5;
    if (is_raw && cell_bytes != TILE_CODE_BYTES) return 5;
    /* header_bytes + record_count * stride, with u64 wrap as in the reference */
    uint64_t required = header_bytes + record_count * record_bytes;
    if (required > len) return 6;
    return 0;
}

/* ---------------------------------------------------------------- primitives */
float oref_silu(float z) { return z / (1.0f + expf(-z)); } /* chpe_engine.zig:159-161 */

void oref_rmsnorm(const float *x, const float *g, float *y, size_t n, float eps) {
    /* rmsNorm: chpe_engine.zig:163-193 */
    float acc[8] = {0};
    size_t i = 0;
    for (; i + 8 <= n; i += 8)
        for (int k = 0; k < 8; k++) acc[k] = acc[k] + x[i + k] * x[i + k];
    float sum_sq = reduce8(acc);
    for (; i < n; i++) sum_sq += x[i] * x[i];
    float mean_sq = sum_sq / (float)n;
    float inv_rms = 1.0f / sqrtf(mean_sq + eps);
    for (i = 0; i < n; i++) y[i] = x[i] * inv_rms * g[i];
}

void oref_apply_rope(float *vec, size_t pos, size_t nh, size_t hd, float rope_theta) {
    /* applyRope: chpe_engine.zig:195-216 */
    float pos_f = (float)pos;
    for (size_t h = 0; h < nh; h++) {
        size_t base = h * hd;
        for (size_t i = 0; i < hd / 2; i++) {
            float freq_exponent = 2.0f * (float)i / (float)hd;
            float freq = 1.0f / powf(rope_theta, freq_exponent);
            float theta = pos_f * freq;
            float c = cosf(theta), s = sinf(theta);
            float x0 = vec[base + i], x1 = vec[base + i + hd / 2];
            vec[base + i] = x0 * c - x1 * s;
            vec[base + i + hd / 2] = x0 * s + x1 * c;
        }
    }
}

/* ---------------------------------------------------------------- cell kernels */
static const float CODEBOOK_W2[4] = {0.0f, 1.0f, -2.0f, -1.0f}; /* chpe_engine.zig:220 */

typedef struct {
    const uint8_t *codes, *payload;
    uint8_t quant_bits;
    uint64_t custom_flags;
    float scale, bias;
    uint32_t rows, cols;
} cell_view;

static cell_view view_cell(const uint8_t *cell) {
    cell_view v;
    v.codes = cell + BYTECODE_HEADER;
    v.payload = cell + PAYLOAD_OFF;
    v.quant_bits = v.payload[20];          /* TileMetadata.quant_bits @20 */
    v.custom_flags = rd64(v.payload + 24); /* TileMetadata.custom_flags @24 */
    v.scale = rdf32(v.payload + 32);       /* TileDims @32 */
    v.bias = rdf32(v.payload + 36);
    v.rows = rd32(v.payload + 40);
    v.cols = rd32(v.payload + 44);
    return v;
}

static inline size_t minz(size_t a, size_t b) { return a < b ? a : b; }

/* outlier term of the 16-row kernels: chpe_engine.zig:244-257, :309-315 */
static void outlier_x(const cell_view *c, const float *x, size_t x_len, float xo[8]) {
    for (int k = 0; k < 8; k++) {
        uint16_t col = rd16(c->payload + 816 + 2 * k);
        xo[k] = col < x_len ? x[col] : 0.0f;
    }
}
static float outlier_row(const cell_view *c, size_t r, const float xo[8]) {
    float p[8];
    for (int k = 0; k < 8; k++) p[k] = oref_f16_to_f32(rd16(c->payload + 560 + 2 * (r * 8 + k))) * xo[k];
    return reduce8(p);
}

static void gemv_w2(const uint8_t *cell, const float *x, size_t x_len, float *y, size_t y_len,
                    size_t row_base, int accumulate) { /* gemvTileW2: chpe_engine.zig:223-323 */
    cell_view c = view_cell(cell);
    size_t rows = c.rows, cols = c.cols;
    int has_g = (c.custom_flags & FLAG_GROUP128) != 0;
    int has_o = has_g && rows == 16;
    float xo[8] = {0};
    if (has_o) outlier_x(&c, x, x_len, xo);
    size_t max_rows = row_base >= y_len ? 0 : minz(rows, y_len - row_base);
    size_t n_groups = minz(cols / 128, x_len / 128), total_groups = cols / 128;
    for (size_t r = 0; r < max_rows; r++) {
        float row_sum = 0.0f;
        size_t rbo = r * (cols / 4);
        if (has_g) {
            for (size_t g = 0; g < n_groups; g++) {
                float scale = oref_f16_to_f32(rd16(c.payload + 48 + 2 * (r * total_groups + g)));
                const uint8_t *gb = c.codes + rbo + g * 32;
                const float *xs = x + g * 128;
                float dv[8] = {0};
                for (size_t j = 0; j < 32; j += 2) {
                    uint8_t b0 = gb[j], b1 = gb[j + 1];
                    float qv[8] = {CODEBOOK_W2[b0 & 3], CODEBOOK_W2[(b0 >> 2) & 3],
                                   CODEBOOK_W2[(b0 >> 4) & 3], CODEBOOK_W2[(b0 >> 6) & 3],
                                   CODEBOOK_W2[b1 & 3], CODEBOOK_W2[(b1 >> 2) & 3],
                                   CODEBOOK_W2[(b1 >> 4) & 3], CODEBOOK_W2[(b1 >> 6) & 3]};
                    for (int k = 0; k < 8; k++) dv[k] = dv[k] + qv[k] * xs[4 * j + k];
                }
                row_sum += reduce8(dv) * scale;
            }
        } else {
            size_t max_quads = minz(cols / 4, x_len / 4);
            for (size_t b = 0; b < max_quads; b++) {
                uint8_t bv = c.codes[rbo + b];
                float w0 = CODEBOOK_W2[bv & 3] * c.scale + c.bias;
                float w1 = CODEBOOK_W2[(bv >> 2) & 3] * c.scale + c.bias;
                float w2 = CODEBOOK_W2[(bv >> 4) & 3] * c.scale + c.bias;
                float w3 = CODEBOOK_W2[(bv >> 6) & 3] * c.scale + c.bias;
                size_t base = b * 4;
                row_sum += w0 * x[base] + w1 * x[base + 1] + w2 * x[base + 2] + w3 * x[base + 3];
            }
        }
        if (has_o) row_sum += outlier_row(&c, r, xo);
        if (accumulate) y[row_base + r] += row_sum; else y[row_base + r] = row_sum;
    }
}

static void gemv_w4(const uint8_t *cell, const float *x, size_t x_len, float *y, size_t y_len,
                    size_t row_base, int accumulate) { /* gemvTileW4: chpe_engine.zig:326-418 */
    cell_view c = view_cell(cell);
    size_t rows = c.rows, cols = c.cols;
    int has_g = (c.custom_flags & FLAG_GROUP128) != 0;
    int has_o = has_g && rows == 16;
    float xo[8] = {0};
    if (has_o) outlier_x(&c, x, x_len, xo);
    size_t max_rows = row_base >= y_len ? 0 : minz(rows, y_len - row_base);
    for (size_t r = 0; r < max_rows; r++) {
        float row_sum = 0.0f;
        size_t rbo = r * (cols / 2);
        if (has_g) {
            size_t n_groups = minz(cols / 128, x_len / 128), total_groups = cols / 128;
            for (size_t g = 0; g < n_groups; g++) {
                float scale = oref_f16_to_f32(rd16(c.payload + 48 + 2 * (r * total_groups + g)));
                const uint8_t *gb = c.codes + rbo + g * 64;
                const float *xs = x + g * 128;
                float group_acc = 0.0f;
                for (size_t j = 0; j < 64; j += 4)
                    for (size_t idx = 0; idx < 4; idx++) {
                        uint8_t bv = gb[j + idx];
                        float q0 = (float)(bv & 0x0F) - 8.0f, q1 = (float)((bv >> 4) & 0x0F) - 8.0f;
                        size_t base = (j + idx) * 2;
                        group_acc += q0 * xs[base] + q1 * xs[base + 1];
                    }
                row_sum += group_acc * scale;
            }
        } else {
            size_t max_pairs = minz(cols / 2, x_len / 2);
            for (size_t b = 0; b < max_pairs; b++) {
                uint8_t bv = c.codes[rbo + b];
                int n0 = (int)(bv & 0x0F) - 8, n1 = (int)((bv >> 4) & 0x0F) - 8;
                float w0 = (float)n0 * c.scale + c.bias, w1 = (float)n1 * c.scale + c.bias;
                size_t base = b * 2;
                row_sum += w0 * x[base] + w1 * x[base + 1];
            }
        }
        if (has_o) row_sum += outlier_row(&c, r, xo);
        if (accumulate) y[row_base + r] += row_sum; else y[row_base + r] = row_sum;
    }
}

static void gemv_w8(const uint8_t *cell, const float *x, size_t x_len, float *y, size_t y_len,
                    size_t row_base, int accumulate) { /* gemvTileW8: chpe_engine.zig:421-472 */
    cell_view c = view_cell(cell);
    size_t rows = c.rows, cols = c.cols;
    size_t max_rows = row_base >= y_len ? 0 : minz(rows, y_len - row_base);
    size_t max_cols = minz(cols, x_len);
    for (size_t r = 0; r < max_rows; r++) {
        const int8_t *rw = (const int8_t *)(c.codes + r * cols);
        float acc[8] = {0};
        size_t i = 0;
        for (; i + 8 <= max_cols; i += 8)
            for (int k = 0; k < 8; k++) acc[k] = acc[k] + (float)rw[i + k] * x[i + k];
        float row_sum = reduce8(acc);
        for (; i < max_cols; i++) row_sum += (float)rw[i] * x[i];
        float final_val = row_sum * c.scale + c.bias;
        if (accumulate) y[row_base + r] += final_val; else y[row_base + r] = final_val;
    }
}

static void gemv_f16(const uint8_t *cell, const float *x, size_t x_len, float *y, size_t y_len,
                     size_t row_base, int accumulate) { /* gemvTileF16: chpe_engine.zig:475-541 */
    cell_view c = view_cell(cell);
    size_t rows = c.rows, cols = c.cols;
    int ieee = (c.custom_flags & FLAG_RAW_FP16) != 0;
    size_t max_rows = row_base >= y_len ? 0 : minz(rows, y_len - row_base);
    size_t max_cols = minz(cols, x_len);
    for (size_t r = 0; r < max_rows; r++) {
        const uint8_t *rw = c.codes + 2 * r * cols;
        float acc[8] = {0};
        size_t i = 0;
        for (; i + 8 <= max_cols; i += 8)
            for (int k = 0; k < 8; k++) {
                uint16_t h = rd16(rw + 2 * (i + k));
                float w = ieee ? oref_f16_to_f32(h) : oref_bf16_to_f32(h);
                acc[k] = fmaf(w, x[i + k], acc[k]);
            }
        float sum = reduce8(acc);
        for (; i < max_cols; i++) {
            uint16_t h = rd16(rw + 2 * i);
            sum += (ieee ? oref_f16_to_f32(h) : oref_bf16_to_f32(h)) * x[i];
        }
        if (accumulate) y[row_base + r] += sum; else y[row_base + r] = sum;
    }
}

static void gemv_f32(const uint8_t *cell, const float *x, size_t x_len, float *y, size_t y_len,
                     size_t row_base, int accumulate) { /* gemvTileF32: chpe_engine.zig:544-581 */
    cell_view c = view_cell(cell);
    size_t rows = c.rows, cols = c.cols;
    size_t max_rows = row_base >= y_len ? 0 : minz(rows, y_len - row_base);
    size_t max_cols = minz(cols, x_len);
    for (size_t r = 0; r < max_rows; r++) {
        const uint8_t *rw = c.codes + 4 * r * cols;
        float acc[8] = {0};
        size_t i = 0;
        for (; i + 8 <= max_cols; i += 8)
            for (int k = 0; k < 8; k++) acc[k] = fmaf(rdf32(rw + 4 * (i + k)), x[i + k], acc[k]);
        float sum = reduce8(acc);
        for (; i < max_cols; i++) sum += rdf32(rw + 4 * i) * x[i];
        if (accumulate) y[row_base + r] += sum; else y[row_base + r] = sum;
    }
}

void oref_gemv_tile_polymorphic(const uint8_t *cell, const float *x, size_t x_len, float *y,
                                size_t y_len, size_t row_base, int accumulate) {
    /* gemvTilePolymorphic: chpe_engine.zig:732-751 (unknown bits fall back to W2) */
    switch (cell[PAYLOAD_OFF + 20]) {
    case 4: gemv_w4(cell, x, x_len, y, y_len, row_base, accumulate); break;
    case 8: gemv_w8(cell, x, x_len, y, y_len, row_base, accumulate); break;
    case 16: gemv_f16(cell, x, x_len, y, y_len, row_base, accumulate); break;
    case 32: gemv_f32(cell, x, x_len, y, y_len, row_base, accumulate); break;
    default: gemv_w2(cell, x, x_len, y, y_len, row_base, accumulate); break;
    }
}

/* flat outliers REPLACE weights: chpe_engine.zig:632-646 (same for 2-bit, :681-693) */
static void flat_outliers(const cell_view *c, size_t wpt, float *tw) {
    uint16_t n = rd16(c->payload + 560);
    if (n > 0 && n <= 64)
        for (size_t m = 0; m < n; m++) {
            uint16_t off = rd16(c->payload + 690 + 2 * m);
            if (off < wpt) tw[off] = oref_f16_to_f32(rd16(c->payload + 562 + 2 * m));
        }
}

void oref_flat_tile_weights(const uint8_t *cell, size_t wpt, float *tw) {
    /* dequant half of gemvCellFlat: chpe_engine.zig:598-699 (tw holds 32768 floats) */
    cell_view c = view_cell(cell);
    int has_g = (c.custom_flags & FLAG_GROUP128) != 0;
    if (c.quant_bits == 4) {
        if (has_g) {
            for (size_t g = 0; g < 256; g++) {
                float scale = oref_f16_to_f32(rd16(c.payload + 48 + 2 * g));
                for (size_t k = 0; k < 64; k++) {
                    uint8_t b = c.codes[g * 64 + k];
                    float q0 = (float)(b & 0x0F) - 8.0f, q1 = (float)((b >> 4) & 0x0F) - 8.0f;
                    tw[g * 128 + k * 2] = q0 * scale;
                    tw[g * 128 + k * 2 + 1] = q1 * scale;
                }
            }
        } else {
            for (size_t k = 0; k < wpt / 2; k++) {
                uint8_t b = c.codes[k];
                float q0 = (float)(b & 0x0F) - 8.0f, q1 = (float)((b >> 4) & 0x0F) - 8.0f;
                tw[k * 2] = q0 * c.scale + c.bias;
                tw[k * 2 + 1] = q1 * c.scale + c.bias;
            }
        }
        flat_outliers(&c, wpt, tw);
    } else if (c.quant_bits == 2) {
        if (has_g) {
            for (size_t g = 0; g < 256; g++) {
                float scale = oref_f16_to_f32(rd16(c.payload + 48 + 2 * g));
                for (size_t k = 0; k < 32; k++) {
                    uint8_t b = c.codes[g * 32 + k];
                    for (int s = 0; s < 4; s++) tw[g * 128 + k * 4 + s] = CODEBOOK_W2[(b >> (2 * s)) & 3] * scale;
                }
            }
        } else {
            for (size_t k = 0; k < wpt / 4; k++) {
                uint8_t b = c.codes[k];
                for (int s = 0; s < 4; s++) tw[k * 4 + s] = CODEBOOK_W2[(b >> (2 * s)) & 3] * c.scale + c.bias;
            }
        }
        flat_outliers(&c, wpt, tw);
    } else {
        memset(tw, 0, 32768 * sizeof(float));
    }
}

/* dot of one segment of materialised weights: chpe_engine.zig:708-722 */
static float seg_dot(const float *w, const float *x, size_t n) {
    float acc[8] = {0};
    size_t k = 0;
    for (; k + 8 <= n; k += 8)
        for (int i = 0; i < 8; i++) acc[i] = fmaf(w[k + i], x[k + i], acc[i]);
    float dot = reduce8(acc);
    for (; k < n; k++) dot += w[k] * x[k];
    return dot;
}

void oref_gemv_cell_flat(const uint8_t *cell, size_t t, size_t wpt, size_t r_total,
                         size_t c_total, const float *x, float *y) {
    /* gemvCellFlat: chpe_engine.zig:584-729 */
    float *tw = malloc(32768 * sizeof(float));
    oref_flat_tile_weights(cell, wpt, tw);
    size_t j = 0, gws = t * wpt, r = gws / c_total, c = gws % c_total;
    while (j < wpt && r < r_total) {
        size_t seg = minz(wpt - j, c_total - c);
        y[r] += seg_dot(tw + j, x + c, seg);
        j += seg;
        c += seg;
        if (c == c_total) { c = 0; r++; }
    }
    free(tw);
}

int oref_unpack_embed_row_cell(const uint8_t *cell, size_t row, float *out, size_t D) {
    /* unpackEmbedRowCell: chpe_engine.zig:1288-1394 */
    cell_view c = view_cell(cell);
    size_t ng = D / 128;
    if (c.quant_bits == 8) {
        if (row >= 8) return 0;
        const int8_t *rb = (const int8_t *)(c.codes + row * D);
        for (size_t g = 0; g < ng; g++) {
            float scale = oref_f16_to_f32(rd16(c.payload + 48 + 2 * (row * ng + g)));
            for (size_t j = 0; j < 128; j++) out[g * 128 + j] = (float)rb[g * 128 + j] * scale;
        }
        return 1;
    }
    if (c.quant_bits == 2) {
        if (row >= 16) return 0;
        const uint8_t *rb = c.codes + row * (D / 4);
        for (size_t g = 0; g < ng; g++) {
            float scale = oref_f16_to_f32(rd16(c.payload + 48 + 2 * (row * ng + g)));
            for (size_t j = 0; j < 32; j++) {
                uint8_t b = rb[g * 32 + j];
                for (int s = 0; s < 4; s++) out[g * 128 + 4 * j + s] = CODEBOOK_W2[(b >> (2 * s)) & 3] * scale;
            }
        }
    } else if ((c.custom_flags & FLAG_GROUP128) || c.quant_bits == 4) {
        if (row >= 16) return 0;
        const uint8_t *rb = c.codes + row * (D / 2);
        for (size_t g = 0; g < ng; g++) {
            float scale = oref_f16_to_f32(rd16(c.payload + 48 + 2 * (row * ng + g)));
            for (size_t j = 0; j < 64; j++) {
                uint8_t b = rb[g * 64 + j];
                float q0 = (float)(b & 0x0F), q1 = (float)((b >> 4) & 0x0F);
                out[g * 128 + 2 * j] = (q0 - 8.0f) * scale;
                out[g * 128 + 2 * j + 1] = (q1 - 8.0f) * scale;
            }
        }
    } else {
        const uint8_t *rb = c.codes + row * (D / 2);
        for (size_t j = 0; j < D / 2; j++) {
            uint8_t b = rb[j];
            float q0 = (float)(b & 0x0F), q1 = (float)((b >> 4) & 0x0F);
            out[2 * j] = (q0 - 8.0f) * c.scale + c.bias;
            out[2 * j + 1] = (q1 - 8.0f) * c.scale + c.bias;
        }
        return 1;
    }
    if (c.custom_flags & FLAG_GROUP128) /* outliers REPLACE (:1335-1343, :1369-1378) */
        for (int k = 0; k < 8; k++) {
            uint16_t col = rd16(c.payload + 816 + 2 * k);
            if (col < D) out[col] = oref_f16_to_f32(rd16(c.payload + 560 + 2 * (row * 8 + k)));
        }
    return 1;
}

/* ---------------------------------------------------------------- attention */
void oref_attention(const float *q, const float *kc, const float *vc, size_t pos, size_t H,
                    size_t KV, size_t hd, float *scores_all, float *out) {
    /* inline GQA attention: chpe_engine.zig:1699-1734 (heads are independent) */
    size_t gqa = H / KV, kvd = KV * hd;
    float scale = 1.0f / sqrtf((float)hd);
#pragma omp parallel for schedule(static)
    for (size_t qh = 0; qh < H; qh++) {
        size_t kv_h = qh / gqa;
        const float *qs = q + qh * hd;
        float *scores = scores_all + qh * (pos + 1);
        float max_score = -1e30f;
        for (size_t t = 0; t <= pos; t++) {
            const float *ks = kc + t * kvd + kv_h * hd;
            float dot = 0.0f;
            for (size_t d = 0; d < hd; d++) dot += qs[d] * ks[d];
            float s = dot * scale;
            scores[t] = s;
            if (s > max_score) max_score = s;
        }
        float sum_exp = 0.0f;
        for (size_t t = 0; t <= pos; t++) {
            float e = expf(scores[t] - max_score);
            scores[t] = e;
            sum_exp += e;
        }
        float inv_sum = 1.0f / sum_exp;
        float *os = out + qh * hd;
        memset(os, 0, hd * sizeof(float));
        for (size_t t = 0; t <= pos; t++) {
            float alpha = scores[t] * inv_sum;
            const float *vs = vc + t * kvd + kv_h * hd;
            for (size_t d = 0; d < hd; d++) os[d] += alpha * vs[d];
        }
    }
}

/* ---------------------------------------------------------------- engine */
struct oref_engine {
    oref_arch arch;
    const uint8_t *bytes;
    size_t len, map_len;
    int owns_map;
    int archive_valid, is_dense, is_raw, is_raw_fp16, map;
    uint8_t quant_bits;
    size_t record_count, stride, wpt, max_seq_len;
    int kv_f16, threads;
    int no_break;  /* test only: skip forwardDecode's non-finite break (a planted deviation) */
    int hybrid;    /* the true Qwen3.5-9B hybrid layers (oref_set_hybrid) */
    float *conv_state, *rec_state, *hy_mix, *hy_conv, *hy_z, *hy_a, *hy_b, *hy_dn, *hy_qg;
    float *hidden, *norm_buf, *norm_gamma, *bias_buf, *q_buf, *k_buf, *v_buf, *attn_out, *gate_buf,
        *up_buf, *mlp_buf, *scores_buf, *logits_buf, *k_cache, *v_cache;
};

static const uint8_t *tile_coded_ptr(const oref_engine *e, size_t idx) {
    /* getTileCodedPtr: chpe_engine.zig:994-1005 */
    if (e->is_raw) return e->bytes + HEADER_BYTES + idx * TILE_CODE_BYTES;
    if (e->is_dense) return e->bytes + HEADER_BYTES + idx * CELL_BYTES + BYTECODE_HEADER;
    return e->bytes + HEADER_BYTES + idx * RECORD_BYTES + PREFETCH_BYTES + BYTECODE_HEADER;
}
static const uint8_t *cell_ptr(const oref_engine *e, size_t idx) {
    /* getCellPointer: chpe_engine.zig:1007-1011 */
    size_t off = HEADER_BYTES + idx * e->stride;
    return e->bytes + (e->is_dense ? off : off + PREFETCH_BYTES);
}

static int engine_init(oref_engine *e, int arch_id, size_t max_seq_len, int kv_f16, int threads) {
    /* CHPEEngine.init: chpe_engine.zig:854-974 */
    if (oref_arch_preset(arch_id, &e->arch)) return -1;
    const uint8_t *b = e->bytes;
    e->quant_bits = 2;
    if (e->len >= 4096) {
        uint32_t magic = rd32(b);
        if (magic == CHPE_MAGIC || magic == ARCHIVE_MAGIC) {
            e->archive_valid = 1;
            e->record_count = (size_t)rd64(b + 16);
            uint64_t rec_b = rd64(b + 32), cell_b = rd64(b + 40), pre_b = rd64(b + 48), flags = rd64(b + 56);
            e->is_dense = pre_b == 0 && rec_b == cell_b && rec_b == CELL_BYTES;
            e->is_raw = rec_b == TILE_CODE_BYTES;
            e->is_raw_fp16 = e->is_raw && (flags & FLAG_RAW_FP16);
            if (e->is_raw_fp16) {
                e->quant_bits = 16;
            } else if (e->is_raw) {
                size_t gib = 1024ull * 1024ull * 1024ull;
                if (arch_id == 1 && ((flags & 0x08) || (e->len < 10 * gib && e->len > 7 * gib)))
                    e->quant_bits = 8;
                else
                    e->quant_bits = 16;
            } else if (e->record_count > 0 &&
                       e->len >= 4096 + (e->is_dense ? CELL_BYTES : RECORD_BYTES)) {
                size_t cell_off = 4096 + (e->is_dense ? 0 : PREFETCH_BYTES);
                e->quant_bits = b[cell_off + PAYLOAD_OFF + 20];
                if (e->quant_bits == 0) e->quant_bits = 2;
            }
        }
    }
    e->stride = e->is_raw ? TILE_CODE_BYTES : (e->is_dense ? CELL_BYTES : RECORD_BYTES);
    if (e->is_raw_fp16 || (e->is_raw && e->quant_bits == 16)) e->wpt = 8192;
    else if (e->quant_bits == 8) e->wpt = 16384;
    else if (e->quant_bits == 4 || e->quant_bits == 2) e->wpt = 32768;
    else e->wpt = 8192;
    e->map = e->arch.hidden_dim == 2048 ? (e->is_raw ? 0 : 1) : (e->arch.hidden_dim == 8192 ? 3 : 2);
    e->max_seq_len = max_seq_len;
    e->kv_f16 = kv_f16;
    e->threads = threads;
    const oref_arch *a = &e->arch;
    size_t D = a->hidden_dim, I = a->intermediate_dim, qd = a->num_attn_heads * a->head_dim,
           kvd = a->num_kv_heads * a->head_dim;
    size_t mp = D > qd ? D : qd;
    if (I > mp) mp = I;
    e->hidden = calloc(D, 4); e->norm_buf = calloc(D, 4); e->norm_gamma = calloc(D, 4);
    e->bias_buf = calloc(mp, 4); e->q_buf = calloc(qd, 4); e->k_buf = calloc(kvd, 4);
    e->v_buf = calloc(kvd, 4); e->attn_out = calloc(D > qd ? D : qd, 4); e->gate_buf = calloc(I, 4);
    e->up_buf = calloc(I, 4); e->mlp_buf = calloc(I, 4);
    e->scores_buf = calloc(a->num_attn_heads * (max_seq_len + 1), 4);
    e->logits_buf = calloc(a->vocab_size, 4);
    e->k_cache = calloc(a->num_layers * max_seq_len * kvd, 4);
    e->v_cache = calloc(a->num_layers * max_seq_len * kvd, 4);
    if (!e->hidden || !e->scores_buf || !e->logits_buf || !e->k_cache || !e->v_cache) return -1;
    return 0;
}

static void set_threads(const oref_engine *e) {
#ifdef _OPENMP
    if (e->threads > 0) omp_set_num_threads(e->threads);
#else
    (void)e;
#endif
}

void oref_set_threads(oref_engine *e, int threads) { e->threads = threads; }

/* Test only: with on == 0 the layer loop never breaks (:1763 removed) -- the deviation a test
 * plants to show that its comparison tells the break from its absence. */
void oref_set_break(oref_engine *e, int on) { e->no_break = on ? 0 : 1; }

oref_engine *oref_open_bytes(const uint8_t *bytes, size_t len, int arch_id, size_t max_seq_len,
                             int kv_f16, int threads) {
    oref_engine *e = calloc(1, sizeof *e);
    e->bytes = bytes;
    e->len = len;
    if (engine_init(e, arch_id, max_seq_len, kv_f16, threads)) { oref_close(e); return NULL; }
    return e;
}

oref_engine *oref_open(const char *path, int arch_id, size_t max_seq_len, int kv_f16, int threads,
                       int *err) {
    /* WeightArchive.openPosix + validate: weight_archive.zig:184-222 */
    if (err) *err = -1;
    int fd = open(path, O_RDONLY);
    if (fd < 0) return NULL;
    struct stat st;
    if (fstat(fd, &st) != 0 || (size_t)st.st_size < HEADER_BYTES) {
        if (err) *err = 1;
        close(fd);
        return NULL;
    }
    size_t len = (size_t)st.st_size, map_len = len + MAP_PAD;
    /* reserve len + pad zero bytes, then map the file over the front: reads that the
     * reference would make past the end of a record stay inside the mapping */
    uint8_t *base = mmap(NULL, map_len, PROT_READ, MAP_PRIVATE | MAP_ANONYMOUS, -1, 0);
    if (base == MAP_FAILED) { close(fd); return NULL; }
    if (mmap(base, len, PROT_READ, MAP_PRIVATE | MAP_FIXED, fd, 0) == MAP_FAILED) {
        munmap(base, map_len);
        close(fd);
        return NULL;
    }
    close(fd);
    madvise(base, len, MADV_SEQUENTIAL);
    madvise(base, len, MADV_WILLNEED);
    int v = oref_validate(base, len);
    if (v) {
        if (err) *err = v;
        munmap(base, map_len);
        return NULL;
    }
    if (arch_id < 0) arch_id = oref_arch_from_path(path);
    oref_engine *e = oref_open_bytes(base, len, arch_id, max_seq_len, kv_f16, threads);
    if (!e) { munmap(base, map_len); return NULL; }
    e->owns_map = 1;
    e->map_len = map_len;
    if (err) *err = 0;
    return e;
}

void oref_close(oref_engine *e) {
    if (!e) return;
    free(e->hidden); free(e->norm_buf); free(e->norm_gamma); free(e->bias_buf); free(e->q_buf);
    free(e->k_buf); free(e->v_buf); free(e->attn_out); free(e->gate_buf); free(e->up_buf);
    free(e->mlp_buf); free(e->scores_buf); free(e->logits_buf); free(e->k_cache); free(e->v_cache);
    free(e->conv_state); free(e->rec_state); free(e->hy_mix); free(e->hy_conv); free(e->hy_z);
    free(e->hy_a); free(e->hy_b); free(e->hy_dn); free(e->hy_qg);
    if (e->owns_map) munmap((void *)e->bytes, e->map_len);
    free(e);
}

const float *oref_logits(const oref_engine *e) { return e->logits_buf; }
const float *oref_hidden(const oref_engine *e) { return e->hidden; }
size_t oref_vocab(const oref_engine *e) { return e->arch.vocab_size; }
size_t oref_hidden_dim(const oref_engine *e) { return e->arch.hidden_dim; }
void oref_engine_info(const oref_engine *e, int64_t o[8]) {
    o[0] = e->is_raw; o[1] = e->is_raw_fp16; o[2] = e->is_dense; o[3] = e->quant_bits;
    o[4] = (int64_t)e->wpt; o[5] = (int64_t)e->record_count; o[6] = e->archive_valid; o[7] = e->map;
}

void oref_unpack_norm(oref_engine *e, size_t tile, float *out, size_t n) {
    /* unpackNorm: chpe_engine.zig:1144-1170 */
    if (!e->archive_valid || tile >= e->record_count) {
        for (size_t i = 0; i < n; i++) out[i] = 1.0f;
        return;
    }
    const uint8_t *p = tile_coded_ptr(e, tile);
    if (e->arch.hidden_dim == 4096 && e->is_raw)
        for (size_t i = 0; i < n; i++) out[i] = oref_bf16_to_f32(rd16(p + 2 * i));
    else
        memcpy(out, p, n * 4);
    int all_zero = 1;
    for (size_t i = 0; i < n; i++) {
        if (!isfinite(out[i])) {
            for (size_t k = 0; k < n; k++) out[k] = 1.0f;
            return;
        }
        if (out[i] != 0.0f) all_zero = 0;
    }
    if (all_zero)
        for (size_t i = 0; i < n; i++) out[i] = 1.0f;
}

void oref_unpack_bias(oref_engine *e, size_t tile, float *out, size_t n) {
    /* unpackBias: chpe_engine.zig:1172-1192 */
    if (!e->archive_valid || tile >= e->record_count) {
        memset(out, 0, n * 4);
        return;
    }
    const uint8_t *p = tile_coded_ptr(e, tile);
    if (e->arch.hidden_dim == 4096 && e->is_raw)
        for (size_t i = 0; i < n; i++) out[i] = oref_bf16_to_f32(rd16(p + 2 * i));
    else
        memcpy(out, p, n * 4);
    for (size_t i = 0; i < n; i++)
        if (!isfinite(out[i])) out[i] = 0.0f;
}

/* dotSegment, raw branches: chpe_engine.zig:1194-1251 (the cell branches below
 * :1252 are unreachable: gemvLinear returns before the raw loop for cells) */
static float dot_segment(const oref_engine *e, const uint8_t *tp, size_t j, size_t n, const float *x) {
    float acc[8] = {0};
    size_t k = 0;
    if (e->is_raw_fp16) {
        const uint8_t *s = tp + 2 * j;
        for (; k + 8 <= n; k += 8)
            for (int i = 0; i < 8; i++) acc[i] = fmaf(oref_f16_to_f32(rd16(s + 2 * (k + i))), x[k + i], acc[i]);
        float sum = reduce8(acc);
        for (; k < n; k++) sum += oref_f16_to_f32(rd16(s + 2 * k)) * x[k];
        return sum;
    }
    if (e->quant_bits == 8) {
        const int8_t *s = (const int8_t *)tp + j;
        for (; k + 8 <= n; k += 8)
            for (int i = 0; i < 8; i++) acc[i] = fmaf((float)s[k + i], x[k + i], acc[i]);
        float sum = reduce8(acc);
        for (; k < n; k++) sum += (float)s[k] * x[k];
        return sum * 0.00373708f;
    }
    const uint8_t *s = tp + 2 * j;
    for (; k + 8 <= n; k += 8)
        for (int i = 0; i < 8; i++) acc[i] = fmaf(oref_bf16_to_f32(rd16(s + 2 * (k + i))), x[k + i], acc[i]);
    float sum = reduce8(acc);
    for (; k < n; k++) sum += oref_bf16_to_f32(rd16(s + 2 * k)) * x[k];
    return sum;
}

void oref_gemv_linear(oref_engine *e, size_t tile_start, size_t num_tiles, const float *x,
                      size_t x_len, float *y, size_t y_len, size_t r_total, size_t c_total,
                      int accumulate, int64_t bias_tile) {
    /* gemvLinear: chpe_engine.zig:1396-1489 */
    set_threads(e);
    if (!accumulate) memset(y, 0, r_total * 4);
    if (!e->archive_valid || tile_start >= e->record_count) {
        if (!accumulate)
            for (size_t r = 0; r < r_total; r++) y[r] = 0.01f * (float)((int)(r % 13) - 6);
        return;
    }
    size_t avail = minz(num_tiles, e->record_count - tile_start);
    if (!e->is_raw) {
        if (c_total > 2048) {
            /* flat tiles in parallel; each tile's segment dots are added to y in tile
             * order afterwards, which is the reference's order of additions */
            const size_t wpt = 32768;
            size_t max_segs = wpt / c_total + 2;
            float *dots = malloc(avail * max_segs * sizeof(float));
            size_t *rows = malloc(avail * max_segs * sizeof(size_t));
            int *nseg = calloc(avail, sizeof(int));
#pragma omp parallel
            {
                float *tw = malloc(32768 * sizeof(float));
#pragma omp for schedule(dynamic, 16)
                for (size_t t = 0; t < avail; t++) {
                    size_t gws = t * wpt, r = gws / c_total, c = gws % c_total, j = 0;
                    if (r >= r_total) continue; /* loop body would not run */
                    oref_flat_tile_weights(cell_ptr(e, tile_start + t), wpt, tw);
                    int ns = 0;
                    while (j < wpt && r < r_total) {
                        size_t seg = minz(wpt - j, c_total - c);
                        dots[t * max_segs + ns] = seg_dot(tw + j, x + c, seg);
                        rows[t * max_segs + ns] = r;
                        ns++;
                        j += seg;
                        c += seg;
                        if (c == c_total) { c = 0; r++; }
                    }
                    nseg[t] = ns;
                }
                free(tw);
            }
            for (size_t t = 0; t < avail; t++)
                for (int s = 0; s < nseg[t]; s++) y[rows[t * max_segs + s]] += dots[t * max_segs + s];
            free(dots); free(rows); free(nseg);
        } else {
            /* 16-row polymorphic cells; row bases are a prefix over dims.rows */
            size_t *rb = malloc((avail + 1) * sizeof(size_t));
            size_t n = 0, row_base = 0;
            for (size_t t = 0; t < avail; t++) {
                if (row_base >= r_total) break;
                uint32_t rows = rd32(cell_ptr(e, tile_start + t) + PAYLOAD_OFF + 40);
                if (rows == 0) break;
                rb[n++] = row_base;
                row_base += rows;
            }
#pragma omp parallel for schedule(dynamic, 4)
            for (size_t t = 0; t < n; t++)
                oref_gemv_tile_polymorphic(cell_ptr(e, tile_start + t), x, x_len, y, y_len, rb[t], accumulate);
            free(rb);
        }
    } else {
        /* raw tiles: rows straddle tiles; each row's segments are added in tile order */
        size_t wpt = e->wpt;
#pragma omp parallel for schedule(static)
        for (size_t r = 0; r < r_total; r++) {
            size_t f0 = r * c_total, f1 = f0 + c_total;
            for (size_t t = f0 / wpt; t < avail && t * wpt < f1; t++) {
                size_t s0 = t * wpt > f0 ? t * wpt : f0, s1 = (t + 1) * wpt < f1 ? (t + 1) * wpt : f1;
                y[r] += dot_segment(e, tile_coded_ptr(e, tile_start + t), s0 - t * wpt, s1 - s0, x + (s0 - f0));
            }
        }
    }
    if (bias_tile >= 0 && (size_t)bias_tile < e->record_count) {
        oref_unpack_bias(e, (size_t)bias_tile, e->bias_buf, r_total);
        for (size_t r = 0; r < r_total; r++) y[r] += e->bias_buf[r];
    }
}

static void synthetic_embed(uint32_t tok, float *out, size_t D) { /* chpe_engine.zig:1493-1498 */
    for (size_t i = 0; i < D; i++) out[i] = 0.05f * (float)((int)((i + tok) % 17) - 8);
}

void oref_unpack_embed_row(oref_engine *e, uint32_t tok, float *out) {
    /* unpackEmbedRow: chpe_engine.zig:1491-1552 */
    size_t D = e->arch.hidden_dim;
    if (!e->archive_valid || e->record_count == 0) { synthetic_embed(tok, out, D); return; }
    if (e->is_raw_fp16 || e->is_raw) {
        size_t per = (e->is_raw_fp16 || e->quant_bits != 8) ? 8192 : 16384;
        size_t rpt = per / D;
        if (rpt > 0) {
            size_t tile = tok / rpt, row = tok % rpt;
            if (tile < e->record_count) {
                const uint8_t *p = tile_coded_ptr(e, tile);
                if (e->is_raw_fp16) {
                    for (size_t i = 0; i < D; i++) out[i] = oref_f16_to_f32(rd16(p + 2 * (row * D + i)));
                } else if (e->quant_bits == 8) {
                    const int8_t *s = (const int8_t *)p + row * D;
                    for (size_t i = 0; i < D; i++) out[i] = (float)s[i] * 0.00373708f;
                } else {
                    for (size_t i = 0; i < D; i++) out[i] = oref_bf16_to_f32(rd16(p + 2 * (row * D + i)));
                }
                return;
            }
        }
    } else {
        size_t tile = tok / 16, row = tok % 16;
        if (tile < e->record_count) {
            oref_unpack_embed_row_cell(cell_ptr(e, tile), row, out, D);
            return;
        }
    }
    synthetic_embed(tok, out, D);
}

static void compute_lm_head(oref_engine *e) {
    /* computeLmHead: chpe_engine.zig:1554-1660 */
    size_t D = e->arch.hidden_dim, V = e->arch.vocab_size;
    float *logits = e->logits_buf;
    const float *xn = e->norm_buf;
    if (!e->archive_valid || e->record_count == 0) {
        for (size_t v = 0; v < V; v++) logits[v] = 0.001f * (float)((int)(v % 13) - 6);
        return;
    }
    int64_t lhs = -1;
    size_t lht = 0;
    if (D == 8192) { lhs = 2181137; lht = 38016; }
    else if (D == 4096) { lhs = 484601; lht = 62080; }
    if (lhs >= 0 && (size_t)lhs < e->record_count) {
        oref_gemv_linear(e, (size_t)lhs, lht, xn, D, logits, V, V, D, 0, -1);
        return;
    }
    set_threads(e);
    if (!e->is_raw) { /* tied embedding cells (:1582-1611) */
        size_t cap = e->record_count;
        size_t *vb = malloc((cap + 1) * sizeof(size_t));
        size_t nc = 0, v = 0;
        for (size_t t = 0; t < cap && v < V; t++) {
            uint32_t rows = rd32(cell_ptr(e, t) + PAYLOAD_OFF + 40);
            vb[nc++] = v;
            v += rows == 0 ? 16 : rows;
        }
#pragma omp parallel
        {
            float *row = calloc(8192 > D ? 8192 : D, sizeof(float)); /* dummy_token_row */
#pragma omp for schedule(dynamic, 8)
            for (size_t t = 0; t < nc; t++) {
                const uint8_t *cell = cell_ptr(e, t);
                uint32_t rows = rd32(cell + PAYLOAD_OFF + 40);
                size_t rpt = rows == 0 ? 16 : rows;
                for (size_t r = 0; r < rpt; r++) {
                    size_t vv = vb[t] + r;
                    if (vv >= V) break;
                    oref_unpack_embed_row_cell(cell, r, row, D); /* stale row if not written */
                    float acc[8] = {0};
                    size_t k = 0;
                    for (; k + 8 <= D; k += 8)
                        for (int i = 0; i < 8; i++) acc[i] = fmaf(xn[k + i], row[k + i], acc[i]);
                    float sum = reduce8(acc);
                    for (; k < D; k++) sum += xn[k] * row[k];
                    logits[vv] = sum;
                }
            }
            free(row);
        }
        free(vb);
        return;
    }
    /* tied embedding in a raw archive (:1613-1659) */
    size_t rpt = 8192 / D;
    if (rpt == 0) rpt = 1;
    size_t tiles = minz(e->record_count, (V + rpt - 1) / rpt);
#pragma omp parallel for schedule(static)
    for (size_t t = 0; t < tiles; t++) {
        const uint8_t *tp = tile_coded_ptr(e, t);
        for (size_t r = 0; r < rpt; r++) {
            size_t v = t * rpt + r;
            if (v >= V) break;
            const uint8_t *rw = tp + 2 * r * D;
            float acc[8] = {0};
            size_t k = 0;
            for (; k + 8 <= D; k += 8)
                for (int i = 0; i < 8; i++) {
                    uint16_t h = rd16(rw + 2 * (k + i));
                    float w = e->is_raw_fp16 ? oref_f16_to_f32(h) : oref_bf16_to_f32(h);
                    acc[i] = fmaf(w, xn[k + i], acc[i]);
                }
            float sum = reduce8(acc);
            for (; k < D; k++) {
                uint16_t h = rd16(rw + 2 * k);
                sum += (e->is_raw_fp16 ? oref_f16_to_f32(h) : oref_bf16_to_f32(h)) * xn[k];
            }
            logits[v] = sum;
        }
    }
}

void oref_compute_lm_head(oref_engine *e, const float *xn, float *logits) {
    /* computeLmHead on a caller's normed hidden state (test hook) */
    memcpy(e->norm_buf, xn, e->arch.hidden_dim * sizeof(float));
    compute_lm_head(e);
    memcpy(logits, e->logits_buf, e->arch.vocab_size * sizeof(float));
}

static float sumsq_seq(const float *v, size_t n) {
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += v[i] * v[i];
    return s;
}

int oref_prefill_synthetic(oref_engine *e, size_t n_pos, uint64_t seed) {
    if (n_pos > e->max_seq_len) return -2;
    const size_t kvd = e->arch.num_kv_heads * e->arch.head_dim;
    for (size_t l = 0; l < e->arch.num_layers; l++)
        for (size_t t = 0; t < n_pos; t++)
            for (size_t i = 0; i < kvd; i++) {
                size_t at = (l * e->max_seq_len + t) * kvd + i;
                uint64_t z = (seed + at) * 0x9E3779B97F4A7C15ull;
                z = (z ^ (z >> 31)) * 0xBF58476D1CE4E5B9ull;
                float k = (float)((z >> 40) & 0xFFFF) / 32768.0f - 1.0f;
                float v = (float)(z >> 48) / 32768.0f - 1.0f;
                if (e->kv_f16) { k = oref_f16_to_f32(f32_to_f16(k)); v = oref_f16_to_f32(f32_to_f16(v)); }
                e->k_cache[at] = k;
                e->v_cache[at] = v;
            }
    return 0;
}

static int forward_layers(oref_engine *e, uint32_t token, size_t pos, size_t n_layers, oref_result *res);

int oref_forward(oref_engine *e, uint32_t token, size_t pos, oref_result *res) {
    return forward_layers(e, token, pos, e->arch.num_layers, res);
}

int oref_forward_layers(oref_engine *e, uint32_t token, size_t pos, size_t n_layers, oref_result *res) {
    /* a timing sample: forwardDecode over the first n_layers layers only */
    return forward_layers(e, token, pos, n_layers < e->arch.num_layers ? n_layers : e->arch.num_layers, res);
}

static int forward_hybrid(oref_engine *e, uint32_t token, size_t pos, size_t n_layers, oref_result *res);

static int forward_layers(oref_engine *e, uint32_t token, size_t pos, size_t n_layers, oref_result *res) {
    /* forwardDecode: chpe_engine.zig:1663-1803 */
    if (e->hybrid) return forward_hybrid(e, token, pos, n_layers, res);
    if (pos >= e->max_seq_len) return -2; /* the reference reads past its KV cache here */
    uint64_t t0 = now_ns();
    set_threads(e);
    const oref_arch *a = &e->arch;
    size_t D = a->hidden_dim, H = a->num_attn_heads, KV = a->num_kv_heads, hd = a->head_dim,
           I = a->intermediate_dim, qd = H * hd, kvd = KV * hd;
    oref_unpack_embed_row(e, token, e->hidden);
    for (size_t l = 0; l < n_layers; l++) {
        oref_layer_info li;
        oref_layer_info_for(e->map, l, &li);
        oref_unpack_norm(e, li.input_norm, e->norm_gamma, D);
        oref_rmsnorm(e->hidden, e->norm_gamma, e->norm_buf, D, a->rms_eps);
        oref_gemv_linear(e, li.q_proj, li.q_tiles, e->norm_buf, D, e->q_buf, qd, qd, D, 0, li.q_bias);
        oref_gemv_linear(e, li.k_proj, li.k_tiles, e->norm_buf, D, e->k_buf, kvd, kvd, D, 0, li.k_bias);
        oref_gemv_linear(e, li.v_proj, li.v_tiles, e->norm_buf, D, e->v_buf, kvd, kvd, D, 0, li.v_bias);
        oref_apply_rope(e->q_buf, pos, H, hd, a->rope_theta);
        oref_apply_rope(e->k_buf, pos, KV, hd, a->rope_theta);
        float *kc = e->k_cache + l * e->max_seq_len * kvd, *vc = e->v_cache + l * e->max_seq_len * kvd;
        for (size_t i = 0; i < kvd; i++) {
            float kk = e->k_buf[i], vv = e->v_buf[i];
            if (e->kv_f16) { kk = oref_f16_to_f32(f32_to_f16(kk)); vv = oref_f16_to_f32(f32_to_f16(vv)); }
            kc[pos * kvd + i] = kk;
            vc[pos * kvd + i] = vv;
        }
        oref_attention(e->q_buf, kc, vc, pos, H, KV, hd, e->scores_buf, e->attn_out);
        oref_gemv_linear(e, li.o_proj, li.o_tiles, e->attn_out, D, e->hidden, D, D, D, 1, -1);
        oref_unpack_norm(e, li.post_norm, e->norm_gamma, D);
        oref_rmsnorm(e->hidden, e->norm_gamma, e->norm_buf, D, a->rms_eps);
        oref_gemv_linear(e, li.gate_proj, li.gate_tiles, e->norm_buf, D, e->gate_buf, I, I, D, 0, -1);
        oref_gemv_linear(e, li.up_proj, li.up_tiles, e->norm_buf, D, e->up_buf, I, I, D, 0, -1);
        for (size_t i = 0; i < I; i++) e->mlp_buf[i] = oref_silu(e->gate_buf[i]) * e->up_buf[i];
        oref_gemv_linear(e, li.down_proj, li.down_tiles, e->mlp_buf, I, e->hidden, D, D, I, 1, -1);
        /* debug-norm block (:1753-1764): only its non-finite break changes results */
        if (l < 3 || (l >= 8 && l <= 16) || !isfinite(e->hidden[0]))
            if (!isfinite(sumsq_seq(e->hidden, D)) && !e->no_break) break;
    }
    oref_unpack_norm(e, oref_final_norm_for(e->map), e->norm_gamma, D);
    oref_rmsnorm(e->hidden, e->norm_gamma, e->norm_buf, D, a->rms_eps);
    compute_lm_head(e);
    float max_logit = -1e30f;
    uint32_t arg = 0;
    int all_finite = 1;
    for (size_t v = 0; v < a->vocab_size; v++) {
        float val = e->logits_buf[v];
        if (!isfinite(val)) all_finite = 0;
        if (val > max_logit) { max_logit = val; arg = (uint32_t)v; }
    }
    float hidden_sq = sumsq_seq(e->hidden, D);
    res->argmax_token = arg;
    res->max_logit = max_logit;
    res->token0_logit = e->logits_buf[0];
    res->elapsed_ns = now_ns() - t0;
    res->hidden_norm = sqrtf(hidden_sq);
    res->all_finite = all_finite;
    return 0;
}

int oref_generate(oref_engine *e, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                  uint32_t *out_tokens, float *top2_gap) {
    /* the reference's caller loop (main.zig:169-184) over the prompt, then greedy
     * feedback of the argmax (the generation loop the reference does not have) */
    if (n_prompt == 0) return -1;
    oref_result r;
    for (size_t p = 0; p < n_prompt; p++)
        if (oref_forward(e, prompt[p], p, &r)) return -2;
    for (size_t i = 0; i < n_gen; i++) {
        out_tokens[i] = r.argmax_token;
        if (top2_gap) {
            float second = -INFINITY;
            for (size_t v = 0; v < e->arch.vocab_size; v++)
                if (v != r.argmax_token && e->logits_buf[v] > second) second = e->logits_buf[v];
            top2_gap[i] = r.max_logit - second;
        }
        if (i + 1 < n_gen && oref_forward(e, r.argmax_token, n_prompt + i, &r)) return -2;
    }
    return 0;
}

/* ---------------------------------------------------------------- the Qwen3.5-9B hybrid
 * The true model of the 9B archive (no reference code: README.md:17,62 only name it; the 9B
 * tensor map names its tensors, qwen35_tensor_map.zig:7-50).  The layer loop keeps
 * forwardDecode's structure (embedding, per layer norm -> token mixer -> residual -> norm ->
 * SwiGLU MLP -> residual, the non-finite break, final norm, LM head, argmax: chpe_engine.zig:
 * 1663-1803); the token mixers follow the library that defines the layer, transformers 5.15.0
 * models/qwen3_5/modeling_qwen3_5.py:
 *   layer l is full attention when l % 4 == 3 (configuration_qwen3_5.py:113-116), else a gated
 *   DeltaNet layer;
 *   full attention (Qwen3_5Attention :629-701): q_proj rows are per head 256 query values then
 *   256 output-gate values (:672-675); RMSNorm of each query and key head (q_norm / k_norm
 *   gains, :677-678); rotary embedding on the first 64 of 256 dims (partial_rotary_factor
 *   0.25, configuration :111; rotate_half pairs (i, i + 32), :546-591) with the reference's
 *   frequency formula (applyRope chpe_engine.zig:195-216 over rot = 64 dims); the KV cache and
 *   attention of forwardDecode (:1693-1734); the output times sigmoid(gate) (:696); o_proj;
 *   gated DeltaNet (Qwen3_5GatedDeltaNet :387-543): in_proj_qkv, in_proj_z, in_proj_a,
 *   in_proj_b; the causal conv1d update + SiLU over the 8192 channels; q, k, v split 2048 /
 *   2048 / 4096; the gated delta rule over 32 value heads (deltanet_oracle.c); the gated
 *   RMSNorm with z; out_proj.
 * Norm tiles hold the effective gain (a converter stores 1 + w for the checkpoints' zero-centred
 * Qwen3_5RMSNorm weights, :720-737).  The recurrent states (conv [24][8192][3], delta rule
 * [24][32][128][128]) start from zero at position 0. */
static int q35_full(size_t l) { return l % 4 == 3; }

typedef struct {
    size_t input_norm, post_norm, gate_proj, up_proj, down_proj;
    size_t q_proj, k_proj, v_proj, o_proj, q_norm, k_norm;
    size_t in_proj_qkv, in_proj_z, in_proj_a, in_proj_b, conv1d, a_log, dt_bias, linear_norm, out_proj;
} q35_records;

static q35_records q35_records_of(size_t l) {
    /* record offsets inside each layer of qwen35_tensor_map.zig:62-1015 */
    q35_records r;
    memset(&r, 0, sizeof r);
    size_t b = 62080;
    for (size_t i = 0; i < l; i++) b += q35_full(i) ? 12804 : 13337;
    r.input_norm = b;
    if (q35_full(l)) {
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

/* n bf16 values from consecutive records' code areas (8192 per record) */
static void q35_bf16_vector(const oref_engine *e, size_t rec, float *out, size_t n) {
    for (size_t i = 0; i < n; i++) {
        const size_t r = rec + i / 8192;
        out[i] = r < e->record_count ? oref_bf16_to_f32(rd16(tile_coded_ptr(e, r) + 2 * (i % 8192))) : 0.0f;
    }
}

/* rotate_half over the first `rot` of hd dims of each head, the reference's angle formula */
static void rope_partial(float *vec, size_t pos, size_t nh, size_t hd, size_t rot, float theta) {
    float pos_f = (float)pos;
    for (size_t h = 0; h < nh; h++) {
        size_t base = h * hd;
        for (size_t i = 0; i < rot / 2; i++) {
            float freq = 1.0f / powf(theta, 2.0f * (float)i / (float)rot);
            float ang = pos_f * freq;
            float c = cosf(ang), s = sinf(ang);
            float x0 = vec[base + i], x1 = vec[base + i + rot / 2];
            vec[base + i] = x0 * c - x1 * s;
            vec[base + i + rot / 2] = x0 * s + x1 * c;
        }
    }
}

int oref_set_hybrid(oref_engine *e, int on) {
    if (!on) { e->hybrid = 0; return 0; }
    if (e->map != 2 || e->is_raw) return -1;  /* the 9B cell archive only */
    const size_t n_lin = 24;
    if (!e->conv_state) {
        e->conv_state = calloc(n_lin * 8192 * 3, 4);
        e->rec_state = calloc(n_lin * 32 * 128 * 128, 4);
        e->hy_mix = calloc(8192, 4); e->hy_conv = calloc(8192, 4); e->hy_z = calloc(4096, 4);
        e->hy_a = calloc(32, 4); e->hy_b = calloc(32, 4); e->hy_dn = calloc(4096, 4); e->hy_qg = calloc(8192, 4);
        if (!e->conv_state || !e->rec_state || !e->hy_qg) return -1;
    }
    e->hybrid = 1;
    return 0;
}

static int forward_hybrid(oref_engine *e, uint32_t token, size_t pos, size_t n_layers, oref_result *res) {
    if (pos >= e->max_seq_len) return -2;
    uint64_t t0 = now_ns();
    set_threads(e);
    const oref_arch *a = &e->arch;
    const size_t D = a->hidden_dim, I = a->intermediate_dim, H = 16, KV = 4, hd = 256, kvd = KV * hd;
    if (pos == 0) {
        memset(e->conv_state, 0, 24 * 8192 * 3 * 4);
        memset(e->rec_state, 0, 24 * 32 * 128 * 128 * 4);
    }
    float gq[256], gk[256], conv_w[8192 * 4], a_log[32], dt_bias[32], lin_norm[128], tmp[256];
    oref_unpack_embed_row(e, token, e->hidden);
    size_t li = 0; /* linear-layer index */
    for (size_t l = 0; l < n_layers; l++) {
        const q35_records r = q35_records_of(l);
        oref_unpack_norm(e, r.input_norm, e->norm_gamma, D);
        oref_rmsnorm(e->hidden, e->norm_gamma, e->norm_buf, D, a->rms_eps);
        if (q35_full(l)) {
            oref_gemv_linear(e, r.q_proj, 2048, e->norm_buf, D, e->hy_qg, 8192, 8192, D, 0, -1);
            oref_gemv_linear(e, r.k_proj, 256, e->norm_buf, D, e->k_buf, kvd, kvd, D, 0, -1);
            oref_gemv_linear(e, r.v_proj, 256, e->norm_buf, D, e->v_buf, kvd, kvd, D, 0, -1);
            q35_bf16_vector(e, r.q_norm, gq, 256);
            q35_bf16_vector(e, r.k_norm, gk, 256);
            for (size_t h = 0; h < H; h++) { /* the query half of each head, RMS-normed */
                oref_rmsnorm(e->hy_qg + h * 512, gq, tmp, hd, a->rms_eps);
                memcpy(e->q_buf + h * hd, tmp, hd * 4);
            }
            for (size_t h = 0; h < KV; h++) {
                oref_rmsnorm(e->k_buf + h * hd, gk, tmp, hd, a->rms_eps);
                memcpy(e->k_buf + h * hd, tmp, hd * 4);
            }
            rope_partial(e->q_buf, pos, H, hd, 64, a->rope_theta);
            rope_partial(e->k_buf, pos, KV, hd, 64, a->rope_theta);
            float *kc = e->k_cache + l * e->max_seq_len * kvd, *vc = e->v_cache + l * e->max_seq_len * kvd;
            for (size_t i = 0; i < kvd; i++) {
                float kk = e->k_buf[i], vv = e->v_buf[i];
                if (e->kv_f16) { kk = oref_f16_to_f32(f32_to_f16(kk)); vv = oref_f16_to_f32(f32_to_f16(vv)); }
                kc[pos * kvd + i] = kk;
                vc[pos * kvd + i] = vv;
            }
            oref_attention(e->q_buf, kc, vc, pos, H, KV, hd, e->scores_buf, e->attn_out);
            for (size_t h = 0; h < H; h++)
                for (size_t d = 0; d < hd; d++) {
                    const float g = e->hy_qg[h * 512 + 256 + d];
                    e->attn_out[h * hd + d] = e->attn_out[h * hd + d] * (1.0f / (1.0f + expf(-g)));
                }
            oref_gemv_linear(e, r.o_proj, 1024, e->attn_out, H * hd, e->hidden, D, D, H * hd, 1, -1);
        } else {
            oref_gemv_linear(e, r.in_proj_qkv, 2048, e->norm_buf, D, e->hy_mix, 8192, 8192, D, 0, -1);
            oref_gemv_linear(e, r.in_proj_z, 1024, e->norm_buf, D, e->hy_z, 4096, 4096, D, 0, -1);
            oref_gemv_linear(e, r.in_proj_a, 8, e->norm_buf, D, e->hy_a, 32, 32, D, 0, -1);
            oref_gemv_linear(e, r.in_proj_b, 8, e->norm_buf, D, e->hy_b, 32, 32, D, 0, -1);
            q35_bf16_vector(e, r.conv1d, conv_w, 8192 * 4);
            q35_bf16_vector(e, r.a_log, a_log, 32);
            q35_bf16_vector(e, r.dt_bias, dt_bias, 32);
            q35_bf16_vector(e, r.linear_norm, lin_norm, 128);
            oref_conv1d_update(8192, 4, e->hy_mix, conv_w, e->conv_state + li * 8192 * 3, e->hy_conv);
            oref_gated_delta_step(32, 16, 128, 128, e->hy_conv, e->hy_conv + 2048, e->hy_conv + 4096, e->hy_a,
                                  e->hy_b, a_log, dt_bias, e->rec_state + li * 32 * 128 * 128, e->hy_dn);
            oref_gated_rmsnorm(32, 128, e->hy_dn, e->hy_z, lin_norm, a->rms_eps, e->attn_out);
            oref_gemv_linear(e, r.out_proj, 1024, e->attn_out, 4096, e->hidden, D, D, 4096, 1, -1);
            li++;
        }
        oref_unpack_norm(e, r.post_norm, e->norm_gamma, D);
        oref_rmsnorm(e->hidden, e->norm_gamma, e->norm_buf, D, a->rms_eps);
        oref_gemv_linear(e, r.gate_proj, 3072, e->norm_buf, D, e->gate_buf, I, I, D, 0, -1);
        oref_gemv_linear(e, r.up_proj, 3072, e->norm_buf, D, e->up_buf, I, I, D, 0, -1);
        for (size_t i = 0; i < I; i++) e->mlp_buf[i] = oref_silu(e->gate_buf[i]) * e->up_buf[i];
        oref_gemv_linear(e, r.down_proj, 3072, e->mlp_buf, I, e->hidden, D, D, I, 1, -1);
        /* forwardDecode's non-finite break (:1753-1764) */
        if (l < 3 || (l >= 8 && l <= 16) || !isfinite(e->hidden[0]))
            if (!isfinite(sumsq_seq(e->hidden, D)) && !e->no_break) break;
    }
    oref_unpack_norm(e, oref_final_norm_for(e->map), e->norm_gamma, D);
    oref_rmsnorm(e->hidden, e->norm_gamma, e->norm_buf, D, a->rms_eps);
    compute_lm_head(e);
    float max_logit = -1e30f;
    uint32_t arg = 0;
    int all_finite = 1;
    for (size_t v = 0; v < a->vocab_size; v++) {
        float val = e->logits_buf[v];
        if (!isfinite(val)) all_finite = 0;
        if (val > max_logit) { max_logit = val; arg = (uint32_t)v; }
    }
    res->argmax_token = arg;
    res->max_logit = max_logit;
    res->token0_logit = e->logits_buf[0];
    res->elapsed_ns = now_ns() - t0;
    res->hidden_norm = sqrtf(sumsq_seq(e->hidden, D));
    res->all_finite = all_finite;
    return 0;
}
