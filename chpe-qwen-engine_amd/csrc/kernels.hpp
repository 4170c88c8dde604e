// kernels.hpp -- argument blocks and launchers of the gfx950 decode kernels.
//
// Each kernel is one stage of CHPEEngine.forwardDecode (src/chpe_engine.zig:1663-1803):
//   embed            unpackEmbedRow                        (:1491-1552, :1288-1394)
//   gemv             gemvLinear / gemvTile* / gemvCellFlat (:1396-1489, :223-729) with the
//                    RMSNorm before it (rmsNorm :163-193) applied to x as it is loaded, and
//                    the bias / residual / SwiGLU / LM-head logits after it in the epilogue
//   attention        RoPE (:195-216) + KV write (:1693-1697) + GQA attention (:1700-1734),
//                    split over the context, then merged by a second launch
//   finish           argmax / all_finite / logits[0] (:1775-1803) and the device-side
//                    advance to the next position
// No kernel communicates between workgroups inside one launch: cross-workgroup reductions
// are separate launches, so no device-scope fence (an L2 write-back + invalidate on this
// multi-die part) is executed anywhere in the step.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

namespace chpe {

// Weight layouts a GEMV launch reads (chosen per tensor by the host plan).
enum class WeightKind : int {
  Raw16 = 0,     // raw archive: contiguous row-major fp16 / bf16 matrix (dotSegment)
  Cell16W4 = 1,  // 16-row cells, 4-bit, GROUP128, rows=16, cols=2048 (gemvTileW4)
  FlatW4 = 2,    // flat 32768-weight tiles, 4-bit, GROUP128 (gemvCellFlat)
  FlatW2 = 3,    // flat tiles, 2-bit, GROUP128
  Cell16Poly = 4,  // 16-row polymorphic cells of any width (gemvTilePolymorphic), per-cell metadata
  Raw8 = 5,        // raw int8 tiles as one row-major matrix, times 0.00373708 (dotSegment :1219-1237)
  FlatPoly = 6,    // flat tiles of any form gemvCellFlat decodes, tile by tile (launch_gemv_flat_poly)
};

enum class GemvMode : int {
  Store = 0,   // y = W x (+ bias)
  Accum = 1,   // y += W x    (o / down projections into the residual stream)
  SwiGlu = 2,  // y = silu(W0 x) * (W1 x)
  Logits = 3,  // logits = W x, plus per-workgroup argmax partials
  QkvRope = 4, // y = W x + bias, then by part role: q rotated (RoPE) into y; k rotated and v
               // stored into the KV cache at the step's position (rounded to the cache type)
};

// kRoleStore: the part's rows stored as computed (no rotation, no KV append) -- the normalised
// input projections of the hybrid layers, whose per-head norms and rotary embedding come after.
// kRoleConv: row c is channel c of the hybrid's depthwise causal conv (RopeArgs::conv_w,
// conv_state): silu(conv over [state, row]) stored, the state shifted (not after a break) -- the
// decode step's in_proj_qkv, with k_dn_conv's arithmetic
enum RopeRole : uint32_t { kRoleQ = 0, kRoleK = 1, kRoleV = 2, kRoleStore = 3, kRoleConv = 4 };
constexpr uint32_t kDnConvTaps = 4;  // the hybrid's conv kernel size (kRoleConv)
// (the conv's weights and state travel in RopeArgs' cache pointers: a launch with a conv part
// has no part that appends a KV row)
struct StepState;

struct RopeArgs {            // QkvRope: applyRope (chpe_engine.zig:195-216) + KV append (:1693-1697)
  StepState* state;          // (also set for the residual launches: StepState::broken)
  const float* cos;          // [head_dim/2]: the step's row of the cos table (staged by k_embed /
  const float* sin;          //   k_finish from the [max_seq][head_dim/2] tables), and of sin
  // this layer: [KV][max_seq][head_dim], f16 or f32; a launch with a kRoleConv part (whose parts
  // append no KV row) holds the conv's [channels][kDnConvTaps] weights here instead
  union {
    void* k_cache;
    const float* conv_w;
  };
  // f32: as k_cache; f16: [KV][max_seq/4][head_dim][4] (4-position blocks); with a kRoleConv
  // part: the conv state [channels][kDnConvTaps - 1], oldest first, shifted in place
  union {
    void* v_cache;
    float* conv_state;
  };
  uint32_t head_dim, max_seq, kv_f16;  // max_seq: cache rows per kv head, a multiple of 16
  uint32_t brk_check;        // the break test this launch makes on its input (see StepState::broken):
                             //   0 none (layer 0), 1 the sum of squares (after layers 0-2 and 8-16),
                             //   2 the first element (after the other layers)
};

constexpr int kMaxParts = 3;
constexpr uint32_t kMaxCorrPerRow = 128;  // flat-tile outliers per output row (two tiles' worth)
constexpr uint32_t kMaxWavesPerUnit = 8;

struct GemvPart {
  const uint8_t* base;        // device address of the tensor's first record
  uint32_t stride;            // record stride in bytes
  uint32_t rows;              // output rows (r_total)
  uint32_t wrows;             // rows the tiles cover (<= rows; FlatW4 only may have fewer): the
                              //   rows past it have no weights (gemvLinear computes only the
                              //   rows its tiles reach), Store / QkvRope give 0 + bias, Accum
                              //   leaves them untouched
  uint32_t unit_begin;        // first work unit of this part
  uint32_t bf16;              // Raw16: 1 = bf16, 0 = fp16
  float* y;                   // output vector
  const float* bias;          // per-row bias (Store), may be null
  const float2* corr;         // Flat: outlier corrections [rows][corr_kmax], zero-padded,
  uint32_t corr_kmax;         //   entry = (column as float bits, w_out - dequantised code)
  uint32_t replace_outliers;  // Cell16W4: outliers replace (tied LM head) instead of add
  uint32_t rope_role;         // QkvRope: RopeRole of this part
  const struct CellReplace* repl;  // Cell16W4 replace mode: per-cell corrections (see below)
  const uint8_t* xcodes;      // Flat tiles on the persistent matrix-core kernel (part 0): the launch's
                              //   codes in that kernel's load order, or null (read from the records)
};

// Replace-mode outliers of one 16-row cell, prepared at load time: entry k replaces column
// col[k] of every row, i.e. adds delta[row][k] = w_out - dequantised code.  Entries that do not
// apply (column out of range, or overridden by a later entry for the same column) have delta 0.
struct CellReplace {
  uint16_t col[8];
  float delta[16][8];
};
static_assert(sizeof(CellReplace) == 528, "");

struct StepResult {  // ForwardResult, src/chpe_engine.zig:803-810 (elapsed measured on the host)
  uint32_t argmax;
  float max_logit;
  float token0_logit;
  float hidden_norm;
  uint32_t all_finite;
  uint32_t pad[3];
};

struct ArgmaxPartial {
  float value;
  uint32_t index;     // 0xffffffff: no candidate
  uint32_t nonfinite;
  uint32_t pad;
};

struct GemvArgs {
  GemvPart part[kMaxParts];
  int n_parts;               // 1; SwiGlu: 2 (gate, up); QkvRope: up to 3 (q, k, v)
  int mode;
  uint32_t C;                // columns (length of x)
  uint32_t n_units;          // row tiles (SwiGlu: a tile is RU/2 gate rows + RU/2 up rows)
  uint32_t n_panels;         // column panels of the layout
  uint32_t waves_per_unit;   // 1, or the K-split width (then one unit per workgroup)
  const float* x;            // input vector (f32)
  const float* gamma;        // RMSNorm gains: x is normalised as it is loaded when non-null
  float eps;
  ArgmaxPartial* partials;   // Logits: one per workgroup
  StepResult* result;        // Logits: workgroup 0 stores the hidden norm
  float* hidden_out;         // Logits (matrix-core kernel): workgroup 0 copies x here when set
  RopeArgs rope;             // QkvRope
};

struct GemvLaunch {  // launch geometry of one GemvArgs
  uint32_t blocks, threads, ru;
  uint32_t cells;  // > 0: the K-split kernel for 16-row cells at 2048 columns, `cells` units per workgroup
  uint32_t flat;   // > 0: the K-split kernel for flat 4-bit tiles, up to `flat` panels per wave
  uint32_t mma;    // > 0: the matrix-core kernel for 16-row cells at 2048 columns, `mma` tiles per workgroup
  uint32_t xs;     // > 0: the input-stationary persistent kernel for flat tiles, `xs` rows per unit
  uint32_t xm;     // > 0: its matrix-core form for flat 4-bit tiles, `xm` rows per unit
};

struct StepState {  // device-resident per-token state read by the captured step
  uint32_t token;
  uint32_t pos;
  uint32_t n_prompt;   // positions teacher-forced from `prompt`
  uint32_t n_steps;
  // forwardDecode's non-finite break (chpe_engine.zig:1753-1764): after layer l the reference
  // leaves the layer loop when the hidden state's sum of squares is not finite, a test it makes
  // after layers 0-2 and 8-16 and whenever hidden[0] is not finite; the final norm and the LM
  // head then see the hidden state of the break.  The q/k/v launch of layer l + 1 makes the test
  // on its input (RopeArgs::brk_check) and sets `broken`; from then on the step's launches write
  // neither the KV cache nor the residual stream.  k_finish clears it for the next step.
  uint32_t broken = 0;
  uint32_t pad[3] = {0, 0, 0};
};

struct EmbedArgs {
  const uint8_t* image;     // archive image base (device), byte 0 = archive byte 0
  uint64_t image_len;       // bytes readable at `image` (archive + zero padding)
  const StepState* state;
  float* hidden;
  uint32_t D;
  int kind;                 // 0 synthetic, 1 raw fp16, 2 raw bf16, 3 raw int8, 4 cell
  uint64_t record_count;
  uint64_t stride;          // record stride
  uint64_t cell_off;        // offset of the cell inside a record
  // the step's RoPE factors: rows `pos` of the [rope_rows][rope_half] cos / sin tables into
  // rope_cur[0, rope_half) / [rope_half, 2 rope_half) (so that the q/k/v launch loads them
  // without waiting for the position)
  const float* rope_cos;
  const float* rope_sin;
  float* rope_cur;
  uint32_t rope_half, rope_rows;
};

struct AttnArgs {
  const StepState* state;
  const float* q;           // [H*hd] rotated queries (the QkvRope GEMV's output)
  const void* k_cache;      // this layer: [KV][max_seq][hd], f16 or f32, rows 0..pos written
  const void* v_cache;      // f32: as k_cache; f16: [KV][max_seq/4][hd][4] (4-position blocks)
  float* out;               // [H*hd]
  float* part_ml;           // [H][n_chunks][2] (chunk max, chunk sum)
  float* part_acc;          // [H][n_chunks][hd]
  uint32_t H, KV, hd, max_seq, n_chunks;  // max_seq: cache rows per kv head, a multiple of 16
  uint32_t chunk;           // positions per chunk: attn_chunk(hd, KV)
  uint32_t kv_f16;
  float scale;              // 1/sqrt(hd)
  uint32_t nq;              // queries of a block step at positions pos .. pos + nq - 1 (rows of q,
                            // out and the partials follow each other); 0 or 1: one query
  const float* gate;        // or null: the merge writes out * sigmoid(g), g the hybrid's output gate
                            //   (query z, head h: gate[z][h][hd + d] of rows [H][2 hd] per query)
};

struct FinishArgs {
  StepState* state;
  const uint32_t* prompt;   // teacher-forced tokens
  const ArgmaxPartial* partials;
  uint32_t n_partials;
  const float* logits;
  StepResult* result;
  uint32_t* out_tokens;     // argmax of every step, indexed by position
  EmbedArgs embed;          // embed_next: the next token's row into embed.hidden (the next step's input)
  uint32_t embed_next;
};

// Workgroup caps of the one-unit-per-wave GEMV (0 = one unit per wave, no cap); the waves of
// a capped grid stride over the remaining units.  Defaults, overridable for measurement by
// CHPE_GEMV_ROWS_BLOCKS / CHPE_GEMV_LOGITS_BLOCKS / CHPE_GEMV_CELLS.
struct GemvTuning {
  uint32_t rows_blocks = 0;
  uint32_t logits_blocks = 2048;
  uint32_t cells = 2;  // units per workgroup of the K-split cell kernel when a launch has >= 2048 units
                       // (1, 2 or 4); CHPE_GEMV_CELLS=0: the one-unit-per-wave kernel instead
  uint32_t flat = 1;   // CHPE_GEMV_FLAT=0: flat 4-bit tiles on the one-workgroup-per-unit K-split by panels
  uint32_t mma = 2;    // 16-row cells at 2048 columns on the matrix-core kernel, 1 or 2 tiles per
                       // workgroup of a launch with >= 1024 tiles (CHPE_GEMV_MMA; 0: off)
  uint32_t mma_logits_blocks = 512;   // persistent workgroups of the matrix-core LM head (2 per CU)
  uint32_t xm = 1;     // flat 4-bit tiles on the matrix-core input-stationary kernel (CHPE_GEMV_XM; 0: off)
  uint32_t xm2 = 1;    // flat 2-bit tiles on it (CHPE_GEMV_XM2; 0: the vector-ALU kernels)
  // its persistent workgroups per CU (CHPE_GEMV_XM_WPC=small,large,logits,wide as below)
  // (small: launches of < 4096 units; in these models only 2-bit ones, whose q/k/v and o ran
  // 0.5 us faster at 3 than at 2)
  uint32_t xm_wpc_small = 3, xm_wpc_large = 3, xm_wpc_logits = 2, xm_wpc_wide = 1;
  // the permuted code copies of the gate/up and LM head launches (xm_layout_bytes;
  // CHPE_XM_LAYOUT=0: the kernel reads the records), and the persistent workgroups per CU of the
  // 4-bit gate/up launches of 4096 units or more at 4 waves (8192 columns) that read such a
  // copy (CHPE_GEMV_XM_WPC_GATEUP; without the copy, and for 2-bit tiles: xm_wpc_large)
  uint32_t xm_layout = 1;
  uint32_t xm_wpc_gateup = 2;
  uint32_t xs = 1;     // flat tiles on the input-stationary persistent kernel (CHPE_GEMV_XS; 0: off)
  // its persistent workgroups per CU (256 CUs): launches of < 4096 units, of more, the LM head,
  // and inputs wider than 8192 columns (CHPE_GEMV_XS_WPC=small,large,logits,wide)
  uint32_t xs_wpc_small = 2, xs_wpc_large = 3, xs_wpc_logits = 6, xs_wpc_wide = 1;
  uint32_t xs_min_units = 4096;  // below this (not the LM head): the older kernels, unless the launch
  uint32_t xm_min_mb = 48;       //   reads at least this many MB of codes (CHPE_GEMV_XM_MIN_MB)
};
const GemvTuning& gemv_tuning();

// Launch geometry: work units, panels and the K-split for a GEMV over `rows[n_parts]` rows of
// C columns; `ru` rows per unit.
GemvLaunch gemv_geometry(WeightKind kind, GemvMode mode, uint32_t C, const uint32_t* rows,
                         int n_parts, uint32_t* n_units, uint32_t* n_panels,
                         uint32_t* waves_per_unit, uint32_t* unit_begin);

// Polymorphic 16-row cells (any of gemvTilePolymorphic's widths, WeightKind::Cell16Poly): the
// cells of one tensor and the first output row of each (the prefix sums of dims.rows), with
// row_base[n_cells] = the rows they cover.
struct PolyPlan {
  const uint32_t* row_base;  // device [n_cells + 1]
  uint32_t n_cells;
};
struct PolyRaw {             // raw row sums per part (device, >= the part's rows each)
  float* y[kMaxParts];
};
constexpr uint32_t kPolyEpilogueBlocks = 64;
// one GEMV over polymorphic cells: the input RMSNorm'ed into xn (when a.gamma is set; xn holds
// C + 1 floats, the last one the input's sum of squares), the raw
// row sums of every part, then the mode's epilogue (a.part[*].y, bias, RoPE / KV append,
// SwiGLU, residual, logits + argmax partials: kPolyEpilogueBlocks of them).  Returns the
// number of argmax partials.
uint32_t launch_gemv_poly(const GemvArgs& a, const PolyPlan* const* plans, float* xn, const PolyRaw& raw,
                          hipStream_t stream);

// Flat tiles of any form (WeightKind::FlatPoly): part p walks n_tiles[p] tiles from its base
// (gemvLinear's available tiles, :1423-1429) over a.part[p].rows x a.C weights; the input
// RMSNorm'ed into xn (C + 1 floats) when a.gamma is set; `part` holds
// flat_poly_part_floats(max n_tiles, C) floats of row-segment sums; then the raw row sums of
// every part and the mode's epilogue as launch_gemv_poly.  Returns the argmax partials' count.
size_t flat_poly_part_floats(uint32_t n_tiles, uint32_t C);
uint32_t launch_gemv_flat_poly(const GemvArgs& a, const uint32_t* n_tiles, float* xn, const PolyRaw& raw,
                               float* part, hipStream_t stream);

// ---- the block step: m <= kMaxBlock tokens at consecutive positions through flat 4- or 2-bit tiles,
// every weight read once for all m tokens (batch-M verify, chunked prefill) ----------------------
constexpr uint32_t kMaxBlock = 32;
constexpr uint32_t kSmallBlock = 8;     // blocks up to this size: k_gemv_mt, token stride 8
constexpr uint32_t kBlockRange = 2048;  // input columns per workgroup of the block GEMV (<= 8 tokens)
constexpr uint32_t kBlockUnit = 16;     // weight rows per unit of the block GEMV

constexpr uint32_t kMaxSsPartials = 4096;  // Σx² partials a block kernel may leave for the next GEMV

// One GEMV input of m tokens as matrix-core operands (k_block_limbs): per token and 128-column
// group the input (RMS-normalised when gamma is set) as exact integers X = x * 2^(30-e), max
// |x| < 2^e, in four signed-byte limbs.  Tokens come in quads T (token 4T + t); nq quads.
struct BlockTables {
  uint4* tb;   // [nq][ng][4 kq][2 h][16]: entry lane 4t + L = limb L of token 4T + t, the 16
               //   columns 32 kq + 16 h .. of the group in the operand byte order
  int4* ci;    // [nq][ng][4]: -8 (4-bit) / -2 (2-bit) * the group's limb sums (limbs 0..3) of token 4T + t
  float* ew;   // [nq][ng][4]: 2^(e - 30) of token 4T + t in the group
  float* xt;   // [C][ts]: the (normalised) input, token-minor (for the outlier corrections)
  float* ss;   // [kMaxBlock]: each token's sum of squares of the raw input (norm GEMVs)
};

// The RMS norm's sum of squares comes as partial sums left by the kernel that wrote the input
// rows (the embedding, an Accum epilogue): ssp[i][t], i < n_ssp, added in a fixed order.
struct BlockGemvArgs {
  GemvArgs g;          // parts, mode, C; g.x = the raw input [m][C], g.gamma; rope: caches and head dim
  BlockTables t;
  uint32_t m, nq;
  uint32_t n_units;    // kBlockUnit-row units over the parts (unit_begin of part p in units)
  uint32_t rows_all;   // kBlockUnit * n_units: rows of the partial-sum buffer
  float* partial;      // [ranges][rows_all][ts]: raw row sums per column range, token-minor
  const float* ssp;    // [n_ssp][kMaxBlock]: partial sums of x^2 of the input rows (with g.gamma)
  uint32_t n_ssp;
  float* ssp_out;      // Accum: [epi_blocks][kMaxBlock] partial sums of y^2 of the updated rows
  const StepState* state;   // position of token 0 (QkvRope)
  const float* rope_cos;    // [rope_rows][head_dim/2] full tables
  const float* rope_sin;
  uint32_t rope_rows;
  ArgmaxPartial* partials;  // Logits: [kMaxBlock][epi_blocks]
  uint32_t epi_blocks;      // set by launch_block_gemv
  uint32_t* brk;            // [kMaxBlock]: token t broke (StepState::broken), cleared by the block's embedding
  uint32_t bits;            // the parts' code width: 4 or 2 (flat tiles)
  uint32_t ranges;          // column ranges of the partial sums (set by launch_block_gemv)
  uint32_t ts;              // token stride of partial and t.xt: kSmallBlock for m <= kSmallBlock
                            // (the verify's few tokens on few cache lines), else kMaxBlock
  // per part, the outlier corrections of the epilogue of more than kSmallBlock tokens: the
  // non-zero entries of g.part[p].corr row after row in entry order, and each row's first entry
  // ([rows + 1]); null when the part has none
  const float2* cpack[kMaxParts];
  const uint32_t* coff[kMaxParts];
};

struct BlockFinishArgs {
  const ArgmaxPartial* partials;  // [kMaxBlock][n_partials]
  uint32_t n_partials, m;
  const float* logits;            // [m][V]
  uint32_t V;
  const float* ss;                // the final-norm input's sums of squares per token
  uint32_t* out_argmax;           // [m]
  StepResult* result;             // the last token's result
};

// embeds m tokens into X [m][D], leaves each row's sum of squares in ssp[0][t] and clears brk[t]
void launch_block_embed(const EmbedArgs& e, const uint32_t* tokens, uint32_t m, float* X, float* ssp,
                        uint32_t* brk, hipStream_t stream);
// the input's operand tables (k_block_limbs), then the block GEMV (k_gemv_mt) and its epilogue;
// launch_block_gemv returns the epilogue's workgroups (Logits / Σy² partials)
void launch_block_limbs(const BlockGemvArgs& a, hipStream_t stream);
uint32_t launch_block_gemv(BlockGemvArgs& a, hipStream_t stream);
// the column ranges (partial sums per output row and token) launch_block_gemv uses for m tokens
// through n_units units of C columns
uint32_t block_gemv_ranges(uint32_t n_units, uint32_t C, uint32_t m);
void launch_block_finish(const BlockFinishArgs& a, hipStream_t stream);

// launchers; all enqueue on `stream` and never synchronise
void launch_embed(const EmbedArgs& a, hipStream_t stream);
void launch_gemv(WeightKind kind, const GemvArgs& a, const GemvLaunch& g, hipStream_t stream);
// The permuted copy of a launch's 4- or 2-bit codes for the persistent matrix-core kernel
// (GemvPart::xcodes): its size in bytes, or 0 where it is not built (another kernel, another
// mode than SwiGlu / Logits, an input that leaves a wave's columns partly empty, 4 GiB or more);
// build_xm_layout enqueues the copy into dst (that many bytes).
size_t xm_layout_bytes(WeightKind kind, const GemvArgs& a, const GemvLaunch& g);
bool build_xm_layout(WeightKind kind, const GemvArgs& a, const GemvLaunch& g, uint8_t* dst, hipStream_t stream);
// Gated-DeltaNet decode step (Qwen3.5 linear-attention layers; deltanet.hip).
constexpr uint32_t kDnMaxTaps = 8;
struct DnConvArgs {         // depthwise causal conv update + SiLU
  const float* x;           // [channels]
  const float* w;           // [channels][taps]
  float* state;             // [channels][taps-1], oldest first; shifted in place
  float* out;               // [channels]
  uint32_t channels, taps;
  const StepState* step;    // or null: after the step's break (StepState::broken) the state stays
};
struct DnStepArgs {         // gated delta rule over the value heads (+ gated RMSNorm)
  const float *q, *k;       // [n_k_heads][head_dim], before the l2 norm
  const float* v;           // [n_v_heads][head_dim]
  const float *a, *b;       // [n_v_heads]: the a / b projections
  const float *A_log, *dt_bias;  // [n_v_heads]
  const float* z;           // [n_v_heads][head_dim] gate of the norm (used when norm_w)
  const float* norm_w;      // [head_dim] or null: then out = S^T q
  float* state;             // [n_v_heads][head_dim][head_dim] f32, updated in place
  float* out;               // [n_v_heads][head_dim]
  uint32_t n_v_heads, n_k_heads;
  float eps;
  const StepState* step;    // or null: after the step's break (StepState::broken) the state stays
};

// A DeltaNet layer's m tokens in order (the block step): conv update + SiLU, the gated delta
// rule and the gated norm per token, each state read once and written once (launch_dn_block).
struct DnBlockArgs {
  const float* x;           // conv input [m][x_stride] (channels used)
  const float* w;           // [channels][taps]
  float* conv_state;        // [channels][taps-1]
  float* conv_out;          // [m][channels]: q [n_k_heads][hd], k, v [n_v_heads][hd] per token
  uint32_t channels, taps, x_stride;
  const float *a, *b;       // [m][ab_stride]
  uint32_t ab_stride;
  const float *A_log, *dt_bias;
  const float* z;           // [m][z_stride]
  uint32_t z_stride;
  const float* norm_w;      // [head_dim]
  float* state;             // [n_v_heads][hd][hd]
  float* out;               // [m][out_stride]
  uint32_t out_stride;
  uint32_t n_v_heads, n_k_heads, head_dim, m;
  float eps;
  const uint32_t* brk;      // [m]: token t broke before this layer (its state updates are skipped)
};
void launch_dn_block(const DnBlockArgs& a, hipStream_t stream);

// The hybrid model's gated full-attention layer around the decode attention kernels
// (transformers' Qwen3_5Attention): per query head the RMS norm (q_norm gains) and the rotary
// embedding of the first `rot` dims (pairs (i, i + rot/2)), into q_out; per kv head the same
// for k (k_norm gains) and both appended to the KV cache at the step's position (as the QkvRope
// epilogue appends them); then, after attention, the output times sigmoid(gate).
struct HybQkArgs {
  const StepState* state;   // position, StepState::broken (no KV append after a break)
  const float* qg;          // [H][2 hd]: per head the query (hd values), then the output gate
  const float* k;           // [KV][hd]
  const float* v;           // [KV][hd]
  const float* q_norm;      // [hd] gains
  const float* k_norm;      // [hd]
  const float* rope_cos;    // [rope_rows][rot/2]
  const float* rope_sin;
  float* q_out;             // [H][hd]
  void* k_cache;            // this layer, as RopeArgs::k_cache / v_cache
  void* v_cache;
  uint32_t H, KV, hd, rot, max_seq, kv_f16, rope_rows;
  float eps;
  // the block step: m tokens at positions pos .. pos + m - 1 (0 or 1: the decode step), the
  // per-token strides of qg, k / v and q_out, and each token's break flag (null: StepState::broken)
  uint32_t m, qg_stride, kv_stride, q_stride;
  const uint32_t* brk;
};
void launch_hyb_qk(const HybQkArgs& a, hipStream_t stream);
bool deltanet_supported(uint32_t n_v_heads, uint32_t n_k_heads, uint32_t head_dim, uint32_t taps);
void launch_dn_conv(const DnConvArgs& a, hipStream_t stream);
void launch_dn_step(const DnStepArgs& a, uint32_t head_dim, hipStream_t stream);

void launch_attention(const AttnArgs& a, hipStream_t stream);  // partial + combine
void launch_attention_partial(const AttnArgs& a, hipStream_t stream);
void launch_attention_combine(const AttnArgs& a, hipStream_t stream);
void launch_finish(const FinishArgs& a, hipStream_t stream);
constexpr uint32_t kAttnMaxChunks = 320;  // chunks of attn_chunk(hd) positions per launch
// device scratch of chpe_attention_noalloc (position + partials), per GPU
constexpr size_t kAttnScratchBytes = size_t(8) << 20;
// positions per attention chunk: 8192 / head_dim (64 at 128, 32 at 256), 128 at head dim 128
// with >= 8 kv heads (the 72B model: enough workgroups per launch at half the partials)
__host__ __device__ constexpr uint32_t attn_chunk_of(uint32_t hd, uint32_t kv) {
  return hd == 128 && kv >= 8 ? 128u : 8192u / hd;
}
inline uint32_t attn_chunk(uint32_t hd, uint32_t kv) { return attn_chunk_of(hd, kv); }
// (hd, query heads per kv head) pairs the attention kernels are built for
bool attention_supported(uint32_t H, uint32_t KV, uint32_t hd);
constexpr uint32_t kMaxLogitsBlocks = 8192;

// Measurement: the next kernel launched by any launcher on this host thread records `start`
// and `stop` when it begins and ends (hipExtLaunchKernelGGL), then the probe is cleared.
struct LaunchProbe {
  hipEvent_t start = nullptr, stop = nullptr;
};
void arm_launch_probe(hipEvent_t start, hipEvent_t stop);
LaunchProbe take_launch_probe();

// Measurement: while on, every launcher on this host thread records the (mangled) name of the
// kernel it would launch, and launches nothing; last_kernel_name() returns the latest one.
void record_kernel_names(bool on);
const char* last_kernel_name();
namespace detail {
extern thread_local bool g_record_names;
extern thread_local const char* g_last_kernel;
}  // namespace detail

// test hooks: dequantise / unpack exactly as the reference materialises weights
void launch_flat_tile_weights(const uint8_t* cell, float* out, hipStream_t stream);
void launch_embed_row_cell(const uint8_t* cell, uint64_t len, uint32_t row, uint32_t D, float* out,
                           int* written, hipStream_t stream);

}  // namespace chpe
