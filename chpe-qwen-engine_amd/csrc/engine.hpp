// engine.hpp -- CHPEEngine for MI355X: the host side of the decode step.
//
// Mirrors the reference engine's interface (src/chpe_engine.zig:820-1804):
//   init(archive bytes, ModelArch, max_seq_len)  -> Engine::create
//   forwardDecode(token, pos) -> ForwardResult    -> Engine::forward
//   logits_buf                                    -> Engine::copy_logits
// The step itself runs on the GPU as one captured hipGraph; the host only writes the
// (token, pos) state and reads back the result.
#pragma once
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "kernels.hpp"
#include "tensor_maps.hpp"

namespace chpe {

struct ModelArch {  // src/chpe_engine.zig:96-146
  int id;           // 0 Qwen2.5-3B, 1 Qwen3.5-9B, 2 Qwen2.5-72B
  const char* name;
  size_t hidden_dim, intermediate_dim, num_layers, num_attn_heads, num_kv_heads, head_dim, vocab_size;
  float rope_theta, rms_eps;
};
bool arch_preset(int id, ModelArch* out);
int arch_from_path(const char* path);  // src/chpe_c_api.zig:29-37

struct ForwardResult {  // src/chpe_engine.zig:803-810
  uint32_t argmax_token;
  float max_logit;
  float token0_logit;
  uint64_t elapsed_ns;
  float hidden_norm;
  bool all_finite;
};

struct EngineConfig {
  int arch_id = 0;
  size_t max_seq_len = 2048;
  bool kv_f16 = false;  // fp16 KV cache (the reference keeps f32)
  bool hybrid = false;  // Qwen3.5-9B (arch 1): the true hybrid layers instead of the reference's
                        //   GQA aliasing (HybLayer)
};

// One projection as the GPU computes it (a gemvLinear call of the reference).
struct ProjPlan {
  WeightKind kind = WeightKind::Raw16;
  const uint8_t* base = nullptr;  // device address of the first record
  uint32_t stride = 0;
  uint32_t rows = 0, cols = 0;
  uint32_t wrows = 0;                  // rows the tiles cover; 0 = all (see GemvPart::wrows)
  uint32_t bf16 = 0;
  uint32_t replace_outliers = 0;
  float* bias = nullptr;               // device, with the reference's non-finite -> 0 rule
  float2* corr = nullptr;              // device [rows][corr_kmax] flat-tile outlier corrections
  uint32_t corr_kmax = 0;
  CellReplace* repl = nullptr;         // device, replace-mode outliers of 16-row cells
  float2* bcorr = nullptr;             // device [rows][bcorr_kmax]: a 16-row cell tensor's outliers as
  uint32_t bcorr_kmax = 0;             //   the block step's per-row corrections (plan_block)
  float2* bpack = nullptr;             // device: the non-zero entries of the block step's corrections
  uint32_t* boff = nullptr;            //   (bcorr, else corr) row after row, and each row's first entry
                                       //   [rows + 1] (plan_packed_corrections)
  uint8_t* xcodes = nullptr;           // device, the decode launch's codes in the persistent
                                       //   matrix-core kernel's load order (see xm_layout_bytes);
                                       //   set on the launch's first part, and passed only to
                                       //   launches of the mode and part count it was built for
  GemvMode xcodes_mode = GemvMode::Store;
  int xcodes_parts = 0;
  PolyPlan poly{};                     // Cell16Poly: the cells' row bases; FlatPoly: n_cells = the tiles
};

// The cells of a 16-row-cell tensor (c_total <= 2048) as gemvLinear walks them (:1430-1442):
// row bases are the prefix sums of dims.rows until rows == 0 or r_total is reached.
// *uniform_w4: every cell is a 16 x c_total group-128 4-bit cell and they cover r_total rows.
// *extent (when set): the bytes from the first cell's start that the polymorphic kernel reads.
void walk_cells(const uint8_t* cells, size_t len, size_t stride, size_t n_avail, size_t r_total, size_t c_total,
                std::vector<uint32_t>* row_base, bool* uniform_w4, uint64_t* extent);

// A flat-tile tensor (gemvCellFlat, src/chpe_engine.zig:584-729) of r_total x c_total weights in
// n_tiles cells at cells + t * stride (host bytes, len readable): checks that the tiles are
// uniformly group-128 4- or 2-bit (*kind), and builds the outlier corrections the GPU adds --
// outliers replace weights (:632-646), the last entry for an offset wins -- as a zero-padded
// [r_total][*corr_kmax] table of (column as float bits, w_out - dequantised code); *corr stays
// empty when no tile has outliers.
bool plan_flat_tiles(const uint8_t* cells, size_t len, size_t stride, size_t n_tiles, size_t r_total,
                     size_t c_total, WeightKind* kind, std::vector<float2>* corr, uint32_t* corr_kmax,
                     std::string* err);

// How a flat-tile tensor of r_total x c_total weights over n_avail available tiles runs: on the
// uniform kernels (kind FlatW4 / FlatW2, wrows rows covered, the correction table) when the
// tiles are uniformly group-128 4- or 2-bit, cover whole rows (a short tensor: 4-bit only) and
// keep to kMaxCorrPerRow outliers per row; otherwise kind FlatPoly over n_tiles tiles (any tile
// form gemvCellFlat decodes, partial rows).
struct FlatPlan {
  WeightKind kind = WeightKind::FlatPoly;
  uint32_t n_tiles = 0, wrows = 0, corr_kmax = 0;
  std::vector<float2> corr;
};
void plan_flat(const uint8_t* cells, size_t len, size_t stride, size_t n_avail, size_t r_total, size_t c_total,
               FlatPlan* out);

struct LayerPlan {
  ProjPlan q, k, v, o, gate, up, down;
  float* gamma_in = nullptr;    // device, unpackNorm rules applied
  float* gamma_post = nullptr;
};

// A layer of the Qwen3.5-9B hybrid (EngineConfig::hybrid; no reference code, README.md:17,62):
// layer l % 4 == 3 is gated full attention -- in0 = q_proj (per head 256 query rows, then 256
// output-gate rows), in1 = k_proj, in2 = v_proj, out = o_proj, with q / k norm gains --, the
// others gated DeltaNet -- in0 = in_proj_qkv, in1 = in_proj_z, in2 = in_proj_a, in3 = in_proj_b,
// out = out_proj, with the conv weights [8192][4], A_log, dt_bias [32] and the gated norm's
// gains [128]; `lin` indexes the DeltaNet layers' state buffers.  The MLP and the two norms are
// the LayerPlan's.  Record offsets: qwen35_records (qwen35_tensor_map.zig:62-1015).
struct HybLayer {
  bool full = false;
  ProjPlan in0, in1, in2, in3, out;
  float *q_norm = nullptr, *k_norm = nullptr;
  float *conv_w = nullptr, *A_log = nullptr, *dt_bias = nullptr, *lin_norm = nullptr;
  uint32_t lin = 0;
  // in_proj_a and in_proj_b as one 64-row part (rows 0-31 a, 32-63 b): their tiles copied next
  // to each other at load, so that the in-projections run as one launch (has_ab)
  ProjPlan ab;
  bool has_ab = false;
};

class Engine {
 public:
  // `bytes` must stay valid for the engine's lifetime only during create() (the archive is
  // copied to the GPU).  Returns null and sets *err on failure.
  static std::unique_ptr<Engine> create(const uint8_t* bytes, size_t len, const EngineConfig& cfg,
                                        std::string* err);
  ~Engine();
  Engine(const Engine&) = delete;
  Engine& operator=(const Engine&) = delete;

  // forwardDecode(token, pos): one step, synchronous.  Returns 0, or -2 if pos >= max_seq_len.
  int forward(uint32_t token, size_t pos, ForwardResult* out);
  // positions 0..n-1 teacher-forced (chpe_forward_tokens); result of the last step
  int forward_tokens(const uint32_t* tokens, size_t n, ForwardResult* out);
  // prompt teacher-forced, then n_gen greedy tokens fed back on the device
  int generate(const uint32_t* prompt, size_t n_prompt, size_t n_gen, uint32_t* out_tokens,
               ForwardResult* last);
  // drafts[0..m) at positions pos..pos+m-1, each step teacher-forced (the KV rows at those
  // positions are overwritten); out_argmax[i] = argmax after draft i
  int verify(const uint32_t* drafts, size_t m, size_t pos, uint32_t* out_argmax, ForwardResult* last);
  // the block step: tokens[0..m), m <= kMaxBlock, at positions pos..pos+m-1 through every layer
  // with each weight read once for all m tokens (flat 4-/2-bit archives: block_ready()), each
  // token's arithmetic that of forwardDecode; KV rows pos..pos+m-1 are written;
  // out_argmax[i] = argmax after token i; the last token's logits become copy_logits()'s and
  // its result *last.  The decode state is not touched.  0, -1 bad arguments or no block step
  // for this archive, -2 past max_seq_len, -3 device error.  (verify() and prefill() then leave
  // the decode state where the sequential steps would: the last argmax at pos + m.)
  // head false: no LM head (out_argmax and last must be null; the prefill's blocks before its last)
  int block_forward(const uint32_t* tokens, size_t m, size_t pos, uint32_t* out_argmax, ForwardResult* last,
                    bool head = true);
  bool block_ready() const { return block_ok_; }
  // positions 0..n-1 teacher-forced in blocks of kMaxBlock (prefill); result and logits of
  // the last position; the decode state is left at (argmax of the last, n)
  int prefill(const uint32_t* tokens, size_t n, ForwardResult* out);
  // enqueue n graph launches continuing from the current device state (no sync); -2 and
  // nothing enqueued when the steps would pass max_seq_len
  int launch_steps(size_t n);
  int sync();
  int copy_logits(float* out) const;   // vocab_size floats of the last step
  int copy_hidden(float* out) const;   // hidden_dim floats (the residual stream)
  int read_result(ForwardResult* out) const;

  const ModelArch& arch() const { return arch_; }
  size_t max_seq_len() const { return cfg_.max_seq_len; }
  hipStream_t stream() const { return stream_; }
  bool archive_valid() const { return archive_valid_; }
  int quant_bits() const { return quant_bits_; }
  bool is_raw() const { return is_raw_; }
  size_t record_count() const { return record_count_; }
  const LayerPlan& layer(size_t l) const { return layers_[l]; }
  const ProjPlan& lm_head() const { return lm_head_; }
  // weight + KV bytes the step reads at position `pos` (the roofline numerator)
  double step_bytes(size_t pos) const;
  // re-launch one stage of one layer alone (measurement): 0 = qkv, 1 = o, 2 = gate/up,
  // 3 = down, 4 = LM head, 5 = attention (at the current position)
  int launch_stage(int stage, size_t layer);
  // run n_steps real steps (greedy, continuing from the device state) launched directly, with
  // an event pair around every launch of `stage`; *avg_ms = mean launch duration
  int time_stage_live(int stage, size_t n_steps, double* avg_ms, size_t* launches);
  // bytes one launch of launch_stage(stage, layer) reads from HBM (weights, scales, outliers)
  double stage_bytes(int stage, size_t layer) const;

 private:
  Engine() = default;
  bool init(const uint8_t* bytes, size_t len, const EngineConfig& cfg, std::string* err);
  bool plan_projection(size_t tile_start, size_t num_tiles, size_t r_total, size_t c_total,
                       size_t x_len, size_t y_len, bool accumulate, int64_t bias_tile,
                       ProjPlan* out, std::string* err);
  bool plan_lm_head(std::string* err);
  // the polymorphic paths' buffers (normalised input, raw row sums), and the FlatPoly row-segment
  // sums for a tensor of flat_tiles tiles of C columns
  bool ensure_poly_buffers(uint32_t flat_tiles, uint32_t C);
  float* upload_vector(const std::vector<float>& v);
  void* dev_alloc(size_t bytes);
  void record_step(hipStream_t st);
  void record_step_hybrid(hipStream_t st);    // (record_step's body for EngineConfig::hybrid)
  bool plan_hybrid(std::string* err);          // the HybLayer plans, vectors and state buffers
  void reset_hybrid_state(hipStream_t st);     // zero recurrent states (a step at position 0)
  EmbedArgs embed_args() const;
  int set_state(const StepState& s);  // host-set (token, pos, ...) and the embedding of its token
  void enqueue_qkv(size_t layer, hipStream_t st);
  RopeArgs rope_args(size_t layer) const;
  // one GEMV launch over n parts (outs[i] receives part i); returns the workgroup count
  uint32_t enqueue_gemv(const ProjPlan* const* parts, float* const* outs, int n, GemvMode mode,
                        const float* x, uint32_t C, const float* gamma, hipStream_t st,
                        const RopeArgs* rope = nullptr, const uint32_t* roles = nullptr);
  // the launch arguments and geometry of enqueue_gemv's launch
  GemvLaunch gemv_args(const ProjPlan* const* parts, float* const* outs, int n, GemvMode mode, const float* x,
                       uint32_t C, const float* gamma, const RopeArgs* rope, const uint32_t* roles, GemvArgs* a) const;
  // the permuted code copies of the decode launches that read them (gate/up, the LM head)
  void build_xm_layouts();
  void build_xm_layout_of(ProjPlan* const* parts, int n, GemvMode mode, uint32_t C, const RopeArgs* rope = nullptr,
                          const uint32_t* roles = nullptr);
  AttnArgs attn_args(size_t layer) const;
  double proj_bytes(const ProjPlan& p) const;
  bool plan_block(std::string* err);
  void record_block(uint32_t m, hipStream_t st);  // the block step of m tokens after its inputs
  // gamma set: the input's Σx² comes as n_ss partials in d_bss_; Accum leaves the updated rows'
  // partials there and returns their count (as it returns the Logits partials' count)
  // roles (QkvRope): the parts' RopeRole (null: q, k, v); pair_dim: the row pairing of the
  // QkvRope epilogue when not the head dim (the hybrid's Store launches: 32)
  uint32_t enqueue_block_gemv(const ProjPlan* const* parts, float* const* outs, int n, GemvMode mode,
                              const float* x, uint32_t C, const float* gamma, uint32_t n_ss, uint32_t m,
                              size_t layer, hipStream_t st, const uint32_t* roles = nullptr, uint32_t pair_dim = 0);
  void record_block_hybrid(uint32_t m, hipStream_t st);  // record_block of the hybrid model

 public:
  // run one projection's GEMV on a caller vector (Store mode, bias included): parity hooks
  int debug_gemv(size_t layer, int which, const float* x, float* y);

 private:

  // archive
  const uint8_t* host_bytes_ = nullptr;
  size_t len_ = 0;
  bool archive_valid_ = false, is_dense_ = false, is_raw_ = false, is_raw_fp16_ = false;
  int quant_bits_ = 2;
  size_t record_count_ = 0, stride_ = 0, wpt_ = 0;
  MapKind map_ = MapKind::Qwen3bRaw;
  ModelArch arch_{};
  EngineConfig cfg_{};

  // device memory
  std::vector<void*> allocs_;
  uint8_t* d_image_ = nullptr;  // archive byte 0
  size_t image_len_ = 0;
  std::vector<LayerPlan> layers_;
  ProjPlan lm_head_;
  float* d_gamma_final_ = nullptr;
  float *d_hidden_ = nullptr, *d_q_ = nullptr, *d_k_ = nullptr, *d_v_ = nullptr, *d_attn_ = nullptr,
        *d_mlp_ = nullptr, *d_logits_ = nullptr;
  void *d_kcache_ = nullptr, *d_vcache_ = nullptr;
  float *d_rope_cos_ = nullptr, *d_rope_sin_ = nullptr, *d_part_ml_ = nullptr, *d_part_acc_ = nullptr;
  uint32_t *d_prompt_ = nullptr, *d_out_tokens_ = nullptr;
  ArgmaxPartial* d_partials_ = nullptr;
  StepResult* d_result_ = nullptr;
  StepState* d_state_ = nullptr;
  StepState* h_state_ = nullptr;      // pinned
  StepResult* h_result_ = nullptr;    // pinned
  int embed_kind_ = 0;
  uint32_t n_chunks_ = 0;
  size_t kv_rows_ = 0;  // cache rows per kv head: max_seq_len rounded up to a 16-position tile

  hipStream_t stream_ = nullptr;
  hipGraph_t graph_ = nullptr;
  hipGraphExec_t graph_exec_ = nullptr;
  bool use_graph_ = true;
  bool embed_fused_ = false;         // k_finish embeds the next token (see init)
  float* d_hidden_out_ = nullptr;    // the last step's final hidden state when embed_fused_
  float* d_rope_cur_ = nullptr;      // the step's cos / sin rows (head_dim floats)
  float* d_xn_ = nullptr;            // polymorphic cells: the RMSNorm'ed input
  PolyRaw poly_raw_{};               // polymorphic cells: raw row sums per part
  float* flat_part_ = nullptr;       // FlatPoly: row-segment sums per tile
  size_t flat_part_floats_ = 0;

  // the hybrid model (EngineConfig::hybrid)
  std::vector<HybLayer> hyb_;
  float *d_hx0_ = nullptr, *d_hx1_ = nullptr, *d_hx2_ = nullptr, *d_hx3_ = nullptr, *d_hconv_ = nullptr;
  float *d_conv_state_ = nullptr, *d_rec_state_ = nullptr;
  size_t conv_state_floats_ = 0, rec_state_floats_ = 0;
  uint32_t rope_dim_ = 0;   // dims of a head the rotary tables cover (head_dim; hybrid: 64)
  std::vector<CellReplace> lm_repl_host_;  // the tied cell LM head's replace tables (for plan_block)
  bool plan_cell_corrections(ProjPlan* p, size_t C, std::string* err);
  bool plan_packed_corrections(const std::vector<float2>& padded, size_t rows, uint32_t kmax, ProjPlan* p);

  // the block step (plan_block): m <= kMaxBlock tokens' activations, operand tables, partials
  bool block_ok_ = false;
  uint32_t *d_btok_ = nullptr, *h_btok_ = nullptr, *d_bout_ = nullptr, *h_bout_ = nullptr;
  StepState *d_bstate_ = nullptr, *h_bstate_ = nullptr;
  uint32_t* d_bbrk_ = nullptr;  // [kMaxBlock] per-token break flags of the block step
  float *d_bx_ = nullptr, *d_bq_ = nullptr, *d_battn_ = nullptr, *d_bmlp_ = nullptr, *d_blog_ = nullptr;
  float *d_bpartial_ = nullptr, *d_bpml_ = nullptr, *d_bpacc_ = nullptr;
  size_t bpart_floats_ = 0;   // d_bpartial_'s capacity
  bool bpart_short_ = false;  // a block GEMV's partial sums did not fit (not launched; the block step fails)
  float* d_bss_ = nullptr;  // [kMaxSsPartials][kMaxBlock]: Σx² partials of the hidden rows for the next norm
  // the hybrid's block activations, [kMaxBlock][rows]: the in-projections' outputs (as d_hx0_ ..
  // d_hx3_) and the conv outputs
  float *d_bhx0_ = nullptr, *d_bhx1_ = nullptr, *d_bhx2_ = nullptr, *d_bhx3_ = nullptr, *d_bhconv_ = nullptr;
  BlockTables btab_{};
  ArgmaxPartial* d_bpartials_ = nullptr;
  // captured block steps, by [with the LM head][token count]; bhead_: the one being recorded has
  // the LM head (the prefill's blocks before its last have none: their logits are not read)
  hipGraph_t bgraph_[2][kMaxBlock + 1] = {};
  hipGraphExec_t bgraph_exec_[2][kMaxBlock + 1] = {};
  bool bhead_ = true;
  int probe_stage_ = -1;                 // stage bracketed by events in record_step
  hipEvent_t* probe_events_ = nullptr;
  size_t probe_next_ = 0;
  int launch_one();
  size_t h_pos_ = 0;  // the device position (StepState::pos) as the launches leave it
};

}  // namespace chpe
