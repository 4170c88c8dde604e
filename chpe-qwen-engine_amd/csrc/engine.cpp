// engine.cpp -- host side of the MI355X decode engine.
//
// init() follows CHPEEngine.init (src/chpe_engine.zig:854-974) for format detection, then
// builds a plan per projection that reproduces gemvLinear's tile walk
// (src/chpe_engine.zig:1396-1489) on the GPU, extracts norm gains / biases with the
// reference's fallback rules (:1144-1192), uploads the archive image and captures the whole
// forwardDecode step (:1663-1803) as one hipGraph.
#include "engine.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>

#include "format.hpp"

namespace chpe {

namespace {

constexpr size_t kImageShift = 64;       // puts every cell's code area on a 128-byte boundary
constexpr size_t kImagePad = 1u << 20;   // zero bytes after the archive (bounded over-reads)

uint64_t now_ns() {
  return uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(
                      std::chrono::steady_clock::now().time_since_epoch())
                      .count());
}

template <typename T>
T rd(const uint8_t* bytes, size_t len, size_t off) {  // little-endian read, zero past the end
  uint8_t buf[sizeof(T)] = {0};
  for (size_t i = 0; i < sizeof(T); ++i)
    if (off + i < len) buf[i] = bytes[off + i];
  T v;
  std::memcpy(&v, buf, sizeof(T));
  return v;
}

#define HIP_TRY(expr)                                                               \
  do {                                                                              \
    hipError_t e_ = (expr);                                                         \
    if (e_ != hipSuccess) {                                                         \
      if (err) *err = std::string(#expr) + ": " + hipGetErrorString(e_);            \
      return false;                                                                 \
    }                                                                               \
  } while (0)

}  // namespace

bool arch_preset(int id, ModelArch* a) {
  switch (id) {
    case 0: *a = {0, "Qwen2.5-3B", 2048, 11008, 36, 16, 2, 128, 151936, 1000000.0f, 1e-6f}; return true;
    case 1: *a = {1, "Qwen3.5-9B", 4096, 12288, 32, 16, 4, 256, 248320, 1000000.0f, 1e-6f}; return true;
    case 2: *a = {2, "Qwen2.5-72B", 8192, 29568, 80, 64, 8, 128, 152064, 1000000.0f, 1e-6f}; return true;
  }
  return false;
}

int arch_from_path(const char* p) {
  if (std::strstr(p, "9B") || std::strstr(p, "9b") || std::strstr(p, "qwen35")) return 1;
  if (std::strstr(p, "72B") || std::strstr(p, "72b")) return 2;
  return 0;
}

std::unique_ptr<Engine> Engine::create(const uint8_t* bytes, size_t len, const EngineConfig& cfg,
                                       std::string* err) {
  std::unique_ptr<Engine> e(new Engine());
  if (!e->init(bytes, len, cfg, err)) return nullptr;
  return e;
}

Engine::~Engine() {
  if (stream_) (void)hipStreamSynchronize(stream_);
  for (int hd = 0; hd < 2; ++hd)
    for (uint32_t m = 0; m <= kMaxBlock; ++m) {
      if (bgraph_exec_[hd][m]) (void)hipGraphExecDestroy(bgraph_exec_[hd][m]);
      if (bgraph_[hd][m]) (void)hipGraphDestroy(bgraph_[hd][m]);
    }
  if (graph_exec_) (void)hipGraphExecDestroy(graph_exec_);
  if (graph_) (void)hipGraphDestroy(graph_);
  for (void* p : allocs_) (void)hipFree(p);
  if (h_state_) (void)hipHostFree(h_state_);
  if (h_result_) (void)hipHostFree(h_result_);
  if (h_btok_) (void)hipHostFree(h_btok_);
  if (h_bout_) (void)hipHostFree(h_bout_);
  if (h_bstate_) (void)hipHostFree(h_bstate_);
  if (stream_) (void)hipStreamDestroy(stream_);
}

void* Engine::dev_alloc(size_t bytes) {
  void* p = nullptr;
  if (hipMalloc(&p, std::max<size_t>(bytes, 256)) != hipSuccess) return nullptr;
  allocs_.push_back(p);
  return p;
}

float* Engine::upload_vector(const std::vector<float>& v) {
  float* d = static_cast<float*>(dev_alloc(v.size() * sizeof(float)));
  if (d) (void)hipMemcpy(d, v.data(), v.size() * sizeof(float), hipMemcpyHostToDevice);
  return d;
}

bool Engine::init(const uint8_t* b, size_t len, const EngineConfig& cfg, std::string* err) {
  cfg_ = cfg;
  host_bytes_ = b;
  len_ = len;
  if (!arch_preset(cfg.arch_id, &arch_)) { *err = "unknown architecture"; return false; }
  if (cfg.hybrid && cfg.arch_id != 1) { *err = "the hybrid layers are Qwen3.5-9B's"; return false; }
  rope_dim_ = uint32_t(cfg.hybrid ? 64 : arch_.head_dim);  // (partial_rotary_factor 0.25 of 256)
  // ---- format detection: CHPEEngine.init, src/chpe_engine.zig:869-918
  if (len >= 4096) {
    const uint32_t magic = rd<uint32_t>(b, len, 0);
    if (magic == kChpeMagic || magic == kArchiveMagic) {
      archive_valid_ = true;
      record_count_ = size_t(rd<uint64_t>(b, len, 16));
      const uint64_t rec_b = rd<uint64_t>(b, len, 32), cell_b = rd<uint64_t>(b, len, 40),
                     pre_b = rd<uint64_t>(b, len, 48), flags = rd<uint64_t>(b, len, 56);
      is_dense_ = pre_b == 0 && rec_b == cell_b && rec_b == kCellBytes;
      is_raw_ = rec_b == kTileCodeBytes;
      is_raw_fp16_ = is_raw_ && (flags & kFlagRawFp16);
      if (is_raw_fp16_) {
        quant_bits_ = 16;
      } else if (is_raw_) {
        const size_t gib = size_t(1) << 30;
        quant_bits_ = (arch_.id == 1 && ((flags & kFlagInt8Hint) || (len < 10 * gib && len > 7 * gib))) ? 8 : 16;
      } else if (record_count_ > 0 && len >= 4096 + (is_dense_ ? kCellBytes : kRecordBytes)) {
        quant_bits_ = b[4096 + (is_dense_ ? 0 : kPrefetchBytes) + kPayloadOff + kMetaQuantBits];
        if (quant_bits_ == 0) quant_bits_ = 2;
      }
    }
  }
  stride_ = is_raw_ ? kTileCodeBytes : (is_dense_ ? kCellBytes : kRecordBytes);
  wpt_ = (is_raw_ && quant_bits_ == 16) ? 8192 : (quant_bits_ == 8 ? 16384 : (quant_bits_ == 4 || quant_bits_ == 2 ? 32768 : 8192));
  map_ = arch_.hidden_dim == 2048 ? (is_raw_ ? MapKind::Qwen3bRaw : MapKind::Qwen3bCell)
                                  : (arch_.hidden_dim == 8192 ? MapKind::Qwen72b : MapKind::Qwen35_9b);
  if (!archive_valid_ || record_count_ == 0) {
    *err = "archive header is not a valid .chpe header (the synthetic-weight fallback of the "
           "reference engine is not built on the GPU path)";
    return false;
  }
  if (cfg.max_seq_len == 0 || cfg.max_seq_len > (1u << 20)) { *err = "bad max_seq_len"; return false; }
  if (!attention_supported(uint32_t(arch_.num_attn_heads), uint32_t(arch_.num_kv_heads),
                           uint32_t(arch_.head_dim))) {
    *err = "attention kernels are built for head_dim 128 with 8 query heads per kv head and "
           "head_dim 256 with 4";
    return false;
  }
  const uint32_t chunk = attn_chunk(uint32_t(arch_.head_dim), uint32_t(arch_.num_kv_heads));
  n_chunks_ = uint32_t((cfg.max_seq_len + chunk - 1) / chunk);
  if (n_chunks_ > kAttnMaxChunks) {
    *err = "max_seq_len exceeds the attention kernel's chunk table (" +
           std::to_string(size_t(kAttnMaxChunks) * chunk) + " positions)";
    return false;
  }

  HIP_TRY(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking));
  // ---- archive image: verbatim, shifted so that code areas are 128-byte aligned
  const size_t shift = is_raw_ ? 0 : kImageShift;
  uint8_t* img = static_cast<uint8_t*>(dev_alloc(shift + len + kImagePad));
  if (!img) { *err = "hipMalloc of the archive image failed"; return false; }
  d_image_ = img + shift;
  image_len_ = len + kImagePad;
  HIP_TRY(hipMemset(img, 0, shift));
  HIP_TRY(hipMemset(d_image_ + len, 0, kImagePad));
  const size_t chunk_bytes = size_t(256) << 20;
  for (size_t off = 0; off < len; off += chunk_bytes)
    HIP_TRY(hipMemcpy(d_image_ + off, b + off, std::min(chunk_bytes, len - off), hipMemcpyHostToDevice));

  // ---- embedding kind (unpackEmbedRow branches)
  embed_kind_ = is_raw_fp16_ ? 1 : (is_raw_ ? (quant_bits_ == 8 ? 3 : 2) : 4);

  // ---- per-layer plans
  const size_t D = arch_.hidden_dim, I = arch_.intermediate_dim,
               qd = arch_.num_attn_heads * arch_.head_dim, kvd = arch_.num_kv_heads * arch_.head_dim;
  auto norm = [&](size_t tile) {  // unpackNorm: src/chpe_engine.zig:1144-1170
    std::vector<float> g(D, 1.0f);
    if (tile >= record_count_) return g;
    const size_t off = is_raw_ ? 4096 + tile * kTileCodeBytes
                               : 4096 + tile * stride_ + (is_dense_ ? 0 : kPrefetchBytes) + kBytecodeHeader;
    const bool bf = arch_.hidden_dim == 4096 && is_raw_;
    bool all_zero = true;
    for (size_t i = 0; i < D; ++i) {
      g[i] = bf ? bf16_to_f32(rd<uint16_t>(b, len, off + 2 * i)) : rd<float>(b, len, off + 4 * i);
      if (!std::isfinite(g[i])) { std::fill(g.begin(), g.end(), 1.0f); return g; }
      if (g[i] != 0.0f) all_zero = false;
    }
    if (all_zero) std::fill(g.begin(), g.end(), 1.0f);
    return g;
  };
  layers_.resize(arch_.num_layers);
  for (size_t l = 0; l < arch_.num_layers; ++l) {
    const LayerInfo li = layer_info(map_, l);
    LayerPlan& L = layers_[l];
    L.gamma_in = upload_vector(norm(li.input_norm));
    L.gamma_post = upload_vector(norm(li.post_norm));
    std::string why;
    auto plan = [&](const char* name, size_t ts, size_t nt, size_t r, size_t c, size_t xl, size_t yl,
                    bool acc, int64_t bt, ProjPlan* p) {
      if (plan_projection(ts, nt, r, c, xl, yl, acc, bt, p, &why)) return true;
      *err = "layer " + std::to_string(l) + " " + name + ": " + why;
      return false;
    };
    if (!plan("q_proj", li.q_proj, li.q_tiles, qd, D, D, qd, false, li.q_bias, &L.q) ||
        !plan("k_proj", li.k_proj, li.k_tiles, kvd, D, D, kvd, false, li.k_bias, &L.k) ||
        !plan("v_proj", li.v_proj, li.v_tiles, kvd, D, D, kvd, false, li.v_bias, &L.v) ||
        !plan("o_proj", li.o_proj, li.o_tiles, D, D, D, D, true, -1, &L.o) ||
        !plan("gate_proj", li.gate_proj, li.gate_tiles, I, D, D, I, false, -1, &L.gate) ||
        !plan("up_proj", li.up_proj, li.up_tiles, I, D, D, I, false, -1, &L.up) ||
        !plan("down_proj", li.down_proj, li.down_tiles, D, I, I, D, true, -1, &L.down))
      return false;
    if (L.gate.kind != L.up.kind) {  // one SwiGLU launch: flat tensors of two forms run tile by tile
      auto flat = [](WeightKind k) { return k == WeightKind::FlatW4 || k == WeightKind::FlatW2 || k == WeightKind::FlatPoly; };
      if (!flat(L.gate.kind) || !flat(L.up.kind)) { *err = "gate/up weight layouts differ"; return false; }
      for (ProjPlan* q : {&L.gate, &L.up}) {
        q->kind = WeightKind::FlatPoly;
        q->corr = nullptr;
        q->corr_kmax = 0;
        q->wrows = 0;
        if (!ensure_poly_buffers(q->poly.n_cells, q->cols)) { *err = "allocation"; return false; }
      }
    }
  }
  d_gamma_final_ = upload_vector(norm(final_norm_record(map_)));
  if (!plan_lm_head(err)) return false;

  // ---- activations, KV cache, RoPE tables, reduction scratch
  const size_t V = arch_.vocab_size, S = cfg.max_seq_len, hd = arch_.head_dim;
  d_hidden_ = static_cast<float*>(dev_alloc(D * 4));
  d_hidden_out_ = static_cast<float*>(dev_alloc(D * 4));
  {  // the next token's embedding moves into k_finish when the LM head runs on the matrix-core
     // kernel (which keeps the step's final hidden state in d_hidden_out_)
    uint32_t rows[kMaxParts] = {lm_head_.rows, 0, 0}, begin[kMaxParts], nu, np, wpu;
    embed_fused_ = gemv_geometry(lm_head_.kind, GemvMode::Logits, uint32_t(D), rows, 1, &nu, &np, &wpu, begin).mma != 0;
  }
  d_q_ = static_cast<float*>(dev_alloc(qd * 4));
  d_k_ = static_cast<float*>(dev_alloc(kvd * 4));
  d_v_ = static_cast<float*>(dev_alloc(kvd * 4));
  d_attn_ = static_cast<float*>(dev_alloc(std::max(D, qd) * 4));
  d_mlp_ = static_cast<float*>(dev_alloc(I * 4));
  d_logits_ = static_cast<float*>(dev_alloc(V * 4));
  const size_t kv_elem = cfg.kv_f16 ? 2 : 4;
  kv_rows_ = (S + 15) / 16 * 16;
  const size_t kv_bytes = arch_.num_layers * kvd * kv_rows_ * kv_elem;
  d_kcache_ = dev_alloc(kv_bytes);
  d_vcache_ = dev_alloc(kv_bytes);
  d_part_ml_ = static_cast<float*>(dev_alloc(arch_.num_attn_heads * n_chunks_ * 2 * 4));
  d_part_acc_ = static_cast<float*>(dev_alloc(arch_.num_attn_heads * n_chunks_ * hd * 4));
  d_partials_ = static_cast<ArgmaxPartial*>(dev_alloc(kMaxLogitsBlocks * sizeof(ArgmaxPartial)));
  d_result_ = static_cast<StepResult*>(dev_alloc(sizeof(StepResult)));
  d_state_ = static_cast<StepState*>(dev_alloc(sizeof(StepState)));
  d_prompt_ = static_cast<uint32_t*>(dev_alloc(S * 4));
  d_out_tokens_ = static_cast<uint32_t*>(dev_alloc(S * 4));
  if (!d_hidden_ || !d_kcache_ || !d_vcache_ || !d_logits_ || !d_part_acc_ || !d_out_tokens_) {
    *err = "device allocation failed";
    return false;
  }
  HIP_TRY(hipMemset(d_hidden_, 0, D * 4));
  HIP_TRY(hipMemset(d_kcache_, 0, kv_bytes));
  HIP_TRY(hipMemset(d_vcache_, 0, kv_bytes));
  HIP_TRY(hipMemset(d_logits_, 0, V * 4));
  HIP_TRY(hipMemset(d_result_, 0, sizeof(StepResult)));
  HIP_TRY(hipMemset(d_state_, 0, sizeof(StepState)));
  // RoPE angles exactly as applyRope computes them (src/chpe_engine.zig:197-206), in f32
  // (the hybrid model rotates the first rope_dim_ = 64 dims of a head: the same formula over
  // 64 dims)
  const size_t rd = rope_dim_;
  std::vector<float> cs(S * (rd / 2)), sn(S * (rd / 2));
  for (size_t p = 0; p < S; ++p) {
    const float pos_f = float(p);
    for (size_t i = 0; i < rd / 2; ++i) {
      const float freq_exponent = 2.0f * float(i) / float(rd);
      const float freq = 1.0f / std::pow(arch_.rope_theta, freq_exponent);
      const float theta = pos_f * freq;
      cs[p * (rd / 2) + i] = std::cos(theta);
      sn[p * (rd / 2) + i] = std::sin(theta);
    }
  }
  d_rope_cos_ = upload_vector(cs);
  d_rope_sin_ = upload_vector(sn);
  d_rope_cur_ = static_cast<float*>(dev_alloc(hd * 4));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&h_state_), sizeof(StepState), hipHostMallocDefault));
  HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&h_result_), sizeof(StepResult), hipHostMallocDefault));
  if (cfg.hybrid && !plan_hybrid(err)) return false;
  {  // the block step for archives whose projections are all flat 4-/2-bit tiles (CHPE_BLOCK=0: off)
    const char* bk = std::getenv("CHPE_BLOCK");
    std::string why;
    if (!(bk && bk[0] == '0') && !plan_block(&why) && !why.empty()) {
      *err = "block step: " + why;
      return false;
    }
  }
  build_xm_layouts();  // the gate/up and LM head codes in the matrix-core kernel's load order
  HIP_TRY(hipDeviceSynchronize());

  // ---- capture the step (CHPE_GRAPH=0 launches the same kernels directly on the stream,
  // which some profilers need)
  const char* g = std::getenv("CHPE_GRAPH");
  use_graph_ = !(g && g[0] == '0');
  if (use_graph_) {
    HIP_TRY(hipStreamBeginCapture(stream_, hipStreamCaptureModeThreadLocal));
    record_step(stream_);
    HIP_TRY(hipStreamEndCapture(stream_, &graph_));
    HIP_TRY(hipGraphInstantiate(&graph_exec_, graph_, nullptr, nullptr, 0));
  }
  return true;
}

int Engine::launch_one() {
  ++h_pos_;  // k_finish advances the device position
  if (use_graph_) return hipGraphLaunch(graph_exec_, stream_) == hipSuccess ? 0 : -3;
  record_step(stream_);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

bool plan_flat_tiles(const uint8_t* cells, size_t len, size_t stride, size_t n_tiles, size_t r_total,
                     size_t c_total, WeightKind* kind, std::vector<float2>* corr, uint32_t* corr_kmax,
                     std::string* err) {
  const uint8_t* b = cells;
  auto cell = [&](size_t t) { return t * stride; };
  corr->clear();
  *corr_kmax = 0;
  if (n_tiles == 0 || n_tiles * kFlatWeights < r_total * c_total) { *err = "flat tensor shorter than its shape"; return false; }
  if (c_total % 128) { *err = "flat tensor width is not a multiple of 128"; return false; }
  const uint8_t bits = rd<uint8_t>(b, len, cell(0) + kPayloadOff + kMetaQuantBits);
  for (size_t t = 0; t < n_tiles; ++t) {
    const size_t pl = cell(t) + kPayloadOff;
    if (rd<uint8_t>(b, len, pl + kMetaQuantBits) != bits ||
        !(rd<uint64_t>(b, len, pl + kMetaCustomFlags) & kFlagGroup128)) {
      *err = "flat tiles are not uniformly group-128 " + std::to_string(bits) + "-bit";
      return false;
    }
  }
  if (bits == 4) *kind = WeightKind::FlatW4;
  else if (bits == 2) *kind = WeightKind::FlatW2;
  else { *err = "flat tiles of " + std::to_string(bits) + " bits"; return false; }
  // outliers replace weights (chpe_engine.zig:632-646): per-row (col, w_out - w_code)
  std::vector<std::vector<std::pair<uint32_t, float>>> by_row;
  const size_t total = r_total * c_total;
  for (size_t t = 0; t < n_tiles; ++t) {
    const size_t pl = cell(t) + kPayloadOff, codes = cell(t) + kBytecodeHeader;
    const uint16_t n = rd<uint16_t>(b, len, pl + kFlatOutlierN);
    if (n == 0 || n > 64) continue;
    std::map<uint32_t, float> last;  // offset -> replacement (the last entry wins)
    for (size_t m = 0; m < n; ++m) {
      const uint16_t off = rd<uint16_t>(b, len, pl + kFlatOutlierOff + 2 * m);
      last[off] = f16_to_f32(rd<uint16_t>(b, len, pl + kFlatOutlierW + 2 * m));
    }
    for (const auto& [off, w] : last) {
      const size_t f = t * kFlatWeights + off;
      if (f >= total) continue;
      const float s = f16_to_f32(rd<uint16_t>(b, len, pl + kGroupScales + 2 * (off / 128)));
      float q;
      if (bits == 4) {
        q = float((rd<uint8_t>(b, len, codes + off / 2) >> (4 * (off & 1))) & 15) - 8.0f;
      } else {
        static const float lut[4] = {0.0f, 1.0f, -2.0f, -1.0f};
        q = lut[(rd<uint8_t>(b, len, codes + off / 4) >> (2 * (off & 3))) & 3];
      }
      if (by_row.empty()) by_row.resize(r_total);
      by_row[f / c_total].push_back({uint32_t(f % c_total), w - q * s});
    }
  }
  if (by_row.empty()) return true;
  size_t kmax = 0;  // fixed stride per row, zero-padded: [r_total][kmax]
  for (const auto& row : by_row) kmax = std::max(kmax, row.size());
  if (kmax > kMaxCorrPerRow) {
    *err = "a row has more than " + std::to_string(kMaxCorrPerRow) + " flat-tile outliers";
    return false;
  }
  kmax = std::max<size_t>(kmax, 1);
  corr->assign(r_total * kmax, make_float2(0.0f, 0.0f));
  for (size_t r = 0; r < r_total; ++r)
    for (size_t k = 0; k < by_row[r].size(); ++k) {
      float cf;
      std::memcpy(&cf, &by_row[r][k].first, 4);
      (*corr)[r * kmax + k] = make_float2(cf, by_row[r][k].second);
    }
  *corr_kmax = uint32_t(kmax);
  return true;
}

void plan_flat(const uint8_t* cells, size_t len, size_t stride, size_t n_avail, size_t r_total, size_t c_total,
               FlatPlan* out) {
  const size_t need = (r_total * c_total + kFlatWeights - 1) / kFlatWeights;
  const size_t use = std::min(n_avail, need);  // (tiles past the shape add nothing, :702)
  const size_t covered = use * kFlatWeights;
  const size_t wrows = use < need ? covered / c_total : r_total;
  std::string why;
  out->corr.clear();
  out->n_tiles = uint32_t(use);
  out->wrows = uint32_t(wrows);
  out->corr_kmax = 0;
  // the uniform kernels: whole rows of uniformly group-128 4- or 2-bit tiles (a short tensor:
  // 4-bit only), at most kMaxCorrPerRow outliers per row
  const bool whole_rows = use == need || covered % c_total == 0;
  if (use > 0 && whole_rows &&
      plan_flat_tiles(cells, len, stride, use, wrows, c_total, &out->kind, &out->corr, &out->corr_kmax, &why) &&
      (wrows == r_total || out->kind == WeightKind::FlatW4))
    return;
  out->kind = WeightKind::FlatPoly;
  out->corr.clear();
  out->corr_kmax = 0;
  out->wrows = uint32_t(r_total);
}

void walk_cells(const uint8_t* b, size_t len, size_t stride, size_t n_avail, size_t r_total, size_t c_total,
                std::vector<uint32_t>* row_base, bool* uniform_w4, uint64_t* extent) {
  size_t rb = 0;
  bool uniform = true;
  unsigned __int128 reach = 0;
  row_base->clear();
  for (size_t t = 0; t < n_avail; ++t) {
    if (rb >= r_total) break;
    const size_t pl = t * stride + kPayloadOff;
    const uint32_t rows = rd<uint32_t>(b, len, pl + kDimsRows);
    if (rows == 0) break;
    const uint32_t cols = rd<uint32_t>(b, len, pl + kDimsCols);
    const uint8_t qb = rd<uint8_t>(b, len, pl + kMetaQuantBits);
    const bool g128 = (rd<uint64_t>(b, len, pl + kMetaCustomFlags) & kFlagGroup128) != 0;
    uniform = uniform && rows == 16 && cols == c_total && qb == 4 && g128;
    // the bytes the polymorphic kernel reads for this cell's used rows: codes at the row stride
    // of its width, group scales past the payload for tall cells
    const unsigned __int128 used = std::min<size_t>(rows, r_total - rb);
    const unsigned __int128 row_bytes = qb == 4 ? cols / 2 : qb == 8 ? cols : qb == 16 ? 2ull * cols
                                        : qb == 32 ? 4ull * cols : cols / 4;
    unsigned __int128 end = t * stride + kPayloadOff + 1024;  // metadata, row outliers
    end = std::max(end, t * stride + kBytecodeHeader + used * row_bytes);
    if (g128 && (qb == 4 || !(qb == 8 || qb == 16 || qb == 32)))
      end = std::max(end, t * stride + kPayloadOff + kGroupScales + 2 * used * (cols / 128));
    reach = std::max(reach, end);
    row_base->push_back(uint32_t(rb));
    rb += rows;
  }
  row_base->push_back(uint32_t(std::min(rb, r_total)));
  *uniform_w4 = uniform && rb == r_total;
  if (extent) *extent = reach > ~uint64_t(0) ? ~uint64_t(0) : uint64_t(reach);
}

bool Engine::plan_projection(size_t tile_start, size_t num_tiles, size_t r_total, size_t c_total,
                             size_t x_len, size_t y_len, bool accumulate, int64_t bias_tile,
                             ProjPlan* p, std::string* err) {
  const uint8_t* b = host_bytes_;
  const size_t len = len_;
  (void)accumulate;
  if (tile_start >= record_count_) {
    *err = "tensor starts past the end of the archive (synthetic-output fallback)";
    return false;
  }
  const size_t avail = std::min(num_tiles, record_count_ - tile_start);
  const size_t cell_off = is_dense_ ? 0 : kPrefetchBytes;
  p->rows = uint32_t(r_total);
  p->cols = uint32_t(c_total);
  if (!is_raw_) {
    auto cell = [&](size_t t) { return 4096 + (tile_start + t) * stride_ + cell_off; };
    p->base = d_image_ + cell(0);
    p->stride = uint32_t(stride_);
    if (c_total > 2048) {  // flat tiles: gemvCellFlat
      // gemvLinear walks the available tiles only (:1423-1429): with fewer tiles than the shape
      // needs (the 9B map's v <- in_proj_a, one tile, :1119) the rows past them get no
      // weights (zero in a fresh output, untouched when accumulating)
      FlatPlan fp;
      plan_flat(b + cell(0), len - cell(0), stride_, avail, r_total, c_total, &fp);
      p->kind = fp.kind;
      p->wrows = fp.wrows;
      p->corr_kmax = fp.corr_kmax;
      if (!fp.corr.empty()) {
        p->corr = static_cast<float2*>(dev_alloc(fp.corr.size() * sizeof(float2)));
        if (!p->corr) { *err = "allocation"; return false; }
        (void)hipMemcpy(p->corr, fp.corr.data(), fp.corr.size() * sizeof(float2), hipMemcpyHostToDevice);
        if ((fp.kind == WeightKind::FlatW4 || fp.kind == WeightKind::FlatW2) &&
            !plan_packed_corrections(fp.corr, r_total, fp.corr_kmax, p)) {
          *err = "allocation";
          return false;
        }
      }
      p->poly.n_cells = fp.n_tiles;
      if (fp.kind == WeightKind::FlatPoly && !ensure_poly_buffers(fp.n_tiles, uint32_t(c_total))) {
        *err = "allocation";
        return false;
      }
    } else {  // 16-row polymorphic cells: row bases are a prefix sum of dims.rows
      std::vector<uint32_t> rb;
      bool uniform = false;
      uint64_t reach = 0;
      walk_cells(b + cell(0), len - cell(0), stride_, avail, r_total, c_total, &rb, &uniform, &reach);
      if (uniform && c_total == 2048 && x_len >= 2048 && y_len >= r_total) {
        p->kind = WeightKind::Cell16W4;
      } else {  // any other mix of widths: the polymorphic kernel, cell by cell
        if (reach > image_len_ - cell(0)) {  // the device image holds the archive + kImagePad
          *err = "polymorphic cells read past the end of the archive";
          return false;
        }
        p->kind = WeightKind::Cell16Poly;
        p->poly.n_cells = uint32_t(rb.size() - 1);
        uint32_t* d = static_cast<uint32_t*>(dev_alloc(rb.size() * 4));
        if (!d) { *err = "allocation"; return false; }
        (void)hipMemcpy(d, rb.data(), rb.size() * 4, hipMemcpyHostToDevice);
        p->poly.row_base = d;
        if (!ensure_poly_buffers(0, 0)) { *err = "allocation"; return false; }
      }
    }
  } else {
    // one row-major matrix over consecutive raw tiles (dotSegment :1194-1251 segment by segment)
    if (avail * wpt_ < r_total * c_total || c_total % (quant_bits_ == 8 ? 16 : 8)) {
      *err = "raw tensor shorter than its shape";
      return false;
    }
    p->kind = quant_bits_ == 8 ? WeightKind::Raw8 : WeightKind::Raw16;
    p->base = d_image_ + 4096 + tile_start * kTileCodeBytes;
    p->stride = uint32_t(kTileCodeBytes);
    p->bf16 = is_raw_fp16_ ? 0 : 1;
  }
  if (bias_tile >= 0 && size_t(bias_tile) < record_count_) {  // unpackBias: :1172-1192
    const size_t off = is_raw_ ? 4096 + size_t(bias_tile) * kTileCodeBytes
                               : 4096 + size_t(bias_tile) * stride_ + cell_off + kBytecodeHeader;
    std::vector<float> bias(r_total);
    const bool bf = arch_.hidden_dim == 4096 && is_raw_;
    for (size_t i = 0; i < r_total; ++i) {
      bias[i] = bf ? bf16_to_f32(rd<uint16_t>(b, len, off + 2 * i)) : rd<float>(b, len, off + 4 * i);
      if (!std::isfinite(bias[i])) bias[i] = 0.0f;
    }
    p->bias = upload_vector(bias);
  }
  return true;
}

bool Engine::ensure_poly_buffers(uint32_t flat_tiles, uint32_t C) {
  if (!d_xn_) {
    const size_t n = std::max({arch_.hidden_dim, arch_.intermediate_dim, arch_.vocab_size,
                               arch_.num_attn_heads * arch_.head_dim});
    d_xn_ = static_cast<float*>(dev_alloc((std::max(arch_.hidden_dim, arch_.intermediate_dim) + 1) * 4));
    for (int i = 0; i < kMaxParts; ++i) poly_raw_.y[i] = static_cast<float*>(dev_alloc(n * 4));
    if (!d_xn_ || !poly_raw_.y[kMaxParts - 1]) return false;
  }
  const size_t need = flat_tiles ? flat_poly_part_floats(flat_tiles, C) : 0;
  if (need > flat_part_floats_) {  // the row-segment sums of the largest FlatPoly tensor
    flat_part_ = static_cast<float*>(dev_alloc(need * 4));
    if (!flat_part_) return false;
    flat_part_floats_ = need;
  }
  return true;
}

bool Engine::plan_lm_head(std::string* err) {
  // computeLmHead: src/chpe_engine.zig:1554-1660
  const size_t D = arch_.hidden_dim, V = arch_.vocab_size;
  size_t start = 0, tiles = 0;
  std::string why;
  if (lm_head_record(D, &start, &tiles) && start < record_count_) {
    if (!plan_projection(start, tiles, V, D, D, V, false, -1, &lm_head_, &why)) {
      *err = "lm_head: " + why;
      return false;
    }
    return true;
  }
  if (!is_raw_) {  // tied embedding cells, outliers replace (unpackEmbedRowCell)
    const size_t n_cells = (V + 15) / 16, cell_off = is_dense_ ? 0 : kPrefetchBytes;
    if (n_cells > record_count_ || D != 2048) { *err = "tied LM head: unsupported shape"; return false; }
    for (size_t t = 0; t < n_cells; ++t) {
      const size_t pl = 4096 + t * stride_ + cell_off + kPayloadOff;
      const uint32_t rows = rd<uint32_t>(host_bytes_, len_, pl + kDimsRows);
      if ((rows != 16 && rows != 0) || host_bytes_[pl + kMetaQuantBits] != 4 ||
          !(rd<uint64_t>(host_bytes_, len_, pl + kMetaCustomFlags) & kFlagGroup128)) {
        *err = "tied LM head: embedding cell " + std::to_string(t) + " is not a 16-row group-128 4-bit cell";
        return false;
      }
    }
    // replace-mode outliers (unpackEmbedRowCell :1369-1378): per cell, entry k sets column
    // col[k] of row n to w_out[n][k]; entries apply in order, so only the last one for a
    // column counts.  Prepared as additive corrections to the dequantised code.
    std::vector<CellReplace> repl(n_cells);
    for (size_t t = 0; t < n_cells; ++t) {
      const size_t cell = 4096 + t * stride_ + cell_off, pl = cell + kPayloadOff;
      CellReplace& R = repl[t];
      for (int k = 0; k < 8; ++k) R.col[k] = rd<uint16_t>(host_bytes_, len_, pl + kRowOutlierCols + 2 * k);
      for (int k = 0; k < 8; ++k) {
        bool live = R.col[k] < D;
        for (int k2 = k + 1; k2 < 8; ++k2) live = live && R.col[k2] != R.col[k];
        for (int n = 0; n < 16; ++n) {
          R.delta[n][k] = 0.0f;
          if (!live) continue;
          const uint32_t col = R.col[k];
          const float w = f16_to_f32(rd<uint16_t>(host_bytes_, len_, pl + kRowOutlierW + 2 * (n * 8 + k)));
          const uint8_t byte = host_bytes_[cell + kBytecodeHeader + n * (D / 2) + col / 2];
          const float q = float((byte >> (4 * (col & 1))) & 15) - 8.0f;
          const float s = f16_to_f32(rd<uint16_t>(host_bytes_, len_, pl + kGroupScales + 2 * (n * (D / 128) + col / 128)));
          R.delta[n][k] = w - q * s;
        }
        if (!live) R.col[k] = 0;
      }
    }
    lm_repl_host_ = repl;
    lm_head_.repl = static_cast<CellReplace*>(dev_alloc(n_cells * sizeof(CellReplace)));
    if (!lm_head_.repl) { *err = "allocation"; return false; }
    (void)hipMemcpy(lm_head_.repl, repl.data(), n_cells * sizeof(CellReplace), hipMemcpyHostToDevice);
    lm_head_.kind = WeightKind::Cell16W4;
    lm_head_.base = d_image_ + 4096 + cell_off;
    lm_head_.stride = uint32_t(stride_);
    lm_head_.rows = uint32_t(V);
    lm_head_.cols = uint32_t(D);
    lm_head_.replace_outliers = 1;
    return true;
  }
  // tied embedding in a raw archive: rows are contiguous 16-bit vectors from record 0
  const size_t rpt = std::max<size_t>(1, 8192 / D);
  const size_t need = (V + rpt - 1) / rpt;
  if (std::min(record_count_, need) < need || D % 8) { *err = "tied raw LM head: archive too short"; return false; }
  lm_head_.kind = WeightKind::Raw16;
  lm_head_.base = d_image_ + 4096;
  lm_head_.stride = uint32_t(kTileCodeBytes);
  lm_head_.rows = uint32_t(V);
  lm_head_.cols = uint32_t(D);
  lm_head_.bf16 = is_raw_fp16_ ? 0 : 1;
  return true;
}

uint32_t Engine::enqueue_gemv(const ProjPlan* const* parts, float* const* outs, int n, GemvMode mode,
                              const float* x, uint32_t C, const float* gamma, hipStream_t st,
                              const RopeArgs* rope, const uint32_t* roles) {
  GemvArgs a{};
  const GemvLaunch g = gemv_args(parts, outs, n, mode, x, C, gamma, rope, roles, &a);
  if (parts[0]->kind == WeightKind::Cell16Poly) {
    const PolyPlan* pp[kMaxParts] = {};
    for (int i = 0; i < n; ++i) pp[i] = &parts[i]->poly;
    return launch_gemv_poly(a, pp, d_xn_, poly_raw_, st);
  }
  if (parts[0]->kind == WeightKind::FlatPoly) {
    uint32_t nt[kMaxParts] = {0, 0, 0};
    for (int i = 0; i < n; ++i) nt[i] = parts[i]->poly.n_cells;
    return launch_gemv_flat_poly(a, nt, d_xn_, poly_raw_, flat_part_, st);
  }
  launch_gemv(parts[0]->kind, a, g, st);
  return g.blocks;
}

GemvLaunch Engine::gemv_args(const ProjPlan* const* parts, float* const* outs, int n, GemvMode mode, const float* x,
                             uint32_t C, const float* gamma, const RopeArgs* rope, const uint32_t* roles,
                             GemvArgs* out) const {
  GemvArgs& a = *out;
  a = GemvArgs{};
  if (rope) a.rope = *rope;
  else a.rope.state = d_state_;  // (the residual launches read StepState::broken)
  a.n_parts = n;
  a.mode = int(mode);
  a.C = C;
  a.x = x;
  a.gamma = gamma;
  a.eps = arch_.rms_eps;
  uint32_t rows[kMaxParts] = {0, 0, 0}, begin[kMaxParts] = {0, 0, 0};
  for (int i = 0; i < n; ++i) rows[i] = parts[i]->rows;
  const GemvLaunch g = gemv_geometry(parts[0]->kind, mode, C, rows, n, &a.n_units, &a.n_panels,
                                     &a.waves_per_unit, begin);
  for (int i = 0; i < n; ++i) {
    const ProjPlan& p = *parts[i];
    GemvPart& gp = a.part[i];
    gp.base = p.base;
    gp.stride = p.stride;
    gp.rows = p.rows;
    gp.wrows = p.wrows ? p.wrows : p.rows;
    gp.unit_begin = begin[i];
    gp.bf16 = p.bf16;
    gp.y = outs[i];
    gp.bias = p.bias;
    gp.corr_kmax = p.corr_kmax;
    gp.corr = p.corr;
    gp.replace_outliers = p.replace_outliers;
    gp.repl = p.repl;
    gp.rope_role = roles ? roles[i] : 0u;
    gp.xcodes = i == 0 && mode == p.xcodes_mode && n == p.xcodes_parts ? p.xcodes : nullptr;
  }
  if (mode == GemvMode::Logits) {
    a.partials = d_partials_;
    a.result = d_result_;
    a.hidden_out = embed_fused_ ? d_hidden_out_ : nullptr;
  }
  return g;
}

void Engine::build_xm_layout_of(ProjPlan* const* parts, int n, GemvMode mode, uint32_t C, const RopeArgs* rope,
                                const uint32_t* roles) {
  GemvArgs a{};
  float* outs[kMaxParts] = {d_mlp_, d_mlp_, d_mlp_};
  const GemvLaunch g = gemv_args(parts, outs, n, mode, d_hidden_, C, nullptr, rope, roles, &a);
  const size_t bytes = xm_layout_bytes(parts[0]->kind, a, g);
  if (bytes == 0) return;
  void* d = nullptr;
  if (hipMalloc(&d, bytes) != hipSuccess) {  // (no copy: the launch reads the records)
    (void)hipGetLastError();
    return;
  }
  allocs_.push_back(d);
  if (build_xm_layout(parts[0]->kind, a, g, static_cast<uint8_t*>(d), stream_)) {
    parts[0]->xcodes = static_cast<uint8_t*>(d);
    parts[0]->xcodes_mode = mode;
    parts[0]->xcodes_parts = n;
  }
}

void Engine::build_xm_layouts() {
  const uint32_t D = uint32_t(arch_.hidden_dim);
  for (size_t l = 0; l < layers_.size(); ++l) {
    LayerPlan& L = layers_[l];
    ProjPlan* gu[2] = {&L.gate, &L.up};
    if (L.gate.kind == L.up.kind && L.gate.rows) build_xm_layout_of(gu, 2, GemvMode::SwiGlu, D);
    // (2-bit tiles: the q/k/v, o and down launches too; xm_layout_bytes decides)
    ProjPlan* o[1] = {&L.o};
    if (L.o.rows) build_xm_layout_of(o, 1, GemvMode::Accum, D);  // (the launch's input length)
    ProjPlan* dn[1] = {&L.down};
    if (L.down.rows) build_xm_layout_of(dn, 1, GemvMode::Accum, uint32_t(arch_.intermediate_dim));
    if (L.q.kind == L.k.kind && L.k.kind == L.v.kind && L.q.rows) {  // one q/k/v launch (enqueue_qkv)
      ProjPlan* qkv[3] = {&L.q, &L.k, &L.v};
      const uint32_t roles[3] = {kRoleQ, kRoleK, kRoleV};
      const RopeArgs rope = rope_args(l);
      build_xm_layout_of(qkv, 3, GemvMode::QkvRope, D, &rope, roles);
    }
  }
  ProjPlan* lm[1] = {&lm_head_};
  if (lm_head_.rows) build_xm_layout_of(lm, 1, GemvMode::Logits, D);
}

void Engine::enqueue_qkv(size_t l, hipStream_t st) {
  // q, k, v in one launch when they share a layout: bias, RoPE on q and k, k and v appended to
  // the layer's KV cache at the step's position, q (rotated) into d_q_
  const LayerPlan& L = layers_[l];
  const uint32_t D = uint32_t(arch_.hidden_dim);
  const ProjPlan* qkv[3] = {&L.q, &L.k, &L.v};
  float* outs[3] = {d_q_, d_k_, d_v_};
  const uint32_t roles[3] = {kRoleQ, kRoleK, kRoleV};
  const RopeArgs rope = rope_args(l);
  if (L.q.kind == L.k.kind && L.k.kind == L.v.kind) {
    enqueue_gemv(qkv, outs, 3, GemvMode::QkvRope, d_hidden_, D, L.gamma_in, st, &rope, roles);
  } else {
    for (int i = 0; i < 3; ++i)
      enqueue_gemv(&qkv[i], &outs[i], 1, GemvMode::QkvRope, d_hidden_, D, L.gamma_in, st, &rope, &roles[i]);
  }
}

RopeArgs Engine::rope_args(size_t l) const {
  const size_t kvd = arch_.num_kv_heads * arch_.head_dim, S = kv_rows_;
  const size_t kv_elem = cfg_.kv_f16 ? 2 : 4;
  RopeArgs r{};
  r.state = d_state_;
  r.cos = d_rope_cur_;
  r.sin = d_rope_cur_ + rope_dim_ / 2;
  r.k_cache = static_cast<uint8_t*>(d_kcache_) + l * kvd * S * kv_elem;
  r.v_cache = static_cast<uint8_t*>(d_vcache_) + l * kvd * S * kv_elem;
  r.head_dim = uint32_t(arch_.head_dim);
  r.max_seq = uint32_t(S);
  r.kv_f16 = cfg_.kv_f16 ? 1 : 0;
  // the break test on the hidden state layer l - 1 left (forwardDecode :1753-1764): the sum of
  // squares after layers 0-2 and 8-16, otherwise hidden[0] (whose non-finite value makes the sum
  // non-finite too)
  const size_t prev = l - 1;
  r.brk_check = l == 0 ? 0u : ((prev < 3 || (prev >= 8 && prev <= 16)) ? 1u : 2u);
  return r;
}

AttnArgs Engine::attn_args(size_t l) const {
  const size_t kvd = arch_.num_kv_heads * arch_.head_dim, S = kv_rows_;
  const size_t kv_elem = cfg_.kv_f16 ? 2 : 4;
  AttnArgs at{};
  at.state = d_state_;
  at.q = d_q_;
  at.k_cache = static_cast<uint8_t*>(d_kcache_) + l * kvd * S * kv_elem;
  at.v_cache = static_cast<uint8_t*>(d_vcache_) + l * kvd * S * kv_elem;
  at.out = d_attn_;
  at.part_ml = d_part_ml_;
  at.part_acc = d_part_acc_;
  at.H = uint32_t(arch_.num_attn_heads);
  at.KV = uint32_t(arch_.num_kv_heads);
  at.hd = uint32_t(arch_.head_dim);
  at.max_seq = uint32_t(S);
  at.n_chunks = n_chunks_;
  at.chunk = attn_chunk(at.hd, at.KV);
  at.kv_f16 = cfg_.kv_f16 ? 1 : 0;
  at.scale = 1.0f / std::sqrt(float(arch_.head_dim));
  return at;
}

EmbedArgs Engine::embed_args() const {
  EmbedArgs e{};
  e.image = d_image_;
  e.image_len = image_len_;
  e.state = d_state_;
  e.hidden = d_hidden_;
  e.D = uint32_t(arch_.hidden_dim);
  e.kind = embed_kind_;
  e.record_count = record_count_;
  e.stride = stride_;
  e.cell_off = is_dense_ ? 0 : kPrefetchBytes;
  e.rope_cos = d_rope_cos_;
  e.rope_sin = d_rope_sin_;
  e.rope_cur = d_rope_cur_;
  e.rope_half = rope_dim_ / 2;
  e.rope_rows = uint32_t(cfg_.max_seq_len);
  return e;
}

int Engine::set_state(const StepState& s) {
  *h_state_ = s;
  h_pos_ = s.pos;
  if (hipMemcpyAsync(d_state_, h_state_, sizeof(StepState), hipMemcpyHostToDevice, stream_) != hipSuccess) return -3;
  if (cfg_.hybrid && s.pos == 0) reset_hybrid_state(stream_);  // a new sequence
  // the first step's input; with embed_fused_ every step's k_finish embeds the next token
  if (embed_fused_) launch_embed(embed_args(), stream_);
  return hipGetLastError() == hipSuccess ? 0 : -3;
}

// One decode step (forwardDecode :1663-1803) on the device: its input hidden state is already in
// place (set_state, or the previous step's k_finish).
void Engine::record_step(hipStream_t st) {
  if (cfg_.hybrid) {
    record_step_hybrid(st);
    return;
  }
  const uint32_t D = uint32_t(arch_.hidden_dim), I = uint32_t(arch_.intermediate_dim);
  if (!embed_fused_) launch_embed(embed_args(), st);
  // begin/end events of every launch of one stage (time_stage_live; never during capture)
  auto mark = [&](int stage) {
    if (probe_stage_ != stage) return;
    arm_launch_probe(probe_events_[probe_next_], probe_events_[probe_next_ + 1]);
    probe_next_ += 2;
  };
  for (size_t l = 0; l < arch_.num_layers; ++l) {
    const LayerPlan& L = layers_[l];
    mark(0);
    enqueue_qkv(l, st);
    const AttnArgs aa = attn_args(l);
    mark(5);
    launch_attention_partial(aa, st);
    mark(6);
    launch_attention_combine(aa, st);
    const ProjPlan* o[1] = {&L.o};
    float* hid[2] = {d_hidden_, d_hidden_};
    mark(1);
    enqueue_gemv(o, hid, 1, GemvMode::Accum, d_attn_, D, nullptr, st);
    const ProjPlan* gu[2] = {&L.gate, &L.up};
    float* mlp[2] = {d_mlp_, d_mlp_};
    mark(2);
    enqueue_gemv(gu, mlp, 2, GemvMode::SwiGlu, d_hidden_, D, L.gamma_post, st);
    const ProjPlan* dn[1] = {&L.down};
    mark(3);
    enqueue_gemv(dn, hid, 1, GemvMode::Accum, d_mlp_, I, nullptr, st);
  }
  const ProjPlan* lm[1] = {&lm_head_};
  float* lg[1] = {d_logits_};
  mark(4);
  const uint32_t n_partials = enqueue_gemv(lm, lg, 1, GemvMode::Logits, d_hidden_, D, d_gamma_final_, st);
  FinishArgs f{d_state_, d_prompt_, d_partials_, n_partials, d_logits_, d_result_, d_out_tokens_, embed_args(),
               embed_fused_ ? 1u : 0u};
  launch_finish(f, st);
}

int Engine::read_result(ForwardResult* out) const {
  if (hipMemcpy(h_result_, d_result_, sizeof(StepResult), hipMemcpyDeviceToHost) != hipSuccess) return -3;
  out->argmax_token = h_result_->argmax;
  out->max_logit = h_result_->max_logit;
  out->token0_logit = h_result_->token0_logit;
  out->hidden_norm = h_result_->hidden_norm;
  out->all_finite = h_result_->all_finite != 0;
  return 0;
}

int Engine::forward(uint32_t token, size_t pos, ForwardResult* out) {
  if (pos >= cfg_.max_seq_len) return -2;  // the reference reads past its KV cache here
  const uint64_t t0 = now_ns();
  if (set_state(StepState{token, uint32_t(pos), 0, 0})) return -3;
  if (launch_one()) return -3;
  if (hipMemcpyAsync(h_result_, d_result_, sizeof(StepResult), hipMemcpyDeviceToHost, stream_) != hipSuccess) return -3;
  if (hipStreamSynchronize(stream_) != hipSuccess) return -3;
  const uint64_t t1 = now_ns();
  out->argmax_token = h_result_->argmax;
  out->max_logit = h_result_->max_logit;
  out->token0_logit = h_result_->token0_logit;
  out->hidden_norm = h_result_->hidden_norm;
  out->all_finite = h_result_->all_finite != 0;
  out->elapsed_ns = t1 - t0;
  return 0;
}

int Engine::launch_steps(size_t n) {
  if (h_pos_ + n > cfg_.max_seq_len) return -2;  // a step at max_seq_len would write past the KV cache
  for (size_t i = 0; i < n; ++i)
    if (launch_one()) return -3;
  return 0;
}

int Engine::time_stage_live(int stage, size_t n_steps, double* avg_ms, size_t* launches) {
  if (stage < 0 || stage > 6 || n_steps == 0) return -1;
  if (cfg_.hybrid && stage != 2 && stage != 3 && stage != 4) return -1;  // (the stages both layer kinds share)
  if (h_pos_ + n_steps > cfg_.max_seq_len) return -2;
  const size_t per_step = stage == 4 ? 1 : arch_.num_layers;
  const size_t n = per_step * n_steps;
  std::vector<hipEvent_t> ev(2 * n, nullptr);
  int rc = 0;
  for (auto& x : ev)
    if (hipEventCreate(&x) != hipSuccess) rc = -3;
  if (rc == 0) {
    probe_stage_ = stage;
    probe_events_ = ev.data();
    probe_next_ = 0;
    for (size_t i = 0; i < n_steps; ++i) record_step(stream_);  // direct launches
    h_pos_ += n_steps;
    probe_stage_ = -1;
    if (hipStreamSynchronize(stream_) != hipSuccess || probe_next_ != 2 * n) rc = -3;
  }
  double total = 0.0;
  for (size_t i = 0; rc == 0 && i < n; ++i) {
    float ms = 0.0f;
    if (hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]) != hipSuccess) rc = -3;
    total += ms;
  }
  for (auto& x : ev)
    if (x) (void)hipEventDestroy(x);
  if (rc == 0) {
    *avg_ms = total / double(n);
    *launches = n;
  }
  return rc;
}

int Engine::sync() { return hipStreamSynchronize(stream_) == hipSuccess ? 0 : -3; }

int Engine::forward_tokens(const uint32_t* toks, size_t n, ForwardResult* out) {
  if (n == 0 || !toks) return -1;
  if (n > cfg_.max_seq_len) return -2;
  if (hipMemcpyAsync(d_prompt_, toks, n * 4, hipMemcpyHostToDevice, stream_) != hipSuccess) return -3;
  if (set_state(StepState{toks[0], 0, uint32_t(n), 0})) return -3;
  if (launch_steps(n - 1)) return -3;
  if (sync()) return -3;
  const uint64_t t0 = now_ns();
  if (launch_steps(1)) return -3;
  if (hipMemcpyAsync(h_result_, d_result_, sizeof(StepResult), hipMemcpyDeviceToHost, stream_) != hipSuccess) return -3;
  if (sync()) return -3;
  const uint64_t t1 = now_ns();
  out->argmax_token = h_result_->argmax;
  out->max_logit = h_result_->max_logit;
  out->token0_logit = h_result_->token0_logit;
  out->hidden_norm = h_result_->hidden_norm;
  out->all_finite = h_result_->all_finite != 0;
  out->elapsed_ns = t1 - t0;
  return 0;
}

int Engine::generate(const uint32_t* prompt, size_t n_prompt, size_t n_gen, uint32_t* out_tokens,
                     ForwardResult* last) {
  if (n_prompt == 0 || !prompt || n_gen == 0) return -1;
  const size_t steps = n_prompt + n_gen - 1;
  if (steps > cfg_.max_seq_len) return -2;
  if (hipMemcpyAsync(d_prompt_, prompt, n_prompt * 4, hipMemcpyHostToDevice, stream_) != hipSuccess) return -3;
  if (set_state(StepState{prompt[0], 0, uint32_t(n_prompt), 0})) return -3;
  if (launch_steps(steps)) return -3;
  if (sync()) return -3;
  if (out_tokens &&
      hipMemcpy(out_tokens, d_out_tokens_ + (n_prompt - 1), n_gen * 4, hipMemcpyDeviceToHost) != hipSuccess)
    return -3;
  if (last && read_result(last)) return -3;
  return 0;
}

int Engine::verify(const uint32_t* drafts, size_t m, size_t pos, uint32_t* out_argmax, ForwardResult* last) {
  if (!drafts || m == 0 || !out_argmax) return -1;
  if (pos + m > cfg_.max_seq_len) return -2;
  if (block_ok_ && m >= 2 && m <= kMaxBlock) {  // every weight read once for the m drafts (one
                                                  // draft: the batch-1 step's kernels are faster)
    ForwardResult r{};
    const int rc = block_forward(drafts, m, pos, out_argmax, &r);
    if (rc) return rc;
    if (last) *last = r;
    // the decode state the sequential path leaves: the last argmax at position pos + m
    if (set_state(StepState{r.argmax_token, uint32_t(pos + m), 0, 0}) || sync()) return -3;
    return 0;
  }
  const uint64_t t0 = now_ns();
  // the drafts take the prompt slots of their positions, so every step is teacher-forced
  if (hipMemcpyAsync(d_prompt_ + pos, drafts, m * 4, hipMemcpyHostToDevice, stream_) != hipSuccess) return -3;
  if (set_state(StepState{drafts[0], uint32_t(pos), uint32_t(pos + m), 0})) return -3;
  if (launch_steps(m)) return -3;
  if (sync()) return -3;
  if (hipMemcpy(out_argmax, d_out_tokens_ + pos, m * 4, hipMemcpyDeviceToHost) != hipSuccess) return -3;
  if (last) {
    if (read_result(last)) return -3;
    last->elapsed_ns = now_ns() - t0;
  }
  return 0;
}

// ---- the block step ---------------------------------------------------------------------------
// Returns false with *err empty when the archive has no block step (a projection that is not
// flat 4- or 2-bit tiles), false with *err set on an allocation failure.
bool Engine::plan_block(std::string* err) {
  block_ok_ = false;
  const size_t D = arch_.hidden_dim, I = arch_.intermediate_dim, V = arch_.vocab_size;
  const size_t qd = arch_.num_attn_heads * arch_.head_dim, kvd = arch_.num_kv_heads * arch_.head_dim;
  // flat 4- or 2-bit tiles, one code width per launch (the q/k/v parts, gate and up alike); 16-row
  // 4-bit group-128 cells at 2048 columns hold their codes and scales exactly as 2048-column flat
  // tiles do (16 rows x 1024 B, f16[16][16]), so the block GEMV reads them as such, their outliers
  // as per-row corrections (plan_cell_corrections)
  auto flat = [](const ProjPlan& p) {
    return p.kind == WeightKind::FlatW4 || p.kind == WeightKind::FlatW2 || (p.kind == WeightKind::Cell16W4 && p.cols == 2048);
  };
  auto bits_of = [](const ProjPlan& p) { return p.kind == WeightKind::FlatW2 ? 2 : 4; };
  for (size_t l = 0; l < layers_.size(); ++l) {
    const LayerPlan& L = layers_[l];
    if (!flat(L.gate) || !flat(L.up) || !flat(L.down) || bits_of(L.up) != bits_of(L.gate)) return false;
    if (cfg_.hybrid) {  // the hybrid's mixers (HybLayer) instead of the q/k/v/o plans
      const HybLayer& H = hyb_[l];
      if (!flat(H.in0) || !flat(H.in1) || !flat(H.in2) || !flat(H.out) || bits_of(H.in1) != bits_of(H.in0) ||
          bits_of(H.in2) != bits_of(H.in0) || (!H.full && !flat(H.in3)) || (H.has_ab && !flat(H.ab)))
        return false;
      continue;
    }
    if (!flat(L.q) || !flat(L.k) || !flat(L.v) || !flat(L.o) || bits_of(L.k) != bits_of(L.q) ||
        bits_of(L.v) != bits_of(L.q))
      return false;
  }
  // (the o projection reads the attention output of qd columns as hidden_dim columns, as the
  // reference's gemvLinear call does, :1737: the two must agree)
  if (!flat(lm_head_) || D % 128 || I % 128 || qd % 128 || qd != D) return false;
  for (LayerPlan& L : layers_)
    for (ProjPlan* p : {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down})
      if (p->kind == WeightKind::Cell16W4 && !plan_cell_corrections(p, p->cols, err)) return false;
  if (lm_head_.kind == WeightKind::Cell16W4 && !plan_cell_corrections(&lm_head_, D, err)) return false;
  auto units = [](size_t rows) { return (rows + kBlockUnit - 1) / kBlockUnit; };
  size_t part_floats = 0;  // ranges x kMaxBlock x rows_all, the largest GEMV at any token count
  auto need = [&](size_t n_units, size_t C) {
    const size_t r = std::max(block_gemv_ranges(uint32_t(n_units), uint32_t(C), kSmallBlock),
                              block_gemv_ranges(uint32_t(n_units), uint32_t(C), kMaxBlock));
    part_floats = std::max(part_floats, r * kBlockUnit * n_units);
  };
  need(units(qd) + 2 * units(kvd), D);
  need(units(D), qd);
  need(2 * units(I), D);
  need(units(D), I);
  need(units(V), D);
  if (cfg_.hybrid) {  // in_proj_qkv + z + a/b (8192 + 4096 + 64 rows), q + k + v (8192 + 2 x 1024), out_proj
    need(units(8192) + units(4096) + units(64), D);
    need(units(8192) + 2 * units(1024), D);
    need(units(D), 4096);
  }
  part_floats *= kMaxBlock;
  const size_t Cmax = std::max({D, I, qd}), ngm = Cmax / 128, nq = (kMaxBlock + 3) / 4;
  const size_t hd = arch_.head_dim, H = arch_.num_attn_heads;
  auto fa = [&](size_t n) { return static_cast<float*>(dev_alloc(n * 4)); };
  d_btok_ = static_cast<uint32_t*>(dev_alloc(kMaxBlock * 4));
  d_bout_ = static_cast<uint32_t*>(dev_alloc(kMaxBlock * 4));
  d_bstate_ = static_cast<StepState*>(dev_alloc(sizeof(StepState)));
  d_bbrk_ = static_cast<uint32_t*>(dev_alloc(kMaxBlock * 4));
  d_bx_ = fa(kMaxBlock * D);
  d_bq_ = fa(kMaxBlock * qd);
  d_battn_ = fa(kMaxBlock * qd);
  d_bmlp_ = fa(kMaxBlock * I);
  d_blog_ = fa(kMaxBlock * V);
  d_bpartial_ = fa(part_floats);
  bpart_floats_ = part_floats;
  d_bpml_ = fa(kMaxBlock * H * n_chunks_ * 2);
  d_bpacc_ = fa(kMaxBlock * H * n_chunks_ * hd);
  d_bss_ = fa(size_t(kMaxSsPartials) * kMaxBlock);
  btab_.tb = static_cast<uint4*>(dev_alloc(nq * ngm * 128 * sizeof(uint4)));
  btab_.ci = static_cast<int4*>(dev_alloc(nq * ngm * 4 * sizeof(int4)));
  btab_.ew = fa(nq * ngm * 4);
  btab_.xt = fa(Cmax * kMaxBlock);
  btab_.ss = fa(kMaxBlock);
  d_bpartials_ = static_cast<ArgmaxPartial*>(dev_alloc(kMaxBlock * 512 * sizeof(ArgmaxPartial)));
  if (cfg_.hybrid) {
    d_bhx0_ = fa(kMaxBlock * 8192);
    d_bhx1_ = fa(kMaxBlock * 4096);
    d_bhx2_ = fa(kMaxBlock * 1024);
    d_bhx3_ = fa(kMaxBlock * 32);
    d_bhconv_ = fa(kMaxBlock * 8192);
    if (!d_bhx0_ || !d_bhx1_ || !d_bhx2_ || !d_bhx3_ || !d_bhconv_) {
      *err = "allocation";
      return false;
    }
  }
  if (!d_btok_ || !d_bout_ || !d_bstate_ || !d_bbrk_ || !d_bx_ || !d_bq_ || !d_battn_ || !d_bmlp_ || !d_blog_ || !d_bpartial_ ||
      !d_bpml_ || !d_bpacc_ || !d_bss_ || !btab_.tb || !btab_.ci || !btab_.ew || !btab_.xt || !btab_.ss ||
      !d_bpartials_) {
    *err = "allocation";
    return false;
  }
  if (hipHostMalloc(reinterpret_cast<void**>(&h_btok_), kMaxBlock * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc(reinterpret_cast<void**>(&h_bout_), kMaxBlock * 4, hipHostMallocDefault) != hipSuccess ||
      hipHostMalloc(reinterpret_cast<void**>(&h_bstate_), sizeof(StepState), hipHostMallocDefault) != hipSuccess) {
    *err = "pinned allocation";
    return false;
  }
  block_ok_ = true;
  return true;
}

// A 16-row cell tensor's outliers for the block step, [rows][8] (column bits, weight): added
// outliers (gemvTileW4 :404-410: the cell's 8 columns, each row's 8 f16 weights times the input
// there, columns past the input giving 0), or for the tied LM head the replace tables' additive
// deltas (w_out - dequantised code, prepared at load).
bool Engine::plan_cell_corrections(ProjPlan* p, size_t C, std::string* err) {
  const size_t rows = p->rows, n_cells = (rows + 15) / 16;
  std::vector<float2> corr(rows * 8, make_float2(0.0f, 0.0f));
  const size_t off0 = size_t(p->base - d_image_);  // (the archive offset of the first cell)
  for (size_t t = 0; t < n_cells; ++t) {
    const size_t pl = off0 + t * p->stride + kPayloadOff;
    for (size_t n = 0; n < 16 && 16 * t + n < rows; ++n)
      for (int k = 0; k < 8; ++k) {
        uint32_t col = 0;
        float w = 0.0f;
        if (p->replace_outliers) {
          const CellReplace& R = lm_repl_host_[t];
          col = R.col[k];
          w = R.delta[n][k];
        } else {
          col = rd<uint16_t>(host_bytes_, len_, pl + kRowOutlierCols + 2 * k);
          w = f16_to_f32(rd<uint16_t>(host_bytes_, len_, pl + kRowOutlierW + 2 * (n * 8 + k)));
        }
        if (col >= C) w = 0.0f;  // (its input is 0: no term)
        const uint32_t cb = w == 0.0f ? 0u : col;  // (the column's bits, as the flat tables hold it)
        float cf;
        std::memcpy(&cf, &cb, 4);
        corr[(16 * t + n) * 8 + k] = make_float2(cf, w);
      }
  }
  p->bcorr = static_cast<float2*>(dev_alloc(corr.size() * sizeof(float2)));
  if (!p->bcorr) {
    *err = "allocation";
    return false;
  }
  (void)hipMemcpy(p->bcorr, corr.data(), corr.size() * sizeof(float2), hipMemcpyHostToDevice);
  p->bcorr_kmax = 8;
  if (!plan_packed_corrections(corr, rows, 8, p)) {
    *err = "allocation";
    return false;
  }
  return true;
}

// The block epilogue's form of a [rows][kmax] correction table: only the entries with a
// non-zero weight (a zero-weight entry -- padding, or an outlier equal to its code's value --
// adds no term), row after row in entry order, and each row's first entry, so that a row's
// loop runs over its own entries instead of the table's widest row.  The terms and their order
// are those of the padded table.
bool Engine::plan_packed_corrections(const std::vector<float2>& padded, size_t rows, uint32_t kmax, ProjPlan* p) {
  std::vector<uint32_t> off(rows + 1);
  std::vector<float2> pk;
  pk.reserve(padded.size());
  for (size_t r = 0; r < rows; ++r) {
    off[r] = uint32_t(pk.size());
    for (uint32_t k = 0; k < kmax; ++k) {
      const float2 e = padded[r * kmax + k];
      if (e.y != 0.0f) pk.push_back(e);  // (a NaN weight stays: it makes the row NaN)
    }
  }
  off[rows] = uint32_t(pk.size());
  if (pk.empty()) pk.push_back(make_float2(0.0f, 0.0f));  // (an allocation; no row reads it)
  p->boff = static_cast<uint32_t*>(dev_alloc(off.size() * sizeof(uint32_t)));
  p->bpack = static_cast<float2*>(dev_alloc(pk.size() * sizeof(float2)));
  if (!p->boff || !p->bpack) return false;
  (void)hipMemcpy(p->boff, off.data(), off.size() * sizeof(uint32_t), hipMemcpyHostToDevice);
  (void)hipMemcpy(p->bpack, pk.data(), pk.size() * sizeof(float2), hipMemcpyHostToDevice);
  return true;
}

uint32_t Engine::enqueue_block_gemv(const ProjPlan* const* parts, float* const* outs, int n, GemvMode mode,
                                    const float* x, uint32_t C, const float* gamma, uint32_t n_ss, uint32_t m,
                                    size_t layer, hipStream_t st, const uint32_t* roles_in, uint32_t pair_dim) {
  BlockGemvArgs b{};
  b.g.n_parts = n;
  b.g.mode = int(mode);
  b.g.C = C;
  b.g.x = x;
  b.g.gamma = gamma;
  b.g.eps = arch_.rms_eps;
  uint32_t units = 0;
  const uint32_t roles[3] = {kRoleQ, kRoleK, kRoleV};
  for (int i = 0; i < n; ++i) {
    const ProjPlan& p = *parts[i];
    GemvPart& gp = b.g.part[i];
    gp.base = p.base;
    gp.stride = p.stride;
    gp.rows = p.rows;
    gp.wrows = p.wrows ? p.wrows : p.rows;
    gp.unit_begin = units;
    gp.y = outs[i];
    gp.bias = p.bias;
    gp.corr = p.bcorr ? p.bcorr : p.corr;
    gp.corr_kmax = p.bcorr ? p.bcorr_kmax : p.corr_kmax;
    b.cpack[i] = gp.corr ? p.bpack : nullptr;
    b.coff[i] = gp.corr ? p.boff : nullptr;
    if (gp.corr && !p.boff) {  // (every block-step part's table has its packed form: plan_projection, plan_block)
      bpart_short_ = true;
      return 1;
    }
    gp.rope_role = mode == GemvMode::QkvRope ? (roles_in ? roles_in[i] : roles[i]) : 0u;
    units += (p.rows + kBlockUnit - 1) / kBlockUnit;
  }
  b.t = btab_;
  b.bits = parts[0]->kind == WeightKind::FlatW2 ? 2u : 4u;  // (16-row cells: 4, read as flat tiles)
  b.m = m;
  b.nq = (m + 3) / 4;
  b.ts = m <= kSmallBlock ? kSmallBlock : kMaxBlock;
  b.n_units = units;
  b.rows_all = kBlockUnit * units;
  b.partial = d_bpartial_;
  b.brk = d_bbrk_;
  if (size_t(block_gemv_ranges(units, C, m)) * b.rows_all * kMaxBlock > bpart_floats_) {  // (the plan's sizes)
    bpart_short_ = true;
    return 1;
  }
  if (mode == GemvMode::QkvRope) {
    b.g.rope = rope_args(layer);
    if (pair_dim) b.g.rope.head_dim = pair_dim;
    b.state = d_bstate_;
    b.rope_cos = d_rope_cos_;
    b.rope_sin = d_rope_sin_;
    b.rope_rows = uint32_t(cfg_.max_seq_len);
  }
  if (mode == GemvMode::Logits) b.partials = d_bpartials_;
  b.ssp = d_bss_;
  b.n_ssp = n_ss;
  if (mode == GemvMode::Accum) b.ssp_out = d_bss_;  // (read by this GEMV's kernels: no gamma)
  launch_block_limbs(b, st);
  return launch_block_gemv(b, st);
}

int Engine::block_forward(const uint32_t* tokens, size_t m, size_t pos, uint32_t* out_argmax, ForwardResult* last,
                          bool head) {
  if (!block_ok_ || !tokens || m == 0 || m > kMaxBlock || (!head && (out_argmax || last))) return -1;
  if (pos + m > cfg_.max_seq_len) return -2;
  const uint64_t t0 = now_ns();
  const uint32_t mm = uint32_t(m);
  hipStream_t st = stream_;
  std::memcpy(h_btok_, tokens, m * 4);
  *h_bstate_ = StepState{tokens[0], uint32_t(pos), 0, 0};
  if (hipMemcpyAsync(d_btok_, h_btok_, m * 4, hipMemcpyHostToDevice, st) != hipSuccess ||
      hipMemcpyAsync(d_bstate_, h_bstate_, sizeof(StepState), hipMemcpyHostToDevice, st) != hipSuccess)
    return -3;
  if (cfg_.hybrid && pos == 0) reset_hybrid_state(st);  // a new sequence (outside the graph)
  bhead_ = head;
  if (use_graph_) {  // one captured graph per (head, token count), captured on first use
    hipGraph_t& g = bgraph_[head ? 1 : 0][m];
    hipGraphExec_t& ge = bgraph_exec_[head ? 1 : 0][m];
    if (!ge) {
      if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) return -3;
      record_block(mm, st);
      if (hipStreamEndCapture(st, &g) != hipSuccess) return -3;
      if (bpart_short_) {
        (void)hipGraphDestroy(g);
        g = nullptr;
        return -3;
      }
      if (hipGraphInstantiate(&ge, g, nullptr, nullptr, 0) != hipSuccess) return -3;
    }
    if (hipGraphLaunch(ge, st) != hipSuccess) return -3;
  } else {
    record_block(mm, st);
    if (bpart_short_) {
      (void)hipStreamSynchronize(st);
      return -3;
    }
  }
  if (!head) return hipStreamSynchronize(st) == hipSuccess ? 0 : -3;
  if (hipMemcpyAsync(h_bout_, d_bout_, m * 4, hipMemcpyDeviceToHost, st) != hipSuccess ||
      hipMemcpyAsync(h_result_, d_result_, sizeof(StepResult), hipMemcpyDeviceToHost, st) != hipSuccess)
    return -3;
  if (hipStreamSynchronize(st) != hipSuccess) return -3;
  if (out_argmax) std::memcpy(out_argmax, h_bout_, m * 4);
  if (last) {
    last->argmax_token = h_result_->argmax;
    last->max_logit = h_result_->max_logit;
    last->token0_logit = h_result_->token0_logit;
    last->hidden_norm = h_result_->hidden_norm;
    last->all_finite = h_result_->all_finite != 0;
    last->elapsed_ns = now_ns() - t0;
  }
  return 0;
}

void Engine::record_block(uint32_t mm, hipStream_t st) {
  if (cfg_.hybrid) {
    record_block_hybrid(mm, st);
    return;
  }
  const uint32_t D = uint32_t(arch_.hidden_dim), I = uint32_t(arch_.intermediate_dim), V = uint32_t(arch_.vocab_size);
  const uint32_t qd = uint32_t(arch_.num_attn_heads * arch_.head_dim);
  launch_block_embed(embed_args(), d_btok_, mm, d_bx_, d_bss_, d_bbrk_, st);
  uint32_t n_ss = 1;  // Σx² partials of the hidden rows in d_bss_
  for (size_t l = 0; l < arch_.num_layers; ++l) {
    const LayerPlan& L = layers_[l];
    const ProjPlan* qkv[3] = {&L.q, &L.k, &L.v};
    float* qo[3] = {d_bq_, nullptr, nullptr};
    enqueue_block_gemv(qkv, qo, 3, GemvMode::QkvRope, d_bx_, D, L.gamma_in, n_ss, mm, l, st);
    AttnArgs at = attn_args(l);
    at.state = d_bstate_;
    at.q = d_bq_;
    at.out = d_battn_;
    at.part_ml = d_bpml_;
    at.part_acc = d_bpacc_;
    at.nq = mm;
    launch_attention(at, st);
    const ProjPlan* o[1] = {&L.o};
    float* hid[1] = {d_bx_};
    n_ss = enqueue_block_gemv(o, hid, 1, GemvMode::Accum, d_battn_, qd, nullptr, 0, mm, l, st);
    const ProjPlan* gu[2] = {&L.gate, &L.up};
    float* mlp[2] = {d_bmlp_, d_bmlp_};
    enqueue_block_gemv(gu, mlp, 2, GemvMode::SwiGlu, d_bx_, D, L.gamma_post, n_ss, mm, l, st);
    const ProjPlan* dn[1] = {&L.down};
    n_ss = enqueue_block_gemv(dn, hid, 1, GemvMode::Accum, d_bmlp_, I, nullptr, 0, mm, l, st);
  }
  if (!bhead_) return;  // (a prefill block before the last: its logits are not read)
  const ProjPlan* lm[1] = {&lm_head_};
  float* lg[1] = {d_blog_};
  const uint32_t eb = enqueue_block_gemv(lm, lg, 1, GemvMode::Logits, d_bx_, D, d_gamma_final_, n_ss, mm, 0, st);
  launch_block_finish(BlockFinishArgs{d_bpartials_, eb, mm, d_blog_, V, btab_.ss, d_bout_, d_result_}, st);
  (void)hipMemcpyAsync(d_logits_, d_blog_ + size_t(mm - 1) * V, size_t(V) * 4, hipMemcpyDeviceToDevice, st);
}

// The hybrid model's block step: record_step_hybrid's layers for m tokens, every weight read once
// (k_gemv_mt), the DeltaNet states rolled over the m tokens in order inside one launch each
// (launch_dn_block), the gated attention layers' q / k norms, rotary embedding and KV append per
// token (k_hyb_qk over the tokens) and the multi-query decode attention.
void Engine::record_block_hybrid(uint32_t mm, hipStream_t st) {
  const uint32_t D = uint32_t(arch_.hidden_dim), I = uint32_t(arch_.intermediate_dim), V = uint32_t(arch_.vocab_size);
  const uint32_t H = uint32_t(arch_.num_attn_heads), KV = uint32_t(arch_.num_kv_heads), hd = uint32_t(arch_.head_dim);
  const uint32_t store[3] = {kRoleStore, kRoleStore, kRoleStore};
  launch_block_embed(embed_args(), d_btok_, mm, d_bx_, d_bss_, d_bbrk_, st);
  uint32_t n_ss = 1;
  for (size_t l = 0; l < arch_.num_layers; ++l) {
    const LayerPlan& L = layers_[l];
    const HybLayer& Hy = hyb_[l];
    float* hid[1] = {d_bx_};
    const ProjPlan* in[3] = {&Hy.in0, &Hy.in1, (!Hy.full && Hy.has_ab) ? &Hy.ab : &Hy.in2};
    float* outs[3] = {d_bhx0_, d_bhx1_, d_bhx2_};
    enqueue_block_gemv(in, outs, 3, GemvMode::QkvRope, d_bx_, D, L.gamma_in, n_ss, mm, l, st, store, 32);
    if (Hy.full) {
      const RopeArgs kv = rope_args(l);
      HybQkArgs q{};
      q.state = d_bstate_;
      q.qg = d_bhx0_;
      q.k = d_bhx1_;
      q.v = d_bhx2_;
      q.q_norm = Hy.q_norm;
      q.k_norm = Hy.k_norm;
      q.rope_cos = d_rope_cos_;
      q.rope_sin = d_rope_sin_;
      q.q_out = d_bq_;
      q.k_cache = kv.k_cache;
      q.v_cache = kv.v_cache;
      q.H = H;
      q.KV = KV;
      q.hd = hd;
      q.rot = rope_dim_;
      q.max_seq = kv.max_seq;
      q.kv_f16 = kv.kv_f16;
      q.rope_rows = uint32_t(cfg_.max_seq_len);
      q.eps = arch_.rms_eps;
      q.m = mm;
      q.qg_stride = 8192;
      q.kv_stride = 1024;
      q.q_stride = H * hd;
      q.brk = d_bbrk_;
      launch_hyb_qk(q, st);
      AttnArgs at = attn_args(l);
      at.state = d_bstate_;
      at.q = d_bq_;
      at.out = d_battn_;
      at.part_ml = d_bpml_;
      at.part_acc = d_bpacc_;
      at.nq = mm;
      at.gate = d_bhx0_;  // (the output gate applied by the merge)
      launch_attention(at, st);
    } else {
      if (!Hy.has_ab) {
        const ProjPlan* inb[1] = {&Hy.in3};
        float* outb[1] = {d_bhx3_};
        enqueue_block_gemv(inb, outb, 1, GemvMode::QkvRope, d_bx_, D, L.gamma_in, n_ss, mm, l, st, store, 32);
      }
      DnBlockArgs dn{};
      dn.x = d_bhx0_;
      dn.w = Hy.conv_w;
      dn.conv_state = d_conv_state_ + size_t(Hy.lin) * 8192 * 3;
      dn.conv_out = d_bhconv_;
      dn.channels = 8192;
      dn.taps = 4;
      dn.x_stride = 8192;
      dn.a = d_bhx2_;
      dn.b = Hy.has_ab ? d_bhx2_ + 32 : d_bhx3_;
      dn.ab_stride = Hy.has_ab ? 64 : 32;
      dn.A_log = Hy.A_log;
      dn.dt_bias = Hy.dt_bias;
      dn.z = d_bhx1_;
      dn.z_stride = 4096;
      dn.norm_w = Hy.lin_norm;
      dn.state = d_rec_state_ + size_t(Hy.lin) * 32 * 128 * 128;
      dn.out = d_battn_;
      dn.out_stride = 4096;
      dn.n_v_heads = 32;
      dn.n_k_heads = 16;
      dn.head_dim = 128;
      dn.m = mm;
      dn.eps = arch_.rms_eps;
      dn.brk = d_bbrk_;
      launch_dn_block(dn, st);
    }
    const ProjPlan* o[1] = {&Hy.out};
    n_ss = enqueue_block_gemv(o, hid, 1, GemvMode::Accum, d_battn_, 4096, nullptr, 0, mm, l, st);
    const ProjPlan* gu[2] = {&L.gate, &L.up};
    float* mlp[2] = {d_bmlp_, d_bmlp_};
    enqueue_block_gemv(gu, mlp, 2, GemvMode::SwiGlu, d_bx_, D, L.gamma_post, n_ss, mm, l, st);
    const ProjPlan* dnp[1] = {&L.down};
    n_ss = enqueue_block_gemv(dnp, hid, 1, GemvMode::Accum, d_bmlp_, I, nullptr, 0, mm, l, st);
  }
  if (!bhead_) return;  // (a prefill block before the last: its logits are not read)
  const ProjPlan* lm[1] = {&lm_head_};
  float* lg[1] = {d_blog_};
  const uint32_t eb = enqueue_block_gemv(lm, lg, 1, GemvMode::Logits, d_bx_, D, d_gamma_final_, n_ss, mm, 0, st);
  launch_block_finish(BlockFinishArgs{d_bpartials_, eb, mm, d_blog_, V, btab_.ss, d_bout_, d_result_}, st);
  (void)hipMemcpyAsync(d_logits_, d_blog_ + size_t(mm - 1) * V, size_t(V) * 4, hipMemcpyDeviceToDevice, st);
}

int Engine::prefill(const uint32_t* tokens, size_t n, ForwardResult* out) {
  if (!tokens || n == 0 || !out) return -1;
  if (n > cfg_.max_seq_len) return -2;
  if (!block_ok_) {  // no block step for this archive: sequential steps
    const int rc = forward_tokens(tokens, n, out);
    if (rc) return rc;
    h_pos_ = n;
    return 0;
  }
  uint32_t am[kMaxBlock];
  for (size_t i = 0; i < n; i += kMaxBlock) {
    const size_t m = std::min<size_t>(kMaxBlock, n - i);
    const bool head = i + m == n;  // (only the last block's logits are read)
    const int rc = block_forward(tokens + i, m, i, head ? am : nullptr, head ? out : nullptr, head);
    if (rc) return rc;
  }
  // continue greedy decoding from here: the last argmax at position n
  if (set_state(StepState{out->argmax_token, uint32_t(n), 0, 0})) return -3;
  return sync();
}

int Engine::copy_logits(float* out) const {
  return hipMemcpy(out, d_logits_, arch_.vocab_size * 4, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -3;
}

int Engine::copy_hidden(float* out) const {
  const float* h = embed_fused_ ? d_hidden_out_ : d_hidden_;
  return hipMemcpy(out, h, arch_.hidden_dim * 4, hipMemcpyDeviceToHost) == hipSuccess ? 0 : -3;
}

double Engine::proj_bytes(const ProjPlan& p) const {
  // algorithmic bytes: codes + group scales + outliers (+ bias); no headers or padding
  const double n = double(p.rows) * p.cols;
  double bytes = 0.0;
  switch (p.kind) {
    case WeightKind::Raw16: bytes = 2.0 * n; break;
    case WeightKind::Raw8: bytes = n; break;
    case WeightKind::Cell16W4: bytes = n / 2 + n / 128 * 2 + double(p.rows / 16) * (16 * 8 * 2 + 8 * 2); break;
    case WeightKind::FlatW4: bytes = n / 2 + n / 128 * 2 + std::ceil(n / kFlatWeights) * (2 + 64 * 4); break;
    case WeightKind::FlatW2: bytes = n / 4 + n / 128 * 2 + std::ceil(n / kFlatWeights) * (2 + 64 * 4); break;
    case WeightKind::Cell16Poly: bytes = double(p.poly.n_cells) * kTileCodeBytes; break;  // the code areas
    case WeightKind::FlatPoly: bytes = double(p.poly.n_cells) * kTileCodeBytes; break;    // (at most)
  }
  if (p.bias) bytes += 4.0 * p.rows;
  return bytes;
}

double Engine::stage_bytes(int stage, size_t l) const {
  const LayerPlan& L = layers_[l];
  switch (stage) {
    case 0: return proj_bytes(L.q) + proj_bytes(L.k) + proj_bytes(L.v);
    case 1: return proj_bytes(L.o);
    case 2: return proj_bytes(L.gate) + proj_bytes(L.up);
    case 3: return proj_bytes(L.down);
    case 4: return proj_bytes(lm_head_);
    case 5:    // K and V rows 0..pos of this layer at the current device position
    case 6: {  // the partials of the chunks active at that position, read once
      StepState st{};
      if (hipStreamSynchronize(stream_) != hipSuccess ||
          hipMemcpy(&st, d_state_, sizeof(st), hipMemcpyDeviceToHost) != hipSuccess)
        return 0.0;
      if (stage == 6) {
        const double chunks =
            std::ceil((double(st.pos) + 1.0) / attn_chunk(uint32_t(arch_.head_dim), uint32_t(arch_.num_kv_heads)));
        return double(arch_.num_attn_heads) * chunks * (arch_.head_dim + 2) * 4.0;
      }
      const double kv_row = double(arch_.num_kv_heads * arch_.head_dim) * (cfg_.kv_f16 ? 2 : 4);
      return 2.0 * kv_row * (double(st.pos) + 1.0);
    }
    default: return 0.0;
  }
}

double Engine::step_bytes(size_t pos) const {
  double bytes = 0.0;
  const double D = double(arch_.hidden_dim);
  if (cfg_.hybrid) {  // weights, norms, the 8 attention layers' KV rows, the DeltaNet states (r + w)
    const double kv_row = double(arch_.num_kv_heads * arch_.head_dim) * (cfg_.kv_f16 ? 2 : 4);
    for (size_t l = 0; l < hyb_.size(); ++l) {
      const HybLayer& H = hyb_[l];
      bytes += proj_bytes(H.in0) + proj_bytes(H.in1) + proj_bytes(H.in2) + proj_bytes(H.out) + 2 * D * 4;
      bytes += stage_bytes(2, l) + stage_bytes(3, l);
      if (H.full) {
        bytes += 2 * 256 * 4 + 2 * kv_row * (double(pos) + 1) + 2 * kv_row;
      } else {
        bytes += proj_bytes(H.in3) + (8192.0 * 4 + 32 * 2 + 128) * 4;  // conv weights, A_log, dt_bias, norm
        bytes += 2.0 * (8192.0 * 3 + 32.0 * 128 * 128) * 4;            // conv and delta-rule states
      }
    }
    return bytes + stage_bytes(4, 0) + D * 4 + D * 0.5625;
  }
  for (size_t l = 0; l < arch_.num_layers; ++l)
    bytes += stage_bytes(0, l) + stage_bytes(1, l) + stage_bytes(2, l) + stage_bytes(3, l) + 2 * D * 4;
  bytes += stage_bytes(4, 0) + D * 4;                        // LM head + final norm
  bytes += D * (is_raw_ ? 2.0 : 0.5625);                     // embedding row
  const double kv_row = double(arch_.num_kv_heads * arch_.head_dim) * (cfg_.kv_f16 ? 2 : 4);
  bytes += double(arch_.num_layers) * 2 * kv_row * (double(pos) + 1);  // K and V read
  bytes += double(arch_.num_layers) * 2 * kv_row;                      // K and V written
  return bytes;
}

bool Engine::plan_hybrid(std::string* err) {
  const size_t D = arch_.hidden_dim;
  if (is_raw_ || D != 4096 || arch_.head_dim != 256 || arch_.num_attn_heads != 16 || arch_.num_kv_heads != 4) {
    *err = "the hybrid layers need the 9B cell archive";
    return false;
  }
  const uint8_t* b = host_bytes_;
  const size_t cell_off = is_dense_ ? 0 : kPrefetchBytes;
  // bf16 vectors: 8192 values per record's code area
  auto bf16vec = [&](size_t rec, size_t n) {
    std::vector<float> v(n, 0.0f);
    for (size_t i = 0; i < n; ++i) {
      const size_t r = rec + i / 8192;
      if (r < record_count_)
        v[i] = bf16_to_f32(rd<uint16_t>(b, len_, 4096 + r * stride_ + cell_off + kBytecodeHeader + 2 * (i % 8192)));
    }
    return upload_vector(v);
  };
  hyb_.resize(arch_.num_layers);
  uint32_t n_lin = 0;
  for (size_t l = 0; l < arch_.num_layers; ++l) {
    const Qwen35Records r = qwen35_records(l);
    HybLayer& H = hyb_[l];
    H.full = r.full_attn;
    std::string why;
    auto plan = [&](const char* name, size_t ts, size_t nt, size_t rows, size_t cols, bool acc, ProjPlan* p) {
      if (plan_projection(ts, nt, rows, cols, cols, rows, acc, -1, p, &why)) return true;
      *err = "hybrid layer " + std::to_string(l) + " " + name + ": " + why;
      return false;
    };
    if (H.full) {
      if (!plan("q_proj", r.q_proj, 2048, 8192, D, false, &H.in0) || !plan("k_proj", r.k_proj, 256, 1024, D, false, &H.in1) ||
          !plan("v_proj", r.v_proj, 256, 1024, D, false, &H.in2) || !plan("o_proj", r.o_proj, 1024, D, 4096, true, &H.out))
        return false;
      H.q_norm = bf16vec(r.q_norm, 256);
      H.k_norm = bf16vec(r.k_norm, 256);
      if (!H.q_norm || !H.k_norm) {
        *err = "allocation";
        return false;
      }
    } else {
      if (!plan("in_proj_qkv", r.in_proj_qkv, 2048, 8192, D, false, &H.in0) ||
          !plan("in_proj_z", r.in_proj_z, 1024, 4096, D, false, &H.in1) ||
          !plan("in_proj_a", r.in_proj_a, 8, 32, D, false, &H.in2) || !plan("in_proj_b", r.in_proj_b, 8, 32, D, false, &H.in3) ||
          !plan("out_proj", r.out_proj, 1024, D, 4096, true, &H.out))
        return false;
      {  // a and b side by side: 4 + 4 whole tiles of 8 rows each, copied record for record
        const size_t na = 4, rec_bytes = stride_;
        if (r.in_proj_a + na <= record_count_ && r.in_proj_b + na <= record_count_ &&
            H.in2.kind == WeightKind::FlatW4 && H.in3.kind == WeightKind::FlatW4 && H.in2.wrows == 32 &&
            H.in3.wrows == 32) {
          std::vector<uint8_t> ab(2 * na * rec_bytes);
          std::memcpy(ab.data(), b + 4096 + r.in_proj_a * rec_bytes, na * rec_bytes);
          std::memcpy(ab.data() + na * rec_bytes, b + 4096 + r.in_proj_b * rec_bytes, na * rec_bytes);
          FlatPlan fp;
          plan_flat(ab.data() + cell_off, ab.size() - cell_off, rec_bytes, 2 * na, 64, D, &fp);
          if (fp.kind == WeightKind::FlatW4 && fp.wrows == 64) {
            uint8_t* d = static_cast<uint8_t*>(dev_alloc(ab.size()));
            float2* dc = fp.corr.empty() ? nullptr : static_cast<float2*>(dev_alloc(fp.corr.size() * sizeof(float2)));
            if (!d || (!fp.corr.empty() && !dc)) {
              *err = "allocation";
              return false;
            }
            (void)hipMemcpy(d, ab.data(), ab.size(), hipMemcpyHostToDevice);
            if (dc) (void)hipMemcpy(dc, fp.corr.data(), fp.corr.size() * sizeof(float2), hipMemcpyHostToDevice);
            H.ab = H.in2;
            H.ab.base = d + cell_off;
            H.ab.stride = uint32_t(rec_bytes);
            H.ab.rows = H.ab.wrows = 64;
            H.ab.corr = dc;
            H.ab.corr_kmax = fp.corr_kmax;
            H.ab.bpack = nullptr;
            H.ab.boff = nullptr;
            if (dc && !plan_packed_corrections(fp.corr, 64, fp.corr_kmax, &H.ab)) {
              *err = "allocation";
              return false;
            }
            H.ab.xcodes = nullptr;
            H.has_ab = true;
          }
        }
      }
      H.conv_w = bf16vec(r.conv1d, 8192 * 4);
      H.A_log = bf16vec(r.a_log, 32);
      H.dt_bias = bf16vec(r.dt_bias, 32);
      H.lin_norm = bf16vec(r.linear_norm, 128);
      if (!H.conv_w || !H.A_log || !H.dt_bias || !H.lin_norm) {
        *err = "allocation";
        return false;
      }
      H.lin = n_lin++;
    }
  }
  auto fa = [&](size_t n) { return static_cast<float*>(dev_alloc(n * 4)); };
  d_hx0_ = fa(8192);
  d_hx1_ = fa(4096);
  d_hx2_ = fa(1024);
  d_hx3_ = fa(32);
  d_hconv_ = fa(8192);
  conv_state_floats_ = size_t(n_lin) * 8192 * 3;
  rec_state_floats_ = size_t(n_lin) * 32 * 128 * 128;
  d_conv_state_ = fa(conv_state_floats_);
  d_rec_state_ = fa(rec_state_floats_);
  if (!d_hx0_ || !d_hx1_ || !d_hx2_ || !d_hx3_ || !d_hconv_ || !d_conv_state_ || !d_rec_state_) {
    *err = "allocation";
    return false;
  }
  reset_hybrid_state(stream_);
  return true;
}

void Engine::reset_hybrid_state(hipStream_t st) {
  (void)hipMemsetAsync(d_conv_state_, 0, conv_state_floats_ * 4, st);
  (void)hipMemsetAsync(d_rec_state_, 0, rec_state_floats_ * 4, st);
}

// One decode step of the Qwen3.5-9B hybrid (the layer loop of forwardDecode :1663-1803 with the
// hybrid token mixers; see HybLayer).  Per layer: the normalised input projections (QkvRope
// launches whose parts have role kRoleStore: rows stored as computed, the break test made),
// then for a full-attention layer the q / k norms and partial rotary embedding with the KV
// append (k_hyb_qk), the decode attention, the output gate, o_proj into the residual; for a
// DeltaNet layer the conv update, the gated delta rule with the gated norm, out_proj into the
// residual; then the MLP as in record_step.
void Engine::record_step_hybrid(hipStream_t st) {
  const uint32_t D = uint32_t(arch_.hidden_dim), I = uint32_t(arch_.intermediate_dim);
  if (!embed_fused_) launch_embed(embed_args(), st);
  // (stage timing: the MLP launches and the LM head, the stages both layer kinds share)
  auto mark = [&](int stage) {
    if (probe_stage_ != stage) return;
    arm_launch_probe(probe_events_[probe_next_], probe_events_[probe_next_ + 1]);
    probe_next_ += 2;
  };
  const uint32_t store[3] = {kRoleStore, kRoleStore, kRoleStore};
  for (size_t l = 0; l < arch_.num_layers; ++l) {
    const LayerPlan& L = layers_[l];
    const HybLayer& H = hyb_[l];
    RopeArgs ra = rope_args(l);
    ra.head_dim = 32;  // (Store parts: rows pair within blocks of 32, a divisor of every part's rows)
    float* hid[1] = {d_hidden_};
    // the normalised in-projections: one launch when the parts share a weight layout, else one
    // launch per part (as enqueue_qkv)
    auto in_proj = [&](const ProjPlan* const* ps, float* const* os, int n, const uint32_t* roles) {
      bool same = true;
      for (int i = 1; i < n; ++i) same = same && ps[i]->kind == ps[0]->kind;
      if (same) {
        enqueue_gemv(ps, os, n, GemvMode::QkvRope, d_hidden_, D, L.gamma_in, st, &ra, roles);
        return;
      }
      for (int i = 0; i < n; ++i) enqueue_gemv(&ps[i], &os[i], 1, GemvMode::QkvRope, d_hidden_, D, L.gamma_in, st, &ra, roles + i);
    };
    if (H.full) {
      const ProjPlan* in[3] = {&H.in0, &H.in1, &H.in2};
      float* outs[3] = {d_hx0_, d_hx1_, d_hx2_};
      in_proj(in, outs, 3, store);
      const RopeArgs kv = rope_args(l);
      HybQkArgs q{};
      q.state = d_state_;
      q.qg = d_hx0_;
      q.k = d_hx1_;
      q.v = d_hx2_;
      q.q_norm = H.q_norm;
      q.k_norm = H.k_norm;
      q.rope_cos = d_rope_cos_;
      q.rope_sin = d_rope_sin_;
      q.q_out = d_q_;
      q.k_cache = kv.k_cache;
      q.v_cache = kv.v_cache;
      q.H = uint32_t(arch_.num_attn_heads);
      q.KV = uint32_t(arch_.num_kv_heads);
      q.hd = uint32_t(arch_.head_dim);
      q.rot = rope_dim_;
      q.max_seq = kv.max_seq;
      q.kv_f16 = kv.kv_f16;
      q.rope_rows = uint32_t(cfg_.max_seq_len);
      q.eps = arch_.rms_eps;
      launch_hyb_qk(q, st);
      AttnArgs aa = attn_args(l);
      aa.gate = d_hx0_;  // (the output gate applied by the merge)
      launch_attention_partial(aa, st);
      launch_attention_combine(aa, st);
      const ProjPlan* o[1] = {&H.out};
      enqueue_gemv(o, hid, 1, GemvMode::Accum, d_attn_, uint32_t(q.H * q.hd), nullptr, st);
    } else {
      // in_proj_qkv's rows go through the causal conv in the launch's epilogue (kRoleConv):
      // d_hconv_ receives silu(conv), the conv state is shifted there
      const ProjPlan* in[3] = {&H.in0, &H.in1, H.has_ab ? &H.ab : &H.in2};
      float* outs[3] = {d_hconv_, d_hx1_, d_hx2_};
      const uint32_t conv_roles[3] = {kRoleConv, kRoleStore, kRoleStore};
      ra.conv_w = H.conv_w;  // (in place of the KV cache pointers: no part appends a KV row)
      ra.conv_state = d_conv_state_ + size_t(H.lin) * 8192 * (kDnConvTaps - 1);
      in_proj(in, outs, 3, conv_roles);
      if (!H.has_ab) {
        const ProjPlan* inb[1] = {&H.in3};
        float* outb[1] = {d_hx3_};
        in_proj(inb, outb, 1, store);
      }
      DnStepArgs dn{};
      dn.q = d_hconv_;
      dn.k = d_hconv_ + 2048;
      dn.v = d_hconv_ + 4096;
      dn.a = d_hx2_;
      dn.b = H.has_ab ? d_hx2_ + 32 : d_hx3_;
      dn.A_log = H.A_log;
      dn.dt_bias = H.dt_bias;
      dn.z = d_hx1_;
      dn.norm_w = H.lin_norm;
      dn.state = d_rec_state_ + size_t(H.lin) * 32 * 128 * 128;
      dn.out = d_attn_;
      dn.n_v_heads = 32;
      dn.n_k_heads = 16;
      dn.eps = arch_.rms_eps;
      dn.step = d_state_;
      launch_dn_step(dn, 128, st);
      const ProjPlan* o[1] = {&H.out};
      enqueue_gemv(o, hid, 1, GemvMode::Accum, d_attn_, 4096, nullptr, st);
    }
    const ProjPlan* gu[2] = {&L.gate, &L.up};
    float* mlp[2] = {d_mlp_, d_mlp_};
    mark(2);
    enqueue_gemv(gu, mlp, 2, GemvMode::SwiGlu, d_hidden_, D, L.gamma_post, st);
    const ProjPlan* dn[1] = {&L.down};
    mark(3);
    enqueue_gemv(dn, hid, 1, GemvMode::Accum, d_mlp_, I, nullptr, st);
  }
  const ProjPlan* lm[1] = {&lm_head_};
  float* lg[1] = {d_logits_};
  mark(4);
  const uint32_t n_partials = enqueue_gemv(lm, lg, 1, GemvMode::Logits, d_hidden_, D, d_gamma_final_, st);
  FinishArgs f{d_state_, d_prompt_, d_partials_, n_partials, d_logits_, d_result_, d_out_tokens_, embed_args(),
               embed_fused_ ? 1u : 0u};
  launch_finish(f, st);
}

int Engine::launch_stage(int stage, size_t l) {
  if (l >= layers_.size()) return -1;
  if (cfg_.hybrid && stage != 2 && stage != 3 && stage != 4) return -1;  // (the MLP and LM head only)
  // q/k/v appends a KV row and attention reads rows up to the device position
  if ((stage == 0 || stage == 5 || stage == 6) && h_pos_ >= cfg_.max_seq_len) return -2;
  const LayerPlan& L = layers_[l];
  const uint32_t D = uint32_t(arch_.hidden_dim), I = uint32_t(arch_.intermediate_dim);
  switch (stage) {
    case 0:
      enqueue_qkv(l, stream_);
      return 0;
    case 1: {  // the step's Accum launch into a scratch vector, not the residual stream
      const ProjPlan* o[1] = {&L.o};
      float* y[1] = {d_q_};
      enqueue_gemv(o, y, 1, GemvMode::Accum, d_attn_, D, nullptr, stream_);
      return 0;
    }
    case 2: {
      const ProjPlan* gu[2] = {&L.gate, &L.up};
      float* y[2] = {d_mlp_, d_mlp_};
      enqueue_gemv(gu, y, 2, GemvMode::SwiGlu, d_hidden_, D, L.gamma_post, stream_);
      return 0;
    }
    case 3: {  // (as stage 1)
      const ProjPlan* dn[1] = {&L.down};
      float* y[1] = {d_attn_};
      enqueue_gemv(dn, y, 1, GemvMode::Accum, d_mlp_, I, nullptr, stream_);
      return 0;
    }
    case 4: {
      const ProjPlan* lm[1] = {&lm_head_};
      float* y[1] = {d_logits_};
      enqueue_gemv(lm, y, 1, GemvMode::Logits, d_hidden_, D, d_gamma_final_, stream_);
      return 0;
    }
    case 5:
      launch_attention_partial(attn_args(l), stream_);
      return 0;
    case 6:
      launch_attention_combine(attn_args(l), stream_);
      return 0;
  }
  return -1;
}

}  // namespace chpe

namespace chpe {

int Engine::debug_gemv(size_t layer, int which, const float* x, float* y) {
  // which: 0 q, 1 k, 2 v, 3 o, 4 gate, 5 up, 6 down, 7 LM head (logits only); the hybrid model
  // has no q/k/v/o plans of the reference's map
  if (which < 7 && layer >= layers_.size()) return -1;
  if (cfg_.hybrid && which >= 0 && which < 4) return -1;
  const ProjPlan* p = nullptr;
  if (which == 7) {
    p = &lm_head_;
  } else {
    const LayerPlan& L = layers_[layer];
    const ProjPlan* all[7] = {&L.q, &L.k, &L.v, &L.o, &L.gate, &L.up, &L.down};
    if (which < 0 || which > 6) return -1;
    p = all[which];
  }
  const size_t C = p->cols, R = p->rows;
  float *dx = nullptr, *dy = nullptr;
  int rc = -3;
  if (hipMalloc(&dx, C * 4) == hipSuccess && hipMalloc(&dy, R * 4) == hipSuccess &&
      hipMemcpy(dx, x, C * 4, hipMemcpyHostToDevice) == hipSuccess) {
    const ProjPlan* one[1] = {p};
    float* ys[1] = {dy};
    enqueue_gemv(one, ys, 1, GemvMode::Store, dx, uint32_t(C), nullptr, stream_);
    if (sync() == 0 && hipMemcpy(y, dy, R * 4, hipMemcpyDeviceToHost) == hipSuccess) rc = 0;
  }
  if (dx) (void)hipFree(dx);
  if (dy) (void)hipFree(dy);
  return rc;
}

}  // namespace chpe
