// c_api.cpp -- the chpe_* C ABI (libchpe.so).
//
// The reference's twelve symbols (src/chpe_c_api.zig:25-143) keep their signatures and
// sentinel semantics; the context owns the engine (device memory) and nothing else: the
// archive is mapped and validated (WeightArchive.openPosix + validate,
// src/weight_archive.zig:152-222), copied to HBM, and unmapped again.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstring>
#include <memory>
#include <string>
#include <vector>

#include "../../include/chpe.h"
#include "engine.hpp"
#include "format.hpp"
#include "src_hash.h"  // CHPE_SRC_HASH: the Makefile's hash of the library's sources

using namespace chpe;

namespace {

thread_local std::string g_last_error;

struct Context {
  std::unique_ptr<Engine> engine;
  ModelArch arch{};
  uint32_t last_argmax = 0;
  float last_max_logit = 0.0f, last_token0_logit = 0.0f, last_hidden_norm = 0.0f;
  uint64_t last_elapsed_ns = 0;
  hipEvent_t ev0 = nullptr, ev1 = nullptr;
};

// WeightArchive.validate: src/weight_archive.zig:152-172
const char* validate(const uint8_t* b, size_t len) {
  if (len < kHeaderBytes) return "FileTooSmall";
  ArchiveHeader h;
  std::memcpy(&h, b, sizeof h);
  if (h.magic != kArchiveMagic && h.magic != kChpeMagic) return "InvalidMagic";
  if (h.version != kArchiveVersion) return "UnsupportedVersion";
  if (h.header_bytes != kHeaderBytes) return "MisalignedHeader";
  const bool standard = h.record_bytes == kRecordBytes && h.prefetch_bytes == kPrefetchBytes;
  const bool dense = h.record_bytes == kCellBytes && h.prefetch_bytes == 0;
  const bool raw = h.record_bytes == kTileCodeBytes && h.prefetch_bytes == 0;
  if (!standard && !dense && !raw) return "BadGeometry";
  if (!raw && h.cell_bytes != kCellBytes) return "BadGeometry";
  if (raw && h.cell_bytes != kTileCodeBytes) return "BadGeometry";
  // header_bytes + record_count * record_bytes > len, without wrapping in 64 bits
  if (h.record_count > (len - h.header_bytes) / h.record_bytes) return "Truncated";
  return nullptr;
}

Context* open_ctx(const char* path, int arch, size_t max_seq_len, bool kv_f16) {
  g_last_error.clear();
  if (!path) { g_last_error = "null path"; return nullptr; }
  const int fd = ::open(path, O_RDONLY);
  if (fd < 0) { g_last_error = std::string("cannot open ") + path; return nullptr; }
  struct stat st;
  if (::fstat(fd, &st) != 0 || size_t(st.st_size) < kHeaderBytes) {
    ::close(fd);
    g_last_error = "FileTooSmall";
    return nullptr;
  }
  const size_t len = size_t(st.st_size);
  void* m = ::mmap(nullptr, len, PROT_READ, MAP_PRIVATE, fd, 0);
  ::close(fd);
  if (m == MAP_FAILED) { g_last_error = "mmap failed"; return nullptr; }
  ::madvise(m, len, MADV_SEQUENTIAL);
  ::madvise(m, len, MADV_WILLNEED);
  const uint8_t* bytes = static_cast<const uint8_t*>(m);
  if (const char* v = validate(bytes, len)) {
    ::munmap(m, len);
    g_last_error = v;
    return nullptr;
  }
  EngineConfig cfg;
  cfg.arch_id = arch < 0 ? arch_from_path(path) : arch == 3 ? 1 : arch;
  cfg.hybrid = arch == 3;
  cfg.max_seq_len = max_seq_len;
  cfg.kv_f16 = kv_f16;
  std::string err;
  auto engine = Engine::create(bytes, len, cfg, &err);
  ::munmap(m, len);
  if (!engine) { g_last_error = err; return nullptr; }
  auto* ctx = new Context();
  ctx->arch = engine->arch();
  ctx->engine = std::move(engine);
  (void)hipEventCreate(&ctx->ev0);
  (void)hipEventCreate(&ctx->ev1);
  return ctx;
}

void remember(Context* c, const ForwardResult& r) {
  c->last_argmax = r.argmax_token;
  c->last_max_logit = r.max_logit;
  c->last_token0_logit = r.token0_logit;
  c->last_hidden_norm = r.hidden_norm;
  c->last_elapsed_ns = r.elapsed_ns;
}

Context* C(void* p) { return static_cast<Context*>(p); }

}  // namespace

extern "C" {

void* chpe_init(const char* archive_path) { return open_ctx(archive_path, -1, 2048, false); }

void* chpe_init_ex(const char* archive_path, int arch, size_t max_seq_len, int kv_f16) {
  if (arch > 3) { g_last_error = "unknown architecture"; return nullptr; }
  return open_ctx(archive_path, arch, max_seq_len, kv_f16 != 0);
}

const char* chpe_last_error(void) { return g_last_error.c_str(); }

const char* chpe_build_id(void) { return CHPE_SRC_HASH; }

int chpe_forward_tokens(void* ctx, const uint32_t* tokens, size_t n, float* out_logits) {
  if (!ctx || !tokens || n == 0) return -1;
  Context* c = C(ctx);
  ForwardResult r{};
  const int rc = c->engine->forward_tokens(tokens, n, &r);
  if (rc) return rc;
  remember(c, r);
  if (out_logits && c->engine->copy_logits(out_logits)) return -3;
  return int(r.argmax_token);
}

int chpe_decode_step(void* ctx, uint32_t token, size_t pos, float* out_logits) {
  if (!ctx) return -1;
  Context* c = C(ctx);
  ForwardResult r{};
  const int rc = c->engine->forward(token, pos, &r);
  if (rc) return rc;
  remember(c, r);
  if (out_logits && c->engine->copy_logits(out_logits)) return -3;
  return int(r.argmax_token);
}

int chpe_generate(void* ctx, const uint32_t* prompt, size_t n_prompt, size_t n_gen, uint32_t* out_tokens) {
  if (!ctx || !prompt || n_prompt == 0 || n_gen == 0 || !out_tokens) return -1;
  Context* c = C(ctx);
  ForwardResult r{};
  const int rc = c->engine->generate(prompt, n_prompt, n_gen, out_tokens, &r);
  if (rc) return rc;
  remember(c, r);
  return 0;
}

int chpe_verify(void* ctx, const uint32_t* drafts, size_t m, size_t pos, uint32_t* out_argmax) {
  if (!ctx || !drafts || m == 0 || !out_argmax) return -1;
  Context* c = C(ctx);
  ForwardResult r{};
  const int rc = c->engine->verify(drafts, m, pos, out_argmax, &r);
  if (rc) return rc;
  remember(c, r);
  return 0;
}

int chpe_prefill(void* ctx, const uint32_t* tokens, size_t num_tokens, float* out_logits) {
  if (!ctx || !tokens || num_tokens == 0) return -1;
  Context* c = C(ctx);
  ForwardResult r{};
  const int rc = c->engine->prefill(tokens, num_tokens, &r);
  if (rc) return rc;
  remember(c, r);
  if (out_logits && c->engine->copy_logits(out_logits)) return -3;
  return int(r.argmax_token);
}

int chpe_block_ready(void* ctx) { return ctx && C(ctx)->engine->block_ready() ? 1 : 0; }

size_t chpe_get_last_logits(void* ctx, float* out, size_t max_len) {
  if (!ctx || !out) return 0;
  Context* c = C(ctx);
  const size_t V = c->arch.vocab_size;
  if (max_len < V) return 0;
  return c->engine->copy_logits(out) == 0 ? V : 0;
}

size_t chpe_get_vocab_size(void* ctx) { return ctx ? C(ctx)->arch.vocab_size : 151936; }
size_t chpe_get_hidden_dim(void* ctx) { return ctx ? C(ctx)->arch.hidden_dim : 2048; }
size_t chpe_get_num_layers(void* ctx) { return ctx ? C(ctx)->arch.num_layers : 36; }
uint64_t chpe_get_last_elapsed_ns(void* ctx) { return ctx ? C(ctx)->last_elapsed_ns : 0; }
uint32_t chpe_get_last_argmax(void* ctx) { return ctx ? C(ctx)->last_argmax : 0; }
float chpe_get_last_max_logit(void* ctx) { return ctx ? C(ctx)->last_max_logit : 0.0f; }
float chpe_get_last_token0_logit(void* ctx) { return ctx ? C(ctx)->last_token0_logit : 0.0f; }
float chpe_get_last_hidden_norm(void* ctx) { return ctx ? C(ctx)->last_hidden_norm : 0.0f; }
size_t chpe_get_max_seq_len(void* ctx) { return ctx ? C(ctx)->engine->max_seq_len() : 0; }

int chpe_get_hidden(void* ctx, float* out) {
  if (!ctx || !out) return -1;
  return C(ctx)->engine->copy_hidden(out);
}

void chpe_free(void* ctx) {
  if (!ctx) return;
  Context* c = C(ctx);
  c->engine.reset();
  if (c->ev0) (void)hipEventDestroy(c->ev0);
  if (c->ev1) (void)hipEventDestroy(c->ev1);
  delete c;
}

int chpe_time_steps(void* ctx, size_t n, float* ms) {
  if (!ctx || !ms) return -1;
  Context* c = C(ctx);
  Engine& e = *c->engine;
  if (hipEventRecord(c->ev0, e.stream()) != hipSuccess) return -3;
  if (const int rc = e.launch_steps(n)) return rc;
  if (hipEventRecord(c->ev1, e.stream()) != hipSuccess) return -3;
  if (hipEventSynchronize(c->ev1) != hipSuccess) return -3;
  if (hipEventElapsedTime(ms, c->ev0, c->ev1) != hipSuccess) return -3;
  ForwardResult r{};
  if (e.read_result(&r) == 0) remember(c, r);
  return 0;
}

int chpe_time_stage(void* ctx, int stage, size_t layer0, size_t layer1, size_t iters, float* ms) {
  if (!ctx || !ms || stage < 0 || stage > 6) return -1;
  Context* c = C(ctx);
  Engine& e = *c->engine;
  if (layer1 > e.arch().num_layers || layer0 >= layer1) return -1;
  if (hipEventRecord(c->ev0, e.stream()) != hipSuccess) return -3;
  for (size_t it = 0; it < iters; ++it)
    for (size_t l = layer0; l < layer1; ++l)
      if (const int rc = e.launch_stage(stage, l)) return rc;
  if (hipEventRecord(c->ev1, e.stream()) != hipSuccess) return -3;
  if (hipEventSynchronize(c->ev1) != hipSuccess) return -3;
  return hipEventElapsedTime(ms, c->ev0, c->ev1) == hipSuccess ? 0 : -3;
}

int chpe_time_stage_live(void* ctx, int stage, size_t n_steps, float* avg_ms) {
  if (!ctx || !avg_ms) return -1;
  Context* c = C(ctx);
  double avg = 0.0;
  size_t n = 0;
  const int rc = c->engine->time_stage_live(stage, n_steps, &avg, &n);
  if (rc) return rc;
  *avg_ms = float(avg);
  ForwardResult r{};
  if (c->engine->read_result(&r) == 0) remember(c, r);
  return 0;
}

const char* chpe_stage_kernel(void* ctx, int stage) {
  thread_local std::string name;
  name.clear();
  if (!ctx) return name.c_str();
  Engine& e = *C(ctx)->engine;
  record_kernel_names(true);  // (the launchers record the names and launch nothing)
  const int rc = e.launch_stage(stage, 0);
  record_kernel_names(false);
  if (rc == 0) name = last_kernel_name();
  return name.c_str();
}

double chpe_stage_bytes(void* ctx, int stage, size_t layer) {
  if (!ctx || layer >= C(ctx)->arch.num_layers) return 0.0;
  return C(ctx)->engine->stage_bytes(stage, layer);
}

double chpe_step_bytes(void* ctx, size_t pos) { return ctx ? C(ctx)->engine->step_bytes(pos) : 0.0; }

int chpe_debug_gemv(void* ctx, size_t layer, int which, const float* x, float* y) {
  if (!ctx || !x || !y) return -1;
  return C(ctx)->engine->debug_gemv(layer, which, x, y);
}

int chpe_debug_flat_tile_weights(const uint8_t* cell, float* out) {
  if (!cell || !out) return -1;
  uint8_t* dc = nullptr;
  float* dout = nullptr;
  int rc = -3;
  if (hipMalloc(&dc, kCellBytes) == hipSuccess && hipMalloc(&dout, kFlatWeights * 4) == hipSuccess &&
      hipMemcpy(dc, cell, kCellBytes, hipMemcpyHostToDevice) == hipSuccess) {
    launch_flat_tile_weights(dc, dout, nullptr);
    if (hipDeviceSynchronize() == hipSuccess &&
        hipMemcpy(out, dout, kFlatWeights * 4, hipMemcpyDeviceToHost) == hipSuccess)
      rc = 0;
  }
  if (dc) (void)hipFree(dc);
  if (dout) (void)hipFree(dout);
  return rc;
}

// One flat-tile GEMV launch (the decode step's kernels for gemvCellFlat tensors) on caller
// cells: the tensor's flat tiles as consecutive 17408-byte cells, copied to the device behind
// the same 64-byte shift and zero tail as the archive image.
int chpe_debug_gemv_raw(int mode, uint32_t rows, uint32_t cols, int kind, const uint8_t* tiles,
                        const uint8_t* tiles_up, size_t n_tiles, const float* x, const float* gamma, float eps, float* y,
                        uint32_t* out_argmax, float* out_hidden_norm) {
  g_last_error.clear();
  const bool norm = mode == int(GemvMode::SwiGlu) || mode == int(GemvMode::Logits);
  if (!tiles || !x || !y || rows == 0 || cols == 0 || kind < 0 || kind > 2 || mode < 0 ||
      mode > int(GemvMode::Logits) || norm != (gamma != nullptr) || (mode == int(GemvMode::SwiGlu)) != (tiles_up != nullptr))
    return -1;
  const size_t wpt = kind == 2 ? 16384 : 8192;
  if (cols % (kind == 2 ? 16u : 8u) || n_tiles * wpt < size_t(rows) * cols) {
    g_last_error = "raw tiles shorter than the matrix, or columns not a multiple of the load width";
    return -1;
  }
  const WeightKind wk = kind == 2 ? WeightKind::Raw8 : WeightKind::Raw16;
  const int n_parts = mode == int(GemvMode::SwiGlu) ? 2 : 1;
  const uint8_t* src[2] = {tiles, tiles_up};
  constexpr size_t kPad = size_t(1) << 20;
  const size_t bytes = n_tiles * kTileCodeBytes;
  std::vector<void*> mem;
  auto alloc = [&](size_t b) -> void* {
    void* d = nullptr;
    if (hipMalloc(&d, b) != hipSuccess) return nullptr;
    mem.push_back(d);
    return d;
  };
  int rc = -3;
  GemvArgs a{};
  a.n_parts = n_parts;
  a.mode = mode;
  a.C = cols;
  a.eps = eps;
  uint32_t prow[kMaxParts] = {rows, rows, 0}, begin[kMaxParts] = {0, 0, 0};
  const GemvLaunch g = gemv_geometry(wk, GemvMode(mode), cols, prow, n_parts, &a.n_units, &a.n_panels,
                                     &a.waves_per_unit, begin);
  float* dx = static_cast<float*>(alloc(size_t(cols) * 4));
  float* dy = static_cast<float*>(alloc(size_t(rows) * 4));
  float* dg = norm ? static_cast<float*>(alloc(size_t(cols) * 4)) : nullptr;
  bool ok = dx && dy && (!norm || dg) && hipMemcpy(dx, x, size_t(cols) * 4, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(dy, y, size_t(rows) * 4, hipMemcpyHostToDevice) == hipSuccess &&
            (!norm || hipMemcpy(dg, gamma, size_t(cols) * 4, hipMemcpyHostToDevice) == hipSuccess);
  for (int i = 0; ok && i < n_parts; ++i) {
    uint8_t* d = static_cast<uint8_t*>(alloc(bytes + kPad));
    ok = d && hipMemset(d, 0, bytes + kPad) == hipSuccess &&
         hipMemcpy(d, src[i], bytes, hipMemcpyHostToDevice) == hipSuccess;
    GemvPart& p = a.part[i];
    p.base = d;
    p.stride = uint32_t(kTileCodeBytes);
    p.rows = rows;
    p.wrows = rows;
    p.unit_begin = begin[i];
    p.y = dy;
    p.bf16 = kind == 1 ? 1 : 0;
  }
  a.x = dx;
  a.gamma = dg;
  StepResult* dres = nullptr;
  StepState* dst = nullptr;
  if (ok && mode == int(GemvMode::Logits)) {
    a.partials = static_cast<ArgmaxPartial*>(alloc(size_t(g.blocks) * sizeof(ArgmaxPartial)));
    dres = static_cast<StepResult*>(alloc(sizeof(StepResult)));
    dst = static_cast<StepState*>(alloc(sizeof(StepState)));
    a.result = dres;
    ok = a.partials && dres && dst && hipMemset(dst, 0, sizeof(StepState)) == hipSuccess;
  }
  if (ok) {
    launch_gemv(wk, a, g, nullptr);
    if (mode == int(GemvMode::Logits)) {
      FinishArgs f{};
      f.state = dst;
      f.partials = a.partials;
      f.n_partials = g.blocks;
      f.logits = dy;
      f.result = dres;
      launch_finish(f, nullptr);
    }
    StepResult r{};
    if (hipDeviceSynchronize() == hipSuccess &&
        hipMemcpy(y, dy, size_t(rows) * 4, hipMemcpyDeviceToHost) == hipSuccess &&
        (!dres || hipMemcpy(&r, dres, sizeof r, hipMemcpyDeviceToHost) == hipSuccess)) {
      if (dres && out_argmax) *out_argmax = r.argmax;
      if (dres && out_hidden_norm) *out_hidden_norm = r.hidden_norm;
      rc = 0;
    }
  }
  for (void* m : mem) (void)hipFree(m);
  return rc;
}

int chpe_debug_gemv_flat(int mode, uint32_t rows, uint32_t cols, const uint8_t* tiles, const uint8_t* tiles_up,
                         size_t n_tiles, const float* x, const float* gamma, float eps, float* y,
                         uint32_t* out_argmax, float* out_hidden_norm) {
  g_last_error.clear();
  const bool norm = mode == int(GemvMode::SwiGlu) || mode == int(GemvMode::Logits);
  if (!tiles || !x || !y || rows == 0 || cols <= 2048 || n_tiles == 0 || mode < 0 || mode > int(GemvMode::Logits) ||
      norm != (gamma != nullptr) || (mode == int(GemvMode::SwiGlu)) != (tiles_up != nullptr))
    return -1;
  const int n_parts = mode == int(GemvMode::SwiGlu) ? 2 : 1;
  const uint8_t* src[2] = {tiles, tiles_up};
  // the engine's plan: the uniform kernels, or tile by tile (FlatPoly) for any other tensor
  FlatPlan fp[2];
  for (int i = 0; i < n_parts; ++i) plan_flat(src[i], n_tiles * kCellBytes, kCellBytes, n_tiles, rows, cols, &fp[i]);
  if (n_parts == 2 && fp[1].kind != fp[0].kind)  // (gate and up share a launch)
    for (int i = 0; i < 2; ++i) {
      fp[i].kind = WeightKind::FlatPoly;
      fp[i].corr.clear();
      fp[i].corr_kmax = 0;
      fp[i].wrows = rows;
    }
  const WeightKind kind = fp[0].kind;
  const bool poly = kind == WeightKind::FlatPoly;
  const size_t used = std::max(fp[0].n_tiles, fp[n_parts - 1].n_tiles);

  constexpr size_t kShift = 64, kPad = size_t(1) << 20;  // as the engine's archive image
  const size_t img = kShift + used * kCellBytes + kPad;
  std::vector<void*> mem;
  auto alloc = [&](size_t bytes) -> void* {
    void* d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return nullptr;
    mem.push_back(d);
    return d;
  };
  int rc = -3;
  GemvArgs a{};
  a.n_parts = n_parts;
  a.mode = mode;
  a.C = cols;
  a.eps = eps;
  uint32_t prow[kMaxParts] = {rows, rows, 0}, begin[kMaxParts] = {0, 0, 0};
  const GemvLaunch g = gemv_geometry(kind, GemvMode(mode), cols, prow, n_parts, &a.n_units, &a.n_panels,
                                     &a.waves_per_unit, begin);
  float* dx = static_cast<float*>(alloc(size_t(cols) * 4));
  float* dy = static_cast<float*>(alloc(size_t(rows) * 4));
  float* dg = norm ? static_cast<float*>(alloc(size_t(cols) * 4)) : nullptr;
  bool ok = dx && dy && (!norm || dg) && hipMemcpy(dx, x, size_t(cols) * 4, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(dy, y, size_t(rows) * 4, hipMemcpyHostToDevice) == hipSuccess &&
            (!norm || hipMemcpy(dg, gamma, size_t(cols) * 4, hipMemcpyHostToDevice) == hipSuccess);
  for (int i = 0; ok && i < n_parts; ++i) {
    uint8_t* d = static_cast<uint8_t*>(alloc(img));
    ok = d && hipMemset(d, 0, img) == hipSuccess &&
         hipMemcpy(d + kShift, src[i], fp[i].n_tiles * kCellBytes, hipMemcpyHostToDevice) == hipSuccess;
    GemvPart& p = a.part[i];
    p.base = d + kShift;
    p.stride = uint32_t(kCellBytes);
    p.rows = rows;
    p.wrows = fp[i].wrows;
    p.unit_begin = begin[i];
    p.y = dy;
    p.corr_kmax = fp[i].corr_kmax;
    if (ok && !fp[i].corr.empty()) {
      float2* dc = static_cast<float2*>(alloc(fp[i].corr.size() * sizeof(float2)));
      ok = dc && hipMemcpy(dc, fp[i].corr.data(), fp[i].corr.size() * sizeof(float2), hipMemcpyHostToDevice) == hipSuccess;
      p.corr = dc;
    }
  }
  a.x = dx;
  a.gamma = dg;
  StepResult* dres = nullptr;
  StepState* dst = nullptr;
  const uint32_t n_partials = poly ? kPolyEpilogueBlocks : g.blocks;
  if (ok && mode == int(GemvMode::Logits)) {
    a.partials = static_cast<ArgmaxPartial*>(alloc(size_t(n_partials) * sizeof(ArgmaxPartial)));
    dres = static_cast<StepResult*>(alloc(sizeof(StepResult)));
    dst = static_cast<StepState*>(alloc(sizeof(StepState)));
    a.result = dres;
    ok = a.partials && dres && dst && hipMemset(dst, 0, sizeof(StepState)) == hipSuccess;
  }
  if (ok && !poly) {  // the permuted code copy where the engine builds one
    const size_t xb = xm_layout_bytes(kind, a, g);
    if (xb) {
      uint8_t* dxc = static_cast<uint8_t*>(alloc(xb));
      ok = dxc && build_xm_layout(kind, a, g, dxc, nullptr);
      a.part[0].xcodes = dxc;
    }
  }
  if (ok && poly) {
    float* xn = static_cast<float*>(alloc((size_t(cols) + 1) * 4));
    float* part = static_cast<float*>(alloc(flat_poly_part_floats(uint32_t(used), cols) * 4));
    PolyRaw raw{};
    for (int i = 0; i < kMaxParts; ++i) raw.y[i] = i < n_parts ? static_cast<float*>(alloc(size_t(rows) * 4)) : nullptr;
    ok = xn && part && raw.y[n_parts - 1];
    const uint32_t nt[kMaxParts] = {fp[0].n_tiles, fp[n_parts - 1].n_tiles, 0};
    if (ok) launch_gemv_flat_poly(a, nt, xn, raw, part, nullptr);
  } else if (ok) {
    launch_gemv(kind, a, g, nullptr);
  }
  if (ok) {
    if (mode == int(GemvMode::Logits)) {
      FinishArgs f{};
      f.state = dst;
      f.partials = a.partials;
      f.n_partials = n_partials;
      f.logits = dy;
      f.result = dres;
      launch_finish(f, nullptr);
    }
    StepResult r{};
    if (hipDeviceSynchronize() == hipSuccess &&
        hipMemcpy(y, dy, size_t(rows) * 4, hipMemcpyDeviceToHost) == hipSuccess &&
        (!dres || hipMemcpy(&r, dres, sizeof r, hipMemcpyDeviceToHost) == hipSuccess)) {
      if (dres && out_argmax) *out_argmax = r.argmax;
      if (dres && out_hidden_norm) *out_hidden_norm = r.hidden_norm;
      rc = 0;
    }
  }
  for (void* p : mem) (void)hipFree(p);
  return rc;
}

// One GEMV over polymorphic 16-row cells (any width, gemvTilePolymorphic) through the engine's
// polymorphic path (the raw row sums cell by cell, then the mode's epilogue).
int chpe_debug_gemv_poly(int mode, uint32_t rows, uint32_t cols, const uint8_t* cells, const uint8_t* cells_up,
                         size_t n_cells, const float* x, const float* gamma, float eps, float* y, uint32_t* out_argmax,
                         float* out_hidden_norm) {
  g_last_error.clear();
  const bool norm = mode == int(GemvMode::SwiGlu) || mode == int(GemvMode::Logits);
  if (!cells || !x || !y || rows == 0 || cols == 0 || n_cells == 0 || mode < 0 || mode > int(GemvMode::Logits) ||
      norm != (gamma != nullptr) || (mode == int(GemvMode::SwiGlu)) != (cells_up != nullptr))
    return -1;
  const int n_parts = mode == int(GemvMode::SwiGlu) ? 2 : 1;
  const uint8_t* src[2] = {cells, cells_up};
  constexpr size_t kShift = 64, kPad = size_t(1) << 20;  // as the engine's archive image
  const size_t img = kShift + n_cells * kCellBytes + kPad;
  std::vector<uint32_t> rb[2];
  for (int i = 0; i < n_parts; ++i) {
    bool uniform = false;
    uint64_t reach = 0;
    walk_cells(src[i], n_cells * kCellBytes, kCellBytes, n_cells, rows, cols, &rb[i], &uniform, &reach);
    if (reach > n_cells * kCellBytes + kPad) {
      g_last_error = "cells read past the end of the given cells";
      return -1;
    }
  }
  std::vector<void*> mem;
  auto alloc = [&](size_t bytes) -> void* {
    void* d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return nullptr;
    mem.push_back(d);
    return d;
  };
  int rc = -3;
  GemvArgs a{};
  a.n_parts = n_parts;
  a.mode = mode;
  a.C = cols;
  a.eps = eps;
  float* dx = static_cast<float*>(alloc(size_t(cols) * 4));
  float* dxn = static_cast<float*>(alloc((size_t(cols) + 1) * 4));
  float* dy = static_cast<float*>(alloc(size_t(rows) * 4));
  float* dg = norm ? static_cast<float*>(alloc(size_t(cols) * 4)) : nullptr;
  PolyRaw raw{};
  PolyPlan plan[2]{};
  const PolyPlan* pp[kMaxParts] = {};
  bool ok = dx && dxn && dy && (!norm || dg) && hipMemcpy(dx, x, size_t(cols) * 4, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(dy, y, size_t(rows) * 4, hipMemcpyHostToDevice) == hipSuccess &&
            (!norm || hipMemcpy(dg, gamma, size_t(cols) * 4, hipMemcpyHostToDevice) == hipSuccess);
  for (int i = 0; ok && i < n_parts; ++i) {
    uint8_t* d = static_cast<uint8_t*>(alloc(img));
    uint32_t* drb = static_cast<uint32_t*>(alloc(rb[i].size() * 4));
    raw.y[i] = static_cast<float*>(alloc(size_t(rows) * 4));
    ok = d && drb && raw.y[i] && hipMemset(d, 0, img) == hipSuccess &&
         hipMemcpy(d + kShift, src[i], n_cells * kCellBytes, hipMemcpyHostToDevice) == hipSuccess &&
         hipMemcpy(drb, rb[i].data(), rb[i].size() * 4, hipMemcpyHostToDevice) == hipSuccess;
    plan[i].row_base = drb;
    plan[i].n_cells = uint32_t(rb[i].size() - 1);
    pp[i] = &plan[i];
    GemvPart& p = a.part[i];
    p.base = d + kShift;
    p.stride = uint32_t(kCellBytes);
    p.rows = rows;
    p.wrows = rows;
    p.y = dy;
  }
  a.x = dx;
  a.gamma = dg;
  StepResult* dres = nullptr;
  StepState* dst = nullptr;
  if (ok && mode == int(GemvMode::Logits)) {
    a.partials = static_cast<ArgmaxPartial*>(alloc(size_t(kPolyEpilogueBlocks) * sizeof(ArgmaxPartial)));
    dres = static_cast<StepResult*>(alloc(sizeof(StepResult)));
    dst = static_cast<StepState*>(alloc(sizeof(StepState)));
    a.result = dres;
    ok = a.partials && dres && dst && hipMemset(dst, 0, sizeof(StepState)) == hipSuccess &&
         hipMemset(dres, 0, sizeof(StepResult)) == hipSuccess;
  }
  if (ok) {
    const uint32_t n_partials = launch_gemv_poly(a, pp, dxn, raw, nullptr);
    if (mode == int(GemvMode::Logits)) {
      FinishArgs f{};
      f.state = dst;
      f.partials = a.partials;
      f.n_partials = n_partials;
      f.logits = dy;
      f.result = dres;
      launch_finish(f, nullptr);
    }
    StepResult r{};
    if (hipDeviceSynchronize() == hipSuccess && hipMemcpy(y, dy, size_t(rows) * 4, hipMemcpyDeviceToHost) == hipSuccess &&
        (mode != int(GemvMode::Logits) || hipMemcpy(&r, dres, sizeof r, hipMemcpyDeviceToHost) == hipSuccess)) {
      if (out_argmax) *out_argmax = r.argmax;
      if (out_hidden_norm) *out_hidden_norm = r.hidden_norm;
      rc = 0;
    }
  }
  for (void* m : mem) (void)hipFree(m);
  return rc;
}

int chpe_debug_gemv_cells(int mode, uint32_t rows, const uint8_t* cells, const uint8_t* cells_up, size_t n_cells,
                          const float* x, const float* gamma, float eps, float* y, uint32_t* out_argmax,
                          float* out_hidden_norm) {
  g_last_error.clear();
  constexpr uint32_t cols = 2048;
  const bool norm = mode == int(GemvMode::SwiGlu) || mode == int(GemvMode::Logits);
  if (!cells || !x || !y || rows == 0 || mode < 0 || mode > int(GemvMode::Logits) || norm != (gamma != nullptr) ||
      (mode == int(GemvMode::SwiGlu)) != (cells_up != nullptr))
    return -1;
  const size_t need = (size_t(rows) + 15) / 16;
  if (n_cells < need) { g_last_error = "fewer cells than the rows need"; return -1; }
  const int n_parts = mode == int(GemvMode::SwiGlu) ? 2 : 1;
  const uint8_t* src[2] = {cells, cells_up};
  for (int i = 0; i < n_parts; ++i)
    for (size_t c = 0; c < need; ++c) {
      const uint8_t* pl = src[i] + c * kCellBytes + kPayloadOff;
      uint64_t flags = 0;
      std::memcpy(&flags, pl + kMetaCustomFlags, 8);
      if (pl[kMetaQuantBits] != 4 || !(flags & kFlagGroup128)) { g_last_error = "cells are not 4-bit group-128"; return -1; }
    }
  constexpr size_t kShift = 64, kPad = size_t(1) << 20;  // as the engine's archive image
  const size_t img = kShift + need * kCellBytes + kPad;
  std::vector<void*> mem;
  auto alloc = [&](size_t bytes) -> void* {
    void* d = nullptr;
    if (hipMalloc(&d, bytes) != hipSuccess) return nullptr;
    mem.push_back(d);
    return d;
  };
  int rc = -3;
  GemvArgs a{};
  a.n_parts = n_parts;
  a.mode = mode;
  a.C = cols;
  a.eps = eps;
  uint32_t prow[kMaxParts] = {rows, rows, 0}, begin[kMaxParts] = {0, 0, 0};
  const GemvLaunch g = gemv_geometry(WeightKind::Cell16W4, GemvMode(mode), cols, prow, n_parts, &a.n_units,
                                     &a.n_panels, &a.waves_per_unit, begin);
  float* dx = static_cast<float*>(alloc(size_t(cols) * 4));
  float* dy = static_cast<float*>(alloc(size_t(rows) * 4));
  float* dg = norm ? static_cast<float*>(alloc(size_t(cols) * 4)) : nullptr;
  bool ok = dx && dy && (!norm || dg) && hipMemcpy(dx, x, size_t(cols) * 4, hipMemcpyHostToDevice) == hipSuccess &&
            hipMemcpy(dy, y, size_t(rows) * 4, hipMemcpyHostToDevice) == hipSuccess &&
            (!norm || hipMemcpy(dg, gamma, size_t(cols) * 4, hipMemcpyHostToDevice) == hipSuccess);
  for (int i = 0; ok && i < n_parts; ++i) {
    uint8_t* d = static_cast<uint8_t*>(alloc(img));
    ok = d && hipMemset(d, 0, img) == hipSuccess &&
         hipMemcpy(d + kShift, src[i], need * kCellBytes, hipMemcpyHostToDevice) == hipSuccess;
    GemvPart& p = a.part[i];
    p.base = d + kShift;
    p.stride = uint32_t(kCellBytes);
    p.rows = rows;
    p.wrows = rows;
    p.unit_begin = begin[i];
    p.y = dy;
  }
  a.x = dx;
  a.gamma = dg;
  StepResult* dres = nullptr;
  StepState* dst = nullptr;
  if (ok && mode == int(GemvMode::Logits)) {
    a.partials = static_cast<ArgmaxPartial*>(alloc(size_t(g.blocks) * sizeof(ArgmaxPartial)));
    dres = static_cast<StepResult*>(alloc(sizeof(StepResult)));
    dst = static_cast<StepState*>(alloc(sizeof(StepState)));
    a.result = dres;
    ok = a.partials && dres && dst && hipMemset(dst, 0, sizeof(StepState)) == hipSuccess;
  }
  if (ok) {
    launch_gemv(WeightKind::Cell16W4, a, g, nullptr);
    if (mode == int(GemvMode::Logits)) {
      FinishArgs f{};
      f.state = dst;
      f.partials = a.partials;
      f.n_partials = g.blocks;
      f.logits = dy;
      f.result = dres;
      launch_finish(f, nullptr);
    }
    StepResult r{};
    if (hipDeviceSynchronize() == hipSuccess &&
        hipMemcpy(y, dy, size_t(rows) * 4, hipMemcpyDeviceToHost) == hipSuccess &&
        (!dres || hipMemcpy(&r, dres, sizeof r, hipMemcpyDeviceToHost) == hipSuccess)) {
      if (dres && out_argmax) *out_argmax = r.argmax;
      if (dres && out_hidden_norm) *out_hidden_norm = r.hidden_norm;
      rc = 0;
    }
  }
  for (void* p : mem) (void)hipFree(p);
  return rc;
}

int chpe_debug_embed_row_cell(const uint8_t* bytes, size_t len, uint32_t row, uint32_t D, float* out) {
  if (!bytes || !out || len < kCellBytes || D == 0 || D % 128) return -1;
  uint8_t* db = nullptr;
  float* dout = nullptr;
  int* dw = nullptr;
  int written = -3;
  if (hipMalloc(&db, len) == hipSuccess && hipMalloc(&dout, D * 4) == hipSuccess &&
      hipMalloc(&dw, sizeof(int)) == hipSuccess &&
      hipMemcpy(db, bytes, len, hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(dout, out, D * 4, hipMemcpyHostToDevice) == hipSuccess) {
    launch_embed_row_cell(db, len, row, D, dout, dw, nullptr);
    int w = 0;
    if (hipDeviceSynchronize() == hipSuccess &&
        hipMemcpy(out, dout, D * 4, hipMemcpyDeviceToHost) == hipSuccess &&
        hipMemcpy(&w, dw, sizeof(int), hipMemcpyDeviceToHost) == hipSuccess)
      written = w;
  }
  if (db) (void)hipFree(db);
  if (dout) (void)hipFree(dout);
  if (dw) (void)hipFree(dw);
  return written;
}

// The decode step's attention kernels on caller data: the caller's f32 rows are laid out as
// the engine's cache holds them (fp16 rounded to nearest even when kv_f16; V in 4-position
// blocks for fp16), and the chunk + merge kernels run once.
// nq queries at positions pos .. pos + nq - 1 (nq 1: the decode step's launch; more: the block
// step's), each over the rows up to its own position
static int debug_attention(uint32_t head_dim, uint32_t heads, uint32_t kv_heads, int kv_f16, uint32_t pos,
                           uint32_t nq, const float* q, const float* k_rows, const float* v_rows, float* out) {
  if (!q || !k_rows || !v_rows || !out || nq == 0 || nq > kMaxBlock || !attention_supported(heads, kv_heads, head_dim))
    return -1;
  const uint32_t chunk = attn_chunk(head_dim, kv_heads), ctx = pos + nq;
  const uint32_t n_chunks = (ctx + chunk - 1) / chunk, rows = n_chunks * chunk;  // a multiple of 16
  if (n_chunks > kAttnMaxChunks) return -1;
  const size_t hd = head_dim, kvd = size_t(kv_heads) * hd, el = kv_f16 ? 2 : 4;
  std::vector<uint8_t> kc(size_t(kv_heads) * rows * hd * el, 0), vc(kc.size(), 0);
  for (size_t t = 0; t < ctx; ++t)
    for (size_t h = 0; h < kv_heads; ++h)
      for (size_t d = 0; d < hd; ++d) {
        const float kv = k_rows[t * kvd + h * hd + d], vv = v_rows[t * kvd + h * hd + d];
        const size_t ka = (h * rows + t) * hd + d;
        if (kv_f16) {
          const size_t va = (h * rows + (t & ~size_t(3))) * hd + d * 4 + (t & 3);
          reinterpret_cast<uint16_t*>(kc.data())[ka] = f32_to_f16(kv);
          reinterpret_cast<uint16_t*>(vc.data())[va] = f32_to_f16(vv);
        } else {
          reinterpret_cast<float*>(kc.data())[ka] = kv;
          reinterpret_cast<float*>(vc.data())[ka] = vv;
        }
      }
  const size_t qn = size_t(nq) * heads * hd;
  void *dk = nullptr, *dv = nullptr;
  float *dq = nullptr, *dout = nullptr, *dml = nullptr, *dacc = nullptr;
  StepState* dst = nullptr;
  StepState st{};
  st.pos = pos;
  int rc = -3;
  if (hipMalloc(&dk, kc.size()) == hipSuccess && hipMalloc(&dv, vc.size()) == hipSuccess &&
      hipMalloc(&dq, qn * 4) == hipSuccess && hipMalloc(&dout, qn * 4) == hipSuccess &&
      hipMalloc(&dml, size_t(nq) * heads * n_chunks * 2 * 4) == hipSuccess &&
      hipMalloc(&dacc, size_t(nq) * heads * n_chunks * hd * 4) == hipSuccess &&
      hipMalloc(&dst, sizeof(StepState)) == hipSuccess &&
      hipMemcpy(dk, kc.data(), kc.size(), hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(dv, vc.data(), vc.size(), hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(dq, q, qn * 4, hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(dst, &st, sizeof st, hipMemcpyHostToDevice) == hipSuccess) {
    AttnArgs a{};
    a.state = dst;
    a.q = dq;
    a.k_cache = dk;
    a.v_cache = dv;
    a.out = dout;
    a.part_ml = dml;
    a.part_acc = dacc;
    a.H = heads;
    a.KV = kv_heads;
    a.hd = head_dim;
    a.max_seq = rows;
    a.n_chunks = n_chunks;
    a.chunk = chunk;
    a.kv_f16 = kv_f16 ? 1 : 0;
    a.scale = 1.0f / std::sqrt(float(head_dim));
    a.nq = nq;
    launch_attention(a, nullptr);
    if (hipDeviceSynchronize() == hipSuccess && hipMemcpy(out, dout, qn * 4, hipMemcpyDeviceToHost) == hipSuccess)
      rc = 0;
  }
  for (void* p : {dk, dv, static_cast<void*>(dq), static_cast<void*>(dout), static_cast<void*>(dml),
                  static_cast<void*>(dacc), static_cast<void*>(dst)})
    if (p) (void)hipFree(p);
  return rc;
}

int chpe_debug_attention(uint32_t head_dim, uint32_t heads, uint32_t kv_heads, int kv_f16, uint32_t pos,
                         const float* q, const float* k_rows, const float* v_rows, float* out) {
  return debug_attention(head_dim, heads, kv_heads, kv_f16, pos, 1, q, k_rows, v_rows, out);
}

int chpe_debug_attention_block(uint32_t head_dim, uint32_t heads, uint32_t kv_heads, int kv_f16, uint32_t pos,
                               uint32_t nq, const float* q, const float* k_rows, const float* v_rows, float* out) {
  return debug_attention(head_dim, heads, kv_heads, kv_f16, pos, nq, q, k_rows, v_rows, out);
}

// One decode step of a gated-DeltaNet layer's recurrent core on caller data (the layers have no
// reference code; see deltanet.hip for the arithmetic's source).
int chpe_debug_deltanet_conv(uint32_t channels, uint32_t taps, const float* x, const float* w, float* state,
                             float* out) {
  if (!x || !w || !state || !out || channels == 0 || taps < 2 || taps > kDnMaxTaps) return -1;
  const size_t nx = channels, nw = size_t(channels) * taps, ns = size_t(channels) * (taps - 1);
  float *dx = nullptr, *dw = nullptr, *ds = nullptr, *dout = nullptr;
  int rc = -3;
  if (hipMalloc(&dx, nx * 4) == hipSuccess && hipMalloc(&dw, nw * 4) == hipSuccess &&
      hipMalloc(&ds, ns * 4) == hipSuccess && hipMalloc(&dout, nx * 4) == hipSuccess &&
      hipMemcpy(dx, x, nx * 4, hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(dw, w, nw * 4, hipMemcpyHostToDevice) == hipSuccess &&
      hipMemcpy(ds, state, ns * 4, hipMemcpyHostToDevice) == hipSuccess) {
    DnConvArgs a{dx, dw, ds, dout, channels, taps, nullptr};
    launch_dn_conv(a, nullptr);
    if (hipDeviceSynchronize() == hipSuccess && hipMemcpy(out, dout, nx * 4, hipMemcpyDeviceToHost) == hipSuccess &&
        hipMemcpy(state, ds, ns * 4, hipMemcpyDeviceToHost) == hipSuccess)
      rc = 0;
  }
  for (float* p : {dx, dw, ds, dout})
    if (p) (void)hipFree(p);
  return rc;
}

int chpe_debug_deltanet_step(uint32_t n_v_heads, uint32_t n_k_heads, uint32_t head_dim, const float* q, const float* k,
                             const float* v, const float* a_in, const float* b_in, const float* A_log,
                             const float* dt_bias, const float* z, const float* norm_w, float eps, float* state,
                             float* out) {
  if (!q || !k || !v || !a_in || !b_in || !A_log || !dt_bias || !state || !out || (norm_w && !z) ||
      !deltanet_supported(n_v_heads, n_k_heads, head_dim, 4))
    return -1;
  const size_t hd = head_dim, nq = n_k_heads * hd, nv = n_v_heads * hd, ns = n_v_heads * hd * hd;
  const float* src[9] = {q, k, v, a_in, b_in, A_log, dt_bias, z, norm_w};
  const size_t cnt[9] = {nq, nq, nv, n_v_heads, n_v_heads, n_v_heads, n_v_heads, nv, hd};
  float* dev[9] = {};
  float *ds = nullptr, *dout = nullptr;
  bool ok = hipMalloc(&ds, ns * 4) == hipSuccess && hipMalloc(&dout, nv * 4) == hipSuccess &&
            hipMemcpy(ds, state, ns * 4, hipMemcpyHostToDevice) == hipSuccess;
  for (int i = 0; ok && i < 9; ++i)
    if (src[i])
      ok = hipMalloc(&dev[i], cnt[i] * 4) == hipSuccess &&
           hipMemcpy(dev[i], src[i], cnt[i] * 4, hipMemcpyHostToDevice) == hipSuccess;
  int rc = -3;
  if (ok) {
    DnStepArgs a{};
    a.q = dev[0];
    a.k = dev[1];
    a.v = dev[2];
    a.a = dev[3];
    a.b = dev[4];
    a.A_log = dev[5];
    a.dt_bias = dev[6];
    a.z = dev[7];
    a.norm_w = dev[8];
    a.state = ds;
    a.out = dout;
    a.n_v_heads = n_v_heads;
    a.n_k_heads = n_k_heads;
    a.eps = eps;
    launch_dn_step(a, head_dim, nullptr);
    if (hipDeviceSynchronize() == hipSuccess && hipMemcpy(out, dout, nv * 4, hipMemcpyDeviceToHost) == hipSuccess &&
        hipMemcpy(state, ds, ns * 4, hipMemcpyDeviceToHost) == hipSuccess)
      rc = 0;
  }
  for (float* p : dev)
    if (p) (void)hipFree(p);
  if (ds) (void)hipFree(ds);
  if (dout) (void)hipFree(dout);
  return rc;
}

}  // extern "C"
