// chpe_fwd -- the reference's CLI (src/main.zig) on the MI355X engine, through libchpe.so's C ABI.
//
// Same flags (main.zig:21-84): a positional archive path or --archive, --tokens-file (raw
// little-endian u32), --out-logits (raw f32[vocab] of the last token), --arch (substring
// "9b"/"9B" or "72b"/"72B" selects the model, else 3B), --bench <iters>, --max-seq-len
// (default 2048), -h/--help; the architecture is otherwise guessed from the archive path as
// main.zig:86-104 does.  Each bench iteration runs the prompt from position 0
// (chpe_forward_tokens, main.zig:169-184).  The receipt goes to stderr in the reference's
// line format (main.zig:189-196), and the spoke JSON file is written when its directory
// exists (main.zig:211-246).  Two flags of its own: --kv-f16 keeps the KV cache in fp16;
// --hybrid runs a Qwen3.5-9B archive through its true hybrid layers (chpe_init_ex arch 3)
// instead of the reference's decode of the 9B map.
#include <fcntl.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/chpe.h"

namespace {

void usage() {
  std::fprintf(stderr,
               "Unified Polymorphic CHPE Forward Engine\n"
               "\n"
               "Usage: chpe_fwd [OPTIONS]\n"
               "\n"
               "Options:\n"
               "  --archive <path>       Path to .chpe weight archive\n"
               "  --tokens-file <path>   Binary little-endian u32 tokens file\n"
               "  --out-logits <path>    Destination binary file for output float logits\n"
               "  --arch <name>          Model architecture (qwen2_5_3b | qwen3_5_9b | qwen2_5_72b)\n"
               "  --bench <iters>        Benchmark iterations (default: 1)\n"
               "  --max-seq-len <len>    Maximum sequence length (default: 2048)\n"
               "  --kv-f16               Keep the KV cache in fp16 (default: f32, as the reference)\n"
               "  --hybrid               Qwen3.5-9B: gated DeltaNet + gated attention layers\n"
               "  -h, --help             Display this help message\n");
}

int arch_of(const std::string& s, bool is_path) {
  auto has = [&](const char* t) { return s.find(t) != std::string::npos; };
  if (has("9b") || has("9B") || (is_path && has("qwen35"))) return 1;
  if (has("72b") || has("72B")) return 2;
  return 0;
}

const char* arch_name(int a) {
  return a == 3 ? "Qwen3.5-9B (hybrid)" : a == 1 ? "Qwen3.5-9B" : (a == 2 ? "Qwen2.5-72B" : "Qwen2.5-3B");
}

uint64_t now_ns() {
  return uint64_t(std::chrono::duration_cast<std::chrono::nanoseconds>(
                      std::chrono::steady_clock::now().time_since_epoch())
                      .count());
}

}  // namespace

int main(int argc, char** argv) {
  std::string archive = "models/warc/Qwen2.5-3B-Instruct.bf16.raw.chpe", tokens_file, out_logits, arch_override;
  size_t bench_iters = 1, max_seq_len = 2048;
  bool kv_f16 = false, hybrid = false;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto next = [&](std::string* dst) {
      if (i + 1 < argc) *dst = argv[++i];
    };
    if (a == "--archive") next(&archive);
    else if (a == "--tokens-file") next(&tokens_file);
    else if (a == "--out-logits") next(&out_logits);
    else if (a == "--arch") next(&arch_override);
    else if (a == "--bench") {
      std::string v;
      next(&v);
      char* end = nullptr;
      const unsigned long long n = std::strtoull(v.c_str(), &end, 10);
      bench_iters = (!v.empty() && end && *end == 0) ? size_t(n) : 1;
    } else if (a == "--max-seq-len") {
      std::string v;
      next(&v);
      char* end = nullptr;
      const unsigned long long n = std::strtoull(v.c_str(), &end, 10);
      max_seq_len = (!v.empty() && end && *end == 0) ? size_t(n) : 2048;
    } else if (a == "--kv-f16") kv_f16 = true;
    else if (a == "--hybrid") hybrid = true;
    else if (a == "--help" || a == "-h") {
      usage();
      return 0;
    } else if (a.rfind("--", 0) != 0) archive = a;
  }
  int arch = arch_override.empty() ? arch_of(archive, true) : arch_of(arch_override, false);
  if (hybrid) {
    if (arch != 1) {
      std::fprintf(stderr, "ERROR: --hybrid needs a Qwen3.5-9B archive\n");
      return 1;
    }
    arch = 3;
  }

  std::fprintf(stderr, "=== [UNIFIED POLYMORPHIC CHPE FORWARD ENGINE] ===\n");
  std::fprintf(stderr, "Archive Path   : %s\n", archive.c_str());
  struct stat st;
  if (::stat(archive.c_str(), &st) != 0) {
    std::fprintf(stderr, "ERROR: Failed to open weight archive '%s': FileNotFound\n", archive.c_str());
    return 1;
  }

  std::vector<uint32_t> prompt;
  if (!tokens_file.empty()) {
    const int fd = ::open(tokens_file.c_str(), O_RDONLY);
    struct stat ts;
    if (fd < 0 || ::fstat(fd, &ts) != 0) {
      std::fprintf(stderr, "ERROR: Failed to open tokens file '%s'\n", tokens_file.c_str());
      if (fd >= 0) ::close(fd);
      return 1;
    }
    prompt.resize(size_t(ts.st_size) / 4);
    if (prompt.empty()) {
      ::close(fd);
      std::fprintf(stderr, "ERROR: EmptyTokensFile\n");
      return 1;
    }
    const ssize_t got = ::read(fd, prompt.data(), prompt.size() * 4);
    ::close(fd);
    if (got != ssize_t(prompt.size() * 4)) {
      std::fprintf(stderr, "ERROR: short read of tokens file '%s'\n", tokens_file.c_str());
      return 1;
    }
    std::fprintf(stderr, "Prompt Tokens  : Loaded %zu tokens from '%s'\n", prompt.size(), tokens_file.c_str());
  } else {
    prompt.push_back(151644);  // <|im_start|>
    std::fprintf(stderr, "Prompt Tokens  : Default single token [%u]\n", prompt[0]);
  }

  void* ctx = chpe_init_ex(archive.c_str(), arch, max_seq_len, kv_f16 ? 1 : 0);
  if (!ctx) {
    std::fprintf(stderr, "ERROR: Failed to open weight archive '%s': %s\n", archive.c_str(), chpe_last_error());
    return 1;
  }
  std::fprintf(stderr, "Model Arch     : %s (%zu layers, D=%zu, vocab=%zu)\n", arch_name(arch),
               chpe_get_num_layers(ctx), chpe_get_hidden_dim(ctx), chpe_get_vocab_size(ctx));
  std::fprintf(stderr, "Archive Size   : %lld bytes (%.2f GB)\n", (long long)st.st_size,
               double(st.st_size) / (1024.0 * 1024.0 * 1024.0));
  std::fprintf(stderr, "Hardware Core  : MI355X (gfx950)\n");
  std::fprintf(stderr, "Execution Loop : Running forward pass over %zu prompt tokens...\n", prompt.size());

  double sum_ms = 0.0;
  for (size_t iter = 0; iter < bench_iters; ++iter) {
    const uint64_t t0 = now_ns();
    const int rc = chpe_forward_tokens(ctx, prompt.data(), prompt.size(), nullptr);
    const double cur_ms = double(now_ns() - t0) / 1e6;
    if (rc < 0) {
      std::fprintf(stderr, "ERROR: forward pass failed (%d)%s\n", rc,
                   rc == -2 ? ": more tokens than --max-seq-len" : "");
      chpe_free(ctx);
      return 1;
    }
    sum_ms += cur_ms;
    if (bench_iters > 1) std::fprintf(stderr, "  [Iter %zu/%zu] Latency: %.2f ms\n", iter + 1, bench_iters, cur_ms);
  }
  if (bench_iters == 0) {
    chpe_free(ctx);
    return 0;
  }
  const double mean_ms = sum_ms / double(bench_iters), throughput = double(prompt.size()) / (mean_ms / 1000.0);
  const size_t V = chpe_get_vocab_size(ctx);
  std::vector<float> logits(V);
  const bool have_logits = chpe_get_last_logits(ctx, logits.data(), V) == V;
  bool finite = have_logits;
  for (float v : logits) finite = finite && std::isfinite(v);

  std::fprintf(stderr, "\n=== [PHYSICAL SILICON EXECUTION RECEIPT] ===\n");
  std::fprintf(stderr, "Argmax Decoded Token ID : %u\n", chpe_get_last_argmax(ctx));
  std::fprintf(stderr, "Maximum Vocab Logit     : %.6f\n", double(chpe_get_last_max_logit(ctx)));
  std::fprintf(stderr, "Token 0 Logit           : %.6f\n", double(chpe_get_last_token0_logit(ctx)));
  std::fprintf(stderr, "Final Hidden Vector Norm: %.6f\n", double(chpe_get_last_hidden_norm(ctx)));
  std::fprintf(stderr, "Mean Latency            : %.2f ms (%.3f s)\n", mean_ms, mean_ms / 1000.0);
  std::fprintf(stderr, "Throughput              : %.2f tokens/sec\n", throughput);
  std::fprintf(stderr, "Numerical Soundness     : %s\n",
               finite ? "100% FINITE (Zero NaN / Zero Inf)" : "FAILED (NaN or Inf present)");

  if (!out_logits.empty() && have_logits) {
    const int fd = ::open(out_logits.c_str(), O_WRONLY | O_CREAT | O_TRUNC, 0644);
    if (fd >= 0) {
      const ssize_t w = ::write(fd, logits.data(), V * 4);
      ::close(fd);
      if (w == ssize_t(V * 4))
        std::fprintf(stderr, "Exported Logits Binary  : %s (%zu floats, %zu bytes)\n", out_logits.c_str(), V, V * 4);
    }
  }

  const char* spoke = "run/spoke_outbox/metal.chpe_fwd.result.json";
  const int fd = ::open(spoke, O_WRONLY | O_CREAT | O_TRUNC, 0644);
  if (fd >= 0) {
    char buf[2048];
    const int n = std::snprintf(
        buf, sizeof buf,
        "{\n  \"benchmark\": \"CHPE Forward Engine\",\n  \"model\": \"%s\",\n  \"archive\": \"%s\",\n"
        "  \"tokens_evaluated\": %zu,\n  \"argmax_token\": %u,\n  \"max_logit\": %.6f,\n  \"token0_logit\": %.6f,\n"
        "  \"hidden_norm\": %.6f,\n  \"mean_latency_ms\": %.2f,\n  \"throughput_tok_s\": %.2f,\n  \"all_finite\": %s\n}\n",
        arch_name(arch), archive.c_str(), prompt.size(), chpe_get_last_argmax(ctx), double(chpe_get_last_max_logit(ctx)),
        double(chpe_get_last_token0_logit(ctx)), double(chpe_get_last_hidden_norm(ctx)), mean_ms, throughput,
        finite ? "true" : "false");
    if (n > 0) (void)!::write(fd, buf, size_t(n));
    ::close(fd);
    std::fprintf(stderr, "Recorded Spoke Telemetry: %s\n", spoke);
  }
  chpe_free(ctx);
  return 0;
}
