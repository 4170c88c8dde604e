// step.hip -- per-token kernels around the layer stack: embedding lookup, the final argmax
// reduction with the device-side advance to the next position, and the dequantisation hooks
// the parity tests use.
#include "device_common.hpp"
#include "kernels.hpp"

namespace chpe {
namespace {
using namespace dev;

// unpackEmbedRowCell (chpe_engine.zig:1288-1394) for one row of the cell at byte offset
// `cell` of the image, workgroup-parallel over columns.  Returns false when the row is out
// of the cell's range (then `out` is left untouched, as in the reference).  Wide rows
// (D >= 4096) read past the cell into the following records, by byte address as on the CPU.
//
// Fast path for the 4-bit group-128 cells when every byte it reads lies inside the image: the
// header, the codes (one 32-bit word per 8 columns), the group scales and the 8 outlier entries
// are all requested before any is used (the step's final kernel waits on this chain once).
constexpr int kEmbedWords = 4;  // 8-column words per thread (D <= 8 * 4 * blockDim.x)
__device__ bool unpack_embed_row_cell_fast(const Image& im, uint64_t cell, uint32_t row, uint32_t D,
                                           float* out, bool* handled) {
  const uint32_t tid = threadIdx.x, nt = blockDim.x, ng = D / 128;
  const uint64_t codes = cell + 64, pl = cell + 16448;
  *handled = false;
  if (row >= 16 || D % 128 != 0 || D > 8 * uint32_t(kEmbedWords) * nt) return false;
  if ((reinterpret_cast<uintptr_t>(im.p) & 3u) != 0 || (cell & 3u) != 0) return false;
  if (cell + 17408 > im.len || codes + uint64_t(row + 1) * (D / 2) > im.len ||
      pl + 48 + 2 * uint64_t(row + 1) * ng > im.len)
    return false;
  const uint8_t* P = im.p;
  const uint32_t qb = P[pl + 20];
  const uint32_t flags = *reinterpret_cast<const uint32_t*>(P + pl + 24);
  uint32_t w[kEmbedWords];
  uint16_t sv[kEmbedWords];
#pragma unroll
  for (int k = 0; k < kEmbedWords; ++k) {
    const uint32_t i0 = (tid + uint32_t(k) * nt) * 8, ic = i0 < D ? i0 : 0u;
    w[k] = *reinterpret_cast<const uint32_t*>(P + codes + uint64_t(row) * (D / 2) + ic / 2);
    sv[k] = *reinterpret_cast<const uint16_t*>(P + pl + 48 + 2 * (uint64_t(row) * ng + ic / 128));
  }
  const uint32_t e = tid < 8 ? tid : 0u;
  const uint32_t ocol = *reinterpret_cast<const uint16_t*>(P + pl + 816 + 2 * e);
  const uint16_t ow = *reinterpret_cast<const uint16_t*>(P + pl + 560 + 2 * (row * 8 + e));
  if (qb != 4 || (flags & 1u) == 0) return false;  // (uniform) the generic path decodes the cell
  *handled = true;
#pragma unroll
  for (int k = 0; k < kEmbedWords; ++k) {
    const uint32_t i0 = (tid + uint32_t(k) * nt) * 8;
    if (i0 < D) {
      const float sc = h2f(sv[k]);
      float v[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = (float((w[k] >> (4 * j)) & 15u) - 8.0f) * sc;
      *reinterpret_cast<float4*>(out + i0) = make_float4(v[0], v[1], v[2], v[3]);
      *reinterpret_cast<float4*>(out + i0 + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
  }
  // outliers replace, in entry order: an entry overridden by a later one for the same column
  // is skipped, so the 8 entries store in parallel (after the row's stores: the barrier)
  __shared__ uint32_t s_oc[8];
  if (tid < 8) s_oc[tid] = ocol;
  __syncthreads();
  if (tid < 8 && ocol < D) {
    bool later = false;
    for (uint32_t j = tid + 1; j < 8; ++j) later |= s_oc[j] == ocol;
    if (!later) out[ocol] = h2f(ow);
  }
  return true;
}

// gi, gn: this thread's index and the thread count of the launch.  The per-tile scale form (the
// 72B and 9B embeddings) is split over all of them; the other forms, whose outliers are stored
// after the row under a workgroup barrier, run in the lead workgroup alone.
__device__ bool unpack_embed_row_cell(const Image& im, uint64_t cell, uint32_t row, uint32_t D,
                                      float* out, uint32_t gi, uint32_t gn, bool lead) {
  const uint64_t codes = cell + 64, pl = cell + 16448;
  const uint8_t qb = im.u8(pl + 20);
  const bool g128 = (im.u64(pl + 24) & 1u) != 0;
  if (qb != 8 && qb != 2 && !g128 && qb != 4) {  // (nibble - 8) * scale + bias (:1384-1394)
    const float scale = im.f32(pl + 32), bias = im.f32(pl + 36);
    for (uint32_t i = gi; i < (D / 2) * 2; i += gn) {
      const uint32_t b = im.u8(codes + uint64_t(row) * (D / 2) + i / 2);
      const float q = float((b >> (4 * (i & 1))) & 15u);
      out[i] = __fadd_rn(__fmul_rn(q - 8.0f, scale), bias);
    }
    return true;
  }
  if (!lead) return true;
  bool handled = false;
  const bool ok = unpack_embed_row_cell_fast(im, cell, row, D, out, &handled);
  if (handled) return ok;
  const uint32_t ng = D / 128;
  const int tid = threadIdx.x, nt = blockDim.x;
  if (qb == 8) {
    if (row >= 8) return false;
    for (uint32_t i = tid; i < ng * 128; i += nt) {
      const float s = h2f(im.u16(pl + 48 + 2 * (row * ng + i / 128)));
      out[i] = float(int8_t(im.u8(codes + uint64_t(row) * D + i))) * s;
    }
    return true;
  }
  if (qb == 2) {
    if (row >= 16) return false;
    for (uint32_t i = tid; i < ng * 128; i += nt) {
      const float s = h2f(im.u16(pl + 48 + 2 * (row * ng + i / 128)));
      const uint32_t b = im.u8(codes + uint64_t(row) * (D / 4) + i / 4);
      out[i] = codebook_w2((b >> (2 * (i & 3))) & 3u) * s;
    }
  } else if (g128 || qb == 4) {
    if (row >= 16) return false;
    for (uint32_t i = tid; i < ng * 128; i += nt) {
      const float s = h2f(im.u16(pl + 48 + 2 * (row * ng + i / 128)));
      const uint32_t b = im.u8(codes + uint64_t(row) * (D / 2) + i / 2);
      out[i] = (float((b >> (4 * (i & 1))) & 15u) - 8.0f) * s;
    }
  }
  if (g128) {  // outliers replace, in entry order (the last entry for a column wins)
    __syncthreads();
    if (tid == 0)
      for (int k = 0; k < 8; ++k) {
        const uint32_t col = im.u16(pl + 816 + 2 * k);
        if (col < D) out[col] = h2f(im.u16(pl + 560 + 2 * (row * 8 + k)));
      }
  }
  return true;
}

// unpackEmbedRow: chpe_engine.zig:1491-1552
// The hidden state of token `tok` (unpackEmbedRow / unpackEmbedRowCell), workgroup-parallel.
// the step's RoPE row (cos then sin of position pos; a position past the tables: none)
__device__ void stage_rope_row(const EmbedArgs& a, uint32_t pos) {
  if (a.rope_cur && pos < a.rope_rows)
    for (uint32_t i = threadIdx.x; i < 2 * a.rope_half; i += blockDim.x)
      a.rope_cur[i] = i < a.rope_half ? a.rope_cos[size_t(pos) * a.rope_half + i]
                                      : a.rope_sin[size_t(pos) * a.rope_half + (i - a.rope_half)];
}

// gi, gn, lead: as unpack_embed_row_cell (one workgroup: threadIdx.x, blockDim.x, true)
__device__ void embed_token(const EmbedArgs& a, uint32_t tok, uint32_t gi, uint32_t gn, bool lead) {
  const uint32_t D = a.D;
  const Image im{a.image, a.image_len};
  const uint32_t tid = gi, nt = gn;
  bool done = false;
  if (a.kind == 1 || a.kind == 2 || a.kind == 3) {
    const uint32_t rpt = (a.kind == 3 ? 16384u : 8192u) / D;
    if (rpt > 0 && tok / rpt < a.record_count) {
      const uint64_t base = 4096 + uint64_t(tok / rpt) * 16384;
      const uint32_t row = tok % rpt;
      for (uint32_t i = tid; i < D; i += nt) {
        const uint64_t e = uint64_t(row) * D + i;
        float v;
        if (a.kind == 1) v = h2f(im.u16(base + 2 * e));
        else if (a.kind == 2) v = bf2f(im.u16(base + 2 * e));
        else v = float(int8_t(im.u8(base + e))) * 0.00373708f;
        a.hidden[i] = v;
      }
      done = true;
    }
  } else if (a.kind == 4) {
    const uint32_t tile = tok / 16, row = tok % 16;
    if (tile < a.record_count) {
      unpack_embed_row_cell(im, 4096 + uint64_t(tile) * a.stride + a.cell_off, row, D, a.hidden, gi, gn, lead);
      done = true;  // an out-of-range row keeps the previous hidden state, as on the CPU
    }
  }
  if (!done)
    for (uint32_t i = tid; i < D; i += nt) a.hidden[i] = 0.05f * float(int((i + tok) % 17u) - 8);
}

// the step's input row over D / 256 workgroups (the 72B and 9B rows are decoded
// byte by byte); workgroup 0 also stages the RoPE row
__global__ void __launch_bounds__(256) k_embed(EmbedArgs a) {
  if (blockIdx.x == 0) stage_rope_row(a, a.state->pos);
  embed_token(a, a.state->token, blockIdx.x * blockDim.x + threadIdx.x, gridDim.x * blockDim.x, blockIdx.x == 0);
}

// the block step's inputs: token blockIdx.x's embedding row into X[blockIdx.x]
// one workgroup per token; then the row's sum of squares (the first layer's RMS norm)
__global__ void __launch_bounds__(256) k_block_embed(EmbedArgs a, const uint32_t* tokens, float* X, float* ssp,
                                                     uint32_t* brk) {
  EmbedArgs e = a;
  if (threadIdx.x == 0) brk[blockIdx.x] = 0u;
  float* row = X + size_t(blockIdx.x) * a.D;
  e.hidden = row;
  embed_token(e, tokens[blockIdx.x], threadIdx.x, blockDim.x, true);
  __syncthreads();  // the workgroup's row writes are visible to it
  float ss = 0.0f;
  for (uint32_t c = threadIdx.x; c < a.D; c += blockDim.x) ss = fmaf(row[c], row[c], ss);
  ss = wave_sum(ss);
  __shared__ float s_ss[4];
  if ((threadIdx.x & 63) == 0) s_ss[threadIdx.x >> 6] = ss;
  __syncthreads();
  if (threadIdx.x == 0) ssp[blockIdx.x] = (s_ss[0] + s_ss[1]) + (s_ss[2] + s_ss[3]);
}

// argmax / all_finite / logits[0] over the LM head's workgroup partials (chpe_engine.zig:
// 1775-1787), then the next position's (token, pos): the prompt while it lasts, else the argmax.
__global__ void __launch_bounds__(256) k_finish(FinishArgs a) {
  // what does not wait for the argmax first: the state, the next position's RoPE row and its
  // prompt token (the step's q/k/v launch has read the current row already)
  const StepState s0 = *a.state;
  const uint32_t next = s0.pos + 1;
  const uint32_t ptok = (a.prompt && next < s0.n_prompt) ? a.prompt[next] : 0u;
  const float logit0 = a.logits[0];
  const EmbedArgs& e = a.embed;
  const uint32_t t = threadIdx.x, rn = 2 * e.rope_half;  // one element per thread when it fits
  const bool rope = a.embed_next && e.rope_cur && next < e.rope_rows;
  const bool rope_regs = rn <= blockDim.x;
  float rv = 0.0f;
  if (rope && rope_regs && t < rn)
    rv = t < e.rope_half ? e.rope_cos[size_t(next) * e.rope_half + t] : e.rope_sin[size_t(next) * e.rope_half + (t - e.rope_half)];
  float bv = -1e30f;
  uint32_t bi = 0xffffffffu, nf = 0;
  for (uint32_t i = threadIdx.x; i < a.n_partials; i += blockDim.x) {
    const ArgmaxPartial p = a.partials[i];
    nf |= p.nonfinite;
    if (better(p.value, p.index, bv, bi)) { bv = p.value; bi = p.index; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = pair_val(bv, o);
    const uint32_t oi = pair_u(bi, o);
    nf |= pair_u(nf, o);
    if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
  }
  if (rope && rope_regs && t < rn) e.rope_cur[t] = rv;
  if (rope && !rope_regs) stage_rope_row(e, next);
  __shared__ float s_v[4];
  __shared__ uint32_t s_i[4], s_nf[4];
  const int w = threadIdx.x >> 6;
  if ((threadIdx.x & 63) == 0) { s_v[w] = bv; s_i[w] = bi; s_nf[w] = nf; }
  __syncthreads();
  __shared__ uint32_t s_next;
  if (threadIdx.x == 0) {
  for (int k = 1; k < int(blockDim.x >> 6); ++k) {
    nf |= s_nf[k];
    if (better(s_v[k], s_i[k], bv, bi)) { bv = s_v[k]; bi = s_i[k]; }
  }
  const uint32_t arg = bi == 0xffffffffu ? 0u : bi;
  StepResult* r = a.result;
  r->argmax = arg;
  r->max_logit = bv;
  r->token0_logit = logit0;
  r->all_finite = nf ? 0u : 1u;
  StepState s = s0;
  if (a.out_tokens) a.out_tokens[s.pos] = arg;
  s.token = (a.prompt && next < s.n_prompt) ? ptok : arg;
  s.pos = next;
  s.n_steps += 1;
  s.broken = 0u;
  *a.state = s;
  s_next = s.token;
  }
  // the next step's input: the embedding row of the next token (one launch less per step)
  if (a.embed_next) {
    __syncthreads();
    embed_token(a.embed, s_next, threadIdx.x, blockDim.x, true);
  }
}

// dequantisation half of gemvCellFlat (chpe_engine.zig:598-699), materialised
__global__ void k_flat_tile_weights(const uint8_t* cell, float* out) {
  const Image im{cell, 17408};
  const uint8_t qb = im.u8(16448 + 20);
  const bool g128 = (im.u64(16448 + 24) & 1u) != 0;
  const float scale = im.f32(16448 + 32), bias = im.f32(16448 + 36);
  for (uint32_t i = threadIdx.x; i < 32768; i += blockDim.x) {
    float w = 0.0f;
    if (qb == 4) {
      const float q = float((im.u8(64 + i / 2) >> (4 * (i & 1))) & 15u) - 8.0f;
      w = g128 ? q * h2f(im.u16(16448 + 48 + 2 * (i / 128))) : __fadd_rn(__fmul_rn(q, scale), bias);
    } else if (qb == 2) {
      const float q = codebook_w2((im.u8(64 + i / 4) >> (2 * (i & 3))) & 3u);
      w = g128 ? q * h2f(im.u16(16448 + 48 + 2 * (i / 128))) : __fadd_rn(__fmul_rn(q, scale), bias);
    }
    out[i] = w;
  }
  __syncthreads();
  if (threadIdx.x == 0 && (qb == 4 || qb == 2)) {
    const uint32_t n = im.u16(16448 + 560);
    if (n > 0 && n <= 64)
      for (uint32_t m = 0; m < n; ++m) {
        const uint32_t off = im.u16(16448 + 690 + 2 * m);
        if (off < 32768) out[off] = h2f(im.u16(16448 + 562 + 2 * m));
      }
  }
}

__global__ void k_embed_row_cell(const uint8_t* cell, uint64_t len, uint32_t row, uint32_t D,
                                 float* out, int* written) {
  const Image im{cell, len};
  const bool w = unpack_embed_row_cell(im, 0, row, D, out, threadIdx.x, blockDim.x, true);
  if (threadIdx.x == 0) *written = w ? 1 : 0;
}

}  // namespace

namespace {
thread_local LaunchProbe g_probe;
}

void arm_launch_probe(hipEvent_t start, hipEvent_t stop) { g_probe = LaunchProbe{start, stop}; }

LaunchProbe take_launch_probe() {
  const LaunchProbe p = g_probe;
  g_probe = LaunchProbe{};
  return p;
}

namespace detail {
thread_local bool g_record_names = false;
thread_local const char* g_last_kernel = nullptr;
}  // namespace detail

void record_kernel_names(bool on) {
  detail::g_record_names = on;
  if (on) detail::g_last_kernel = nullptr;
}

const char* last_kernel_name() { return detail::g_last_kernel ? detail::g_last_kernel : ""; }

void launch_embed(const EmbedArgs& a, hipStream_t st) {
  launch_kernel(k_embed, dim3(a.D > 256 ? (a.D + 255) / 256 : 1), dim3(256), st, a);
}

void launch_block_embed(const EmbedArgs& e, const uint32_t* tokens, uint32_t m, float* X, float* ssp, uint32_t* brk,
                        hipStream_t st) {
  launch_kernel(k_block_embed, dim3(m), dim3(256), st, e, tokens, X, ssp, brk);
}

void launch_finish(const FinishArgs& a, hipStream_t st) {
  launch_kernel(k_finish, dim3(1), dim3(256), st, a);
}

void launch_flat_tile_weights(const uint8_t* cell, float* out, hipStream_t st) {
  hipLaunchKernelGGL(k_flat_tile_weights, dim3(1), dim3(256), 0, st, cell, out);
}

void launch_embed_row_cell(const uint8_t* cell, uint64_t len, uint32_t row, uint32_t D, float* out,
                           int* written, hipStream_t st) {
  hipLaunchKernelGGL(k_embed_row_cell, dim3(1), dim3(256), 0, st, cell, len, row, D, out, written);
}

}  // namespace chpe
