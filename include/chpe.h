/* chpe.h -- C ABI of the MI355X decode engine (libchpe.so).
 *
 * The first twelve symbols are the reference's C ABI (src/chpe_c_api.zig:25-143) with the
 * same signatures, ownership and sentinel-value error behaviour; each one cites the
 * reference symbol it replaces.  Behaviour kept on purpose:
 *   - chpe_init guesses the architecture from the path ("9B"/"9b"/"qwen35" -> Qwen3.5-9B,
 *     "72B"/"72b" -> Qwen2.5-72B, else Qwen2.5-3B) and fixes max_seq_len at 2048;
 *   - chpe_forward_tokens restarts at position 0 on every call (teacher-forced prompt);
 *   - getters on a NULL context return the 3B defaults (vocab/hidden/layers) or 0.
 * One deliberate difference: where the reference reads past its KV cache (more tokens than
 * max_seq_len), chpe_forward_tokens returns -2.
 *
 * Symbols after those twelve are additions; they have no counterpart in the reference.
 * A context is not re-entrant (one engine state); separate contexts are independent.
 */
#ifndef CHPE_H
#define CHPE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* chpe_c_api.zig:25-48 `chpe_init`: mmap + validate the archive, build the engine.
 * Returns NULL on any error. */
void *chpe_init(const char *archive_path);

/* chpe_c_api.zig:50-78 `chpe_forward_tokens`: decode positions 0..num_tokens-1.
 * Returns the last argmax, -1 if ctx/tokens is NULL or num_tokens == 0, -2 if num_tokens
 * exceeds the context's max_seq_len, -3 on a device error.  out_logits (optional) receives
 * vocab_size floats of the last step. */
int chpe_forward_tokens(void *ctx, const uint32_t *tokens, size_t num_tokens, float *out_logits);

/* chpe_c_api.zig:80-87 `chpe_get_last_logits`: copies vocab_size floats of the last step;
 * returns vocab_size, or 0 if ctx/out is NULL or max_len < vocab_size. */
size_t chpe_get_last_logits(void *ctx, float *out_logits, size_t max_len);

size_t chpe_get_vocab_size(void *ctx);   /* chpe_c_api.zig:89-93 */
size_t chpe_get_hidden_dim(void *ctx);   /* chpe_c_api.zig:95-99 */
size_t chpe_get_num_layers(void *ctx);   /* chpe_c_api.zig:101-105 */
uint64_t chpe_get_last_elapsed_ns(void *ctx);   /* chpe_c_api.zig:107-111 */
uint32_t chpe_get_last_argmax(void *ctx);       /* chpe_c_api.zig:113-117 */
float chpe_get_last_max_logit(void *ctx);       /* chpe_c_api.zig:119-123 */
float chpe_get_last_token0_logit(void *ctx);    /* chpe_c_api.zig:125-129 */
float chpe_get_last_hidden_norm(void *ctx);     /* chpe_c_api.zig:131-135 */

/* chpe_c_api.zig:137-143 `chpe_free`: releases the engine, its device memory and the map. */
void chpe_free(void *ctx);

/* ---------------- additions (no counterpart in the reference) ---------------- */

/* chpe_init with an explicit architecture (0 = Qwen2.5-3B, 1 = Qwen3.5-9B,
 * 2 = Qwen2.5-72B, 3 = Qwen3.5-9B with its true hybrid layers -- gated DeltaNet and gated
 * full attention with q / k norms and partial rotary embedding, recurrent states cleared at
 * position 0; the 9B cell archive only --, -1 = guess from the path), max_seq_len and
 * KV-cache type (kv_f16 != 0: fp16 KV cache in HBM; 0: f32 as the reference).  Arch 1 is the
 * reference's decode of the 9B map (its GQA aliasing, chpe_engine.zig:1663-1803). */
void *chpe_init_ex(const char *archive_path, int arch, size_t max_seq_len, int kv_f16);

/* One forwardDecode(token, pos) (src/chpe_engine.zig:1663) on the context's current KV
 * cache.  Returns the argmax, -1 bad args, -2 pos >= max_seq_len, -3 device error. */
int chpe_decode_step(void *ctx, uint32_t token, size_t pos, float *out_logits);

/* Teacher-forced prompt (positions 0..n_prompt-1), then n_gen greedy tokens with the argmax
 * fed back on the device (n_prompt + n_gen - 1 steps).  out_tokens[n_gen].  Returns 0,
 * -1 bad args, -2 too long for max_seq_len, -3 device error. */
int chpe_generate(void *ctx, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                  uint32_t *out_tokens);

/* Batch-M verify: drafts[0..m) consumed at positions pos..pos+m-1 over the cache built by
 * earlier calls, out_argmax[i] = the argmax after draft i.  Equal to m sequential
 * chpe_decode_step(ctx, drafts[i], pos + i) calls (the reference has no verify code; its
 * equivalent is m forwardDecode calls, src/chpe_engine.zig:1663-1803, whose KV write at pos
 * overwrites the row, :1693-1697): on archives of flat 4- or 2-bit tiles or 4-bit 16-row cells
 * (chpe_block_ready) and
 * 2 <= m <= 32 as one block step that reads every weight once for the m drafts, with each draft's
 * arithmetic that of the decode step up to the order of the float sums; otherwise m replays of
 * the decode step, bit-identical.  last_* report the final step; chpe_get_last_logits gives
 * its logits.  Returns 0, -1 bad args, -2 pos + m > max_seq_len, -3 device error. */
int chpe_verify(void *ctx, const uint32_t *drafts, size_t m, size_t pos, uint32_t *out_argmax);
/* Prefill: positions 0..num_tokens-1 teacher-forced as chpe_forward_tokens, in block steps of
 * up to 32 tokens that read every weight once per block (archives of flat 4- or 2-bit tiles or
 * 4-bit 16-row cells; others:
 * the sequential steps).  Each token's arithmetic is the decode step's up to the order of the
 * float sums; the KV cache holds the same rows.  Leaves the decode state at (the last argmax,
 * num_tokens).  Returns the last argmax, -1 bad args, -2 too long, -3 device error;
 * out_logits (optional) receives the last position's logits. */
int chpe_prefill(void *ctx, const uint32_t *tokens, size_t num_tokens, float *out_logits);
/* 1 when the archive runs the block step (every projection flat 4- or 2-bit tiles or 4-bit 16-row
 * cells at 2048 columns, one width per launch: q/k/v alike, gate/up alike), else 0. */
int chpe_block_ready(void *ctx);

/* Message of the last failed chpe_init / chpe_init_ex on this thread ("" if none). */
const char *chpe_last_error(void);
/* The first 16 hex digits of the SHA-256 of the sources this library was built from (the
 * Makefile's LIBSRC list), so that a caller can tell a library built from other sources. */
const char *chpe_build_id(void);

size_t chpe_get_max_seq_len(void *ctx);
/* hidden_dim floats of the residual stream after the last step. */
int chpe_get_hidden(void *ctx, float *out);

/* Timing: enqueue `n` decode steps that continue from the device state (greedy feedback),
 * bracketed by HIP events on the engine's stream; *ms = elapsed milliseconds. */
int chpe_time_steps(void *ctx, size_t n, float *ms);
/* Launch one stage alone (0 q/k/v, 1 o, 2 gate+up, 3 down, 4 LM head, 5 attention over the
 * context chunks, 6 merge of the chunks) for each layer in [layer0, layer1), `iters` times,
 * between HIP events; *ms = total.  The step's own kernels and arguments, except that o and
 * down add into scratch vectors (not the residual stream) and the LM head's logits replace the
 * last step's; stage 0 writes the KV row at the device position, which the next step
 * overwrites.  The hybrid model (arch 3): stages 2-4 only. */
int chpe_time_stage(void *ctx, int stage, size_t layer0, size_t layer1, size_t iters, float *ms);
/* Run n_steps real decode steps (greedy feedback, continuing from the device state), launched
 * without the graph and with a HIP event pair around every launch of `stage` (numbering as
 * above); *avg_ms = mean duration of one launch of that stage inside the step. */
int chpe_time_stage_live(void *ctx, int stage, size_t n_steps, float *avg_ms);
/* Algorithmic HBM bytes: of one stage launch for `layer` (stage 5: at the current position),
 * and of a whole step at `pos`. */
double chpe_stage_bytes(void *ctx, int stage, size_t layer);
double chpe_step_bytes(void *ctx, size_t pos);
/* The (mangled) name of the kernel that runs `stage` of layer 0 (numbering as above; the last
 * launch of the stage), looked up without launching anything (the decode state is untouched);
 * "" on error. */
const char *chpe_stage_kernel(void *ctx, int stage);

/* Parity hooks: one projection's GEMV on a caller vector (which: 0 q, 1 k, 2 v, 3 o,
 * 4 gate, 5 up, 6 down, 7 LM head), bias included, no norm; y gets the output rows.  -1 for
 * which 0-3 on the hybrid model (arch 3), whose mixers are not the reference map's q/k/v/o. */
int chpe_debug_gemv(void *ctx, size_t layer, int which, const float *x, float *y);
/* Materialised weights of one flat 32768-weight tile (gemvCellFlat's dequantisation),
 * computed by the GPU from the 17408-byte cell. */
int chpe_debug_flat_tile_weights(const uint8_t *cell, float *out32768);
/* One flat-tile GEMV (gemvCellFlat, src/chpe_engine.zig:584-729, as gemvLinear drives it for
 * tensors wider than 2048 columns, :1396-1489) through the decode step's kernels, on a rows x
 * cols tensor given as n_tiles consecutive 17408-byte cells, planned as the engine plans a
 * tensor: uniformly group-128 4- or 2-bit tiles on the uniform kernels, any other tile form,
 * a mix of forms or fewer tiles than the shape needs (a short tensor) tile by tile; outliers
 * replace weights.  mode 0: y = W x; 1: y += W x; 2: y = silu(W rmsnorm(x)) * (U rmsnorm(x))
 * with U in tiles_up; 3: y = W rmsnorm(x) (the LM head's logits) with *out_argmax (first index
 * of the maximum) and *out_hidden_norm = |x| (both optional).  rmsnorm uses gamma and eps;
 * gamma is given exactly in modes 2 and 3.  Returns 0, -1 on bad arguments or tiles
 * (chpe_last_error), -3 on a device error. */
int chpe_debug_gemv_flat(int mode, uint32_t rows, uint32_t cols, const uint8_t *tiles,
                         const uint8_t *tiles_up, size_t n_tiles, const float *x, const float *gamma,
                         float eps, float *y, uint32_t *out_argmax, float *out_hidden_norm);
/* One 16-row-cell GEMV at 2048 columns (gemvTileW4, src/chpe_engine.zig:326-418, per cell of
 * 16 rows; outliers added) through the decode step's kernels on caller cells: `cells` (and
 * `cells_up` for mode 2) hold ceil(rows/16) consecutive 17408-byte 4-bit group-128 cells; mode
 * and the other arguments as for chpe_debug_gemv_flat (x has 2048 floats; mode 3 writes the
 * logits, the first index of the maximum and the norm of x).  Returns 0, -1 on bad arguments
 * or cells (chpe_last_error), -3 on a device error. */
int chpe_debug_gemv_cells(int mode, uint32_t rows, const uint8_t *cells, const uint8_t *cells_up,
                          size_t n_cells, const float *x, const float *gamma, float eps, float *y,
                          uint32_t *out_argmax, float *out_hidden_norm);
/* One GEMV over raw tiles read as one row-major rows x cols matrix (gemvLinear's raw path,
 * src/chpe_engine.zig:1455-1488, dotSegment :1194-1251): kind 0 IEEE fp16, 1 bf16, 2 int8 with
 * each dot times 0.00373708; n_tiles consecutive 16384-byte tiles.  Modes and the other
 * arguments as for chpe_debug_gemv_flat.  Returns 0, -1 on bad arguments, -3 on a device error. */
int chpe_debug_gemv_raw(int mode, uint32_t rows, uint32_t cols, int kind, const uint8_t *tiles,
                        const uint8_t *tiles_up, size_t n_tiles, const float *x, const float *gamma, float eps,
                        float *y, uint32_t *out_argmax, float *out_hidden_norm);
/* One GEMV over polymorphic 16-row cells of any width (gemvTilePolymorphic,
 * src/chpe_engine.zig:732-751: 2-bit codebook, 4-bit, int8 with a per-row scale and bias,
 * fp16 / bf16, f32; group-128 scales or the tile's scale and bias; outliers added to group-128
 * cells of 16 rows) through the engine's polymorphic path, on n_cells consecutive 17408-byte
 * cells covering `rows` rows as gemvLinear walks them (row bases = prefix sums of dims.rows);
 * x has `cols` floats.  Modes and the other arguments as for chpe_debug_gemv_flat.  Returns 0,
 * -1 on bad arguments, -3 on a device error. */
int chpe_debug_gemv_poly(int mode, uint32_t rows, uint32_t cols, const uint8_t *cells, const uint8_t *cells_up,
                         size_t n_cells, const float *x, const float *gamma, float eps, float *y,
                         uint32_t *out_argmax, float *out_hidden_norm);
/* unpackEmbedRowCell on the GPU over `len` bytes starting at a cell (rows of wide tensors
 * read past the cell).  Returns 1 if written, 0 if the row is out of range, <0 on error. */
int chpe_debug_embed_row_cell(const uint8_t *bytes, size_t len, uint32_t row, uint32_t D,
                              float *out);
/* The decode step's attention (chunk + merge kernels) on caller data: q [heads][head_dim]
 * rotated queries, k_rows / v_rows [pos+1][kv_heads*head_dim] f32 (the layout of the
 * reference's KVCache rows, src/chpe_engine.zig:755-801); kv_f16 rounds them to fp16 first,
 * as the fp16 cache holds them.  out [heads][head_dim] (the attention loop :1700-1734).
 * 0 on success, -1 bad arguments or unsupported shape, -3 device error. */
int chpe_debug_attention(uint32_t head_dim, uint32_t heads, uint32_t kv_heads, int kv_f16, uint32_t pos,
                         const float *q, const float *k_rows, const float *v_rows, float *out);
/* No counterpart in the reference (it attends one position per forwardDecode call).  The block
 * step's attention on caller data: nq <= 32 queries q [nq][heads][head_dim] at positions
 * pos .. pos+nq-1, query z over rows 0..pos+z of k_rows / v_rows [pos+nq][kv_heads*head_dim]
 * (the fp16 cache and more than 4 queries: the multi-query launch); out [nq][heads][head_dim].
 * 0 on success, -1 bad arguments or unsupported shape, -3 device error. */
int chpe_debug_attention_block(uint32_t head_dim, uint32_t heads, uint32_t kv_heads, int kv_f16, uint32_t pos,
                               uint32_t nq, const float *q, const float *k_rows, const float *v_rows, float *out);
/* No counterpart in the reference.  The decode step's attention (chunk + merge kernels) on
 * caller device buffers, allocating nothing: for callers that cannot allocate (code under HIP
 * graph capture, serving loops, harnesses that forbid hipMalloc).  q [heads][head_dim] f32
 * rotated queries; k_cache [kv_heads][max_seq][head_dim] and v_cache in the engine's cache
 * layout (f32: as k_cache; kv_f16: fp16, k as above, v [kv_heads][max_seq/4][head_dim][4]),
 * rows 0..pos written; out [heads][head_dim] f32; all device pointers on the current device.
 * max_seq: cache rows per kv head, a multiple of 16, > pos.  stream: a hipStream_t (null: the
 * default stream); the call only enqueues.  The chunk partials live in a per-GPU device array
 * of 8 MiB (heads * ceil((pos+1)/chunk) * (head_dim + 2) * 4 bytes must fit, chunk = 8192 /
 * head_dim positions, 128 at head_dim 128 with >= 8 kv heads); calls that overlap on one GPU
 * race on it.  Returns 0, -1 bad arguments
 * or unsupported shape, -2 the partials exceed the scratch, -3 device error. */
int chpe_attention_noalloc(uint32_t head_dim, uint32_t heads, uint32_t kv_heads, int kv_f16, uint32_t pos,
                           uint32_t max_seq, const float *q, const void *k_cache, const void *v_cache,
                           float *out, void *stream);
/* Gated-DeltaNet (Qwen3.5 linear-attention layers) decode-step kernels on caller data.  The
 * reference has no code for these layers (README claims only); the arithmetic is the gated
 * delta rule as defined by transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py.
 * conv: causal depthwise conv over [state, x] + SiLU (:200-217); w [channels][taps], state
 * [channels][taps-1] (oldest first), updated in place; out [channels].
 * step: q, k [n_k_heads][head_dim] before the l2 norm, v [n_v_heads][head_dim], a, b, A_log,
 * dt_bias [n_v_heads] (:331-380, :497-502); state [n_v_heads][head_dim][head_dim] f32, updated in
 * place; out [n_v_heads][head_dim] = S^T q, or with norm_w (and z [n_v_heads][head_dim]) the
 * gated RMSNorm of it (:168-184).  head_dim 64 or 128.  0 on success, -1 bad arguments, -3
 * device error. */
int chpe_debug_deltanet_conv(uint32_t channels, uint32_t taps, const float *x, const float *w, float *state,
                             float *out);
int chpe_debug_deltanet_step(uint32_t n_v_heads, uint32_t n_k_heads, uint32_t head_dim, const float *q,
                             const float *k, const float *v, const float *a, const float *b, const float *A_log,
                             const float *dt_bias, const float *z, const float *norm_w, float eps, float *state,
                             float *out);

#ifdef __cplusplus
}
#endif
#endif
