/* chpe_oracle.h -- CPU restatement of the reference decode path (test infrastructure).
 *
 * THIS IS THE ORACLE, NOT THE PRODUCT.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py load it, and only as the checker / the timed CPU
 * baseline.  The engine (libchpe.so) never links it.
 *
 * It restates, in plain C, `CHPEEngine.forwardDecode` and everything it calls in the
 * reference (src/chpe_engine.zig), with the reference's float arithmetic structure:
 *   - `@Vector(8,f32)` accumulators are 8 independent lanes; `@reduce(.Add)` is the
 *     ordered sum lane0+lane1+...+lane7 (LLVM ordered fadd reduction);
 *   - `@mulAdd` is fmaf(); every other `a*b + c` is a rounded multiply then add
 *     (built with -ffp-contract=off, -fno-fast-math);
 *   - expf/powf/sinf/cosf come from the C library (the reference uses Zig's own;
 *     those few ulps are the only deliberate source of difference).
 * Row-parallel OpenMP keeps every output row's summation order, so the result is
 * bit-identical for any thread count.
 *
 * Parity pinning (what each function is checked against) is listed in the header
 * comment of chpe_oracle.c.
 */
#ifndef CHPE_ORACLE_H
#define CHPE_ORACLE_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- model presets: src/chpe_engine.zig:96-146 ---- */
typedef struct {
    int id; /* 0 = Qwen2.5-3B, 1 = Qwen3.5-9B, 2 = Qwen2.5-72B */
    size_t hidden_dim, intermediate_dim, num_layers, num_attn_heads, num_kv_heads, head_dim,
        vocab_size;
    float rope_theta, rms_eps;
} oref_arch;

int oref_arch_preset(int id, oref_arch *out);
/* arch guess from a path: src/main.zig:97-103, src/chpe_c_api.zig:29-37 */
int oref_arch_from_path(const char *path);

/* ---- layer map: src/chpe_engine.zig:1017-1142 ---- */
typedef struct {
    size_t input_norm, q_proj, q_tiles, k_proj, k_tiles, v_proj, v_tiles, o_proj, o_tiles,
        post_norm, gate_proj, gate_tiles, up_proj, up_tiles, down_proj, down_tiles;
    int64_t q_bias, k_bias, v_bias; /* -1 = null */
} oref_layer_info;

/* map: 0 = 3B raw (qwen3b_geometry.zig:48-79), 1 = 3B cell (qwen3b_tensor_map.zig),
 *      2 = 9B (qwen35_tensor_map.zig), 3 = 72B (qwen72b_tensor_map.zig) */
int oref_layer_info_for(int map, size_t layer, oref_layer_info *out);
size_t oref_final_norm_for(int map);

/* ---- archive validation: src/weight_archive.zig:152-172 ----
 * returns 0 ok, else 1 FileTooSmall, 2 InvalidMagic, 3 UnsupportedVersion,
 * 4 MisalignedHeader, 5 BadGeometry, 6 Truncated */
int oref_validate(const uint8_t *bytes, size_t len);

/* ---- primitives (src/chpe_engine.zig:157-216) ---- */
float oref_silu(float z);
void oref_rmsnorm(const float *x, const float *gamma, float *y, size_t n, float eps);
void oref_apply_rope(float *vec, size_t pos, size_t num_heads, size_t head_dim, float theta);
float oref_f16_to_f32(uint16_t h);
/* element-wise: f32 -> f16 round-to-nearest-even (the fp16 KV cache), f16 -> f32 */
void oref_f32_to_f16_n(const float *x, uint16_t *out, size_t n);
void oref_f16_to_f32_n(const uint16_t *h, float *out, size_t n);
float oref_bf16_to_f32(uint16_t h);

/* ---- cell kernels on one 17408-byte cell (src/chpe_engine.zig:223-751, 1288-1394) ---- */
void oref_gemv_tile_polymorphic(const uint8_t *cell, const float *x, size_t x_len, float *y,
                                size_t y_len, size_t row_base, int accumulate);
/* materialised weights of a flat tile (the `tile_weights` array, :584-699) */
void oref_flat_tile_weights(const uint8_t *cell, size_t wpt, float *tile_weights);
void oref_gemv_cell_flat(const uint8_t *cell, size_t t, size_t wpt, size_t r_total,
                         size_t c_total, const float *x, float *y);
/* returns 1 if `out` was written, 0 if the row was out of range (out left untouched) */
int oref_unpack_embed_row_cell(const uint8_t *cell, size_t row_in_tile, float *out, size_t D);

/* ---- attention for one layer (src/chpe_engine.zig:1699-1734) ----
 * k_cache / v_cache: [>= pos+1][kv_heads*head_dim] f32. out: [heads*head_dim]. */
void oref_attention(const float *q, const float *k_cache, const float *v_cache, size_t pos,
                    size_t heads, size_t kv_heads, size_t head_dim, float *scores, float *out);

/* ---- gated-DeltaNet decode step (no reference code; deltanet_oracle.c) ----
 * conv: x [channels], w [channels][taps], state [channels][taps-1] (oldest first, updated),
 * out [channels] = silu(causal depthwise conv).  step: q, k [n_k_heads][dk] (before the l2
 * norm), v [n_v_heads][dv], a, b, A_log, dt_bias [n_v_heads], state [n_v_heads][dk][dv]
 * (updated), out [n_v_heads][dv].  gated rmsnorm: out = w * (x * rsqrt(mean x^2 + eps)) * silu(z)
 * per head of dv values. */
void oref_conv1d_update(size_t channels, size_t taps, const float *x, const float *w, float *state,
                        float *out);
void oref_gated_delta_step(size_t n_v_heads, size_t n_k_heads, size_t dk, size_t dv, const float *q,
                           const float *k, const float *v, const float *a, const float *b,
                           const float *A_log, const float *dt_bias, float *state, float *out);
void oref_gated_rmsnorm(size_t n, size_t dv, const float *x, const float *z, const float *w, float eps,
                        float *out);

/* ---- engine (src/chpe_engine.zig:854-1803) ---- */
typedef struct {
    uint32_t argmax_token;
    float max_logit, token0_logit;
    uint64_t elapsed_ns;
    float hidden_norm;
    int all_finite;
} oref_result;

typedef struct oref_engine oref_engine;

/* Opens + mmaps + validates (weight_archive.zig:184-222), then CHPEEngine.init.
 * arch_id < 0: guess from path.  kv_f16 != 0 stores K/V rounded to fp16 (the
 * fp16-KV variant of the same algorithm).  threads <= 0: all cores.
 * Returns NULL on error; *err (if non-NULL) gets the validation code or -1. */
oref_engine *oref_open(const char *path, int arch_id, size_t max_seq_len, int kv_f16,
                       int threads, int *err);
/* Same over caller-owned bytes (no validation: CHPEEngine.init on raw bytes, as the
 * reference's own mock-archive tests do). */
oref_engine *oref_open_bytes(const uint8_t *bytes, size_t len, int arch_id,
                             size_t max_seq_len, int kv_f16, int threads);
void oref_close(oref_engine *e);
int oref_forward(oref_engine *e, uint32_t token, size_t pos, oref_result *res);
/* worker threads of the row-parallel loops (results do not depend on it) */
void oref_set_threads(oref_engine *e, int threads);
void oref_set_break(oref_engine *e, int on);  /* test only: 0 removes the non-finite break */
/* The true Qwen3.5-9B hybrid layers on the 9B cell archive (24 gated-DeltaNet layers, 8 gated
 * full-attention layers with q/k norms and partial rotary embedding) instead of the
 * reference's GQA aliasing; 0 ok, -1 not a 9B cell archive or out of memory. */
int oref_set_hybrid(oref_engine *e, int on);
/* the same step over the first n_layers layers only (a CPU timing sample) */
int oref_forward_layers(oref_engine *e, uint32_t token, size_t pos, size_t n_layers, oref_result *res);
/* Timing aid (no reference counterpart): fill K/V cache rows 0..n_pos-1 of every layer with
 * seeded values in [-1, 1) (fp16-rounded in kv_f16 mode), so that oref_forward can be timed at
 * position n_pos without decoding a prompt first.  Returns -2 if n_pos > max_seq_len. */
int oref_prefill_synthetic(oref_engine *e, size_t n_pos, uint64_t seed);
const float *oref_logits(const oref_engine *e);
const float *oref_hidden(const oref_engine *e);
size_t oref_vocab(const oref_engine *e);
size_t oref_hidden_dim(const oref_engine *e);
/* engine flags after init: is_raw, is_raw_fp16, is_dense, quant_bits, wpt, record_count */
void oref_engine_info(const oref_engine *e, int64_t out[8]);
/* one gemvLinear call against the engine's archive (src/chpe_engine.zig:1396-1489) */
void oref_gemv_linear(oref_engine *e, size_t tile_start, size_t num_tiles, const float *x,
                      size_t x_len, float *y, size_t y_len, size_t r_total, size_t c_total,
                      int accumulate, int64_t bias_tile);
/* norm / bias unpack with the reference's fallbacks (:1144-1192) */
void oref_unpack_norm(oref_engine *e, size_t tile, float *out, size_t n);
void oref_unpack_bias(oref_engine *e, size_t tile, float *out, size_t n);
void oref_unpack_embed_row(oref_engine *e, uint32_t token, float *out);
/* computeLmHead (chpe_engine.zig:1554-1660) on `xn` (hidden_dim floats, already normed):
 * vocab_size logits into `logits` */
void oref_compute_lm_head(oref_engine *e, const float *xn, float *logits);

/* Teacher-forced prompt (positions 0..n_prompt-1) then greedy feedback for n_gen
 * tokens.  out_tokens[n_gen]; top2_gap[n_gen] (optional) = max logit - runner-up. */
int oref_generate(oref_engine *e, const uint32_t *prompt, size_t n_prompt, size_t n_gen,
                  uint32_t *out_tokens, float *top2_gap);

#ifdef __cplusplus
}
#endif
#endif
