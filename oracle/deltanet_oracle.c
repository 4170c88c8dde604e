/* deltanet_oracle.c -- CPU restatement of one decode step of a gated-DeltaNet
 * (linear-attention) layer of Qwen3.5.  TEST INFRASTRUCTURE (the oracle), never the product.
 *
 * The reference engine has no code for these layers (its README only claims them), so this
 * follows the published algorithm: the gated delta rule of Yang, Kautz and Hatamizadeh,
 * "Gated Delta Networks: Improving Mamba2 with Delta Rule" (ICLR 2025),
 *     S_t = exp(g_t) S_{t-1} + k_t (beta_t (v_t - (exp(g_t) S_{t-1})^T k_t))^T,  o_t = S_t^T q_t,
 * in the form and with the surrounding arithmetic of the third-party library that defines the
 * Qwen3.5 layer, transformers 5.15.0 (models/qwen3_5/modeling_qwen3_5.py):
 *     causal_conv1d_update ........ :200-217 (depthwise causal conv over [state, x], SiLU)
 *     l2norm ...................... :242-245 (x * rsqrt(sum x^2 + 1e-6))
 *     torch_recurrent_gated_delta_rule :331-380 (q scaled by 1/sqrt(dk), S decayed first)
 *     beta = sigmoid(b), g = -exp(A_log) * softplus(a + dt_bias) ... :497-499
 *     q/k heads repeated to the value heads (repeat_interleave) ..... :500-502
 *     Qwen3_5RMSNormGated ......... :168-184, applied per value head at :539
 *                                   (RMSNorm over a head, * weight, * silu(z))
 *
 * Parity pinning (tests/test_oracle_deltanet.py): float64 brute force on random inputs;
 * invariants (beta = 0 => S_t = exp(g) S_{t-1}; g -> -inf with beta = 1 => S_t = k v^T for a
 * unit k; a zero state gives o = (q.k) beta v); and fixtures written by the library's own
 * torch routines (tests/golden/make_deltanet_fixtures.py).
 */
#include <math.h>
#include <stddef.h>
#include <string.h>

#include "chpe_oracle.h"

static float silu_f(float x) { return x / (1.0f + expf(-x)); }

/* torch.nn.functional.softplus, beta 1, threshold 20 */
static float softplus_f(float x) { return x > 20.0f ? x : log1pf(expf(x)); }

void oref_conv1d_update(size_t channels, size_t taps, const float *x, const float *w, float *state,
                        float *out) {
    for (size_t c = 0; c < channels; c++) {
        float *st = state + c * (taps - 1);
        const float *wc = w + c * taps;
        float acc = 0.0f;
        for (size_t k = 0; k + 1 < taps; k++) acc += wc[k] * st[k];
        acc += wc[taps - 1] * x[c];
        out[c] = silu_f(acc);
        for (size_t k = 0; k + 2 < taps; k++) st[k] = st[k + 1];
        st[taps - 2] = x[c];
    }
}

static void l2norm_f(const float *x, size_t n, float *y) {
    float s = 0.0f;
    for (size_t i = 0; i < n; i++) s += x[i] * x[i];
    const float inv = 1.0f / sqrtf(s + 1e-6f);
    for (size_t i = 0; i < n; i++) y[i] = x[i] * inv;
}

void oref_gated_delta_step(size_t n_v_heads, size_t n_k_heads, size_t dk, size_t dv, const float *q,
                           const float *k, const float *v, const float *a, const float *b,
                           const float *A_log, const float *dt_bias, float *state, float *out) {
    float qn[512], kn[512], kv[512];
    if (dk > 512 || dv > 512 || n_k_heads == 0 || n_v_heads % n_k_heads) return;
    const size_t rep = n_v_heads / n_k_heads;
    const float scale = 1.0f / sqrtf((float)dk);
    for (size_t h = 0; h < n_v_heads; h++) {
        const size_t kh = h / rep;
        l2norm_f(q + kh * dk, dk, qn);
        l2norm_f(k + kh * dk, dk, kn);
        for (size_t i = 0; i < dk; i++) qn[i] *= scale;
        const float beta = 1.0f / (1.0f + expf(-b[h]));
        const float g = -expf(A_log[h]) * softplus_f(a[h] + dt_bias[h]);
        const float decay = expf(g);
        float *S = state + h * dk * dv; /* [dk][dv] */
        for (size_t i = 0; i < dk * dv; i++) S[i] *= decay;
        for (size_t j = 0; j < dv; j++) {
            float m = 0.0f;
            for (size_t i = 0; i < dk; i++) m += S[i * dv + j] * kn[i];
            kv[j] = m;
        }
        const float *vh = v + h * dv;
        for (size_t j = 0; j < dv; j++) {
            const float delta = (vh[j] - kv[j]) * beta;
            for (size_t i = 0; i < dk; i++) S[i * dv + j] += kn[i] * delta;
        }
        float *oh = out + h * dv;
        for (size_t j = 0; j < dv; j++) {
            float o = 0.0f;
            for (size_t i = 0; i < dk; i++) o += S[i * dv + j] * qn[i];
            oh[j] = o;
        }
    }
}

void oref_gated_rmsnorm(size_t n, size_t dv, const float *x, const float *z, const float *w, float eps,
                        float *out) {
    for (size_t h = 0; h < n; h++) {
        const float *xh = x + h * dv, *zh = z + h * dv;
        float s = 0.0f;
        for (size_t j = 0; j < dv; j++) s += xh[j] * xh[j];
        const float r = 1.0f / sqrtf(s / (float)dv + eps);
        for (size_t j = 0; j < dv; j++) out[h * dv + j] = w[j] * (xh[j] * r) * silu_f(zh[j]);
    }
}
