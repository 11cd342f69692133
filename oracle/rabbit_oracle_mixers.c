/*
 * rabbit_oracle_mixers.c -- scalar CPU restatement of Qwen 3.8's two token mixers.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker; never part of the product path). Compiled with
 * -ffp-contract=off: every product and sum is rounded on its own, in the order the cited Rust code
 * performs it; transcendentals are the C library's expf / logf / log1pf / powf / sinf / cosf /
 * sqrtf, the functions Rust's f32 methods call on this platform.
 *
 *   Gated DeltaNet, one token (qwen38/generate.rs:196-219 minus the input / output projections):
 *     ShortConvState::step        kimi_linear/short_conv.rs:58-85
 *     gdn::step_token             qwen38/gdn.rs:142-196
 *       activate_and_split        qwen38/gdn.rs:96-106 (swish, kimi_linear/ops.rs:22-24)
 *       prepare_qk                qwen38/gdn.rs:110-118 (l2_norm, kimi_linear/ops.rs:34-40)
 *       key_head_of               qwen38/gdn.rs:62-65
 *       alpha_from_decay          qwen38/gdn.rs:76-80 -> decay_gate kimi_linear/kda.rs:65-76,
 *                                 softplus kimi_linear/kda.rs:28-30
 *       beta_from_projection      qwen38/gdn.rs:85-87 (sigmoid)
 *       KdaState::step            kimi_linear/kda.rs:132-166
 *       head_output_gate_silu     qwen38/gdn.rs:122-128 (rmsnorm kimi_linear/ops.rs:46-53)
 *   GQA attention, one token (qwen38/generate.rs:226-255 minus the projections):
 *     split_query_gate            qwen38/attention.rs:122-133
 *     norm_heads                  qwen38/attention.rs:138-143 (rmsnorm_1p qwen38/ops.rs:25-33)
 *     rope_half                   qwen38/attention.rs:160-172
 *     KvCache::push               qwen38/attention.rs:76-82
 *     attend                      qwen38/attention.rs:190-217 (softmax glm52/attention.rs:88-98)
 *     apply_output_gate           qwen38/attention.rs:221-226
 *
 * Parity pins (tests/test_oracle_mixers.py): the reference's own tests for these functions
 * (qwen38/gdn.rs:234-424, qwen38/attention.rs:228-391, kimi_linear/kda.rs tests' naive form),
 * restated, plus float64 transcriptions of the formulas on random inputs.
 */
#include "rabbit_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* kimi_linear/ops.rs:22-28 */
static float swishf(float x) { return x / (1.0f + expf(-x)); }
static float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }

/* kimi_linear/kda.rs:28-30: x.max(0.0) + (-x.abs()).exp().ln_1p() */
static float softplusf(float x) { return fmaxf(x, 0.0f) + log1pf(expf(-fabsf(x))); }

/* kimi_linear/ops.rs:34-40: sum_sq as a sequential f32 fold, scale = 1 / max(sqrt(sum_sq), eps). */
static void l2_norm(float *x, size_t n, float eps) {
    float sum_sq = 0.0f;
    for (size_t i = 0; i < n; i++) sum_sq += x[i] * x[i];
    float scale = 1.0f / fmaxf(sqrtf(sum_sq), eps);
    for (size_t i = 0; i < n; i++) x[i] *= scale;
}

void orc_short_conv_step(float *history, size_t d_inner, size_t kernel, const float *x, const float *weight,
                         float *out) {
    size_t hist_len = kernel - 1;
    for (size_t c = 0; c < d_inner; c++) {
        const float *hist = history + c * hist_len;
        const float *w = weight + c * kernel;
        float acc = 0.0f;
        for (size_t t = 0; t < hist_len; t++) acc += w[t] * hist[t];
        acc += w[hist_len] * x[c];
        out[c] = acc;
    }
    for (size_t c = 0; c < d_inner; c++) {
        float *h = history + c * hist_len;
        for (size_t t = 0; t + 1 < hist_len; t++) h[t] = h[t + 1];
        if (hist_len > 0) h[hist_len - 1] = x[c];
    }
}

/* kimi_linear/kda.rs:65-76 with lower_bound None: alpha = exp(-exp(a_log) * softplus(g + dt_bias)). */
float orc_gdn_alpha(float a_log, float a, float dt_bias) {
    float neg_exp_a_log = -expf(a_log);
    return expf(neg_exp_a_log * softplusf(a + dt_bias));
}

/* kimi_linear/kda.rs:132-166 for one head: s[d_k * d_v] row-major, alpha broadcast. */
void orc_kda_step(float *s, size_t d_k, size_t d_v, const float *q, const float *k, const float *v, float alpha,
                  float beta, float *o) {
    for (size_t i = 0; i < d_k; i++)
        for (size_t j = 0; j < d_v; j++) s[i * d_v + j] *= alpha;
    float *c = (float *)calloc(d_v, sizeof(float));
    for (size_t i = 0; i < d_k; i++)
        for (size_t j = 0; j < d_v; j++) c[j] += k[i] * s[i * d_v + j];
    for (size_t i = 0; i < d_k; i++) {
        float bk = beta * k[i];
        for (size_t j = 0; j < d_v; j++) s[i * d_v + j] += bk * (v[j] - c[j]);
    }
    for (size_t j = 0; j < d_v; j++) o[j] = 0.0f;
    for (size_t i = 0; i < d_k; i++)
        for (size_t j = 0; j < d_v; j++) o[j] += q[i] * s[i * d_v + j];
    free(c);
}

/* qwen38/gdn.rs:110-118: l2-normalise q and k (eps 1e-6, gdn.rs:57), then q *= 1 / sqrt(d_k). */
void orc_gdn_prepare_qk(float *q, float *k, size_t d_k) {
    l2_norm(q, d_k, 1e-6f);
    l2_norm(k, d_k, 1e-6f);
    float scale = 1.0f / sqrtf((float)d_k);
    for (size_t i = 0; i < d_k; i++) q[i] *= scale;
}

/* qwen38/gdn.rs:122-128: rmsnorm(o, norm_weight, eps), then o *= swish(z). */
void orc_gdn_output_gate(float *o, const float *norm_weight, const float *z, size_t d_v, float eps) {
    orc_rmsnorm(o, norm_weight, d_v, eps);
    for (size_t j = 0; j < d_v; j++) o[j] *= swishf(z[j]);
}

int orc_gdn_step_token(float *states, size_t n_v, size_t d_k, size_t d_v, float *qkv, size_t key_dim,
                       const float *z, const float *a, const float *b, const float *a_log, const float *dt_bias,
                       const float *norm_weight, float eps, float *out) {
    size_t value_dim = n_v * d_v;
    if (n_v == 0 || d_k == 0 || key_dim == 0 || key_dim % d_k) return -1;
    size_t n_k = key_dim / d_k;
    if (n_v % n_k) return -1;
    /* activate_and_split: SiLU over the whole conv row, then q | k | v */
    for (size_t i = 0; i < 2 * key_dim + value_dim; i++) qkv[i] = swishf(qkv[i]);
    float *qp = (float *)malloc(key_dim * sizeof(float)), *kp = (float *)malloc(key_dim * sizeof(float));
    memcpy(qp, qkv, key_dim * sizeof(float));
    memcpy(kp, qkv + key_dim, key_dim * sizeof(float));
    const float *vall = qkv + 2 * key_dim;
    /* prepare_qk once per K head */
    for (size_t kh = 0; kh < n_k; kh++) orc_gdn_prepare_qk(qp + kh * d_k, kp + kh * d_k, d_k);
    size_t n_rep = n_v / n_k;
    for (size_t h = 0; h < n_v; h++) {
        size_t kh = h / n_rep; /* key_head_of: repeat_interleave blocks */
        float alpha = orc_gdn_alpha(a_log[h], a[h], dt_bias[h]);
        float beta = sigmoidf_(b[h]);
        float *o = out + h * d_v;
        orc_kda_step(states + h * d_k * d_v, d_k, d_v, qp + kh * d_k, kp + kh * d_k, vall + h * d_v, alpha, beta, o);
        orc_gdn_output_gate(o, norm_weight, z + h * d_v, d_v, eps);
    }
    free(qp);
    free(kp);
    return 0;
}

/* ---- GQA -------------------------------------------------------------------------------------- */
void orc_rope_half(float *v, size_t rope_dim, size_t pos, float theta) {
    size_t half = rope_dim / 2;
    for (size_t j = 0; j < half; j++) {
        float inv = powf(theta, -2.0f * (float)j / (float)rope_dim);
        float ang = (float)pos * inv;
        float sn = sinf(ang), cs = cosf(ang);
        float a = v[j], b = v[j + half];
        v[j] = a * cs - b * sn;
        v[j + half] = b * cs + a * sn;
    }
}

/* glm52/attention.rs:88-98 */
static void softmax(float *x, size_t n) {
    float m = -1e30f;
    for (size_t i = 0; i < n; i++) m = fmaxf(m, x[i]);
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) {
        x[i] = expf(x[i] - m);
        sum += x[i];
    }
    for (size_t i = 0; i < n; i++) x[i] /= sum;
}

void orc_gqa_attend(const float *q, size_t n_heads, const float *k_cache, const float *v_cache, size_t positions,
                    size_t n_kv, size_t head_dim, float scale, float *out) {
    size_t n_rep = n_heads / n_kv;
    float *scores = (float *)malloc((positions ? positions : 1) * sizeof(float));
    for (size_t h = 0; h < n_heads; h++) {
        size_t kvh = h / n_rep;
        const float *qh = q + h * head_dim;
        for (size_t t = 0; t < positions; t++) {
            const float *k = k_cache + (t * n_kv + kvh) * head_dim;
            float dot = 0.0f;
            for (size_t d = 0; d < head_dim; d++) dot += qh[d] * k[d];
            scores[t] = dot * scale;
        }
        softmax(scores, positions);
        float *dst = out + h * head_dim;
        for (size_t d = 0; d < head_dim; d++) dst[d] = 0.0f;
        for (size_t t = 0; t < positions; t++) {
            const float *v = v_cache + (t * n_kv + kvh) * head_dim;
            float w = scores[t];
            for (size_t d = 0; d < head_dim; d++) dst[d] += w * v[d];
        }
    }
    free(scores);
}

int orc_gqa_step(const float *qg, const float *k_in, const float *v_in, size_t n_heads, size_t n_kv, size_t head_dim,
                 const float *q_norm, const float *k_norm, float eps, size_t rope_dim, float theta, float attn_scale,
                 float *k_cache, float *v_cache, size_t pos, float *ctx) {
    if (n_kv == 0 || n_heads % n_kv || rope_dim > head_dim || rope_dim % 2) return -1;
    size_t qw = n_heads * head_dim, kw = n_kv * head_dim;
    float *q = (float *)malloc(qw * sizeof(float)), *gate = (float *)malloc(qw * sizeof(float));
    float *k = (float *)malloc(kw * sizeof(float));
    /* split_query_gate: per head [query(head_dim), gate(head_dim)] */
    for (size_t h = 0; h < n_heads; h++) {
        memcpy(q + h * head_dim, qg + h * 2 * head_dim, head_dim * sizeof(float));
        memcpy(gate + h * head_dim, qg + h * 2 * head_dim + head_dim, head_dim * sizeof(float));
    }
    memcpy(k, k_in, kw * sizeof(float));
    for (size_t h = 0; h < n_heads; h++) orc_rmsnorm_1p(q + h * head_dim, q_norm, head_dim, eps);
    for (size_t h = 0; h < n_kv; h++) orc_rmsnorm_1p(k + h * head_dim, k_norm, head_dim, eps);
    for (size_t h = 0; h < n_heads; h++) orc_rope_half(q + h * head_dim, rope_dim, pos, theta);
    for (size_t h = 0; h < n_kv; h++) orc_rope_half(k + h * head_dim, rope_dim, pos, theta);
    /* KvCache::push at position pos */
    memcpy(k_cache + pos * kw, k, kw * sizeof(float));
    memcpy(v_cache + pos * kw, v_in, kw * sizeof(float));
    orc_gqa_attend(q, n_heads, k_cache, v_cache, pos + 1, n_kv, head_dim, attn_scale, ctx);
    /* apply_output_gate: ctx *= sigmoid(gate) */
    for (size_t i = 0; i < qw; i++) ctx[i] *= sigmoidf_(gate[i]);
    free(q);
    free(gate);
    free(k);
    return 0;
}
