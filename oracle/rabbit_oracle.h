/*
 * rabbit_oracle.h -- CPU restatement of ferrumox/rabbit's routed-expert dequant-matmul path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product library (rabbit_amd/) links, loads or calls
 * this code.  It is the parity checker for the HIP kernels (tests/, __graft_entry__.smoke()) and
 * the CPU baseline that bench.py times beside the GPU ("kind": "port").
 *
 * Every function restates one function of the reference (Rust, /root/reference/src) with the
 * same operation order, so that a scalar restatement reproduces the reference's fp32 results
 * bit for bit: the file is compiled with -ffp-contract=off because rustc never fuses a*b+c.
 * Citations are path:line inside the reference.
 *
 * Layouts (quant.rs:92-110):
 *   MXFP4  [rows, cols]: data u8[rows * ceil(cols/2)], low nibble first;
 *                        block_scale u8[rows * ceil(cols/32)] (E8M0, one per 32-element block).
 *   I4G    [rows, cols]: data u8[rows * ceil(cols/2)] holding value+8, low nibble first;
 *                        scale f32[rows * ceil(cols/gs)], scale[row*ngroups + g].
 *   F32    [rows, cols]: row-major f32.
 */
#ifndef RABBIT_ORACLE_H
#define RABBIT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ORC_QT_F32 = 0, ORC_QT_I4_GROUPED = 1, ORC_QT_MXFP4 = 2 };
enum { ORC_ACT_SILU = 0, ORC_ACT_SITU = 1 };

/* Activation (glm52/moe.rs:49-52): Silu, or Situ { beta, linear_beta: Option<f32> }. */
typedef struct {
    int kind;              /* ORC_ACT_* */
    float beta;
    float linear_beta;
    int has_linear_beta;
} orc_act;
enum { ORC_FAMILY_QWEN38 = 0, ORC_FAMILY_GLM52 = 1, ORC_FAMILY_KIMI_K3 = 2 };

/* One quantized matrix, mirrors QT / QTKind (quant.rs:77-110). Host pointers. */
typedef struct {
    size_t rows, cols;
    int kind;
    const void *data;
    const void *scale;
    size_t group_size;
} orc_qt;

/* Mirrors ExpertSlot / GateUp (expert_cache.rs:640-650). */
typedef struct {
    uint32_t eid;
    int fused;             /* 0: gate + up separate; 1: gate_up [2i, d] */
    orc_qt gate, up, gate_up, down;
} orc_slot;

/* --- quant.rs ------------------------------------------------------------------------------ */
float orc_e2m1_decode(uint8_t nibble);                                   /* quant.rs:353-356 */
float orc_e8m0_decode(uint8_t byte);                                     /* quant.rs:391-396 */
void orc_row_f32(const orc_qt *w, size_t row, float *out);               /* quant.rs:280-341 */
size_t orc_resident_bytes(const orc_qt *w);                              /* quant.rs:214-228 */

/* --- kernels.rs (scalar tiers: the parity oracle) ------------------------------------------ */
void orc_matmul(float *y, const float *x, const float *w, size_t s, size_t i, size_t o);
void orc_matmul_mxfp4_scalar(float *y, const float *x, const uint8_t *data, const uint8_t *block_scale,
                             size_t s, size_t i, size_t o);
void orc_matmul_i4_grouped(float *y, const float *x, const uint8_t *q4, const float *scale,
                           size_t group_size, size_t s, size_t i, size_t o);
/* matmul_qt with the scalar MXFP4 tier (simd=0) or the dispatching SIMD tier (simd=1). */
void orc_matmul_qt(float *y, const float *x, const orc_qt *w, size_t s, int simd);

/* --- kernels.rs SIMD tiers (CPU baseline; rabbit_oracle_simd.c) ----------------------------- */
int orc_cpu_has_avx512(void);
int orc_cpu_has_avx2(void);
void orc_matmul_mxfp4_avx2(float *y, const float *x, const uint8_t *data, const uint8_t *block_scale,
                           size_t s, size_t i, size_t o);
void orc_matmul_mxfp4_avx512(float *y, const float *x, const uint8_t *data, const uint8_t *block_scale,
                             size_t s, size_t i, size_t o);
/* kernels.rs:233-244: AVX-512F/BW > AVX2 > scalar. Returns the tier used (512, 2, 0). */
int orc_matmul_mxfp4(float *y, const float *x, const uint8_t *data, const uint8_t *block_scale,
                     size_t s, size_t i, size_t o);
void orc_set_threads(int n);
int orc_get_threads(void);

/* --- routers --------------------------------------------------------------------------------- */
/* qwen38::moe::route (qwen38/moe.rs:41-76) for one token. Returns k' = min(k, n). */
size_t orc_route_softmax(const float *logits, size_t n, size_t k, int32_t *ids, float *w);
/* glm52::moe::route for one token given its router logits (glm52/moe.rs:131-260):
 * sigmoid, choice = p + bias (bias may be NULL = 0), rank_top_grouped, normalize_and_scale. */
size_t orc_route_sigmoid(const float *logits, const float *bias, size_t n, size_t k, int norm_topk,
                         float routed_scale, size_t n_group, size_t topk_group, int32_t *ids, float *w);
/* unique_experts (glm52/moe.rs:333-344). ids is [s, k]; returns the count written to uniq. */
size_t orc_unique_experts(const int32_t *ids, size_t s, size_t k, int32_t *uniq);

float orc_siluf(float x);                                                /* glm52/moe.rs:33-35 */
float orc_sigmoid(float x);                                              /* kimi_linear/ops.rs:26-28 */

/* Activation::combine (glm52/moe.rs:58-70): silu(g) * u, or
 * (beta * tanh(g / beta)) * (1 / (1 + exp(-g))) * u' with u' = linear_beta * tanh(u / linear_beta)
 * when linear_beta is set (else u). */
float orc_act_combine(const orc_act *a, float g, float u);

/* apply_single_expert (glm52/moe.rs:463-513): accumulates into out[s, d]. _act: with an
 * activation (NULL = Silu). */
void orc_apply_single_expert(const orc_slot *slot, const int32_t *ids, const float *wts, size_t s,
                             size_t k, const float *x, size_t d, size_t i, int simd, float *out);
void orc_apply_single_expert_act(const orc_slot *slot, const int32_t *ids, const float *wts, size_t s,
                                 size_t k, const float *x, size_t d, size_t i, int simd, const orc_act *act,
                                 float *out);

/* One MoE layer's weights (router + shared expert), by family. */
typedef struct {
    int family;                 /* ORC_FAMILY_* */
    size_t hidden, moe_inter, n_experts, topk;
    const float *router;        /* f32 [n_experts, hidden] */
    const float *router_bias;   /* GLM/K3 post-sigmoid selection bias [n_experts] or NULL */
    const float *logit_bias;    /* synthetic pre-activation logit skew [n_experts] or NULL */
    int norm_topk;
    float routed_scale;
    size_t n_group, topk_group;
    int has_shared;
    orc_slot shared;            /* shared expert (eid ignored) */
    const float *shared_gate;   /* Qwen: f32 [hidden] sigmoid gate vector; NULL = ungated */
    const orc_slot *const *experts; /* experts[eid] (routed pool) */
} orc_moe_layer;

/* qwen38::generate::moe_forward (qwen38/generate.rs:262-351) and glm52::moe::moe
 * (glm52/moe.rs:350-451) with every expert resident. out[s, hidden] is overwritten.
 * ids_out / w_out (optional, [s, topk]) receive the routing. Returns 0, or -1 on a missing expert. */
int orc_moe_forward(const orc_moe_layer *L, const float *x, size_t s, int simd, float *out,
                    int32_t *ids_out, float *w_out);
/* Router logits plus optional synthetic skew, [s, n_experts] (generate.rs:279-281). */
void orc_router_logits(const orc_moe_layer *L, const float *x, size_t s, float *logits);

/* The layer's routing alone (the router half of moe_forward / moe): ids, w [s, min(topk, E)]. */
void orc_moe_route(const orc_moe_layer *L, const float *x, size_t s, int32_t *ids, float *w);

/* K3's latent MoE (kimi_k3/moe.rs:64-116): route x [s, hidden] with L's router at full width,
 * x_latent = matmul_qt(x, down_proj [moe_hidden, hidden]), every unique routed expert
 * (L->experts, shaped for moe_hidden) accumulated at moe_hidden with `act`, optional rmsnorm of
 * each summed row (norm [moe_hidden], eps), then out = matmul_qt(routed, up_proj [hidden,
 * moe_hidden]) (overwritten; no shared expert). Returns 0, or -1 on a missing expert. */
typedef struct {
    size_t moe_hidden;
    orc_qt down_proj, up_proj;
    const float *norm;     /* NULL: no norm */
    float eps;
    orc_act act;
} orc_latent;
int orc_latent_moe(const orc_moe_layer *L, const orc_latent *lw, const float *x, size_t s, int simd, float *out,
                   int32_t *ids_out, float *w_out);

/* --- norms and the MoE sublayer ----------------------------------------------------------- */
/* kimi_linear/ops.rs:46-53 rmsnorm, in place: r = 1 / sqrt((sum_f64(v^2) / n) as f32 + eps), then
 * v[i] *= r * w[i]. */
void orc_rmsnorm(float *v, const float *w, size_t n, float eps);
/* qwen38/ops.rs:25-33 rmsnorm_1p, in place: the same r, then v[i] *= r * (1 + w[i]). */
void orc_rmsnorm_1p(float *v, const float *w, size_t n, float eps);
/* The MoE half of a Qwen 3.8 decoder layer (qwen38/generate.rs:397-413): per token row,
 * nrm = rmsnorm_1p(x, post_ln), then x += moe_forward(nrm). x[s, hidden] is updated in place. */
int orc_moe_sublayer(const orc_moe_layer *L, float *x, size_t s, const float *post_ln, float eps, int simd,
                     int32_t *ids_out, float *w_out);

/* --- Qwen 3.8 token mixers (rabbit_oracle_mixers.c) ---------------------------------------- */
/* kimi_linear/short_conv.rs:58-85: out[c] = sum_t w[c,t] hist[c,t] + w[c,K-1] x[c], then the
 * per-channel history [d_inner, kernel - 1] shifts in x. weight is [d_inner, kernel]. */
void orc_short_conv_step(float *history, size_t d_inner, size_t kernel, const float *x, const float *weight,
                         float *out);
/* kimi_linear/kda.rs:65-76 (lower_bound None) for one scalar gate. */
float orc_gdn_alpha(float a_log, float a, float dt_bias);
/* kimi_linear/kda.rs:132-166 for one head with a broadcast alpha: s [d_k, d_v] updated, o [d_v]. */
void orc_kda_step(float *s, size_t d_k, size_t d_v, const float *q, const float *k, const float *v, float alpha,
                  float beta, float *o);
/* qwen38/gdn.rs:110-118 (q, k of one K head, in place) and :122-128 (one head's output gate). */
void orc_gdn_prepare_qk(float *q, float *k, size_t d_k);
void orc_gdn_output_gate(float *o, const float *norm_weight, const float *z, size_t d_v, float eps);
/* qwen38/gdn.rs:142-196: states [n_v, d_k, d_v] updated; qkv [2 key_dim + n_v d_v] is the
 * post-convolution row (SiLU applied in place); out [n_v d_v]. Returns -1 on a bad shape. */
int orc_gdn_step_token(float *states, size_t n_v, size_t d_k, size_t d_v, float *qkv, size_t key_dim,
                       const float *z, const float *a, const float *b, const float *a_log, const float *dt_bias,
                       const float *norm_weight, float eps, float *out);
/* qwen38/attention.rs:160-172, one head in place. */
void orc_rope_half(float *v, size_t rope_dim, size_t pos, float theta);
/* qwen38/attention.rs:190-217 over cache positions 0..positions-1 ([positions, n_kv, head_dim]). */
void orc_gqa_attend(const float *q, size_t n_heads, const float *k_cache, const float *v_cache, size_t positions,
                    size_t n_kv, size_t head_dim, float scale, float *out);
/* qwen38/generate.rs:226-255 between the projections: split q|gate per head, (1+w) RMSNorm of the q
 * and k heads, partial RoPE, push k / v at position pos, attend over positions 0..pos, sigmoid gate.
 * ctx [n_heads head_dim]. Returns -1 on a bad shape. */
int orc_gqa_step(const float *qg, const float *k_in, const float *v_in, size_t n_heads, size_t n_kv, size_t head_dim,
                 const float *q_norm, const float *k_norm, float eps, size_t rope_dim, float theta, float attn_scale,
                 float *k_cache, float *v_cache, size_t pos, float *ctx);

/* --- synthetic workload generator (shared bit-for-bit with rabbit_amd's device generator) --- */
uint64_t orc_synth_mix64(uint64_t z);
void orc_synth_mxfp4(uint8_t *data, uint8_t *scale, size_t rows, size_t cols, uint64_t seed,
                     uint32_t exp_lo, uint32_t exp_hi);
void orc_synth_i4g(uint8_t *data, float *scale, size_t rows, size_t cols, size_t gs, uint64_t seed,
                   float s_lo, float s_hi);

#ifdef __cplusplus
}
#endif
#endif
