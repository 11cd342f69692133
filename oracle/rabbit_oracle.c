/*
 * rabbit_oracle.c -- scalar CPU restatement of rabbit's routed-expert path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline; never part of the product path).
 * Compiled with -ffp-contract=off: every product and sum below is rounded on its own, in the
 * order the cited Rust code performs it.
 *
 * Parity pins (tests/test_oracle_golden.py): e2m1/e8m0 against the reference's KATs
 * (quant.rs:858-905, expert_cache.rs:1557-1566), matmul against kernels.rs:1323-1331, the MXFP4
 * two-block KAT (kernels.rs:1388-1406), the grouped-int4 two-group KAT (kernels.rs:1408-1428),
 * the router KATs (qwen38/moe.rs:115-182, glm52/moe.rs:920-961), the fused == separate KAT
 * (glm52/moe.rs:592-626), and exact fp64 brute force on small shapes.
 */
#include "rabbit_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static int g_threads = 0; /* 0 = OpenMP default */

void orc_set_threads(int n) { g_threads = n; }
int orc_get_threads(void) {
#ifdef _OPENMP
    return g_threads > 0 ? g_threads : omp_get_max_threads();
#else
    return 1;
#endif
}
int orc_nthreads_internal(void) { return orc_get_threads(); }

static size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }

/* quant.rs:348 E2M1_MAGNITUDES, quant.rs:353-356 e2m1_decode. */
static const float E2M1_MAG[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};

float orc_e2m1_decode(uint8_t nibble) {
    float mag = E2M1_MAG[nibble & 0x7];
    return (nibble & 0x8) ? -mag : mag;
}

/* quant.rs:391-396: byte 0 -> the subnormal 2^-127 (bits 1<<22); otherwise the byte is the f32
 * biased exponent field, so byte 255 gives +inf bits. */
float orc_e8m0_decode(uint8_t byte) {
    uint32_t bits = byte == 0 ? (1u << 22) : ((uint32_t)byte << 23);
    float f;
    memcpy(&f, &bits, sizeof f);
    return f;
}

/* QT::row_f32, quant.rs:280-341 (F32 :284, I4Grouped :312-324, MxFp4 :325-339). */
void orc_row_f32(const orc_qt *w, size_t row, float *out) {
    size_t cols = w->cols;
    if (w->kind == ORC_QT_F32) {
        memcpy(out, (const float *)w->data + row * cols, cols * sizeof(float));
        return;
    }
    size_t rb = div_ceil(cols, 2);
    const uint8_t *wr = (const uint8_t *)w->data + row * rb;
    if (w->kind == ORC_QT_I4_GROUPED) {
        size_t ng = div_ceil(cols, w->group_size);
        const float *srow = (const float *)w->scale + row * ng;
        for (size_t k = 0; k < cols; k++) {
            uint8_t byte = wr[k >> 1];
            uint8_t nib = (k & 1) == 0 ? (byte & 0xF) : (byte >> 4);
            out[k] = (float)((int)nib - 8) * srow[k / w->group_size];
        }
        return;
    }
    size_t bpr = div_ceil(cols, 32);
    const uint8_t *bsr = (const uint8_t *)w->scale + row * bpr;
    for (size_t k = 0; k < cols; k++) {
        uint8_t byte = wr[k >> 1];
        uint8_t nib = (k & 1) == 0 ? (byte & 0xF) : (byte >> 4);
        out[k] = orc_e2m1_decode(nib) * orc_e8m0_decode(bsr[k / 32]);
    }
}

/* QT::resident_bytes, quant.rs:214-228. */
size_t orc_resident_bytes(const orc_qt *w) {
    switch (w->kind) {
    case ORC_QT_F32: return w->rows * w->cols * 4;
    case ORC_QT_I4_GROUPED:
        return w->rows * div_ceil(w->cols, 2) + w->rows * div_ceil(w->cols, w->group_size) * 4;
    default: return w->rows * div_ceil(w->cols, 2) + w->rows * div_ceil(w->cols, 32);
    }
}

/* kernels.rs:113-124 matmul: y[s,o] = sum_k x[s,k]*w[o,k], a left-to-right fold of rounded
 * products (Iterator::sum). Modern Rust's f32 Sum starts the fold at -0.0, which only differs
 * from +0.0 when every product is -0.0. Rows are independent, so the row-parallel loop gives
 * the same bits as rayon's par_chunks_mut. */
void orc_matmul(float *y, const float *x, const float *w, size_t s, size_t i, size_t o) {
#pragma omp parallel for schedule(static) num_threads(orc_nthreads_internal())
    for (long oi = 0; oi < (long)o; oi++) {
        const float *wr = w + (size_t)oi * i;
        for (size_t si = 0; si < s; si++) {
            const float *xs = x + si * i;
            float a = -0.0f;
            for (size_t k = 0; k < i; k++) a += xs[k] * wr[k];
            y[si * o + (size_t)oi] = a;
        }
    }
}

/* kernels.rs:247-267 matmul_mxfp4_scalar: a += (x[k] * e2m1(n)) * e8m0(s[k/32]). */
void orc_matmul_mxfp4_scalar(float *y, const float *x, const uint8_t *data, const uint8_t *block_scale,
                             size_t s, size_t i, size_t o) {
    size_t rb = div_ceil(i, 2), bpr = div_ceil(i, 32);
#pragma omp parallel for schedule(static) num_threads(orc_nthreads_internal())
    for (long oi = 0; oi < (long)o; oi++) {
        const uint8_t *w = data + (size_t)oi * rb;
        const uint8_t *bs = block_scale + (size_t)oi * bpr;
        for (size_t si = 0; si < s; si++) {
            const float *xs = x + si * i;
            float a = 0.0f;
            for (size_t k = 0; k < i; k++) {
                uint8_t byte = w[k >> 1];
                uint8_t nib = (k & 1) == 0 ? (byte & 0xF) : (byte >> 4);
                a += xs[k] * orc_e2m1_decode(nib) * orc_e8m0_decode(bs[k / 32]);
            }
            y[si * o + (size_t)oi] = a;
        }
    }
}

/* kernels.rs:276-296 matmul_i4_grouped: a += (x[k] * f32(n-8)) * scale[row, k/gs]. */
void orc_matmul_i4_grouped(float *y, const float *x, const uint8_t *q4, const float *scale,
                           size_t group_size, size_t s, size_t i, size_t o) {
    size_t rb = div_ceil(i, 2), ng = div_ceil(i, group_size);
#pragma omp parallel for schedule(static) num_threads(orc_nthreads_internal())
    for (long oi = 0; oi < (long)o; oi++) {
        const uint8_t *w = q4 + (size_t)oi * rb;
        const float *sc = scale + (size_t)oi * ng;
        for (size_t si = 0; si < s; si++) {
            const float *xs = x + si * i;
            float a = 0.0f;
            for (size_t k = 0; k < i; k++) {
                uint8_t byte = w[k >> 1];
                uint8_t nib = (k & 1) == 0 ? (byte & 0xF) : (byte >> 4);
                a += xs[k] * (float)((int)nib - 8) * sc[k / group_size];
            }
            y[si * o + (size_t)oi] = a;
        }
    }
}

/* kernels.rs:1104-1123 matmul_qt, restricted to the formats on this path. */
void orc_matmul_qt(float *y, const float *x, const orc_qt *w, size_t s, int simd) {
    switch (w->kind) {
    case ORC_QT_F32: orc_matmul(y, x, (const float *)w->data, s, w->cols, w->rows); break;
    case ORC_QT_I4_GROUPED:
        orc_matmul_i4_grouped(y, x, (const uint8_t *)w->data, (const float *)w->scale, w->group_size, s,
                              w->cols, w->rows);
        break;
    default:
        if (simd)
            orc_matmul_mxfp4(y, x, (const uint8_t *)w->data, (const uint8_t *)w->scale, s, w->cols, w->rows);
        else
            orc_matmul_mxfp4_scalar(y, x, (const uint8_t *)w->data, (const uint8_t *)w->scale, s, w->cols,
                                    w->rows);
    }
}

/* ----------------------------------------------------------------------------------------------
 * Routers
 * -------------------------------------------------------------------------------------------- */

/* qwen38/moe.rs:41-76: running top-k by logit (strict > keeps the lower id first on ties), then a
 * max-subtracted softmax over the k winners, in selection order. */
size_t orc_route_softmax(const float *logits, size_t n, size_t k, int32_t *ids, float *w) {
    if (k > n) k = n;
    if (k == 0) return 0;
    size_t len = 0;
    for (size_t id = 0; id < n; id++) {
        float l = logits[id];
        size_t pos = len;
        for (size_t p = 0; p < len; p++) {
            if (l > w[p]) { pos = p; break; }
        }
        if (pos == len) {
            if (len < k) { ids[len] = (int32_t)id; w[len] = l; len++; }
            continue;
        }
        size_t last = len < k ? len : k - 1; /* drop the tail when full (top.pop()) */
        for (size_t q = last; q > pos; q--) { ids[q] = ids[q - 1]; w[q] = w[q - 1]; }
        ids[pos] = (int32_t)id;
        w[pos] = l;
        if (len < k) len++;
    }
    float mx = w[0], sum = 0.0f;
    for (size_t p = 0; p < len; p++) {
        w[p] = expf(w[p] - mx);
        sum += w[p];
    }
    for (size_t p = 0; p < len; p++) w[p] /= sum;
    return len;
}

/* glm52/moe.rs:148-168 rank_top / :172-189 rank_top_within: repeated strict-> scans from
 * bv = -1e30 over the not-yet-taken (and allowed) experts; the stored value is the plain
 * sigmoid, not the biased choice. */
static size_t rank_top_within(const float *choice, const float *p, size_t n, size_t k, const unsigned char *allowed,
                              int32_t *ids, float *w) {
    unsigned char *taken = (unsigned char *)calloc(n, 1);
    size_t cnt = 0;
    if (allowed) {
        size_t na = 0;
        for (size_t e = 0; e < n; e++) na += allowed[e] ? 1 : 0;
        if (k > na) k = na;
    } else if (k > n) {
        k = n;
    }
    for (size_t t = 0; t < k; t++) {
        long best = -1;
        float bv = -1e30f;
        for (size_t e = 0; e < n; e++) {
            if (!taken[e] && (!allowed || allowed[e]) && choice[e] > bv) { bv = choice[e]; best = (long)e; }
        }
        if (best < 0) break;
        taken[best] = 1;
        ids[cnt] = (int32_t)best;
        w[cnt] = p[best];
        cnt++;
    }
    free(taken);
    return cnt;
}

/* glm52/moe.rs:194-208 top2_sum. */
static float top2_sum(const float *v, size_t n) {
    float t1 = -INFINITY, t2 = -INFINITY;
    for (size_t e = 0; e < n; e++) {
        if (v[e] > t1) { t2 = t1; t1 = v[e]; }
        else if (v[e] > t2) { t2 = v[e]; }
    }
    return isfinite(t2) ? t1 + t2 : t1;
}

/* glm52/moe.rs:131-260: router_scores (sigmoid, choice = p + bias), rank_top_grouped,
 * normalize_and_scale. */
size_t orc_route_sigmoid(const float *logits, const float *bias, size_t n, size_t k, int norm_topk,
                         float routed_scale, size_t n_group, size_t topk_group, int32_t *ids, float *w) {
    float *p = (float *)malloc(n * sizeof(float));
    float *choice = (float *)malloc(n * sizeof(float));
    for (size_t e = 0; e < n; e++) {
        p[e] = 1.0f / (1.0f + expf(-logits[e]));
        choice[e] = p[e] + (bias ? bias[e] : 0.0f);
    }
    size_t cnt;
    if (n_group <= 1) {
        cnt = rank_top_within(choice, p, n, k, NULL, ids, w);
    } else {
        size_t gsz = n / n_group;
        float *gscore = (float *)malloc(n_group * sizeof(float));
        size_t *order = (size_t *)malloc(n_group * sizeof(size_t));
        for (size_t g = 0; g < n_group; g++) { gscore[g] = top2_sum(choice + g * gsz, gsz); order[g] = g; }
        /* sort by score desc, group index asc (glm52/moe.rs:221) */
        for (size_t a = 1; a < n_group; a++) {
            size_t cur = order[a], b = a;
            while (b > 0 && (gscore[order[b - 1]] < gscore[cur] ||
                             (gscore[order[b - 1]] == gscore[cur] && order[b - 1] > cur))) {
                order[b] = order[b - 1];
                b--;
            }
            order[b] = cur;
        }
        unsigned char *allowed = (unsigned char *)calloc(n, 1);
        for (size_t t = 0; t < topk_group && t < n_group; t++)
            for (size_t e = 0; e < gsz; e++) allowed[order[t] * gsz + e] = 1;
        cnt = rank_top_within(choice, p, n, k, allowed, ids, w);
        free(allowed);
        free(order);
        free(gscore);
    }
    if (norm_topk) {
        float sum = -0.0f;
        for (size_t t = 0; t < cnt; t++) sum += w[t];
        sum += 1e-20f;
        for (size_t t = 0; t < cnt; t++) w[t] /= sum;
    }
    for (size_t t = 0; t < cnt; t++) w[t] *= routed_scale;
    free(choice);
    free(p);
    return cnt;
}

/* glm52/moe.rs:333-344 unique_experts: first-occurrence order over tokens, then slots. */
size_t orc_unique_experts(const int32_t *ids, size_t s, size_t k, int32_t *uniq) {
    size_t cnt = 0;
    for (size_t t = 0; t < s * k; t++) {
        int seen = 0;
        for (size_t u = 0; u < cnt; u++) if (uniq[u] == ids[t]) { seen = 1; break; }
        if (!seen) uniq[cnt++] = ids[t];
    }
    return cnt;
}

float orc_siluf(float x) { return x / (1.0f + expf(-x)); }
float orc_sigmoid(float x) { return 1.0f / (1.0f + expf(-x)); }

/* glm52/moe.rs:58-70 Activation::combine */
float orc_act_combine(const orc_act *a, float g, float u) {
    if (!a || a->kind == ORC_ACT_SILU) return orc_siluf(g) * u;
    if (a->has_linear_beta) u = a->linear_beta * tanhf(u / a->linear_beta);
    const float situ = a->beta * tanhf(g / a->beta) * (1.0f / (1.0f + expf(-g)));
    return situ * u;
}

void orc_apply_single_expert(const orc_slot *slot, const int32_t *ids, const float *wts, size_t s,
                             size_t k, const float *x, size_t d, size_t i, int simd, float *out) {
    orc_apply_single_expert_act(slot, ids, wts, s, k, x, d, i, simd, NULL, out);
}

/* glm52/moe.rs:463-513 apply_single_expert */
void orc_apply_single_expert_act(const orc_slot *slot, const int32_t *ids, const float *wts, size_t s,
                                 size_t k, const float *x, size_t d, size_t i, int simd, const orc_act *act,
                                 float *out) {
    size_t *rows = (size_t *)malloc((s ? s : 1) * sizeof(size_t));
    float *rw = (float *)malloc((s ? s : 1) * sizeof(float));
    size_t nr = 0;
    for (size_t si = 0; si < s; si++) {
        for (size_t t = 0; t < k; t++) {
            if (ids[si * k + t] == (int32_t)slot->eid) { rows[nr] = si; rw[nr] = wts[si * k + t]; nr++; break; }
        }
    }
    if (nr == 0) { free(rows); free(rw); return; }
    float *xg = (float *)malloc(nr * d * sizeof(float));
    for (size_t r = 0; r < nr; r++) memcpy(xg + r * d, x + rows[r] * d, d * sizeof(float));
    float *gg = (float *)malloc(nr * i * sizeof(float));
    if (!slot->fused) {
        float *uu = (float *)malloc(nr * i * sizeof(float));
        orc_matmul_qt(gg, xg, &slot->gate, nr, simd);
        orc_matmul_qt(uu, xg, &slot->up, nr, simd);
        for (size_t z = 0; z < nr * i; z++) gg[z] = orc_act_combine(act, gg[z], uu[z]);
        free(uu);
    } else {
        float *gu = (float *)malloc(nr * 2 * i * sizeof(float));
        orc_matmul_qt(gu, xg, &slot->gate_up, nr, simd);
        for (size_t r = 0; r < nr; r++)
            for (size_t c = 0; c < i; c++) gg[r * i + c] = orc_act_combine(act, gu[r * 2 * i + c], gu[r * 2 * i + i + c]);
        free(gu);
    }
    float *hh = (float *)malloc(nr * d * sizeof(float));
    orc_matmul_qt(hh, gg, &slot->down, nr, simd);
    for (size_t r = 0; r < nr; r++)
        for (size_t dd = 0; dd < d; dd++) out[rows[r] * d + dd] += rw[r] * hh[r * d + dd];
    free(hh);
    free(gg);
    free(xg);
    free(rw);
    free(rows);
}

/* kimi_linear/ops.rs:46-53: the f64 sum of squares in element order, (ms / n) rounded to f32. */
static float orc_rms_scale(const float *v, size_t n, float eps) {
    double ms = 0.0;
    for (size_t i = 0; i < n; i++) ms += (double)v[i] * (double)v[i];
    return 1.0f / sqrtf((float)(ms / (double)n) + eps);
}

void orc_rmsnorm(float *v, const float *w, size_t n, float eps) {
    const float r = orc_rms_scale(v, n, eps);
    for (size_t i = 0; i < n; i++) v[i] *= r * w[i];
}

/* qwen38/ops.rs:25-33 */
void orc_rmsnorm_1p(float *v, const float *w, size_t n, float eps) {
    const float r = orc_rms_scale(v, n, eps);
    for (size_t i = 0; i < n; i++) v[i] *= r * (1.0f + w[i]);
}

/* qwen38/generate.rs:397-413: nrm = rmsnorm_1p(x) row by row, tmp = moe_forward(nrm), x += tmp. */
int orc_moe_sublayer(const orc_moe_layer *L, float *x, size_t s, const float *post_ln, float eps, int simd,
                     int32_t *ids_out, float *w_out) {
    const size_t d = L->hidden;
    float *nrm = (float *)malloc((s ? s : 1) * d * sizeof(float));
    float *tmp = (float *)malloc((s ? s : 1) * d * sizeof(float));
    memcpy(nrm, x, s * d * sizeof(float));
    for (size_t si = 0; si < s; si++) orc_rmsnorm_1p(nrm + si * d, post_ln, d, eps);
    const int rc = orc_moe_forward(L, nrm, s, simd, tmp, ids_out, w_out);
    if (rc == 0)
        for (size_t z = 0; z < s * d; z++) x[z] += tmp[z];
    free(tmp);
    free(nrm);
    return rc;
}

/* qwen38/generate.rs:279-281 (router matmul) plus the synthetic pre-activation skew. */
void orc_router_logits(const orc_moe_layer *L, const float *x, size_t s, float *logits) {
    orc_matmul(logits, x, L->router, s, L->hidden, L->n_experts);
    if (L->logit_bias)
        for (size_t si = 0; si < s; si++)
            for (size_t e = 0; e < L->n_experts; e++) logits[si * L->n_experts + e] += L->logit_bias[e];
}

/* qwen38/generate.rs:262-351 (Qwen: softmax router, sigmoid-gated shared expert) and
 * glm52/moe.rs:350-451 (GLM/K3: sigmoid router, ungated shared expert). Every routed expert is
 * resident, so experts are applied in unique_experts order and the shared expert is added last. */
/* qwen38/generate.rs:279-287 / glm52/moe.rs:365-376: router logits, then the family's route. */
void orc_moe_route(const orc_moe_layer *L, const float *x, size_t s, int32_t *ids, float *wts) {
    size_t E = L->n_experts, k = L->topk;
    if (k > E) k = E;
    float *logits = (float *)malloc((s ? s : 1) * E * sizeof(float));
    orc_router_logits(L, x, s, logits);
    for (size_t si = 0; si < s; si++) {
        if (L->family == ORC_FAMILY_QWEN38)
            orc_route_softmax(logits + si * E, E, k, ids + si * k, wts + si * k);
        else
            orc_route_sigmoid(logits + si * E, L->router_bias, E, k, L->norm_topk, L->routed_scale,
                              L->n_group, L->topk_group, ids + si * k, wts + si * k);
    }
    free(logits);
}

/* kimi_k3/moe.rs:64-116 latent_moe */
int orc_latent_moe(const orc_moe_layer *L, const orc_latent *lw, const float *x, size_t s, int simd, float *out,
                   int32_t *ids_out, float *w_out) {
    const size_t mh = lw->moe_hidden, i = L->moe_inter, E = L->n_experts;
    size_t k = L->topk;
    if (k > E) k = E;
    int32_t *ids = (int32_t *)malloc((s ? s : 1) * (k ? k : 1) * sizeof(int32_t));
    float *wts = (float *)malloc((s ? s : 1) * (k ? k : 1) * sizeof(float));
    orc_moe_route(L, x, s, ids, wts);
    if (ids_out) memcpy(ids_out, ids, s * k * sizeof(int32_t));
    if (w_out) memcpy(w_out, wts, s * k * sizeof(float));
    float *xl = (float *)malloc((s ? s : 1) * mh * sizeof(float));
    float *routed = (float *)calloc((s ? s : 1) * mh, sizeof(float));
    orc_matmul_qt(xl, x, &lw->down_proj, s, simd);
    int32_t *uniq = (int32_t *)malloc((s ? s : 1) * (k ? k : 1) * sizeof(int32_t));
    const size_t nu = orc_unique_experts(ids, s, k, uniq);
    int rc = 0;
    for (size_t u = 0; u < nu; u++) {
        const orc_slot *slot = L->experts[uniq[u]];
        if (!slot) { rc = -1; break; }
        orc_apply_single_expert_act(slot, ids, wts, s, k, xl, mh, i, simd, &lw->act, routed);
    }
    if (lw->norm)
        for (size_t si = 0; si < s; si++) orc_rmsnorm(routed + si * mh, lw->norm, mh, lw->eps);
    orc_matmul_qt(out, routed, &lw->up_proj, s, simd);
    free(uniq);
    free(routed);
    free(xl);
    free(wts);
    free(ids);
    return rc;
}

int orc_moe_forward(const orc_moe_layer *L, const float *x, size_t s, int simd, float *out,
                    int32_t *ids_out, float *w_out) {
    size_t d = L->hidden, i = L->moe_inter, E = L->n_experts, k = L->topk;
    if (k > E) k = E;
    int32_t *ids = (int32_t *)malloc((s ? s : 1) * (k ? k : 1) * sizeof(int32_t));
    float *wts = (float *)malloc((s ? s : 1) * (k ? k : 1) * sizeof(float));
    orc_moe_route(L, x, s, ids, wts);
    if (ids_out) memcpy(ids_out, ids, s * k * sizeof(int32_t));
    if (w_out) memcpy(w_out, wts, s * k * sizeof(float));
    memset(out, 0, s * d * sizeof(float));

    float *shared = NULL;
    if (L->has_shared) {
        size_t si_ = L->shared.fused ? L->shared.gate_up.rows / 2 : L->shared.gate.rows;
        float *sg = (float *)malloc(s * si_ * sizeof(float));
        shared = (float *)malloc(s * d * sizeof(float));
        if (!L->shared.fused) {
            float *su = (float *)malloc(s * si_ * sizeof(float));
            orc_matmul_qt(sg, x, &L->shared.gate, s, simd);
            orc_matmul_qt(su, x, &L->shared.up, s, simd);
            for (size_t z = 0; z < s * si_; z++) sg[z] = orc_siluf(sg[z]) * su[z];
            free(su);
        } else {
            float *gu = (float *)malloc(s * 2 * si_ * sizeof(float));
            orc_matmul_qt(gu, x, &L->shared.gate_up, s, simd);
            for (size_t r = 0; r < s; r++)
                for (size_t c = 0; c < si_; c++)
                    sg[r * si_ + c] = orc_siluf(gu[r * 2 * si_ + c]) * gu[r * 2 * si_ + si_ + c];
            free(gu);
        }
        orc_matmul_qt(shared, sg, &L->shared.down, s, simd);
        free(sg);
        if (L->shared_gate) {
            for (size_t si = 0; si < s; si++) {
                float lg = -0.0f;
                for (size_t c = 0; c < d; c++) lg += x[si * d + c] * L->shared_gate[c];
                float sc = orc_sigmoid(lg);
                for (size_t c = 0; c < d; c++) shared[si * d + c] *= sc;
            }
        }
    }

    int32_t *uniq = (int32_t *)malloc((s ? s : 1) * (k ? k : 1) * sizeof(int32_t));
    size_t nu = orc_unique_experts(ids, s, k, uniq);
    int rc = 0;
    for (size_t u = 0; u < nu; u++) {
        const orc_slot *slot = L->experts[uniq[u]];
        if (!slot) { rc = -1; break; }
        orc_apply_single_expert(slot, ids, wts, s, k, x, d, i, simd, out);
    }
    if (shared) {
        for (size_t z = 0; z < s * d; z++) out[z] += shared[z];
        free(shared);
    }
    free(uniq);
    free(wts);
    free(ids);
    return rc;
}

/* ----------------------------------------------------------------------------------------------
 * Synthetic workload generator. Counter-based (splitmix64 finaliser over an index), so any byte
 * of any tensor can be regenerated independently; rabbit_amd's device generator produces the
 * same bytes. Data: byte j of 8-byte word w is bits [8j, 8j+8) of mix64(seed_d + w), so every
 * nibble is uniform over 0..15. MXFP4 scale byte idx: exp_lo + floor(hi32(mix64(seed_s + idx)) *
 * (exp_hi - exp_lo + 1) / 2^32). I4G scale idx: s_lo + (s_hi - s_lo) * u with u the top 24 bits
 * of mix64(seed_s + idx) times 2^-24, each operation rounded separately.
 * -------------------------------------------------------------------------------------------- */
uint64_t orc_synth_mix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void synth_bytes(uint8_t *data, size_t nbytes, uint64_t seed_d) {
#pragma omp parallel for schedule(static) num_threads(orc_nthreads_internal())
    for (long w = 0; w < (long)((nbytes + 7) / 8); w++) {
        uint64_t h = orc_synth_mix64(seed_d + (uint64_t)w);
        for (size_t j = 0; j < 8; j++) {
            size_t b = (size_t)w * 8 + j;
            if (b < nbytes) data[b] = (uint8_t)(h >> (8 * j));
        }
    }
}

void orc_synth_mxfp4(uint8_t *data, uint8_t *scale, size_t rows, size_t cols, uint64_t seed,
                     uint32_t exp_lo, uint32_t exp_hi) {
    uint64_t seed_d = orc_synth_mix64(seed * 2 + 1), seed_s = orc_synth_mix64(seed * 2 + 2);
    synth_bytes(data, rows * div_ceil(cols, 2), seed_d);
    size_t ns = rows * div_ceil(cols, 32);
    uint64_t span = (uint64_t)(exp_hi - exp_lo + 1);
#pragma omp parallel for schedule(static) num_threads(orc_nthreads_internal())
    for (long idx = 0; idx < (long)ns; idx++) {
        uint64_t h = orc_synth_mix64(seed_s + (uint64_t)idx);
        scale[idx] = (uint8_t)(exp_lo + (((h >> 32) * span) >> 32));
    }
}

void orc_synth_i4g(uint8_t *data, float *scale, size_t rows, size_t cols, size_t gs, uint64_t seed,
                   float s_lo, float s_hi) {
    uint64_t seed_d = orc_synth_mix64(seed * 2 + 1), seed_s = orc_synth_mix64(seed * 2 + 2);
    synth_bytes(data, rows * div_ceil(cols, 2), seed_d);
    size_t ns = rows * div_ceil(cols, gs);
    float span = s_hi - s_lo;
#pragma omp parallel for schedule(static) num_threads(orc_nthreads_internal())
    for (long idx = 0; idx < (long)ns; idx++) {
        uint64_t h = orc_synth_mix64(seed_s + (uint64_t)idx);
        float u = (float)(uint32_t)(h >> 40) * 0x1p-24f;
        float t = span * u;
        scale[idx] = s_lo + t;
    }
}
