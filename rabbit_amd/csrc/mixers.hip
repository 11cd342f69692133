// mixers.hip -- Qwen 3.8's token mixers for one decode token: Gated DeltaNet and GQA attention.
//
// The parts between the input and output projections (the projections are rbt_matmul_qt_d):
//
//   Gated DeltaNet (qwen38/generate.rs:196-219):
//     k_gdn_conv   the depthwise causal conv over q|k|v (kimi_linear/short_conv.rs:58-85) and its
//                  history shift, then SiLU (qwen38/gdn.rs:96-106); one thread per channel.
//     k_gdn_head   one workgroup per V head: its K head's q and k l2-normalised and q scaled
//                  (gdn.rs:110-118), the scalar decay and write strength (gdn.rs:76-87,
//                  kimi_linear/kda.rs:65-76), the delta-rule update of the head's [d_k, d_v] state
//                  and the readout o = S^T q (kimi_linear/kda.rs:132-166), then RMSNorm(o) * silu(z)
//                  (gdn.rs:122-128). The state stays in HBM between tokens; each workgroup reads and
//                  writes its head's once (64 KB each way at d_k = d_v = 128).
//   GQA attention (qwen38/generate.rs:226-255):
//     k_gqa_prep     per query head: the head's query slice of q_proj's per-head [query, gate] row
//                    (attention.rs:122-133), (1 + w) RMSNorm (attention.rs:138-143) and partial
//                    rotate-half RoPE (attention.rs:160-172); per KV head: the same for k, and k, v
//                    appended at position pos of the cache [cap, n_kv, head_dim] (attention.rs:76-82).
//     k_gqa_scores   per (KV head, chunk of 64 positions): the group's query heads' scores, each a
//                    sequential fp32 dot product over head_dim times the scale (attention.rs:203-206),
//                    and the chunk's softmax partials: max, sum of exp(s - max), exp-weighted V.
//     k_gqa_combine  per query head: the chunks merged (softmax over the whole cache,
//                    glm52/attention.rs:88-98, attention.rs:207-215), times sigmoid(gate)
//                    (attention.rs:221-226).
//
// Arithmetic: products and sums round on their own (-ffp-contract=off). Norm and softmax
// reductions that the reference runs sequentially run in a fixed parallel order here, so outputs
// agree with the reference to fp32 accumulation accuracy, not bit for bit. exp, log1p, pow, sin and
// cos are evaluated in fp64 and rounded to fp32, which gives the correctly rounded fp32 value the
// reference's libm calls return.
#include "rbt_device.h"
#include "rbt_internal.h"

namespace rbt {

__device__ __forceinline__ float mx_exp(float x) { return (float)exp((double)x); }
__device__ __forceinline__ float mx_silu(float x) { return __fdiv_rn(x, __fadd_rn(1.0f, mx_exp(-x))); }
__device__ __forceinline__ float mx_sigmoid(float x) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, mx_exp(-x))); }

// ---- Gated DeltaNet --------------------------------------------------------------------------
// hist [C, K - 1] oldest first, w [C, K]: y[c] = silu(sum_t w[c,t] hist[c,t] + w[c,K-1] x[c]).
__global__ __launch_bounds__(256) void k_gdn_conv(float *__restrict__ hist, const float *__restrict__ x,
                                                  const float *__restrict__ w, int C, int K, float *__restrict__ y) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const int hl = K - 1;
  float *h = hist + (long)c * hl;
  const float *wc = w + (long)c * K;
  const float xc = x[c];
  float acc = 0.0f;
  for (int t = 0; t < hl; t++) acc = __fadd_rn(acc, __fmul_rn(wc[t], h[t]));
  acc = __fadd_rn(acc, __fmul_rn(wc[hl], xc));
  for (int t = 0; t + 1 < hl; t++) h[t] = h[t + 1];
  if (hl > 0) h[hl - 1] = xc;
  y[c] = mx_silu(acc);
}

constexpr int GDN_MAXR = 64;  // state rows per thread held in registers

// One V head per workgroup of 256 threads. Thread t owns column j = t % d_v and rows
// i = g, g + G, ... (g = t / d_v, G = 256 / d_v); d_v divides 256 and d_k <= GDN_MAXR * G.
// act: the conv output after SiLU, [q (key_dim) | k (key_dim) | v (n_v d_v)].
__global__ __launch_bounds__(256) void k_gdn_head(float *__restrict__ states, const float *__restrict__ act,
                                                  int key_dim, int n_v, int n_k, int d_k, int d_v,
                                                  const float *__restrict__ z, const float *__restrict__ a,
                                                  const float *__restrict__ b, const float *__restrict__ a_log,
                                                  const float *__restrict__ dt_bias,
                                                  const float *__restrict__ norm_w, float eps,
                                                  float *__restrict__ out) {
  extern __shared__ float sm[];
  float *qs = sm, *ks = sm + d_k, *vs = sm + 2 * d_k, *part = sm + 2 * d_k + d_v;  // part [G][d_v]
  __shared__ float coef[4];
  const int h = blockIdx.x, t = threadIdx.x;
  const int kh = h / (n_v / n_k);  // key_head_of (gdn.rs:62-65)
  const int G = 256 / d_v, j = t % d_v, g = t / d_v;
  for (int i = t; i < d_k; i += 256) {
    qs[i] = act[kh * d_k + i];
    ks[i] = act[key_dim + kh * d_k + i];
  }
  for (int i = t; i < d_v; i += 256) vs[i] = act[2 * key_dim + h * d_v + i];
  __syncthreads();
  // prepare_qk (gdn.rs:110-118): l2_norm's sequential f32 sum of squares (kimi_linear/ops.rs:34-40)
  // for q on thread 0 and k on thread 64, the decay and write strength on thread 128
  if (t == 0 || t == 64) {
    float *v = t == 0 ? qs : ks;
    float ss = 0.0f;
    for (int i = 0; i < d_k; i++) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
    coef[t == 0 ? 0 : 1] = __fdiv_rn(1.0f, fmaxf(rbt_sqrt_rn(ss), 1e-6f));
  } else if (t == 128) {
    // alpha = exp(-exp(a_log) * softplus(a + dt_bias)), softplus(x) = max(x, 0) + ln_1p(exp(-|x|))
    const float x = __fadd_rn(a[h], dt_bias[h]);
    const float sp = __fadd_rn(fmaxf(x, 0.0f), (float)log1p((double)mx_exp(-fabsf(x))));
    coef[2] = mx_exp(__fmul_rn(-mx_exp(a_log[h]), sp));
    coef[3] = mx_sigmoid(b[h]);
  }
  __syncthreads();
  const float qscale = __fdiv_rn(1.0f, rbt_sqrt_rn((float)d_k));
  const float sq = coef[0], sk = coef[1], alpha = coef[2], beta = coef[3];
  // this thread's rows of the state, scaled by alpha (kda.rs:140-144)
  float *S = states + (long)h * d_k * d_v;
  const int nr = (d_k - g + G - 1) / G;
  float s[GDN_MAXR];
#pragma unroll
  for (int r = 0; r < GDN_MAXR; r++)
    if (r < nr) s[r] = __fmul_rn(S[(long)(g + G * r) * d_v + j], alpha);
  // c[j] = sum_i k_i S[i, j] (kda.rs:146-151)
  float c = 0.0f;
#pragma unroll
  for (int r = 0; r < GDN_MAXR; r++)
    if (r < nr) c = __fadd_rn(c, __fmul_rn(__fmul_rn(ks[g + G * r], sk), s[r]));
  part[g * d_v + j] = c;
  __syncthreads();
  float cj = 0.0f;
  for (int q = 0; q < G; q++) cj = __fadd_rn(cj, part[q * d_v + j]);
  __syncthreads();
  // S[i, j] += (beta k_i) (v_j - c_j) (kda.rs:153-158), then o[j] = sum_i q_i S[i, j] (:160-165)
  const float dv = __fsub_rn(vs[j], cj);
  float o = 0.0f;
#pragma unroll
  for (int r = 0; r < GDN_MAXR; r++)
    if (r < nr) {
      const int i = g + G * r;
      const float ki = __fmul_rn(ks[i], sk);
      s[r] = __fadd_rn(s[r], __fmul_rn(__fmul_rn(beta, ki), dv));
      S[(long)i * d_v + j] = s[r];
      o = __fadd_rn(o, __fmul_rn(__fmul_rn(__fmul_rn(qs[i], sq), qscale), s[r]));
    }
  part[g * d_v + j] = o;
  __syncthreads();
  if (t < d_v) {
    float oj = 0.0f;
    for (int q = 0; q < G; q++) oj = __fadd_rn(oj, part[q * d_v + t]);
    vs[t] = oj;
  }
  __syncthreads();
  // head_output_gate_silu (gdn.rs:122-128): rmsnorm (kimi_linear/ops.rs:46-53, the f64 sum of
  // squares in order) then * silu(z)
  if (t == 0) {
    double ms = 0.0;
    for (int i = 0; i < d_v; i++) ms += (double)vs[i] * (double)vs[i];
    coef[0] = __fdiv_rn(1.0f, rbt_sqrt_rn(__fadd_rn((float)(ms / (double)d_v), eps)));
  }
  __syncthreads();
  if (t < d_v) {
    const float r = coef[0];
    const float on = __fmul_rn(vs[t], __fmul_rn(r, norm_w[t]));
    out[(long)h * d_v + t] = __fmul_rn(on, mx_silu(z[(long)h * d_v + t]));
  }
}

// ---- GQA --------------------------------------------------------------------------------------
// (1 + w) RMSNorm of one head_dim-wide row in LDS (qwen38/ops.rs:25-33: f64 sum of squares in order)
// and the rotate-half RoPE of its first rope_dim entries (attention.rs:160-172), in place.
__device__ void gqa_norm_rope(float *v, const float *__restrict__ w, int hd, float eps, int rope_dim, int pos,
                              float theta, float *rs) {
  const int t = threadIdx.x;
  if (t == 0) {
    double ms = 0.0;
    for (int i = 0; i < hd; i++) ms += (double)v[i] * (double)v[i];
    rs[0] = __fdiv_rn(1.0f, rbt_sqrt_rn(__fadd_rn((float)(ms / (double)hd), eps)));
  }
  __syncthreads();
  const float r = rs[0];
  for (int i = t; i < hd; i += blockDim.x) v[i] = __fmul_rn(v[i], __fmul_rn(r, __fadd_rn(1.0f, w[i])));
  __syncthreads();
  const int half = rope_dim / 2;
  for (int jj = t; jj < half; jj += blockDim.x) {
    const float e = __fdiv_rn(__fmul_rn(-2.0f, (float)jj), (float)rope_dim);
    const float inv = (float)pow((double)theta, (double)e);
    const float ang = __fmul_rn((float)pos, inv);
    const float sn = (float)sin((double)ang), cs = (float)cos((double)ang);
    const float x0 = v[jj], x1 = v[jj + half];
    v[jj] = __fsub_rn(__fmul_rn(x0, cs), __fmul_rn(x1, sn));
    v[jj + half] = __fadd_rn(__fmul_rn(x1, cs), __fmul_rn(x0, sn));
  }
  __syncthreads();
}

// Workgroups [0, n_heads): query heads -> qp [n_heads, hd]; [n_heads, n_heads + n_kv): KV heads ->
// cache row pos. blockDim >= 64, hd <= 1024.
__global__ __launch_bounds__(256) void k_gqa_prep(const float *__restrict__ qg, const float *__restrict__ kin,
                                                  const float *__restrict__ vin, int n_heads, int n_kv, int hd,
                                                  const float *__restrict__ qn, const float *__restrict__ kn,
                                                  float eps, int rope_dim, int pos, float theta,
                                                  float *__restrict__ qp, float *__restrict__ kc,
                                                  float *__restrict__ vc) {
  extern __shared__ float row[];
  __shared__ float rs[1];
  const int b = blockIdx.x, t = threadIdx.x;
  const bool query = b < n_heads;
  const int kvh = b - n_heads;
  const float *src = query ? qg + (long)b * 2 * hd : kin + (long)kvh * hd;
  for (int i = t; i < hd; i += blockDim.x) row[i] = src[i];
  __syncthreads();
  gqa_norm_rope(row, query ? qn : kn, hd, eps, rope_dim, pos, theta, rs);
  const long kw = (long)n_kv * hd;
  if (query) {
    for (int i = t; i < hd; i += blockDim.x) qp[(long)b * hd + i] = row[i];
  } else {
    for (int i = t; i < hd; i += blockDim.x) {
      kc[(long)pos * kw + (long)kvh * hd + i] = row[i];
      vc[(long)pos * kw + (long)kvh * hd + i] = vin[(long)kvh * hd + i];
    }
  }
}

constexpr int GQA_CHUNK = 64;  // positions per scores workgroup

// grid (n_kv, chunks), 256 threads. The n_rep query heads of KV head kvh against positions
// [c * 64, min(P, c * 64 + 64)): scores into LDS (thread per (head, position), a sequential dot
// product), then per head m = max, l = sum exp(s - m), acc[d] = sum exp(s - m) v[d].
// part: [n_kv, chunks, n_rep, 2 + hd] = (m, l, acc).
__global__ __launch_bounds__(256) void k_gqa_scores(const float *__restrict__ qp, const float *__restrict__ kc,
                                                    const float *__restrict__ vc, int P, int n_heads, int n_kv, int hd,
                                                    float scale, float *__restrict__ part) {
  extern __shared__ float sm[];
  const int n_rep = n_heads / n_kv, kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x;
  const int p0 = ch * GQA_CHUNK, np = min(GQA_CHUNK, P - p0);
  float *qs = sm;                        // [n_rep, hd]
  float *sc = sm + n_rep * hd;           // [n_rep, GQA_CHUNK]
  float *st = sc + n_rep * GQA_CHUNK;    // [n_rep, 2]
  for (int i = t; i < n_rep * hd; i += 256) qs[i] = qp[(long)kvh * n_rep * hd + i];
  __syncthreads();
  const long kw = (long)n_kv * hd;
  for (int u = t; u < n_rep * np; u += 256) {
    const int r = u / np, p = u - r * np;
    const float *k = kc + (long)(p0 + p) * kw + (long)kvh * hd;
    const float *q = qs + r * hd;
    float dot = 0.0f;
    for (int d = 0; d < hd; d++) dot = __fadd_rn(dot, __fmul_rn(q[d], k[d]));
    sc[r * GQA_CHUNK + p] = __fmul_rn(dot, scale);
  }
  __syncthreads();
  if (t < n_rep) {
    float m = -1e30f;
    for (int p = 0; p < np; p++) m = fmaxf(m, sc[t * GQA_CHUNK + p]);
    float l = 0.0f;
    for (int p = 0; p < np; p++) {
      const float e = mx_exp(__fsub_rn(sc[t * GQA_CHUNK + p], m));
      sc[t * GQA_CHUNK + p] = e;
      l = __fadd_rn(l, e);
    }
    st[2 * t] = m;
    st[2 * t + 1] = l;
  }
  __syncthreads();
  const int nch = gridDim.y;
  for (int u = t; u < n_rep * hd; u += 256) {
    const int r = u / hd, d = u - r * hd;
    float acc = 0.0f;
    for (int p = 0; p < np; p++)
      acc = __fadd_rn(acc, __fmul_rn(sc[r * GQA_CHUNK + p], vc[(long)(p0 + p) * kw + (long)kvh * hd + d]));
    float *o = part + ((long)(kvh * nch + ch) * n_rep + r) * (2 + hd);
    o[2 + d] = acc;
    if (d == 0) {
      o[0] = st[2 * r];
      o[1] = st[2 * r + 1];
    }
  }
}

// One query head per workgroup: the chunks' partials merged, divided by the softmax sum, times
// sigmoid of the head's gate slice of q_proj's row.
__global__ __launch_bounds__(256) void k_gqa_combine(const float *__restrict__ part, const float *__restrict__ qg,
                                                     int n_heads, int n_kv, int hd, int nch,
                                                     float *__restrict__ ctx) {
  const int h = blockIdx.x, n_rep = n_heads / n_kv, kvh = h / n_rep, r = h - kvh * n_rep;
  auto P = [&](int c) { return part + ((long)(kvh * nch + c) * n_rep + r) * (2 + hd); };
  float M = -1e30f;
  for (int c = 0; c < nch; c++) M = fmaxf(M, P(c)[0]);
  float L = 0.0f;
  for (int c = 0; c < nch; c++) L = __fadd_rn(L, __fmul_rn(P(c)[1], mx_exp(__fsub_rn(P(c)[0], M))));
  for (int d = threadIdx.x; d < hd; d += blockDim.x) {
    float acc = 0.0f;
    for (int c = 0; c < nch; c++) acc = __fadd_rn(acc, __fmul_rn(P(c)[2 + d], mx_exp(__fsub_rn(P(c)[0], M))));
    const float g = qg[(long)h * 2 * hd + hd + d];
    ctx[(long)h * hd + d] = __fmul_rn(__fdiv_rn(acc, L), mx_sigmoid(g));
  }
}

// ---- launchers ----------------------------------------------------------------------------------
bool gdn_ok(int n_v, int n_k, int d_k, int d_v) {
  return n_v > 0 && n_k > 0 && n_v % n_k == 0 && d_v > 0 && d_v <= 256 && 256 % d_v == 0 && d_k > 0 &&
         d_k <= GDN_MAXR * (256 / d_v);
}

hipError_t launch_gdn(const Ctx &c, float *conv_hist, const float *conv_w, int K, float *states,
                      const float *qkv_pre, const float *z, const float *a, const float *b, const float *a_log,
                      const float *dt_bias, const float *norm_w, float eps, int n_v, int n_k, int d_k, int d_v,
                      float *act, float *out) {
  if (!gdn_ok(n_v, n_k, d_k, d_v) || K < 1) return hipErrorInvalidValue;
  const int key_dim = n_k * d_k, C = 2 * key_dim + n_v * d_v;
  launch_k(c, k_gdn_conv, dim3((C + 255) / 256), dim3(256), conv_hist, qkv_pre, conv_w, C, K, act);
  const unsigned lds = (unsigned)((2 * d_k + d_v + 256) * sizeof(float));
  launch_ks(c, k_gdn_head, dim3(n_v), dim3(256), lds, states, (const float *)act, key_dim, n_v, n_k, d_k, d_v, z, a,
            b, a_log, dt_bias, norm_w, eps, out);
  return hipGetLastError();
}

bool gqa_ok(int n_heads, int n_kv, int hd, int rope_dim) {
  return n_kv > 0 && n_heads % n_kv == 0 && hd > 0 && hd <= 1024 && rope_dim >= 0 && rope_dim % 2 == 0 &&
         rope_dim <= hd && (size_t)(n_heads / n_kv) * (hd + GQA_CHUNK + 2) * sizeof(float) <= 64 * 1024;
}

size_t gqa_part_floats(int n_heads, int n_kv, int hd, int positions) {
  const int nch = (positions + GQA_CHUNK - 1) / GQA_CHUNK;
  return (size_t)n_kv * nch * (n_heads / n_kv) * (2 + hd);
}

hipError_t launch_gqa(const Ctx &c, const float *qg, const float *k, const float *v, int n_heads, int n_kv, int hd,
                      const float *qn, const float *kn, float eps, int rope_dim, float theta, float scale, int pos,
                      float *kc, float *vc, float *qp, float *part, float *ctx) {
  if (!gqa_ok(n_heads, n_kv, hd, rope_dim) || pos < 0) return hipErrorInvalidValue;
  const int P = pos + 1, nch = (P + GQA_CHUNK - 1) / GQA_CHUNK, n_rep = n_heads / n_kv;
  launch_ks(c, k_gqa_prep, dim3(n_heads + n_kv), dim3(256), (unsigned)(hd * sizeof(float)), qg, k, v, n_heads, n_kv,
            hd, qn, kn, eps, rope_dim, pos, theta, qp, kc, vc);
  const unsigned lds = (unsigned)(n_rep * (hd + GQA_CHUNK + 2) * sizeof(float));
  launch_ks(c, k_gqa_scores, dim3(n_kv, nch), dim3(256), lds, (const float *)qp, (const float *)kc,
            (const float *)vc, P, n_heads, n_kv, hd, scale, part);
  launch_k(c, k_gqa_combine, dim3(n_heads), dim3(256), (const float *)part, qg, n_heads, n_kv, hd, nch, ctx);
  return hipGetLastError();
}

}  // namespace rbt
