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
//     k_gqa_chunk    per (KV head, chunk of 64 positions), on the matrix cores: the group's query
//                    heads' scores q . k times the scale (attention.rs:203-206) and the chunk's softmax
//                    partials: max, sum of exp(s - max), exp-weighted V (each K and V row read once).
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
// KT: the kernel size when it is known at compile time (its loads then all go out together, one
// wait), 0 for any K.
template <int KT>
__global__ __launch_bounds__(256) void k_gdn_conv(float *__restrict__ hist, const float *__restrict__ x,
                                                  const float *__restrict__ w, int C, int K, float *__restrict__ y) {
  const int c = blockIdx.x * 256 + threadIdx.x;
  if (c >= C) return;
  const int hl = (KT > 0 ? KT : K) - 1;
  float *h = hist + (long)c * hl;
  const float *wc = w + (long)c * (hl + 1);
  float acc = 0.0f;
  if constexpr (KT > 0) {
    float wv[KT], hv[KT > 1 ? KT - 1 : 1];
#pragma unroll
    for (int t = 0; t < KT; t++) wv[t] = wc[t];
#pragma unroll
    for (int t = 0; t < KT - 1; t++) hv[t] = h[t];
    const float xc = x[c];
#pragma unroll
    for (int t = 0; t < KT - 1; t++) acc = __fadd_rn(acc, __fmul_rn(wv[t], hv[t]));
    acc = __fadd_rn(acc, __fmul_rn(wv[KT - 1], xc));
#pragma unroll
    for (int t = 0; t + 1 < KT - 1; t++) h[t] = hv[t + 1];
    if (KT > 1) h[KT - 2] = xc;
    y[c] = mx_silu(acc);
  } else {
    const float xc = x[c];
    for (int t = 0; t < hl; t++) acc = __fadd_rn(acc, __fmul_rn(wc[t], h[t]));
    acc = __fadd_rn(acc, __fmul_rn(wc[hl], xc));
    for (int t = 0; t + 1 < hl; t++) h[t] = h[t + 1];
    if (hl > 0) h[hl - 1] = xc;
    y[c] = mx_silu(acc);
  }
}

constexpr int GDN_NT = 512;   // threads per head workgroup
constexpr int GDN_MAXR = 16;  // state rows per thread held in registers (float4 each)

// One V head per workgroup of GDN_NT threads. Thread t owns the four columns 4 jq .. 4 jq + 3
// (jq = t % (d_v / 4)) of rows i = g, g + G, ... (g = t / (d_v / 4), G = GDN_NT / (d_v / 4)); d_v is a
// multiple of 4 with d_v / 4 dividing GDN_NT and d_v <= GDN_NT, d_k is even and d_k <= GDN_MAXR G.
// q, k, v, z and the norm weight are requested first, then the head's state rows; the norms and gates
// are prepared while the state arrives (loads complete in order, so those issued after the state
// rows would wait for them).
// NR > 0: every thread holds exactly NR rows (d_k = NR G), and the row loads are unconditional, so the
// compiler's waits for the loads issued before them do not also wait for them.
// act: the conv output after SiLU, [q (key_dim) | k (key_dim) | v (n_v d_v)].
template <int NR>
__global__ __launch_bounds__(GDN_NT) void k_gdn_head(float *__restrict__ states, const float *__restrict__ act,
                                                     int key_dim, int n_v, int n_k, int d_k, int d_v,
                                                     const float *__restrict__ z, const float *__restrict__ a,
                                                     const float *__restrict__ b, const float *__restrict__ a_log,
                                                     const float *__restrict__ dt_bias,
                                                     const float *__restrict__ norm_w, float eps,
                                                     float *__restrict__ out) {
  extern __shared__ float sm[];
  const int QN = d_v / 4, G = GDN_NT / QN;
  float *qs = sm, *ks = sm + d_k, *vs = sm + 2 * d_k, *part = sm + 2 * d_k + d_v;  // part [G][d_v]
  __shared__ float coef[4];
  const int h = blockIdx.x, t = threadIdx.x;
  const int kh = h / (n_v / n_k);  // key_head_of (gdn.rs:62-65)
  const int jq = t % QN, g = t / QN;
  constexpr int MR = NR > 0 ? NR : GDN_MAXR;
  const int nr = NR > 0 ? NR : g < d_k ? (d_k - g + G - 1) / G : 0;
  // (clamped indices rather than branches, so that nothing here waits for the state rows)
  const int ti = min(t, d_k - 1), tj = min(t, d_v - 1);
  const float q0 = act[kh * d_k + ti], k0 = act[key_dim + kh * d_k + ti], v0 = act[2 * key_dim + h * d_v + tj];
  const float zj = z[(long)h * d_v + tj], nwj = norm_w[tj];
  const float ah = a[h], dth = dt_bias[h], alh = a_log[h], bh = b[h];
  __builtin_amdgcn_sched_barrier(0);  // the state rows are requested only now
  // this thread's rows: Sp[r * rs] is S[g + G r][4 jq .. 4 jq + 3] (32-bit offsets: the head's state
  // is d_k d_v < 2^31 floats)
  float4 *Sp = reinterpret_cast<float4 *>(states + (long)h * d_k * d_v) + g * QN + jq;
  const int rs = G * QN;
  float4 s[MR];
#pragma unroll
  for (int r = 0; r < MR; r++)
    if (NR > 0 || r < nr) s[r] = Sp[r * rs];
  // the values loaded first are taken here, before anything could move their loads after the rows'
  // (threads past d_k or d_v store the same value as the last one)
  float zv = zj, nw = nwj;
  asm volatile("" : "+v"(zv), "+v"(nw));
  qs[ti] = q0;
  ks[ti] = k0;
  vs[tj] = v0;
  for (int i = t + GDN_NT; i < d_k; i += GDN_NT) {
    qs[i] = act[kh * d_k + i];
    ks[i] = act[key_dim + kh * d_k + i];
  }
  __syncthreads();
  // prepare_qk (gdn.rs:110-118): l2_norm's sequential f32 sum of squares (kimi_linear/ops.rs:34-40)
  // for q on thread 0 and k on thread 64, the decay and write strength on thread 128
  if (t == 0 || t == 64) {
    float *v = t == 0 ? qs : ks;
    float ss = 0.0f;
    int i = 0;
    for (; i + 16 <= d_k; i += 16) {  // in order; sixteen LDS reads in flight at a time
      float x[16];
#pragma unroll
      for (int u = 0; u < 16; u++) x[u] = v[i + u];
#pragma unroll
      for (int u = 0; u < 16; u++) ss = __fadd_rn(ss, __fmul_rn(x[u], x[u]));
    }
    for (; i < d_k; i++) ss = __fadd_rn(ss, __fmul_rn(v[i], v[i]));
    coef[t == 0 ? 0 : 1] = __fdiv_rn(1.0f, fmaxf(rbt_sqrt_rn(ss), 1e-6f));
  } else if (t == 128) {
    // alpha = exp(-exp(a_log) * softplus(a + dt_bias)), softplus(x) = max(x, 0) + ln_1p(exp(-|x|))
    const float x = __fadd_rn(ah, dth);
    const float sp = __fadd_rn(fmaxf(x, 0.0f), (float)log1p((double)mx_exp(-fabsf(x))));
    coef[2] = mx_exp(__fmul_rn(-mx_exp(alh), sp));
    coef[3] = mx_sigmoid(bh);
  }
  __syncthreads();
  const float qscale = __fdiv_rn(1.0f, rbt_sqrt_rn((float)d_k));
  const float sq = coef[0], sk = coef[1], alpha = coef[2], beta = coef[3];
  // S *= alpha (kda.rs:140-144); c[j] = sum_i k_i S[i, j] (kda.rs:146-151)
  float4 c = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < MR; r++)
    if (NR > 0 || r < nr) {
      s[r] = make_float4(__fmul_rn(s[r].x, alpha), __fmul_rn(s[r].y, alpha), __fmul_rn(s[r].z, alpha),
                         __fmul_rn(s[r].w, alpha));
      const float ki = __fmul_rn(ks[g + G * r], sk);
      c.x = __fadd_rn(c.x, __fmul_rn(ki, s[r].x));
      c.y = __fadd_rn(c.y, __fmul_rn(ki, s[r].y));
      c.z = __fadd_rn(c.z, __fmul_rn(ki, s[r].z));
      c.w = __fadd_rn(c.w, __fmul_rn(ki, s[r].w));
    }
  reinterpret_cast<float4 *>(part)[g * QN + jq] = c;
  __syncthreads();
  float4 cj = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int q = 0; q < G; q++) {
    const float4 p = reinterpret_cast<const float4 *>(part)[q * QN + jq];
    cj = make_float4(__fadd_rn(cj.x, p.x), __fadd_rn(cj.y, p.y), __fadd_rn(cj.z, p.z), __fadd_rn(cj.w, p.w));
  }
  __syncthreads();
  // S[i, j] += (beta k_i) (v_j - c_j) (kda.rs:153-158), then o[j] = sum_i q_i S[i, j] (:160-165)
  const float4 v4 = reinterpret_cast<const float4 *>(vs)[jq];
  const float4 dv = make_float4(__fsub_rn(v4.x, cj.x), __fsub_rn(v4.y, cj.y), __fsub_rn(v4.z, cj.z),
                                __fsub_rn(v4.w, cj.w));
  float4 o = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
  for (int r = 0; r < MR; r++)
    if (NR > 0 || r < nr) {
      const int i = g + G * r;
      const float bk = __fmul_rn(beta, __fmul_rn(ks[i], sk));
      s[r].x = __fadd_rn(s[r].x, __fmul_rn(bk, dv.x));
      s[r].y = __fadd_rn(s[r].y, __fmul_rn(bk, dv.y));
      s[r].z = __fadd_rn(s[r].z, __fmul_rn(bk, dv.z));
      s[r].w = __fadd_rn(s[r].w, __fmul_rn(bk, dv.w));
      Sp[r * rs] = s[r];
      const float qi = __fmul_rn(__fmul_rn(qs[i], sq), qscale);
      o.x = __fadd_rn(o.x, __fmul_rn(qi, s[r].x));
      o.y = __fadd_rn(o.y, __fmul_rn(qi, s[r].y));
      o.z = __fadd_rn(o.z, __fmul_rn(qi, s[r].z));
      o.w = __fadd_rn(o.w, __fmul_rn(qi, s[r].w));
    }
  reinterpret_cast<float4 *>(part)[g * QN + jq] = o;
  __syncthreads();
  if (t < d_v) {
    float oj = 0.0f;
    for (int q = 0; q < G; q++) oj = __fadd_rn(oj, part[q * d_v + t]);
    vs[t] = oj;
  }
  __syncthreads();
  // head_output_gate_silu (gdn.rs:122-128): rmsnorm (kimi_linear/ops.rs:46-53: an f64 sum of
  // squares, here per lane of wave 0 then a butterfly; f64 sums of fp32 squares round to the same
  // fp32 in any order but for rare ties) then * silu(z)
  if (t < 64) {
    double ms = 0.0;
    for (int i = t; i < d_v; i += 64) ms += (double)vs[i] * (double)vs[i];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) ms += __shfl_xor(ms, d, 64);
    if (t == 0) coef[0] = __fdiv_rn(1.0f, rbt_sqrt_rn(__fadd_rn((float)(ms / (double)d_v), eps)));
  }
  __syncthreads();
  if (t < d_v) {
    const float r = coef[0];
    const float on = __fmul_rn(vs[t], __fmul_rn(r, nw));
    out[(long)h * d_v + t] = __fmul_rn(on, mx_silu(zv));
  }
}

// ---- GQA --------------------------------------------------------------------------------------
// sin and cos of an fp32 angle (|x| < 2^22) in fp64, light on registers: x minus the nearest
// multiple k of pi/2 (Cody and Waite's reduction with pi/2 split into three doubles; the first fma
// is exact since x - k c1 is a multiple of 2^-52 below 1 in magnitude), then the Taylor series of
// sin and cos on |r| <= pi/4 + ulp to degree 21 and 22 (truncation error below 2e-25), and the
// quadrant k mod 4. Rounded to fp32, this gives the fp32 rounding of the exact values, as fp64
// library calls do, without their large-argument paths.
__device__ __forceinline__ void mx_sincos(float xf, float &sn, float &cs) {
  constexpr double c1 = 1.5707963267948966, c2 = 6.123233995736766e-17, c3 = -1.4973849048591698e-33;
  const double x = xf, k = rint(x * 0.6366197723675814);
  double r = fma(-k, c1, x);
  r = fma(-k, c2, r);
  r = fma(-k, c3, r);
  const double r2 = r * r;
  // 1 / n! for n = 0 .. 22 (each factorial is exact in fp64, so each quotient is correctly rounded)
  constexpr double f[23] = {1.0, 1.0, 1.0 / 2, 1.0 / 6, 1.0 / 24, 1.0 / 120, 1.0 / 720, 1.0 / 5040,
                            1.0 / 40320, 1.0 / 362880, 1.0 / 3628800, 1.0 / 39916800, 1.0 / 479001600,
                            1.0 / 6227020800.0, 1.0 / 87178291200.0, 1.0 / 1307674368000.0,
                            1.0 / 20922789888000.0, 1.0 / 355687428096000.0, 1.0 / 6402373705728000.0,
                            1.0 / 121645100408832000.0, 1.0 / 2432902008176640000.0,
                            1.0 / 51090942171709440000.0, 1.0 / 1124000727777607680000.0};
  // sin r = r sum_{n<=10} (-r^2)^n / (2n+1)!, cos r = sum_{n<=11} (-r^2)^n / (2n)!, by Horner
  double ps = f[21], pc = -f[22];
#pragma unroll
  for (int n = 10; n >= 0; n--) {
    if (n < 10) ps = (n & 1 ? -f[2 * n + 1] : f[2 * n + 1]) + r2 * ps;
    pc = (n & 1 ? -f[2 * n] : f[2 * n]) + r2 * pc;
  }
  const double sr = r * ps, cr = pc;
  const int q = (int)((long long)k & 3);
  sn = (float)(q == 0 ? sr : q == 1 ? cr : q == 2 ? -sr : -cr);
  cs = (float)(q == 0 ? cr : q == 1 ? -sr : q == 2 ? -cr : sr);
}

// One workgroup of 256 threads per head: workgroups [0, n_heads) take the query heads -> qp
// [n_heads, hd]; [n_heads, n_heads + n_kv) the KV heads -> cache row pos. Each head's row gets the
// (1 + w) RMSNorm (qwen38/ops.rs:25-33: f64 sum of squares in order) and the rotate-half RoPE of its
// first rope_dim entries (attention.rs:160-172). NPT = entries per thread (hd <= 256 NPT).
// Every global load is issued at entry (the row, the norm's weights and, for KV heads, the value
// row; clamped indices, so none sits behind a branch), and the rotation's sines and cosines, which
// depend on nothing loaded, are computed while those loads travel.
template <int NPT>
__global__ __launch_bounds__(256) void k_gqa_prep(const float *__restrict__ qg, const float *__restrict__ kin,
                                                  const float *__restrict__ vin, int n_heads, int n_kv, int hd,
                                                  const float *__restrict__ qn, const float *__restrict__ kn,
                                                  float eps, int rope_dim, int pos, float theta,
                                                  float *__restrict__ qp, float *__restrict__ kc,
                                                  float *__restrict__ vc) {
  constexpr int NP = (NPT + 1) / 2;  // rotated pairs per thread (rope_dim / 2 <= hd / 2 <= 128 NPT)
  extern __shared__ float row[];
  __shared__ float rs[1];
  const int b = blockIdx.x, t = threadIdx.x;
  const bool query = b < n_heads;
  const int kvh = query ? 0 : b - n_heads;  // query heads load KV head 0's value row and drop it
  const float *src = query ? qg + (long)b * 2 * hd : kin + (long)kvh * hd;
  const float *w = query ? qn : kn;
  const float *vr = vin + (long)kvh * hd;
  float xr[NPT], wr[NPT], vv[NPT];
#pragma unroll
  for (int k = 0; k < NPT; k++) xr[k] = src[min(t + 256 * k, hd - 1)];
#pragma unroll
  for (int k = 0; k < NPT; k++) wr[k] = w[min(t + 256 * k, hd - 1)];
#pragma unroll
  for (int k = 0; k < NPT; k++) vv[k] = vr[min(t + 256 * k, hd - 1)];
  __builtin_amdgcn_sched_barrier(0);
  const int half = rope_dim / 2;
  float sn[NP], cs[NP];
#pragma unroll
  for (int k = 0; k < NP; k++) {
    const int jj = min(t + 256 * k, max(half, 1) - 1);
    const float e = __fdiv_rn(__fmul_rn(-2.0f, (float)jj), (float)max(rope_dim, 2));
    const float inv = (float)pow((double)theta, (double)e);
    mx_sincos(__fmul_rn((float)pos, inv), sn[k], cs[k]);
  }
#pragma unroll
  for (int k = 0; k < NPT; k++)
    if (t + 256 * k < hd) row[t + 256 * k] = xr[k];
  __syncthreads();
  if (t == 0) {
    double ms = 0.0;
    int i = 0;
    for (; i + 32 <= hd; i += 32) {  // in order; 32 LDS reads in flight at a time
      float x[32];
#pragma unroll
      for (int u = 0; u < 32; u++) x[u] = row[i + u];
#pragma unroll
      for (int u = 0; u < 32; u++) ms += (double)x[u] * (double)x[u];
    }
    for (; i < hd; i++) ms += (double)row[i] * (double)row[i];
    rs[0] = __fdiv_rn(1.0f, rbt_sqrt_rn(__fadd_rn((float)(ms / (double)hd), eps)));
  }
  __syncthreads();
  const float r = rs[0];
#pragma unroll
  for (int k = 0; k < NPT; k++)
    if (t + 256 * k < hd) row[t + 256 * k] = __fmul_rn(xr[k], __fmul_rn(r, __fadd_rn(1.0f, wr[k])));
  __syncthreads();
#pragma unroll
  for (int k = 0; k < NP; k++) {
    const int jj = t + 256 * k;
    if (jj < half) {
      const float x0 = row[jj], x1 = row[jj + half];
      row[jj] = __fsub_rn(__fmul_rn(x0, cs[k]), __fmul_rn(x1, sn[k]));
      row[jj + half] = __fadd_rn(__fmul_rn(x1, cs[k]), __fmul_rn(x0, sn[k]));
    }
  }
  __syncthreads();
  const long kw = (long)n_kv * hd;
#pragma unroll
  for (int k = 0; k < NPT; k++) {
    const int i = t + 256 * k;
    if (i >= hd) break;
    if (query) {
      qp[(long)b * hd + i] = row[i];
    } else {
      kc[(long)pos * kw + (long)kvh * hd + i] = row[i];
      vc[(long)pos * kw + (long)kvh * hd + i] = vv[k];
    }
  }
}

constexpr int GQA_CHUNK = 64;  // positions per workgroup (16 per wave)
constexpr int GQA_MAXREP = 16;  // query heads per KV head (the MFMA tile's rows)

typedef float gq4 __attribute__((ext_vector_type(4)));

// grid (n_kv, chunks), 256 threads. The n_rep (<= 16) query heads of KV head kvh against positions
// [64 c, min(P, 64 c + 64)), on the matrix cores (v_mfma_f32_16x16x4_f32, fp32 products and sums):
//   scores  S[head][pos] = (q_head . k_pos) * scale: wave w takes positions 16 w .. 16 w + 15; lane l
//           (n = l % 16, kq = l / 16) loads 16 bytes of head n's query and of position n's key at
//           dims 16 g + 4 kq .. +3, and MFMA m of group g uses their component m (A[n][kq], B[kq][n]).
//   softmax partials per head over the chunk: m = max S, e = exp(S - m) (LDS), l = sum e.
//   values  O[head][d] = sum_pos e[head][pos] v_pos[d]: wave w takes dims 64 b .. 64 b + 63
//           (b = w, w + 4, ...) as four strided 16-dim tiles (tile c = dims 64 b + 4 n + c), so lane l's
//           16-byte load of v_pos[64 b + 4 n .. +3] feeds the four tiles' MFMAs (A[n][kq] = e[n][pos]).
// part: [n_kv, chunks, n_rep, 4 + hd] = (m, l, -, -, O), rows 16-byte aligned.
__global__ __launch_bounds__(256) void k_gqa_chunk(const float *__restrict__ qp, const float *__restrict__ kc,
                                                   const float *__restrict__ vc, int P, int n_heads, int n_kv, int hd,
                                                   float scale, float *__restrict__ part) {
  __shared__ float es[GQA_MAXREP][GQA_CHUNK + 4];
  __shared__ float wm[4][GQA_MAXREP], wl[4][GQA_MAXREP], hm[GQA_MAXREP];
  const int n_rep = n_heads / n_kv, kvh = blockIdx.x, ch = blockIdx.y, t = threadIdx.x;
  const int w = t >> 6, lane = t & 63, n = lane & 15, kq = lane >> 4;
  const int p0 = ch * GQA_CHUNK, np = min(GQA_CHUNK, P - p0);
  const long kw = (long)n_kv * hd;
  const int pl = 16 * w + n;  // this lane's position (B column) within the chunk
  const bool live = pl < np;
  const float *qrow = qp + ((long)kvh * n_rep + min(n, n_rep - 1)) * hd + 4 * kq;
  const float *krow = kc + (long)(p0 + min(pl, np - 1)) * kw + (long)kvh * hd + 4 * kq;
  gq4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int g = 0; g < hd / 16; g++) {
    const float4 qv = *reinterpret_cast<const float4 *>(qrow + 16 * g);
    const float4 kv = *reinterpret_cast<const float4 *>(krow + 16 * g);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.x, kv.x, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.y, kv.y, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.z, kv.z, acc, 0, 0, 0);
    acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv.w, kv.w, acc, 0, 0, 0);
  }
  // the values of this wave's first dim block, requested before the softmax needs the scores
  const int nb = hd / 64;
  float4 vpre[GQA_CHUNK / 4];
  if (w < nb) {
    const float *vcol = vc + (long)kvh * hd + 64 * w + 4 * n;
#pragma unroll
    for (int st = 0; st < GQA_CHUNK / 4; st++) {
      const int pp = 4 * st + kq;
      vpre[st] = pp < np ? *reinterpret_cast<const float4 *>(vcol + (long)(p0 + pp) * kw) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  }
  // lane l holds S[4 kq + i][position pl], i = 0..3
  float sv[4], mx[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    sv[i] = live ? __fmul_rn(acc[i], scale) : -INFINITY;
    float m = sv[i];
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
    mx[i] = m;
  }
  if (n == 0)
#pragma unroll
    for (int i = 0; i < 4; i++) wm[w][4 * kq + i] = mx[i];
  __syncthreads();
  if (t < GQA_MAXREP) hm[t] = fmaxf(fmaxf(wm[0][t], wm[1][t]), fmaxf(wm[2][t], wm[3][t]));
  __syncthreads();
  float ls[4];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int hh = 4 * kq + i;
    const float e = live ? mx_exp(__fsub_rn(sv[i], hm[hh])) : 0.0f;
    es[hh][pl] = e;
    float l = e;
#pragma unroll
    for (int d = 1; d < 16; d <<= 1) l = __fadd_rn(l, __shfl_xor(l, d, 64));
    ls[i] = l;
  }
  if (n == 0)
#pragma unroll
    for (int i = 0; i < 4; i++) wl[w][4 * kq + i] = ls[i];
  __syncthreads();
  const int nch = gridDim.y;
  float *base = part + ((long)(kvh * nch + ch) * n_rep) * (4 + hd);
  if (t < n_rep) {
    base[(long)t * (4 + hd)] = hm[t];
    base[(long)t * (4 + hd) + 1] = __fadd_rn(__fadd_rn(wl[0][t], wl[1][t]), __fadd_rn(wl[2][t], wl[3][t]));
  }
  // values: wave w, dim blocks b = w, w + 4, ... (the first one prefetched)
  for (int b = w; b < nb; b += 4) {
    gq4 o[4] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
    const float *vcol = vc + (long)kvh * hd + 64 * b + 4 * n;
#pragma unroll
    for (int st = 0; st < GQA_CHUNK / 4; st++) {
      const int pp = 4 * st + kq;
      const float a = es[n][pp];
      const float4 vv = b == w ? vpre[st]
                               : (pp < np ? *reinterpret_cast<const float4 *>(vcol + (long)(p0 + pp) * kw)
                                          : make_float4(0.f, 0.f, 0.f, 0.f));
      o[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vv.x, o[0], 0, 0, 0);
      o[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vv.y, o[1], 0, 0, 0);
      o[2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vv.z, o[2], 0, 0, 0);
      o[3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, vv.w, o[3], 0, 0, 0);
    }
    // lane l holds O[4 kq + i][64 b + 4 n + c] in o[c][i]
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int hh = 4 * kq + i;
      if (hh < n_rep)
        *reinterpret_cast<float4 *>(base + (long)hh * (4 + hd) + 4 + 64 * b + 4 * n) =
            make_float4(o[0][i], o[1][i], o[2][i], o[3][i]);
    }
  }
}

// One query head per workgroup: the chunks' partials merged (each chunk's O and l scaled by
// exp(m_c - M), M the largest m_c), divided by the softmax sum, times sigmoid of the head's gate.
__global__ __launch_bounds__(256) void k_gqa_combine(const float *__restrict__ part, const float *__restrict__ qg,
                                                     int n_heads, int n_kv, int hd, int nch,
                                                     float *__restrict__ ctx) {
  extern __shared__ float fc[];  // [nch] chunk scales, then [nch] scaled sums
  __shared__ float red[4], tot[2];
  const int h = blockIdx.x, n_rep = n_heads / n_kv, kvh = h / n_rep, r = h - kvh * n_rep, t = threadIdx.x;
  const long stride = (long)n_rep * (4 + hd);
  const float *P0 = part + ((long)kvh * nch * n_rep + r) * (4 + hd);
  float m = -INFINITY;
  for (int c = t; c < nch; c += 256) m = fmaxf(m, P0[c * stride]);
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
  if ((t & 63) == 0) red[t >> 6] = m;
  __syncthreads();
  const float M = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  float *lc = fc + nch;  // [nch] each chunk's l scaled
  for (int c = t; c < nch; c += 256) {
    const float f = mx_exp(__fsub_rn(P0[c * stride], M));
    fc[c] = f;
    lc[c] = __fmul_rn(P0[c * stride + 1], f);
  }
  __syncthreads();
  if (t == 0) {
    float L = 0.0f;
    int c = 0;
    for (; c + 16 <= nch; c += 16) {  // in order; sixteen LDS reads in flight at a time
      float x[16];
#pragma unroll
      for (int u = 0; u < 16; u++) x[u] = lc[c + u];
#pragma unroll
      for (int u = 0; u < 16; u++) L = __fadd_rn(L, x[u]);
    }
    for (; c < nch; c++) L = __fadd_rn(L, lc[c]);
    tot[0] = L;
  }
  __syncthreads();
  const float L = tot[0];
  for (int d = t; d < hd; d += 256) {
    // the chunks' terms in chunk order; their loads issued sixteen at a time (each batch waits
    // one round trip to L2)
    constexpr int CB = 16;
    float acc = 0.0f;
    int c = 0;
    for (; c + CB <= nch; c += CB) {
      float xv[CB];
#pragma unroll
      for (int u = 0; u < CB; u++) xv[u] = P0[(long)(c + u) * stride + 4 + d];
#pragma unroll
      for (int u = 0; u < CB; u++) acc = __fadd_rn(acc, __fmul_rn(xv[u], fc[c + u]));
    }
    for (; c < nch; c++) acc = __fadd_rn(acc, __fmul_rn(P0[c * stride + 4 + d], fc[c]));
    const float g = qg[(long)h * 2 * hd + hd + d];
    ctx[(long)h * hd + d] = __fmul_rn(__fdiv_rn(acc, L), mx_sigmoid(g));
  }
}

// ---- launchers ----------------------------------------------------------------------------------
bool gdn_ok(int n_v, int n_k, int d_k, int d_v) {
  return n_v > 0 && n_k > 0 && n_v % n_k == 0 && d_v > 0 && d_v % 4 == 0 && d_v <= GDN_NT &&
         GDN_NT % (d_v / 4) == 0 && d_k > 0 && d_k % 2 == 0 && d_k <= GDN_MAXR * (GDN_NT / (d_v / 4));
}

hipError_t launch_gdn(const Ctx &c, float *conv_hist, const float *conv_w, int K, float *states,
                      const float *qkv_pre, const float *z, const float *a, const float *b, const float *a_log,
                      const float *dt_bias, const float *norm_w, float eps, int n_v, int n_k, int d_k, int d_v,
                      float *act, float *out) {
  if (!gdn_ok(n_v, n_k, d_k, d_v) || K < 1) return hipErrorInvalidValue;
  const int key_dim = n_k * d_k, C = 2 * key_dim + n_v * d_v;
  launch_k(c, K == 4 ? k_gdn_conv<4> : K == 3 ? k_gdn_conv<3> : K == 2 ? k_gdn_conv<2> : k_gdn_conv<0>,
           dim3((C + 255) / 256), dim3(256), conv_hist, qkv_pre, conv_w, C, K, act);
  const unsigned lds = (unsigned)((2 * d_k + d_v + 4 * GDN_NT) * sizeof(float));
  const int G = GDN_NT / (d_v / 4);
  auto head = d_k == 8 * G ? k_gdn_head<8> : d_k == 4 * G ? k_gdn_head<4> : d_k == 16 * G ? k_gdn_head<16>
              : d_k == 2 * G ? k_gdn_head<2> : k_gdn_head<0>;
  launch_ks(c, head, dim3(n_v), dim3(GDN_NT), lds, states, (const float *)act, key_dim, n_v, n_k, d_k, d_v, z, a,
            b, a_log, dt_bias, norm_w, eps, out);
  return hipGetLastError();
}

bool gqa_ok(int n_heads, int n_kv, int hd, int rope_dim) {
  return n_kv > 0 && n_heads % n_kv == 0 && n_heads / n_kv <= GQA_MAXREP && hd > 0 && hd % 64 == 0 &&
         hd <= 1024 && rope_dim >= 0 && rope_dim % 2 == 0 && rope_dim <= hd;
}

size_t gqa_part_floats(int n_heads, int n_kv, int hd, int positions) {
  const int nch = (positions + GQA_CHUNK - 1) / GQA_CHUNK;
  return (size_t)n_kv * nch * (n_heads / n_kv) * (4 + hd);
}

hipError_t launch_gqa(const Ctx &c, const float *qg, const float *k, const float *v, int n_heads, int n_kv, int hd,
                      const float *qn, const float *kn, float eps, int rope_dim, float theta, float scale, int pos,
                      float *kc, float *vc, float *qp, float *part, float *ctx) {
  if (!gqa_ok(n_heads, n_kv, hd, rope_dim) || pos < 0) return hipErrorInvalidValue;
  const int P = pos + 1, nch = (P + GQA_CHUNK - 1) / GQA_CHUNK;
  if ((size_t)nch * 2 * sizeof(float) > 48 * 1024) return hipErrorInvalidValue;  // the combine's chunk scales
  auto prep = hd <= 256 ? k_gqa_prep<1> : hd <= 512 ? k_gqa_prep<2> : k_gqa_prep<4>;
  launch_ks(c, prep, dim3(n_heads + n_kv), dim3(256), (unsigned)(hd * sizeof(float)), qg, k, v, n_heads, n_kv, hd,
            qn, kn, eps, rope_dim, pos, theta, qp, kc, vc);
  launch_k(c, k_gqa_chunk, dim3(n_kv, nch), dim3(256), (const float *)qp, (const float *)kc, (const float *)vc, P,
           n_heads, n_kv, hd, scale, part);
  launch_ks(c, k_gqa_combine, dim3(n_heads), dim3(256), (unsigned)(2 * nch * sizeof(float)), (const float *)part, qg,
            n_heads, n_kv, hd, nch, ctx);
  return hipGetLastError();
}

}  // namespace rbt
