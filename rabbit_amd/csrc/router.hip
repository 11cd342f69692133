// router.hip -- router logits, top-k selection and token -> expert grouping for gfx950.
//
// The reference computes every router logit as a left-to-right fp32 fold of rounded products
// (kernels.rs:113-124, Iterator::sum) and selects on it; a tree reduction on the GPU would round
// differently and could flip a near-tie at the k / k+1 boundary. Selection here is exact anyway:
//
//  1. Logits with certified intervals (k_router_logits_b / _t / _w, and inside k_router1): the
//     products p_k = fl32(x_k w_k) exactly as the reference forms them, summed in fp64 (S), with a
//     rigorous bound B on |L_ref - S|, where L_ref is the reference's sequential fp32 result. With
//     S_j the exact prefix sums, u = 2^-24, u' = u/(1-u) and T = sum_j |S_j|, the fold's error
//     obeys |L_ref - S| <= u' T / (1 - n u'). T needs every prefix sum (a parallel fp64 scan);
//     extra slack covers the fp64 arithmetic itself. Batches of 64+ tokens instead fold every
//     logit as the reference does (k_router_logits_exact), four folds per lane.
//  2. Selection (select3_body, and its register fast path select4_fast): the fp32 interval
//     [lo, hi] that must contain L_ref is pushed through the monotone key map (logit bias,
//     sigmoid, selection bias), top-k is taken on the midpoints with the reference's tie rule
//     (higher key first, lower expert id on ties), and then certified: every expert whose key
//     interval could reach the selected set, or overlaps another winner's, gets its exact
//     sequential fp32 fold recomputed (same operations in the same order as the reference). After
//     that, every relevant comparison is either strict or an exact tie, so the ids are the
//     reference's ids. One token: k_router1 runs logits, selection and the shared expert's gate/up
//     in one launch, and may leave the exact folds to the gate/up launch (k_xgateup1f).
//  3. k_group (several tokens): unique_experts order (glm52/moe.rs:333-344), per-expert token
//     lists in token order, and per-token pick lists ordered by first occurrence.
#include "rbt_device.h"
#include "rbt_gemv.h"
#include "rbt_internal.h"
#include "rbt_xmfma.h"

namespace rbt {

// ------------------------------------------------------------------------------------------------
// 1. logits with certified error bound
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ double block_excl_scan_256(double v, double *sh, double *total) {
  // inclusive wave scan
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  double inc = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    double o = __shfl_up(inc, d, 64);
    if (lane >= d) inc += o;
  }
  if (lane == 63) sh[wid] = inc;
  __syncthreads();
  double off = 0.0, tot = 0.0;
  for (int w = 0; w < 4; w++) {
    if (w < wid) off += sh[w];
    tot += sh[w];
  }
  __syncthreads();
  *total = tot;
  return off + inc - v;
}

__device__ __forceinline__ double block_sum_256(double v, double *sh) {
  v = rbt_wave_sum_d(v);
  const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
  if (lane == 0) sh[wid] = v;
  __syncthreads();
  double t = sh[0] + sh[1] + sh[2] + sh[3];
  __syncthreads();
  return t;
}

constexpr int ROUTER_MAXC = 32;  // cached products per thread (H <= 8192 keeps them in registers)

// Rows 0..E-1 are router rows; row E (when sgate != nullptr) is the shared-expert gate vector.
__global__ __launch_bounds__(256) void k_router_logits(const float *__restrict__ x, int S, int H,
                                                       const float *__restrict__ W, int E,
                                                       const float *__restrict__ sgate, double *__restrict__ mid,
                                                       double *__restrict__ bnd, int erows) {
  __shared__ double sh[4];
  const int e = blockIdx.x;
  const float *w = e < E ? W + (size_t)e * H : sgate;
  const int t = threadIdx.x;
  const int c = (H + 255) / 256;
  const int k0 = t * c;
  const int k1 = min(k0 + c, H);
  const double u1 = 5.9604648328104515e-08;  // u/(1-u), u = 2^-24 (rounded up)
  const double e64 = 1.1102230246251565e-16; // 2^-53
  for (int s = 0; s < S; s++) {
    const float *xs = x + (size_t)s * H;
    float pc[ROUTER_MAXC];
    double run = 0.0, pabs = 0.0;
    if (c <= ROUTER_MAXC) {
#pragma unroll
      for (int j = 0; j < ROUTER_MAXC; j++) {
        int k = k0 + j;
        float p = (j < c && k < k1) ? __fmul_rn(xs[k], w[k]) : 0.0f;
        pc[j] = p;
        run += (double)p;
        pabs += fabs((double)p);
      }
    } else {
      for (int k = k0; k < k1; k++) {
        float p = __fmul_rn(xs[k], w[k]);
        run += (double)p;
        pabs += fabs((double)p);
      }
    }
    double total;
    double pre = block_excl_scan_256(run, sh, &total);
    double T = 0.0;
    if (c <= ROUTER_MAXC) {
#pragma unroll
      for (int j = 0; j < ROUTER_MAXC; j++) {
        if (j < c && k0 + j < k1) {
          pre += (double)pc[j];
          T += fabs(pre);
        }
      }
    } else {
      for (int k = k0; k < k1; k++) {
        pre += (double)__fmul_rn(xs[k], w[k]);
        T += fabs(pre);
      }
    }
    T = block_sum_256(T, sh);
    double P = block_sum_256(pabs, sh);
    if (t == 0) {
      double n = (double)H;
      double slack = 4.0 * n * e64 * (P + T) + n * n * e64 * P;
      double Tu = T * (1.0 + 4.0 * n * e64) + slack;
      double B = (u1 * Tu) / (1.0 - n * u1) + slack;
      B = B * (1.0 + 1e-9) + 1e-300;
      mid[(size_t)s * erows + e] = total;
      bnd[(size_t)s * erows + e] = B;
    }
  }
}

// Fast path (H % 256 == 0): one wave per router row. The row is walked in chunks of 256 elements,
// lane l taking the 4 consecutive elements [4l, 4l+4) of each chunk with one 16-byte load (so each
// load instruction reads 1 KB contiguous); a wave-wide fp64 exclusive scan per chunk gives every
// prefix sum S_j for the bound term T.
__device__ __forceinline__ double wave_incl_scan_d(double v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    double o = __shfl_up(v, d, 64);
    if (lane >= d) v += o;
  }
  return v;
}

__global__ __launch_bounds__(256) void k_router_logits_w(const float *__restrict__ x, int S, int H,
                                                         const float *__restrict__ W, int E,
                                                         const float *__restrict__ sgate, double *__restrict__ mid,
                                                         double *__restrict__ bnd, int erows) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= erows) return;
  const float4 *w4 = reinterpret_cast<const float4 *>(row < E ? W + (size_t)row * H : sgate);
  const double u1 = 5.9604648328104515e-08;   // u/(1-u), u = 2^-24 (rounded up)
  const double e64 = 1.1102230246251565e-16;  // 2^-53
  const int nch = H / 256;
  for (int s = 0; s < S; s++) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)s * H);
    double base = 0.0, T = 0.0, Pa = 0.0;
    for (int c = 0; c < nch; c++) {
      const float4 xv = x4[c * 64 + lane], wv = w4[c * 64 + lane];
      const double p0 = (double)__fmul_rn(xv.x, wv.x), p1 = (double)__fmul_rn(xv.y, wv.y);
      const double p2 = (double)__fmul_rn(xv.z, wv.z), p3 = (double)__fmul_rn(xv.w, wv.w);
      const double l1 = p0 + p1, l2 = l1 + p2, l3 = l2 + p3;
      const double inc = wave_incl_scan_d(l3);
      const double pre = base + (inc - l3);
      T += fabs(pre + p0) + fabs(pre + l1) + fabs(pre + l2) + fabs(pre + l3);
      Pa += fabs(p0) + fabs(p1) + fabs(p2) + fabs(p3);
      base += __shfl(inc, 63, 64);
    }
    T = rbt_wave_sum_d(T);
    Pa = rbt_wave_sum_d(Pa);
    if (lane == 0) {
      const double n = (double)H;
      const double slack = 8.0 * n * e64 * (Pa + T) + n * n * e64 * Pa;
      const double Tu = T * (1.0 + 8.0 * n * e64) + slack;
      double B = (u1 * Tu) / (1.0 - n * u1) + slack;
      B = B * (1.0 + 1e-9) + 1e-300;
      mid[(size_t)s * erows + row] = base;
      bnd[(size_t)s * erows + row] = B;
    }
  }
}

// Transposed variant (H % 256 == 0, H <= 8192): one 64-thread workgroup per router row. The wave
// loads the row and x with coalesced 16-byte loads, forms the products and stores them to LDS so
// that lane l then owns the contiguous segment [l*H/64, (l+1)*H/64): one sequential fp64 prefix per
// lane and a single wave scan give every prefix sum S_j. The segment stride is padded by 4 floats
// so the 16-byte LDS reads of neighbouring lanes fall in different banks.
constexpr int RT_MAXH = 8192;
// LDS stride of a thread's segment of seg products (seg a multiple of 4): every thread reads its
// segment with 16-byte loads, which are conflict-free when the stride in 16-byte units is odd (an even
// stride puts neighbouring lanes on the same banks: at seg = 28 the plain seg + 4 = 32 dwords maps all
// 64 lanes onto two bank groups).
__device__ __forceinline__ int rt_segp(int seg) { return ((seg >> 2) & 1) ? seg : seg + 4; }


__global__ __launch_bounds__(64) void k_router_logits_t(const float *__restrict__ x, int S, int H,
                                                        const float *__restrict__ W, int E,
                                                        const float *__restrict__ sgate, double *__restrict__ mid,
                                                        double *__restrict__ bnd, int erows) {
  __shared__ float lp[RT_MAXH + 4 * 64];
  const int lane = threadIdx.x;
  const int row = blockIdx.x;
  const float4 *w4 = reinterpret_cast<const float4 *>(row < E ? W + (size_t)row * H : sgate);
  const int seg = H / 64;      // elements per lane segment
  const int segp = rt_segp(seg);  // padded segment stride in LDS
  const int nch = H / 256;     // coalesced chunks (one float4 per lane)
  const double u1 = 5.9604648328104515e-08;   // u/(1-u), u = 2^-24 (rounded up)
  const double e64 = 1.1102230246251565e-16;  // 2^-53
  constexpr int MAXCH = RT_MAXH / 256;
  float4 wv[MAXCH];
#pragma unroll
  for (int c = 0; c < MAXCH; c++)
    if (c < nch) wv[c] = w4[c * 64 + lane];
  for (int s = 0; s < S; s++) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)s * H);
    float4 xv[MAXCH];
#pragma unroll
    for (int c = 0; c < MAXCH; c++)
      if (c < nch) xv[c] = x4[c * 64 + lane];
#pragma unroll
    for (int c = 0; c < MAXCH; c++) {
      if (c < nch) {
        const int j = c * 256 + 4 * lane;            // first of this lane's 4 elements
        const int dst = (j / seg) * segp + (j % seg); // 4 consecutive elements stay in one segment
        float4 p;
        p.x = __fmul_rn(xv[c].x, wv[c].x);
        p.y = __fmul_rn(xv[c].y, wv[c].y);
        p.z = __fmul_rn(xv[c].z, wv[c].z);
        p.w = __fmul_rn(xv[c].w, wv[c].w);
        *reinterpret_cast<float4 *>(&lp[dst]) = p;
      }
    }
    __syncthreads();
    const float *mine = lp + lane * segp;
    double loc = 0.0, pa = 0.0;
    for (int t = 0; t < seg; t += 4) {
      const float4 p = *reinterpret_cast<const float4 *>(mine + t);
      loc += (double)p.x;
      loc += (double)p.y;
      loc += (double)p.z;
      loc += (double)p.w;
      pa += fabs((double)p.x) + fabs((double)p.y) + fabs((double)p.z) + fabs((double)p.w);
    }
    const double inc = wave_incl_scan_d(loc);
    double pre = inc - loc, T = 0.0;
    for (int t = 0; t < seg; t += 4) {
      const float4 p = *reinterpret_cast<const float4 *>(mine + t);
      pre += (double)p.x;
      T += fabs(pre);
      pre += (double)p.y;
      T += fabs(pre);
      pre += (double)p.z;
      T += fabs(pre);
      pre += (double)p.w;
      T += fabs(pre);
    }
    T = rbt_wave_sum_d(T);
    pa = rbt_wave_sum_d(pa);
    const double total = __shfl(inc, 63, 64);
    if (lane == 0) {
      const double n = (double)H;
      const double slack = 8.0 * n * e64 * (pa + T) + n * n * e64 * pa;
      const double Tu = T * (1.0 + 8.0 * n * e64) + slack;
      double B = (u1 * Tu) / (1.0 - n * u1) + slack;
      B = B * (1.0 + 1e-9) + 1e-300;
      mid[(size_t)s * erows + row] = total;
      bnd[(size_t)s * erows + row] = B;
    }
    __syncthreads();
  }
}

// Block variant (H % 1024 == 0, H <= 8192): one 256-thread workgroup per router row; coalesced
// loads, products through padded LDS, thread t owns the contiguous segment [t*H/256, (t+1)*H/256),
// then a block-wide fp64 scan. Four times less serial fp64 work per thread than one wave per row.
__global__ __launch_bounds__(256) void k_router_logits_b(const float *__restrict__ x, int S, int H,
                                                         const float *__restrict__ W, int E,
                                                         const float *__restrict__ sgate, double *__restrict__ mid,
                                                         double *__restrict__ bnd, int erows) {
  __shared__ float lp[RT_MAXH + 4 * 256];
  __shared__ double sh[4];
  const int t = threadIdx.x;
  const int row = blockIdx.x;
  const float4 *w4 = reinterpret_cast<const float4 *>(row < E ? W + (size_t)row * H : sgate);
  const int seg = H / 256;   // elements per thread segment
  const int segp = rt_segp(seg);  // padded stride
  const int nch = H / 1024;  // coalesced chunks (one float4 per thread)
  const double u1 = 5.9604648328104515e-08;   // u/(1-u), u = 2^-24 (rounded up)
  const double e64 = 1.1102230246251565e-16;  // 2^-53
  constexpr int MAXCH = RT_MAXH / 1024;
  float4 wv[MAXCH];
#pragma unroll
  for (int c = 0; c < MAXCH; c++)
    if (c < nch) wv[c] = w4[c * 256 + t];
  for (int s = 0; s < S; s++) {
    const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)s * H);
#pragma unroll
    for (int c = 0; c < MAXCH; c++) {
      if (c < nch) {
        const float4 xv = x4[c * 256 + t];
        const int j = c * 1024 + 4 * t;
        const int dst = (j / seg) * segp + (j % seg);
        float4 p;
        p.x = __fmul_rn(xv.x, wv[c].x);
        p.y = __fmul_rn(xv.y, wv[c].y);
        p.z = __fmul_rn(xv.z, wv[c].z);
        p.w = __fmul_rn(xv.w, wv[c].w);
        *reinterpret_cast<float4 *>(&lp[dst]) = p;
      }
    }
    __syncthreads();
    const float *mine = lp + t * segp;
    double loc = 0.0, pa = 0.0;
    for (int q = 0; q < seg; q += 4) {
      const float4 p = *reinterpret_cast<const float4 *>(mine + q);
      loc += (double)p.x;
      loc += (double)p.y;
      loc += (double)p.z;
      loc += (double)p.w;
      pa += fabs((double)p.x) + fabs((double)p.y) + fabs((double)p.z) + fabs((double)p.w);
    }
    double total;
    double pre = block_excl_scan_256(loc, sh, &total);
    double T = 0.0;
    for (int q = 0; q < seg; q += 4) {
      const float4 p = *reinterpret_cast<const float4 *>(mine + q);
      pre += (double)p.x;
      T += fabs(pre);
      pre += (double)p.y;
      T += fabs(pre);
      pre += (double)p.z;
      T += fabs(pre);
      pre += (double)p.w;
      T += fabs(pre);
    }
    T = block_sum_256(T, sh);
    pa = block_sum_256(pa, sh);
    if (t == 0) {
      const double n = (double)H;
      const double slack = 8.0 * n * e64 * (pa + T) + n * n * e64 * pa;
      const double Tu = T * (1.0 + 8.0 * n * e64) + slack;
      double B = (u1 * Tu) / (1.0 - n * u1) + slack;
      B = B * (1.0 + 1e-9) + 1e-300;
      mid[(size_t)s * erows + row] = total;
      bnd[(size_t)s * erows + row] = B;
    }
    __syncthreads();
  }
}

// Exact logits for a batch of tokens: logit[t, e] = fold(-0.0, +) of fl32(x[t, k] * w[e, k]) over
// k ascending, the reference's own sequential sum (kernels.rs:113-124), so selection needs no
// certification. Each lane carries four independent folds (2 tokens x 2 rows); a workgroup covers
// 32 tokens x 32 router rows, with 256-column chunks of both operands staged through LDS (the
// next chunk is loaded while the current one is folded). Rows E (when sgate is set) and beyond
// read the shared-gate vector; rows past erows and tokens past S are computed on clamped inputs
// and not written.
constexpr int RX_T = 32, RX_E = 32, RX_KC = 256, RX_PAD = 4;
constexpr int RX_EXACT_MIN_S = 64;  // from this batch size the exact folds beat the certified sums
__global__ __launch_bounds__(256) void k_router_logits_exact(const float *__restrict__ x, int S, int H,
                                                             const float *__restrict__ W, int E,
                                                             const float *__restrict__ sgate, float *__restrict__ logits,
                                                             int erows) {
  __shared__ __attribute__((aligned(16))) float xs[2][RX_T][RX_KC + RX_PAD];
  __shared__ __attribute__((aligned(16))) float ws[2][RX_E][RX_KC + RX_PAD];
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int t0 = blockIdx.y * RX_T, e0 = blockIdx.x * RX_E;
  // staging: thread tid moves row tid / 8, 32 consecutive floats (8 x float4) of each operand
  const int sr = tid >> 3, sc = (tid & 7) * 32;
  const float *xrow = x + (size_t)min(t0 + sr, S - 1) * H;
  const int er = min(e0 + sr, erows - 1);
  const float *wrow = er < E ? W + (size_t)er * H : sgate;
  float4 stx[8], stw[8];
  auto load_chunk = [&](int c) {
    const float4 *px = reinterpret_cast<const float4 *>(xrow + c * RX_KC + sc);
    const float4 *pw = reinterpret_cast<const float4 *>(wrow + c * RX_KC + sc);
#pragma unroll
    for (int i = 0; i < 8; i++) {
      stx[i] = px[i];
      stw[i] = pw[i];
    }
  };
  auto store_chunk = [&](int b) {
#pragma unroll
    for (int i = 0; i < 8; i++) {
      *reinterpret_cast<float4 *>(&xs[b][sr][sc + 4 * i]) = stx[i];
      *reinterpret_cast<float4 *>(&ws[b][sr][sc + 4 * i]) = stw[i];
    }
  };
  // lane's folds: tokens 16 (wave >> 1) + 2 (lane & 7) + {0, 1}, rows 16 (wave & 1) + 2 (lane >> 3) + {0, 1}
  const int lt = 16 * (wave >> 1) + 2 * (lane & 7), le = 16 * (wave & 1) + 2 * (lane >> 3);
  float a00 = -0.0f, a01 = -0.0f, a10 = -0.0f, a11 = -0.0f;
  const int nch = H / RX_KC;
  load_chunk(0);
  store_chunk(0);
  if (nch > 1) load_chunk(1);
  __syncthreads();
  for (int c = 0; c < nch; c++) {
    const int b = c & 1;
    const float *x0 = xs[b][lt], *x1 = xs[b][lt + 1], *w0 = ws[b][le], *w1 = ws[b][le + 1];
#pragma unroll 4
    for (int k = 0; k < RX_KC; k += 4) {
      const float4 xa = *reinterpret_cast<const float4 *>(x0 + k), xb = *reinterpret_cast<const float4 *>(x1 + k);
      const float4 wa = *reinterpret_cast<const float4 *>(w0 + k), wb = *reinterpret_cast<const float4 *>(w1 + k);
      a00 = __fadd_rn(a00, __fmul_rn(xa.x, wa.x));
      a01 = __fadd_rn(a01, __fmul_rn(xa.x, wb.x));
      a10 = __fadd_rn(a10, __fmul_rn(xb.x, wa.x));
      a11 = __fadd_rn(a11, __fmul_rn(xb.x, wb.x));
      a00 = __fadd_rn(a00, __fmul_rn(xa.y, wa.y));
      a01 = __fadd_rn(a01, __fmul_rn(xa.y, wb.y));
      a10 = __fadd_rn(a10, __fmul_rn(xb.y, wa.y));
      a11 = __fadd_rn(a11, __fmul_rn(xb.y, wb.y));
      a00 = __fadd_rn(a00, __fmul_rn(xa.z, wa.z));
      a01 = __fadd_rn(a01, __fmul_rn(xa.z, wb.z));
      a10 = __fadd_rn(a10, __fmul_rn(xb.z, wa.z));
      a11 = __fadd_rn(a11, __fmul_rn(xb.z, wb.z));
      a00 = __fadd_rn(a00, __fmul_rn(xa.w, wa.w));
      a01 = __fadd_rn(a01, __fmul_rn(xa.w, wb.w));
      a10 = __fadd_rn(a10, __fmul_rn(xb.w, wa.w));
      a11 = __fadd_rn(a11, __fmul_rn(xb.w, wb.w));
    }
    if (c + 1 < nch) {
      store_chunk(b ^ 1);
      if (c + 2 < nch) load_chunk(c + 2);
    }
    __syncthreads();
  }
  const int ta = t0 + lt, ea = e0 + le;
  if (ta < S && ea < erows) logits[(size_t)ta * erows + ea] = a00;
  if (ta < S && ea + 1 < erows) logits[(size_t)ta * erows + ea + 1] = a01;
  if (ta + 1 < S && ea < erows) logits[(size_t)(ta + 1) * erows + ea] = a10;
  if (ta + 1 < S && ea + 1 < erows) logits[(size_t)(ta + 1) * erows + ea + 1] = a11;
}

// ------------------------------------------------------------------------------------------------
// 2. per-token selection
// ------------------------------------------------------------------------------------------------
// sigmoid as the reference writes it, 1/(1 + exp(-v)), with exp correctly rounded to f32 (the
// reference calls the platform libm's expf).
__device__ __forceinline__ float sigmoid_ref(float v) {
  float e = (float)exp(-(double)v);
  return __fdiv_rn(1.0f, __fadd_rn(1.0f, e));
}

struct SelParams {
  int family;  // RBT_FAMILY_*
  int E, erows, k, H, S;
  const float *logit_bias;   // may be null
  const float *router_bias;  // may be null
  int norm_topk;
  float routed_scale;
  int n_group, topk_group;
  const float *x;  // [S, H] for exact recomputation
  const float *W;  // [E, H]
};

// Selection key of one logit value for the family (monotone non-decreasing in the logit).
__device__ __forceinline__ float sel_key(const SelParams &P, int e, float l) {
  if (P.logit_bias) l = __fadd_rn(l, P.logit_bias[e]);
  if (P.family == RBT_FAMILY_QWEN38) return l;
  float p = sigmoid_ref(l);
  return P.router_bias ? __fadd_rn(p, P.router_bias[e]) : p;
}

// Same map with the expert's bias values already loaded (lb/rb ignored when the pointer is null).
__device__ __forceinline__ float sel_key_v(const SelParams &P, float lb, float rb, float l) {
  if (P.logit_bias) l = __fadd_rn(l, lb);
  if (P.family == RBT_FAMILY_QWEN38) return l;
  const float p = sigmoid_ref(l);
  return P.router_bias ? __fadd_rn(p, rb) : p;
}

// (key desc, id asc) ordering: true if (ka, a) ranks before (kb, b).
__device__ __forceinline__ bool ranks_before(float ka, int a, float kb, int b) {
  return ka > kb || (ka == kb && a < b);
}

constexpr int SEL_MAXE = 2048;
constexpr int SEL_MAXK = 64;
constexpr int SEL_NC = 64;  // most candidates the fast selection ranks (one per lane)

// Top-k over keys[] restricted to allowed (nullptr = all); writes out[0..k). One wave.
__device__ void wave_topk(const float *keys, const unsigned char *allowed, int E, int k, int *out) {
  const int lane = threadIdx.x & 63;
  __shared__ unsigned char taken[SEL_MAXE];
  for (int e = lane; e < E; e += 64) taken[e] = 0;
  __syncthreads();
  for (int r = 0; r < k; r++) {
    float bk = -INFINITY;
    int bi = 0x7fffffff;
    for (int e = lane; e < E; e += 64) {
      if (taken[e] || (allowed && !allowed[e])) continue;
      if (bi == 0x7fffffff || ranks_before(keys[e], e, bk, bi)) { bk = keys[e]; bi = e; }
    }
#pragma unroll
    for (int m = 32; m >= 1; m >>= 1) {
      float ok = __shfl_xor(bk, m, 64);
      int oi = __shfl_xor(bi, m, 64);
      if (oi != 0x7fffffff && (bi == 0x7fffffff || ranks_before(ok, oi, bk, bi))) { bk = ok; bi = oi; }
    }
    if (lane == 0) {
      out[r] = bi;
      if (bi != 0x7fffffff) taken[bi] = 1;
    }
    __syncthreads();
  }
}

// The reference's sequential logit: fold(-0.0, +) of fl32(x_k * w_k), k ascending.
__device__ float exact_logit(const float *xs, const float *w, int H) {
  float a = -0.0f;
  for (int k = 0; k < H; k++) a = __fadd_rn(a, __fmul_rn(xs[k], w[k]));
  return a;
}

__global__ __launch_bounds__(64) void k_router_select_grouped(SelParams P, const double *__restrict__ mid,
                                                      const double *__restrict__ bnd, int32_t *__restrict__ ids,
                                                      float *__restrict__ wts, float *__restrict__ sh_scale,
                                                      int *__restrict__ stats) {
  __shared__ float klo[SEL_MAXE], khi[SEL_MAXE], kmid[SEL_MAXE], lmid[SEL_MAXE];
  __shared__ unsigned char exact[SEL_MAXE], allowed[SEL_MAXE];
  __shared__ int sel[SEL_MAXK];
  __shared__ int amb_list[SEL_MAXE];
  __shared__ int namb;
  __shared__ float kth_lo;
  const int lane = threadIdx.x;
  const int s = blockIdx.x;
  const int E = P.E, k = P.k;
  const double *ms = mid + (size_t)s * P.erows;
  const double *bs = bnd + (size_t)s * P.erows;

  for (int e = lane; e < E; e += 64) {
    double m = ms[e], b = bs[e];
    float lo = __double2float_rd(m - b * (1.0 + 1e-12));
    float hi = __double2float_ru(m + b * (1.0 + 1e-12));
    float md = __double2float_rn(m);
    if (md < lo) md = lo;
    if (md > hi) md = hi;
    lmid[e] = md;
    klo[e] = sel_key(P, e, lo);
    khi[e] = sel_key(P, e, hi);
    kmid[e] = sel_key(P, e, md);
    exact[e] = (lo == hi);
  }
  if (lane == 0) namb = 0;
  __syncthreads();

  // Group restriction (rank_top_grouped, glm52/moe.rs:214-229) needs group scores from the keys;
  // for n_group > 1 every group's top-2 sum must itself be certain, so its experts are made exact.
  const bool grouped = P.family != RBT_FAMILY_QWEN38 && P.n_group > 1;
  if (grouped) {
    for (int e = lane; e < E; e += 64) {
      if (!exact[e]) {
        float l = exact_logit(P.x + (size_t)s * P.H, P.W + (size_t)e * P.H, P.H);
        lmid[e] = l;
        klo[e] = khi[e] = kmid[e] = sel_key(P, e, l);
        exact[e] = 1;
      }
    }
    __syncthreads();
    if (lane == 0) {
      int gsz = E / P.n_group;
      float gs[64];
      int ord[64];
      for (int g = 0; g < P.n_group; g++) {
        float t1 = -INFINITY, t2 = -INFINITY;
        for (int e = g * gsz; e < (g + 1) * gsz; e++) {
          float v = kmid[e];
          if (v > t1) { t2 = t1; t1 = v; }
          else if (v > t2) { t2 = v; }
        }
        gs[g] = isfinite(t2) ? __fadd_rn(t1, t2) : t1;
        ord[g] = g;
      }
      for (int a = 1; a < P.n_group; a++) {
        int cur = ord[a], b = a;
        while (b > 0 && (gs[ord[b - 1]] < gs[cur] || (gs[ord[b - 1]] == gs[cur] && ord[b - 1] > cur))) {
          ord[b] = ord[b - 1];
          b--;
        }
        ord[b] = cur;
      }
      for (int e = 0; e < E; e++) allowed[e] = 0;
      for (int t = 0; t < P.topk_group && t < P.n_group; t++)
        for (int e = ord[t] * gsz; e < (ord[t] + 1) * gsz; e++) allowed[e] = 1;
    }
    __syncthreads();
  }
  int kk = k;
  if (grouped) {
    int na = 0;
    for (int e = 0; e < E; e++) na += allowed[e];
    if (kk > na) kk = na;
  }

  wave_topk(kmid, grouped ? allowed : nullptr, E, kk, sel);

  // Certify: R = experts whose upper key reaches the lowest selected lower key.
  if (lane == 0) {
    float m = INFINITY;
    for (int r = 0; r < kk; r++) m = fminf(m, klo[sel[r]]);
    kth_lo = m;
  }
  // R as a list (set semantics: its order does not matter).
  __shared__ int rlist[SEL_MAXE];
  __shared__ int nr;
  if (lane == 0) nr = 0;
  __syncthreads();
  for (int e = lane; e < E; e += 64) {
    if ((grouped && !allowed[e]) || khi[e] < kth_lo) continue;
    rlist[atomicAdd(&nr, 1)] = e;
  }
  __syncthreads();
  const int nR = nr;
  for (int j = lane; j < nR; j += 64) {
    const int e = rlist[j];
    if (exact[e]) continue;
    // e is in R and not exact: ambiguous if its interval overlaps any other member of R.
    bool a = false;
    for (int m = 0; m < nR && !a; m++) {
      const int f = rlist[m];
      if (f != e && klo[e] <= khi[f] && klo[f] <= khi[e]) a = true;
    }
    if (a) amb_list[atomicAdd(&namb, 1)] = e;
  }
  __syncthreads();
  const int na = namb;
  if (na > 0) {
    for (int j = lane; j < na; j += 64) {
      int e = amb_list[j];
      float l = exact_logit(P.x + (size_t)s * P.H, P.W + (size_t)e * P.H, P.H);
      lmid[e] = l;
      klo[e] = khi[e] = kmid[e] = sel_key(P, e, l);
      exact[e] = 1;
    }
    __syncthreads();
    wave_topk(kmid, grouped ? allowed : nullptr, E, kk, sel);
  }
  if (lane == 0 && stats) atomicAdd(stats, na);

  // Weights.
  if (lane == 0) {
    int32_t *io = ids + (size_t)s * k;
    float *wo = wts + (size_t)s * k;
    if (P.family == RBT_FAMILY_QWEN38) {
      // qwen38/moe.rs:66-74: softmax over the winners' logits, max-subtracted.
      float lv[SEL_MAXK];
      for (int r = 0; r < kk; r++) {
        int e = sel[r];
        lv[r] = P.logit_bias ? __fadd_rn(lmid[e], P.logit_bias[e]) : lmid[e];
      }
      float mx = lv[0], sum = 0.0f;
      for (int r = 0; r < kk; r++) {
        lv[r] = (float)exp((double)__fsub_rn(lv[r], mx));
        sum = __fadd_rn(sum, lv[r]);
      }
      for (int r = 0; r < kk; r++) {
        io[r] = sel[r];
        wo[r] = __fdiv_rn(lv[r], sum);
      }
    } else {
      // glm52/moe.rs:231-241: weight = plain sigmoid; norm_topk; routed_scale.
      float wv[SEL_MAXK];
      for (int r = 0; r < kk; r++) {
        int e = sel[r];
        float l = P.logit_bias ? __fadd_rn(lmid[e], P.logit_bias[e]) : lmid[e];
        wv[r] = sigmoid_ref(l);
      }
      if (P.norm_topk) {
        float sum = -0.0f;
        for (int r = 0; r < kk; r++) sum = __fadd_rn(sum, wv[r]);
        sum = __fadd_rn(sum, 1e-20f);
        for (int r = 0; r < kk; r++) wv[r] = __fdiv_rn(wv[r], sum);
      }
      for (int r = 0; r < kk; r++) {
        io[r] = sel[r];
        wo[r] = __fmul_rn(wv[r], P.routed_scale);
      }
    }
    for (int r = kk; r < k; r++) {
      io[r] = -1;
      wo[r] = 0.0f;
    }
    if (sh_scale) {
      float gl = (P.erows > E) ? __double2float_rn(ms[E]) : 0.0f;
      sh_scale[s] = (P.erows > E) ? sigmoid_ref(gl) : 1.0f;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Exact recomputation of one router logit (selection near-ties)
// ------------------------------------------------------------------------------------------------
// The reference's sequential fold, computed by one whole wave: lanes form the products of a block
// of 64 x 32 elements in parallel (the next block's loads are already in flight), then the running
// fp32 sum walks the block lane by lane: lane l adds its 32 products in order and v_readlane hands
// the sum to lane l+1. Same operations in the same order as the reference; only the serial chain
// of adds remains on the critical path. Needs H % 4 == 0 and 16-byte aligned rows (else the plain
// loop below).
__device__ float exact_logit_wave(const float *__restrict__ xs, const float *__restrict__ w, int H) {
  const int lane = threadIdx.x & 63;
  if ((H & 3) || ((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(w)) & 15)) {
    float acc = -0.0f;
    for (int i = 0; i < H; i++) acc = __fadd_rn(acc, __fmul_rn(xs[i], w[i]));
    return acc;
  }
  const float4 *x4 = reinterpret_cast<const float4 *>(xs);
  const float4 *w4 = reinterpret_cast<const float4 *>(w);
  const int H4 = H >> 2;
  float acc = -0.0f;
  float4 xa[8], wa[8];
  auto fetch = [&](int base4) {
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const int k = min(base4 + 8 * lane + j, H4 - 1);
      xa[j] = x4[k];
      wa[j] = w4[k];
    }
  };
  fetch(0);
  for (int base = 0; base < H; base += 2048) {
    float p[32];
#pragma unroll
    for (int j = 0; j < 8; j++) {
      p[4 * j + 0] = __fmul_rn(xa[j].x, wa[j].x);
      p[4 * j + 1] = __fmul_rn(xa[j].y, wa[j].y);
      p[4 * j + 2] = __fmul_rn(xa[j].z, wa[j].z);
      p[4 * j + 3] = __fmul_rn(xa[j].w, wa[j].w);
    }
    if (base + 2048 < H) fetch((base + 2048) >> 2);
    const int n = min(2048, H - base);
    const int full = n >> 5;  // lanes whose 32 products are all in range
    for (int l = 0; l < full; l++) {
      if (lane == l) {
#pragma unroll
        for (int j = 0; j < 32; j++) acc = __fadd_rn(acc, p[j]);
      }
      acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), l));
    }
    if ((full << 5) < n) {  // partial tail lane
      if (lane == full)
        for (int j = 0; j < n - (full << 5); j++) acc = __fadd_rn(acc, p[j]);
      acc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), full));
    }
  }
  return acc;
}


// The same fold with the serial chain on one lane, for a wave that has a 2 x 1024-float LDS buffer
// of its own: the wave forms the products of 1024-element blocks in parallel into the buffer, in
// element order, and lane 0 walks the previous block with 16-byte LDS reads (two groups of eight in
// flight) and dependent adds, the next block's loads already in flight. No exec-mask or readlane
// hand-offs sit on the chain. Same operations in the same order as the reference. Needs H % 1024 ==
// 0 and 16-byte aligned rows (else exact_logit_wave).
__device__ float exact_logit_lds(const float *__restrict__ xs, const float *__restrict__ w, int H,
                                 float (*buf)[1024]) {
  const int lane = threadIdx.x & 63;
  if ((H & 1023) || ((reinterpret_cast<uintptr_t>(xs) | reinterpret_cast<uintptr_t>(w)) & 15))
    return exact_logit_wave(xs, w, H);
  const float4 *x4 = reinterpret_cast<const float4 *>(xs);
  const float4 *w4 = reinterpret_cast<const float4 *>(w);
  const int nb = H >> 10;
  float4 xa[4], wa[4];
  auto fetch = [&](int b) {
#pragma unroll
    for (int j = 0; j < 4; j++) {
      xa[j] = x4[256 * b + 64 * j + lane];
      wa[j] = w4[256 * b + 64 * j + lane];
    }
  };
  auto put = [&](int b) {
    float4 *d = reinterpret_cast<float4 *>(buf[b & 1]);
#pragma unroll
    for (int j = 0; j < 4; j++)
      d[64 * j + lane] = make_float4(__fmul_rn(xa[j].x, wa[j].x), __fmul_rn(xa[j].y, wa[j].y),
                                     __fmul_rn(xa[j].z, wa[j].z), __fmul_rn(xa[j].w, wa[j].w));
  };
  fetch(0);
  put(0);
  if (nb > 1) fetch(1);
  float acc = -0.0f;
  for (int b = 0; b < nb; b++) {
    if (lane == 0) {
      const float4 *pb = reinterpret_cast<const float4 *>(buf[b & 1]);
      float4 a[8], c[8];
#pragma unroll
      for (int u = 0; u < 8; u++) a[u] = pb[u];
      for (int i = 0; i < 256; i += 16) {
#pragma unroll
        for (int u = 0; u < 8; u++) c[u] = pb[i + 8 + u];
#pragma unroll
        for (int u = 0; u < 8; u++) {
          acc = __fadd_rn(acc, a[u].x);
          acc = __fadd_rn(acc, a[u].y);
          acc = __fadd_rn(acc, a[u].z);
          acc = __fadd_rn(acc, a[u].w);
        }
        const int jn = (i + 16) & 255;  // past the block: wraps to its start (read, unused)
#pragma unroll
        for (int u = 0; u < 8; u++) a[u] = pb[jn + u];
#pragma unroll
        for (int u = 0; u < 8; u++) {
          acc = __fadd_rn(acc, c[u].x);
          acc = __fadd_rn(acc, c[u].y);
          acc = __fadd_rn(acc, c[u].z);
          acc = __fadd_rn(acc, c[u].w);
        }
      }
    }
    if (b + 1 < nb) {
      put(b + 1);
      if (b + 2 < nb) fetch(b + 2);
    }
  }
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(acc), 0));
}

// ------------------------------------------------------------------------------------------------
// Selection helpers: order-preserving key bits (0 is left for "no expert"), lane masks, and the
// one-token job-table outputs.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t ord_key(float f) {
  const uint32_t b = __float_as_uint(f + 0.0f);  // -0 -> +0: equal keys compare equal
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

__device__ __forceinline__ unsigned long long lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return (lane == 0) ? 0ull : (~0ull >> (64 - lane));
}

struct GroupOut {
  const RbtExpertDev *table;
  const RbtExpertDev *shared_dev;
  RbtExpertDev *pair_job;
  int *pair_tok, *tok_pair;
  float *tok_w;
  int *err;
  RbtExpertDev *down_job;  // optional (one token): winners in slot order, then the shared expert
  int *down_slot;          // their pair slots
  int shared_slot;         // pair slot of the shared expert
};

__host__ __device__ inline GroupOut group_out(const GroupArgs &g, int k) {
  return GroupOut{g.table,    g.shared_dev, g.pair_job, g.pair_tok, g.tok_pair,
                  g.tok_w,    g.err,        g.down_job, g.down_slot, g.shared_slot >= 0 ? g.shared_slot : k};
}

// Copy of a job-table entry field by field (a struct temporary ends up in scratch memory).
__device__ __forceinline__ void copy_job(RbtExpertDev *dst, const RbtExpertDev *src) {
  const uint8_t *gd = src->gd, *ud = src->ud, *dd = src->dd;
  const void *gs = src->gs, *us = src->us, *ds = src->ds;
  dst->gd = gd;
  dst->gs = gs;
  dst->ud = ud;
  dst->us = us;
  dst->dd = dd;
  dst->ds = ds;
}

// ------------------------------------------------------------------------------------------------
// Selection v3 (n_group <= 1), one workgroup of 256 threads per token; wave 0 selects, all four
// waves recompute ambiguous logits exactly.
//  * Keys: expert e = lane + 64 m of wave 0 holds its key interval [klo, khi] (logit interval through
//    the family's monotone key map) and the order-preserving bits of its midpoint key (0 = no
//    expert, so no validity masks are needed in the hot loop).
//  * Top-k: the candidates are the keys at or above the kk-th largest of the 64 lane maxima (found
//    by bisection over 32 key bits with one ballot per bit); at least kk keys reach it, so every
//    winner is a candidate. The candidates (usually a few more than kk) are ranked by midpoint key
//    desc, id asc, as the reference's strict-> scans order them (qwen38/moe.rs:48-58,
//    glm52/moe.rs:170-186), and the first kk win. More than 64 candidates (many equal keys) fall
//    back to a bisection for the kk-th largest key over all keys with the same tie rule.
//  * Certification, in registers: the set is certain when every inexact winner's lower key is
//    above every loser's upper key and every inexact loser's upper key is below every winner's lower
//    key (wave min / max); the order is certain when every pair of winners has disjoint intervals
//    or is a pair of exact values. Intervals that fail are recomputed as the reference computes
//    them (exact_logit_wave) and become points; the selection then repeats until nothing is
//    ambiguous (checking every pair makes one recomputation pass enough in practice).
//  * The winners' job-table entries are loaded by their candidate lanes while the selection is
//    certified and written in rank order at the end.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ float wave_min_f(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fminf(v, __shfl_xor(v, d, 64));
  return v;
}
__device__ __forceinline__ float wave_max_f(float v) {
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
  return v;
}

// LDS of the selection (one token per workgroup).
struct SelLds {
  int c_id[SEL_MAXK];  // winners in id order (bisection path)
  uint32_t c_ku[SEL_MAXK];
  float c_lo[SEL_MAXK], c_hi[SEL_MAXK], c_l[SEL_MAXK];
  int r_id[SEL_MAXK];  // winners in rank order
  float r_l[SEL_MAXK], r_lo[SEL_MAXK], r_hi[SEL_MAXK];
  float s_w[SEL_MAXK];
  // every expert once for set membership, plus at most two per adjacent winner pair for order
  int amb[SEL_MAXE + 2 * SEL_MAXK];
  float amb_val[SEL_MAXE + 2 * SEL_MAXK];
  int namb;
  int q_id[SEL_NC];  // candidates (fast path)
  uint32_t q_ku[SEL_NC];
  float q_lo[SEL_NC], q_hi[SEL_NC], q_l[SEL_NC];
};

// Routing weights of the kk winners (L.r_id, L.r_l in rank order) into L.s_w, by wave 0: computed
// by the lanes in parallel, the sums in rank order.
__device__ __forceinline__ void winner_weights(SelLds &L, const SelParams &P, int kk) {
  const int lane = threadIdx.x & 63;
  float lv = 0.0f;
  if (lane < kk) {
    const int e = L.r_id[lane];
    lv = P.logit_bias ? __fadd_rn(L.r_l[lane], P.logit_bias[e]) : L.r_l[lane];
  }
  if (P.family == RBT_FAMILY_QWEN38) {
    // qwen38/moe.rs:66-74: softmax over the winners' logits, max-subtracted.
    const float mx = __shfl(lv, 0, 64);
    if (lane < kk) L.s_w[lane] = (float)exp((double)__fsub_rn(lv, mx));
    __builtin_amdgcn_wave_barrier();
    float sum = 0.0f;
    for (int r = 0; r < kk; r++) sum = __fadd_rn(sum, L.s_w[r]);
    if (lane < kk) L.s_w[lane] = __fdiv_rn(L.s_w[lane], sum);
  } else {
    // glm52/moe.rs:231-241: weight = plain sigmoid; norm_topk; routed_scale.
    if (lane < kk) L.s_w[lane] = sigmoid_ref(lv);
    __builtin_amdgcn_wave_barrier();
    if (P.norm_topk) {
      float sum = -0.0f;
      for (int r = 0; r < kk; r++) sum = __fadd_rn(sum, L.s_w[r]);
      sum = __fadd_rn(sum, 1e-20f);
      if (lane < kk) L.s_w[lane] = __fdiv_rn(L.s_w[lane], sum);
    }
    if (lane < kk) L.s_w[lane] = __fmul_rn(L.s_w[lane], P.routed_scale);
  }
  __builtin_amdgcn_wave_barrier();
}

// Selection keys of one expert from its logit interval: key at the clamped midpoint (kmid, and its
// order key ku), and the interval of keys [klo, khi] (a point when the logit interval is).
__device__ __forceinline__ void sel_keys(const SelParams &P, double mv, double bv, float lb, float rb, float &lmid,
                                         uint32_t &ku, float &klo, float &khi) {
  const float lo = __double2float_rd(mv - bv * (1.0 + 1e-12));
  const float hi = __double2float_ru(mv + bv * (1.0 + 1e-12));
  const float md = fminf(fmaxf(__double2float_rn(mv), lo), hi);
  lmid = md;
  const float kmid = sel_key_v(P, lb, rb, md);
  ku = ord_key(kmid);
  if (lo == hi) {
    klo = khi = kmid;
  } else {
    klo = sel_key_v(P, lb, rb, lo);
    khi = sel_key_v(P, lb, rb, hi);
  }
}

// MW: the keys of all experts are computed by the four waves together (for the sigmoid families
// each key costs three fp64-exp sigmoids) and handed to wave 0 through kbuf, LDS of 4 * 64 * MAXM
// words; otherwise wave 0 computes them alone and kbuf is unused.
template <int MAXM, bool MW = false>
__device__ __forceinline__ void select3_body(SelLds &L, const SelParams &P, const double *__restrict__ mid,
                                             const double *__restrict__ bnd, int32_t *__restrict__ ids,
                                             float *__restrict__ wts, float *__restrict__ sh_scale,
                                             int *__restrict__ stats, const GroupOut &G, int grp, int s,
                                             float *kbuf = nullptr) {
  int(&c_id)[SEL_MAXK] = L.c_id;
  uint32_t(&c_ku)[SEL_MAXK] = L.c_ku;
  float(&c_lo)[SEL_MAXK] = L.c_lo, (&c_hi)[SEL_MAXK] = L.c_hi, (&c_l)[SEL_MAXK] = L.c_l;
  int(&r_id)[SEL_MAXK] = L.r_id;
  float(&r_l)[SEL_MAXK] = L.r_l, (&r_lo)[SEL_MAXK] = L.r_lo, (&r_hi)[SEL_MAXK] = L.r_hi;
  float(&s_w)[SEL_MAXK] = L.s_w;
  int(&amb)[SEL_MAXE + 2 * SEL_MAXK] = L.amb;
  float(&amb_val)[SEL_MAXE + 2 * SEL_MAXK] = L.amb_val;
  int &namb = L.namb;
  int(&q_id)[SEL_NC] = L.q_id;
  uint32_t(&q_ku)[SEL_NC] = L.q_ku;
  float(&q_lo)[SEL_NC] = L.q_lo, (&q_hi)[SEL_NC] = L.q_hi, (&q_l)[SEL_NC] = L.q_l;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int E = P.E, k = P.k, kk = min(P.k, P.E);
  const double *ms = mid + (size_t)s * P.erows;
  const double *bs = bnd + (size_t)s * P.erows;

  float klo[MAXM], khi[MAXM], lmid[MAXM], lbv[MAXM], rbv[MAXM];
  uint32_t ku[MAXM];
  if (MW) {
    constexpr int MQ = (MAXM + 3) / 4, NE = 64 * MAXM;
    {
      double mv[MQ], bv[MQ];
      float lb[MQ], rb[MQ];
#pragma unroll
      for (int i = 0; i < MQ; i++) {
        const int e = min(lane + 64 * (wave + 4 * i), E - 1);  // unconditional (in-bounds) loads batch together
        mv[i] = ms[e];
        bv[i] = bs[e];
        lb[i] = P.logit_bias ? P.logit_bias[e] : 0.0f;
        rb[i] = P.router_bias ? P.router_bias[e] : 0.0f;
      }
#pragma unroll
      for (int i = 0; i < MQ; i++) {
        const int e = lane + 64 * (wave + 4 * i);
        if (wave + 4 * i < MAXM && e < E) {
          float lm, kl, kh;
          uint32_t u;
          sel_keys(P, mv[i], bv[i], lb[i], rb[i], lm, u, kl, kh);
          kbuf[e] = kl;
          kbuf[NE + e] = kh;
          kbuf[2 * NE + e] = lm;
          kbuf[3 * NE + e] = __uint_as_float(u);
          kbuf[4 * NE + e] = lb[i];  // the biases too: wave 0 reads them from LDS, not memory again
          kbuf[5 * NE + e] = rb[i];
        }
      }
    }
    __syncthreads();
    if (wave == 0) {
#pragma unroll
      for (int m = 0; m < MAXM; m++) {
        const int e = min(lane + 64 * m, E - 1);
        lbv[m] = kbuf[4 * NE + e];
        rbv[m] = kbuf[5 * NE + e];
        const bool in = lane + 64 * m < E;
        ku[m] = in ? __float_as_uint(kbuf[3 * NE + e]) : 0u;
        klo[m] = in ? kbuf[e] : -INFINITY;
        khi[m] = in ? kbuf[NE + e] : -INFINITY;
        lmid[m] = in ? kbuf[2 * NE + e] : -INFINITY;
      }
    }
  } else if (wave == 0) {
    double mv[MAXM], bv[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; m++) {
      const int e = min(lane + 64 * m, E - 1);  // unconditional (in-bounds) loads batch together
      mv[m] = ms[e];
      bv[m] = bs[e];
      lbv[m] = P.logit_bias ? P.logit_bias[e] : 0.0f;
      rbv[m] = P.router_bias ? P.router_bias[e] : 0.0f;
    }
#pragma unroll
    for (int m = 0; m < MAXM; m++) {
      ku[m] = 0;
      klo[m] = khi[m] = lmid[m] = -INFINITY;
      if (lane + 64 * m < E) sel_keys(P, mv[m], bv[m], lbv[m], rbv[m], lmid[m], ku[m], klo[m], khi[m]);
    }
  }
  int total_amb = 0;
  // fast path state of the last pass: the lane's candidate, its rank and its job-table entry
  bool fast = false;
  int my_rank = -1, my_id = 0;
  const uint8_t *pf_gd = nullptr, *pf_ud = nullptr, *pf_dd = nullptr;
  const void *pf_gs = nullptr, *pf_us = nullptr, *pf_ds = nullptr;
  for (;;) {
    if (wave == 0) {
      // Candidates: the keys at or above M, the kk-th largest of the 64 lane maxima. The maxima of
      // kk lanes reach M, so at least kk keys do and the kk winners are all candidates; usually
      // only a few more than kk keys qualify.
      uint32_t lmax = 0;
#pragma unroll
      for (int m = 0; m < MAXM; m++) lmax = max(lmax, ku[m]);
      uint32_t M = 0;
#pragma unroll 1
      for (int bit = 31; bit >= 0; bit--) {
        const uint32_t cand = M | (1u << bit);
        M = __popcll(__ballot(lmax >= cand)) >= kk ? cand : M;
      }
      int nc = 0;
#pragma unroll
      for (int m = 0; m < MAXM; m++) nc += __popcll(__ballot(ku[m] >= M));
      fast = nc <= SEL_NC && M != 0;  // M = 0 only if some key maps to 0 (a NaN): bisection path
      if (fast) {
        uint32_t cm = 0;
        int base = 0;
#pragma unroll
        for (int m = 0; m < MAXM; m++) {
          const bool c = ku[m] >= M;
          const unsigned long long cb = __ballot(c);
          if (c) {
            const int at = base + __popcll(cb & lanemask_lt());
            q_id[at] = lane + 64 * m;
            q_ku[at] = ku[m];
            q_lo[at] = klo[m];
            q_hi[at] = khi[m];
            q_l[at] = lmid[m];
            cm |= 1u << m;
          }
          base += __popcll(cb);
        }
        float hi_out = -INFINITY;  // upper keys of the non-candidates (never winners)
#pragma unroll
        for (int m = 0; m < MAXM; m++)
          if (!((cm >> m) & 1u) && ku[m] != 0) hi_out = fmaxf(hi_out, khi[m]);
        __builtin_amdgcn_wave_barrier();
        // rank of candidate `lane` among the candidates: key desc, id asc
        float clo = INFINITY, chi = -INFINITY, cl = 0.0f;
        my_rank = -1;
        if (lane < nc) {
          const uint32_t my = q_ku[lane];
          my_id = q_id[lane];
          clo = q_lo[lane];
          chi = q_hi[lane];
          cl = q_l[lane];
          int rank = 0, j = 0;
          for (; j + 8 <= nc; j += 8) {  // eight candidates' LDS reads in flight at once
            uint32_t o[8];
            int oi[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
              o[u] = q_ku[j + u];
              oi[u] = q_id[j + u];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) rank += (o[u] > my) || (o[u] == my && oi[u] < my_id);
          }
          for (; j < nc; j++) {
            const uint32_t o = q_ku[j];
            rank += (o > my) || (o == my && q_id[j] < my_id);
          }
          my_rank = rank;
          if (grp) {  // the job-table entry, in flight while the selection is certified
            const RbtExpertDev *src = G.table + my_id;
            pf_gd = src->gd;
            pf_gs = src->gs;
            pf_ud = src->ud;
            pf_us = src->us;
            pf_dd = src->dd;
            pf_ds = src->ds;
          }
        }
        const bool iw = my_rank >= 0 && my_rank < kk;
        const float lo_sel = wave_min_f(iw ? clo : INFINITY);
        const float hi_uns = wave_max_f(fmaxf(hi_out, (lane < nc && !iw) ? chi : -INFINITY));
        if (iw) {
          r_id[my_rank] = my_id;
          r_l[my_rank] = cl;
          r_lo[my_rank] = clo;
          r_hi[my_rank] = chi;
        }
        if (lane == 0) namb = 0;
        __builtin_amdgcn_wave_barrier();
        // set membership: inexact experts on the wrong side of the other side's bound
#pragma unroll
        for (int m = 0; m < MAXM; m++)
          if (!((cm >> m) & 1u) && ku[m] != 0 && klo[m] != khi[m] && khi[m] >= lo_sel)
            amb[atomicAdd(&namb, 1)] = lane + 64 * m;
        const bool cexact = clo == chi;
        bool amb_me = lane < nc && !cexact && (iw ? clo <= hi_uns : chi >= lo_sel);
        // order: every pair of winners must be strictly ordered or an exact tie-broken pair (checking
        // all pairs, not only neighbours, keeps one recomputation pass enough)
        if (iw && !cexact) {
          int q = 0;
          for (; q + 8 <= kk; q += 8) {  // eight winners' LDS reads in flight at once
            float ql[8], qh[8];
#pragma unroll
            for (int u = 0; u < 8; u++) {
              ql[u] = r_lo[q + u];
              qh[u] = r_hi[q + u];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
              const int qq = q + u;
              const bool sure = qq < my_rank ? ql[u] > chi : (qq > my_rank ? clo > qh[u] : true);
              amb_me |= !sure;
            }
          }
          for (; q < kk; q++) {
            const float ql = r_lo[q], qh = r_hi[q];
            const bool sure = q < my_rank ? ql > chi : (q > my_rank ? clo > qh : true);
            amb_me |= !sure;
          }
        }
        if (amb_me) amb[atomicAdd(&namb, 1)] = my_id;
      } else {
        // k-th largest midpoint key
        uint32_t T = 0;
  #pragma unroll 1
        for (int bit = 31; bit >= 0; bit--) {
          const uint32_t cand = T | (1u << bit);
          int cnt = 0;
#pragma unroll
          for (int m = 0; m < MAXM; m++) cnt += __popcll(__ballot(ku[m] >= cand));
          T = cnt >= kk ? cand : T;
        }
        int ngt = 0;
#pragma unroll
        for (int m = 0; m < MAXM; m++) ngt += __popcll(__ballot(ku[m] > T));
        const int need = kk - ngt;
        uint32_t win = 0;
        int taken_eq = 0, base = 0;
        float lo_sel = INFINITY, hi_uns = -INFINITY;
#pragma unroll
        for (int m = 0; m < MAXM; m++) {
          const unsigned long long eq = __ballot(ku[m] == T);
          const bool weq = ku[m] == T && (taken_eq + __popcll(eq & lanemask_lt())) < need;
          taken_eq += __popcll(eq);
          const bool w = ku[m] > T || weq;
          const unsigned long long wm = __ballot(w);
          if (w) {
            const int at = base + __popcll(wm & lanemask_lt());
            c_id[at] = lane + 64 * m;
            c_ku[at] = ku[m];
            c_lo[at] = klo[m];
            c_hi[at] = khi[m];
            c_l[at] = lmid[m];
            win |= 1u << m;
            lo_sel = fminf(lo_sel, klo[m]);
          } else if (ku[m] != 0) {
            hi_uns = fmaxf(hi_uns, khi[m]);
          }
          base += __popcll(wm);
        }
        lo_sel = wave_min_f(lo_sel);
        hi_uns = wave_max_f(hi_uns);
        if (lane == 0) namb = 0;
        __builtin_amdgcn_wave_barrier();
        // set membership: inexact experts on the wrong side of the other side's bound
#pragma unroll
        for (int m = 0; m < MAXM; m++) {
          const bool inexact = ku[m] != 0 && klo[m] != khi[m];
          const bool a = inexact && (((win >> m) & 1u) ? klo[m] <= hi_uns : khi[m] >= lo_sel);
          if (a) amb[atomicAdd(&namb, 1)] = lane + 64 * m;
        }
        // order: rank the winners by midpoint (key desc, id asc), then check adjacent intervals
        if (lane < kk) {
          const uint32_t my = c_ku[lane];
          const int id = c_id[lane];
          int rank = 0;
          for (int j = 0; j < kk; j++) {
            const uint32_t o = c_ku[j];
            rank += (o > my) || (o == my && c_id[j] < id);
          }
          r_id[rank] = id;
          r_l[rank] = c_l[lane];
          r_lo[rank] = c_lo[lane];
          r_hi[rank] = c_hi[lane];
        }
        __builtin_amdgcn_wave_barrier();
        if (lane + 1 < kk) {
          const bool ea = r_lo[lane] == r_hi[lane], eb = r_lo[lane + 1] == r_hi[lane + 1];
          if (!(r_lo[lane] > r_hi[lane + 1]) && !(ea && eb)) {
            // a winner already counted for set membership may be added twice: harmless
            if (!ea) amb[atomicAdd(&namb, 1)] = r_id[lane];
            if (!eb) amb[atomicAdd(&namb, 1)] = r_id[lane + 1];
          }
        }
      }
    }
    __syncthreads();
    const int na = namb;
    if (na == 0) break;
    total_amb += na;
    for (int j = wave; j < na; j += 4) {
      const float l = exact_logit_wave(P.x + (size_t)s * P.H, P.W + (size_t)amb[j] * P.H, P.H);
      if (lane == 0) amb_val[j] = l;
    }
    __syncthreads();
    if (wave == 0) {
      for (int j = 0; j < na; j++) {
        const int e = amb[j];
        if ((e & 63) == lane) {
          const int mm = e >> 6;
          const float l = amb_val[j];
#pragma unroll
          for (int m = 0; m < MAXM; m++)
            if (m == mm) {
              const float key = sel_key_v(P, lbv[m], rbv[m], l);
              lmid[m] = l;
              klo[m] = khi[m] = key;
              ku[m] = ord_key(key);
            }
        }
      }
    }
    __syncthreads();
  }
  if (wave == 0) {
    if (lane == 0 && stats && total_amb) atomicAdd(stats, total_amb);
    winner_weights(L, P, kk);
    int32_t *io = ids + (size_t)s * k;
    float *wo = wts + (size_t)s * k;
    for (int r = lane; r < k; r += 64) {
      io[r] = r < kk ? r_id[r] : -1;
      wo[r] = r < kk ? s_w[r] : 0.0f;
    }
    if (lane == 0 && sh_scale) sh_scale[s] = (P.erows > E) ? sigmoid_ref(__double2float_rn(ms[E])) : 1.0f;
    if (grp) {
      // single token: pair j = slot j; the shared expert is at G.shared_slot
      auto put = [&](int r, const uint8_t *gd, const void *gs, const uint8_t *ud, const void *us, const uint8_t *dd,
                     const void *ds) {
        RbtExpertDev *dst = G.pair_job + r;
        dst->gd = gd;
        dst->gs = gs;
        dst->ud = ud;
        dst->us = us;
        dst->dd = dd;
        dst->ds = ds;
        if (G.down_job && r < kk) {
          RbtExpertDev *dn = G.down_job + r;
          dn->gd = gd;
          dn->gs = gs;
          dn->ud = ud;
          dn->us = us;
          dn->dd = dd;
          dn->ds = ds;
          G.down_slot[r] = r;
        }
      };
      if (fast && my_rank >= 0 && my_rank < kk) {
        // winners of the fast path: the entries their candidate lanes loaded during certification
        if (pf_gd == nullptr || pf_dd == nullptr) atomicOr(G.err, 1);
        put(my_rank, pf_gd, pf_gs, pf_ud, pf_us, pf_dd, pf_ds);
      }
      for (int r = lane; r <= k; r += 64) {
        if (r < k) {
          if (!fast || r >= kk) {
            const RbtExpertDev *src = G.table + (r < kk ? r_id[r] : 0);
            const bool use = r < kk;
            const uint8_t *gd = use ? src->gd : nullptr, *ud = use ? src->ud : nullptr;
            const uint8_t *dd = use ? src->dd : nullptr;
            const void *gs = use ? src->gs : nullptr, *us = use ? src->us : nullptr;
            const void *ds = use ? src->ds : nullptr;
            if (use && (gd == nullptr || dd == nullptr)) atomicOr(G.err, 1);
            put(r, gd, gs, ud, us, dd, ds);
          }
          G.pair_tok[r] = 0;
          G.tok_pair[r] = r < kk ? r : -1;
          G.tok_w[r] = r < kk ? s_w[r] : 0.0f;
        } else {
          copy_job(G.pair_job + G.shared_slot, G.shared_dev);
          if (G.shared_slot == k) G.pair_tok[k] = 0;
          if (G.down_job) {
            copy_job(G.down_job + kk, G.shared_dev);
            G.down_slot[kk] = G.shared_slot;
          }
        }
      }
    }
  }
}

template <int MAXM>
__global__ __launch_bounds__(256) void k_router_select3(SelParams P, const double *__restrict__ mid,
                                                        const double *__restrict__ bnd, int32_t *__restrict__ ids,
                                                        float *__restrict__ wts, float *__restrict__ sh_scale,
                                                        int *__restrict__ stats, GroupOut G, int grp) {
  __shared__ SelLds L;
  __shared__ float kbuf[6 * 64 * MAXM];
  select3_body<MAXM, true>(L, P, mid, bnd, ids, wts, sh_scale, stats, G, grp, blockIdx.x, kbuf);
}

// One token with a shared expert: workgroup 0 selects; the other workgroups stream the shared
// expert's gate/up (it does not depend on the routing) on the CUs the selection leaves idle.
template <int MAXM, int NCH>
__global__ __launch_bounds__(256) void k_router_select3_sh(SelParams P, const double *__restrict__ mid,
                                                           const double *__restrict__ bnd, int32_t *__restrict__ ids,
                                                           float *__restrict__ wts, float *__restrict__ sh_scale,
                                                           int *__restrict__ stats, GroupOut G, int grp,
                                                           const RbtExpertDev *__restrict__ shared_dev,
                                                           const float *__restrict__ x, int I,
                                                           __bf16 *__restrict__ hp_shared) {
  __shared__ union {
    SelLds sel;
    GuLds gu;
  } L;
  if (blockIdx.x == 0)
    select3_body<MAXM>(L.sel, P, mid, bnd, ids, wts, sh_scale, stats, G, grp, 0);
  else
    xgateup1_body<NCH>(L.gu, shared_dev, 1, x, I, hp_shared, blockIdx.x - 1, gridDim.x - 1);
}

// One token of the latent MoE: workgroup 0 selects (writing the pair list); the other workgroups,
// one per CU, run the latent down projection x_latent = down_proj . x (kimi_k3/moe.rs:64-80) as the
// decode GEMV does, since it does not depend on the routing: it streams while the selection (and
// any exact fold it needs) runs.
template <int MAXM, int NB, bool I4G>
__global__ __launch_bounds__(256) void k_router_select3_dp(SelParams P, const double *__restrict__ mid,
                                                           const double *__restrict__ bnd, int32_t *__restrict__ ids,
                                                           float *__restrict__ wts, float *__restrict__ sh_scale,
                                                           int *__restrict__ stats, GroupOut G, RbtExpertDev proj,
                                                           int cols, int rows, float *__restrict__ xl) {
  __shared__ SelLds L;
  __shared__ float kbuf[6 * 64 * MAXM];
  if (blockIdx.x == 0)
    select3_body<MAXM, true>(L, P, mid, bnd, ids, wts, sh_scale, stats, G, 1, 0, kbuf);
  else
    decode_gemv_body<NB, 64, 1, MODE_DOWN, I4G, 1, 1>(nullptr, proj, 1, nullptr, P.x, nullptr, 0, cols, rows, xl, 0,
                                                      nullptr, 0.0f, (blockIdx.x - 1) * 4 + (threadIdx.x >> 6),
                                                      (gridDim.x - 1) * 4);
}

// Routing from precomputed logits (rbt_route_*_topk): the logits are exact inputs, so the
// interval is a point (bound 0) and the same selection code applies.
__global__ void k_logits_to_mid(const float *__restrict__ logits, size_t n, double *__restrict__ mid,
                                double *__restrict__ bnd) {
  size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) {
    mid[i] = (double)logits[i];
    bnd[i] = 0.0;
  }
}

// ------------------------------------------------------------------------------------------------
// 3. grouping: pairs (token, slot) ordered by (unique_experts position, token).
//   pair_job[p]   -> expert device view (table lookup), or the shared expert for p >= S*k
//   pair_tok[p]   -> token index
//   tok_pair[t*k + j] -> the t-th token's pairs sorted by unique_experts position
//   tok_w[t*k + j]    -> matching routing weight
// One workgroup; thread e handles expert e. The picks (ids, weights) and the per-token pair lists
// are kept in LDS when they fit (stage != 0): every expert's thread walks all the picks, and the
// per-token sort is a chain of dependent accesses, each a memory round trip in global memory.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void k_group(const int32_t *__restrict__ ids, const float *__restrict__ wts, int S,
                                                int k, int E, const RbtExpertDev *__restrict__ table,
                                                const RbtExpertDev *__restrict__ shared_dev, RbtExpertDev *pair_job,
                                                int *pair_tok, int *tok_pair, float *tok_w, int *err, int *nuniq,
                                                int stage) {
  extern __shared__ int smem[];
  __shared__ int uniq;
  int *first = smem;       // [E]
  int *cnt = smem + E;     // [E]
  int *off = smem + 2 * E; // [E]
  const int P = S * k;
  // staged: the picks and the per-token pair lists live in LDS ([P] each)
  int *sid = smem + 3 * E;
  float *swt = reinterpret_cast<float *>(smem + 3 * E + P);
  int *stp = smem + 3 * E + 2 * P;
  float *stw = reinterpret_cast<float *>(smem + 3 * E + 3 * P);
  const int32_t *pid = stage ? sid : ids;
  const float *pwt = stage ? swt : wts;
  int *tp_all = stage ? stp : tok_pair;
  float *tw_all = stage ? stw : tok_w;
  if (threadIdx.x == 0) uniq = 0;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    first[e] = 0x7fffffff;
    cnt[e] = 0;
  }
  // Slots without a pick (grouped routing can select fewer than k) stay empty: null job, no pair.
  for (int p = threadIdx.x; p < P; p += blockDim.x) {
    if (stage) {
      sid[p] = ids[p];
      swt[p] = wts[p];
    }
    pair_job[p] = RbtExpertDev{};
    pair_tok[p] = 0;
    tp_all[p] = -1;
    tw_all[p] = 0.0f;
  }
  __syncthreads();
  for (int p = threadIdx.x; p < P; p += blockDim.x) {
    int e = pid[p];
    if (e >= 0 && e < E) {
      atomicMin(&first[e], p);
      atomicAdd(&cnt[e], 1);
    }
  }
  __syncthreads();
  // off[e]: the picks of the experts first picked before e -- an exclusive prefix sum over the picks
  // in order of cnt[e] at each expert's first pick (chunks of 1024 picks, wave scans and a carry)
  __shared__ int wsum[16], carry;
  if (threadIdx.x == 0) carry = 0;
  __syncthreads();
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  for (int base = 0; base < P; base += 1024) {
    const int p = base + (int)threadIdx.x;
    int e = -1, v = 0;
    if (p < P) {
      e = pid[p];
      if (e >= 0 && e < E && first[e] == p) v = cnt[e];
    }
    int incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int o = __shfl_up(incl, d, 64);
      if (lane >= d) incl += o;
    }
    if (lane == 63) wsum[wave] = incl;
    __syncthreads();
    int woff = carry, tot = 0;
    for (int w2 = 0; w2 < 16; w2++) {
      if (w2 < wave) woff += wsum[w2];
      tot += wsum[w2];
    }
    if (v) {
      off[e] = woff + incl - v;
      atomicAdd(&uniq, 1);
    }
    __syncthreads();
    if (threadIdx.x == 0) carry += tot;
    __syncthreads();
  }
  if (threadIdx.x == 0 && nuniq) *nuniq = uniq;
  for (int e = threadIdx.x; e < E; e += blockDim.x) {
    if (cnt[e] == 0) continue;
    int c = 0;
    RbtExpertDev J = table[e];
    if (J.gd == nullptr || J.dd == nullptr) atomicOr(err, 1);
    for (int q = first[e]; q < P; q++) {  // pairs in token order (q = t k + j), from the first pick
      if (pid[q] == e) {
        int p = off[e] + c++;
        pair_job[p] = J;
        pair_tok[p] = q / k;
        tp_all[q] = p;  // unsorted for now
        tw_all[q] = pwt[q];
      }
    }
  }
  __syncthreads();
  // shared-expert pairs, and per-token sort of the picks by pair index (= first-occurrence order)
  for (int t = threadIdx.x; t < S; t += blockDim.x) {
    pair_job[P + t] = *shared_dev;
    pair_tok[P + t] = t;
    int *tp = tp_all + t * k;
    float *tw = tw_all + t * k;
    for (int a = 1; a < k; a++) {
      int cp = tp[a];
      float cw = tw[a];
      int b = a;
      while (b > 0 && (unsigned)tp[b - 1] > (unsigned)cp) {
        tp[b] = tp[b - 1];
        tw[b] = tw[b - 1];
        b--;
      }
      tp[b] = cp;
      tw[b] = cw;
    }
  }
  if (stage) {
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
      tok_pair[p] = stp[p];
      tok_w[p] = stw[p];
    }
  }
}

// ------------------------------------------------------------------------------------------------
// combine: out[t, d] = sum over t's picks (unique_experts order) of w * y[pair, d], accumulated in
// fp32 with separate roundings (glm52/moe.rs:508-512), then + shared (qwen38/generate.rs:346-349)
// scaled by the token's shared gate (qwen38/generate.rs:316-322) when gated.
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_combine(const float *__restrict__ y, int S, int k, int H,
                                                 const int *__restrict__ tok_pair, const float *__restrict__ tok_w,
                                                 const float *__restrict__ sh_scale, int has_shared, int gated,
                                                 float *__restrict__ out) {
  size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (size_t)S * H) return;
  int t = (int)(idx / H), d = (int)(idx % H);
  float acc = 0.0f;
  // pairs in slot order, 16 at a time: the slots' pair ids and weights, then their rows, each
  // group of loads issued together (a pair-by-pair walk waits on two loads per pair)
  constexpr int CH = 16;
  for (int j0 = 0; j0 < k; j0 += CH) {
    int pp[CH];
    float ww[CH], vv[CH];
#pragma unroll
    for (int u = 0; u < CH; u++) {
      const int j = min(j0 + u, k - 1);
      pp[u] = tok_pair[t * k + j];
      ww[u] = tok_w[t * k + j];
    }
#pragma unroll
    for (int u = 0; u < CH; u++) vv[u] = y[(size_t)max(pp[u], 0) * H + d];
#pragma unroll
    for (int u = 0; u < CH; u++)
      if (j0 + u < k && pp[u] >= 0) acc = __fadd_rn(acc, __fmul_rn(ww[u], vv[u]));
  }
  if (has_shared) {
    float sh = y[((size_t)S * k + t) * H + d];
    if (gated) sh = __fmul_rn(sh, sh_scale[t]);
    acc = __fadd_rn(acc, sh);
  }
  out[idx] = acc;
}

// Single-token routing writes the grouping directly: pair j = slot j.
__global__ void k_group_s1(const int32_t *__restrict__ ids, const float *__restrict__ wts, int k, int E,
                           const RbtExpertDev *__restrict__ table, const RbtExpertDev *__restrict__ shared_dev,
                           RbtExpertDev *pair_job, int *pair_tok, int *tok_pair, float *tok_w, int *err) {
  int j = threadIdx.x;
  if (j < k) {
    int e = ids[j];
    RbtExpertDev J = {};
    if (e >= 0 && e < E) J = table[e];
    if (e >= 0 && (J.gd == nullptr || J.dd == nullptr)) atomicOr(err, 1);
    pair_job[j] = J;
    pair_tok[j] = 0;
    tok_pair[j] = e >= 0 ? j : -1;
    tok_w[j] = wts[j];
  } else if (j == k) {
    pair_job[k] = *shared_dev;
    pair_tok[k] = 0;
  }
}

// ------------------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_router_logits_tk(const float *__restrict__ x, int S, int H,
                                                          const float *__restrict__ W, int E,
                                                          const float *__restrict__ sgate, double *__restrict__ mid,
                                                          double *__restrict__ bnd, int erows);

hipError_t launch_router_logits(const Ctx &c, const float *x, int S, int H, const float *W, int E, const float *sgate,
                                double *mid, double *bnd) {
  int erows = E + (sgate ? 1 : 0);
  bool aligned = ((uintptr_t)x % 16 == 0) && ((uintptr_t)W % 16 == 0) && (!sgate || (uintptr_t)sgate % 16 == 0);
  if (H % 1024 == 0 && H <= RT_MAXH && aligned && S > 1)
    launch_k(c, k_router_logits_tk, dim3(erows, (S + 3) / 4), dim3(256), x, S, H, W, E, sgate, mid, bnd, erows);
  else if (H % 1024 == 0 && H <= RT_MAXH && aligned)
    launch_k(c, k_router_logits_b, dim3(erows), dim3(256), x, S, H, W, E, sgate, mid, bnd, erows);
  else if (H % 256 == 0 && H <= RT_MAXH && aligned)
    launch_k(c, k_router_logits_t, dim3(erows), dim3(64), x, S, H, W, E, sgate, mid, bnd, erows);
  else if (H % 256 == 0 && aligned)
    launch_k(c, k_router_logits_w, dim3((erows + 3) / 4), dim3(256), x, S, H, W, E, sgate, mid,
                       bnd, erows);
  else
    launch_k(c, k_router_logits, dim3(erows), dim3(256), x, S, H, W, E, sgate, mid, bnd, erows);
  return hipGetLastError();
}

bool router_exact_ok(int S, int H) { return S >= RX_EXACT_MIN_S && H % RX_KC == 0; }

hipError_t launch_router_logits_exact(const Ctx &c, const float *x, int S, int H, const float *W, int E,
                                      const float *sgate, float *logits) {
  const int erows = E + (sgate ? 1 : 0);
  if (H % RX_KC != 0 || ((uintptr_t)x | (uintptr_t)W | (uintptr_t)(sgate ? sgate : W)) % 16 != 0)
    return hipErrorInvalidValue;
  const dim3 grid((erows + RX_E - 1) / RX_E, (S + RX_T - 1) / RX_T);
  launch_k(c, k_router_logits_exact, grid, dim3(256), x, S, H, W, E, sgate, logits, erows);
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// Batched router logits on the matrix cores, certified (prefill batches). The selection needs, per
// (token, router row), a midpoint and a rigorous bound on its distance to the reference's
// sequential fp32 fold (kernels.rs:113-124); the ambiguous experts are then folded exactly by the
// selection itself. Here, per 32-column step of a (token, row) pair:
//   the products run on v_mfma_f32_16x16x4_f32 in two chains of four (columns 8 g + q and
//   8 g + 4 + q of lane group g), restarted every step; the chains' sum joins an fp64 sum;
//   sum |x| |w| accumulates over the steps on v_mfma_f32_16x16x32_bf16 from |x| and |w| cut to
//   bf16 (the same 32 columns, each lane's eight in its natural slot);
//   the prefix bound collects |sum after the step|: each partial sum S_i of a step lies within
//   min(|start| + P_<=i, |end| + P_>i) <= (|start| + |end| + P) / 2 of zero (P the step's
//   sum |x| |w|), so the step's 32 sums total at most 16 (|start| + |end|) + 16 P, and over a part
//   at most 32 sum_steps |end| + 16 sum |x| |w|.
// Error model of the matrix cores (addends aligned to the largest and truncated, then one rounding:
// at most 11 u; measured on MI355X at most 2 u, u = 2^-24): one MFMA output is within
// 16 u (sum |products| + |accumulator|) of the exact value, so a chain of four is within 64 u of its
// step's sum |x| |w|; the bf16 magnitude chain of 32 steps reads at least (1 - 64 u)^33 of its
// exact value; cutting to bf16 loses less than 2^-7 of a value.
// The reference's fold error is at most u T / (1 - n u), T the sum of its partial sums' magnitudes;
// its products' rounding is at most u sum |x| |w|.
// ------------------------------------------------------------------------------------------------
constexpr int RB_STEP = 32;  // columns per step
constexpr int RB_WGT = 64;   // tokens and rows per workgroup (four waves of 32 x 32)

struct RbRec {  // one K part of one (token, row): sum, prefix-magnitude sum, sum |xh| |wh|
  double s;
  float t, a;
};

typedef float rbf4 __attribute__((ext_vector_type(4)));
typedef __bf16 rbh8 __attribute__((ext_vector_type(8)));

// |v| cut to bf16 (toward zero), eight values: the high halves of each pair, sign bits cleared
__device__ __forceinline__ rbh8 rb_abs8(rbf4 lo, rbf4 hi) {
  uint4 u;
  u.x = __builtin_amdgcn_perm(__float_as_uint(lo[1]), __float_as_uint(lo[0]), 0x07060302u) & 0x7fff7fffu;
  u.y = __builtin_amdgcn_perm(__float_as_uint(lo[3]), __float_as_uint(lo[2]), 0x07060302u) & 0x7fff7fffu;
  u.z = __builtin_amdgcn_perm(__float_as_uint(hi[1]), __float_as_uint(hi[0]), 0x07060302u) & 0x7fff7fffu;
  u.w = __builtin_amdgcn_perm(__float_as_uint(hi[3]), __float_as_uint(hi[2]), 0x07060302u) & 0x7fff7fffu;
  return *reinterpret_cast<rbh8 *>(&u);
}

// One workgroup: 64 tokens x 64 rows over the columns of K part z (H / ks of them); wave w takes
// tokens 32 (w >> 1) .. +31 and rows 32 (w & 1) .. +31 as 2 x 2 tiles of 16 x 16. Workgroups are
// dealt to the eight XCDs in contiguous runs of (token tile, row tile, part) so that one XCD's
// workgroups share token tiles in its L2. Row E (with sgate) is the shared-expert gate vector; rows
// and tokens past the ends are computed on clamped inputs and not stored.
__global__ __launch_bounds__(256) void k_rcert(const float *__restrict__ x, int S, int H,
                                               const float *__restrict__ W, const float *__restrict__ sgate, int E,
                                               int erows, int n_t, int n_e, int ks, RbRec *__restrict__ out) {
  const int nwg = n_t * n_e * ks, run = (nwg + 7) / 8;
  const int L = (blockIdx.x & 7) * run + (blockIdx.x >> 3);
  if (L >= nwg) return;
  const int z = L % ks, et = (L / ks) % n_e, tt = L / (ks * n_e);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  const int t0 = tt * RB_WGT + 32 * (w >> 1), e0 = et * RB_WGT + 32 * (w & 1);
  const int kc = H / ks, k0 = z * kc;
  const float *xp[2], *wp[2];
#pragma unroll
  for (int j = 0; j < 2; j++) {
    xp[j] = x + (long)min(t0 + 16 * j + r, S - 1) * H + k0 + 8 * g;
    const int e = min(e0 + 16 * j + r, erows - 1);
    wp[j] = (e < E ? W + (long)e * H : sgate) + k0 + 8 * g;
  }
  // operands of one step: [token or row tile][columns 8 g .. +3, 8 g + 4 .. +7]
  rbf4 pa[2][2], pb[2][2], qa[2][2], qb[2][2];
  auto load = [&](rbf4 (&A)[2][2], rbf4 (&B)[2][2], int k) {
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int h = 0; h < 2; h++) {
        A[j][h] = *reinterpret_cast<const rbf4 *>(xp[j] + k + 4 * h);
        B[j][h] = *reinterpret_cast<const rbf4 *>(wp[j] + k + 4 * h);
      }
    __builtin_amdgcn_sched_barrier(0);  // keep the loads where they are issued: a full step ahead
  };
  double sd[2][2][4], td[2][2][4];
  rbf4 ab[2][2];
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int b = 0; b < 2; b++) {
      ab[a][b] = rbf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int i = 0; i < 4; i++) sd[a][b][i] = td[a][b][i] = 0.0;
    }
  auto step = [&](rbf4 (&A)[2][2], rbf4 (&B)[2][2]) {
    // opaque operands: the compiler may not reload them here (which would wait on the whole latency)
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
      for (int h = 0; h < 2; h++) asm volatile("" : "+v"(A[j][h]), "+v"(B[j][h]));
    rbh8 xa[2], wa[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      xa[j] = rb_abs8(A[j][0], A[j][1]);
      wa[j] = rb_abs8(B[j][0], B[j][1]);
    }
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
      for (int b = 0; b < 2; b++) {
        rbf4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = c0;
#pragma unroll
        for (int q = 0; q < 4; q++) {
          c0 = __builtin_amdgcn_mfma_f32_16x16x4f32(A[a][0][q], B[b][0][q], c0, 0, 0, 0);
          c1 = __builtin_amdgcn_mfma_f32_16x16x4f32(A[a][1][q], B[b][1][q], c1, 0, 0, 0);
        }
        ab[a][b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(xa[a], wa[b], ab[a][b], 0, 0, 0);
#pragma unroll
        for (int i = 0; i < 4; i++) {
          sd[a][b][i] += (double)(c0[i] + c1[i]);
          td[a][b][i] += fabs(sd[a][b][i]);
        }
      }
  };
  const int ns = kc / RB_STEP;  // even
  load(pa, pb, 0);
  for (int i = 0; i < ns; i += 2) {
    load(qa, qb, RB_STEP * (i + 1));
    step(pa, pb);
    load(pa, pb, RB_STEP * min(i + 2, ns - 2));  // past the end: a step again, unused
    step(qa, qb);
  }
#pragma unroll
  for (int a = 0; a < 2; a++)
#pragma unroll
    for (int b = 0; b < 2; b++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int t = t0 + 16 * a + 4 * g + i, e = e0 + 16 * b + r;
        if (t < S && e < erows) out[((long)z * S + t) * erows + e] = RbRec{sd[a][b][i], (float)td[a][b][i], ab[a][b][i]};
      }
}

// mid / bnd [S, erows] from the ks parts, joined in column order: A = sum |x| |w| bound, the prefix
// bound of a part shifted by the sum before it (and that sum's error), then the fold, product and
// midpoint errors.
__global__ __launch_bounds__(256) void k_rcomb(const RbRec *__restrict__ part, int S, int H, int erows, int ks,
                                               double *__restrict__ mid, double *__restrict__ bnd) {
  const long idx = (long)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (long)S * erows) return;
  const double u = 5.9604644775390625e-08, ub = 0.0078125, e64 = 1.1102230246251565e-16, n = (double)H;
  const double kc = n / ks, steps = kc / RB_STEP;
  // sum |xh| |wh| (cut values, 32-product MFMA chain over the steps) -> sum |x| |w|
  const double infl = 1.0 / ((1.0 - ub) * (1.0 - ub) * (1.0 - 64.0 * u * (steps + 1.0))) * (1.0 + 2.0 * u);
  const double per_mid = 64.01 * u + u * (1.0 + 64.01 * u);  // two chains of four, then their fp32 sum
  const double per = per_mid + u;                             // + the reference's product rounding
  double s = 0.0, T = 0.0, A = 0.0;
  for (int z = 0; z < ks; z++) {
    const RbRec o = part[(long)z * S * erows + idx];
    const double az = (double)o.a * infl;
    const double tz = RB_STEP * (double)o.t * (1.0 + 2.0 * u) + 0.5 * RB_STEP * az + kc * per * az;  // o.t >= 0
    T += tz + kc * (fabs(s) + per * A);
    s += o.s;
    A += az;
  }
  double B = u * T * (1.0 + 4.0 * u) / (1.0 - n * u) + per * A + 4.0 * n * e64 * A;
  B = B * (1.0 + 1e-9) + 1e-28;
  mid[idx] = s;
  bnd[idx] = B;
}

static int router_bounded_ks(const RouterArgs &a, int erows) {
  const long tiles = (long)((a.S + RB_WGT - 1) / RB_WGT) * ((erows + RB_WGT - 1) / RB_WGT);
  int ks = 8;
  while (ks > 1 && (tiles * 4 * (ks / 2) >= 2048 || a.H % (2 * RB_STEP * ks) != 0)) ks /= 2;
  return ks;
}

bool router_bounded_ok(const RouterArgs &a) {
  return a.S >= 1 && a.E >= 1 && a.H % (2 * RB_STEP) == 0 && a.H > 0 && a.n_group <= 1;
}

size_t router_bounded_scratch(const RouterArgs &a, int erows) {
  return (size_t)router_bounded_ks(a, erows) * a.S * erows * sizeof(RbRec);
}

hipError_t launch_router_bounded(const Ctx &c, const RouterArgs &a, const float *sgate, double *mid, double *bnd,
                                 void *scratch) {
  const int erows = a.E + (sgate ? 1 : 0);
  if (!router_bounded_ok(a)) return hipErrorInvalidValue;
  if (((uintptr_t)a.x | (uintptr_t)a.W | (uintptr_t)(sgate ? sgate : a.x)) % 16 != 0) return hipErrorInvalidValue;
  const int ks = router_bounded_ks(a, erows);
  const int n_t = (a.S + RB_WGT - 1) / RB_WGT, n_e = (erows + RB_WGT - 1) / RB_WGT;
  const int nwg = n_t * n_e * ks, run = (nwg + 7) / 8;
  RbRec *part = static_cast<RbRec *>(scratch);
  launch_k(c, k_rcert, dim3(8 * run), dim3(256), a.x, a.S, a.H, a.W, sgate, a.E, erows, n_t, n_e, ks, part);
  const long nout = (long)a.S * erows;
  launch_k(c, k_rcomb, dim3((unsigned)((nout + 255) / 256)), dim3(256), (const RbRec *)part, a.S, a.H, erows, ks,
           mid, bnd);
  return hipGetLastError();
}

static SelParams sel_params(const RouterArgs &a);

bool router_select_dp_ok(const RouterArgs &a, int kind, int cols, int rows) {
  const int nblk = cols / 32;
  return a.S == 1 && !(a.n_group > 1 && a.family != RBT_FAMILY_QWEN38) && a.E <= 64 * 16 && rows > 0 &&
         cols % 32 == 0 && nblk > 64 && nblk <= 256 && (kind == RBT_QT_MXFP4 || kind == RBT_QT_I4_GROUPED);
}

hipError_t launch_router_select_dp(const Ctx &c, const RouterArgs &a, const double *mid, const double *bnd,
                                   int32_t *ids, float *wts, float *sh_scale, int *stats, const GroupArgs &grp,
                                   const RbtExpertDev &proj, int kind, int cols, int rows, float *xl) {
  if (!router_select_dp_ok(a, kind, cols, rows) || c.num_cu < 1) return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  const GroupOut G = group_out(grp, a.k);
  const int m = (a.E + 63) / 64, nb = (cols / 32 + 63) / 64;
  const bool i4 = kind == RBT_QT_I4_GROUPED;
  const dim3 grid(1 + c.num_cu);
#define RBT_DP(M, NB_)                                                                                               {                                                                                                                    if (i4)                                                                                                              launch_k(c, (k_router_select3_dp<M, NB_, true>), grid, dim3(256), P, mid, bnd, ids, wts, sh_scale, stats, G,                proj, cols, rows, xl);                                                                                  else                                                                                                                 launch_k(c, (k_router_select3_dp<M, NB_, false>), grid, dim3(256), P, mid, bnd, ids, wts, sh_scale, stats,                  G, proj, cols, rows, xl);                                                                             }
#define RBT_DP_NB(M)   { if (nb == 2) RBT_DP(M, 2) else if (nb == 3) RBT_DP(M, 3) else RBT_DP(M, 4) }
  if (m <= 4)
    RBT_DP_NB(4)
  else if (m <= 8)
    RBT_DP_NB(8)
  else
    RBT_DP_NB(16)
#undef RBT_DP_NB
#undef RBT_DP
  return hipGetLastError();
}

hipError_t launch_router_select(const Ctx &c, const RouterArgs &a, const double *mid, const double *bnd, int32_t *ids,
                                float *wts, float *sh_scale, int *stats, const GroupArgs *grp, const SharedGateUp *sgu) {
  SelParams P;
  P.family = a.family;
  P.E = a.E;
  P.erows = a.erows;
  P.k = a.k;
  P.H = a.H;
  P.S = a.S;
  P.logit_bias = a.logit_bias;
  P.router_bias = a.router_bias;
  P.norm_topk = a.norm_topk;
  P.routed_scale = a.routed_scale;
  P.n_group = a.n_group;
  P.topk_group = a.topk_group;
  P.x = a.x;
  P.W = a.W;
  if (a.n_group > 1 && a.family != RBT_FAMILY_QWEN38) {
    launch_k(c, k_router_select_grouped, dim3(a.S), dim3(64), P, mid, bnd, ids, wts, sh_scale,
                       stats);
  } else {
    GroupOut G{};
    int g = 0;
    if (grp && a.S == 1) {
      G = group_out(*grp, a.k);
      g = 1;
    }
    const int m = (a.E + 63) / 64;
    if (sgu && a.S == 1 && m <= 8 && (sgu->K == 8192 || sgu->K == 7168)) {
      const dim3 grid(max(2, c.num_cu));
      if (m <= 4) {
        if (sgu->K == 8192)
          launch_k(c, (k_router_select3_sh<4, 16>), grid, dim3(256), P, mid, bnd, ids, wts, sh_scale,
                             stats, G, g, sgu->dev, sgu->x, sgu->I, sgu->hp);
        else
          launch_k(c, (k_router_select3_sh<4, 14>), grid, dim3(256), P, mid, bnd, ids, wts, sh_scale,
                             stats, G, g, sgu->dev, sgu->x, sgu->I, sgu->hp);
      } else {
        if (sgu->K == 8192)
          launch_k(c, (k_router_select3_sh<8, 16>), grid, dim3(256), P, mid, bnd, ids, wts, sh_scale,
                             stats, G, g, sgu->dev, sgu->x, sgu->I, sgu->hp);
        else
          launch_k(c, (k_router_select3_sh<8, 14>), grid, dim3(256), P, mid, bnd, ids, wts, sh_scale,
                             stats, G, g, sgu->dev, sgu->x, sgu->I, sgu->hp);
      }
      return hipGetLastError();
    }
    if (sgu) return hipErrorInvalidValue;
    if (m <= 4)
      launch_k(c, k_router_select3<4>, dim3(a.S), dim3(256), P, mid, bnd, ids, wts, sh_scale, stats,
                         G, g);
    else if (m <= 8)
      launch_k(c, k_router_select3<8>, dim3(a.S), dim3(256), P, mid, bnd, ids, wts, sh_scale, stats,
                         G, g);
    else if (m <= 16)
      launch_k(c, k_router_select3<16>, dim3(a.S), dim3(256), P, mid, bnd, ids, wts, sh_scale,
                         stats, G, g);
    else
      launch_k(c, k_router_select3<32>, dim3(a.S), dim3(256), P, mid, bnd, ids, wts, sh_scale,
                         stats, G, g);
  }
  return hipGetLastError();
}

// ------------------------------------------------------------------------------------------------
// One token on the matrix cores, in three launches and with no workgroup waiting for another:
//  1. k_router1: two (or four) router rows per workgroup with the block variant's arithmetic (fp64
//     segment sums, block scans, the certified bound), writing mid / bnd and a 16-byte key record
//     per expert, and the shared-expert gate row (sh_scale). Nothing else: every workgroup's loads
//     go out at once and the rows' reduction is the whole critical path.
//  2. k_xgateup1s (num_cu workgroups): every workgroup runs the selection itself from the key
//     records (identical inputs and code, hence an identical result), so the routing reaches the
//     streaming workgroups without a cross-workgroup hand-off. Workgroup 0 publishes ids, weights and
//     the down launch's job list; every workgroup streams its share of the routed pairs' and then
//     the shared expert's gate/up (pair slot nr: 11 pairs balanced over the grid at C1).
//     When the certified intervals left the decision open, workgroup 0 instead folds the undecided
//     logits exactly and decides, while the others stream every candidate.
//  3. k_xdown1 (xgemm.hip).
// ------------------------------------------------------------------------------------------------

// Key record of one expert: the key interval, the order-preserving bits of the midpoint key and the
// midpoint logit, computed exactly as the selection's own key setup does from (mid, bnd).
struct KeyRec {
  float klo, khi;
  uint32_t ku;
  float lm;
};

__device__ __forceinline__ KeyRec make_key_rec(const SelParams &P, int e, double mv, double bv) {
  const float lbv = P.logit_bias ? P.logit_bias[e] : 0.0f;
  const float rbv = P.router_bias ? P.router_bias[e] : 0.0f;
  const float lo = __double2float_rd(mv - bv * (1.0 + 1e-12));
  const float hi = __double2float_ru(mv + bv * (1.0 + 1e-12));
  const float md = fminf(fmaxf(__double2float_rn(mv), lo), hi);
  KeyRec r;
  r.lm = md;
  const float kmid = sel_key_v(P, lbv, rbv, md);
  r.ku = ord_key(kmid);
  if (lo == hi) {
    r.klo = r.khi = kmid;
  } else {
    r.klo = sel_key_v(P, lbv, rbv, lo);
    r.khi = sel_key_v(P, lbv, rbv, hi);
  }
  return r;
}

// The selection's result in the LDS of one gate/up workgroup: the routed pairs (T: slot c holds
// expert T.id[c], its midpoint order key and logit, and whether its logit must be folded exactly),
// their job-table entries, and the general path's outputs when it runs.
struct PairLds {
  D1Task T;
  RbtExpertDev pj[D1_NC + 1];  // the routed pairs, then the shared expert
  int status;
  int fb_ids[SEL_MAXK];
  float fb_w[SEL_MAXK];
};

// One token, wave 0: the fast path of the selection above from the key records, in registers (DPP
// reductions, readlane loops over the candidates), into LDS only. The threshold M is the kk-th
// largest lane maximum, taken by kk rounds of wave maximum that each retire one lane; candidates,
// ranking, set and order certification are those of the general path. Returns (every lane):
//  1  certified: the kk winners in rank order at slots 0..kk-1 (L.r_id / L.r_l set as well);
//  2  deferred: the winners in midpoint rank order, then the candidates that might still win, the
//     undecided ones flagged for an exact fold (Q.T.pending = 1);
//  0  the general path is needed (a NaN key, more than SEL_NC candidates, or more undecided
//     candidates than the pair slots beyond top-k).
// rv[m]: the key record of expert lane + 64 m (clamped to E - 1; load_key_recs), table: the job
// table (may be LDS).
template <int MAXM>
__device__ __forceinline__ void load_key_recs(const KeyRec *__restrict__ rec, int E, float4 (&rv)[MAXM]) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int m = 0; m < MAXM; m++) rv[m] = *reinterpret_cast<const float4 *>(rec + min(lane + 64 * m, E - 1));
}

template <int MAXM>
__device__ __forceinline__ int select_pairs(SelLds &L, PairLds &Q, const SelParams &P, const float4 (&rv)[MAXM],
                            const RbtExpertDev *__restrict__ table) {
  const int lane = threadIdx.x & 63;
  const int E = P.E, k = P.k, kk = min(P.k, P.E);
  uint32_t ku[MAXM];
  float klo[MAXM], khi[MAXM], lm[MAXM];
#pragma unroll
  for (int m = 0; m < MAXM; m++) {
    const float4 v = rv[m];
    const bool ok = lane + 64 * m < E;
    klo[m] = ok ? v.x : -INFINITY;
    khi[m] = ok ? v.y : -INFINITY;
    ku[m] = ok ? __float_as_uint(v.z) : 0u;
    lm[m] = v.w;
  }
  uint32_t cur = 0;
#pragma unroll
  for (int m = 0; m < MAXM; m++) cur = max(cur, ku[m]);
  // M: the kk-th largest of the lanes' largest keys (with multiplicity), found bit by bit as the
  // largest value that at least kk of them reach; every expert at or above it is a candidate (at
  // least kk of them, so every winner is one)
  uint32_t M = 0;
#pragma unroll
  for (int b = 31; b >= 0; b--) {
    const uint32_t c = M | (1u << b);
    if (__popcll(__ballot(cur >= c)) >= kk) M = c;
  }
  if (M == 0) return 0;  // a key maps to 0 (a NaN), or fewer than kk experts
  int nc = 0;
#pragma unroll
  for (int m = 0; m < MAXM; m++) nc += __popcll(__ballot(ku[m] >= M));
  if (nc > SEL_NC) return 0;
  uint32_t cm = 0;
  int base = 0;
#pragma unroll
  for (int m = 0; m < MAXM; m++) {
    const bool c = ku[m] >= M;
    const unsigned long long cb = __ballot(c);
    if (c) {
      const int at = base + __popcll(cb & lanemask_lt());
      L.q_id[at] = lane + 64 * m;
      L.q_ku[at] = ku[m];
      L.q_lo[at] = klo[m];
      L.q_hi[at] = khi[m];
      L.q_l[at] = lm[m];
      cm |= 1u << m;
    }
    base += __popcll(cb);
  }
  float hi_out = -INFINITY;  // upper keys of the non-candidates (never winners)
#pragma unroll
  for (int m = 0; m < MAXM; m++)
    if (!((cm >> m) & 1u) && ku[m] != 0) hi_out = fmaxf(hi_out, khi[m]);
  __builtin_amdgcn_wave_barrier();
  const bool cand = lane < nc;
  const uint32_t cku = cand ? L.q_ku[lane] : 0u;
  const int cid = cand ? L.q_id[lane] : 0x7fffffff;
  const float clo = cand ? L.q_lo[lane] : INFINITY, chi = cand ? L.q_hi[lane] : -INFINITY;
  const float cl = cand ? L.q_l[lane] : 0.0f;
  // the candidate's job-table entry, in flight while the selection is certified
  const uint8_t *pf_gd = nullptr, *pf_ud = nullptr, *pf_dd = nullptr;
  const void *pf_gs = nullptr, *pf_us = nullptr, *pf_ds = nullptr;
  if (cand) {
    const RbtExpertDev *src = table + cid;
    pf_gd = src->gd;
    pf_gs = src->gs;
    pf_ud = src->ud;
    pf_us = src->us;
    pf_dd = src->dd;
    pf_ds = src->ds;
  }
  // rank among the candidates: key desc, id asc
  int rank = 0;
  for (int j = 0; j < nc; j++) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)cku, j);
    const int oid = __builtin_amdgcn_readlane(cid, j);
    rank += (o > cku) || (o == cku && oid < cid);
  }
  if (!cand) rank = SEL_NC;
  const bool iw = rank < kk;
  const float lo_sel = rbt_wave_min_f(iw ? clo : INFINITY);
  const float hi_uns = rbt_wave_max_f(fmaxf(hi_out, (cand && !iw) ? chi : -INFINITY));
  // set membership: inexact experts on the wrong side of the other side's bound (nflag: the lane's
  // non-candidate keys that might still win; cflag: the lane's candidate is not certain)
  uint32_t nflag = 0;
#pragma unroll
  for (int m = 0; m < MAXM; m++)
    if (!((cm >> m) & 1u) && ku[m] != 0 && klo[m] != khi[m] && khi[m] >= lo_sel) nflag |= 1u << m;
  const bool cexact = clo == chi;
  bool cflag = cand && !cexact && (iw ? clo <= hi_uns : chi >= lo_sel);
  // order: every pair of winners strictly ordered, or both exact. The winners are ranked by their
  // midpoint keys, which their intervals hold, so that holds iff it holds for each winner and the
  // next one in rank order; only when some adjacent pair fails does the pairwise scan run, which
  // flags every non-exact winner that overlaps another.
  if (iw) {
    L.r_lo[rank] = clo;
    L.r_hi[rank] = chi;
  }
  __builtin_amdgcn_wave_barrier();
  bool bad = false;
  if (iw && rank + 1 < kk) {
    const float nlo = L.r_lo[rank + 1], nhi = L.r_hi[rank + 1];
    bad = !(cexact && nlo == nhi) && !(clo > nhi);
  }
  if (__ballot(bad) != 0) {
    for (int j = 0; j < nc; j++) {
      const int rj = __builtin_amdgcn_readlane(rank, j);
      const float lj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(clo), j));
      const float hj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(chi), j));
      if (iw && !cexact && rj < kk && rj != rank) cflag |= !(rj < rank ? lj > chi : clo > hj);
    }
  }
  D1Task &T = Q.T;
  auto task = [&](int slot, int id, uint32_t key, float logit, int flag) {
    T.id[slot] = id;
    T.ku[slot] = key;
    T.lm[slot] = logit;
    T.flag[slot] = flag;
  };
  auto put = [&](int slot) {
    RbtExpertDev *dst = Q.pj + slot;
    dst->gd = pf_gd;
    dst->gs = pf_gs;
    dst->ud = pf_ud;
    dst->us = pf_us;
    dst->dd = pf_dd;
    dst->ds = pf_ds;
  };
  if (__ballot(cflag || nflag != 0) != 0) {
    // Not certain: the routed pairs are the winners in midpoint rank order, then the candidates
    // that might still win; workgroup 0 folds the flagged logits exactly and decides.
    const bool undec = cand && !iw && cflag;
    const unsigned long long um = __ballot(undec);
    const int nuc = __popcll(um);
    int nun = 0;
#pragma unroll
    for (int m = 0; m < MAXM; m++) nun += __popcll(__ballot((nflag >> m) & 1u));
    const int nr = kk + nuc + nun;
    if (nr > min(k + D1_KX, D1_NC)) return 0;
    if (iw) {
      task(rank, cid, cku, cl, cflag ? 1 : 0);
      put(rank);
    }
    if (undec) {
      const int slot = kk + __popcll(um & lanemask_lt());
      task(slot, cid, cku, cl, 1);
      put(slot);
    }
    int nb = kk + nuc;
#pragma unroll
    for (int m = 0; m < MAXM; m++) {
      const bool f = (nflag >> m) & 1u;
      const unsigned long long fb = __ballot(f);
      if (f) {
        const int slot = nb + __popcll(fb & lanemask_lt()), id = lane + 64 * m;
        task(slot, id, ku[m], lm[m], 1);
        copy_job(Q.pj + slot, table + id);
      }
      nb += __popcll(fb);
    }
    if (lane == 0) {
      T.nr = nr;
      T.pending = 1;
    }
    return 2;
  }
  // certified: the winners in rank order
  if (iw) {
    L.r_id[rank] = cid;
    L.r_l[rank] = cl;
    task(rank, cid, cku, cl, 0);
    put(rank);
  }
  if (lane == 0) {
    T.nr = kk;
    T.pending = 0;
  }
  return 1;
}

// NR (1 or 2) router rows by the whole workgroup at once (one pass, shared scans and sums; per row
// the block variant's arithmetic, with the cross-lane sums through DPP, which only reorders fp64
// additions that the bound's slack covers): xv, wa, wb hold the thread's float4 chunks c * 256 + t
// of x and of the rows (wb unused when NR is 1).
template <int NR>
struct LgLds {
  __attribute__((aligned(16))) float lp[NR][RT_MAXH + 4 * 256];
  double sh[16];
};

__device__ __forceinline__ void store_key_rec(KeyRec *dst, const KeyRec &r) {
  const unsigned long long a = ((unsigned long long)__float_as_uint(r.khi) << 32) | __float_as_uint(r.klo);
  const unsigned long long b = ((unsigned long long)__float_as_uint(r.lm) << 32) | r.ku;
  unsigned long long *d = reinterpret_cast<unsigned long long *>(dst);
  d[0] = a;
  d[1] = b;
}

// KP/rec: when KP is set, the finishing threads also store the key records of rows ea and eb
// (-1: none), row b's at rec_b + eb when rec_b is given (two tokens of one router row).
// logits_rows_blk in two phases: the products into LDS (the inputs are dead after it), then the
// sums, the scan, the bound and the outputs.
template <int NR>
__device__ __forceinline__ void logits_rows_store(LgLds<NR> &L, const float4 (&xv)[RT_MAXH / 1024],
                                                  const float4 (&wa)[RT_MAXH / 1024],
                                                  const float4 (&wb)[RT_MAXH / 1024], int H) {
  static_assert(NR == 1 || NR == 2, "one or two rows");
  const int t = threadIdx.x;
  const int seg = H / 256, segp = rt_segp(seg), nch = H / 1024;
#pragma unroll
  for (int c = 0; c < RT_MAXH / 1024; c++) {
    if (c < nch) {
      const int j = c * 1024 + 4 * t;
      const int dst = (j / seg) * segp + (j % seg);
      float4 p;
      p.x = __fmul_rn(xv[c].x, wa[c].x);
      p.y = __fmul_rn(xv[c].y, wa[c].y);
      p.z = __fmul_rn(xv[c].z, wa[c].z);
      p.w = __fmul_rn(xv[c].w, wa[c].w);
      *reinterpret_cast<float4 *>(&L.lp[0][dst]) = p;
      if constexpr (NR == 2) {
        float4 q;
        q.x = __fmul_rn(xv[c].x, wb[c].x);
        q.y = __fmul_rn(xv[c].y, wb[c].y);
        q.z = __fmul_rn(xv[c].z, wb[c].z);
        q.w = __fmul_rn(xv[c].w, wb[c].w);
        *reinterpret_cast<float4 *>(&L.lp[NR - 1][dst]) = q;
      }
    }
  }
}

template <int NR>
__device__ __forceinline__ void logits_rows_finish(LgLds<NR> &L, int H, double *mid_a, double *bnd_a, double *mid_b,
                                                   double *bnd_b, const SelParams *KP = nullptr,
                                                   KeyRec *rec = nullptr, int ea = -1, int eb = -1,
                                                   KeyRec *rec_b = nullptr) {
  const int t = threadIdx.x, lane = t & 63, wid = t >> 6;
  const int seg = H / 256, segp = rt_segp(seg);
  const double u1 = 5.9604648328104515e-08;   // u/(1-u), u = 2^-24 (rounded up)
  const double e64 = 1.1102230246251565e-16;  // 2^-53
  __syncthreads();
  const float *ma = L.lp[0] + t * segp, *mb = L.lp[NR - 1] + t * segp;
  double la = 0.0, pa = 0.0, lb = 0.0, pb = 0.0;
  for (int q = 0; q < seg; q += 4) {
    const float4 p = *reinterpret_cast<const float4 *>(ma + q);
    la += (double)p.x;
    la += (double)p.y;
    la += (double)p.z;
    la += (double)p.w;
    pa += fabs((double)p.x) + fabs((double)p.y) + fabs((double)p.z) + fabs((double)p.w);
    if constexpr (NR == 2) {
      const float4 r = *reinterpret_cast<const float4 *>(mb + q);
      lb += (double)r.x;
      lb += (double)r.y;
      lb += (double)r.z;
      lb += (double)r.w;
      pb += fabs((double)r.x) + fabs((double)r.y) + fabs((double)r.z) + fabs((double)r.w);
    }
  }
  // exclusive block scan of the segment sums (wave scans, then wave offsets through LDS)
  const double ia = rbt_wave_scan_d(la);
  const double ib = NR == 2 ? rbt_wave_scan_d(lb) : 0.0;
  if (lane == 63) {
    L.sh[wid] = ia;
    L.sh[4 + wid] = ib;
  }
  __syncthreads();
  double offa = 0.0, offb = 0.0, tota = 0.0, totb = 0.0;
  for (int w = 0; w < 4; w++) {
    if (w < wid) {
      offa += L.sh[w];
      offb += L.sh[4 + w];
    }
    tota += L.sh[w];
    totb += L.sh[4 + w];
  }
  __syncthreads();
  double prea = offa + ia - la, preb = offb + ib - lb, Ta = 0.0, Tb = 0.0;
  for (int q = 0; q < seg; q += 4) {
    const float4 p = *reinterpret_cast<const float4 *>(ma + q);
    prea += (double)p.x;
    Ta += fabs(prea);
    prea += (double)p.y;
    Ta += fabs(prea);
    prea += (double)p.z;
    Ta += fabs(prea);
    prea += (double)p.w;
    Ta += fabs(prea);
    if constexpr (NR == 2) {
      const float4 r = *reinterpret_cast<const float4 *>(mb + q);
      preb += (double)r.x;
      Tb += fabs(preb);
      preb += (double)r.y;
      Tb += fabs(preb);
      preb += (double)r.z;
      Tb += fabs(preb);
      preb += (double)r.w;
      Tb += fabs(preb);
    }
  }
  Ta = rbt_wave_total_d(Ta);
  pa = rbt_wave_total_d(pa);
  if (NR == 2) {
    Tb = rbt_wave_total_d(Tb);
    pb = rbt_wave_total_d(pb);
  }
  if (lane == 0) {
    L.sh[wid] = Ta;
    L.sh[4 + wid] = pa;
    L.sh[8 + wid] = Tb;
    L.sh[12 + wid] = pb;
  }
  __syncthreads();
  // row a finishes on thread 0, row b on thread 64 (another wave), in parallel
  if (t == 0 || (NR == 2 && t == 64)) {
    const bool rowb = t == 64;
    const double n = (double)H;
    const double T = rowb ? L.sh[8] + L.sh[9] + L.sh[10] + L.sh[11] : L.sh[0] + L.sh[1] + L.sh[2] + L.sh[3];
    const double P = rowb ? L.sh[12] + L.sh[13] + L.sh[14] + L.sh[15] : L.sh[4] + L.sh[5] + L.sh[6] + L.sh[7];
    const double tot = rowb ? totb : tota;
    // B = u1 Tu / (1 - n u1) + slack, with 1/(1 - x) <= 1 + x + 2 x^2 (x = n u1 <= 1/2) in place of
    // the division; the final factor covers the fp64 roundings
    const double x = n * u1;
    const double slack = 8.0 * n * e64 * (P + T) + n * n * e64 * P;
    const double Tu = T * (1.0 + 8.0 * n * e64) + slack;
    double B = u1 * Tu * (1.0 + x + 2.0 * x * x) + slack;
    B = B * (1.0 + 1e-9) + 1e-300;
    double *mo = rowb ? mid_b : mid_a, *bo = rowb ? bnd_b : bnd_a;
    if (mo) {
      *mo = tot;
      *bo = B;
      const int e = rowb ? eb : ea;
      if (KP && e >= 0) store_key_rec((rowb && rec_b ? rec_b : rec) + e, make_key_rec(*KP, e, tot, B));
    }
  }
  __syncthreads();  // lp and sh are rewritten next
}

template <int NR>
__device__ __forceinline__ void logits_rows_blk(LgLds<NR> &L, const float4 (&xv)[RT_MAXH / 1024],
                                                const float4 (&wa)[RT_MAXH / 1024],
                                                const float4 (&wb)[RT_MAXH / 1024], int H, double *mid_a,
                                                double *bnd_a, double *mid_b, double *bnd_b,
                                                const SelParams *KP = nullptr, KeyRec *rec = nullptr, int ea = -1,
                                                int eb = -1, KeyRec *rec_b = nullptr) {
  logits_rows_store<NR>(L, xv, wa, wb, H);
  logits_rows_finish<NR>(L, H, mid_a, bnd_a, mid_b, bnd_b, KP, rec, ea, eb, rec_b);
}

typedef float rbt_f4v __attribute__((ext_vector_type(4)));

// rmsnorm_1p of the token (qwen38/ops.rs:25-33) in the workgroup: r = 1 / sqrt((sum_f64(v^2) / n)
// as f32 + eps), v[i] *= r * (1 + w[i]), every fp32 operation rounded on its own. The squares are
// exact in fp64 and summed in the registers' order (thread t: its chunks' elements 1024 c + 4 t ..
// +3, then the wave totals in fixed order), so every workgroup gets the same r; the sum differs from
// the reference's sequential one (and from k_rmsnorm's order) in the last fp64 bits only, which
// change the fp32 mean square only within a few fp64 ulps of an fp32 rounding boundary.
template <int NR>
__device__ __forceinline__ void norm1p_chunks(LgLds<NR> &L, float4 (&xv)[RT_MAXH / 1024],
                                              const float4 (&wv)[RT_MAXH / 1024], int H, float eps) {
  constexpr int MC = RT_MAXH / 1024;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6, nch = H / 1024;
  double acc = 0.0;
#pragma unroll
  for (int c = 0; c < MC; c++)
    if (c < nch) {
      acc += (double)xv[c].x * (double)xv[c].x;
      acc += (double)xv[c].y * (double)xv[c].y;
      acc += (double)xv[c].z * (double)xv[c].z;
      acc += (double)xv[c].w * (double)xv[c].w;
    }
  acc = rbt_wave_total_d(acc);
  if (lane == 0) L.sh[wave] = acc;
  __syncthreads();
  const double ms = (L.sh[0] + L.sh[1]) + (L.sh[2] + L.sh[3]);
  const float r = __fdiv_rn(1.0f, rbt_sqrt_rn(__fadd_rn((float)(ms / (double)H), eps)));
#pragma unroll
  for (int c = 0; c < MC; c++) {
    xv[c].x = __fmul_rn(xv[c].x, __fmul_rn(r, __fadd_rn(1.0f, wv[c].x)));
    xv[c].y = __fmul_rn(xv[c].y, __fmul_rn(r, __fadd_rn(1.0f, wv[c].y)));
    xv[c].z = __fmul_rn(xv[c].z, __fmul_rn(r, __fadd_rn(1.0f, wv[c].z)));
    xv[c].w = __fmul_rn(xv[c].w, __fmul_rn(r, __fadd_rn(1.0f, wv[c].w)));
  }
  __syncthreads();  // L.sh is the rows' scratch next
}

// Workgroup b computes RPW router rows: rows RPW b .. RPW b + RPW - 1 of the E router rows followed
// by the shared-expert gate row (row E, when sgate is given: its fp64 sum gives sh_scale; it has no
// key record). The rows' loads are issued together, then the rows are reduced two at a time.
// With nw (the MoE sublayer), P.x is the raw token and every workgroup first normalises it
// (rmsnorm_1p with weights nw, eps) for its rows; workgroup 0 writes the normalised token to xn.
template <int RPW, bool NORM>
__device__ __forceinline__ void router1_body(LgLds<RPW == 1 ? 1 : 2> &L, const SelParams &P,
                                             const float *__restrict__ sgate, double *__restrict__ mid,
                                             double *__restrict__ bnd, float *__restrict__ sh_scale,
                                             KeyRec *__restrict__ rec, const float *__restrict__ nw, float eps,
                                             float *__restrict__ xn, int b) {
  constexpr int MC = RT_MAXH / 1024, NR = RPW == 1 ? 1 : 2;
  const int t = threadIdx.x;
  const int H = P.H, E = P.E, nch = H / 1024;
  if (sgate == nullptr && b == 0 && t == 0) sh_scale[0] = 1.0f;
  const int Rn = E + (sgate != nullptr ? 1 : 0), r0 = RPW * b;
  if (r0 >= Rn && !(NORM && b == 0)) return;
  const float4 *x4 = reinterpret_cast<const float4 *>(P.x);
  float4 xv[MC], w[RPW][MC], wv[MC];
  // the token (and the norm's weights) first: the memory counter retires loads in issue order, so
  // the norm waits for them only, not for the rows' loads behind them
#pragma unroll
  for (int c = 0; c < MC; c++) xv[c] = x4[min(c, nch - 1) * 256 + t];
  if (NORM) {
    const float4 *n4 = reinterpret_cast<const float4 *>(nw);
#pragma unroll
    for (int c = 0; c < MC; c++) wv[c] = n4[min(c, nch - 1) * 256 + t];
  }
  // unconditional loads (chunks past the row repeat its last one; rows past the end read row 0):
  // no waits between the rows
#pragma unroll
  for (int j = 0; j < RPW; j++) {
    const int r = r0 + j;
    const float4 *w4 =
        reinterpret_cast<const float4 *>(r < E ? P.W + (size_t)r * H : (r == E && sgate != nullptr ? sgate : P.W));
#pragma unroll
    for (int c = 0; c < MC; c++) {
      const rbt_f4v v =
          __builtin_nontemporal_load(reinterpret_cast<const rbt_f4v *>(w4 + min(c, nch - 1) * 256 + t));
      w[j][c] = make_float4(v[0], v[1], v[2], v[3]);
    }
  }
  // (the norm below is kept after the rows' loads: placed before them, its use of the weights
  // made the rows wait for the token and the weights to land)
  __builtin_amdgcn_sched_barrier(0);
  if (NORM) {
    norm1p_chunks<NR>(L, xv, wv, H, eps);
    if (b == 0) {
#pragma unroll
      for (int c = 0; c < MC; c++)
        if (c < nch) reinterpret_cast<float4 *>(xn)[c * 256 + t] = xv[c];
    }
    if (r0 >= Rn) return;
  }
#pragma unroll
  for (int j = 0; j < RPW; j += NR) {
    const int ra = r0 + j, rb = ra + 1;
    if (ra < Rn)
      logits_rows_blk<NR>(L, xv, w[j], w[j + NR - 1], H, mid + ra, bnd + ra, NR == 2 && rb < Rn ? mid + rb : nullptr,
                          NR == 2 && rb < Rn ? bnd + rb : nullptr, &P, rec, ra < E ? ra : -1,
                          NR == 2 && rb < E ? rb : -1);
  }
  // gated shared expert: sigmoid of the fp32-rounded gate logit (qwen38/moe.rs:78-83); the row's
  // sum was stored before the last barrier of logits_rows_blk
  if (sgate != nullptr && r0 <= E && E < r0 + RPW && t == 0) sh_scale[0] = sigmoid_ref(__double2float_rn(mid[E]));
}

template <int RPW, bool NORM>
__global__ __launch_bounds__(256) void k_router1(SelParams P, const float *__restrict__ sgate,
                                                 double *__restrict__ mid, double *__restrict__ bnd,
                                                 float *__restrict__ sh_scale, KeyRec *__restrict__ rec,
                                                 const float *__restrict__ nw, float eps, float *__restrict__ xn) {
  __shared__ LgLds<RPW == 1 ? 1 : 2> L;
  router1_body<RPW, NORM>(L, P, sgate, mid, bnd, sh_scale, rec, nw, eps, xn, blockIdx.x);
}

// One token of K3's latent MoE: the router rows' key records (router1_body, workgroups 0 .. E - 1)
// and the latent down projection xl = Dp . x (proj1_body, workgroups E .. E + npj - 1, four waves of
// at most two rows each) in one launch. Both read only the token, and each alone is bound by its
// latency (router rows 10 us for 26 MB, the projection 8 us for 16 MB), not by HBM: together 15.4
// us (the projection's workgroups first: 15.9).
union RouterProjLds {
  LgLds<1> lg;
  PjLds pj;
};
template <bool I4G, int NB>
__global__ __launch_bounds__(256) void k_router1_proj(SelParams P, double *__restrict__ mid, double *__restrict__ bnd,
                                                      float *__restrict__ sh_scale, KeyRec *__restrict__ rec,
                                                      const uint8_t *__restrict__ pd, const uint8_t *__restrict__ ps,
                                                      int mh, float *__restrict__ xl, int npj) {
  __shared__ RouterProjLds U;
  if ((int)blockIdx.x >= P.E)
    proj1_body<I4G, false, NB, 4, 2>(U.pj, pd, ps, P.x, P.H, mh, xl, nullptr, 0.0f, blockIdx.x - P.E, npj);
  else
    router1_body<1, false>(U.lg, P, nullptr, mid, bnd, sh_scale, rec, nullptr, 0.0f, nullptr, blockIdx.x);
}

// Certified logits of a decode batch, one (row, token) per workgroup: a smaller LDS footprint than
// the two-at-a-time form, so four workgroups share a CU; the row is read from HBM once and its
// other tokens' reads hit L2 when the router's row count is a multiple of the XCD count (the grid's
// tokens of one row are then dispatched to one XCD).
__global__ __launch_bounds__(256) void k_router_logits_t1(const float *__restrict__ x, int S, int H,
                                                          const float *__restrict__ W, int E,
                                                          const float *__restrict__ sgate, double *__restrict__ mid,
                                                          double *__restrict__ bnd, int erows) {
  constexpr int MC = RT_MAXH / 1024;
  __shared__ LgLds<1> L;
  const int t = threadIdx.x, row = blockIdx.x, s = blockIdx.y, nch = H / 1024;
  const float4 *w4 = reinterpret_cast<const float4 *>(row < E ? W + (size_t)row * H : sgate);
  const float4 *x4 = reinterpret_cast<const float4 *>(x + (size_t)s * H);
  float4 wv[MC], xv[MC];
#pragma unroll
  for (int c = 0; c < MC; c++) xv[c] = x4[min(c, nch - 1) * 256 + t];
#pragma unroll
  for (int c = 0; c < MC; c++) wv[c] = w4[min(c, nch - 1) * 256 + t];
  logits_rows_blk<1>(L, wv, xv, xv, H, mid + (size_t)s * erows + row, bnd + (size_t)s * erows + row, nullptr,
                     nullptr);
}

// The selection of a decode batch, one workgroup per token: the four waves form the token's key
// records from its intervals (sel_keys: three fp64 sigmoids per expert for the sigmoid families),
// then wave 0 runs the one-token fast path (select_pairs); when it certifies, the winners' weights
// and ids; otherwise (an open decision, ties beyond the candidate window, NaN keys) the general
// path from the intervals, exact folds included (select3_body). Writes ids / wts / sh_scale of the
// token as k_router_select3 does.
template <int MAXM>
__global__ __launch_bounds__(256) void k_router_select_rec(SelParams P, const double *__restrict__ mid,
                                                           const double *__restrict__ bnd,
                                                           const RbtExpertDev *__restrict__ table,
                                                           int32_t *__restrict__ ids, float *__restrict__ wts,
                                                           float *__restrict__ sh_scale, int *__restrict__ stats,
                                                           __bf16 *__restrict__ xb3) {
  __shared__ SelLds L;
  __shared__ PairLds Q;
  __shared__ __attribute__((aligned(16))) float4 kr[64 * MAXM];
  __shared__ float kbuf[6 * 64 * MAXM];
  const int s = blockIdx.x, t = threadIdx.x, lane = t & 63;
  const int E = P.E, k = P.k, kk = min(P.k, P.E);
  const double *ms = mid + (size_t)s * P.erows, *bs = bnd + (size_t)s * P.erows;
  for (int e = t; e < E; e += 256) {
    const float lb = P.logit_bias ? P.logit_bias[e] : 0.0f;
    const float rb = P.router_bias ? P.router_bias[e] : 0.0f;
    float lm, kl, kh;
    uint32_t u;
    sel_keys(P, ms[e], bs[e], lb, rb, lm, u, kl, kh);
    kr[e] = make_float4(kl, kh, __uint_as_float(u), lm);
  }
  __syncthreads();
  if (t < 64) {
    float4 rv[MAXM];
#pragma unroll
    for (int m = 0; m < MAXM; m++) rv[m] = kr[min(lane + 64 * m, E - 1)];
    const int r = select_pairs<MAXM>(L, Q, P, rv, table);
    if (r == 1) {
      winner_weights(L, P, kk);
      for (int j = lane; j < k; j += 64) {
        ids[(size_t)s * k + j] = j < kk ? L.r_id[j] : -1;
        wts[(size_t)s * k + j] = j < kk ? L.s_w[j] : 0.0f;
      }
      if (lane == 0 && sh_scale) sh_scale[s] = (P.erows > E) ? sigmoid_ref(__double2float_rn(ms[E])) : 1.0f;
    }
    if (lane == 0) Q.status = r;
  } else if (xb3 != nullptr) {
    // waves 1-3 meanwhile: the token's three exact bf16 parts for the grouped decode GEMMs (x = hi +
    // mid + lo, each the bf16 rounding of the remainder; rows 3 s + part of xb3)
    const int H = P.H;
    const float4 *x4 = reinterpret_cast<const float4 *>(P.x + (size_t)s * H);
    __bf16 *o0 = xb3 + (size_t)(3 * s) * H, *o1 = o0 + H, *o2 = o1 + H;
    for (int q = t - 64; q < H / 4; q += 192) {
      const float4 v = x4[q];
      const float e4[4] = {v.x, v.y, v.z, v.w};
      __bf16 hh[4], mm[4], ll[4];
#pragma unroll
      for (int e = 0; e < 4; e++) split3(e4[e], hh[e], mm[e], ll[e]);
      typedef __bf16 b4v __attribute__((ext_vector_type(4)));
      *reinterpret_cast<b4v *>(o0 + 4 * q) = b4v{hh[0], hh[1], hh[2], hh[3]};
      *reinterpret_cast<b4v *>(o1 + 4 * q) = b4v{mm[0], mm[1], mm[2], mm[3]};
      *reinterpret_cast<b4v *>(o2 + 4 * q) = b4v{ll[0], ll[1], ll[2], ll[3]};
    }
  }
  __syncthreads();
  if (Q.status != 1) select3_body<MAXM, true>(L, P, mid, bnd, ids, wts, sh_scale, stats, GroupOut{}, 0, s, kbuf);
}

// Certified logits of a small batch: workgroup (row, q) computes router row `row` (or the shared
// gate row, row == E) against tokens 4q .. 4q + 3, two at a time with the two-row arithmetic (the
// products are the same with the row and the tokens swapped). The row is read once per four tokens.
__global__ __launch_bounds__(256) void k_router_logits_tk(const float *__restrict__ x, int S, int H,
                                                          const float *__restrict__ W, int E,
                                                          const float *__restrict__ sgate, double *__restrict__ mid,
                                                          double *__restrict__ bnd, int erows) {
  constexpr int MC = RT_MAXH / 1024;
  __shared__ LgLds<2> L;
  const int t = threadIdx.x, row = blockIdx.x, nch = H / 1024;
  const int s0 = 4 * blockIdx.y;
  const float4 *w4 = reinterpret_cast<const float4 *>(row < E ? W + (size_t)row * H : sgate);
  float4 wv[MC], xa[MC], xb[MC];
  auto load = [&](const float4 *p, float4(&v)[MC]) {
#pragma unroll
    for (int c = 0; c < MC; c++) v[c] = p[min(c, nch - 1) * 256 + t];
  };
  load(w4, wv);
  for (int s = s0; s < min(S, s0 + 4); s += 2) {
    const int s1 = min(s + 1, S - 1);
    load(reinterpret_cast<const float4 *>(x + (size_t)s * H), xa);
    load(reinterpret_cast<const float4 *>(x + (size_t)s1 * H), xb);
    const bool two = s + 1 < S;
    logits_rows_blk<2>(L, wv, xa, xb, H, mid + (size_t)s * erows + row, bnd + (size_t)s * erows + row,
                       two ? mid + (size_t)(s + 1) * erows + row : nullptr,
                       two ? bnd + (size_t)(s + 1) * erows + row : nullptr);
  }
}

// ------------------------------------------------------------------------------------------------
// Workgroup 0 of the gate/up launch, after a certified selection: ids, weights, tok_pair / tok_w
// and the down launch's job list (the winners in rank order at pair slots 0..kk-1, then the shared
// expert at its slot). Wave 0.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ void publish_certified(SelLds &L, const PairLds &Q, const SelParams &P, const GroupOut &G,
                                  int32_t *__restrict__ ids, float *__restrict__ wts) {
  const int lane = threadIdx.x & 63;
  const int k = P.k, kk = min(P.k, P.E);
  winner_weights(L, P, kk);
  for (int r = lane; r <= k; r += 64) {
    if (r < k) {
      ids[r] = r < kk ? L.r_id[r] : -1;
      wts[r] = r < kk ? L.s_w[r] : 0.0f;
      G.tok_pair[r] = r < kk ? r : -1;
      G.tok_w[r] = r < kk ? L.s_w[r] : 0.0f;
      if (r < kk) {
        if (Q.pj[r].gd == nullptr || Q.pj[r].dd == nullptr) atomicOr(G.err, 1);
        copy_job(G.down_job + r, Q.pj + r);
        G.down_slot[r] = r;
      }
    } else {
      copy_job(G.down_job + kk, G.shared_dev);
      G.down_slot[kk] = G.shared_slot;
    }
  }
}

// Workgroup 0 after a deferred selection: folds the flagged logits as the reference does (the
// sequential fp32 sum, four waves in parallel), ranks the candidates with exact keys where they
// were folded and midpoint keys elsewhere (an unflagged candidate's interval is disjoint from every
// other candidate's, so its midpoint orders it), and writes ids, weights, tok_pair / tok_w and the
// down job list.
__device__ __forceinline__ void d1_finish(SelLds &L, float (*fold)[2][1024], const SelParams &P, const D1Task *__restrict__ T,
                          const GroupOut &G, int32_t *__restrict__ ids, float *__restrict__ wts,
                          int *__restrict__ stats) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int k = P.k, kk = min(P.k, P.E);
  const int nc = T->nr;
  if (threadIdx.x == 0) L.namb = 0;
  __syncthreads();
  if (wave == 0 && lane < nc && T->flag[lane]) L.amb[atomicAdd(&L.namb, 1)] = lane;
  __syncthreads();
  const int na = L.namb;
  for (int j = wave; j < na; j += 4) {
    const int c = L.amb[j];
    const float l = exact_logit_lds(P.x, P.W + (size_t)T->id[c] * P.H, P.H, fold[wave]);
    if (lane == 0) L.amb_val[j] = l;
  }
  __syncthreads();
  if (wave != 0) return;
  // candidate `lane` (pair slot `lane`) with its final key: exact where folded
  const bool cand = lane < nc;
  const int id = cand ? T->id[lane] : 0x7fffffff;
  uint32_t key = cand ? T->ku[lane] : 0u;
  float lm = cand ? T->lm[lane] : 0.0f;
  for (int j = 0; j < na; j++)
    if (L.amb[j] == lane) {
      lm = L.amb_val[j];
      const float lb = P.logit_bias ? P.logit_bias[id] : 0.0f;
      const float rb = P.router_bias ? P.router_bias[id] : 0.0f;
      key = ord_key(sel_key_v(P, lb, rb, lm));
    }
  int rank = 0;
  for (int j = 0; j < nc; j++) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_readlane((int)key, j);
    const int oid = __builtin_amdgcn_readlane(id, j);
    rank += (o > key) || (o == key && oid < id);
  }
  if (cand && rank < kk) {
    L.r_id[rank] = id;
    L.r_l[rank] = lm;
    L.q_id[rank] = lane;  // pair slot of the rank-th winner
  }
  __builtin_amdgcn_wave_barrier();
  winner_weights(L, P, kk);
  for (int r = lane; r <= k; r += 64) {
    if (r < k) {
      ids[r] = r < kk ? L.r_id[r] : -1;
      wts[r] = r < kk ? L.s_w[r] : 0.0f;
      // the consumers of the job list (the down launches, the combine) index their rows by rank,
      // not by the winner's gate/up slot (down_slot)
      G.tok_pair[r] = r < kk ? r : -1;
      G.tok_w[r] = r < kk ? L.s_w[r] : 0.0f;
      if (r < kk) {
        const RbtExpertDev *src = G.table + L.r_id[r];
        if (src->gd == nullptr || src->dd == nullptr) atomicOr(G.err, 1);
        copy_job(G.down_job + r, src);
        G.down_slot[r] = L.q_id[r];
      }
    } else {
      copy_job(G.down_job + kk, G.shared_dev);
      G.down_slot[kk] = G.shared_slot;
    }
  }
  if (lane == 0 && stats && na) atomicAdd(stats, na);
}

// After the general selection (select3_body, the same in every workgroup), the workgroup's routed
// pairs: the winners in rank order (L.r_id, left by wave 0 in every workgroup, the publishing one
// included), their job-table entries, nr = kk, nothing pending. Ends with a
// workgroup barrier.
__device__ __forceinline__ void fallback_pairs(const SelLds &L, PairLds &Q, const RbtExpertDev *__restrict__ tab,
                                               int kk) {
  __syncthreads();
  const int t = threadIdx.x;
  if (t < 64) {
    for (int r = t; r < kk; r += 64) {
      const int e = L.r_id[r];
      Q.T.id[r] = e;
      copy_job(Q.pj + r, tab + e);
    }
    if (t == 0) {
      Q.T.nr = kk;
      Q.T.pending = 0;
    }
  }
  __syncthreads();
}

// gup (optional) counts the routed pairs the launch streams (for the benchmark's byte accounting).
// xg: the gate/up activation (K = 512 NCH values; the router's own token in a plain layer, the
// latent token in K3's latent MoE); h = act(g, u), as three bf16 parts or (HF32) fp32.
// A workgroup stages the job-table entries of up to 64 MAXM experts in LDS.
template <int MAXM, int NCH, bool HF32>
__global__ __launch_bounds__(256) void k_xgateup1s(SelParams P, const KeyRec *__restrict__ rec,
                                                   const double *__restrict__ mid, const double *__restrict__ bnd,
                                                   GroupOut G, int32_t *__restrict__ ids, float *__restrict__ wts,
                                                   int *__restrict__ stats, int *__restrict__ gup, int I,
                                                   __bf16 *__restrict__ hp, int has_shared, RbtExpertDev shv,
                                                   const float *__restrict__ xg, RbtAct act) {
  __shared__ union {
    GuLds gu;
    __attribute__((aligned(16))) float fold[4][2][1024];  // workgroup 0, deferred: exact_logit_lds's blocks
  } U;
  __shared__ SelLds S;
  __shared__ PairLds Q;
  const int t = threadIdx.x, lane = t & 63;
  const bool streamer = blockIdx.x > 0;
  const int E = P.E, kk = min(P.k, P.E);
  // The key records (wave 0) and the activation are in flight together; the selection loads each
  // candidate's job-table entry while it certifies.
  float4 rv[MAXM];
  if (t < 64) load_key_recs<MAXM>(rec, E, rv);
  float4 xv[xg_nv<NCH>()];
  xgateup1_load_x<NCH>(xg, xv);
  xgateup1_stage_x<NCH>(U.gu, xv);
  // The shared expert's gate/up does not depend on the routing: when every workgroup holds at most
  // two of its 4-row units, each unit is two half units (waves 2j, 2j + 1), whose loads go out now
  // and land during the selection (issued after the selection's own inputs have landed, which they
  // would otherwise delay). The routed pairs then balance over the grid without it.
  const int tpp = I >> 2;
  const bool shpro = NCH % 2 == 0 && !HF32 && has_shared && shv.gd && shv.ud && shv.gs && shv.us &&
                     tpp <= 2 * (int)gridDim.x;
  const int s0 = shpro ? (int)((long)blockIdx.x * tpp / gridDim.x) : 0;
  const int nsu = shpro ? (int)((long)(blockIdx.x + 1) * tpp / gridDim.x) - s0 : 0;
  // Wave 0 selects first: its half goes out after the selection (loads issued ahead of the selection
  // would hold its issue slots until the memory pipeline has room for all of them). Waves 1-3 issue
  // theirs after the staging barrier, so that the selection does not wait for those issues.
  ShHalf<NCH> sh;
  if ((t >> 6) < 2 * nsu) {
    sh.su = s0 + (t >> 7);
    sh.hf = (t >> 6) & 1;
  }
  lds_barrier();  // the staged activation
  if constexpr (NCH % 2 == 0)
    if (t >= 64 && sh.su >= 0) xgateup1_sh_issue<NCH>(sh, shv);
  if (t < 64) {
    const int r = select_pairs<MAXM>(S, Q, P, rv, G.table);
    if (t == 0) Q.status = r;
  }
  if constexpr (NCH % 2 == 0)
    if (t < 64 && sh.su >= 0) xgateup1_sh_issue<NCH>(sh, shv);
  lds_barrier();
  const int st = Q.status;
  // the shared expert streams as the pair after the routed ones: its h lands at pair slot nr
  GroupOut Gs = G;
  if (st == 0) {
    // the general path (exact recomputes until certain), the same in every workgroup; workgroup 0
    // writes the outputs, the others take the winners as their pairs
    if (!streamer) {
      Gs.shared_slot = kk;
      select3_body<MAXM>(S, P, mid, bnd, ids, wts, nullptr, stats, Gs, 1, 0);
    } else {
      select3_body<MAXM>(S, P, mid, bnd, Q.fb_ids, Q.fb_w, nullptr, nullptr, G, 0, 0);
    }
    fallback_pairs(S, Q, G.table, kk);
  }
  // A deferred decision: workgroup 0 folds and decides while the others stream every candidate.
  // Otherwise workgroup 0 publishes the routing (the general path already did) and streams its
  // share like the rest.
  const bool pending = st == 2;
  const int nr = Q.T.nr;
  Gs.shared_slot = nr;
  const bool decider = !streamer && pending;  // folds and decides; streams no routed pair
  if (!streamer) {
    if (t == 0 && gup) atomicAdd(gup, nr + has_shared);
    if (st == 1 && t < 64) publish_certified(S, Q, P, Gs, ids, wts);
  }
  if (has_shared && !shpro && t == 0) copy_job(Q.pj + nr, G.shared_dev);
  __syncthreads();
  if (!decider || shpro) {
    // the routed pairs (and the shared expert unless it went out early), balanced over the grid;
    // the deciding workgroup only multiplies its shared half units
    const int wg = pending ? blockIdx.x - 1 : blockIdx.x, nwg = pending ? gridDim.x - 1 : gridDim.x;
    xgateup1_run<NCH, true, true, HF32>(U.gu, Q.pj, decider ? 0 : nr + (has_shared && !shpro), xv, xg, I, hp,
                                        decider ? 0 : wg, decider ? 1 : nwg, &sh, act);
    if (shpro) {
      __syncthreads();
      xgateup1_sh_combine(U.gu, s0, nsu, nr, I, hp);
    }
  }
  if (decider) {
    __syncthreads();
    d1_finish(S, U.fold, P, &Q.T, Gs, ids, wts, stats);  // U.gu's staged activation is not needed
  }
}

// One token through the decode GEMVs (grouped int4, or any format the matrix-core kernels do not
// take), as the three-launch decode does it on the matrix cores: every workgroup selects from the
// key records (k_router1), workgroup 0 publishes the routing and the down job list, and the grid's
// waves run the fused gate/up + activation GEMV over the routed pairs and the shared expert (the
// pair after them), h in fp32 at the pairs' slots. A deferred decision: workgroup 0 folds and decides
// while the other workgroups stream every candidate.
template <int MAXM, int NB, bool I4G>
__global__ __launch_bounds__(256) void k_gu1s_gemv(SelParams P, const KeyRec *__restrict__ rec,
                                                   const double *__restrict__ mid, const double *__restrict__ bnd,
                                                   GroupOut G, int32_t *__restrict__ ids, float *__restrict__ wts,
                                                   int *__restrict__ stats, int I, float *__restrict__ h,
                                                   int has_shared, RbtAct act) {
  __shared__ __attribute__((aligned(16))) float fold[4][2][1024];  // workgroup 0, deferred
  __shared__ SelLds S;
  __shared__ PairLds Q;
  const int t = threadIdx.x, lane = t & 63;
  const bool streamer = blockIdx.x > 0;
  const int E = P.E, kk = min(P.k, P.E);
  float4 rv[MAXM];
  if (t < 64) load_key_recs<MAXM>(rec, E, rv);
  if (t < 64) {
    const int r = select_pairs<MAXM>(S, Q, P, rv, G.table);
    if (t == 0) Q.status = r;
  }
  lds_barrier();
  const int st = Q.status;
  GroupOut Gs = G;
  if (st == 0) {
    if (!streamer) {
      Gs.shared_slot = kk;
      select3_body<MAXM>(S, P, mid, bnd, ids, wts, nullptr, stats, Gs, 1, 0);
    } else {
      select3_body<MAXM>(S, P, mid, bnd, Q.fb_ids, Q.fb_w, nullptr, nullptr, G, 0, 0);
    }
    fallback_pairs(S, Q, G.table, kk);
  }
  const bool pending = st == 2;
  const int nr = Q.T.nr;
  Gs.shared_slot = nr;
  const bool decider = !streamer && pending;
  if (!streamer && st == 1 && t < 64) publish_certified(S, Q, P, Gs, ids, wts);
  if (has_shared && t == 0) copy_job(Q.pj + nr, G.shared_dev);
  __syncthreads();
  if (!decider) {
    const int wg = pending ? blockIdx.x - 1 : blockIdx.x, nwg = pending ? gridDim.x - 1 : gridDim.x;
    gu_act_body<NB, I4G>(Q.pj, RbtExpertDev{}, nr + has_shared, nullptr, P.x, nullptr, 0, P.H, I, act, h,
                         wg * 4 + (t >> 6), nwg * 4);
  } else {
    d1_finish(S, fold, P, &Q.T, Gs, ids, wts, stats);
  }
}

static SelParams sel_params(const RouterArgs &a) {
  SelParams P{};
  P.family = a.family;
  P.E = a.E;
  P.erows = a.erows;
  P.k = a.k;
  P.H = a.H;
  P.S = a.S;
  P.logit_bias = a.logit_bias;
  P.router_bias = a.router_bias;
  P.norm_topk = a.norm_topk;
  P.routed_scale = a.routed_scale;
  P.n_group = a.n_group;
  P.topk_group = a.topk_group;
  P.x = a.x;
  P.W = a.W;
  return P;
}

bool router_batch_ok(const RouterArgs &a) {
  const bool aligned = ((uintptr_t)a.x % 16 == 0) && ((uintptr_t)a.W % 16 == 0);
  return a.S >= 2 && a.H % 1024 == 0 && a.H <= RT_MAXH && aligned && a.E <= 1024 && a.k <= SEL_MAXK &&
         !(a.n_group > 1 && a.family != RBT_FAMILY_QWEN38);
}

hipError_t launch_router_batch(const Ctx &c, const RouterArgs &a, const float *sgate, double *mid, double *bnd,
                               const RbtExpertDev *table, int32_t *ids, float *wts, float *sh_scale, int *stats,
                               __bf16 *xb3) {
  if (!router_batch_ok(a) || (sgate && (uintptr_t)sgate % 16 != 0) || !table) return hipErrorInvalidValue;
  if (xb3 && ((uintptr_t)a.x % 16 != 0 || (uintptr_t)xb3 % 8 != 0 || a.H % 4 != 0)) return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  launch_k(c, k_router_logits_t1, dim3(a.erows, a.S), dim3(256), a.x, a.S, a.H, a.W, a.E, sgate, mid, bnd, a.erows);
  const int m = (a.E + 63) / 64;
  if (m <= 4)
    launch_k(c, k_router_select_rec<4>, dim3(a.S), dim3(256), P, (const double *)mid, (const double *)bnd, table, ids,
             wts, sh_scale, stats, xb3);
  else if (m <= 8)
    launch_k(c, k_router_select_rec<8>, dim3(a.S), dim3(256), P, (const double *)mid, (const double *)bnd, table, ids,
             wts, sh_scale, stats, xb3);
  else
    launch_k(c, k_router_select_rec<16>, dim3(a.S), dim3(256), P, (const double *)mid, (const double *)bnd, table,
             ids, wts, sh_scale, stats, xb3);
  return hipGetLastError();
}

bool router1_ok(const RouterArgs &a, int num_cu, const SharedGateUp *sgu) {
  const bool aligned = ((uintptr_t)a.x % 16 == 0) && ((uintptr_t)a.W % 16 == 0);
  return a.S == 1 && !(a.n_group > 1 && a.family != RBT_FAMILY_QWEN38) && a.E <= 512 && a.k + D1_KX <= D1_NC &&
         (a.H == 8192 || a.H == 7168) && aligned && a.E <= 2 * num_cu && num_cu >= 2 &&
         (sgu == nullptr || sgu->K == a.H);
}

hipError_t launch_router1(const Ctx &c, const RouterArgs &a, const float *sgate, double *mid, double *bnd,
                          float *sh_scale, void *rec_buf, const float *nw, float eps, float *xn) {
  KeyRec *rec = reinterpret_cast<KeyRec *>(rec_buf);
  if (!router1_ok(a, c.num_cu, nullptr) || (sgate && (uintptr_t)sgate % 16 != 0)) return hipErrorInvalidValue;
  if (nw && (!xn || ((uintptr_t)nw | (uintptr_t)xn) % 16 != 0)) return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  // one row per workgroup while the grid fits the chip at once (the rows' reduction is on the
  // critical path: C1's 513 rows take 9.5 us as 257 x 2 rows, 11.8 us as 129 x 4)
  const int rn = a.E + (sgate ? 1 : 0);
  if (rn <= 4 * c.num_cu)  // four one-row workgroups fit on a CU
    launch_k(c, nw ? k_router1<1, true> : k_router1<1, false>, dim3(rn), dim3(256), P, sgate, mid, bnd, sh_scale, rec,
             nw, eps, xn);
  else
    launch_k(c, nw ? k_router1<2, true> : k_router1<2, false>, dim3((rn + 1) / 2), dim3(256), P, sgate, mid, bnd,
             sh_scale, rec, nw, eps, xn);
  return hipGetLastError();
}

hipError_t launch_router1_latent(const Ctx &c, const RouterArgs &a, double *mid, double *bnd, float *sh_scale,
                                 void *rec_buf, int mh, int I) {
  if (!router1_latent_ok(a, c.num_cu, mh, I)) return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  launch_k(c, k_router1<1, false>, dim3(a.E), dim3(256), P, nullptr, mid, bnd, sh_scale,
           reinterpret_cast<KeyRec *>(rec_buf), nullptr, 0.0f, nullptr);
  return hipGetLastError();
}

bool router1_proj_ok(const RouterArgs &a, int num_cu, int mh, int I, int kind, size_t gs) {
  const bool fmt = kind == RBT_QT_MXFP4 || (kind == RBT_QT_I4_GROUPED && gs == 32);
  return fmt && router1_latent_ok(a, num_cu, mh, I) && a.H % 32 == 0 && a.H <= PJ_MAXC &&
         (long)mh <= 2L * 4 * (2 * num_cu);
}

hipError_t launch_router1_proj(const Ctx &c, const RouterArgs &a, double *mid, double *bnd, float *sh_scale,
                               void *rec_buf, int mh, int I, int kind, size_t gs, const void *data, const void *scale,
                               float *xl) {
  if (!router1_proj_ok(a, c.num_cu, mh, I, kind, gs) || ((uintptr_t)data | (uintptr_t)xl) % 16 != 0)
    return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  const int npj = 2 * c.num_cu;  // 8 waves per CU, two rows each
  const dim3 grid(npj + a.E), block(256);
  KeyRec *rec = reinterpret_cast<KeyRec *>(rec_buf);
  const uint8_t *pd = (const uint8_t *)data, *ps = (const uint8_t *)scale;
  // hidden 7168 or 8192: four 32-value blocks per lane
  if (kind == RBT_QT_I4_GROUPED)
    launch_k(c, k_router1_proj<true, 4>, grid, block, P, mid, bnd, sh_scale, rec, pd, ps, mh, xl, npj);
  else
    launch_k(c, k_router1_proj<false, 4>, grid, block, P, mid, bnd, sh_scale, rec, pd, ps, mh, xl, npj);
  return hipGetLastError();
}

hipError_t launch_xgateup1s(const Ctx &c, const RouterArgs &a, const void *rec_buf, const double *mid,
                            const double *bnd, const GroupArgs &grp, int32_t *ids, float *wts, int *stats, int *gup,
                            int I, __bf16 *hp, bool has_shared) {
  if (I % 4 != 0 || c.num_cu < 2 || !grp.down_job || !grp.down_slot || !router1_ok(a, c.num_cu, nullptr))
    return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  const GroupOut G = group_out(grp, a.k);
  const KeyRec *rec = reinterpret_cast<const KeyRec *>(rec_buf);
  const dim3 grid(c.num_cu);
  const bool m4 = a.E <= 256;
  const RbtAct act{};
#define RBT_GU1S(M, N)                                                                                              \
  launch_k(c, k_xgateup1s<M, N, false>, grid, dim3(256), P, rec, mid, bnd, G, ids, wts, stats, gup, I, hp,          \
           (int)has_shared, grp.shv, a.x, act)
  if (a.H == 8192) {
    if (m4)
      RBT_GU1S(4, 16);
    else
      RBT_GU1S(8, 16);
  } else {
    if (m4)
      RBT_GU1S(4, 14);
    else
      RBT_GU1S(8, 14);
  }
#undef RBT_GU1S
  return hipGetLastError();
}

bool router1_latent_ok(const RouterArgs &a, int num_cu, int mh, int I) {
  const bool aligned = ((uintptr_t)a.x % 16 == 0) && ((uintptr_t)a.W % 16 == 0);
  return a.S == 1 && !(a.n_group > 1 && a.family != RBT_FAMILY_QWEN38) && a.E <= 1024 && a.E <= 4 * num_cu &&
         a.k + D1_KX <= D1_NC && (a.H == 8192 || a.H == 7168) && aligned && num_cu >= 2 && mh == 3584 &&
         I % 4 == 0 && (long)a.k * (I / 4) >= 4L * num_cu;
}

hipError_t launch_xgateup1s_latent(const Ctx &c, const RouterArgs &a, const void *rec_buf, const double *mid,
                                   const double *bnd, const GroupArgs &grp, int32_t *ids, float *wts, int *stats,
                                   int *gup, const float *xl, int mh, int I, float *h, const RbtAct &act) {
  if (!grp.down_job || !grp.down_slot || !router1_latent_ok(a, c.num_cu, mh, I) || (uintptr_t)xl % 16 != 0)
    return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  const GroupOut G = group_out(grp, a.k);
  const KeyRec *rec = reinterpret_cast<const KeyRec *>(rec_buf);
  launch_k(c, k_xgateup1s<16, 7, true>, dim3(c.num_cu), dim3(256), P, rec, mid, bnd, G, ids, wts, stats, gup, I,
           reinterpret_cast<__bf16 *>(h), 0, RbtExpertDev{}, xl, act);
  return hipGetLastError();
}

bool gu1s_gemv_ok(const RouterArgs &a, int num_cu, int kind, size_t gs, int I) {
  const bool aligned = ((uintptr_t)a.x % 16 == 0) && ((uintptr_t)a.W % 16 == 0);
  return a.S == 1 && !(a.n_group > 1 && a.family != RBT_FAMILY_QWEN38) && a.E <= 512 && a.E <= 4 * num_cu &&
         a.k + D1_KX <= D1_NC && a.H % 1024 == 0 && a.H <= RT_MAXH && aligned && num_cu >= 2 &&
         gu_act_ok(a.H, kind, gs) && I > 0;
}

hipError_t launch_gu1s_gemv(const Ctx &c, const RouterArgs &a, const void *rec_buf, const double *mid,
                            const double *bnd, const GroupArgs &grp, int32_t *ids, float *wts, int *stats, int kind,
                            size_t gs, int I, float *h, bool has_shared) {
  if (!grp.down_job || !grp.down_slot || !gu1s_gemv_ok(a, c.num_cu, kind, gs, I)) return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  const GroupOut G = group_out(grp, a.k);
  const KeyRec *rec = reinterpret_cast<const KeyRec *>(rec_buf);
  const dim3 grid(c.num_cu);
  const RbtAct act{};
  const bool i4 = kind == RBT_QT_I4_GROUPED, m4 = a.E <= 256;
  const int nb = (a.H / 32 + 63) / 64;
#define RBT_G1(M, NB_)                                                                                          \
  {                                                                                                             \
    if (i4)                                                                                                     \
      launch_k(c, k_gu1s_gemv<M, NB_, true>, grid, dim3(256), P, rec, mid, bnd, G, ids, wts, stats, I, h,        \
               (int)has_shared, act);                                                                           \
    else                                                                                                        \
      launch_k(c, k_gu1s_gemv<M, NB_, false>, grid, dim3(256), P, rec, mid, bnd, G, ids, wts, stats, I, h,       \
               (int)has_shared, act);                                                                           \
  }
  if (nb <= 2) {
    if (m4) RBT_G1(4, 2) else RBT_G1(8, 2)
  } else {
    if (m4) RBT_G1(4, 3) else RBT_G1(8, 3)
  }
#undef RBT_G1
  return hipGetLastError();
}

hipError_t launch_router1_any(const Ctx &c, const RouterArgs &a, double *mid, double *bnd, float *sh_scale,
                              const float *sgate, void *rec_buf) {
  if (a.S != 1 || a.H % 1024 != 0 || a.H > RT_MAXH || ((uintptr_t)a.x | (uintptr_t)a.W) % 16 != 0 ||
      (sgate && (uintptr_t)sgate % 16 != 0))
    return hipErrorInvalidValue;
  const SelParams P = sel_params(a);
  KeyRec *rec = reinterpret_cast<KeyRec *>(rec_buf);
  const int rn = a.E + (sgate ? 1 : 0);
  if (rn <= 4 * c.num_cu)
    launch_k(c, k_router1<1, false>, dim3(rn), dim3(256), P, sgate, mid, bnd, sh_scale, rec, nullptr, 0.0f, nullptr);
  else
    launch_k(c, k_router1<2, false>, dim3((rn + 1) / 2), dim3(256), P, sgate, mid, bnd, sh_scale, rec, nullptr, 0.0f,
             nullptr);
  return hipGetLastError();
}

hipError_t launch_logits_to_mid(const Ctx &c, const float *logits, size_t n, double *mid, double *bnd) {
  if (n == 0) return hipSuccess;
  launch_k(c, k_logits_to_mid, dim3((unsigned)((n + 255) / 256)), dim3(256), logits, n, mid, bnd);
  return hipGetLastError();
}

hipError_t launch_group(const Ctx &c, const int32_t *ids, const float *wts, int S, int k, int E,
                        const RbtExpertDev *table, const RbtExpertDev *shared_dev, RbtExpertDev *pair_job,
                        int *pair_tok, int *tok_pair, float *tok_w, int *err, int *nuniq) {
  if (S == 1) {
    launch_k(c, k_group_s1, dim3(1), dim3(((k + 1 + 63) / 64) * 64), ids, wts, k, E, table,
                       shared_dev, pair_job, pair_tok, tok_pair, tok_w, err);
  } else {
    // the picks go to LDS too while they fit (64 KB)
    const size_t base = (size_t)3 * E * sizeof(int), picks = (size_t)4 * S * k * sizeof(int);
    const int stage = base + picks <= 65536 ? 1 : 0;
    const size_t smem = base + (stage ? picks : 0);
    launch_ks(c, k_group, dim3(1), dim3(1024), (unsigned)smem, ids, wts, S, k, E, table, shared_dev, pair_job,
              pair_tok, tok_pair, tok_w, err, nuniq, stage);
  }
  return hipGetLastError();
}

hipError_t launch_combine(const Ctx &c, const float *y, int S, int k, int H, const int *tok_pair, const float *tok_w,
                          const float *sh_scale, int has_shared, int gated, float *out) {
  size_t n = (size_t)S * H;
  launch_k(c, k_combine, dim3((unsigned)((n + 255) / 256)), dim3(256), y, S, k, H, tok_pair, tok_w,
                     sh_scale, has_shared, gated, out);
  return hipGetLastError();
}

}  // namespace rbt
