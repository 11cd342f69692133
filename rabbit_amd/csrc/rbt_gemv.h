// rbt_gemv.h -- the decode GEMV's device code (gemv.hip), shared with kernels that run it beside
// other work in one launch (router.hip: the latent projection beside the one-token selection).
//
// Decode GEMV: y[S,O] = x[S,I] . W^T with W in MXFP4 or grouped int4 (kernels.rs:228-296), one token
// per weight row. A row is split over LPR lanes (16, 32 or 64); lane q owns the 32-element blocks
// b = q + LPR*j (j < NB). One block of MXFP4 is 16 bytes of E2M1 nibbles (one global_load_dwordx4)
// plus one E8M0 byte; one block of grouped int4 (group_size 32) is 16 bytes of nibbles plus one f32
// scale. The lane's slice of x (32*NB floats) lives in registers for as many rows as the wave
// processes, so HBM traffic is the weight bytes alone. Each wave streams a contiguous run of rows;
// consecutive lanes read consecutive 16-byte blocks, so every load instruction covers LPR*16
// contiguous bytes per row. The per-row partial sums are reduced over the LPR lanes with a
// butterfly. Accumulation is fp32 with fused multiply-add; the reference's sequential sum is
// reassociated (within the 1e-5 relative-L2 contract), the dequantized weight itself is exact.
#pragma once
#include "rbt_device.h"
#include "rbt_internal.h"

namespace rbt {

// ------------------------------------------------------------------------------------------------
// MXFP4 block dot: 32 E2M1 codes (one uint4) times 32 activations, scaled by the block's E8M0.
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ float fp4_dword_dot(uint32_t w, float sc, const float *xv, float acc) {
  rbt_f2 v0 = RBT_FP4X2(w, sc, 0);
  rbt_f2 v1 = RBT_FP4X2(w, sc, 1);
  rbt_f2 v2 = RBT_FP4X2(w, sc, 2);
  rbt_f2 v3 = RBT_FP4X2(w, sc, 3);
  acc = __builtin_fmaf(xv[0], v0.x, acc);
  acc = __builtin_fmaf(xv[1], v0.y, acc);
  acc = __builtin_fmaf(xv[2], v1.x, acc);
  acc = __builtin_fmaf(xv[3], v1.y, acc);
  acc = __builtin_fmaf(xv[4], v2.x, acc);
  acc = __builtin_fmaf(xv[5], v2.y, acc);
  acc = __builtin_fmaf(xv[6], v3.x, acc);
  acc = __builtin_fmaf(xv[7], v3.y, acc);
  return acc;
}

// Grouped int4: nibble n encodes n-8. Returns sum_k x_k * n_k (unsigned codes); the caller folds in
// -8 * sum_k x_k and the group scale.
__device__ __forceinline__ float i4_dword_dot(uint32_t w, const float *xv, float acc) {
  uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
  acc = __builtin_fmaf(xv[0], (float)(lo & 0xFFu), acc);
  acc = __builtin_fmaf(xv[1], (float)(hi & 0xFFu), acc);
  acc = __builtin_fmaf(xv[2], (float)((lo >> 8) & 0xFFu), acc);
  acc = __builtin_fmaf(xv[3], (float)((hi >> 8) & 0xFFu), acc);
  acc = __builtin_fmaf(xv[4], (float)((lo >> 16) & 0xFFu), acc);
  acc = __builtin_fmaf(xv[5], (float)((hi >> 16) & 0xFFu), acc);
  acc = __builtin_fmaf(xv[6], (float)(lo >> 24), acc);
  acc = __builtin_fmaf(xv[7], (float)(hi >> 24), acc);
  return acc;
}

template <int NB, int LPR>
__device__ __forceinline__ void load_x_slice(float (&xr)[NB][32], float (&xs)[NB], const float *__restrict__ x,
                                             int q, int nblk) {
  // unconditional loads from a clamped (in-bounds) block, then zeroed: no branches around loads,
  // so the compiler can count outstanding loads instead of draining them.
  const rbt_gf4 *xg = (const rbt_gf4 *)x;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int b = q + LPR * j;
    const bool ok = b < nblk;
    const int bb = ok ? b : nblk - 1;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const float4 v = xg[8 * bb + t];
      xr[j][4 * t + 0] = ok ? v.x : 0.0f;
      xr[j][4 * t + 1] = ok ? v.y : 0.0f;
      xr[j][4 * t + 2] = ok ? v.z : 0.0f;
      xr[j][4 * t + 3] = ok ? v.w : 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < NB; j++) {
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 32; t++) s += xr[j][t];
    xs[j] = s;
  }
}

// rmsnorm of a row held as a whole wave's x slice (64 lanes, blocks q + 64j), in place:
// r = 1/sqrt((sum_f64(v^2) / n) as f32 + eps), v *= r * w (kimi_linear/ops.rs:46-53), then the
// block sums again as load_x_slice forms them. The fp64 sum runs in another order than k_rmsnorm's.
template <int NB>
__device__ __forceinline__ void norm_x_slice(float (&xr)[NB][32], float (&xs)[NB], const float *__restrict__ w,
                                             float eps, int q, int nblk, int n) {
  // the weights' loads go out first and land while the sum of squares is reduced
  const rbt_gf4 *wg = (const rbt_gf4 *)w;
  float4 wv[NB][8];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int bb = min(q + 64 * j, nblk - 1);
#pragma unroll
    for (int t = 0; t < 8; t++) wv[j][t] = wg[8 * bb + t];
  }
  double acc = 0.0;
#pragma unroll
  for (int j = 0; j < NB; j++)
#pragma unroll
    for (int t = 0; t < 32; t++) acc += (double)xr[j][t] * (double)xr[j][t];  // zero past the row
  acc = rbt_wave_total_d(acc);
  const float r = __fdiv_rn(1.0f, rbt_sqrt_rn(__fadd_rn((float)(acc / (double)n), eps)));
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const bool ok = q + 64 * j < nblk;
#pragma unroll
    for (int t = 0; t < 8; t++) {
      const float4 v = wv[j][t];
      xr[j][4 * t + 0] = ok ? __fmul_rn(xr[j][4 * t + 0], __fmul_rn(r, v.x)) : 0.0f;
      xr[j][4 * t + 1] = ok ? __fmul_rn(xr[j][4 * t + 1], __fmul_rn(r, v.y)) : 0.0f;
      xr[j][4 * t + 2] = ok ? __fmul_rn(xr[j][4 * t + 2], __fmul_rn(r, v.z)) : 0.0f;
      xr[j][4 * t + 3] = ok ? __fmul_rn(xr[j][4 * t + 3], __fmul_rn(r, v.w)) : 0.0f;
    }
  }
#pragma unroll
  for (int j = 0; j < NB; j++) {
    float s = 0.0f;
#pragma unroll
    for (int t = 0; t < 32; t++) s += xr[j][t];
    xs[j] = s;
  }
}



// ------------------------------------------------------------------------------------------------
// Decode kernel over a job table. Each job u is one expert (or one plain matrix); MODE selects the
// matrix and the activation:
//   MODE_DOWN   : y[u*y_stride + r] = down_u[r] . x_u                         (r < rows)
//   MODE_STACKED: gate_u and up_u as one [2*half, cols] matrix: rows [0, half) are gate's, rows
//                 [half, 2*half) up's; y[u*y_stride + r] = that row . x_u     (r < rows = 2*half)
//   MODE_ACT    : like MODE_DOWN, but the activation is built on the fly from a stacked gate/up
//                 result g|u (2*cols floats): x_k = silu(g_k) * u_k (glm52/moe.rs:33-80).
// x_u = x + tok(u)*x_stride with tok(u) = x_index[u] (or u when x_index is null).
// The flattened (job, row) range is split into equal contiguous runs, one per wave. An iteration
// covers U * (64/LPR) consecutive rows; the next iteration's blocks are loaded before the current
// one is reduced (double buffering), so a wave keeps two iterations of weight bytes in flight. With
// U > 1 the host guarantees rows % (U * 64/LPR) == 0 (an iteration never straddles two jobs). A
// job whose weights are absent (null pointers) yields zeros.
// ------------------------------------------------------------------------------------------------
enum { MODE_DOWN = 0, MODE_STACKED = 1, MODE_ACT = 2, MODE_NORM = 3 };  // NORM: MODE_DOWN of rmsnorm(x)

template <int NB, int U>
struct DecodeFrag {
  rbt_u4 w[U][NB];
  uint32_t sb[U][NB];  // E8M0 byte (MXFP4) or f32 bits (I4G)
};

// Loads the blocks of IPI = U * (64/LPR) consecutive rows starting at `row` (a row pointer into
// `d`, rows rb bytes apart; scales `sc`, nblk per row). Lane (sub, q) takes rows row + u*RPI + sub.
// Every load is unconditional (blocks past nblk re-read block nblk-1; block_dots drops them), so
// the loop body is straight-line and the next iteration's loads stay in flight during this one's
// arithmetic.
template <int NB, int LPR, int U, bool I4G>
__device__ __forceinline__ void frag_load(DecodeFrag<NB, U> &f, const uint8_t *__restrict__ d,
                                          const uint8_t *__restrict__ sc, int row, int q, int sub, int nblk,
                                          unsigned rb, int sstride) {
  constexpr int RPI = RBT_WAVE / LPR;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const unsigned r = (unsigned)(row + u * RPI + sub);
    const rbt_gu4 *rp = (const rbt_gu4 *)(d + (size_t)r * rb);
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int b = q + LPR * j;
      const int bb = min(b, nblk - 1);
      f.w[u][j] = __builtin_nontemporal_load(rp + bb);
      if (I4G)
        f.sb[u][j] = ((const rbt_gu32 *)sc)[(size_t)r * sstride + bb];
      else
        f.sb[u][j] = ((const rbt_gu8 *)sc)[(size_t)r * sstride + bb];
    }
  }
}

// Blocks b = q + LPR*j past nblk hold a re-read of block nblk-1 (frag_load) and contribute nothing.
template <int NB, int LPR, bool I4G>
__device__ __forceinline__ float block_dots(const rbt_u4 (&w)[NB], const uint32_t (&sb)[NB], const float (&xr)[NB][32],
                                            const float (&xs)[NB], int q, int nblk) {
  float r = 0.0f;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    float a = 0.0f;
    if (I4G) {
      a = i4_dword_dot(w[j].x, &xr[j][0], a);
      a = i4_dword_dot(w[j].y, &xr[j][8], a);
      a = i4_dword_dot(w[j].z, &xr[j][16], a);
      a = i4_dword_dot(w[j].w, &xr[j][24], a);
      // sum_k x_k (n_k - 8) = sum_k x_k n_k - 8 sum_k x_k, then the group scale.
      const float t = __builtin_fmaf(__builtin_fmaf(-8.0f, xs[j], a), __uint_as_float(sb[j]), r);
      r = (q + LPR * j < nblk) ? t : r;
    } else {
      const float sc = rbt_e8m0(sb[j]);
      a = fp4_dword_dot(w[j].x, sc, &xr[j][0], a);
      a = fp4_dword_dot(w[j].y, sc, &xr[j][8], a);
      a = fp4_dword_dot(w[j].z, sc, &xr[j][16], a);
      a = fp4_dword_dot(w[j].w, sc, &xr[j][24], a);
      r += (q + LPR * j < nblk) ? a : 0.0f;
    }
  }
  return r;
}

// x slice for MODE_ACT: x_k = silu(g_k) * u_k from a stacked gate/up result. The producer may have
// split its rows into PARTS column ranges: gu holds PARTS partial gate vectors, then PARTS partial
// up vectors (cols floats each), summed here.
template <int PARTS>
__device__ __forceinline__ float4 sum_parts(const float *__restrict__ p, int cols, int off) {
  float4 v = *reinterpret_cast<const float4 *>(p + off);
#pragma unroll
  for (int h = 1; h < PARTS; h++) {
    const float4 w = *reinterpret_cast<const float4 *>(p + h * cols + off);
    v.x += w.x;
    v.y += w.y;
    v.z += w.z;
    v.w += w.w;
  }
  return v;
}

template <int NB, int LPR, int PARTS>
__device__ __forceinline__ void load_act_slice(float (&xr)[NB][32], float (&xs)[NB], const float *__restrict__ gu,
                                               int q, int nblk, int cols) {
#pragma unroll
  for (int j = 0; j < NB; j++) {
    const int b = q + LPR * j;
    float s = 0.0f;
    if (b < nblk) {
#pragma unroll
      for (int t = 0; t < 8; t++) {
        const float4 g = sum_parts<PARTS>(gu, cols, 32 * b + 4 * t);
        const float4 u = sum_parts<PARTS>(gu + PARTS * cols, cols, 32 * b + 4 * t);
        xr[j][4 * t + 0] = rbt_silu(g.x) * u.x;
        xr[j][4 * t + 1] = rbt_silu(g.y) * u.y;
        xr[j][4 * t + 2] = rbt_silu(g.z) * u.z;
        xr[j][4 * t + 3] = rbt_silu(g.w) * u.w;
      }
#pragma unroll
      for (int t = 0; t < 32; t++) s += xr[j][t];
    } else {
#pragma unroll
      for (int t = 0; t < 32; t++) xr[j][t] = 0.0f;
    }
    xs[j] = s;
  }
}

template <int NB, int LPR, int U, bool I4G>
__device__ __forceinline__ void frag_reduce_store(const DecodeFrag<NB, U> &f, const float (&xr)[NB][32],
                                                  const float (&xs)[NB], float *__restrict__ yrow, int q, int sub,
                                                  int nblk) {
  constexpr int RPI = RBT_WAVE / LPR;
#pragma unroll
  for (int u = 0; u < U; u++) {
    float a = block_dots<NB, LPR, I4G>(f.w[u], f.sb[u], xr, xs, q, nblk);
    a = rbt_group_sum<LPR>(a);
    if (q == 0) yrow[u * RPI + sub] = a;
    // one row at a time: keeps the scheduler from decoding every row's nibbles up front, which
    // would cost 32 registers per block and halve the waves per SIMD.
    __builtin_amdgcn_sched_barrier(0);
  }
}

// The decode GEMV of one wave: wave `wave` of `nwaves` (the kernel's whole grid, or the part of a
// grid that runs it beside other work).
template <int NB, int LPR, int U, int MODE, bool I4G, int CS, int PARTS>
__device__ __forceinline__ void decode_gemv_body(const RbtExpertDev *__restrict__ jobs, RbtExpertDev single,
                                                 int njobs, const int *__restrict__ njobs_dev,
                                                 const float *__restrict__ x, const int *__restrict__ x_index,
                                                 long x_stride, int cols, int rows, float *__restrict__ y,
                                                 long y_stride, const float *__restrict__ nw, float eps, int wave_in,
                                                 int nwaves) {
  static_assert(MODE != MODE_NORM || (LPR == 64 && CS == 1), "the norm needs the whole row in one wave");
  constexpr int RPI = RBT_WAVE / LPR;  // rows side by side in one wave
  constexpr int IPI = U * RPI;         // rows per iteration
  const int lane = threadIdx.x & (RBT_WAVE - 1);
  const int q = lane % LPR, sub = lane / LPR;
  const int wave = __builtin_amdgcn_readfirstlane(wave_in);
  int nj = njobs;
  if (njobs_dev) nj = min(nj, *njobs_dev);
  // Each logical row of `cols` columns is processed as CS column ranges ("parts"), so a lane's x
  // slice covers cols/CS columns. A segment is a run of rows of one matrix and one part: per job,
  // MODE_STACKED has 2*CS segments (gate parts, then up parts), the other modes CS. `rows` counts
  // logical rows per job (2*half for MODE_STACKED); segment lengths are multiples of IPI.
  const int seg = MODE == MODE_STACKED ? rows / 2 : rows;
  const int nseg_job = (rows / seg) * CS;
  const int total = nj * seg * nseg_job;
  int per = (total + nwaves - 1) / nwaves;
  per = ((per + IPI - 1) / IPI) * IPI;
  int pos = wave * per;
  if (pos >= total) return;
  const int end = min(pos + per, total);

  const int pcols = cols / CS;  // columns of one part
  const int nblk = pcols / 32;
  const unsigned rb = (unsigned)cols / 2;

  float xr[NB][32];
  float xs[NB];
  long cur = -1;
  DecodeFrag<NB, U> f0, f1;

  while (pos < end) {
    // one segment: rows [r, r1) of matrix (job, part)
    const int sidx = pos / seg;
    const int job = sidx / nseg_job, sj = sidx - job * nseg_job;
    const int mat = sj / CS, h = sj - mat * CS;  // matrix (gate/up for MODE_STACKED), column part
    int r = pos - sidx * seg;
    const int r1 = min(seg, r + (end - pos));
    pos += r1 - r;
    const RbtExpertDev J = jobs ? jobs[job] : single;
    const uint8_t *d = MODE == MODE_STACKED ? (mat ? J.ud : J.gd) : J.dd;
    const uint8_t *sc = reinterpret_cast<const uint8_t *>(MODE == MODE_STACKED ? (mat ? J.us : J.gs) : J.ds);
    float *yrow = y + (long)job * y_stride + (long)sj * seg;
    if (d == nullptr) {
      for (int rr = r + lane; rr < r1; rr += RBT_WAVE) yrow[rr] = 0.0f;
      continue;
    }
    d += (size_t)h * (pcols / 2);                         // part h of every row
    sc += (size_t)h * nblk * (I4G ? 4 : 1);
    // ping-pong over iterations of IPI rows: the next iteration's blocks are in flight while the
    // current one is reduced. The first weight loads go out before the activation slice is read.
    frag_load<NB, LPR, U, I4G>(f0, d, sc, r, q, sub, nblk, rb, CS * nblk);
    const long tok = x_stride == 0 ? 0 : (x_index ? (long)x_index[job] : (long)job);
    if (tok * CS + h != cur) {
      if (MODE == MODE_ACT)
        load_act_slice<NB, LPR, PARTS>(xr, xs, x + tok * x_stride, q, nblk, cols);
      else
        load_x_slice<NB, LPR>(xr, xs, x + tok * x_stride + (long)h * pcols, q, nblk);
      if constexpr (MODE == MODE_NORM) norm_x_slice<NB>(xr, xs, nw, eps, q, nblk, cols);
      cur = tok * CS + h;
    }
    // The prefetch is unconditional: past the segment's last iteration it re-reads that iteration
    // (rlast), so every load sits in straight-line code.
    const int rlast = r1 - IPI;
    while (true) {
      frag_load<NB, LPR, U, I4G>(f1, d, sc, min(r + IPI, rlast), q, sub, nblk, rb, CS * nblk);
      frag_reduce_store<NB, LPR, U, I4G>(f0, xr, xs, yrow + r, q, sub, nblk);
      if (r + IPI >= r1) break;
      frag_load<NB, LPR, U, I4G>(f0, d, sc, min(r + 2 * IPI, rlast), q, sub, nblk, rb, CS * nblk);
      frag_reduce_store<NB, LPR, U, I4G>(f1, xr, xs, yrow + r + IPI, q, sub, nblk);
      r += 2 * IPI;
      if (r >= r1) break;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Gate/up and the activation in one pass, for rows of 2049..6144 columns (one token per pair, one
// column part): a wave takes a contiguous run of (pair, r) items; for each it streams gate row r and
// up row r of the pair's expert, reduces both as k_decode_gemv does (block_dots, the wave sum), and
// lane 0 writes h[p, r] = act(g, u). Below 4096 columns the g and u values are the stacked kernel's,
// so h is bit-identical to k_decode_gemv (stacked) + k_swiglu; from 4096 columns on the stacked
// kernel sums two column parts (g0 + g1) where this one reduces the whole row, so the two agree
// only within the fp32 accumulation tolerance there. The gate|up scratch and one launch are saved.
// Two items in flight per wave.
template <int NB, bool I4G>
__device__ __forceinline__ void frag_load_gu(DecodeFrag<NB, 2> &f, const RbtExpertDev &J, int row, int q, int nblk,
                                             unsigned rb) {
#pragma unroll
  for (int m = 0; m < 2; m++) {
    const uint8_t *d = m ? J.ud : J.gd;
    const uint8_t *sc = reinterpret_cast<const uint8_t *>(m ? J.us : J.gs);
    const rbt_gu4 *rp = (const rbt_gu4 *)(d + (size_t)row * rb);
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int bb = min(q + 64 * j, nblk - 1);
      f.w[m][j] = __builtin_nontemporal_load(rp + bb);
      if (I4G)
        f.sb[m][j] = ((const rbt_gu32 *)sc)[(size_t)row * nblk + bb];
      else
        f.sb[m][j] = ((const rbt_gu8 *)sc)[(size_t)row * nblk + bb];
    }
  }
}

// The wave's gate and up sums of one row, as values uniform across the wave (lane 0's total, which
// is what the stacked kernel stores).
template <int NB, bool I4G>
__device__ __forceinline__ void frag_gu_sums(const DecodeFrag<NB, 2> &f, const float (&xr)[NB][32],
                                             const float (&xs)[NB], int q, int nblk, float &g, float &u) {
  g = block_dots<NB, 64, I4G>(f.w[0], f.sb[0], xr, xs, q, nblk);
  g = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rbt_group_sum<64>(g)), 0));
  __builtin_amdgcn_sched_barrier(0);
  u = block_dots<NB, 64, I4G>(f.w[1], f.sb[1], xr, xs, q, nblk);
  u = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(rbt_group_sum<64>(u)), 0));
  __builtin_amdgcn_sched_barrier(0);
}

// The wave `wave_in` of `nwaves` (the kernel's grid, or the part of a grid that runs it beside other
// work): its contiguous run of (pair, row) items. `jobs` may point at LDS.
template <int NB, bool I4G>
__device__ __forceinline__ void gu_act_body(const RbtExpertDev *__restrict__ jobs, RbtExpertDev single, int njobs,
                                            const int *__restrict__ njobs_dev, const float *__restrict__ x,
                                            const int *__restrict__ x_index, long x_stride, int cols, int I,
                                            const RbtAct &act, float *__restrict__ h, int wave_in, int nwaves) {
  const int q = threadIdx.x & (RBT_WAVE - 1);
  const int wave = __builtin_amdgcn_readfirstlane(wave_in);
  int nj = njobs;
  if (njobs_dev) nj = min(nj, *njobs_dev);
  const int total = nj * I;
  const int per = (total + nwaves - 1) / nwaves;
  int pos = wave * per;
  if (pos >= total) return;
  const int end = min(pos + per, total);
  const int nblk = cols / 32;
  const unsigned rb = (unsigned)cols / 2;
  float xr[NB][32];
  float xs[NB];
  long cur = -1;
  DecodeFrag<NB, 2> f0, f1;
  while (pos < end) {
    // one run: rows [r, r1) of pair `job`
    const int job = pos / I;
    int r = pos - job * I;
    const int r1 = min(I, r + (end - pos));
    pos += r1 - r;
    const RbtExpertDev J = jobs ? jobs[job] : single;
    float *hrow = h + (long)job * I;
    if (J.gd == nullptr || J.ud == nullptr) {  // no expert: g = u = 0, act(0, 0) = 0
      for (int rr = r + q; rr < r1; rr += RBT_WAVE) hrow[rr] = 0.0f;
      continue;
    }
    frag_load_gu<NB, I4G>(f0, J, r, q, nblk, rb);
    const long tok = x_stride == 0 ? 0 : (x_index ? (long)x_index[job] : (long)job);
    if (tok != cur) {
      load_x_slice<NB, 64>(xr, xs, x + tok * x_stride, q, nblk);
      cur = tok;
    }
    // rows' sums collect in lane (row - wb) of a 64-row window; the activation then runs once per
    // window on all lanes (on one lane per row it would serialise the whole wave)
    int wb = r;
    float gk = 0.0f, uk = 0.0f;
    auto take = [&](const DecodeFrag<NB, 2> &f, int rr) {
      float g, u;
      frag_gu_sums<NB, I4G>(f, xr, xs, q, nblk, g, u);
      if (q == rr - wb) {
        gk = g;
        uk = u;
      }
      if (rr - wb == RBT_WAVE - 1 || rr + 1 == r1) {
        if (q <= rr - wb) hrow[wb + q] = rbt_act(act, gk, uk);
        wb = rr + 1;
      }
    };
    const int rlast = r1 - 1;
    while (true) {
      frag_load_gu<NB, I4G>(f1, J, min(r + 1, rlast), q, nblk, rb);
      take(f0, r);
      if (r + 1 >= r1) break;
      frag_load_gu<NB, I4G>(f0, J, min(r + 2, rlast), q, nblk, rb);
      take(f1, r + 1);
      r += 2;
      if (r >= r1) break;
    }
  }
}

// ------------------------------------------------------------------------------------------------
// One token through one matrix (a projection of up to 8192 columns, MXFP4 or grouped int4 with
// groups of 32). The decode GEMV above keeps a slice of x per wave in registers, which at one
// matrix of long rows means every wave reloads all of x for two or three rows and runs at one
// wave per SIMD. Here each workgroup stages x once in LDS (32-value blocks padded to 36 floats, so
// lanes reading consecutive blocks hit distinct banks) and each wave holds only its rows' weights:
// a wave's (at most PJ_RW) rows go out as one batch of loads at kernel entry, ahead of the staging.
// Per row the lane arithmetic is block_dots' (blocks q + 64 j, the same fused multiply-adds and
// -8 fold) and the wave sum rbt_group_sum<64>; the block sums of x for the fold are added as a
// tree. NORM: x is first replaced by rmsnorm(x) * nw (norm_x_slice's arithmetic; the fp64 sum of
// squares is formed over the workgroup, in another order).
// ------------------------------------------------------------------------------------------------
constexpr int PJ_MAXC = 8192, PJ_RW = 4;  // columns, rows per wave

struct PjLds {
  __attribute__((aligned(16))) float xs[PJ_MAXC / 32 * 36];
  float bsum[PJ_MAXC / 32];
  double red[16];
};

// Workgroup wg of nwg (NW waves each) runs rows [r0, r1) of its waves, at most RW per wave.
template <bool I4G, bool NORM, int NB, int NW, int RW = PJ_RW>
__device__ __forceinline__ void proj1_body(PjLds &L, const uint8_t *__restrict__ d, const uint8_t *__restrict__ sc,
                                           const float *__restrict__ x, int cols, int rows, float *__restrict__ y,
                                           const float *__restrict__ nw, float eps, int wg, int nwg) {
  static_assert(NW <= 16, "the reduction slots");
  float *xs = L.xs, *bsum = L.bsum;
  double *red = L.red;
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int nblk = cols / 32;
  const long NWT = (long)nwg * NW, wi = (long)wg * NW + w;
  const int r0 = (int)(wi * rows / NWT), r1 = (int)((wi + 1) * rows / NWT);
  const unsigned rb = (unsigned)cols / 2;
  // x first (one float4 per thread and step): the memory counter retires loads in issue order, so
  // the staging below waits for x only, not for the weights issued after it
  constexpr int XV = PJ_MAXC / 4 / (64 * NW);
  const int n4 = cols / 4;
  float4 xv4[XV], nw4[NORM ? XV : 1];
#pragma unroll
  for (int k = 0; k < XV; k++) xv4[k] = ((const rbt_gf4 *)x)[min(t + 64 * NW * k, n4 - 1)];
  if (NORM)  // the norm's weights too (loaded after the rows, waiting for them would wait for the rows)
#pragma unroll
    for (int k = 0; k < XV; k++) nw4[k] = ((const rbt_gf4 *)nw)[min(t + 64 * NW * k, n4 - 1)];
  __builtin_amdgcn_sched_barrier(0);
  // the wave's rows (clamped: a wave without rows re-reads row 0 and stores nothing)
  rbt_u4 wr[RW][NB];
  uint32_t sb[RW][NB];
#pragma unroll
  for (int u = 0; u < RW; u++) {
    const int r = r1 > r0 ? min(r0 + u, r1 - 1) : 0;
    const rbt_gu4 *rp = (const rbt_gu4 *)(d + (size_t)r * rb);
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int bb = min(lane + 64 * j, nblk - 1);
      wr[u][j] = __builtin_nontemporal_load(rp + bb);
      sb[u][j] = I4G ? ((const rbt_gu32 *)sc)[(size_t)r * nblk + bb] : ((const rbt_gu8 *)sc)[(size_t)r * nblk + bb];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // x into LDS (with the norm: after scaling), and for grouped int4 the 32-value block sums (chunk
  // sums added over the block's eight lanes). Barriers here are LDS-only: the weights stay in flight.
  double sq = 0.0;
  auto put = [&](int i, const float4 &v) {
    *reinterpret_cast<float4 *>(&xs[(i >> 3) * 36 + 4 * (i & 7)]) = v;
    if (I4G) {
      const float bsv = rbt_group_sum<8>(__fadd_rn(__fadd_rn(__fadd_rn(v.x, v.y), v.z), v.w));
      if ((i & 7) == 0) bsum[i >> 3] = bsv;
    }
  };
#pragma unroll
  for (int k = 0; k < XV; k++) {
    const int i = t + 64 * NW * k;
    if (i < n4) {
      const float4 v = xv4[k];
      if (NORM)
        sq += (double)v.x * v.x + (double)v.y * v.y + (double)v.z * v.z + (double)v.w * v.w;
      else
        put(i, v);
    }
  }
  if (NORM) {
    sq = rbt_wave_total_d(sq);
    if (lane == 0) red[w] = sq;
    lds_barrier();
    double tot = 0.0;
#pragma unroll
    for (int i = 0; i < NW; i++) tot += red[i];
    const float r = __fdiv_rn(1.0f, rbt_sqrt_rn(__fadd_rn((float)(tot / (double)cols), eps)));
#pragma unroll
    for (int k = 0; k < XV; k++) {
      const int i = t + 64 * NW * k;
      if (i < n4) {
        const float4 g = nw4[k];
        float4 v = xv4[k];
        v.x = __fmul_rn(v.x, __fmul_rn(r, g.x));
        v.y = __fmul_rn(v.y, __fmul_rn(r, g.y));
        v.z = __fmul_rn(v.z, __fmul_rn(r, g.z));
        v.w = __fmul_rn(v.w, __fmul_rn(r, g.w));
        put(i, v);
      }
    }
  }
  lds_barrier();
#pragma unroll
  for (int u = 0; u < RW; u++) {
    if (r0 + u >= r1) break;
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < NB; j++) {
      const int b = lane + 64 * j;
      const int bb = min(b, nblk - 1);
      float xv[32];
#pragma unroll
      for (int k = 0; k < 8; k++) {
        const float4 v = *reinterpret_cast<const float4 *>(&xs[bb * 36 + 4 * k]);
        xv[4 * k] = v.x;
        xv[4 * k + 1] = v.y;
        xv[4 * k + 2] = v.z;
        xv[4 * k + 3] = v.w;
      }
      float a = 0.0f;
      if (I4G) {
        a = i4_dword_dot(wr[u][j].x, &xv[0], a);
        a = i4_dword_dot(wr[u][j].y, &xv[8], a);
        a = i4_dword_dot(wr[u][j].z, &xv[16], a);
        a = i4_dword_dot(wr[u][j].w, &xv[24], a);
        const float tt = __builtin_fmaf(__builtin_fmaf(-8.0f, bsum[bb], a), __uint_as_float(sb[u][j]), acc);
        acc = b < nblk ? tt : acc;
      } else {
        const float scv = rbt_e8m0(sb[u][j]);
        a = fp4_dword_dot(wr[u][j].x, scv, &xv[0], a);
        a = fp4_dword_dot(wr[u][j].y, scv, &xv[8], a);
        a = fp4_dword_dot(wr[u][j].z, scv, &xv[16], a);
        a = fp4_dword_dot(wr[u][j].w, scv, &xv[24], a);
        acc += b < nblk ? a : 0.0f;
      }
    }
    acc = rbt_group_sum<64>(acc);
    if (lane == 0) y[r0 + u] = acc;
  }
}


}  // namespace rbt
