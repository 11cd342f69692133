// gemv.hip -- dequant-GEMV kernels for gfx950: y[S,O] = x[S,I] . W^T with W in MXFP4, grouped
// int4 or f32 (kernels.rs:113-124, :228-296).
//
// Two families:
//  * Decode kernels (one token per weight row, the hot path). A row is split over LPR lanes
//    (16, 32 or 64); lane q owns the 32-element blocks b = q + LPR*j (j < NB). One block of MXFP4
//    is 16 bytes of E2M1 nibbles (one global_load_dwordx4) plus one E8M0 byte; one block of
//    grouped int4 (group_size 32) is 16 bytes of nibbles plus one f32 scale. The lane's slice of
//    x (32*NB floats) lives in registers for as many rows as the wave processes, so HBM traffic is
//    the weight bytes alone. Each wave streams a contiguous run of rows; consecutive lanes read
//    consecutive 16-byte blocks, so every load instruction covers LPR*16 contiguous bytes per row.
//    The per-row partial sums are reduced over the LPR lanes with a butterfly.
//  * Generic kernels for any shape, alignment and token count (tails, odd columns, partial
//    blocks), one wave per output row.
//
// Accumulation is fp32 with fused multiply-add; the reference's sequential sum is reassociated
// (within the 1e-5 relative-L2 contract), the dequantized weight itself is exact.
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
#pragma unroll
  for (int j = 0; j < NB; j++) {
    int b = q + LPR * j;
    float s = 0.0f;
    if (b < nblk) {
      const float4 *p = reinterpret_cast<const float4 *>(x + 32 * b);
#pragma unroll
      for (int t = 0; t < 8; t++) {
        float4 v = p[t];
        xr[j][4 * t + 0] = v.x;
        xr[j][4 * t + 1] = v.y;
        xr[j][4 * t + 2] = v.z;
        xr[j][4 * t + 3] = v.w;
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

// Partial dot of one MXFP4 row over this lane's blocks.
template <int NB, int LPR>
__device__ __forceinline__ float row_dot_mxfp4(const uint8_t *__restrict__ rowd, const uint8_t *__restrict__ rows,
                                               int q, int nblk, const float (&xr)[NB][32]) {
  rbt_u4 w[NB];
  uint32_t sb[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    int b = q + LPR * j;
    if (b < nblk) {
      w[j] = __builtin_nontemporal_load(reinterpret_cast<const rbt_u4 *>(rowd) + b);
      sb[j] = rows[b];
    } else {
      w[j] = rbt_u4{0u, 0u, 0u, 0u};
      sb[j] = 127;
    }
  }
  float acc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    float sc = rbt_e8m0(sb[j]);
    float a = 0.0f;
    a = fp4_dword_dot(w[j].x, sc, &xr[j][0], a);
    a = fp4_dword_dot(w[j].y, sc, &xr[j][8], a);
    a = fp4_dword_dot(w[j].z, sc, &xr[j][16], a);
    a = fp4_dword_dot(w[j].w, sc, &xr[j][24], a);
    acc[j] = a;
  }
  float r = 0.0f;
#pragma unroll
  for (int j = 0; j < NB; j++) r += acc[j];
  return r;
}

// Partial dot of one grouped-int4 row (group_size 32) over this lane's blocks.
template <int NB, int LPR>
__device__ __forceinline__ float row_dot_i4g(const uint8_t *__restrict__ rowd, const float *__restrict__ rows, int q,
                                             int nblk, const float (&xr)[NB][32], const float (&xs)[NB]) {
  rbt_u4 w[NB];
  float sc[NB];
#pragma unroll
  for (int j = 0; j < NB; j++) {
    int b = q + LPR * j;
    if (b < nblk) {
      w[j] = __builtin_nontemporal_load(reinterpret_cast<const rbt_u4 *>(rowd) + b);
      sc[j] = rows[b];
    } else {
      w[j] = rbt_u4{0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u};
      sc[j] = 0.0f;
    }
  }
  float r = 0.0f;
#pragma unroll
  for (int j = 0; j < NB; j++) {
    float a = 0.0f;
    a = i4_dword_dot(w[j].x, &xr[j][0], a);
    a = i4_dword_dot(w[j].y, &xr[j][8], a);
    a = i4_dword_dot(w[j].z, &xr[j][16], a);
    a = i4_dword_dot(w[j].w, &xr[j][24], a);
    // sum_k x_k (n_k - 8) = sum_k x_k n_k - 8 sum_k x_k, then the group scale.
    r = __builtin_fmaf(__builtin_fmaf(-8.0f, xs[j], a), sc[j], r);
  }
  return r;
}

// ------------------------------------------------------------------------------------------------
// Decode kernel over a job table. Each job u is one expert (or one plain matrix):
//   GATEUP: y[u*y_stride + r] = silu(gate_u[r] . x_u) * (up_u[r] . x_u), r < rows
//   else:   y[u*y_stride + r] = down_u[r] . x_u
// with x_u = x + tok(u)*x_stride, tok(u) = x_index[u] (or u when x_index is null). The flattened
// (job, row) range is split into equal contiguous runs, one per wave, so a wave reloads its x slice
// only when the token changes. A job whose weights are absent (null pointers) yields zeros.
// ------------------------------------------------------------------------------------------------
template <int NB, int LPR, bool GATEUP, bool I4G>
__global__ __launch_bounds__(256) void k_decode_gemv(const RbtExpertDev *__restrict__ jobs, RbtExpertDev single,
                                                     int njobs, const int *__restrict__ njobs_dev,
                                                     const float *__restrict__ x, const int *__restrict__ x_index,
                                                     long x_stride, int cols, int rows, float *__restrict__ y,
                                                     long y_stride) {
  constexpr int RPI = RBT_WAVE / LPR;  // rows per wave iteration
  const int lane = threadIdx.x & (RBT_WAVE - 1);
  const int q = lane % LPR, sub = lane / LPR;
  const long nwaves = (long)gridDim.x * (blockDim.x / RBT_WAVE);
  const long wave = (long)blockIdx.x * (blockDim.x / RBT_WAVE) + threadIdx.x / RBT_WAVE;
  int nj = njobs;
  if (njobs_dev) nj = min(nj, *njobs_dev);
  const long total = (long)nj * rows;
  long per = (total + nwaves - 1) / nwaves;
  per = ((per + RPI - 1) / RPI) * RPI;
  const long begin = wave * per;
  if (begin >= total) return;
  const long end = min(begin + per, total);

  const int nblk = cols / 32;
  const size_t rb = (size_t)cols / 2;
  const size_t sstride = (size_t)nblk;  // scale elements per row (u8 for MXFP4, f32 for I4G)

  float xr[NB][32];
  float xs[NB];
  long cur = -1;

  for (long base = begin; base < end; base += RPI) {
    const long item = base + sub;
    const bool valid = item < end;
    const int u = valid ? (int)(item / rows) : (int)((end - 1) / rows);
    const int r = valid ? (int)(item % rows) : 0;
    const long tok = x_stride == 0 ? 0 : (x_index ? (long)x_index[u] : (long)u);
    if (tok != cur) {
      load_x_slice<NB, LPR>(xr, xs, x + tok * x_stride, q, nblk);
      cur = tok;
    }
    const RbtExpertDev J = jobs ? jobs[u] : single;
    float a = 0.0f, b = 0.0f;
    if (GATEUP) {
      if (J.gd && J.ud) {
        if (I4G) {
          a = row_dot_i4g<NB, LPR>(J.gd + r * rb, reinterpret_cast<const float *>(J.gs) + r * sstride, q, nblk, xr, xs);
          b = row_dot_i4g<NB, LPR>(J.ud + r * rb, reinterpret_cast<const float *>(J.us) + r * sstride, q, nblk, xr, xs);
        } else {
          a = row_dot_mxfp4<NB, LPR>(J.gd + r * rb, reinterpret_cast<const uint8_t *>(J.gs) + r * sstride, q, nblk, xr);
          b = row_dot_mxfp4<NB, LPR>(J.ud + r * rb, reinterpret_cast<const uint8_t *>(J.us) + r * sstride, q, nblk, xr);
        }
      }
      b = rbt_group_sum<LPR>(b);
    } else if (J.dd) {
      if (I4G)
        a = row_dot_i4g<NB, LPR>(J.dd + r * rb, reinterpret_cast<const float *>(J.ds) + r * sstride, q, nblk, xr, xs);
      else
        a = row_dot_mxfp4<NB, LPR>(J.dd + r * rb, reinterpret_cast<const uint8_t *>(J.ds) + r * sstride, q, nblk, xr);
    }
    a = rbt_group_sum<LPR>(a);
    if (valid && q == 0) y[(long)u * y_stride + r] = GATEUP ? rbt_silu(a) * b : a;
  }
}

// Same contract as k_decode_gemv for any shape (odd columns, partial blocks, any group size):
// one wave per (job, row), lane t takes bytes t, t+64, ...
template <bool GATEUP>
__global__ __launch_bounds__(256) void k_pair_generic(const RbtExpertDev *__restrict__ jobs, RbtExpertDev single,
                                                      int njobs, const int *__restrict__ njobs_dev, int kind, int gs,
                                                      const float *__restrict__ x, const int *__restrict__ x_index,
                                                      long x_stride, int cols, int rows, float *__restrict__ y,
                                                      long y_stride) {
  const int lane = threadIdx.x & 63;
  const long item = (long)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  int nj = njobs;
  if (njobs_dev) nj = min(nj, *njobs_dev);
  if (item >= (long)nj * rows) return;
  const int u = (int)(item / rows), r = (int)(item % rows);
  const RbtExpertDev J = jobs ? jobs[u] : single;
  const float *xs = x + (x_stride == 0 ? 0 : (x_index ? (long)x_index[u] : (long)u) * x_stride);
  const size_t rb = ((size_t)cols + 1) / 2;
  const size_t ns = kind == RBT_QT_MXFP4 ? ((size_t)cols + 31) / 32 : ((size_t)cols + gs - 1) / gs;
  float acc[2] = {0.0f, 0.0f};
  for (int m = 0; m < (GATEUP ? 2 : 1); m++) {
    const uint8_t *w = GATEUP ? (m == 0 ? J.gd : J.ud) : J.dd;
    const void *sc = GATEUP ? (m == 0 ? J.gs : J.us) : J.ds;
    if (!w) continue;
    w += (size_t)r * rb;
    float a = 0.0f;
    for (size_t bi = lane; bi < rb; bi += 64) {
      uint32_t byte = w[bi];
      for (int h = 0; h < 2; h++) {
        size_t k = 2 * bi + h;
        if (k >= (size_t)cols) break;
        uint32_t nib = h ? (byte >> 4) : (byte & 0xF);
        float wv;
        if (kind == RBT_QT_MXFP4)
          wv = rbt_e2m1(nib) * rbt_e8m0(reinterpret_cast<const uint8_t *>(sc)[r * ns + k / 32]);
        else
          wv = (float)((int)nib - 8) * reinterpret_cast<const float *>(sc)[r * ns + k / gs];
        a = __builtin_fmaf(xs[k], wv, a);
      }
    }
    acc[m] = rbt_group_sum<64>(a);
  }
  if (lane == 0) y[(long)u * y_stride + r] = GATEUP ? rbt_silu(acc[0]) * acc[1] : acc[0];
}

// ------------------------------------------------------------------------------------------------
// Generic kernels: any S, I, O, alignment. One wave per output row; lane t takes bytes t, t+64, ...
// ------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_mxfp4_generic(float *__restrict__ y, const float *__restrict__ x,
                                                       const uint8_t *__restrict__ data,
                                                       const uint8_t *__restrict__ bscale, int s, int i, int o) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  if (row >= o) return;
  const size_t rb = ((size_t)i + 1) / 2, bpr = ((size_t)i + 31) / 32;
  const uint8_t *w = data + row * rb;
  const uint8_t *bs = bscale + row * bpr;
  for (int si = 0; si < s; si++) {
    const float *xs = x + (size_t)si * i;
    float acc = 0.0f;
    for (size_t bi = lane; bi < rb; bi += 64) {
      uint32_t byte = w[bi];
      size_t k = 2 * bi;
      float sc = rbt_e8m0(bs[k / 32]);
      acc = __builtin_fmaf(xs[k], rbt_e2m1(byte & 0xF) * sc, acc);
      if (k + 1 < (size_t)i) acc = __builtin_fmaf(xs[k + 1], rbt_e2m1(byte >> 4) * sc, acc);
    }
    acc = rbt_group_sum<64>(acc);
    if (lane == 0) y[(size_t)si * o + row] = acc;
  }
}

__global__ __launch_bounds__(256) void k_i4g_generic(float *__restrict__ y, const float *__restrict__ x,
                                                     const uint8_t *__restrict__ q4, const float *__restrict__ scale,
                                                     int gs, int s, int i, int o) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  if (row >= o) return;
  const size_t rb = ((size_t)i + 1) / 2, ng = ((size_t)i + gs - 1) / gs;
  const uint8_t *w = q4 + row * rb;
  const float *sc = scale + row * ng;
  for (int si = 0; si < s; si++) {
    const float *xs = x + (size_t)si * i;
    float acc = 0.0f;
    for (size_t bi = lane; bi < rb; bi += 64) {
      uint32_t byte = w[bi];
      size_t k = 2 * bi;
      acc = __builtin_fmaf(xs[k], (float)((int)(byte & 0xF) - 8) * sc[k / gs], acc);
      if (k + 1 < (size_t)i) acc = __builtin_fmaf(xs[k + 1], (float)((int)(byte >> 4) - 8) * sc[(k + 1) / gs], acc);
    }
    acc = rbt_group_sum<64>(acc);
    if (lane == 0) y[(size_t)si * o + row] = acc;
  }
}

__global__ __launch_bounds__(256) void k_f32_generic(float *__restrict__ y, const float *__restrict__ x,
                                                     const float *__restrict__ w, int s, int i, int o) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * (blockDim.x / 64) + threadIdx.x / 64;
  if (row >= o) return;
  const float *wr = w + (size_t)row * i;
  for (int si = 0; si < s; si++) {
    const float *xs = x + (size_t)si * i;
    float acc = 0.0f;
    for (int k = lane; k < i; k += 64) acc = __builtin_fmaf(xs[k], wr[k], acc);
    acc = rbt_group_sum<64>(acc);
    if (lane == 0) y[(size_t)si * o + row] = acc;
  }
}

// Dequantize rows [row0, row0 + nrows) bit-exactly (QT::row_f32, quant.rs:280-341): one IEEE f32
// multiply of the exact element by the exact scale, as the reference does.
__global__ void k_dequant_rows(float *__restrict__ out, int kind, const void *__restrict__ data,
                               const void *__restrict__ scale, size_t cols, size_t gs, size_t row0, size_t nrows) {
  size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  size_t total = nrows * cols;
  for (; idx < total; idx += (size_t)gridDim.x * blockDim.x) {
    size_t r = row0 + idx / cols, k = idx % cols;
    if (kind == RBT_QT_F32) {
      out[idx] = reinterpret_cast<const float *>(data)[r * cols + k];
      continue;
    }
    size_t rb = (cols + 1) / 2;
    uint32_t byte = reinterpret_cast<const uint8_t *>(data)[r * rb + (k >> 1)];
    uint32_t nib = (k & 1) ? (byte >> 4) : (byte & 0xF);
    if (kind == RBT_QT_MXFP4) {
      size_t bpr = (cols + 31) / 32;
      out[idx] = __fmul_rn(rbt_e2m1(nib), rbt_e8m0(reinterpret_cast<const uint8_t *>(scale)[r * bpr + k / 32]));
    } else {
      size_t ng = (cols + gs - 1) / gs;
      out[idx] = __fmul_rn((float)((int)nib - 8), reinterpret_cast<const float *>(scale)[r * ng + k / gs]);
    }
  }
}

// ------------------------------------------------------------------------------------------------
// Host-side launchers.
// ------------------------------------------------------------------------------------------------
static int grid_for_rows(long rows) { return (int)((rows + 3) / 4); }

hipError_t launch_generic(const Ctx &c, int kind, float *y, const float *x, const void *data, const void *scale,
                          size_t gs, size_t s, size_t i, size_t o) {
  dim3 grid(grid_for_rows((long)o)), block(256);
  if (kind == RBT_QT_MXFP4)
    hipLaunchKernelGGL(k_mxfp4_generic, grid, block, 0, c.stream, y, x, (const uint8_t *)data,
                       (const uint8_t *)scale, (int)s, (int)i, (int)o);
  else if (kind == RBT_QT_I4_GROUPED)
    hipLaunchKernelGGL(k_i4g_generic, grid, block, 0, c.stream, y, x, (const uint8_t *)data, (const float *)scale,
                       (int)gs, (int)s, (int)i, (int)o);
  else
    hipLaunchKernelGGL(k_f32_generic, grid, block, 0, c.stream, y, x, (const float *)data, (int)s, (int)i, (int)o);
  return hipGetLastError();
}

hipError_t launch_dequant(const Ctx &c, float *out, int kind, const void *data, const void *scale, size_t cols,
                          size_t gs, size_t row0, size_t nrows) {
  size_t total = nrows * cols;
  size_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks == 0) return hipSuccess;
  hipLaunchKernelGGL(k_dequant_rows, dim3((unsigned)blocks), dim3(256), 0, c.stream, out, kind, data, scale, cols, gs,
                     row0, nrows);
  return hipGetLastError();
}

// Picks (LPR, NB) for a row of `cols` elements: the fewest lanes per row that keep NB <= 4, so a
// lane's x slice is at most 128 registers.
bool decode_shape_ok(size_t cols, int kind, size_t gs) {
  if (cols == 0 || cols % 32 != 0) return false;
  if (kind == RBT_QT_I4_GROUPED && gs != 32) return false;
  if (kind != RBT_QT_MXFP4 && kind != RBT_QT_I4_GROUPED) return false;
  return cols / 32 <= 256;  // up to 8192 columns
}

template <int NB, int LPR, bool GATEUP, bool I4G>
static hipError_t launch_decode_t(const Ctx &c, const RbtExpertDev *jobs, const RbtExpertDev &single, int njobs,
                                  const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols,
                                  int rows, float *y, long y_stride) {
  constexpr int RPI = RBT_WAVE / LPR;
  long total = (long)njobs * rows;
  // About 8 waves per CU; each wave takes an equal contiguous run of rows (computed in-kernel from
  // the actual job count).
  long waves = (long)c.num_cu * 8;
  long iters = (total + RPI - 1) / RPI;
  if (waves > iters) waves = iters;
  if (waves < 1) waves = 1;
  int blocks = (int)((waves + 3) / 4);
  hipLaunchKernelGGL((k_decode_gemv<NB, LPR, GATEUP, I4G>), dim3(blocks), dim3(256), 0, c.stream, jobs, single, njobs,
                     njobs_dev, x, x_index, x_stride, cols, rows, y, y_stride);
  return hipGetLastError();
}

template <bool GATEUP, bool I4G>
static hipError_t launch_decode_k(const Ctx &c, const RbtExpertDev *jobs, const RbtExpertDev &single, int njobs,
                                  const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols,
                                  int rows, float *y, long y_stride) {
#define RBT_DEC(NB, LPR) \
  return launch_decode_t<NB, LPR, GATEUP, I4G>(c, jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols, rows, y, y_stride)
  int nblk = cols / 32;
  if (nblk <= 16) RBT_DEC(1, 16);
  if (nblk <= 32) RBT_DEC(2, 16);
  if (nblk <= 48) RBT_DEC(3, 16);
  if (nblk <= 64) RBT_DEC(4, 16);
  if (nblk <= 96) RBT_DEC(3, 32);
  if (nblk <= 128) RBT_DEC(4, 32);
  if (nblk <= 192) RBT_DEC(3, 64);
  RBT_DEC(4, 64);
#undef RBT_DEC
}

hipError_t launch_decode(const Ctx &c, bool gateup, int kind, const RbtExpertDev *jobs, const RbtExpertDev &single,
                         int njobs, const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols,
                         int rows, float *y, long y_stride) {
  if (njobs <= 0 || rows <= 0) return hipSuccess;
  if (kind == RBT_QT_I4_GROUPED)
    return gateup ? launch_decode_k<true, true>(c, jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols, rows, y, y_stride)
                  : launch_decode_k<false, true>(c, jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols, rows, y, y_stride);
  return gateup ? launch_decode_k<true, false>(c, jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols, rows, y, y_stride)
                : launch_decode_k<false, false>(c, jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols, rows, y, y_stride);
}

hipError_t launch_pair_generic(const Ctx &c, bool gateup, int kind, size_t gs, const RbtExpertDev *jobs,
                               const RbtExpertDev &single, int njobs, const int *njobs_dev, const float *x,
                               const int *x_index, long x_stride, int cols, int rows, float *y, long y_stride) {
  long items = (long)njobs * rows;
  if (items <= 0) return hipSuccess;
  dim3 grid((unsigned)((items + 3) / 4)), block(256);
  if (gateup)
    hipLaunchKernelGGL(k_pair_generic<true>, grid, block, 0, c.stream, jobs, single, njobs, njobs_dev, kind, (int)gs, x,
                       x_index, x_stride, cols, rows, y, y_stride);
  else
    hipLaunchKernelGGL(k_pair_generic<false>, grid, block, 0, c.stream, jobs, single, njobs, njobs_dev, kind, (int)gs, x,
                       x_index, x_stride, cols, rows, y, y_stride);
  return hipGetLastError();
}

}  // namespace rbt
