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
#include <algorithm>

#include "rbt_device.h"
#include "rbt_gemv.h"
#include "rbt_internal.h"

namespace rbt {
template <int NB, int LPR, int U, int MODE, bool I4G, int CS, int PARTS>
__global__ __launch_bounds__(256) void k_decode_gemv(const RbtExpertDev *__restrict__ jobs, RbtExpertDev single,
                                                     int njobs, const int *__restrict__ njobs_dev,
                                                     const float *__restrict__ x, const int *__restrict__ x_index,
                                                     long x_stride, int cols, int rows, float *__restrict__ y,
                                                     long y_stride, const float *__restrict__ nw, float eps) {
  decode_gemv_body<NB, LPR, U, MODE, I4G, CS, PARTS>(jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols,
                                                     rows, y, y_stride, nw, eps,
                                                     blockIdx.x * (blockDim.x / RBT_WAVE) + threadIdx.x / RBT_WAVE,
                                                     gridDim.x * (blockDim.x / RBT_WAVE));
}

// Activation between the stacked gate/up GEMV and the down GEMV: h[p, k] = act(g, u) with g and
// u summed over the producer's column parts (gu per pair: PARTS gate vectors, then PARTS up vectors
// of `half` floats each). The activation rounds as the reference writes it (glm52/moe.rs:33-35,
// :58-70).
template <int PARTS>
__global__ __launch_bounds__(256) void k_swiglu(const float *__restrict__ gu, long gu_stride, int half, int npairs,
                                                const int *__restrict__ npairs_dev, RbtAct act, float *__restrict__ h) {
  int np = npairs;
  if (npairs_dev) np = min(np, *npairs_dev);
  const long n = (long)np * half;
  for (long idx = (long)blockIdx.x * blockDim.x + threadIdx.x; idx < n; idx += (long)gridDim.x * blockDim.x) {
    const long p = idx / half, k = idx - p * half;
    const float *g = gu + p * gu_stride;
    float gv = g[k], uv = g[PARTS * half + k];
#pragma unroll
    for (int j = 1; j < PARTS; j++) {
      gv += g[j * half + k];
      uv += g[(PARTS + j) * half + k];
    }
    h[idx] = rbt_act(act, gv, uv);
  }
}

// k_decode_gu_act: gate/up and the activation in one pass (gu_act_body, rbt_gemv.h).
template <int NB, bool I4G>
__global__ __launch_bounds__(256) void k_decode_gu_act(const RbtExpertDev *__restrict__ jobs, RbtExpertDev single,
                                                       int njobs, const int *__restrict__ njobs_dev,
                                                       const float *__restrict__ x, const int *__restrict__ x_index,
                                                       long x_stride, int cols, int I, RbtAct act,
                                                       float *__restrict__ h) {
  gu_act_body<NB, I4G>(jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols, I, act, h,
                       blockIdx.x * (blockDim.x / RBT_WAVE) + threadIdx.x / RBT_WAVE,
                       gridDim.x * (blockDim.x / RBT_WAVE));
}

bool gu_act_ok(size_t cols, int kind, size_t gs) {
  // (8192 columns would take four blocks per lane: 256 registers, one wave per SIMD)
  return decode_shape_ok(cols, kind, gs) && cols > 2048 && cols <= 6144;
}

hipError_t launch_gu_act(const Ctx &c, int kind, const RbtExpertDev *jobs, const RbtExpertDev &single, int njobs,
                         const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols, int I,
                         float *h, const RbtAct &act) {
  const long total = (long)njobs * I;
  if (total <= 0) return hipSuccess;
  if (total >= (1L << 31) || cols > 8192 || cols % 32 != 0) return hipErrorInvalidValue;
  long waves = (long)c.num_cu * 8;
  if (waves > total) waves = total;
  const int blocks = (int)((waves + 3) / 4);
  const int nb = (cols / 32 + 63) / 64;  // blocks per lane: 2 up to 4096 columns, 3 to 6144, 4 beyond
#define RBT_GUA(NB_)                                                                                              \
  {                                                                                                               \
    if (kind == RBT_QT_I4_GROUPED)                                                                                \
      launch_k(c, k_decode_gu_act<NB_, true>, dim3(blocks), dim3(256), jobs, single, njobs, njobs_dev, x, x_index, \
               x_stride, cols, I, act, h);                                                                        \
    else                                                                                                          \
      launch_k(c, k_decode_gu_act<NB_, false>, dim3(blocks), dim3(256), jobs, single, njobs, njobs_dev, x,        \
               x_index, x_stride, cols, I, act, h);                                                               \
  }
  if (nb <= 2)
    RBT_GUA(2)
  else if (nb == 3)
    RBT_GUA(3)
  else
    RBT_GUA(4)
#undef RBT_GUA
  return hipGetLastError();
}

hipError_t launch_swiglu(const Ctx &c, const float *gu, long gu_stride, int half, int npairs, const int *npairs_dev,
                         int parts, float *h, const RbtAct &act) {
  const long n = (long)npairs * half;
  if (n <= 0) return hipSuccess;
  const int blocks = (int)std::min<long>((n + 255) / 256, (long)c.num_cu * 4);
  if (parts == 2)
    launch_k(c, k_swiglu<2>, dim3(blocks), dim3(256), gu, gu_stride, half, npairs, npairs_dev,
                       act, h);
  else
    launch_k(c, k_swiglu<1>, dim3(blocks), dim3(256), gu, gu_stride, half, npairs, npairs_dev,
                       act, h);
  return hipGetLastError();
}

// Same contract as k_decode_gemv for any shape (odd columns, partial blocks, any group size):
// one wave per (job, row), lane t takes bytes t, t+64, ...
template <bool GATEUP>
__global__ __launch_bounds__(256) void k_pair_generic(const RbtExpertDev *__restrict__ jobs, RbtExpertDev single,
                                                      int njobs, const int *__restrict__ njobs_dev, int kind, int gs,
                                                      const float *__restrict__ x, const int *__restrict__ x_index,
                                                      long x_stride, int cols, int rows, float *__restrict__ y,
                                                      long y_stride, RbtAct act) {
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
  if (lane == 0) y[(long)u * y_stride + r] = GATEUP ? rbt_act(act, acc[0], acc[1]) : acc[0];
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
    launch_k(c, k_mxfp4_generic, grid, block, y, x, (const uint8_t *)data,
                       (const uint8_t *)scale, (int)s, (int)i, (int)o);
  else if (kind == RBT_QT_I4_GROUPED)
    launch_k(c, k_i4g_generic, grid, block, y, x, (const uint8_t *)data, (const float *)scale,
                       (int)gs, (int)s, (int)i, (int)o);
  else
    launch_k(c, k_f32_generic, grid, block, y, x, (const float *)data, (int)s, (int)i, (int)o);
  return hipGetLastError();
}

hipError_t launch_dequant(const Ctx &c, float *out, int kind, const void *data, const void *scale, size_t cols,
                          size_t gs, size_t row0, size_t nrows) {
  size_t total = nrows * cols;
  size_t blocks = (total + 255) / 256;
  if (blocks > 65536) blocks = 65536;
  if (blocks == 0) return hipSuccess;
  launch_k(c, k_dequant_rows, dim3((unsigned)blocks), dim3(256), out, kind, data, scale, cols, gs,
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

template <int NB, int LPR, int U, int MODE, bool I4G, int CS, int PARTS>
static hipError_t launch_decode_t(const Ctx &c, const RbtExpertDev *jobs, const RbtExpertDev &single, int njobs,
                                  const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols,
                                  int rows, float *y, long y_stride, int wpc, const float *nw, float eps) {
  constexpr int IPI = U * (RBT_WAVE / LPR);
  const long total = (long)njobs * rows * CS;
  if (total >= (1L << 31)) return hipErrorInvalidValue;
  // wpc waves per CU; each wave takes an equal contiguous run of rows (recomputed in-kernel from
  // the actual job count).
  long waves = (long)c.num_cu * wpc;
  long iters = (total + IPI - 1) / IPI;
  if (waves > iters) waves = iters;
  if (waves < 1) waves = 1;
  int blocks = (int)((waves + 3) / 4);
  launch_k(c, (k_decode_gemv<NB, LPR, U, MODE, I4G, CS, PARTS>), dim3(blocks), dim3(256), jobs,
                     single, njobs, njobs_dev, x, x_index, x_stride, cols, rows, y, y_stride, nw, eps);
  return hipGetLastError();
}

// Kernel shape per row length. Long rows (hidden = 6144..8192 columns) are split into two column
// parts of a whole wave each (x slice <= 128 floats per lane before the split, <= 64 after); short
// rows (moe_inter = 2048) take 32 lanes, two rows side by side and two unrolled.
// The stacked gate/up producer's split count is what the MODE_ACT consumer sums (parts_of()).
static int long_split(int cols) { return cols >= 4096 && cols % 64 == 0 && (cols / 64) % 32 == 0 ? 2 : 1; }

template <int MODE, bool I4G, int PARTS>
static hipError_t launch_decode_k(const Ctx &c, const RbtExpertDev *jobs, const RbtExpertDev &single, int njobs,
                                  const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols,
                                  int rows, float *y, long y_stride, const float *nw, float eps) {
#define RBT_DEC(NB, LPR, U, CS)                                                                                    \
  return launch_decode_t<NB, LPR, U, MODE, I4G, CS, PARTS>(c, jobs, single, njobs, njobs_dev, x, x_index, x_stride, \
                                                           cols, rows, y, y_stride, wpc, nw, eps)
  const int seg = MODE == MODE_STACKED ? rows / 2 : rows;  // rows of one matrix
  // One matrix of rows longer than 2048 columns (a projection): every wave reloads the whole x
  // slice for few rows, so half the waves, each with twice the rows, read less of it in total
  // (3584 x 7168 grouped int4: 10.3 us against 14.7 us at 8 waves per CU).
  const int wpc = ((MODE == MODE_DOWN || MODE == MODE_NORM) && njobs == 1 && cols > 2048) ? 4 : 8;
  const int nblk = cols / 32;
  if constexpr (MODE != MODE_NORM) {  // the norm keeps a row in one wave: none of the 16-lane shapes
  if (MODE == MODE_STACKED && long_split(cols) == 2 && seg % 2 == 0) {  // parts summed by MODE_ACT
    const int pblk = cols / 64;  // blocks per part
    if (pblk <= 64) RBT_DEC(1, 64, 2, 2);
    if (pblk <= 128) RBT_DEC(2, 64, 2, 2);
  }
  if (nblk <= 64 && nblk > 32 && seg % 4 == 0) RBT_DEC(1, 64, 4, 1);  // one x copy per wave
  if (nblk <= 64 && seg % 4 == 0) {
    if (nblk <= 16) RBT_DEC(1, 16, 1, 1);
    if (nblk <= 32) RBT_DEC(2, 16, 1, 1);
  }
  }
  if (nblk <= 64) RBT_DEC(1, 64, 1, 1);
  if (nblk <= 128) {  // 2080..4096 columns: two rows per iteration (K3's 3584 / 3072: 5.1 and 4.1 TB/s, U=1 4.4 and 3.5)
    if (seg % 2 == 0) RBT_DEC(2, 64, 2, 1);
    RBT_DEC(2, 64, 1, 1);
  }
  if (nblk <= 192) RBT_DEC(3, 64, 1, 1);
  RBT_DEC(4, 64, 1, 1);
#undef RBT_DEC
}

int decode_parts(int cols) { return long_split(cols); }

// k_proj1: one token through one matrix (proj1_body, rbt_gemv.h), one workgroup per CU.
constexpr int PJ_NW = 8;  // waves per workgroup of k_proj1

template <bool I4G, bool NORM, int NB>
__global__ __launch_bounds__(64 * PJ_NW) void k_proj1(const uint8_t *__restrict__ d, const uint8_t *__restrict__ sc,
                                                      const float *__restrict__ x, int cols, int rows,
                                                      float *__restrict__ y, const float *__restrict__ nw,
                                                      float eps) {
  __shared__ PjLds L;
  proj1_body<I4G, NORM, NB, PJ_NW>(L, d, sc, x, cols, rows, y, nw, eps, blockIdx.x, gridDim.x);
}

bool proj1_ok(int kind, size_t gs, int cols, int rows, int num_cu) {
  const bool fmt = kind == RBT_QT_MXFP4 || (kind == RBT_QT_I4_GROUPED && gs == 32);
  return fmt && cols % 32 == 0 && cols >= 64 * 32 && cols <= PJ_MAXC && rows > 0 &&
         (long)rows <= (long)PJ_RW * PJ_NW * num_cu;
}

hipError_t launch_proj1(const Ctx &c, int kind, size_t gs, const void *data, const void *scale, const float *x,
                        int cols, int rows, float *y, const float *nw, float eps) {
  if (!proj1_ok(kind, gs, cols, rows, c.num_cu) || ((uintptr_t)x | (uintptr_t)data) % 16 != 0 ||
      (nw && (uintptr_t)nw % 16 != 0))
    return hipErrorInvalidValue;
  const bool i4 = kind == RBT_QT_I4_GROUPED;
  const int nb = (cols / 32 + 63) / 64;
  const uint8_t *d = (const uint8_t *)data, *sc = (const uint8_t *)scale;
#define RBT_PJ(I4, NORM, NB_)                                                                                 \
  launch_k(c, k_proj1<I4, NORM, NB_>, dim3(c.num_cu), dim3(64 * PJ_NW), d, sc, x, cols, rows, y, nw, eps); \
  return hipGetLastError()
#define RBT_PJ_NB(I4, NORM)      \
  {                              \
    if (nb <= 2) {               \
      RBT_PJ(I4, NORM, 2);       \
    } else {                     \
      RBT_PJ(I4, NORM, 4);       \
    }                            \
  }
  if (i4) {
    if (nw) RBT_PJ_NB(true, true) else RBT_PJ_NB(true, false)
  } else {
    if (nw) RBT_PJ_NB(false, true) else RBT_PJ_NB(false, false)
  }
#undef RBT_PJ_NB
#undef RBT_PJ
}

// mode: 0 = plain rows (down / single matrix), 1 = stacked gate|up rows, 2 = plain rows with the
// SiLU-gated activation built from a stacked g|u input produced with `parts` column parts.
hipError_t launch_decode(const Ctx &c, int mode, int kind, const RbtExpertDev *jobs, const RbtExpertDev &single,
                         int njobs, const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols,
                         int rows, float *y, long y_stride, int parts, const float *nw, float eps) {
  if (njobs <= 0 || rows <= 0) return hipSuccess;
  const bool i4 = kind == RBT_QT_I4_GROUPED;
#define RBT_MODE(M, P)                                                                                              \
  return i4 ? launch_decode_k<M, true, P>(c, jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols, rows, y,   \
                                          y_stride, nw, eps)                                                        \
            : launch_decode_k<M, false, P>(c, jobs, single, njobs, njobs_dev, x, x_index, x_stride, cols, rows, y,  \
                                           y_stride, nw, eps)
  if (mode == MODE_NORM) {
    if (nw == nullptr || cols % 32 != 0 || cols > 64 * 32 * 4) return hipErrorInvalidValue;
    RBT_MODE(MODE_NORM, 1);
  }
  if (mode == MODE_STACKED) RBT_MODE(MODE_STACKED, 1);
  if (mode == MODE_ACT) {
    if (parts == 2) RBT_MODE(MODE_ACT, 2);
    RBT_MODE(MODE_ACT, 1);
  }
  RBT_MODE(MODE_DOWN, 1);
#undef RBT_MODE
}

// ------------------------------------------------------------------------------------------------
// One token: the down GEMV over a rank-ordered job list (the kk winners, then the shared expert)
// with the ordered combine fused. Workgroup b owns output rows [R0, R1) (whole iterations of IPI
// rows) of every job; its waves deal out the (job, row) items job-major in equal contiguous runs, so
// a wave reloads its x slice (the job's h row, at slots[job]) once per job of its run. Each row is
// computed as k_decode_gemv computes it (same blocks per lane, same reductions: bit-identical row
// sums). The sums land in LDS; thread r then combines row R0 + r in rank order with separate
// roundings, as k_combine does (acc = 0, acc += w_j y_j, then + the shared row, scaled by
// sh_scale[0] when gated; glm52/moe.rs:508-512, qwen38/generate.rs:303-349), and writes it. The
// combine's launch and its re-read of every row sum are saved.
// ------------------------------------------------------------------------------------------------
constexpr int DC_MAXJ = 33, DC_MAXR = 64;

template <int NB, int LPR, int U, int NW, bool I4G>
__global__ __launch_bounds__(64 * NW) void k_down1c(const RbtExpertDev *__restrict__ jobs,
                                                       const int *__restrict__ slots, int kk, int has_shared,
                                                       const float *__restrict__ h, long h_stride, int cols,
                                                       int rows, const float *__restrict__ tok_w,
                                                       const float *__restrict__ sh_scale, int gated,
                                                       float *__restrict__ out) {
  constexpr int RPI = RBT_WAVE / LPR, IPI = U * RPI;
  __shared__ float ys[DC_MAXJ][DC_MAXR];
  const int nj = kk + (has_shared ? 1 : 0);
  const int lane = threadIdx.x & (RBT_WAVE - 1), q = lane % LPR, sub = lane / LPR;
  const int w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int ntile = rows / IPI;
  const int T0 = (int)((long)blockIdx.x * ntile / gridDim.x), T1 = (int)((long)(blockIdx.x + 1) * ntile / gridDim.x);
  const int R0 = T0 * IPI, nr = (T1 - T0) * IPI;
  const int total = nj * nr;
  int per = (total + NW - 1) / NW;
  per = ((per + IPI - 1) / IPI) * IPI;
  int pos = w * per;
  const int end = min(pos + per, total);
  const int nblk = cols / 32;
  const unsigned rb = (unsigned)cols / 2;
  float xr[NB][32];
  float xs[NB];
  DecodeFrag<NB, U> f0, f1;
  while (pos < end) {
    // one job's rows [r, r1) of the workgroup's block
    const int job = pos / nr;
    int r = pos - job * nr;
    const int r1 = min(nr, r + (end - pos));
    pos += r1 - r;
    const RbtExpertDev J = jobs[job];
    const uint8_t *d = J.dd;
    const uint8_t *sc = reinterpret_cast<const uint8_t *>(J.ds);
    float *yrow = ys[job];
    if (d == nullptr) {
      for (int rr = r + lane; rr < r1; rr += RBT_WAVE) yrow[rr] = 0.0f;
      continue;
    }
    // the first weights go out before the x slice is read; then ping-pong as k_decode_gemv
    frag_load<NB, LPR, U, I4G>(f0, d, sc, R0 + r, q, sub, nblk, rb, nblk);
    load_x_slice<NB, LPR>(xr, xs, h + (long)slots[job] * h_stride, q, nblk);
    const int rlast = r1 - IPI;
    while (true) {
      frag_load<NB, LPR, U, I4G>(f1, d, sc, R0 + min(r + IPI, rlast), q, sub, nblk, rb, nblk);
      frag_reduce_store<NB, LPR, U, I4G>(f0, xr, xs, yrow + r, q, sub, nblk);
      if (r + IPI >= r1) break;
      frag_load<NB, LPR, U, I4G>(f0, d, sc, R0 + min(r + 2 * IPI, rlast), q, sub, nblk, rb, nblk);
      frag_reduce_store<NB, LPR, U, I4G>(f1, xr, xs, yrow + r + IPI, q, sub, nblk);
      r += 2 * IPI;
      if (r >= r1) break;
    }
  }
  __syncthreads();
  const int t = threadIdx.x;
  if (t < nr) {
    float acc = 0.0f;
    for (int j = 0; j < kk; j++) acc = __fadd_rn(acc, __fmul_rn(tok_w[j], ys[j][t]));
    if (has_shared) {
      float sh = ys[kk][t];
      if (gated) sh = __fmul_rn(sh, sh_scale[0]);
      acc = __fadd_rn(acc, sh);
    }
    out[R0 + t] = acc;
  }
}

// Blocks per lane as k_decode_gemv's MODE_DOWN takes them for these columns (so the sums are the
// same bits; the rows per iteration do not change them): 1025..2048 columns one block per lane, in
// 8 waves with 4 rows per iteration (C2's inter 2048: 18.6 us against 19.9 in 16 waves); 2049..4096
// two, in 16 waves with one row per iteration (K3's 3584 x 3072: 23.1 us against 24.5 with 2 rows,
// whose 16-wave build spills, and 24.4 in 8 waves with 2 rows). Returns the rows per iteration.
static int down1c_ipi(int cols) {
  const int nblk = cols / 32;
  return nblk > 32 && nblk <= 64 ? 4 : nblk > 64 && nblk <= 128 ? 1 : 0;
}

bool down1c_ok(int kind, size_t gs, int njobs, int cols, int rows, int num_cu) {
  if (!decode_shape_ok((size_t)cols, kind, gs) || njobs < 1 || njobs > DC_MAXJ || num_cu <= 0) return false;
  const int ipi = down1c_ipi(cols);
  if (ipi == 0 || rows <= 0 || rows % ipi != 0) return false;
  const int ntile = rows / ipi;
  return (long)ipi * ((ntile + num_cu - 1) / num_cu) <= DC_MAXR;
}

hipError_t launch_down1c(const Ctx &c, int kind, size_t gs, const RbtExpertDev *jobs, const int *slots, int kk,
                         int has_shared, const float *h, long h_stride, int cols, int rows, const float *tok_w,
                         const float *sh_scale, int gated, float *out) {
  const int nj = kk + (has_shared ? 1 : 0);
  if (!down1c_ok(kind, gs, nj, cols, rows, c.num_cu) || (gated && !sh_scale)) return hipErrorInvalidValue;
  const bool i4 = kind == RBT_QT_I4_GROUPED;
  const dim3 grid(c.num_cu);
#define RBT_DC(NB, U, NW)                                                                                           \
  {                                                                                                                 \
    if (i4)                                                                                                         \
      launch_k(c, k_down1c<NB, 64, U, NW, true>, grid, dim3(64 * NW), jobs, slots, kk, has_shared, h, h_stride,     \
               cols, rows, tok_w, sh_scale, gated, out);                                                            \
    else                                                                                                            \
      launch_k(c, k_down1c<NB, 64, U, NW, false>, grid, dim3(64 * NW), jobs, slots, kk, has_shared, h, h_stride,    \
               cols, rows, tok_w, sh_scale, gated, out);                                                            \
  }
  if (down1c_ipi(cols) == 4)
    RBT_DC(1, 4, 8)
  else
    RBT_DC(2, 1, 16)
#undef RBT_DC
  return hipGetLastError();
}

hipError_t launch_pair_generic(const Ctx &c, bool gateup, int kind, size_t gs, const RbtExpertDev *jobs,
                               const RbtExpertDev &single, int njobs, const int *njobs_dev, const float *x,
                               const int *x_index, long x_stride, int cols, int rows, float *y, long y_stride,
                               const RbtAct &act) {
  long items = (long)njobs * rows;
  if (items <= 0) return hipSuccess;
  dim3 grid((unsigned)((items + 3) / 4)), block(256);
  if (gateup)
    launch_k(c, k_pair_generic<true>, grid, block, jobs, single, njobs, njobs_dev, kind, (int)gs, x,
                       x_index, x_stride, cols, rows, y, y_stride, act);
  else
    launch_k(c, k_pair_generic<false>, grid, block, jobs, single, njobs, njobs_dev, kind, (int)gs, x,
                       x_index, x_stride, cols, rows, y, y_stride, act);
  return hipGetLastError();
}

}  // namespace rbt
