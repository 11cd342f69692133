// norm.hip -- RMS norms of token rows and the residual add of the MoE sublayer.
//
// rmsnorm (kimi_linear/ops.rs:46-53) and rmsnorm_1p (qwen38/ops.rs:25-33) compute
//   r = 1 / sqrt((sum_f64(v^2) / n) as f32 + eps),   v[i] *= r * w[i]   (or r * (1 + w[i]))
// with every fp32 operation rounded on its own, as the reference does. The squares are exact in
// fp64; their sum is a parallel fp64 reduction (the reference's is sequential), so the fp32 mean
// square equals the reference's unless the exact value lies within a few fp64 ulps of an fp32
// rounding boundary. One workgroup per row.
#include "rbt_device.h"
#include "rbt_internal.h"

namespace rbt {

template <bool ONE_PLUS>
__global__ __launch_bounds__(256) void k_rmsnorm(const float *__restrict__ x, const float *__restrict__ w, float eps,
                                                 float *__restrict__ y, int n) {
  // rows up to 256 * R elements stay in registers: the row and the weights are loaded once, all
  // loads issued together (an element-by-element walk waits on memory once per element). Thread t
  // holds elements 1024 c + 4 t + e (c < R / 4, e < 4) and sums their squares in that order, the
  // order the one-token router launch uses when it normalises the token itself (router.hip
  // norm1p_chunks), so both give the same row bit for bit.
  constexpr int R = 32;
  __shared__ double part[4];
  const float *xr = x + (long)blockIdx.x * n;
  float *yr = y + (long)blockIdx.x * n;
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const bool held = n <= 256 * R;
  float v[R], wv[R];
  double acc = 0.0;
  if (held) {
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int i = 1024 * (j >> 2) + 4 * t + (j & 3);
      v[j] = i < n ? xr[i] : 0.0f;
      wv[j] = i < n ? w[i] : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < R; j++) acc += (double)v[j] * (double)v[j];
  } else {
    for (int i = t; i < n; i += 256) {
      const double e = (double)xr[i];
      acc += e * e;
    }
  }
  acc = rbt_wave_total_d(acc);
  if (lane == 0) part[wave] = acc;
  __syncthreads();
  const double ms = (part[0] + part[1]) + (part[2] + part[3]);
  const float r = __fdiv_rn(1.0f, rbt_sqrt_rn(__fadd_rn((float)(ms / (double)n), eps)));
  if (held) {
#pragma unroll
    for (int j = 0; j < R; j++) {
      const int i = 1024 * (j >> 2) + 4 * t + (j & 3);
      const float s = ONE_PLUS ? __fmul_rn(r, __fadd_rn(1.0f, wv[j])) : __fmul_rn(r, wv[j]);
      if (i < n) yr[i] = __fmul_rn(v[j], s);
    }
  } else {
    for (int i = t; i < n; i += 256) {
      const float s = ONE_PLUS ? __fmul_rn(r, __fadd_rn(1.0f, w[i])) : __fmul_rn(r, w[i]);
      yr[i] = __fmul_rn(xr[i], s);
    }
  }
}

// x[i] += t[i] (qwen38/generate.rs:411-413).
__global__ void k_add_rows(float *__restrict__ x, const float *__restrict__ t, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    x[i] = __fadd_rn(x[i], t[i]);
}

hipError_t launch_rmsnorm(const Ctx &c, const float *x, const float *w, float eps, float *y, size_t rows, size_t n,
                          bool one_plus) {
  if (rows == 0 || n == 0) return hipSuccess;
  if (n > (size_t)INT32_MAX || rows > (size_t)INT32_MAX) return hipErrorInvalidValue;
  if (one_plus)
    launch_k(c, k_rmsnorm<true>, dim3((unsigned)rows), dim3(256), x, w, eps, y, (int)n);
  else
    launch_k(c, k_rmsnorm<false>, dim3((unsigned)rows), dim3(256), x, w, eps, y, (int)n);
  return hipGetLastError();
}

hipError_t launch_add_rows(const Ctx &c, float *x, const float *t, size_t n) {
  if (n == 0) return hipSuccess;
  const size_t blocks = std::min<size_t>((n + 255) / 256, (size_t)c.num_cu * 8);
  launch_k(c, k_add_rows, dim3((unsigned)blocks), dim3(256), x, t, n);
  return hipGetLastError();
}

}  // namespace rbt
