// synth.hip -- synthetic expert weights generated in place in HBM (benchmarks and tests).
//
// Counter-based: every 8-byte word and every scale is a pure function of (seed, index), so a
// 13.7 GB resident pool is filled without a host staging copy, and any byte can be regenerated on
// the host bit for bit. Data: byte j of word w is bits [8j, 8j+8) of mix64(seed_d + w). MXFP4
// scale idx: exp_lo + floor(hi32(mix64(seed_s + idx)) * (exp_hi - exp_lo + 1) / 2^32). I4G scale
// idx: s_lo + (s_hi - s_lo) * u, u = (top 24 bits of mix64(seed_s + idx)) * 2^-24, each operation
// rounded on its own. seed_d = mix64(2*seed + 1), seed_s = mix64(2*seed + 2). mix64 is the
// splitmix64 finaliser.
#include "rbt_device.h"
#include "rbt_internal.h"

namespace rbt {

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

__global__ void k_synth_bytes(uint8_t *__restrict__ data, size_t nbytes, uint64_t seed_d) {
  size_t nw = (nbytes + 7) / 8;
  for (size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x; w < nw; w += (size_t)gridDim.x * blockDim.x) {
    uint64_t h = mix64(seed_d + w);
    size_t b0 = w * 8;
    if (b0 + 8 <= nbytes && ((uintptr_t)(data + b0) & 7) == 0) {
      *reinterpret_cast<uint64_t *>(data + b0) = h;
    } else {
      for (int j = 0; j < 8; j++)
        if (b0 + j < nbytes) data[b0 + j] = (uint8_t)(h >> (8 * j));
    }
  }
}

__global__ void k_synth_e8m0(uint8_t *__restrict__ scale, size_t n, uint64_t seed_s, uint32_t lo, uint64_t span) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint64_t h = mix64(seed_s + i);
    scale[i] = (uint8_t)(lo + (((h >> 32) * span) >> 32));
  }
}

__global__ void k_synth_f32scale(float *__restrict__ scale, size_t n, uint64_t seed_s, float lo, float hi) {
  float span = __fsub_rn(hi, lo);
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    uint64_t h = mix64(seed_s + i);
    float u = __fmul_rn((float)(uint32_t)(h >> 40), 0x1p-24f);
    scale[i] = __fadd_rn(lo, __fmul_rn(span, u));
  }
}

static unsigned grid_for(size_t n) {
  size_t g = (n + 255) / 256;
  if (g > 65536) g = 65536;
  return (unsigned)(g ? g : 1);
}

hipError_t launch_synth_mxfp4(const Ctx &c, uint8_t *data, uint8_t *scale, size_t rows, size_t cols, uint64_t seed,
                              uint32_t lo, uint32_t hi) {
  uint64_t sd = mix64(seed * 2 + 1), ss = mix64(seed * 2 + 2);
  size_t nb = rows * ((cols + 1) / 2), ns = rows * ((cols + 31) / 32);
  launch_k(c, k_synth_bytes, dim3(grid_for((nb + 7) / 8)), dim3(256), data, nb, sd);
  launch_k(c, k_synth_e8m0, dim3(grid_for(ns)), dim3(256), scale, ns, ss, lo,
                     (uint64_t)(hi - lo + 1));
  return hipGetLastError();
}

hipError_t launch_synth_i4g(const Ctx &c, uint8_t *data, float *scale, size_t rows, size_t cols, size_t gs,
                            uint64_t seed, float lo, float hi) {
  uint64_t sd = mix64(seed * 2 + 1), ss = mix64(seed * 2 + 2);
  size_t nb = rows * ((cols + 1) / 2), ns = rows * ((cols + gs - 1) / gs);
  launch_k(c, k_synth_bytes, dim3(grid_for((nb + 7) / 8)), dim3(256), data, nb, sd);
  launch_k(c, k_synth_f32scale, dim3(grid_for(ns)), dim3(256), scale, ns, ss, lo, hi);
  return hipGetLastError();
}

}  // namespace rbt
