// rbt_device.h -- gfx950 device helpers shared by the kernels.
//
// Wave size is 64 on CDNA4. All device code is built with -ffp-contract=off: the combine and
// activation math rounds every product and sum separately (as the reference does); the dot-product
// inner loops use explicit fmaf.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define RBT_WAVE 64

typedef float rbt_f2 __attribute__((ext_vector_type(2)));
typedef unsigned int rbt_u4 __attribute__((ext_vector_type(4)));

// e8m0_decode (quant.rs:391-396): byte 0 is the subnormal 2^-127, every other byte is the f32
// biased exponent field (255 -> +inf).
__device__ __forceinline__ float rbt_e8m0(uint32_t b) {
  return __uint_as_float(b == 0 ? (1u << 22) : (b << 23));
}

// e2m1_decode (quant.rs:353-356) by bit construction: sign bit 3, exponent bits 2..1 (bias 1),
// mantissa bit 0. exp 0 is the subnormal {0, 0.5}; code 8 gives -0.0.
__device__ __forceinline__ float rbt_e2m1(uint32_t n) {
  uint32_t e = (n >> 1) & 3u, m = n & 1u;
  uint32_t mag = e ? (((125u + e + 1u) << 23) | (m << 22)) : (m ? 0x3F000000u : 0u);
  return __uint_as_float(mag | ((n & 8u) << 28));
}

// Two E2M1 codes (byte `sel` of `w`: low nibble -> .x, high nibble -> .y), each times `scale`,
// in one v_cvt_scalef32_pk_f32_fp4.
#define RBT_FP4X2(w, scale, sel) __builtin_amdgcn_cvt_scalef32_pk_f32_fp4((w), (scale), (sel))

__device__ __forceinline__ float rbt_silu(float g) { return g / (1.0f + expf(-g)); }
__device__ __forceinline__ float rbt_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

// Butterfly sum over groups of `width` lanes (width a power of two <= 64).
template <int WIDTH>
__device__ __forceinline__ float rbt_group_sum(float v) {
#pragma unroll
  for (int m = WIDTH / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, RBT_WAVE);
  return v;
}

__device__ __forceinline__ double rbt_wave_sum_d(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, RBT_WAVE);
  return v;
}

// Device view of one expert: gate/up/down as separate (data, scale) pointers. A fused gate_up
// tensor is presented as two views into the same allocation.
struct RbtExpertDev {
  const uint8_t *gd;
  const void *gs;
  const uint8_t *ud;
  const void *us;
  const uint8_t *dd;
  const void *ds;
};
