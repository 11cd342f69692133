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
// Global-address-space views (addrspace 1): loads through them are global_load_* rather than
// flat_load_*, which count only in vmcnt and let the compiler keep several loads in flight.
// The host compilation pass only parses device functions, and HIP's float4 class has no
// address-space-qualified constructors there, so it sees plain types.
#if defined(__HIP_DEVICE_COMPILE__)
#define RBT_GLOBAL __attribute__((address_space(1)))
#else
#define RBT_GLOBAL
#endif
typedef RBT_GLOBAL const rbt_u4 rbt_gu4;
typedef RBT_GLOBAL const float4 rbt_gf4;
typedef RBT_GLOBAL const uint32_t rbt_gu32;
typedef RBT_GLOBAL const uint8_t rbt_gu8;

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

// Activation::combine (glm52/moe.rs:58-70): silu(g) * u, or Situ
// (beta * tanh(g / beta)) * (1 / (1 + exp(-g))) * u' with u' = lbeta * tanh(u / lbeta) when has_lb.
// Each fp32 operation rounded on its own, in the reference's order (tanh and exp are the device's).
struct RbtAct {
  int kind = 0;  // 0: Silu, 1: Situ (RBT_ACT_*)
  float beta = 0.0f, lbeta = 0.0f;
  int has_lb = 0;
};
__device__ __forceinline__ float rbt_act(const RbtAct &a, float g, float u) {
  if (a.kind != 1) return rbt_silu(g) * u;
  if (a.has_lb) u = __fmul_rn(a.lbeta, tanhf(__fdiv_rn(u, a.lbeta)));
  const float situ = __fmul_rn(__fmul_rn(a.beta, tanhf(__fdiv_rn(g, a.beta))), __fdiv_rn(1.0f, __fadd_rn(1.0f, expf(-g))));
  return __fmul_rn(situ, u);
}

// Correctly rounded fp32 square root for positive normal x. v_sqrt_f32 is only faithful (within
// one ulp), so the neighbours of its result are tested with one fma residual each and the rounded
// value picked: the lowering LLVM uses for a correctly rounded llvm.sqrt.f32.
__device__ __forceinline__ float rbt_sqrt_rn(float x) {
  const float s = __builtin_amdgcn_sqrtf(x);
  const float sd = __int_as_float(__float_as_int(s) - 1), su = __int_as_float(__float_as_int(s) + 1);
  const float rd = __builtin_fmaf(-sd, s, x), ru = __builtin_fmaf(-su, s, x);
  const float r = rd <= 0.0f ? sd : s;
  return ru > 0.0f ? su : r;
}
__device__ __forceinline__ float rbt_sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

// v + (v from another lane of the same 16-lane DPP row), one v_add_f32_dpp.
template <int CTRL>
__device__ __forceinline__ float rbt_dpp_add(float v) {
  return v + __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}

// Barrier for LDS hand-offs only: global loads in flight stay in flight (__syncthreads' release
// fence waits for every outstanding load of the wave first).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Sum over aligned groups of WIDTH lanes (WIDTH a power of two <= 64). Within a 16-lane row the
// butterfly runs on DPP (quad_perm xor 1, xor 2, row_half_mirror, row_mirror); every lane of the
// group ends with the sum for WIDTH <= 32. For WIDTH = 64 the total is valid in lanes 0..31.
template <int WIDTH>
__device__ __forceinline__ float rbt_group_sum(float v) {
  if (WIDTH >= 2) v = rbt_dpp_add<0xB1>(v);   // quad_perm [1,0,3,2]
  if (WIDTH >= 4) v = rbt_dpp_add<0x4E>(v);   // quad_perm [2,3,0,1]
  if (WIDTH >= 8) v = rbt_dpp_add<0x141>(v);  // row_half_mirror
  if (WIDTH >= 16) v = rbt_dpp_add<0x140>(v); // row_mirror
  if (WIDTH >= 32) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // xor 16
  if (WIDTH >= 64) v += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  return v;
}

__device__ __forceinline__ double rbt_wave_sum_d(double v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, RBT_WAVE);
  return v;
}

// fp64 DPP move (both halves) with 0.0 in lanes whose source is outside the row or masked.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ double rbt_dpp0_d(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(v);
  const int lo = __builtin_amdgcn_update_dpp(0, (int)(unsigned)b, CTRL, ROW_MASK, BANK_MASK, false);
  const int hi = __builtin_amdgcn_update_dpp(0, (int)(unsigned)(b >> 32), CTRL, ROW_MASK, BANK_MASK, false);
  return __longlong_as_double((long long)(((unsigned long long)(unsigned)hi << 32) | (unsigned)lo));
}

// Inclusive wave scan (sum) with DPP: row_shr 1, 2, 4, 8 scan each row of 16 lanes, then
// row_bcast:15 adds row 0's total into row 1 (and row 2's into row 3) and row_bcast:31 adds
// rows 0-1 into rows 2-3. No LDS traffic (cross-lane shuffles go through it).
__device__ __forceinline__ double rbt_wave_scan_d(double v) {
  v += rbt_dpp0_d<0x111, 0xf, 0xf>(v);
  v += rbt_dpp0_d<0x112, 0xf, 0xf>(v);
  v += rbt_dpp0_d<0x114, 0xf, 0xf>(v);
  v += rbt_dpp0_d<0x118, 0xf, 0xf>(v);
  v += rbt_dpp0_d<0x142, 0xa, 0xf>(v);
  v += rbt_dpp0_d<0x143, 0xc, 0xf>(v);
  return v;
}

// 32-bit DPP moves with a given fill for lanes whose source is outside the row or masked.
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ uint32_t rbt_dpp_u(uint32_t fill, uint32_t v) {
  return (uint32_t)__builtin_amdgcn_update_dpp((int)fill, (int)v, CTRL, ROW_MASK, BANK_MASK, false);
}
template <int CTRL, int ROW_MASK, int BANK_MASK>
__device__ __forceinline__ float rbt_dpp_f(float fill, float v) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(fill), __float_as_int(v), CTRL, ROW_MASK, BANK_MASK, false));
}

// Wave maximum / minimum over the DPP scan pattern (as rbt_wave_scan_d); every lane gets the result.
__device__ __forceinline__ uint32_t rbt_wave_max_u(uint32_t v) {
  v = max(v, rbt_dpp_u<0x111, 0xf, 0xf>(0u, v));
  v = max(v, rbt_dpp_u<0x112, 0xf, 0xf>(0u, v));
  v = max(v, rbt_dpp_u<0x114, 0xf, 0xf>(0u, v));
  v = max(v, rbt_dpp_u<0x118, 0xf, 0xf>(0u, v));
  v = max(v, rbt_dpp_u<0x142, 0xa, 0xf>(0u, v));
  v = max(v, rbt_dpp_u<0x143, 0xc, 0xf>(0u, v));
  return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ float rbt_wave_min_f(float v) {
  v = fminf(v, rbt_dpp_f<0x111, 0xf, 0xf>(INFINITY, v));
  v = fminf(v, rbt_dpp_f<0x112, 0xf, 0xf>(INFINITY, v));
  v = fminf(v, rbt_dpp_f<0x114, 0xf, 0xf>(INFINITY, v));
  v = fminf(v, rbt_dpp_f<0x118, 0xf, 0xf>(INFINITY, v));
  v = fminf(v, rbt_dpp_f<0x142, 0xa, 0xf>(INFINITY, v));
  v = fminf(v, rbt_dpp_f<0x143, 0xc, 0xf>(INFINITY, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
__device__ __forceinline__ float rbt_wave_max_f(float v) {
  v = fmaxf(v, rbt_dpp_f<0x111, 0xf, 0xf>(-INFINITY, v));
  v = fmaxf(v, rbt_dpp_f<0x112, 0xf, 0xf>(-INFINITY, v));
  v = fmaxf(v, rbt_dpp_f<0x114, 0xf, 0xf>(-INFINITY, v));
  v = fmaxf(v, rbt_dpp_f<0x118, 0xf, 0xf>(-INFINITY, v));
  v = fmaxf(v, rbt_dpp_f<0x142, 0xa, 0xf>(-INFINITY, v));
  v = fmaxf(v, rbt_dpp_f<0x143, 0xc, 0xf>(-INFINITY, v));
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

// Wave total through the DPP scan (the value of lane 63, in every lane).
__device__ __forceinline__ double rbt_wave_total_d(double v) {
  const unsigned long long b = (unsigned long long)__double_as_longlong(rbt_wave_scan_d(v));
  const unsigned lo = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)b, 63);
  const unsigned hi = (unsigned)__builtin_amdgcn_readlane((int)(unsigned)(b >> 32), 63);
  return __longlong_as_double((long long)(((unsigned long long)hi << 32) | lo));
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
