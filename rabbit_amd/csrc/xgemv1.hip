// xgemv1.hip -- one token through one MXFP4 matrix (matmul_mxfp4, kernels.rs:233-267) or through one
// expert (apply_single_expert, glm52/moe.rs:463-513) on the matrix cores, balanced over the chip.
//
// A single token's product is too small to stream in steady state (5.9-17.8 MB: one to three
// microseconds of HBM time), so the work is cut into as many items as the chip has wave slots and
// every wave issues all of its loads at entry. Item = (4-row tile, K part): the K range (NCH steps
// of 512 columns) is split in KS parts, so a matrix of O rows gives O/4 * KS items; a workgroup of
// eight waves holds 8 / KS consecutive tiles with all of their parts, and the parts' row sums meet in
// LDS, summed in part order (fixed: the result does not depend on timing). Lane layout, the exact
// three-part bf16 split of the activation and the MFMA tile are those of the one-token gate/up
// (rbt_xmfma.h); each lane reads its block's E8M0 byte from one dword per step.
//
// Modes:
//   GU   gate and up of one expert (two matrices, the same items), h = act(g, u) written as three
//        bf16 parts hp[part * I + r] for a following PIN launch;
//   PIN  the activation is such a three-part h (the down product), staged as is;
//   else the activation is fp32 x, split into parts while staged.
// Output (not GU): y[r] = row sum, or with an accumulate weight (apply_single_expert)
// out[r] = out[r] + w * row sum, with separate roundings (glm52/moe.rs:508-512).
#include "rbt_device.h"
#include "rbt_internal.h"
#include "rbt_xmfma.h"

namespace rbt {

constexpr int XV_W = 8;  // waves per workgroup (one item each)

template <int NCH, int KS, bool GU, bool PIN>
__global__ __launch_bounds__(64 * XV_W) void k_xgemv1(const uint8_t *__restrict__ d0, const uint8_t *__restrict__ s0,
                                                      const uint8_t *__restrict__ d1, const uint8_t *__restrict__ s1,
                                                      const void *__restrict__ xin, int O, __bf16 *__restrict__ hp,
                                                      float *__restrict__ y, const int32_t *__restrict__ ids,
                                                      const float *__restrict__ wts, int k, int eid, RbtAct act) {
  constexpr int K = NCH * 512, stride = K + XG_PAD, SR = K >> 5;
  constexpr int NM = GU ? 2 : 1;                       // matrices per item
  constexpr int SPI = (NCH + KS - 1) / KS;             // most steps of one part
  constexpr int TPW = XV_W / KS;                       // tiles per workgroup
  static_assert(XV_W % KS == 0, "a workgroup holds whole tiles");
  __shared__ __attribute__((aligned(16))) __bf16 xs[3 * stride];
  __shared__ __attribute__((aligned(16))) __bf16 zb[32];
  __shared__ float part[TPW][KS][4][NM];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6, g = lane >> 4, col = lane & 15;
  const int rho = col >> 2, kap = col & 3;
  // apply_single_expert: lane j's routing slot (k <= 64) is requested first, with everything else,
  // and looked at only after the products, before anything is stored (a token that did not pick the
  // expert returns there): the check costs no trip to memory of its own. Without ids the loads read
  // a valid address and go unused.
  const int jl = min(lane, max(k, 1) - 1);
  const int32_t idl = *(ids != nullptr ? ids + jl : reinterpret_cast<const int32_t *>(xin));
  const float wtl = *(ids != nullptr ? wts + jl : reinterpret_cast<const float *>(xin));
  const int tile = blockIdx.x * TPW + w / KS, kp = w % KS;
  const int c0 = kp * NCH / KS, c1 = (kp + 1) * NCH / KS;  // this item's steps
  const long row0 = 4L * min(tile, O / 4 - 1);
  // the activation first (the memory counter retires loads in issue order: waiting for it then does
  // not mean waiting for the weights issued behind it)
  constexpr int NT = 64 * XV_W;
  constexpr int XQ = PIN ? (3 * K / 8 + NT - 1) / NT : (K / 4 + NT - 1) / NT;  // 16-byte pieces per thread
  rbt_u4 xr[XQ];
#pragma unroll
  for (int i = 0; i < XQ; i++) {
    const int e = t + NT * i;
    if (PIN)
      xr[i] = *(const rbt_gu4 *)((const uint8_t *)xin + 16L * min(e, 3 * K / 8 - 1));
    else
      xr[i] = *(const rbt_gu4 *)((const uint8_t *)xin + 16L * min(e, K / 4 - 1));
  }
  // every load of the item at once: codes (16 bytes of the lane's row per step) and the dword of
  // E8M0 bytes that holds the lane's block
  rbt_u4 wd[NM][SPI];
  uint32_t sd[NM][SPI];
  const uint8_t *dm[2] = {d0, d1};
  const uint8_t *sm[2] = {s0, s1};
#pragma unroll
  for (int m = 0; m < NM; m++) {
    const uint8_t *rowp = dm[m] + (row0 + rho) * (K >> 1) + 64 * kap + 16 * g;
    const uint8_t *srow = sm[m] + (row0 + rho) * SR + 4 * kap;
#pragma unroll
    for (int c = 0; c < SPI; c++) {
      const int cc = min(c0 + c, c1 - 1);  // past the part's end: its last step again (never used)
      wd[m][c] = __builtin_nontemporal_load((const rbt_gu4 *)(rowp + 256 * cc));
      sd[m][c] = *(const rbt_gu32 *)(srow + 16 * cc);
    }
  }
  // stage the activation's three bf16 parts
  if (t < 32) zb[t] = (__bf16)0.0f;
#pragma unroll
  for (int i = 0; i < XQ; i++) {
    const int e = t + NT * i;
    if (PIN) {
      if (e < 3 * K / 8) {
        const int p = e / (K / 8), q = e - p * (K / 8);
        *reinterpret_cast<rbt_u4 *>(&xs[p * stride + 8 * q]) = xr[i];
      }
    } else if (e < K / 4) {
      const float f[4] = {__uint_as_float(xr[i].x), __uint_as_float(xr[i].y), __uint_as_float(xr[i].z),
                          __uint_as_float(xr[i].w)};
#pragma unroll
      for (int j = 0; j < 4; j++) {
        __bf16 hh, mm, ll;
        split3(f[j], hh, mm, ll);
        xs[4 * e + j] = hh;
        xs[stride + 4 * e + j] = mm;
        xs[2 * stride + 4 * e + j] = ll;
      }
    }
  }
  lds_barrier();  // the staged parts (the weight loads stay in flight)
  const int bq = col >> 2, bpart = col & 3;
  const char *bp = bpart < 3 ? reinterpret_cast<const char *>(xs + bpart * stride + 128 * bq + 32 * g)
                             : reinterpret_cast<const char *>(zb);
  const int binc = bpart < 3 ? 1024 : 0;
  const uint32_t sh = 8u * (uint32_t)g;
  xf4 acc[NM];
#pragma unroll
  for (int m = 0; m < NM; m++) acc[m] = xf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < SPI; c++) {
    if (c0 + c < c1) {
      const XB B = xb_read(bp + binc * (c0 + c));
#pragma unroll
      for (int m = 0; m < NM; m++) xmma_s(wd[m][c], xe8m0((sd[m][c] >> sh) & 0xFFu), B, acc[m]);
    }
  }
  // the token's weight for this expert: its first slot that holds eid (glm52/moe.rs:465-470), the same
  // in every wave
  const unsigned long long hit = __ballot(lane < k && idl == eid);
  if (ids != nullptr && hit == 0) return;  // not picked: nothing to do
  const float wv = ids != nullptr ? __shfl(wtl, (int)__ffsll(hit) - 1, 64) : 1.0f;
#pragma unroll
  for (int m = 0; m < NM; m++) {
    const float v = row_dot(acc[m], col);
    if (col == 0) part[w / KS][kp][g][m] = v;  // lane 16 g: row row0 + g
  }
  __syncthreads();
  if (t < 4 * TPW) {
    const int tl = t >> 2, r = t & 3, tt = blockIdx.x * TPW + tl;
    if (4 * tt < O) {
      float sv[NM];
#pragma unroll
      for (int m = 0; m < NM; m++) {
        float s = part[tl][0][r][m];
#pragma unroll
        for (int p = 1; p < KS; p++) s += part[tl][p][r][m];
        sv[m] = s;
      }
      const long rr = 4L * tt + r;
      if constexpr (GU) {
        const float hv = rbt_act(act, sv[0], sv[1]);
        __bf16 hh, mm, ll;
        split3(hv, hh, mm, ll);
        hp[rr] = hh;
        hp[(long)O + rr] = mm;
        hp[2L * O + rr] = ll;
      } else if (ids != nullptr) {
        y[rr] = __fadd_rn(y[rr], __fmul_rn(wv, sv[0]));
      } else {
        y[rr] = sv[0];
      }
    }
  }
}

// ---- launchers --------------------------------------------------------------------------------
// K parts per tile for O rows: enough items (O/4 * KS) to give every wave slot of the chip one.
static int xgemv1_ks(int O, int num_cu) {
  const long tiles = O / 4, want = (long)XV_W * num_cu;
  return tiles >= want ? 1 : (2 * tiles >= want ? 2 : 4);
}

template <int NCH, bool GU, bool PIN>
static hipError_t xgemv1_go(const Ctx &c, int ks, const uint8_t *d0, const uint8_t *s0, const uint8_t *d1,
                            const uint8_t *s1, const void *xin, int O, __bf16 *hp, float *y, const int32_t *ids,
                            const float *wts, int k, int eid, const RbtAct &act) {
  const int tiles = O / 4;
  if (ks == 1)
    launch_k(c, k_xgemv1<NCH, 1, GU, PIN>, dim3((tiles + XV_W - 1) / XV_W), dim3(64 * XV_W), d0, s0, d1, s1, xin, O,
             hp, y, ids, wts, k, eid, act);
  else if (ks == 2)
    launch_k(c, k_xgemv1<NCH, 2, GU, PIN>, dim3((tiles + XV_W / 2 - 1) / (XV_W / 2)), dim3(64 * XV_W), d0, s0, d1,
             s1, xin, O, hp, y, ids, wts, k, eid, act);
  else
    launch_k(c, k_xgemv1<NCH, 4, GU, PIN>, dim3((tiles + XV_W / 4 - 1) / (XV_W / 4)), dim3(64 * XV_W), d0, s0, d1,
             s1, xin, O, hp, y, ids, wts, k, eid, act);
  return hipGetLastError();
}

bool xgemv1_ok(size_t cols, size_t rows, int num_cu) {
  const int nch = (int)(cols / 512);
  if (cols % 512 != 0 || rows % 4 != 0 || rows == 0 || num_cu <= 0) return false;
  if (nch != 4 && nch != 7 && nch != 8 && nch != 14 && nch != 16) return false;
  // at most two workgroups of eight waves per CU in flight over the launch's items (one per wave);
  // larger products stream better through the decode GEMV
  const int ks = xgemv1_ks((int)rows, num_cu);
  return (long)(rows / 4) * ks <= 2L * XV_W * num_cu && ks <= nch;
}

hipError_t launch_xgemv1(const Ctx &c, const uint8_t *data, const uint8_t *scale, const float *x, int I, int O,
                         float *y) {
  if (!xgemv1_ok((size_t)I, (size_t)O, c.num_cu) || ((uintptr_t)x | (uintptr_t)data) % 16 != 0 ||
      (uintptr_t)scale % 4 != 0)
    return hipErrorInvalidValue;
  const int ks = xgemv1_ks(O, c.num_cu);
  const RbtAct none{};
  switch (I / 512) {
    case 4: return xgemv1_go<4, false, false>(c, ks, data, scale, nullptr, nullptr, x, O, nullptr, y, nullptr, nullptr, 0, 0, none);
    case 7: return xgemv1_go<7, false, false>(c, ks, data, scale, nullptr, nullptr, x, O, nullptr, y, nullptr, nullptr, 0, 0, none);
    case 8: return xgemv1_go<8, false, false>(c, ks, data, scale, nullptr, nullptr, x, O, nullptr, y, nullptr, nullptr, 0, 0, none);
    case 14: return xgemv1_go<14, false, false>(c, ks, data, scale, nullptr, nullptr, x, O, nullptr, y, nullptr, nullptr, 0, 0, none);
    case 16: return xgemv1_go<16, false, false>(c, ks, data, scale, nullptr, nullptr, x, O, nullptr, y, nullptr, nullptr, 0, 0, none);
  }
  return hipErrorInvalidValue;
}

bool xexpert1_ok(size_t d, size_t i, int num_cu) {
  return (d == 8192 || d == 7168) && i == 2048 && xgemv1_ok(d, i, num_cu) && xgemv1_ok(i, d, num_cu);
}

hipError_t launch_xexpert1(const Ctx &c, const RbtExpertDev &J, const float *x, int d, int i, const int32_t *ids,
                           const float *wts, int k, int eid, __bf16 *hp, float *out, const RbtAct &act) {
  if (!xexpert1_ok((size_t)d, (size_t)i, c.num_cu) || !J.gd || !J.ud || !J.dd || !J.gs || !J.us || !J.ds ||
      ((uintptr_t)x | (uintptr_t)J.gd | (uintptr_t)J.ud | (uintptr_t)J.dd) % 16 != 0 ||
      ((uintptr_t)J.gs | (uintptr_t)J.us | (uintptr_t)J.ds) % 4 != 0 || k < 1 || k > 64)
    return hipErrorInvalidValue;
  const uint8_t *gs = (const uint8_t *)J.gs, *us = (const uint8_t *)J.us, *ds = (const uint8_t *)J.ds;
  const int ksg = xgemv1_ks(i, c.num_cu), ksd = xgemv1_ks(d, c.num_cu);
  hipError_t e = d == 8192 ? xgemv1_go<16, true, false>(c, ksg, J.gd, gs, J.ud, us, x, i, hp, nullptr, ids, wts, k, eid, act)
                           : xgemv1_go<14, true, false>(c, ksg, J.gd, gs, J.ud, us, x, i, hp, nullptr, ids, wts, k, eid, act);
  if (e != hipSuccess) return e;
  return xgemv1_go<4, false, true>(c, ksd, J.dd, ds, nullptr, nullptr, hp, d, nullptr, out, ids, wts, k, eid, act);
}

}  // namespace rbt
