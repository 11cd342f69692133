// rbt_xmfma.h -- MFMA helpers for the MXFP4 decode products (gfx950) and the balanced one-token
// gate/up body, shared by xgemm.hip and router.hip (the router launch also runs the shared
// expert's gate/up on the CUs its selection leaves idle).
//
// Lane layout (v_mfma_f32_16x16x32_bf16): lane l supplies A[l%16][8*(l/16) + 0..7] and
// B[8*(l/16) + 0..7][l%16] and receives D[4*(l/16) + i][l%16]. A rows are "virtual rows"
// v = 4*rho + kappa (weight row rho of a 4-row tile restricted to column quarter kappa of a
// 512-column step); B column 4*kappa' + p holds activation part p of quarter kappa'.
#pragma once

#include "rbt_device.h"
#include "rbt_internal.h"

namespace rbt {

typedef __bf16 xb8 __attribute__((ext_vector_type(8)));
typedef __bf16 xb2 __attribute__((ext_vector_type(2)));
typedef float xf4 __attribute__((ext_vector_type(4)));

constexpr int XG_PAD = 8;        // bf16 padding between the LDS part rows (bank spread)

// 8 E2M1 codes (one dword) -> 8 bf16, scaled by the block's E8M0 value.
__device__ __forceinline__ xb8 fp4x8_bf16(uint32_t w, float sc) {
  const xb2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0);
  const xb2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1);
  const xb2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2);
  const xb2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3);
  return xb8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// x = hi + mid + lo, each part the bf16 rounding of the remainder (the remainders are exact in
// fp32: x and hi agree to within one bf16 ulp).
__device__ __forceinline__ void split3(float x, __bf16 &h, __bf16 &m, __bf16 &l) {
  h = (__bf16)x;
  const float r1 = x - (float)h;
  m = (__bf16)r1;
  const float r2 = r1 - (float)m;
  l = (__bf16)r2;
}

// The four B operands of one step: lane l (column j = l%16: quarter j/4, part j%4) reads 8 values
// of its part per MFMA; lanes of part 3 read a 64-byte zero block (their pointer does not move).
struct XB {
  xb8 b[4];
};
__device__ __forceinline__ XB xb_read(const char *bp) {
  XB r;
#pragma unroll
  for (int m = 0; m < 4; m++) r.b[m] = *reinterpret_cast<const xb8 *>(bp + 16 * m);
  return r;
}

// acc += A(codes, scale) . B: the four MFMAs of one 16-byte chunk.
__device__ __forceinline__ void xmma_s(const rbt_u4 &w, float sc, const XB &B, xf4 &acc) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(w.x, sc), B.b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(w.y, sc), B.b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(w.z, sc), B.b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(w.w, sc), B.b[3], acc, 0, 0, 0);
}

// E8M0 byte -> f32 (e8m0_decode, quant.rs:391-396): 0 -> 2^-127, 255 -> the +inf bits.
__device__ __forceinline__ float xe8m0(uint32_t b) { return __uint_as_float(max(b << 23, 0x400000u)); }

// Dot product of weight row l/16 of the tile from the accumulator (see the tile-shape notes): the
// lane's useful entry is acc[(l%16)/4] unless its part is 3; the 16 lanes of the row group sum
// them (every lane of the group ends with the same value).
__device__ __forceinline__ float row_dot(const xf4 &acc, int col) {
  const int kq = col >> 2;
  float v = kq == 0 ? acc[0] : kq == 1 ? acc[1] : kq == 2 ? acc[2] : acc[3];
  v = (col & 3) == 3 ? 0.0f : v;
  return rbt_group_sum<16>(v);
}

// ------------------------------------------------------------------------------------------------
// gate/up for one token (every pair reads the same x): balanced over the whole chip. The work is
// U = npairs * I/4 units, unit u = (pair u / (I/4), 4-row tile u % (I/4)) of gate and of up; wave i
// of the grid takes units [i U / NW, (i+1) U / NW), so every CU streams the same number of bytes
// (a workgroup per CU; per-pair grids leave a third of the CUs with twice the work at small pair
// counts). A wave runs its units as one stream of (unit, step) iterations, XG1_D of them in flight
// (2 chunks of 16 bytes per lane each), and keeps each unit's scale bytes (4 rows x K/32 bytes of
// gate and of up) in a private LDS window loaded one unit ahead.
// ------------------------------------------------------------------------------------------------
// Workgroup wg of nwg (the caller's grid, or its part of one) runs the body; hp points at pair 0's
// output parts.
// LDS of the one-token gate/up (sized for K = 8192).
struct GuLds {
  __attribute__((aligned(16))) __bf16 xs[3 * (8192 + XG_PAD)];
  __attribute__((aligned(16))) __bf16 zb[32];
  __attribute__((aligned(16))) uint8_t sw[4][2][2][4][256];  // [wave][buffer][matrix][row][byte]
  float sp[4][4][2];  // [wave][row of the unit][gate, up]: a shared half unit's row sums
};

// The shared expert's half unit that a wave of the one-token gate/up takes before its routed units:
// rows 4 su .. 4 su + 3 of the shared gate and up, steps hf D .. hf D + D - 1 (D = NCH / 2, the
// ring's depth). The shared expert does not depend on the routing, so the caller issues these loads
// before the selection and they land while it runs. The two halves of a unit belong to waves 2j and
// 2j + 1 of one workgroup, which leave their row sums in GuLds::sp; the caller adds them after a
// barrier (xgateup1_sh_combine).
template <int NCH>
struct ShHalf {
  int su = -1, hf = 0;  // su < 0: no half for this wave
  rbt_u4 ring[NCH % 2 == 0 ? NCH / 2 : 1][2];
  rbt_u4 sv[2];  // the lane's scale pieces of the unit (as the body's window loads)
};

template <int NCH>
__device__ __forceinline__ void xgateup1_sh_issue(ShHalf<NCH> &s, const RbtExpertDev &J) {
  static_assert(NCH % 2 == 0, "half units need an even step count");
  constexpr int K = NCH * 512, SR = K >> 5, D = NCH / 2;
  const int lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15, rho = col >> 2, kap = col & 3;
  const int s_row = (lane >> 4) & 3, s_off = min(16 * (lane & 15), SR - 16);
  const long row0 = 4L * s.su;
  s.sv[0] = *(const rbt_gu4 *)((const uint8_t *)J.gs + (row0 + s_row) * SR + s_off);
  s.sv[1] = *(const rbt_gu4 *)((const uint8_t *)J.us + (row0 + s_row) * SR + s_off);
  const long off = (row0 + rho) * (K >> 1) + 64 * kap + 16 * g + 256L * D * s.hf;
#pragma unroll
  for (int d = 0; d < D; d++) {
    s.ring[d][0] = __builtin_nontemporal_load((const rbt_gu4 *)(J.gd + off + 256 * d));
    s.ring[d][1] = __builtin_nontemporal_load((const rbt_gu4 *)(J.ud + off + 256 * d));
  }
}

// h of the workgroup's shared units [s0, s0 + nsu) from the halves' row sums (after a barrier that
// follows every wave's half): gate and up are each the first half's sum plus the second's.
__device__ __forceinline__ void xgateup1_sh_combine(const GuLds &L, int s0, int nsu, int slot, int I,
                                                    __bf16 *__restrict__ hp) {
  const int t = threadIdx.x;
  if (t < 4 * nsu) {
    const int j = t >> 2, r = t & 3;
    const float gv = __fadd_rn(L.sp[2 * j][r][0], L.sp[2 * j + 1][r][0]);
    const float uv = __fadd_rn(L.sp[2 * j][r][1], L.sp[2 * j + 1][r][1]);
    const float hv = rbt_silu(gv) * uv;
    __bf16 hh, mm, ll;
    split3(hv, hh, mm, ll);
    const long rr = 4L * (s0 + j) + r;
    hp[((long)slot * 3 + 0) * I + rr] = hh;
    hp[((long)slot * 3 + 1) * I + rr] = mm;
    hp[((long)slot * 3 + 2) * I + rr] = ll;
  }
}

// The token's activation, thread t's float4 chunks t + 256 j (the first step of the body, issued
// early by callers that have other work before the body proper).
template <int NCH>
constexpr int xg_nv() { return (NCH * 128 + 255) / 256; }  // float4 chunks of K = 512 NCH values per thread

template <int NCH>
__device__ __forceinline__ void xgateup1_load_x(const float *__restrict__ x, float4 (&xv)[xg_nv<NCH>()]) {
  const rbt_gf4 *s4 = (const rbt_gf4 *)x;
#pragma unroll
  for (int j = 0; j < xg_nv<NCH>(); j++) xv[j] = s4[min((int)threadIdx.x + 256 * j, NCH * 128 - 1)];
}

// The activation's three bf16 parts (and the zero block) into the body's LDS; the body's first
// barrier publishes them.
template <int NCH>
__device__ __forceinline__ void xgateup1_stage_x(GuLds &L, const float4 (&xv)[xg_nv<NCH>()]) {
  constexpr int stride = NCH * 512 + XG_PAD;
  if (threadIdx.x < 32) L.zb[threadIdx.x] = (__bf16)0.0f;
#pragma unroll
  for (int j = 0; j < xg_nv<NCH>(); j++) {
    const int q = threadIdx.x + 256 * j;
    if (q >= NCH * 128) break;
    const float e4[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      __bf16 hh, mm, ll;
      split3(e4[e], hh, mm, ll);
      L.xs[4 * q + e] = hh;
      L.xs[stride + 4 * q + e] = mm;
      L.xs[2 * stride + 4 * q + e] = ll;
    }
  }
}

// The body with the activation already in registers (xgateup1_load_x), or, with STAGED, already in
// LDS (xgateup1_stage_x, xv unused); `jobs` may point at LDS.
// With SH, a wave whose sh.su >= 0 first multiplies its preloaded shared half unit (scales into
// window buffer 1, row sums into L.sp) while its first routed unit's loads go out. h = act(g, u)
// (rbt_act: SiLU by default); with HF32 it is stored as one fp32 value per row (pair p's rows at
// hp + 2 I p as floats) instead of three bf16 parts.
template <int NCH, bool STAGED = false, bool SH = false, bool HF32 = false>
__device__ __forceinline__ void xgateup1_run(GuLds &L, const RbtExpertDev *__restrict__ jobs, int npairs,
                                             const float4 (&xv)[xg_nv<NCH>()], const float *__restrict__ x, int I,
                                             __bf16 *__restrict__ hp, int wg, int nwg,
                                             const ShHalf<NCH> *sh = nullptr, const RbtAct &act = RbtAct{}) {
  // ring depth: half a unit, so step c < D prefetches step c + D of the same unit and step c >= D
  // the first half of the next unit (slots and the unit epilogue are compile-time positions)
  // (an odd step count keeps a whole unit in flight)
  constexpr int K = NCH * 512, stride = K + XG_PAD, SR = K >> 5, D = NCH % 2 == 0 ? NCH / 2 : NCH;
  static_assert(K <= 8192, "GuLds holds K <= 8192");
  __bf16 *xs = L.xs;
  __bf16 *zb = L.zb;
  uint8_t(&sw)[4][2][2][4][256] = L.sw;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int rho = col >> 2, kap = col & 3;
  const int tpp = I >> 2;  // 4-row tiles per pair
  const long U = (long)npairs * tpp, NW = 4L * nwg, wi = 4L * wg + w;
  const int u0 = (int)(wi * U / NW), u1 = (int)((wi + 1) * U / NW);
  // the wave's units span at most two pairs (U / NW < I / 4)
  const int pa = min(u0 / tpp, max(npairs - 1, 0)), pb = min(pa + 1, max(npairs - 1, 0));
  RbtExpertDev JA{}, JB{};
  if (u1 > u0) {
    JA = jobs[pa];
    JB = jobs[pb];
  }
  const bool live = u1 > u0 && JA.gd != nullptr && JA.ud != nullptr && JB.gd != nullptr && JB.ud != nullptr;
  const bool shw = SH && sh->su >= 0;  // this wave has a shared half
  // lane pointers of unit u (clamped to the wave's last unit): codes of gate / up at step 0, and the
  // lane's scale piece (16 bytes of row (lane >> 4) & 3, clamped at the row end)
  const int s_row = (lane >> 4) & 3, s_off = min(16 * (lane & 15), SR - 16);
  struct UPtr {
    const uint8_t *g, *u, *gs, *us;
  };
  auto uptr = [&](int u) {
    UPtr r;
    if (u >= u1) {
      // past the wave's units: reads of the activation vector (cached, a few KB), never used
      r.g = r.u = (const uint8_t *)x + 64 * kap + 16 * g;
      r.gs = r.us = (const uint8_t *)x + s_off;
      return r;
    }
    const int pp = u / tpp;
    const RbtExpertDev &J = pp == pa ? JA : JB;
    const long row0 = 4L * (u - pp * tpp);
    r.g = J.gd + (row0 + rho) * (K >> 1) + 64 * kap + 16 * g;
    r.u = J.ud + (row0 + rho) * (K >> 1) + 64 * kap + 16 * g;
    r.gs = (const uint8_t *)J.gs + (row0 + s_row) * SR + s_off;
    r.us = (const uint8_t *)J.us + (row0 + s_row) * SR + s_off;
    return r;
  };
  rbt_u4 ring[D][2], sv[2];
  UPtr cur{}, nxt{};
  if (live) {
    cur = uptr(u0);
    nxt = uptr(u0 + 1);
    sv[0] = *(const rbt_gu4 *)cur.gs;
    sv[1] = *(const rbt_gu4 *)cur.us;
    if (!shw) {
#pragma unroll
      for (int d = 0; d < D; d++) {
        ring[d][0] = __builtin_nontemporal_load((const rbt_gu4 *)(cur.g + 256 * d));
        ring[d][1] = __builtin_nontemporal_load((const rbt_gu4 *)(cur.u + 256 * d));
      }
    }
  }
  if (!STAGED) xgateup1_stage_x<NCH>(L, xv);
  auto sstore = [&](int buf) {
    *reinterpret_cast<rbt_u4 *>(&sw[w][buf][0][s_row][16 * (lane & 15)]) = sv[0];
    *reinterpret_cast<rbt_u4 *>(&sw[w][buf][1][s_row][16 * (lane & 15)]) = sv[1];
  };
  const int bq = col >> 2, bpart = col & 3;
  const char *bp = bpart < 3 ? reinterpret_cast<const char *>(xs + bpart * stride + 128 * bq + 32 * g)
                             : reinterpret_cast<const char *>(zb);
  const int binc = bpart < 3 ? 1024 : 0;  // bytes per step (512 bf16)
  if constexpr (SH && NCH % 2 == 0) if (shw) {
    // the shared half: its scales into window buffer 1 (its loads landed during the selection),
    // then its steps, each refilled with the same step of the first routed unit
    *reinterpret_cast<rbt_u4 *>(&sw[w][1][0][s_row][16 * (lane & 15)]) = sh->sv[0];
    *reinterpret_cast<rbt_u4 *>(&sw[w][1][1][s_row][16 * (lane & 15)]) = sh->sv[1];
    const uint8_t(*win)[4][256] = sw[w][1];
    xf4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < D; c++) {
      const int cs = sh->hf * D + c;
      const XB B = xb_read(bp + binc * cs);
      const int sb = 16 * cs + 4 * kap + g;
      const rbt_u4 cg = sh->ring[c][0], cu = sh->ring[c][1];
      if (live) {
        ring[c][0] = __builtin_nontemporal_load((const rbt_gu4 *)(cur.g + 256 * c));
        ring[c][1] = __builtin_nontemporal_load((const rbt_gu4 *)(cur.u + 256 * c));
      }
      xmma_s(cg, xe8m0(win[0][rho][sb]), B, ag);
      xmma_s(cu, xe8m0(win[1][rho][sb]), B, au);
      __builtin_amdgcn_sched_barrier(0);
    }
    const float gv = row_dot(ag, col), uv = row_dot(au, col);
    if (col == 0) {  // lane 16 g: row g of the unit
      L.sp[w][g][0] = gv;
      L.sp[w][g][1] = uv;
    }
  }
  if (live) {
    sstore(0);
    sv[0] = *(const rbt_gu4 *)nxt.gs;  // scales of the next unit (the last unit's own, if none)
    sv[1] = *(const rbt_gu4 *)nxt.us;
  }
  __syncthreads();
  if (!live) {
    // a missing expert is reported by the grouping (error flag); zero this wave's rows of h
    for (int u = u0; u < u1; u++) {
      const int pp = u / tpp;
      if (HF32) {
        if (lane < 4) reinterpret_cast<float *>(hp)[(long)pp * I + 4L * (u - pp * tpp) + lane] = 0.0f;
      } else if (lane < 12) {
        hp[((long)pp * 3 + lane / 4) * I + 4L * (u - pp * tpp) + (lane & 3)] = (__bf16)0.0f;
      }
    }
    return;
  }
  for (int u = u0; u < u1; u++) {
    const uint8_t(*win)[4][256] = sw[w][(u - u0) & 1];
    xf4 ag = {0.f, 0.f, 0.f, 0.f}, au = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < NCH; c++) {
      const int d = c % D;
      const XB B = xb_read(bp + binc * c);
      const int sb = 16 * c + 4 * kap + g;
      const rbt_u4 cg = ring[d][0], cu = ring[d][1];
      // refill: step c + D of this unit, or of the next one past the unit's end
      const uint8_t *rg = c + D < NCH ? cur.g + 256 * (c + D) : nxt.g + 256 * (c + D - NCH);
      const uint8_t *ru = c + D < NCH ? cur.u + 256 * (c + D) : nxt.u + 256 * (c + D - NCH);
      ring[d][0] = __builtin_nontemporal_load((const rbt_gu4 *)rg);
      ring[d][1] = __builtin_nontemporal_load((const rbt_gu4 *)ru);
      xmma_s(cg, xe8m0(win[0][rho][sb]), B, ag);
      xmma_s(cu, xe8m0(win[1][rho][sb]), B, au);
      __builtin_amdgcn_sched_barrier(0);
    }
    // unit done: h for its 4 rows
    const float gv = row_dot(ag, col), uv = row_dot(au, col);
    const int pp = u / tpp;
    if (col == 0) {  // lane 16*g: row 4 t + g of the unit's pair
      const float hv = rbt_act(act, gv, uv);
      const long rr = 4L * (u - pp * tpp) + g;
      if (HF32) {
        reinterpret_cast<float *>(hp)[(long)pp * I + rr] = hv;
      } else {
        __bf16 hh, mm, ll;
        split3(hv, hh, mm, ll);
        hp[((long)pp * 3 + 0) * I + rr] = hh;
        hp[((long)pp * 3 + 1) * I + rr] = mm;
        hp[((long)pp * 3 + 2) * I + rr] = ll;
      }
    }
    // next unit's scales into the other window, then look one unit further ahead
    sstore((u + 1 - u0) & 1);
    cur = nxt;
    nxt = uptr(u + 2);
    sv[0] = *(const rbt_gu4 *)nxt.gs;
    sv[1] = *(const rbt_gu4 *)nxt.us;
  }
}



template <int NCH>
__device__ __forceinline__ void xgateup1_body(GuLds &L, const RbtExpertDev *__restrict__ jobs, int npairs,
                                              const float *__restrict__ x, int I, __bf16 *__restrict__ hp, int wg,
                                              int nwg) {
  float4 xv[xg_nv<NCH>()];
  xgateup1_load_x<NCH>(x, xv);
  xgateup1_run<NCH>(L, jobs, npairs, xv, x, I, hp, wg, nwg);
}

}  // namespace rbt
