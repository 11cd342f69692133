// xgemm.hip -- MXFP4 expert products on the matrix cores (gfx950 MFMA), decode shapes.
//
// Weights: each lane loads 16 bytes (32 E2M1 codes, one 32-element block) of one weight row and
// turns them into bf16 with v_cvt_scalef32_pk_bf16_fp4, which applies the block's E8M0 scale in the
// same instruction. e2m1 * 2^(s-127) has at most two significant bits, so the bf16 weight equals
// the reference's dequantized weight (quant.rs:325-339) for every scale the weights use in
// practice: normal values are exact, only blocks whose scaled codes fall below 2^-126 (scale bytes
// 0..2) reach the matrix core as bf16 subnormals.
//
// Activations: x (fp32) is split exactly into three bf16 parts hi + mid + lo (each the bf16
// rounding of what the previous parts leave), and the parts are three columns of the MFMA's B
// operand. Products of bf16 values are exact in fp32 and the matrix core accumulates in fp32, so the
// result has fp32-accumulation accuracy (the 1e-5 relative-L2 contract), like an FMA chain with a
// different association.
//
// Tile shape: v_mfma_f32_16x16x32_bf16 multiplies a 16x32 A tile by a 32x16 B tile. Lane l
// supplies A[l%16][8*(l/16) + 0..7] and B[8*(l/16) + 0..7][l%16] and receives D[4*(l/16) + i][l%16],
// i = 0..3. The 16 A rows here are "virtual rows" v = 4*rho + kappa: weight row rho (0..3) of a
// 4-row tile, restricted to column quarter kappa, where a 512-column step is cut into four
// 128-column quarters. Lane l (rho = (l%16)/4, kappa = l%4, g = l/16) loads 16 bytes = 32 codes of
// its row at columns 512*c + 128*kappa + 32*g, so one load instruction reads 4 rows x 256
// contiguous bytes (streams of 16 rows x 64 bytes run at two thirds of the bandwidth on this part).
// B column j = 4*kappa' + p holds activation part p (< 3; p = 3 is zero) at quarter kappa'. Only
// the D entries with kappa' == kappa are used: lane l's useful value is acc[(l%16)/4] for weight
// row l/16, and the 12 useful lanes of a 16-lane row group sum to that row's dot product.
//
// Work split:
//   k_xgateup : a wave owns 16 gate and 16 up rows (four 4-row tiles each) of one (expert, token)
//               pair over all columns; the four waves of a workgroup share the pair's activation
//               parts in LDS. Output h = silu(g) * u (glm52/moe.rs:33-80) as three bf16 parts.
//   k_xdown   : a wave owns one 4-row tile of the output for every pair of the call, one pair after
//               the other (the pair's h parts in LDS), and accumulates the ordered combine of
//               qwen38/generate.rs:303-349 / glm52/moe.rs:508-512 in place -> out.
#include "rbt_device.h"
#include "rbt_internal.h"
#include "rbt_xmfma.h"

namespace rbt {

constexpr int XD_MAXP = 80;  // pairs per down launch (partial tiles kept in LDS)

struct XChunk {
  rbt_u4 w;    // 32 E2M1 codes of this lane's row at its 32 columns of the step
  uint32_t s;  // the row's four E8M0 bytes of this lane's quarter (blocks 16*step + 4*kappa .. +3)
};

// One 512-column step of a lane's row: `row` points at the lane's 16 bytes of step 0 (row start +
// 64*kappa + 16*g), `srow` at its quarter's scale dword of step 0 (scale row + 4*kappa, 4-byte
// aligned). A step is 256 bytes of codes and 16 scale bytes.
__device__ __forceinline__ void xload(XChunk &c, const uint8_t *row, const uint8_t *srow, int step) {
  c.w = __builtin_nontemporal_load((const rbt_gu4 *)(row + 256 * step));
  c.s = *(const rbt_gu32 *)(srow + 16 * step);
}

// acc0/acc1 += A(chunk) . B: even and odd MFMAs go to separate accumulators (two independent
// dependency chains); the caller adds them in a fixed order.
// E8M0 byte -> f32 scale, max(b << 23, 2^-127 bits): byte 0 is 2^-127, 255 the +inf bits
// (e8m0_decode, quant.rs:391-396). Written as volatile asm so it stays in the step that multiplies
// the chunk: as plain code, instruction selection places the byte test right after the byte's
// load, four steps early, and the compiler then waits for that load there.
// `sh` = 8 * (lane's block within the dword).
__device__ __forceinline__ float e8m0_inplace(uint32_t sw, uint32_t sh) {
  uint32_t r;
  asm volatile("v_bfe_u32 %0, %1, %2, 8\n\tv_lshlrev_b32 %0, 23, %0\n\tv_max_u32 %0, 0x400000, %0"
               : "=&v"(r)
               : "v"(sw), "v"(sh));
  return __uint_as_float(r);
}

// acc += A(step) . B: the four MFMAs of the lane's 32 codes (8 per MFMA).
__device__ __forceinline__ void xmma1(const XChunk &c, uint32_t sh, const XB &B, xf4 &acc) {
  const float sc = e8m0_inplace(c.s, sh);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(c.w.x, sc), B.b[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(c.w.y, sc), B.b[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(c.w.z, sc), B.b[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(fp4x8_bf16(c.w.w, sc), B.b[3], acc, 0, 0, 0);
}

// ------------------------------------------------------------------------------------------------
// gate/up: grid (I/64, npairs), 256 threads. Wave w owns rows 16*(4*blockIdx.x + w) .. +15 of gate
// and of up for pair p = blockIdx.y, as four 4-row tiles, over all K = 512*NCH columns. The step
// loop is fully unrolled: the loads of step c + XG_DEPTH are issued while step c multiplies.
// h = silu(gate . x) * (up . x) goes out as three bf16 parts hp[(p*3 + part)*I + r].
// ------------------------------------------------------------------------------------------------
constexpr int XG_DEPTH = 2;  // steps in flight per wave (8 KB of codes each)

// Block scales of a wave's rows go through a wave-private LDS window. A group of 4 steps needs
// 64 scale bytes per row (blocks 64 G .. 64 G + 63); the wave's 32 rows (16 gate, 16 up) are
// 128 pieces of 16 bytes, two per lane, loaded one group ahead and stored after the current group
// has read its window. A lane then reads the one byte of each chunk from LDS instead of issuing a
// 4-byte global load per chunk and step (16x fewer scale requests to the memory pipeline).
struct XScale {
  const uint8_t *p[2];  // piece i: matrix i (gate, up), row lane/4 of the wave, bytes 16 (lane % 4)
  int last;             // last valid 16-byte offset of a row's scale bytes
  rbt_u4 v[2];
  __device__ __forceinline__ void load(int G) {
    const int off = min(64 * G, last);  // past the row end: a valid address, never read back
#pragma unroll
    for (int i = 0; i < 2; i++) v[i] = *(const rbt_gu4 *)(p[i] + off);
  }
};

template <int NCH>
__global__ __launch_bounds__(256) void k_xgateup(const RbtExpertDev *__restrict__ jobs, const int *__restrict__ tok,
                                                 const float *__restrict__ x, long x_stride, int I,
                                                 __bf16 *__restrict__ hp) {
  constexpr int K = NCH * 512, stride = K + XG_PAD, XV = K / 1024, SR = K >> 5;
  __shared__ __attribute__((aligned(16))) __bf16 xs[3 * stride];
  __shared__ __attribute__((aligned(16))) __bf16 zb[32];
  __shared__ __attribute__((aligned(16))) uint8_t sw[4][2][32][64];  // [wave][buffer][row][byte]
  const int p = blockIdx.y;
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int rho = col >> 2, kap = col & 3;
  const RbtExpertDev J = jobs[p];
  const long r0 = 16L * (4 * blockIdx.x + w);  // first row of the wave
  if (J.gd == nullptr || J.ud == nullptr) {
    for (int e = threadIdx.x; e < 3 * 64; e += 256)
      hp[((long)p * 3 + e / 64) * I + 64 * blockIdx.x + (e & 63)] = (__bf16)0.0f;
    return;
  }
  // activation first (the oldest loads in flight), then the scale window and the weight ring
  float4 xv[XV];
  {
    const rbt_gf4 *s4 = (const rbt_gf4 *)(x + (long)tok[p] * x_stride);
#pragma unroll
    for (int j = 0; j < XV; j++) xv[j] = s4[threadIdx.x + 256 * j];
  }
  XScale S;
  S.last = SR - 16 * ((lane & 3) + 1);
#pragma unroll
  for (int i = 0; i < 2; i++)
    S.p[i] = (const uint8_t *)(i ? J.us : J.gs) + (r0 + (lane >> 2)) * SR + 16 * (lane & 3);
  S.load(0);
  __builtin_amdgcn_sched_barrier(0);
  // lane pointers: tile t, matrix m (0 gate, 1 up)
  const uint8_t *wrow[2][4];
#pragma unroll
  for (int m = 0; m < 2; m++)
#pragma unroll
    for (int t = 0; t < 4; t++) wrow[m][t] = (m ? J.ud : J.gd) + (r0 + 4 * t + rho) * (K >> 1) + 64 * kap + 16 * g;
  rbt_u4 ring[XG_DEPTH][2][4];
#pragma unroll
  for (int d = 0; d < XG_DEPTH; d++) {
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
      for (int t = 0; t < 4; t++) ring[d][m][t] = __builtin_nontemporal_load((const rbt_gu4 *)(wrow[m][t] + 256 * d));
    __builtin_amdgcn_sched_barrier(0);
  }
  if (threadIdx.x < 32) zb[threadIdx.x] = (__bf16)0.0f;
#pragma unroll
  for (int j = 0; j < XV; j++) {
    const int q = threadIdx.x + 256 * j;
    const float e4[4] = {xv[j].x, xv[j].y, xv[j].z, xv[j].w};
#pragma unroll
    for (int e = 0; e < 4; e++) {
      __bf16 hh, mm, ll;
      split3(e4[e], hh, mm, ll);
      xs[4 * q + e] = hh;
      xs[stride + 4 * q + e] = mm;
      xs[2 * stride + 4 * q + e] = ll;
    }
  }
  // scale window of group 0, and group 1 in flight
#pragma unroll
  for (int i = 0; i < 2; i++) *reinterpret_cast<rbt_u4 *>(&sw[w][0][(lane >> 2) + 16 * i][16 * (lane & 3)]) = S.v[i];
  if (NCH > 4) S.load(1);
  __syncthreads();

  const int bq = col >> 2, bpart = col & 3;
  const char *bp = bpart < 3 ? reinterpret_cast<const char *>(xs + bpart * stride + 128 * bq + 32 * g)
                             : reinterpret_cast<const char *>(zb);
  const int binc = bpart < 3 ? 1024 : 0;  // bytes per step (512 bf16)
  xf4 acc[2][4];
#pragma unroll
  for (int m = 0; m < 2; m++)
#pragma unroll
    for (int t = 0; t < 4; t++) acc[m][t] = xf4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < NCH; c++) {
    const int d = c % XG_DEPTH;
    const XB B = xb_read(bp + binc * c);
    const uint8_t(*win)[64] = sw[w][(c >> 2) & 1];
    const int sb = 16 * (c & 3) + 4 * kap + g;
#pragma unroll
    for (int m = 0; m < 2; m++)
#pragma unroll
      for (int t = 0; t < 4; t++) xmma_s(ring[d][m][t], xe8m0(win[16 * m + 4 * t + rho][sb]), B, acc[m][t]);
    if (c + XG_DEPTH < NCH) {
#pragma unroll
      for (int m = 0; m < 2; m++)
#pragma unroll
        for (int t = 0; t < 4; t++)
          ring[d][m][t] = __builtin_nontemporal_load((const rbt_gu4 *)(wrow[m][t] + 256 * (c + XG_DEPTH)));
    }
    if ((c & 3) == 3 && c + 1 < NCH) {
      // group (c + 1) / 4 -> its window (this wave read the other buffer's last bytes just above)
      const int G = (c + 1) >> 2;
#pragma unroll
      for (int i = 0; i < 2; i++)
        *reinterpret_cast<rbt_u4 *>(&sw[w][G & 1][(lane >> 2) + 16 * i][16 * (lane & 3)]) = S.v[i];
      if (4 * (G + 1) < NCH) S.load(G + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
#pragma unroll
  for (int t = 0; t < 4; t++) {
    const float gv = row_dot(acc[0][t], col), uv = row_dot(acc[1][t], col);
    if (col == 0) {  // lane 16*g: row r0 + 4t + g
      const float hv = rbt_silu(gv) * uv;
      __bf16 hh, mm, ll;
      split3(hv, hh, mm, ll);
      const long rr = r0 + 4 * t + g;
      hp[((long)p * 3 + 0) * I + rr] = hh;
      hp[((long)p * 3 + 1) * I + rr] = mm;
      hp[((long)p * 3 + 2) * I + rr] = ll;
    }
  }
}

// gate/up for one token: the balanced body (rbt_xmfma.h) over the whole grid.
template <int NCH>
__global__ __launch_bounds__(256) void k_xgateup1(const RbtExpertDev *__restrict__ jobs, int npairs,
                                                  const float *__restrict__ x, int I, __bf16 *__restrict__ hp) {
  __shared__ GuLds L;
  xgateup1_body<NCH>(L, jobs, npairs, x, I, hp, blockIdx.x, gridDim.x);
}

// ------------------------------------------------------------------------------------------------
// down + combine: grid (H/16), 256 threads. Wave w owns output rows 16*blockIdx.x + 4w .. +3 (one
// tile) over all I = 512*NCH columns, for every pair of the call in pair order, with each pair's h
// parts (hp, bf16) staged in LDS by the whole workgroup. The ordered combine of
//   out[t, r] = sum_j w[t,j] * y_{pair(t,j)}[r]   (pairs in tok_pair order, separate roundings)
//             + shared_t[r] * sh_scale[t]         (has_shared; the scale only when gated)
// is accumulated per (token, row) in LDS as the pairs arrive: pairs are grouped in the order
// tok_pair lists them (first occurrence), so each token's terms come in its own order, and the
// shared pairs [S*k, S*k + S) come last. Requires npairs <= XD_MAXP, S <= 16.
// ------------------------------------------------------------------------------------------------
constexpr int XD_DEPTH = 8;  // (pair, step) chunks in flight per wave: two pairs of NCH = 4 steps

template <int NCH>
__global__ __launch_bounds__(256) void k_xdown(const RbtExpertDev *__restrict__ jobs, int npairs,
                                               const __bf16 *__restrict__ hp, int I, int H, int S, int k,
                                               const int *__restrict__ tok, const int *__restrict__ tok_pair,
                                               const float *__restrict__ tok_w, const float *__restrict__ sh_scale,
                                               int has_shared, int gated, float *__restrict__ out) {
  constexpr int KD = NCH * 512, stride = KD + XG_PAD, SRD = KD >> 5;
  constexpr int HV = 3 * KD / 8 / 256;  // 16-byte pieces of a pair's parts per thread
  static_assert(SRD == 64, "a row's scale bytes are four 16-byte pieces");
  __shared__ __attribute__((aligned(16))) __bf16 hs[2][3 * stride];
  __shared__ float oacc[16][16];  // [token][row of the workgroup]
  __shared__ float pw[XD_MAXP];   // weight of each pair (routing weight or shared scale)
  __shared__ int ptok[XD_MAXP];   // token of each pair (-1: adds nothing)
  __shared__ const uint8_t *pd[XD_MAXP];  // down codes / scales of each pair (a live pair's for null jobs)
  __shared__ const uint8_t *ps[XD_MAXP];
  __shared__ int plive[XD_MAXP];
  __shared__ __attribute__((aligned(16))) uint8_t sw[4][2][4][4][64];  // [wave][buffer][pair of group][row][byte]
  __shared__ __attribute__((aligned(16))) __bf16 zb[32];
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, g = lane >> 4, col = lane & 15;
  const int rho = col >> 2, kap = col & 3;
  const int P = S * k;
  if (threadIdx.x < 32) zb[threadIdx.x] = (__bf16)0.0f;
  oacc[threadIdx.x >> 4][threadIdx.x & 15] = 0.0f;
  for (int pp = threadIdx.x; pp < npairs; pp += 256) {
    float wv = 0.0f;
    int tt = pp < P ? tok[pp] : pp - P;
    if (pp < P) {
      for (int j = 0; j < k; j++)
        if (tok_pair[tt * k + j] == pp) wv = tok_w[tt * k + j];
    } else {
      wv = gated ? sh_scale[tt] : 1.0f;
    }
    const RbtExpertDev J = jobs[pp];
    plive[pp] = J.dd != nullptr && J.ds != nullptr;
    pd[pp] = J.dd;
    ps[pp] = (const uint8_t *)J.ds;
    pw[pp] = wv;
    ptok[pp] = (pp < P || has_shared) ? tt : -1;
  }
  __syncthreads();
  // Pairs with a null job read the rows of the first live pair (valid memory) and add nothing.
  int live0 = -1;
  for (int pp = 0; pp < npairs && live0 < 0; pp++)
    if (plive[pp]) live0 = pp;
  if (live0 < 0) {
    const int t = threadIdx.x >> 4, rr = threadIdx.x & 15;
    if (t < S) out[(long)t * H + 16 * blockIdx.x + rr] = 0.0f;
    return;
  }
  __syncthreads();
  for (int pp = threadIdx.x; pp < npairs; pp += 256)
    if (!plive[pp]) {
      pd[pp] = pd[live0];
      ps[pp] = ps[live0];
      ptok[pp] = -1;
    }
  __syncthreads();
  const int tile_r0 = 16 * blockIdx.x + 4 * w;
  const long wrow = (long)(tile_r0 + rho) * (KD >> 1) + 64 * kap + 16 * g;  // lane's code offset in a matrix
  // chunk (pair q, step c) of the lane; past the last pair the loads read the cached activation
  // parts instead (never used)
  const uint8_t *dummy = reinterpret_cast<const uint8_t *>(hp) + 64 * kap + 16 * g;
  auto chunk = [&](int q, int c) {
    const uint8_t *a = q < npairs ? pd[min(q, npairs - 1)] + wrow : dummy;
    return __builtin_nontemporal_load((const rbt_gu4 *)(a + 256 * c));
  };
  // scale window of pair group G (4 pairs): lane l holds pair 4G + l/16, row (l/4) % 4, bytes 16 (l % 4)
  const int s_q = lane >> 4, s_row = (lane >> 2) & 3, s_seg = lane & 3;
  auto sload = [&](int G) {
    return *(const rbt_gu4 *)(ps[min(4 * G + s_q, npairs - 1)] + (long)(tile_r0 + s_row) * SRD + 16 * s_seg);
  };
  auto sstore = [&](int buf, const rbt_u4 &v) {
    *reinterpret_cast<rbt_u4 *>(&sw[w][buf][s_q][s_row][16 * s_seg]) = v;
  };
  rbt_u4 hv[2][HV];
  auto load_h = [&](int q, rbt_u4 (&dst)[HV]) {
    const rbt_gu4 *s4 = (const rbt_gu4 *)(hp + (long)min(q, npairs - 1) * 3 * KD);
#pragma unroll
    for (int j = 0; j < HV; j++) dst[j] = s4[threadIdx.x + 256 * j];
  };
  auto store_h = [&](int buf, const rbt_u4 (&src)[HV]) {
#pragma unroll
    for (int j = 0; j < HV; j++) {
      const int e = 8 * (threadIdx.x + 256 * j);  // element in [0, 3*KD)
      const int part = e / KD, kk = e - part * KD;
      *reinterpret_cast<rbt_u4 *>(&hs[buf][part * stride + kk]) = src[j];
    }
  };
  // prologue: h of pairs 0 and 1, scale windows of groups 0 (stored) and 1 (in flight), codes of
  // pairs 0 and 1 in the ring
  load_h(0, hv[0]);
  load_h(1, hv[1]);
  rbt_u4 sv = sload(0);
  rbt_u4 ring[2 * NCH];
#pragma unroll
  for (int i = 0; i < 2 * NCH; i++) ring[i] = chunk(i / NCH, i % NCH);
  store_h(0, hv[0]);
  sstore(0, sv);
  sv = sload(1);
  __syncthreads();
  const int bq = col >> 2, bpart = col & 3;
  const int boff = bpart < 3 ? 2 * (bpart * stride + 128 * bq + 32 * g) : -1;
  const int binc = bpart < 3 ? 1024 : 0;
  const int ngroups = (npairs + 3) / 4;
  for (int G = 0; G < ngroups; G++) {
#pragma unroll
    for (int h4 = 0; h4 < 4; h4++) {
      const int cp = 4 * G + h4, hb = h4 & 1;
      // h of pair cp + 2 (stored to LDS at the end of pair cp + 1)
      load_h(cp + 2, hv[hb]);
      const char *bp = boff >= 0 ? reinterpret_cast<const char *>(hs[hb]) + boff : reinterpret_cast<const char *>(zb);
      const uint8_t(*win)[64] = sw[w][G & 1][h4];
      xf4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int c = 0; c < NCH; c++) {
        const int slot = hb * NCH + c;
        const XB B = xb_read(bp + binc * c);
        const rbt_u4 cw = ring[slot];
        ring[slot] = chunk(cp + 2, c);
        xmma_s(cw, xe8m0(win[rho][16 * c + 4 * kap + g]), B, acc);
        __builtin_amdgcn_sched_barrier(0);
      }
      const float y = row_dot(acc, col);
      if (cp < npairs) {
        const int tt = ptok[cp];
        if (col == 0 && tt >= 0) {  // lane 16*g: row tile_r0 + g
          float &o = oacc[tt][4 * w + g];
          o = __fadd_rn(o, __fmul_rn(pw[cp], y));
        }
      }
      store_h(hb ^ 1, hv[hb ^ 1]);  // h of pair cp + 1 (loaded during pair cp - 1)
      __syncthreads();
    }
    sstore((G + 1) & 1, sv);
    sv = sload(G + 2);
  }
  const int t = threadIdx.x >> 4, rr = threadIdx.x & 15;
  if (t < S) out[(long)t * H + 16 * blockIdx.x + rr] = oacc[t][rr];
}

// ------------------------------------------------------------------------------------------------
// down + combine for one token, balanced over the whole chip: one workgroup of XD1_NW waves per CU.
// Workgroup b owns the 4-row output tiles [T0, T1) (an equal share of H/4) and the units
// (tile, pair) over them, u = pair * nt + tile (a wave's units are consecutive tiles of one pair:
// runs of contiguous weight rows), dealt evenly over its waves. Every pair's h
// parts are staged in LDS once (no per-pair barriers); a wave streams its units' 16-byte code chunks
// with four units (16 chunks) in flight, block scales for four units at a time through a
// wave-private LDS window (one 16-byte load per lane), and leaves each unit's four row sums in LDS.
// The ordered combine then runs per output row over the pair list: the winners in slot (rank)
// order, the shared pair last:
//   out[r] = (...(w_0 y_0[r] + w_1 y_1[r]) + ...) + w_s y_s[r]   (separate roundings)
// the reference's order (qwen38/generate.rs:303-349). The pair list is compact (its h may sit at
// any pair slot), so the launch covers exactly the experts that are combined.
// ------------------------------------------------------------------------------------------------
constexpr int XD1_NP = 11;   // pairs whose h fits in LDS (top-10 + shared at I = 2048)
constexpr int XD1_NW = 8;    // waves per workgroup
constexpr int XD1_TPW = 16;  // most 4-row tiles per workgroup



template <int NCH>
__global__ __launch_bounds__(64 * XD1_NW) void k_xdown1(const RbtExpertDev *__restrict__ jobs,
                                                        const int *__restrict__ slots, int kk,
                                                        const __bf16 *__restrict__ hp, int H,
                                                        const float *__restrict__ tok_w,
                                                        const float *__restrict__ sh_scale, int has_shared,
                                                        int gated, float *__restrict__ out, int accumulate,
                                                        const uint8_t *__restrict__ sh_dd,
                                                        const uint8_t *__restrict__ sh_ds) {
  // pairs: the kk winners in slot order (jobs[j], h at pair slot slots[j], weight tok_w[j]), then
  // the shared expert (jobs[kk], h at slots[kk], weight sh_scale when gated, else 1)
  const int npairs = kk + (has_shared ? 1 : 0);
  // With the shared expert's pointers given (sh_dd, sh_ds), the waves take it first: its first
  // window goes out at entry, before the pair tables land (the combine keeps the pair order).
  const bool shf = has_shared && sh_dd != nullptr && sh_ds != nullptr;
  auto pp_of = [&](int q) { return shf ? (q == 0 ? npairs - 1 : q - 1) : q; };  // pair of processing slot q
  constexpr int KD = NCH * 512, stride = KD + XG_PAD, SRD = KD >> 5;
  constexpr int PPP = 3 * KD / 8;                                  // 16-byte pieces of one pair's parts
  constexpr int HI = (XD1_NP * PPP + 64 * XD1_NW - 1) / (64 * XD1_NW);  // pieces per thread
  static_assert(NCH == 4 && SRD == 64, "a unit is 4 rows x 4 chunks with 64 scale bytes per row");
  __shared__ __attribute__((aligned(16))) __bf16 hs[XD1_NP][3 * stride];
  __shared__ __attribute__((aligned(16))) uint8_t sw[XD1_NW][2][4][4][64];  // [wave][buffer][unit][row][byte]
  __shared__ float yb[XD1_TPW][XD1_NP][4];  // row sums per (tile, pair)
  __shared__ float pw[XD1_NP];
  __shared__ const uint8_t *pd[XD1_NP];
  __shared__ const uint8_t *ps[XD1_NP];
  __shared__ int plive[XD1_NP], padd[XD1_NP];
  __shared__ __attribute__((aligned(16))) __bf16 zb[32];
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, col = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rho = col >> 2, kap = col & 3;
  const int ntile = H >> 2;
  const int T0 = (int)((long)blockIdx.x * ntile / gridDim.x), T1 = (int)((long)(blockIdx.x + 1) * ntile / gridDim.x);
  const int nt = T1 - T0;
  const int NU = nt * npairs;
  // Wave w takes units w, w + NW, w + 2 NW, ... (its i-th unit is uu(i)): the eight waves move
  // through the pairs together, so a window touches the pages of a few experts at a time instead of
  // every expert's at the start (each new page costs the CU a translation miss).
  const int nu = NU > w ? (NU - w + XD1_NW - 1) / XD1_NW : 0;
  auto uu = [&](int i) { return w + XD1_NW * i; };
  const uint8_t *hb8 = reinterpret_cast<const uint8_t *>(hp);
  const uint8_t *dummy = hb8 + 64 * kap + 16 * g;
  const int s_q = lane >> 4, s_row = (lane >> 2) & 3, s_seg = lane & 3;
  rbt_u4 ring[4][NCH];
  const bool early = shf && nu > 0 && uu(0) < nt;  // the wave's first unit is a shared-expert tile
  if (early) {
    const uint8_t *c0 = sh_dd + (long)(4 * (T0 + uu(0)) + rho) * (KD >> 1) + 64 * kap + 16 * g;
#pragma unroll
    for (int c = 0; c < NCH; c++) ring[0][c] = __builtin_nontemporal_load((const rbt_gu4 *)(c0 + 256 * c));
  }
  __builtin_amdgcn_sched_barrier(0);
  // Prologue. vmcnt counts loads in issue order, so everything the staging barrier waits for (the h
  // parts, the pair tables, the first scale window) is issued before the first window's weights:
  // the h pieces come from L2 while the weights (128 KB per CU, all CUs at once) take the HBM's time,
  // and waiting for the h pieces then does not mean waiting for the weights.
  // Pair tables first, as one vector load per lane (lane p: pair p's pointers, slot and weight;
  // clamped): the table was written by the previous launch, possibly on another XCD, so every load
  // of it is a trip to memory, and chains of dependent scalar loads would pay that trip each time.
  const int tp = min(lane, npairs - 1);
  const RbtExpertDev *J = jobs + tp;
  const uint8_t *t_dd = J->dd;
  const uint8_t *t_ds = (const uint8_t *)J->ds;
  const int t_slot = slots[tp];
  const float t_w = tp < kk ? tok_w[min(tp, kk - 1)] : (gated ? sh_scale[0] : 1.0f);
  auto lane_ptr = [](const uint8_t *p, int l) -> const uint8_t * {
    const uint64_t v = reinterpret_cast<uint64_t>(p);
    const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l);
    const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
    return reinterpret_cast<const uint8_t *>(((uint64_t)hi << 32) | lo);
  };
  // First window (units 0 .. 3 of the wave): pointers from the tables' lanes (the pair is
  // wave-uniform).
  const uint8_t *cp[4], *sp[4];
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int u = uu(j);
    cp[j] = dummy;
    sp[j] = hb8 + 16 * s_seg;
    if (j < nu) {
      const int q = u / nt, pp = pp_of(q), tl = u - q * nt;
      const bool shq = shf && q == 0;
      const uint8_t *dd = shq ? sh_dd : lane_ptr(t_dd, pp);
      const uint8_t *ds = shq ? sh_ds : lane_ptr(t_ds, pp);
      if (dd != nullptr && ds != nullptr) {
        cp[j] = dd + (long)(4 * (T0 + tl) + rho) * (KD >> 1) + 64 * kap + 16 * g;
        sp[j] = ds + (long)(4 * (T0 + tl) + s_row) * SRD + 16 * s_seg;
      }
    }
  }
  // h parts of every pair: pieces e = tid + 512 i (clamped reads stay inside the pair list), in an
  // order rotated by workgroup so that the grid does not read the same lines at the same time.
  // Piece row ii spans pairs ii*512/PPP and the next one (their slots from the tables' lanes).
  const int npc = npairs * PPP;
  rbt_u4 hr[HI];
  const int rot = blockIdx.x % HI;
#pragma unroll
  for (int i = 0; i < HI; i++) {
    const int ii = i + rot < HI ? i + rot : i + rot - HI;
    const int e = min(tid + 64 * XD1_NW * ii, npc - 1), pp = e / PPP;
    const int pa = min(64 * XD1_NW * ii / PPP, npairs - 1), pb = min(pa + 1, npairs - 1);
    const int sa = __builtin_amdgcn_readlane(t_slot, pa), sb = __builtin_amdgcn_readlane(t_slot, pb);
    const long slot = pp == pa ? sa : sb;
    hr[i] = *(const rbt_gu4 *)(hp + 8L * (slot * PPP + (e - pp * PPP)));
  }
  rbt_u4 sv = *(const rbt_gu4 *)(s_q == 0 ? sp[0] : s_q == 1 ? sp[1] : s_q == 2 ? sp[2] : sp[3]);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 4; j++)
    if (j > 0 || !early) {
#pragma unroll
      for (int c = 0; c < NCH; c++) ring[j][c] = __builtin_nontemporal_load((const rbt_gu4 *)(cp[j] + 256 * c));
    }
  __builtin_amdgcn_sched_barrier(0);
  if (tid < 32) zb[tid] = (__bf16)0.0f;
  if (w == 0 && lane < npairs) {
    const int live = t_dd != nullptr && t_ds != nullptr;
    plive[lane] = live;
    padd[lane] = live;
    pd[lane] = t_dd;
    ps[lane] = t_ds;
    pw[lane] = t_w;
  }
#pragma unroll
  for (int i = 0; i < HI; i++) {
    const int ii = i + rot < HI ? i + rot : i + rot - HI;
    const int e = tid + 64 * XD1_NW * ii;
    if (e < npc) {
      const int pp = e / PPP, q = e - pp * PPP;
      *reinterpret_cast<rbt_u4 *>(&hs[pp][(q / (KD / 8)) * stride + 8 * (q % (KD / 8))]) = hr[i];
    }
  }
  // lane pointer of the wave's unit i (chunk 0); past its units or for a null job: cached dummy bytes
  auto uptr = [&](int i) -> const uint8_t * {
    if (i >= nu) return dummy;
    const int u = uu(i), q = u / nt, pp = pp_of(q), tl = u - q * nt;
    return plive[pp] ? pd[pp] + (long)(4 * (T0 + tl) + rho) * (KD >> 1) + 64 * kap + 16 * g : dummy;
  };
  // scale window of the wave's units ib .. ib+3: lane l holds unit ib + l/16, row (l/4) % 4, bytes
  // 16 (l % 4)
  auto sload = [&](int ib) {
    const int i = ib + s_q;
    const uint8_t *p = hb8 + 16 * s_seg;
    if (i < nu) {
      const int u = uu(i), q = u / nt, pp = pp_of(q), tl = u - q * nt;
      if (plive[pp]) p = ps[pp] + (long)(4 * (T0 + tl) + s_row) * SRD + 16 * s_seg;
    }
    return *(const rbt_gu4 *)p;
  };
  auto sstore = [&](int buf, const rbt_u4 &v) {
    *reinterpret_cast<rbt_u4 *>(&sw[w][buf][s_q][s_row][16 * s_seg]) = v;
  };
  sstore(0, sv);
  lds_barrier();  // tables, h parts, first scale windows
  sv = sload(4);
  const int bq = col >> 2, bpart = col & 3;
  const int boff = bpart < 3 ? 2 * (bpart * stride + 128 * bq + 32 * g) : -1;
  const int binc = bpart < 3 ? 1024 : 0;
  int buf = 0;
  for (int ib = 0; ib < nu; ib += 4) {
    const uint8_t(*win)[4][64] = sw[w][buf];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = ib + j;
      const uint8_t *np = uptr(i + 4);
      rbt_u4 cw[NCH];
#pragma unroll
      for (int c = 0; c < NCH; c++) {
        cw[c] = ring[j][c];
        ring[j][c] = __builtin_nontemporal_load((const rbt_gu4 *)(np + 256 * c));
      }
      if (i < nu) {
        const int u = uu(i), q = u / nt, pp = pp_of(q), tl = u - q * nt;
        const char *bp = boff >= 0 ? reinterpret_cast<const char *>(hs[pp]) + boff : reinterpret_cast<const char *>(zb);
        xf4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NCH; c++) {
          const XB B = xb_read(bp + binc * c);
          xmma_s(cw[c], xe8m0(win[j][rho][16 * c + 4 * kap + g]), B, acc);
        }
        const float y = row_dot(acc, col);
        if (col == 0) yb[tl][pp][g] = y;  // lane 16 g: row 4 (T0 + tl) + g
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    buf ^= 1;
    sstore(buf, sv);
    sv = sload(ib + 8);
  }
  __syncthreads();
  if (tid < 4 * nt) {
    const int tl = tid >> 2, r = tid & 3;
    float o = 0.0f;
    for (int pp = 0; pp < npairs; pp++)
      if (padd[pp]) o = __fadd_rn(o, __fmul_rn(pw[pp], yb[tl][pp][r]));
    if (accumulate) o = __fadd_rn(out[4 * (T0 + tl) + r], o);  // x += layer(x) (qwen38/generate.rs:411-413)
    out[4 * (T0 + tl) + r] = o;
  }
}

// ------------------------------------------------------------------------------------------------
// down for one token, pair-major: the U = npairs * H/4 units (pair q, 4-row output tile) in pair
// order are dealt as contiguous runs over every wave of the grid (wave i of NW: units
// [i U / NW, (i + 1) U / NW)). A wave streams consecutive 4 KB tiles of one expert's down rows and a
// workgroup's run (XD2_NW waves x U / NW units, 352 KB at C1) covers at most two experts, so the
// workgroup stages the h parts of at most two pairs (24 KB of LDS, against all eleven pairs' 135 KB
// when a workgroup owns output rows of every pair) and touches few pages. Each unit's four row sums
// go to yy[pair][row]; k_combine1 then forms the ordered combine over the pairs.
// Processing order: with the shared expert's down pointers given (sh_dd, sh_ds), the shared expert
// is processed first (q = 0), so the waves whose run lies in it issue their first window from kernel
// arguments, before the pair tables land (its h slot still comes from the table); yy keeps the pair
// list's order (the winners, then the shared expert at npairs - 1).
// ------------------------------------------------------------------------------------------------
constexpr int XD2_NW = 8;     // waves per workgroup
constexpr int XD2_NP = 2;     // pairs whose h a workgroup stages
constexpr int XD2_TB = 16;    // output tiles per block of the fused combine (64 rows)
constexpr int XD2_MAXB = 32;  // blocks one workgroup can complete
constexpr int XD2_MAXU = (XD2_MAXB - 4) * XD2_TB;  // most units of one workgroup (xdown2_ok)
constexpr int XC1_MAXP = 64;  // pairs of the combine
constexpr bool XD2_FUSED = true;  // the combine in the down launch (else k_combine1)

template <int NCH, bool FC>
__global__ __launch_bounds__(64 * XD2_NW) void k_xdown2(const RbtExpertDev *__restrict__ jobs,
                                                        const int *__restrict__ slots, int npairs,
                                                        const __bf16 *__restrict__ hp, int H,
                                                        float *__restrict__ yy, const uint8_t *__restrict__ sh_dd,
                                                        const uint8_t *__restrict__ sh_ds, int kk, int gated,
                                                        const float *__restrict__ tok_w,
                                                        const float *__restrict__ sh_scale, float *__restrict__ out,
                                                        int accumulate, unsigned *__restrict__ cnt) {
  constexpr int KD = NCH * 512, stride = KD + XG_PAD, SRD = KD >> 5;
  constexpr int PPP = 3 * KD / 8;                                        // 16-byte pieces of one pair's parts
  constexpr int HI = (XD2_NP * PPP + 64 * XD2_NW - 1) / (64 * XD2_NW);  // pieces per thread
  static_assert(NCH == 4 && SRD == 64, "a unit is 4 rows x 4 chunks with 64 scale bytes per row");
  __shared__ __attribute__((aligned(16))) __bf16 hs[XD2_NP][3 * stride];
  __shared__ __attribute__((aligned(16))) uint8_t sw[XD2_NW][2][4][4][64];  // [wave][buffer][unit][row][byte]
  __shared__ __attribute__((aligned(16))) __bf16 zb[32];
  __shared__ float pw[XC1_MAXP];  // FC: the combine's pair weights and liveness
  __shared__ int plive[XC1_MAXP];
  __shared__ int lastb[XD2_MAXB], nlast;
  __shared__ float yl[FC ? 4 * XD2_MAXU : 1];  // FC: the row sums of the workgroup's units [b0, b1)
  const int tid = threadIdx.x, lane = tid & 63, g = lane >> 4, col = lane & 15;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int rho = col >> 2, kap = col & 3;
  const int nt = H >> 2;
  const bool shf = sh_dd != nullptr && sh_ds != nullptr;
  // FC: pair j's liveness and combine weight, loaded by lane j of wave 1 now (independent loads, no
  // waits) and put in LDS after the stream
  uint64_t f_dd = 0, f_ds = 0;
  float f_w = 0.0f, f_s = 0.0f;
  if (FC && w == 1) {
    const int jl = min(lane, npairs - 1);
    f_dd = reinterpret_cast<uint64_t>(jobs[jl].dd);
    f_ds = reinterpret_cast<uint64_t>(jobs[jl].ds);
    f_w = tok_w[min(jl, max(kk - 1, 0))];
    f_s = sh_scale[0];
  }
  if (FC && tid == 0) nlast = 0;
  // pair-list index of processing pair q
  auto pl_of = [&](int q) { return shf ? (q == 0 ? npairs - 1 : q - 1) : q; };
  const long U = (long)npairs * nt, NWT = (long)gridDim.x * XD2_NW, wi = (long)blockIdx.x * XD2_NW + w;
  const int u0 = (int)(wi * U / NWT), nu = (int)((wi + 1) * U / NWT) - u0;
  const int b0 = (int)((long)blockIdx.x * XD2_NW * U / NWT);
  const int b1 = (int)((long)(blockIdx.x + 1) * XD2_NW * U / NWT);
  const int qa = b0 / nt, qb = min(max(b1 - 1, b0) / nt, npairs - 1);  // the workgroup's pairs (qb <= qa + 1)
  const uint8_t *hb8 = reinterpret_cast<const uint8_t *>(hp);
  const uint8_t *dummy = hb8 + 64 * kap + 16 * g;
  const int s_q = lane >> 4, s_row = (lane >> 2) & 3, s_seg = lane & 3;
  // The workgroup's two pairs (local 0 = qa, 1 = qb): down pointers and h slots, from the kernel
  // arguments for the shared expert, else from the tables (lane l loads local pair l & 1).
  const uint8_t *pdd[XD2_NP], *pds[XD2_NP];
  int pslot[XD2_NP];
  {
    const int ql = min(qa + (lane & 1), qb), pl = pl_of(ql);
    const bool tab = !(shf && ql == 0);
    // the three table loads unconditionally (one trip to memory), then the choice
    const uint8_t *j_dd = jobs[pl].dd;
    const uint8_t *j_ds = (const uint8_t *)jobs[pl].ds;
    const int t_slot = slots[pl];  // the shared expert's h slot is decided on the device (after the routed pairs)
    const uint8_t *t_dd = tab ? j_dd : sh_dd;
    const uint8_t *t_ds = tab ? j_ds : sh_ds;
    auto lane_ptr = [](const uint8_t *p, int l) -> const uint8_t * {
      const uint64_t v = reinterpret_cast<uint64_t>(p);
      const uint32_t lo = __builtin_amdgcn_readlane((uint32_t)v, l);
      const uint32_t hi = __builtin_amdgcn_readlane((uint32_t)(v >> 32), l);
      return reinterpret_cast<const uint8_t *>(((uint64_t)hi << 32) | lo);
    };
#pragma unroll
    for (int i = 0; i < XD2_NP; i++) {
      pdd[i] = lane_ptr(t_dd, i);
      pds[i] = lane_ptr(t_ds, i);
      pslot[i] = __builtin_amdgcn_readlane(t_slot, i);
    }
  }
  const bool live[XD2_NP] = {pdd[0] != nullptr && pds[0] != nullptr, pdd[1] != nullptr && pds[1] != nullptr};
  // lane pointers of the wave's unit i: codes at chunk 0, and its piece of the scale window
  auto uptr = [&](int i) -> const uint8_t * {
    if (i >= nu) return dummy;
    const int u = u0 + i, q = u / nt, tl = u - q * nt, lq = q - qa;
    const uint8_t *dd = lq == 0 ? pdd[0] : pdd[1];
    return (lq == 0 ? live[0] : live[1]) ? dd + (long)(4 * tl + rho) * (KD >> 1) + 64 * kap + 16 * g : dummy;
  };
  auto sload = [&](int ib) {
    const int i = ib + s_q;
    const uint8_t *p = hb8 + 16 * s_seg;
    if (i < nu) {
      const int u = u0 + i, q = u / nt, tl = u - q * nt, lq = q - qa;
      if (lq == 0 ? live[0] : live[1]) p = (lq == 0 ? pds[0] : pds[1]) + (long)(4 * tl + s_row) * SRD + 16 * s_seg;
    }
    return *(const rbt_gu4 *)p;
  };
  // h parts of the workgroup's pairs first (vmcnt counts loads in issue order: waiting for them then
  // does not mean waiting for the weights issued after them)
  const int npc = (qb - qa + 1) * PPP;
  rbt_u4 hr[HI];
#pragma unroll
  for (int i = 0; i < HI; i++) {
    const int e = min(tid + 64 * XD2_NW * i, npc - 1), lq = e / PPP;
    const long slot = lq == 0 ? pslot[0] : pslot[1];
    hr[i] = *(const rbt_gu4 *)(hp + 8L * (slot * PPP + (e - lq * PPP)));
  }
  rbt_u4 sv = sload(0);
  rbt_u4 ring[4][NCH];
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const uint8_t *cp = uptr(j);
#pragma unroll
    for (int c = 0; c < NCH; c++) ring[j][c] = __builtin_nontemporal_load((const rbt_gu4 *)(cp + 256 * c));
  }
  __builtin_amdgcn_sched_barrier(0);
  if (tid < 32) zb[tid] = (__bf16)0.0f;
#pragma unroll
  for (int i = 0; i < HI; i++) {
    const int e = tid + 64 * XD2_NW * i;
    if (e < npc) {
      const int lq = e / PPP, r = e - lq * PPP;
      *reinterpret_cast<rbt_u4 *>(&hs[lq][(r / (KD / 8)) * stride + 8 * (r % (KD / 8))]) = hr[i];
    }
  }
  auto sstore = [&](int buf, const rbt_u4 &v) {
    *reinterpret_cast<rbt_u4 *>(&sw[w][buf][s_q][s_row][16 * s_seg]) = v;
  };
  sstore(0, sv);
  lds_barrier();  // h parts, first scale windows
  sv = sload(4);
  const int bq = col >> 2, bpart = col & 3;
  const int boff = bpart < 3 ? 2 * (bpart * stride + 128 * bq + 32 * g) : -1;
  const int binc = bpart < 3 ? 1024 : 0;
  int buf = 0;
  for (int ib = 0; ib < nu; ib += 4) {
    const uint8_t(*win)[4][64] = sw[w][buf];
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = ib + j;
      const uint8_t *np = uptr(i + 4);
      rbt_u4 cw[NCH];
#pragma unroll
      for (int c = 0; c < NCH; c++) {
        cw[c] = ring[j][c];
        ring[j][c] = __builtin_nontemporal_load((const rbt_gu4 *)(np + 256 * c));
      }
      if (i < nu) {
        const int u = u0 + i, q = u / nt, tl = u - q * nt, lq = q - qa;
        const char *bp = boff >= 0 ? reinterpret_cast<const char *>(hs[lq]) + boff : reinterpret_cast<const char *>(zb);
        xf4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < NCH; c++) {
          const XB B = xb_read(bp + binc * c);
          xmma_s(cw[c], xe8m0(win[j][rho][16 * c + 4 * kap + g]), B, acc);
        }
        const float y = row_dot(acc, col);
        if (col == 0) {
          const float yv = (lq == 0 ? live[0] : live[1]) ? y : 0.0f;
          if constexpr (FC)
            yl[4 * (u - b0) + g] = yv;  // written to yy in one pass after the stream
          else
            yy[(long)pl_of(q) * H + 4 * tl + g] = yv;
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    buf ^= 1;
    sstore(buf, sv);
    sv = sload(ib + 8);
  }
  if constexpr (FC) {
    // The ordered combine by the last contributor of each block of XD2_TB output tiles: the
    // workgroup adds the tiles it wrote to the block's arrival counter once its rows of yy are
    // complete; the workgroup that completes npairs x (the block's tiles) combines the block and
    // returns the counter to 0. No workgroup waits for another. The rows of yy, the counters and
    // the combine's reads are device-scope atomic accesses, performed at the device's point of
    // coherence (no cache of one XCD holds them), so no cache-wide write-back or invalidate is
    // needed: a row store completes (vmcnt 0) before the counter add that announces it, and the
    // combine reads after its add has seen every announcement.
    // The workgroup's rows of yy leave in one coalesced pass (device-scope stores inside the stream
    // loop, one per unit, slowed the weight stream by about a tenth).
    __syncthreads();
    for (int e = tid; e < 4 * (b1 - b0); e += 64 * XD2_NW) {
      const int u = b0 + (e >> 2), q = u / nt, tl = u - q * nt;
      __hip_atomic_store(yy + (long)pl_of(q) * H + 4 * tl + (e & 3), yl[e], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);  // at the device's coherence point
    }
    __builtin_amdgcn_s_waitcnt(0);  // this thread's rows of yy are complete
    if (w == 1 && lane < npairs) {
      asm volatile("" : "+v"(f_dd), "+v"(f_ds), "+v"(f_w), "+v"(f_s));  // used here, so waited for here
      plive[lane] = f_dd != 0 && f_ds != 0;
      pw[lane] = lane < kk ? f_w : (gated ? f_s : 1.0f);
    }
    __syncthreads();
    // the workgroup's segments: pair qa's tiles [ta0, ta1), then pair qb's [0, tb1) when qb > qa
    const int ta0 = b0 - qa * nt, ta1 = min(b1, (qa + 1) * nt) - qa * nt, tb1 = qb > qa ? b1 - qb * nt : 0;
    const int na = ta1 > ta0 ? (ta1 - 1) / XD2_TB - ta0 / XD2_TB + 1 : 0;
    const int nb = tb1 > 0 ? (tb1 - 1) / XD2_TB + 1 : 0;
    if (tid < na + nb) {
      const bool sa = tid < na;
      const int blk = sa ? ta0 / XD2_TB + tid : tid - na;
      const int lo = max(blk * XD2_TB, sa ? ta0 : 0), hi = min((blk + 1) * XD2_TB, sa ? ta1 : tb1);
      const unsigned n = (unsigned)(hi - lo);
      const unsigned tgt = (unsigned)npairs * (unsigned)(min((blk + 1) * XD2_TB, nt) - blk * XD2_TB);
      const unsigned old = __hip_atomic_fetch_add(&cnt[blk], n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (old + n == tgt) lastb[atomicAdd(&nlast, 1)] = blk;
    }
    __syncthreads();
    const int nl = nlast;
    if (nl > 0) {
      constexpr int RB = 4 * XD2_TB;  // rows per block
      for (int i0 = 0; i0 < nl; i0 += 64 * XD2_NW / RB) {
        const int i = i0 + tid / RB;
        if (i < nl) {
          const int r = lastb[i] * RB + tid % RB;
          if (r < H) {
            constexpr int CH = 16;  // the rows of 16 pairs in flight at once
            float o = 0.0f;
            for (int j0 = 0; j0 < npairs; j0 += CH) {
              float v[CH];
#pragma unroll
              for (int u = 0; u < CH; u++)
                v[u] = __hip_atomic_load(yy + (long)min(j0 + u, npairs - 1) * H + r, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
              for (int u = 0; u < CH; u++)
                if (j0 + u < npairs && plive[j0 + u]) o = __fadd_rn(o, __fmul_rn(pw[j0 + u], v[u]));
            }
            if (accumulate) o = __fadd_rn(out[r], o);
            out[r] = o;
          }
        }
      }
      if (tid < nl) __hip_atomic_store(&cnt[lastb[tid]], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
}

// The ordered combine of one token over the pair list of the down launch (yy rows: the kk winners
// in rank order, then the shared expert):
//   out[r] = (...(w_0 y_0[r] + w_1 y_1[r]) + ...) + s y_s[r]   (s: the shared gate when gated, else 1)
// with separate roundings, the reference's order (qwen38/generate.rs:303-349); a pair whose job is
// null (reported through the error flag) is left out. With accumulate, out[r] + (that) in one
// rounding (x += layer(x), qwen38/generate.rs:411-413).

__global__ __launch_bounds__(256) void k_combine1(const float *__restrict__ yy, const RbtExpertDev *__restrict__ jobs,
                                                  int kk, int has_shared, int gated,
                                                  const float *__restrict__ tok_w,
                                                  const float *__restrict__ sh_scale, int H,
                                                  float *__restrict__ out, int accumulate) {
  // the rows and the pair tables go out together (lane l of every wave reads pair l's entry)
  const int npairs = kk + (has_shared ? 1 : 0);
  const int lane = threadIdx.x & 63;
  const int r = min((int)(blockIdx.x * 256 + threadIdx.x), H - 1);
  constexpr int CH = 16;
  float o = 0.0f;
  for (int j0 = 0; j0 < npairs; j0 += 64) {
    const int jl = min(j0 + lane, npairs - 1);
    const int lv = jobs[jl].dd != nullptr && jobs[jl].ds != nullptr;
    const float lw = jl < kk ? tok_w[jl] : (gated ? sh_scale[0] : 1.0f);
    for (int j1 = j0; j1 < min(j0 + 64, npairs); j1 += CH) {
      float v[CH];
#pragma unroll
      for (int u = 0; u < CH; u++) v[u] = yy[(long)min(j1 + u, npairs - 1) * H + r];
#pragma unroll
      for (int u = 0; u < CH; u++) {
        const int j = j1 + u;
        const int live = __builtin_amdgcn_readlane(lv, min(j - j0, 63));
        const float wj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(lw), min(j - j0, 63)));
        if (j < npairs && live) o = __fadd_rn(o, __fmul_rn(wj, v[u]));
      }
    }
  }
  if ((int)(blockIdx.x * 256 + threadIdx.x) >= H) return;
  if (accumulate) o = __fadd_rn(out[r], o);
  out[r] = o;
}

bool xdown2_ok(int npairs, size_t i, int H, int num_cu) {
  if (i != 2048 || H % 4 != 0 || num_cu <= 0 || npairs < 1 || npairs > XC1_MAXP) return false;
  const long U = (long)npairs * (H / 4), per = (U + num_cu - 1) / num_cu;
  // a workgroup's run spans at most two pairs; the fused combine's blocks: its counters, and the
  // blocks a workgroup can complete
  return per <= H / 4 && per <= XD2_MAXU && (H / 4 + XD2_TB - 1) / XD2_TB <= CNT_N && per / XD2_TB + 4 <= XD2_MAXB;
}

hipError_t launch_xdown2(const Ctx &c, const RbtExpertDev *down_job, const int *down_slot, int kk, const __bf16 *hp,
                         int I, int H, const float *tok_w, const float *sh_scale, int has_shared, int gated,
                         float *yy, float *out, bool accumulate, const uint8_t *sh_dd, const uint8_t *sh_ds) {
  const int npairs = kk + (has_shared ? 1 : 0);
  if (!xdown2_ok(npairs, (size_t)I, H, c.num_cu)) return hipErrorInvalidValue;
  const bool shf = has_shared && sh_dd != nullptr && sh_ds != nullptr;
  // phase events: the start at the down kernel's start, the end after the combine (the context is
  // the one the caller holds: per-kernel profiling files events under it)
  Ctx &m = const_cast<Ctx &>(c);
  const hipEvent_t ts = c.t_start, te = c.t_stop;
  m.t_stop = nullptr;
  if (XD2_FUSED && c.d_cnt) {
    m.t_stop = te;
    launch_k(c, k_xdown2<4, true>, dim3(c.num_cu), dim3(64 * XD2_NW), down_job, down_slot, npairs, hp, H, yy,
             shf ? sh_dd : nullptr, shf ? sh_ds : nullptr, kk, gated, tok_w, sh_scale, out, (int)accumulate, c.d_cnt);
    return hipGetLastError();
  }
  launch_k(c, k_xdown2<4, false>, dim3(c.num_cu), dim3(64 * XD2_NW), down_job, down_slot, npairs, hp, H, yy,
           shf ? sh_dd : nullptr, shf ? sh_ds : nullptr, kk, gated, tok_w, sh_scale, out, (int)accumulate,
           (unsigned *)nullptr);
  m.t_start = nullptr;
  launch_k(c, k_combine1, dim3((H + 255) / 256), dim3(256), (const float *)yy, down_job, kk, has_shared, gated, tok_w,
           sh_scale, H, out, (int)accumulate);
  m.t_start = ts;
  m.t_stop = te;
  if (te) {
    const hipError_t e = hipEventRecord(te, c.stream);
    if (e != hipSuccess) return e;
  }
  return hipGetLastError();
}

bool xdown1_ok(int npairs, size_t i) { return i == 2048 && npairs >= 1 && npairs <= XD1_NP; }

hipError_t launch_xdown1(const Ctx &c, const RbtExpertDev *down_job, const int *down_slot, int kk, const __bf16 *hp,
                         int I, int H, const float *tok_w, const float *sh_scale, int has_shared, int gated,
                         float *out, bool accumulate, const uint8_t *sh_dd,
                         const uint8_t *sh_ds) {
  const int grid = c.num_cu;
  if (!xdown1_ok(kk + (has_shared ? 1 : 0), I) || H % 4 != 0 || grid <= 0 || (H / 4 + grid - 1) / grid > XD1_TPW)
    return hipErrorInvalidValue;
  launch_k(c, k_xdown1<4>, dim3(grid), dim3(64 * XD1_NW), down_job, down_slot, kk, hp, H, tok_w, sh_scale,
           has_shared, gated, out, (int)accumulate, sh_dd, sh_ds);
  return hipGetLastError();
}

bool xgemm_ok(int kind, size_t d, size_t i, int S, int k, int has_shared) {
  if (kind != RBT_QT_MXFP4) return false;
  if ((d != 8192 && d != 7168) || i % 64 != 0) return false;  // gate/up: K = 512 * NCH
  if (i != 2048 || d % 16 != 0) return false;                 // down: K = 2048
  const long np = (long)S * k + (has_shared ? S : 0);
  return np <= XD_MAXP && S <= 16;
}

hipError_t launch_xgateup1(const Ctx &c, const RbtExpertDev *jobs, int npairs, const float *x, int K, int I,
                           __bf16 *hp) {
  if (npairs <= 0) return hipSuccess;
  if (I % 4 != 0 || (long)npairs * (I / 4) < 4L * c.num_cu) return hipErrorInvalidValue;
  const dim3 grid(c.num_cu);
  if (K == 8192)
    launch_k(c, k_xgateup1<16>, grid, dim3(256), jobs, npairs, x, I, hp);
  else if (K == 7168)
    launch_k(c, k_xgateup1<14>, grid, dim3(256), jobs, npairs, x, I, hp);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_xgateup(const Ctx &c, const RbtExpertDev *jobs, const int *tok, int npairs, const float *x,
                          long x_stride, int K, int I, __bf16 *hp) {
  if (npairs <= 0) return hipSuccess;
  const dim3 grid(I / 64, npairs);
  if (K == 8192)
    launch_k(c, k_xgateup<16>, grid, dim3(256), jobs, tok, x, x_stride, I, hp);
  else if (K == 7168)
    launch_k(c, k_xgateup<14>, grid, dim3(256), jobs, tok, x, x_stride, I, hp);
  else
    return hipErrorInvalidValue;
  return hipGetLastError();
}

hipError_t launch_xdown(const Ctx &c, const RbtExpertDev *jobs, int npairs, const __bf16 *hp, int I, int H, int S,
                        int k, const int *tok, const int *tok_pair, const float *tok_w, const float *sh_scale,
                        int has_shared, int gated, float *out) {
  if (npairs <= 0 || npairs > XD_MAXP || I != 2048 || S > 16) return hipErrorInvalidValue;
  launch_k(c, k_xdown<4>, dim3(H / 16), dim3(256), jobs, npairs, hp, I, H, S, k, tok, tok_pair,
                     tok_w, sh_scale, has_shared, gated, out);
  return hipGetLastError();
}

}  // namespace rbt
