// prefill.hip -- MoE-layer prefill (many tokens per call) on the matrix cores, MXFP4 experts.
//
// The reference runs a prefill layer as apply_single_expert per unique expert (glm52/moe.rs:453-513,
// called in unique_experts order by qwen38/generate.rs:327-342): gather the expert's tokens, three
// matmul_mxfp4 calls with s = the expert's token count (kernels.rs:233), SiLU * up, and
// out[t] += w * y. Here the same products run as grouped GEMMs over every expert of the call:
//
//   k_pgroup   token -> expert grouping: one segment per unique expert in first-occurrence order
//              (unique_experts, glm52/moe.rs:333-344), its tokens in token order (the reference's
//              gather order, glm52/moe.rs:465-470), the shared expert as the last segment (all S
//              tokens); a tile table cuts segments into chunks of PF_TCH tokens.
//   k_to_bf16  x (fp32) -> bf16, the MFMA operand.
//   k_pgateup  per (tile, 64-row block): h = silu(gate . x) * (up . x) as bf16.
//   k_pdown    per (tile, 64-row block): y = down . h, fp32, one row per (expert, token) pair.
//   k_combine  (router.hip) out[t] = sum over t's picks in unique_experts order of w * y, then
//              + the shared expert's y (gated for Qwen), each product and sum rounded separately.
//
// GEMM tiling (v_mfma_f32_16x16x32_bf16, D[16x16] += A[16x32] . B[32x16]): A rows are 16 weight
// rows, B columns are 16 tokens. Lane l (r = l % 16, g = l / 16) loads 16 bytes = 32 E2M1 codes
// of weight row r at columns 128 s + 32 g .. +31 of step s: exactly one 32-element MXFP4 block, so
// one E8M0 byte scales them all. v_cvt_scalef32_pk_bf16_fp4 turns the codes into bf16 with the
// block scale applied (e2m1 * 2^(b-127) has two significant bits, so the bf16 value is the
// reference's dequantized weight, quant.rs:325-339, whenever it is a normal number). The four
// MFMAs of a step use the codes' four dwords; MFMA m covers columns 128 s + 32 g + 8 m .. +7 in
// lane group g, so the B lane (token r, group g) supplies the same 8 columns of its token's row.
// Lane l receives D[4 g + i][r]: rows 4g..4g+3 of the wave's 16 for token r.
//
// Weights stream from HBM once per tile (non-temporal loads); the activations (x or h, bf16) are
// small and stay in the caches across the row blocks of a tile.
#include "rbt_device.h"
#include "rbt_internal.h"

namespace rbt {

typedef __bf16 pb8 __attribute__((ext_vector_type(8)));
typedef __bf16 pb4 __attribute__((ext_vector_type(4)));
typedef __bf16 pb2 __attribute__((ext_vector_type(2)));
typedef float pf4 __attribute__((ext_vector_type(4)));

// ------------------------------------------------------------------------------------------------
// grouping
// ------------------------------------------------------------------------------------------------
__device__ __forceinline__ unsigned long long pg_lanemask_lt() {
  const int lane = threadIdx.x & 63;
  return (lane == 0) ? 0ull : (~0ull >> (64 - lane));
}

// Exclusive prefix sum over the 1024 threads of the block; *total gets the sum. `ws` holds 17 ints.
__device__ int pg_block_scan(int v, int *ws, int *total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int incl = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int o = __shfl_up(incl, d, 64);
    if (lane >= d) incl += o;
  }
  if (lane == 63) ws[wave] = incl;
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int i = 0; i < 16; i++) {
      const int c = ws[i];
      ws[i] = run;
      run += c;
    }
    ws[16] = run;
  }
  __syncthreads();
  const int r = ws[wave] + incl - v;
  *total = ws[16];
  __syncthreads();
  return r;
}

__device__ __forceinline__ uint32_t pg_load(const uint32_t *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One workgroup of 1024 threads. ids / wts are [S, k] (id -1 = no pick). bits / pc are scratch of
// E * ceil(S/32) words each. Outputs:
//   segs[u]     u < U: unique expert u (first-occurrence order), its pair offset and token count;
//               u = U (has_shared): the shared expert, pairs [S*k, S*k + S), all tokens.
//   tiles[i]    (segment, first token of the chunk of at most tch tokens), *ntiles = count.
//   pair_tok[p] token of pair p; routed pairs are [0, n_routed) in segment order, tokens
//               ascending within a segment; the shared pair of token t is S*k + t.
//   tok_pair / tok_w [t*k + j]: token t's pairs and routing weights sorted by pair index, i.e. in
//               unique_experts order (-1 / 0 for missing picks, placed last).
// SMALL (E * ceil(S / 32) <= PG_SMALLW): the token bitmaps and their prefix counts live in LDS
// (bits / pc unused); otherwise in the global scratch.
constexpr int PG_SMALLW = 8192;  // words: C4 (512 experts x 512 tokens) keeps its bitmaps in LDS
template <bool SMALL>
__global__ __launch_bounds__(1024) void k_pgroup(const int32_t *__restrict__ ids, const float *__restrict__ wts, int S,
                                                 int k, int E, int has_shared, const RbtExpertDev *__restrict__ table,
                                                 uint32_t *__restrict__ gbits, uint32_t *__restrict__ gpc,
                                                 PSeg *__restrict__ segs, PTile *__restrict__ tiles,
                                                 int *__restrict__ ntiles, int *__restrict__ pair_tok,
                                                 int *__restrict__ tok_pair, float *__restrict__ tok_w,
                                                 int *__restrict__ err, int *__restrict__ nuniq, int tch) {
  __shared__ int first[PG_MAXE], cnt[PG_MAXE], rank[PG_MAXE], byrank[PG_MAXE], segoff[PG_MAXE + 1];
  __shared__ uint32_t lbits[SMALL ? PG_SMALLW : 1], lpc[SMALL ? PG_SMALLW : 1];
  __shared__ int ws[17];
  __shared__ int carry_s;
  uint32_t *bits = SMALL ? lbits : gbits, *pc = SMALL ? lpc : gpc;
  auto bload = [&](const uint32_t *q) -> uint32_t { return SMALL ? *q : pg_load(q); };
  const int tid = threadIdx.x;
  const int W = (S + 31) >> 5;
  const int P = S * k;
  for (int e = tid; e < E; e += 1024) {
    first[e] = 0x7fffffff;
    cnt[e] = 0;
  }
  for (long i = tid; i < (long)E * W; i += 1024) bits[i] = 0u;
  if (!SMALL) __threadfence();
  __syncthreads();
  // counts, first occurrences, token bitmaps
  for (int p = tid; p < P; p += 1024) {
    const int e = ids[p];
    if (e >= 0 && e < E) {
      const int t = p / k;
      atomicAdd(&cnt[e], 1);
      atomicMin(&first[e], p);
      atomicOr(&bits[(long)e * W + (t >> 5)], 1u << (t & 31));
      const RbtExpertDev J = table[e];
      if (J.gd == nullptr || J.ud == nullptr || J.dd == nullptr) atomicOr(err, 1);
    }
  }
  if (!SMALL) __threadfence();
  __syncthreads();
  // rank of each used expert: the number of first occurrences before its own
  if (tid == 0) carry_s = 0;
  __syncthreads();
  for (int base = 0; base < P; base += 1024) {
    const int p = base + tid;
    int e = -1;
    bool fl = false;
    if (p < P) {
      e = ids[p];
      fl = e >= 0 && e < E && first[e] == p;
    }
    int tot;
    const int ex = pg_block_scan(fl ? 1 : 0, ws, &tot);
    const int c0 = carry_s;
    if (fl) {
      rank[e] = c0 + ex;
      byrank[c0 + ex] = e;
    }
    __syncthreads();
    if (tid == 0) carry_s = c0 + tot;
    __syncthreads();
  }
  const int U = carry_s;
  // segment offsets in rank order (two ranks per thread)
  {
    const int u0 = 2 * tid, u1 = 2 * tid + 1;
    const int c0 = u0 < U ? cnt[byrank[u0]] : 0, c1 = u1 < U ? cnt[byrank[u1]] : 0;
    int tot;
    const int ex = pg_block_scan(c0 + c1, ws, &tot);
    if (u0 < U) segoff[u0] = ex;
    if (u1 < U) segoff[u1] = ex + c0;
    if (tid == 0) segoff[U] = tot;
  }
  __syncthreads();
  // segments and tiles
  {
    const int nseg = U + (has_shared ? 1 : 0);
    const int u0 = 2 * tid, u1 = 2 * tid + 1;
    auto seg_cnt = [&](int u) { return u < U ? cnt[byrank[u]] : S; };
    const int n0 = u0 < nseg ? (seg_cnt(u0) + tch - 1) / tch : 0;
    const int n1 = u1 < nseg ? (seg_cnt(u1) + tch - 1) / tch : 0;
    int tot;
    const int ex = pg_block_scan(n0 + n1, ws, &tot);
    if (u0 < nseg) {
      segs[u0] = PSeg{u0 < U ? byrank[u0] : -1, u0 < U ? segoff[u0] : P, seg_cnt(u0), 0};
      for (int c = 0; c < n0; c++) tiles[ex + c] = PTile{u0, c * tch};
    }
    if (u1 < nseg) {
      segs[u1] = PSeg{u1 < U ? byrank[u1] : -1, u1 < U ? segoff[u1] : P, seg_cnt(u1), 0};
      for (int c = 0; c < n1; c++) tiles[ex + n0 + c] = PTile{u1, c * tch};
    }
    if (tid == 0) {
      *ntiles = tot;
      if (nuniq) *nuniq = U;
    }
  }
  // per-expert prefix counts of the token bitmap words
  for (int e = tid; e < E; e += 1024) {
    if (cnt[e] == 0) continue;
    uint32_t run = 0;
    for (int w = 0; w < W; w++) {
      pc[(long)e * W + w] = run;
      run += __popc(bload(&bits[(long)e * W + w]));
    }
  }
  if (!SMALL) __threadfence();
  __syncthreads();
  // Pairs, one thread per (token, pick). The slot of (t, e) within e's segment is the number of
  // earlier tokens that picked e. Token t's picks are written in pair order, which is
  // unique_experts order (segments are in rank order): pick j goes to position
  // #{j' : key(j') < key(j)}, with key = rank of the expert, and missing picks after every real one
  // in slot order.
  for (int p = tid; p < P; p += 1024) {
    const int t = p / k, j = p - t * k;
    const int32_t *ti = ids + (long)t * k;
    const int e = ti[j];
    const bool v = e >= 0 && e < E;
    const int kj = v ? rank[e] : E + j;
    int pos = 0;
    for (int j2 = 0; j2 < k; j2++) {
      const int e2 = ti[j2];
      pos += ((e2 >= 0 && e2 < E) ? rank[e2] : E + j2) < kj;
    }
    int pr = -1;
    if (v) {
      const long wi = (long)e * W + (t >> 5);
      const int slot = (int)(bload(&pc[wi]) + __popc(bload(&bits[wi]) & ((1u << (t & 31)) - 1u)));
      pr = segoff[rank[e]] + slot;
      pair_tok[pr] = t;
    }
    tok_pair[(long)t * k + pos] = pr;
    tok_w[(long)t * k + pos] = v ? wts[(long)t * k + j] : 0.0f;
    if (has_shared && j == 0) pair_tok[P + t] = t;
  }
}

// x (fp32) -> bf16, round to nearest even. vec: x and xb allow 16- and 8-byte accesses.
__global__ __launch_bounds__(256) void k_to_bf16(const float *__restrict__ x, long n, __bf16 *__restrict__ xb,
                                                 int vec) {
  const long i = 4 * ((long)blockIdx.x * 256 + threadIdx.x);
  if (vec && i + 3 < n) {
    const float4 v = *reinterpret_cast<const float4 *>(x + i);
    *reinterpret_cast<pb4 *>(xb + i) = pb4{(__bf16)v.x, (__bf16)v.y, (__bf16)v.z, (__bf16)v.w};
  } else {
    for (long j = i; j < min(n, i + 4); j++) xb[j] = (__bf16)x[j];
  }
}

// ------------------------------------------------------------------------------------------------
// grouped GEMMs
// ------------------------------------------------------------------------------------------------
// 8 E2M1 codes (one dword) -> 8 bf16 scaled by the block's E8M0 value.
__device__ __forceinline__ pb8 pf_fp4x8(uint32_t w, float sc) {
  const pb2 a = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 0);
  const pb2 b = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 1);
  const pb2 c = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 2);
  const pb2 d = __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w, sc, 3);
  return pb8{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

// E8M0 byte -> f32 scale (e8m0_decode, quant.rs:391-396): byte 0 is 2^-127, 255 the +inf bits.
__device__ __forceinline__ float pf_e8m0(uint32_t b) { return __uint_as_float(b == 0 ? (1u << 22) : (b << 23)); }

// Tile decode shared by both GEMMs.
struct PfTile {
  RbtExpertDev J;
  int pbase;  // first pair of the tile
  int M;      // tokens in the tile (1..PF_TCH)
  bool ok;
};

__device__ __forceinline__ PfTile pf_tile(int ti, const PTile *__restrict__ tiles, const PSeg *__restrict__ segs,
                                          const RbtExpertDev *__restrict__ table,
                                          const RbtExpertDev *__restrict__ shared_dev, int tch = PF_TCH) {
  PfTile r;
  const PTile T = tiles[ti];
  const PSeg G = segs[T.seg];
  r.J = G.eid >= 0 ? table[G.eid] : *shared_dev;
  r.pbase = G.off + T.c0;
  r.M = min(tch, G.cnt - T.c0);
  // a missing expert is reported by k_pgroup (error flag); its tiles compute nothing
  r.ok = r.M > 0 && r.J.gd != nullptr && r.J.ud != nullptr && r.J.dd != nullptr;
  return r;
}

// A operand of one K step: the lane's 32 codes (16 bytes) and the scale dword holding its block's
// E8M0 byte (byte g of the dword at 4 * step).
struct PfA {
  rbt_u4 w;
  uint32_t s;
};

__device__ __forceinline__ void pf_load_a(PfA &a, const uint8_t *row, const uint8_t *srow, int s) {
  a.w = __builtin_nontemporal_load((const rbt_gu4 *)(row + 64 * s));
  a.s = *(const rbt_gu32 *)(srow + 4 * s);
}

__device__ __forceinline__ void pf_decode(const PfA &a, int g, pb8 (&A)[4]) {
  const float sc = pf_e8m0((a.s >> (8 * g)) & 0xffu);
  A[0] = pf_fp4x8(a.w.x, sc);
  A[1] = pf_fp4x8(a.w.y, sc);
  A[2] = pf_fp4x8(a.w.z, sc);
  A[3] = pf_fp4x8(a.w.w, sc);
}

constexpr int PF_RBG = 8;         // workgroups per tile: each takes 1/8 of the rows (contiguous)
constexpr int PB_STRIDE = 128 + 8;  // bf16 per LDS token row of a step (272 B: rows 4 banks apart)

// The tile's activations for one K step (nt * 16 tokens x 128 columns, bf16) go through LDS: the
// workgroup loads them with one coalesced 16-byte load per thread per 16 tokens (a token's 256
// bytes are 16 consecutive lanes) and every wave reads its MFMA B operands from LDS. Thread t
// stages token 16 q + t / 16, bytes 16 (t % 16) .. +15 of the step.
//
// Load order and the in-order memory counter: a wave waits for a global load by waiting until at
// most N younger loads are outstanding, so every load it depends on must be as old as the weight
// loads of the same step. Iteration `it` therefore issues the weight loads for it + D and the
// activation loads for it + 1 + D together (register rings of depth D), and stores the activations
// of it + 1 (issued D iterations earlier) to the LDS buffer the next iteration reads.
template <int NTV>
struct PfStage {
  rbt_u4 v[NTV];
};

template <int NTV>
__device__ __forceinline__ void pf_stage_load(PfStage<NTV> &st, const __bf16 *const (&src)[NTV], int s) {
#pragma unroll
  for (int q = 0; q < NTV; q++) st.v[q] = *(const rbt_gu4 *)(src[q] + 128 * s);
}

template <int NTV>
__device__ __forceinline__ void pf_stage_store(const PfStage<NTV> &st, __bf16 (*buf)[PB_STRIDE]) {
  const int j = threadIdx.x >> 4, c = (threadIdx.x & 15) * 8;
#pragma unroll
  for (int q = 0; q < NTV; q++) *reinterpret_cast<rbt_u4 *>(&buf[16 * q + j][c]) = st.v[q];
}

// B operand of MFMA m for column block q: token 16 q + r, columns 32 g + 8 m .. +7 of the step.
__device__ __forceinline__ pb8 pf_b(const __bf16 (*buf)[PB_STRIDE], int q, int m, int r, int g) {
  return *reinterpret_cast<const pb8 *>(&buf[16 * q + r][32 * g + 8 * m]);
}

// Weight staging. An MFMA reads 16 rows x 64 bytes per K step, but streams of 16 rows x 64 bytes run
// at about two thirds of the bandwidth of 4 rows x 256 contiguous bytes on this part. So each
// wave loads its tiles' K groups (4 steps = 256 bytes per row) as 4 rows x 256 bytes per
// instruction (lane l: row 4 q + l / 16 of the 16-row tile, bytes 16 (l % 16) .. +15 of the group),
// writes them to its own LDS area at a PW_STRIDE-byte row stride, and every step reads the MFMA
// layout back (lane (r, g): row r, bytes 16 (4 d + g) .. +15 of step d). The 272-byte stride puts
// the 16 rows of a read 4 banks apart, and a wave reads its area only after its own writes, in
// order, so no barrier is needed.
constexpr int PW_STRIDE = 256 + 16;       // bytes per staged weight row (one K group)
constexpr int PW_TILE = 16 * PW_STRIDE;   // bytes per staged 16-row tile

// LDS of one pf_gemm workgroup: the activation double buffer (2 x 16 NTV token rows) then each
// wave's staged weights (NM TILES tiles).
constexpr int pf_lds_bytes(int NM, int NTV, int TILES) {
  return 2 * 16 * NTV * PB_STRIDE * 2 + 4 * NM * TILES * PW_TILE;
}

// One tile x row-block group. Wave w owns TILES 16-row tiles (16 TILES contiguous rows) of each
// of NM matrices per row block (gate/up: NM = 2, down: NM = 1); a row block is 64 TILES rows, and
// the workgroup walks `per` of them: blocks rb0, rb0 + rbs, rb0 + 2 rbs, ...
//
// The weights stream in groups of 4 K steps (512 columns): at the start of a group the wave writes
// the group loaded a group ago to its LDS area, then issues every load of the next group at once,
// the codes (4 per tile, see above) and, per 16-row tile, one 16-byte load of its 4 steps' E8M0
// bytes (byte 4 s + g of a row is the block of lane group g). The group in flight
// (NM * TILES * 4 KB per wave) covers the memory latency while the current group computes.
// NM = 2 writes hb = bf16(silu(g) * u), NM = 1 writes y (fp32).
//
// DEC (the grouped decode): a 16-column block holds five tokens' three bf16 activation parts
// (column 3 m + p: token 5 q + m, part p; column 15 unused), so the products are fp32-exact and the
// epilogue sums each token's three columns (lanes r0, r0 + 1, r0 + 2 of the row group) before the
// activation: NM = 2 writes h as three bf16 parts (rows 3 pair + part of hb), NM = 1 writes y.
// rbs: row blocks between a workgroup's consecutive blocks (PF_RBG for prefill, 1 for decode).
// lds: pf_lds_bytes(NM, NTV, TILES) bytes of LDS.
template <int NM, int NTV, int TILES, bool DEC = false, bool SL = false>
__device__ __forceinline__ void pf_gemm(const PfTile &T, const __bf16 *const (&src)[NTV], const uint8_t *const (&a)[NM],
                                        const uint8_t *const (&sc)[NM], long rowb, long rows, int rb0, int per,
                                        int nsteps, int out_cols, __bf16 *__restrict__ hb, float *__restrict__ y,
                                        uint8_t *lds, int rbs = PF_RBG) {
  constexpr int G = 4;  // K steps per group
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63, r = lane & 15, g = lane >> 4;
  constexpr int BR = 64 * TILES;                                         // rows per row block
  const long blk_a = (long)rbs * BR * rowb, blk_s = (long)rbs * BR * rows;  // between own blocks
  const int total = per * nsteps;
  if (total <= 0) return;  // no row block for this workgroup (uniform)
  __bf16(*bs)[16 * NTV][PB_STRIDE] = reinterpret_cast<__bf16(*)[16 * NTV][PB_STRIDE]>(lds);
  uint8_t *const wl = lds + 2 * 16 * NTV * PB_STRIDE * 2 + w * (NM * TILES * PW_TILE);  // this wave's area
  const uint8_t *pa[NM][TILES], *ps[NM][TILES], *pl[NM][TILES];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int t = 0; t < TILES; t++) {
      const long row0 = (long)rb0 * BR + 16 * TILES * w + 16 * t;  // first row of the tile
      pa[m][t] = a[m] + (row0 + (lane >> 4)) * rowb + 16 * (lane & 15);
      ps[m][t] = sc[m] + (row0 + r) * rows;
      pl[m][t] = sc[m] + (row0 + (lane >> 2)) * rows + 16 * (lane & 3);
    }
  // Scale lines: a row's E8M0 bytes for four groups (2048 columns) are 64 contiguous bytes. One
  // 16-byte load per lane and tile (row lane / 4, bytes 16 (lane % 4) .. +15 of the line) reads the
  // tile's 16 rows x 64 bytes at once, and each group's 16 bytes reach their MFMA lanes by shuffles.
  // Loading each group's 16 bytes of a row on its own touches every line four times, a group apart.
  const int nlines = nsteps / (4 * G);  // lines per row of a row block
  const bool sline = SL && nsteps % (4 * G) == 0 && rows == 64 * nlines;  // SL: the down GEMMs (the gate/up ones
  // have no registers to spare at their occupancy)
  rbt_u4 sl[NM][TILES];
  auto sl_load = [&](int rb, int j) {
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int t = 0; t < TILES; t++) sl[m][t] = *(const rbt_gu4 *)(pl[m][t] + (long)rb * blk_s + 64 * j);
  };
  // next group to fetch (past the end: the last group again, never used)
  int f_rb = 0, f_s = 0;
  rbt_u4 nw[NM][TILES][4], ns[NM][TILES];
  auto fetch_group = [&]() {
    const int rb = min(f_rb, per - 1);
    const int st = f_rb < per ? f_s : nsteps - G;
    const long oa = (long)rb * blk_a + 64 * st, os = (long)rb * blk_s + 4 * st;
#pragma unroll
    for (int q = 0; q < 4; q++)
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int t = 0; t < TILES; t++)
          nw[m][t][q] = __builtin_nontemporal_load((const rbt_gu4 *)(pa[m][t] + oa + 4 * q * rowb));
    if (!sline) {
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int t = 0; t < TILES; t++) ns[m][t] = *(const rbt_gu4 *)(ps[m][t] + os);
    }
    f_s += G;
    if (f_s == nsteps) {
      f_s = 0;
      ++f_rb;
    }
  };
  // activation stage ring: slot (it + 1) % G holds the activations of iteration it + 1, loaded in
  // the same group batch as the weights it is used with
  PfStage<NTV> st[G];
  int a_s = 1 % nsteps;
  int a_n = 1;
  auto stage_next = [&](PfStage<NTV> &dst) {
    pf_stage_load<NTV>(dst, src, a_n < total ? a_s : 0);
    if (++a_s == nsteps) a_s = 0;
    ++a_n;
  };
  {
    PfStage<NTV> s0;
    pf_stage_load<NTV>(s0, src, 0);
#pragma unroll
    for (int d = 0; d < G; d++) stage_next(st[(d + 1) % G]);
    if (sline) sl_load(0, 0);
    fetch_group();
    pf_stage_store<NTV>(s0, bs[0]);
  }
  __syncthreads();
  pf4 acc[NM][TILES][NTV];
#pragma unroll
  for (int m = 0; m < NM; m++)
#pragma unroll
    for (int t = 0; t < TILES; t++)
#pragma unroll
      for (int q = 0; q < NTV; q++) acc[m][t][q] = pf4{0.f, 0.f, 0.f, 0.f};
  int c_rb = 0, c_s = 0;  // group being computed
  for (int it0 = 0; it0 < total; it0 += G) {
    rbt_u4 cs[NM][TILES];
    if (sline) {
      // this group's 16 bytes of row r: lane 4 r + group holds them; the next row block's line
      // goes out once the last group's bytes are taken
      const int gq = c_s / G, src = 4 * r + (gq & 3);
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int t = 0; t < TILES; t++)
          cs[m][t] = rbt_u4{(uint32_t)__shfl((int)sl[m][t].x, src, 64), (uint32_t)__shfl((int)sl[m][t].y, src, 64),
                            (uint32_t)__shfl((int)sl[m][t].z, src, 64), (uint32_t)__shfl((int)sl[m][t].w, src, 64)};
      if ((gq & 3) == 3) {
        const int j = (gq >> 2) + 1;
        if (j < nlines)
          sl_load(c_rb, j);
        else if (c_rb + 1 < per)
          sl_load(c_rb + 1, 0);
      }
    }
    // the group loaded a group ago -> this wave's LDS area (rows at PW_STRIDE)
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int t = 0; t < TILES; t++) {
        if (!sline) cs[m][t] = ns[m][t];
        uint8_t *wt = wl + (m * TILES + t) * PW_TILE + (lane >> 4) * PW_STRIDE + 16 * (lane & 15);
#pragma unroll
        for (int q = 0; q < 4; q++) *reinterpret_cast<rbt_u4 *>(wt + 4 * q * PW_STRIDE) = nw[m][t][q];
      }
    fetch_group();
#pragma unroll
    for (int d = 0; d < G; d++) {
      const int buf = d & 1;  // iteration it reads LDS buffer it & 1 (nsteps even)
      // activations of it + 1 (loaded a group ago) -> the other LDS buffer
      pf_stage_store<NTV>(st[(d + 1) % G], bs[buf ^ 1]);
      stage_next(st[(d + 1) % G]);
      rbt_u4 cw[NM][TILES];
#pragma unroll
      for (int m = 0; m < NM; m++)
#pragma unroll
        for (int t = 0; t < TILES; t++)
          cw[m][t] = *reinterpret_cast<const rbt_u4 *>(wl + (m * TILES + t) * PW_TILE + r * PW_STRIDE + 16 * (4 * d + g));
#pragma unroll
      for (int k4 = 0; k4 < 4; k4++) {
        pb8 bv[NTV];
#pragma unroll
        for (int q = 0; q < NTV; q++) bv[q] = pf_b(bs[buf], q, k4, r, g);
#pragma unroll
        for (int m = 0; m < NM; m++)
#pragma unroll
          for (int t = 0; t < TILES; t++) {
            const rbt_u4 sv = cs[m][t];
            const uint32_t sw = d == 0 ? sv.x : d == 1 ? sv.y : d == 2 ? sv.z : sv.w;
            const float scl = pf_e8m0((sw >> (8 * g)) & 0xffu);
            const rbt_u4 c = cw[m][t];
            const uint32_t code = k4 == 0 ? c.x : k4 == 1 ? c.y : k4 == 2 ? c.z : c.w;
            const pb8 av = pf_fp4x8(code, scl);
#pragma unroll
            for (int q = 0; q < NTV; q++)
              acc[m][t][q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(av, bv[q], acc[m][t][q], 0, 0, 0);
          }
      }
      __syncthreads();
    }
    c_s += G;
    if (!DEC && NM == 1 && c_s == nsteps) {
      // down, row block done: y leaves in whole cache lines, non-temporal. The wave's 16 NTV tokens x
      // 16 TILES rows go through its LDS area (idle until the next group's write, which follows in
      // program order) token-major, then each token's rows are stored as one contiguous run (256
      // bytes at TILES = 4) instead of 64-byte pieces of 16 rows 32 KB apart. Stores share the
      // in-order vector memory counter with the weight loads, so their acknowledgements delay the
      // waits that follow them; streaming stores and one row block per workgroup (PF_DN_RBG) keep that
      // cost down (k_pdown at C4: 1041 -> 980 us; without any y store it runs in 863 us).
      constexpr int RW = 16 * TILES, CPT = RW / 4;  // rows per token run, 16-byte chunks in it
      constexpr int YS = 16 * NTV * (RW * 4 + 16) <= NM * TILES * PW_TILE ? RW * 4 + 16 : RW * 4;
      static_assert(16 * NTV * YS <= NM * TILES * PW_TILE, "staged y fits the wave's area");
#pragma unroll
      for (int t = 0; t < TILES; t++)
#pragma unroll
        for (int q = 0; q < NTV; q++) {
          *reinterpret_cast<pf4 *>(wl + (16 * q + r) * YS + (16 * t + 4 * g) * 4) = acc[0][t][q];
          acc[0][t][q] = pf4{0.f, 0.f, 0.f, 0.f};
        }
      const long row0 = (long)(rb0 + rbs * c_rb) * BR + 16 * TILES * w;
#pragma unroll
      for (int k = 0; k < NTV * CPT / 4; k++) {
        const int c = lane + 64 * k, tok = c / CPT, ch = c - tok * CPT;
        const pf4 v = *reinterpret_cast<const pf4 *>(wl + tok * YS + 16 * ch);
        if (tok < T.M) __builtin_nontemporal_store(v, reinterpret_cast<pf4 *>(y + (long)(T.pbase + tok) * out_cols + row0 + 4 * ch));
      }
      c_s = 0;
      ++c_rb;
    } else if (c_s == nsteps) {  // row block done (wave-uniform)
#pragma unroll
      for (int t = 0; t < TILES; t++) {
        const int orow = (rb0 + rbs * c_rb) * BR + 16 * TILES * w + 16 * t + 4 * g;
#pragma unroll
        for (int q = 0; q < NTV; q++) {
          const int j = 16 * q + r;
          if (DEC) {
            // token 5 q + r / 3 on lanes r = 0, 3, .., 12: its parts hi + mid + lo, in that order
            pf4 sum[NM];
#pragma unroll
            for (int m = 0; m < NM; m++)
#pragma unroll
              for (int i = 0; i < 4; i++) {
                const float v0 = acc[m][t][q][i];
                const float v1 = __shfl_down(v0, 1, 16), v2 = __shfl_down(v0, 2, 16);
                sum[m][i] = __fadd_rn(__fadd_rn(v0, v1), v2);
              }
            const int tl = 5 * q + r / 3;
            if (r % 3 == 0 && r < 15 && tl < T.M) {
              const long pr = T.pbase + tl;
              if (NM == 2) {
                pb4 hp[3];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                  const float hv = __fmul_rn(rbt_silu(sum[0][i]), sum[NM - 1][i]);
                  const __bf16 hh = (__bf16)hv;
                  const float r1 = __fsub_rn(hv, (float)hh);
                  const __bf16 mm = (__bf16)r1;
                  hp[0][i] = hh;
                  hp[1][i] = mm;
                  hp[2][i] = (__bf16)__fsub_rn(r1, (float)mm);
                }
#pragma unroll
                for (int p = 0; p < 3; p++)
                  *reinterpret_cast<pb4 *>(hb + (pr * 3 + p) * out_cols + orow) = hp[p];
              } else {
                *reinterpret_cast<float4 *>(y + pr * out_cols + orow) =
                    float4{sum[0][0], sum[0][1], sum[0][2], sum[0][3]};
              }
            }
          } else if (j < T.M) {
            if (NM == 2) {
              pb4 hv;
#pragma unroll
              for (int i = 0; i < 4; i++) hv[i] = (__bf16)(rbt_silu(acc[0][t][q][i]) * acc[NM - 1][t][q][i]);
              *reinterpret_cast<pb4 *>(hb + (long)(T.pbase + j) * out_cols + orow) = hv;
            } else {
              *reinterpret_cast<float4 *>(y + (long)(T.pbase + j) * out_cols + orow) =
                  float4{acc[0][t][q][0], acc[0][t][q][1], acc[0][t][q][2], acc[0][t][q][3]};
            }
          }
#pragma unroll
          for (int m = 0; m < NM; m++) acc[m][t][q] = pf4{0.f, 0.f, 0.f, 0.f};
        }
      }
      c_s = 0;
      ++c_rb;
    }
  }
}

// Gate/up: grid = ntiles_max * PF_RBG workgroups of 256 threads; workgroup (tile, gi) owns rows
// [gi * I / PF_RBG, (gi + 1) * I / PF_RBG) of gate and of up for the tile's tokens, over all H
// columns. Output hb[pair, I] = bf16(silu(g) * u) (glm52/moe.rs:33-80 Activation::Silu).
constexpr int PF_GU_LDS = pf_lds_bytes(2, 1, 2) > pf_lds_bytes(2, 4, 1) ? pf_lds_bytes(2, 1, 2) : pf_lds_bytes(2, 4, 1);
constexpr int PF_DN_LDS = pf_lds_bytes(1, 1, 4) > pf_lds_bytes(1, 4, 1) ? pf_lds_bytes(1, 1, 4) : pf_lds_bytes(1, 4, 1);
static_assert(pf_lds_bytes(2, 2, 1) <= PF_GU_LDS && pf_lds_bytes(1, 2, 2) <= PF_DN_LDS, "LDS sizes");
static_assert(2 * PF_GU_LDS <= 160 * 1024 && 2 * PF_DN_LDS <= 160 * 1024, "two workgroups per CU");

// Workgroup -> (tile, row-block group): the RBG workgroups of a tile are consecutive dispatch
// slots of one XCD (workgroups are dealt to the eight XCDs round robin), so the tile's
// activations come into that XCD's L2 once and its RBG x per row blocks re-read them there.
// The grid is a multiple of 8 RBG workgroups.
template <int RBG = PF_RBG>
__device__ __forceinline__ void pf_tile_of_block(int &ti, int &gi) {
  const int xcd = blockIdx.x & 7, slot = blockIdx.x >> 3;
  gi = slot % RBG;
  ti = (slot / RBG) * 8 + xcd;
}
// Down: 32 workgroups per tile, so that at TILES = 4 (256-row blocks of 8192 rows) each takes one row
// block and its y stores are its last memory operations.
constexpr int PF_DN_RBG = 32;

__global__ __launch_bounds__(256) void k_pgateup(const PTile *__restrict__ tiles, const int *__restrict__ ntiles,
                                                 const PSeg *__restrict__ segs, const RbtExpertDev *__restrict__ table,
                                                 const RbtExpertDev *__restrict__ shared_dev,
                                                 const int *__restrict__ pair_tok, const __bf16 *__restrict__ xb,
                                                 int S, int H, int I, __bf16 *__restrict__ hb) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[PF_GU_LDS];
  int ti, gi;
  pf_tile_of_block(ti, gi);
  if (ti >= *ntiles) return;
  const PfTile T = pf_tile(ti, tiles, segs, table, shared_dev);
  if (!T.ok) return;
  const int nt = (T.M + 15) >> 4;
  const int nsteps = H >> 7;
  // row blocks of BR rows, dealt round-robin to the PF_RBG workgroups of the tile
  auto per_of = [&](int br) { return (I / br - gi + PF_RBG - 1) / PF_RBG; };
  const long rowb = (long)(H >> 1), rows = (long)(H >> 5);
  const uint8_t *const a[2] = {T.J.gd, T.J.ud};
  const uint8_t *const sc[2] = {(const uint8_t *)T.J.gs, (const uint8_t *)T.J.us};
  auto src_of = [&](int q) {
    const int tok = min(max(pair_tok[T.pbase + min(16 * q + (int)(threadIdx.x >> 4), T.M - 1)], 0), S - 1);
    return xb + (long)tok * H + (threadIdx.x & 15) * 8;
  };
  switch (nt) {
    case 1: {
      const __bf16 *src[1] = {src_of(0)};
      pf_gemm<2, 1, 2>(T, src, a, sc, rowb, rows, gi, per_of(128), nsteps, I, hb, nullptr, lds);
    } break;
    case 2: {
      const __bf16 *src[2] = {src_of(0), src_of(1)};
      pf_gemm<2, 2, 1>(T, src, a, sc, rowb, rows, gi, per_of(64), nsteps, I, hb, nullptr, lds);
    } break;
    default: {
      const __bf16 *src[4] = {src_of(0), src_of(1), src_of(2), src_of(3)};
      pf_gemm<2, 4, 1>(T, src, a, sc, rowb, rows, gi, per_of(64), nsteps, I, hb, nullptr, lds);
    } break;
  }
}

// Down: grid = ntiles_max * PF_DN_RBG, 256 threads; workgroup (tile, gi) takes the tile's row blocks
// gi, gi + PF_DN_RBG, .. over all I columns; y[pair, H] fp32.
__global__ __launch_bounds__(256) void k_pdown(const PTile *__restrict__ tiles, const int *__restrict__ ntiles,
                                               const PSeg *__restrict__ segs, const RbtExpertDev *__restrict__ table,
                                               const RbtExpertDev *__restrict__ shared_dev,
                                               const __bf16 *__restrict__ hb, int I, int H, float *__restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[PF_DN_LDS];
  int ti, gi;
  pf_tile_of_block<PF_DN_RBG>(ti, gi);
  if (ti >= *ntiles) return;
  const PfTile T = pf_tile(ti, tiles, segs, table, shared_dev);
  if (!T.ok) return;
  const int nt = (T.M + 15) >> 4;
  const int nsteps = I >> 7;
  auto per_of = [&](int br) { return (H / br - gi + PF_DN_RBG - 1) / PF_DN_RBG; };
  const long rowb = (long)(I >> 1), rows = (long)(I >> 5);
  const uint8_t *const a[1] = {T.J.dd};
  const uint8_t *const sc[1] = {(const uint8_t *)T.J.ds};
  auto src_of = [&](int q) {
    return hb + (long)(T.pbase + min(16 * q + (int)(threadIdx.x >> 4), T.M - 1)) * I + (threadIdx.x & 15) * 8;
  };
  switch (nt) {
    case 1: {
      const __bf16 *src[1] = {src_of(0)};
      pf_gemm<1, 1, 4, false, true>(T, src, a, sc, rowb, rows, gi, per_of(256), nsteps, H, nullptr, y, lds, PF_DN_RBG);
    } break;
    case 2: {
      const __bf16 *src[2] = {src_of(0), src_of(1)};
      pf_gemm<1, 2, 2, false, true>(T, src, a, sc, rowb, rows, gi, per_of(128), nsteps, H, nullptr, y, lds, PF_DN_RBG);
    } break;
    default: {
      const __bf16 *src[4] = {src_of(0), src_of(1), src_of(2), src_of(3)};
      pf_gemm<1, 4, 1, false, true>(T, src, a, sc, rowb, rows, gi, per_of(64), nsteps, H, nullptr, y, lds, PF_DN_RBG);
    } break;
  }
}

// ------------------------------------------------------------------------------------------------
// grouped decode (a few tokens per call, fp32-accurate): the tile GEMMs above with each token's
// activation as three bf16 parts hi + mid + lo (split3: exact) in three MFMA columns, five tokens
// per 16-column block and two blocks per tile (PD_TCH = 10 tokens: the two-block GEMMs keep two
// workgroups per CU), summed in the epilogue. Every unique expert's
// weights stream once per call however many of the call's tokens picked it. The work is the
// (tile, row block) units of all tiles, dealt evenly over a fixed grid (the tile count is on the
// device), so a handful of experts still fills the chip.
// ------------------------------------------------------------------------------------------------
// x [S, H] fp32 -> xb3 [3 S, H] bf16: row 3 t + p is part p of token t.
__global__ __launch_bounds__(256) void k_split3(const float *__restrict__ x, int S, int H, __bf16 *__restrict__ xb3) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= (long)S * H) return;
  const long t = i / H, c = i - t * H;
  const float v = x[i];
  const __bf16 hh = (__bf16)v;
  const float r1 = __fsub_rn(v, (float)hh);
  const __bf16 mm = (__bf16)r1;
  xb3[(3 * t) * H + c] = hh;
  xb3[(3 * t + 1) * H + c] = mm;
  xb3[(3 * t + 2) * H + c] = (__bf16)__fsub_rn(r1, (float)mm);
}

// Row (token part) of virtual column jv of block q in a tile: token 5 q + jv / 3 (clamped to the
// tile), part jv % 3; column 15 repeats column 0 (its products are never read).
__device__ __forceinline__ void pd_col(int q, int jv, int M, int &tl, int &part) {
  if (jv >= 15) jv = 0;
  tl = min(5 * q + jv / 3, M - 1);
  part = jv % 3;
}

// Units u = tile * RB + row block over all tiles, workgroup b taking [b U / nwg, (b + 1) U / nwg):
// consecutive row blocks of one tile run as one pf_gemm call.
template <bool GATEUP>
__device__ __forceinline__ void pd_units(const PTile *__restrict__ tiles, const int *__restrict__ ntiles,
                                         const PSeg *__restrict__ segs, const RbtExpertDev *__restrict__ table,
                                         const RbtExpertDev *__restrict__ shared_dev,
                                         const int *__restrict__ pair_tok, const __bf16 *__restrict__ src_rows,
                                         int S, int K, int O, int RB, __bf16 *__restrict__ hb3, float *__restrict__ y,
                                         uint8_t *lds) {
  constexpr int TILES = GATEUP ? 1 : 2;
  const int U = *ntiles * RB, nwg = gridDim.x, b = blockIdx.x;
  const int u0 = (int)((long)b * U / nwg), u1 = (int)((long)(b + 1) * U / nwg);
  const long rowb = K >> 1, rows = K >> 5;
  const int nsteps = K >> 7;
  const int jv = threadIdx.x >> 4;
  for (int u = u0; u < u1;) {
    const int ti = u / RB, rb0 = u - ti * RB, per = min(u1 - u, RB - rb0);
    u += per;
    const PfTile T = pf_tile(ti, tiles, segs, table, shared_dev, PD_TCH);
    if (!T.ok) continue;  // a missing expert is reported by k_pgroup; its rows compute nothing
    const int nt = (T.M + 4) / 5;
    auto src_of = [&](int q) {
      int tl, part;
      pd_col(q, jv, T.M, tl, part);
      long row;
      if (GATEUP) {
        const int tok = min(max(pair_tok[T.pbase + tl], 0), S - 1);
        row = 3L * tok + part;
      } else {
        row = 3L * (T.pbase + tl) + part;
      }
      return src_rows + row * K + (threadIdx.x & 15) * 8;
    };
    const uint8_t *const ga[2] = {T.J.gd, T.J.ud};
    const uint8_t *const gs[2] = {(const uint8_t *)T.J.gs, (const uint8_t *)T.J.us};
    const uint8_t *const da[1] = {T.J.dd};
    const uint8_t *const ds[1] = {(const uint8_t *)T.J.ds};
#define RBT_PD(NTV_)                                                                                          \
  {                                                                                                           \
    const __bf16 *src[NTV_];                                                                                  \
    for (int q = 0; q < NTV_; q++) src[q] = src_of(q);                                                        \
    if (GATEUP)                                                                                               \
      pf_gemm<2, NTV_, TILES, true>(T, src, ga, gs, rowb, rows, rb0, per, nsteps, O, hb3, nullptr, lds, 1);   \
    else                                                                                                      \
      pf_gemm<1, NTV_, TILES, true, true>(T, src, da, ds, rowb, rows, rb0, per, nsteps, O, nullptr, y, lds, 1);     \
  }
    if (nt == 1)
      RBT_PD(1)
    else
      RBT_PD(2)
#undef RBT_PD
    __syncthreads();  // the next tile's first activation step reuses the LDS buffers
  }
}

// Gate/up: hb3 [3 pairs, I] bf16 (h parts). Row blocks of 64 rows (RB = I / 64). Three workgroups
// per CU (52 KB of LDS, four waves each): a workgroup keeps one K group of its rows in flight, so
// the chip's loads in flight grow with the workgroups per CU (C3: 90 -> 79 us per call against one
// per CU; two per CU balance no better than one).
__global__ __launch_bounds__(256) void k_dgateup(const PTile *__restrict__ tiles, const int *__restrict__ ntiles,
                                                 const PSeg *__restrict__ segs, const RbtExpertDev *__restrict__ table,
                                                 const RbtExpertDev *__restrict__ shared_dev,
                                                 const int *__restrict__ pair_tok, const __bf16 *__restrict__ xb3,
                                                 int S, int H, int I, __bf16 *__restrict__ hb3) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[pf_lds_bytes(2, 2, 1)];
  pd_units<true>(tiles, ntiles, segs, table, shared_dev, pair_tok, xb3, S, H, I, I / 64, hb3, nullptr, lds);
}

// Down: y [pairs, H] fp32. Row blocks of 128 rows (RB = H / 128).
__global__ __launch_bounds__(256) void k_ddown(const PTile *__restrict__ tiles, const int *__restrict__ ntiles,
                                               const PSeg *__restrict__ segs, const RbtExpertDev *__restrict__ table,
                                               const RbtExpertDev *__restrict__ shared_dev,
                                               const __bf16 *__restrict__ hb3, int I, int H, float *__restrict__ y) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[pf_lds_bytes(1, 2, 2)];
  pd_units<false>(tiles, ntiles, segs, table, shared_dev, nullptr, hb3, 0, I, H, H / 128, nullptr, y, lds);
}

// ------------------------------------------------------------------------------------------------
// launchers
// ------------------------------------------------------------------------------------------------
bool prefill_ok(int kind, size_t d, size_t i, size_t n_experts, size_t k) {
  if (kind != RBT_QT_MXFP4) return false;
  // K steps of 128 columns (gate/up: 4 in flight, down: 8), PF_RBG groups of 64-row blocks
  if (d % 512 != 0 || i % 1024 != 0 || d > (1u << 20) || i > (1u << 20)) return false;
  // segments: every expert plus the shared one within PG_MAXE
  return n_experts + 1 <= (size_t)PG_MAXE && k <= 64;
}

long prefill_max_tiles(int S, int k, int E, int has_shared) {
  const long P = (long)S * k;
  const long nseg = std::min<long>(E, P) + (has_shared ? 1 : 0);
  return nseg + (P + (has_shared ? S : 0) + PF_TCH - 1) / PF_TCH;
}

hipError_t launch_pgroup(const Ctx &c, const int32_t *ids, const float *wts, int S, int k, int E, int has_shared,
                         const RbtExpertDev *table, uint32_t *bits, uint32_t *pc, PSeg *segs, PTile *tiles,
                         int *ntiles, int *pair_tok, int *tok_pair, float *tok_w, int *err, int *nuniq, int tch) {
  if (E > PG_MAXE || tch < 1) return hipErrorInvalidValue;
  if ((long)E * ((S + 31) / 32) <= PG_SMALLW)
    launch_k(c, k_pgroup<true>, dim3(1), dim3(1024), ids, wts, S, k, E, has_shared, table, bits, pc, segs, tiles,
             ntiles, pair_tok, tok_pair, tok_w, err, nuniq, tch);
  else
    launch_k(c, k_pgroup<false>, dim3(1), dim3(1024), ids, wts, S, k, E, has_shared, table, bits, pc, segs, tiles,
             ntiles, pair_tok, tok_pair, tok_w, err, nuniq, tch);
  return hipGetLastError();
}

bool dgemm_ok(int kind, size_t d, size_t i, size_t n_experts, size_t k) {
  // gate/up: 64-row blocks over I, K groups of 512 columns over H; down: 128-row blocks over H,
  // K groups of 512 columns over I
  return kind == RBT_QT_MXFP4 && d % 512 == 0 && i % 512 == 0 && d <= (1u << 20) && i <= (1u << 20) &&
         n_experts + 1 <= (size_t)PG_MAXE && k <= 64;
}

long dgemm_max_tiles(int S, int k, int E, int has_shared) {
  const long P = (long)S * k;
  const long nseg = std::min<long>(E, P) + (has_shared ? 1 : 0);
  return nseg + (P + (has_shared ? S : 0) + PD_TCH - 1) / PD_TCH;
}

hipError_t launch_split3(const Ctx &c, const float *x, int S, int H, __bf16 *xb3) {
  const long n = (long)S * H;
  if (n <= 0) return hipSuccess;
  launch_k(c, k_split3, dim3((unsigned)((n + 255) / 256)), dim3(256), x, S, H, xb3);
  return hipGetLastError();
}

hipError_t launch_dgateup(const Ctx &c, const PTile *tiles, const int *ntiles, const PSeg *segs,
                          const RbtExpertDev *table, const RbtExpertDev *shared_dev, const int *pair_tok,
                          const __bf16 *xb3, int S, int H, int I, __bf16 *hb3) {
  if (H % 512 || I % 64) return hipErrorInvalidValue;
  launch_k(c, k_dgateup, dim3(3 * c.num_cu), dim3(256), tiles, ntiles, segs, table, shared_dev, pair_tok, xb3, S, H,
           I, hb3);
  return hipGetLastError();
}

hipError_t launch_ddown(const Ctx &c, const PTile *tiles, const int *ntiles, const PSeg *segs,
                        const RbtExpertDev *table, const RbtExpertDev *shared_dev, const __bf16 *hb3, int I, int H,
                        float *y) {
  if (I % 512 || H % 128) return hipErrorInvalidValue;
  launch_k(c, k_ddown, dim3(2 * c.num_cu), dim3(256), tiles, ntiles, segs, table, shared_dev, hb3, I, H, y);
  return hipGetLastError();
}

hipError_t launch_to_bf16(const Ctx &c, const float *x, long n, __bf16 *xb) {
  if (n <= 0) return hipSuccess;
  const long threads = (n + 3) / 4;
  const int vec = ((uintptr_t)x % 16 == 0) && ((uintptr_t)xb % 8 == 0);
  launch_k(c, k_to_bf16, dim3((unsigned)((threads + 255) / 256)), dim3(256), x, n, xb, vec);
  return hipGetLastError();
}

hipError_t launch_pgateup(const Ctx &c, const PTile *tiles, const int *ntiles, long max_tiles, const PSeg *segs,
                          const RbtExpertDev *table, const RbtExpertDev *shared_dev, const int *pair_tok,
                          const __bf16 *xb, int S, int H, int I, __bf16 *hb) {
  const long blocks = (max_tiles + 7) / 8 * 8 * PF_RBG;  // pf_tile_of_block: a multiple of 64
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffffL || H % 512 || I % 1024) return hipErrorInvalidValue;
  launch_k(c, k_pgateup, dim3((unsigned)blocks), dim3(256), tiles, ntiles, segs, table,
                     shared_dev, pair_tok, xb, S, H, I, hb);
  return hipGetLastError();
}

hipError_t launch_pdown(const Ctx &c, const PTile *tiles, const int *ntiles, long max_tiles, const PSeg *segs,
                        const RbtExpertDev *table, const RbtExpertDev *shared_dev, const __bf16 *hb, int I, int H,
                        float *y) {
  const long blocks = (max_tiles + 7) / 8 * 8 * PF_DN_RBG;  // pf_tile_of_block
  if (blocks <= 0) return hipSuccess;
  if (blocks > 0x7fffffffL || H % 512 || I % 1024) return hipErrorInvalidValue;
  launch_k(c, k_pdown, dim3((unsigned)blocks), dim3(256), tiles, ntiles, segs, table, shared_dev,
                     hb, I, H, y);
  return hipGetLastError();
}

}  // namespace rbt
