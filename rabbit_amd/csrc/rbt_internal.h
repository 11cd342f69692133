// rbt_internal.h -- host-side declarations shared by the library's translation units.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <string>

#include "../../include/rabbit_amd.h"
#include "rbt_device.h"

namespace rbt {

struct Ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int num_cu = 256;
  // Profiling: when set, the next timed launch records these events itself at the kernel's start
  // and end (hipExtLaunchKernelGGL), so the interval excludes dispatch gaps.
  hipEvent_t t_start = nullptr, t_stop = nullptr;
  // Per-kernel profiling: when set, every launch records a start/end event pair of its own
  // (kernel_events in api.hip hands them out and files them under the kernel).
  bool kprof = false;
  // Arrival counters (CNT_N, device memory, zeroed at creation): a kernel that counts arrivals on
  // them returns each to 0 before it ends.
  unsigned *d_cnt = nullptr;
};
constexpr int CNT_N = 1024;

// Events for one profiled launch of `fn` (false when none could be created: the launch is untimed).
bool kernel_events(const Ctx &c, const void *fn, hipEvent_t *start, hipEvent_t *stop);

// Launch on the context's stream with `smem` bytes of dynamic LDS; timed by the dispatch when the
// context holds phase events or profiles every kernel.
template <typename K, typename... A>
inline void launch_ks(const Ctx &c, K kernel, dim3 grid, dim3 block, unsigned smem, A... args) {
  hipEvent_t s = c.t_start, e = c.t_stop;
  if (!s && c.kprof && !kernel_events(c, reinterpret_cast<const void *>(kernel), &s, &e)) s = e = nullptr;
  if (s)
    hipExtLaunchKernelGGL(kernel, grid, block, smem, c.stream, s, e, 0, args...);
  else
    hipLaunchKernelGGL(kernel, grid, block, smem, c.stream, args...);
}

template <typename K, typename... A>
inline void launch_k(const Ctx &c, K kernel, dim3 grid, dim3 block, A... args) {
  launch_ks(c, kernel, grid, block, 0u, args...);
}

struct RouterArgs {
  int family, E, erows, k, H, S;
  const float *logit_bias, *router_bias;
  int norm_topk;
  float routed_scale;
  int n_group, topk_group;
  const float *x, *W;
};

// shards.hip: base names, shapes and the packed tensor's suffix of one MXFP4 expert's three
// matrices in read order (ExpertNaming::tensor_specs / packed_suffix, expert_cache.rs:154-208).
int mxfp4_specs(int naming, uint32_t layer, uint32_t eid, size_t hidden, size_t moe_inter, std::string base[3],
                size_t rows[3], size_t cols[3], const char **packed_suffix);

// norm.hip: rmsnorm (kimi_linear/ops.rs:46) or, with one_plus, rmsnorm_1p (qwen38/ops.rs:25) of
// rows x n (x may equal y); x += t over n floats.
hipError_t launch_rmsnorm(const Ctx &c, const float *x, const float *w, float eps, float *y, size_t rows, size_t n,
                          bool one_plus);
hipError_t launch_add_rows(const Ctx &c, float *x, const float *t, size_t n);

// gemv.hip
// One token: the down GEMV over the job list jobs[0 .. kk + has_shared) (the winners in rank
// order, then the shared expert; h rows at h + slots[j] * h_stride) with the ordered combine fused:
// out[r] = sum_j w_j y_j in rank order, then + the shared row (times sh_scale[0] when gated), the
// rounding sequence of launch_combine; the row sums are the bits of launch_decode's MODE_DOWN.
// One workgroup per CU. cols 1025..4096 (MXFP4 or grouped int4 with groups of 32).
bool down1c_ok(int kind, size_t gs, int njobs, int cols, int rows, int num_cu);
hipError_t launch_down1c(const Ctx &c, int kind, size_t gs, const RbtExpertDev *jobs, const int *slots, int kk,
                         int has_shared, const float *h, long h_stride, int cols, int rows, const float *tok_w,
                         const float *sh_scale, int gated, float *out);
hipError_t launch_generic(const Ctx &c, int kind, float *y, const float *x, const void *data, const void *scale,
                          size_t gs, size_t s, size_t i, size_t o);
hipError_t launch_dequant(const Ctx &c, float *out, int kind, const void *data, const void *scale, size_t cols,
                          size_t gs, size_t row0, size_t nrows);
bool decode_shape_ok(size_t cols, int kind, size_t gs);
// Decode GEMV over a job table (see gemv.hip). jobs == nullptr uses `single` for every job.
// njobs_dev (optional) caps the job count from device memory.
// mode: 0 = plain rows, 1 = stacked gate|up rows (raw dots), 2 = plain rows whose activation is
// silu(g) * u built from a stacked g|u input, 3 = plain rows of rmsnorm(x) with weight nw and eps
// (each x row normalised in the wave that reads it; rows up to 8192 columns).
enum { DECODE_DOWN = 0, DECODE_STACKED = 1, DECODE_ACT = 2, DECODE_NORM = 3 };
// parts: for DECODE_ACT, the column-part count the stacked producer used (decode_parts(hidden)).
hipError_t launch_decode(const Ctx &c, int mode, int kind, const RbtExpertDev *jobs, const RbtExpertDev &single,
                         int njobs, const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols,
                         int rows, float *y, long y_stride, int parts = 1, const float *nw = nullptr,
                         float eps = 0.0f);
// Gate/up and the activation in one pass into h [njobs, I] (rows of 2049..6144 columns, the shapes
// decode_shape_ok accepts): bit-identical to the stacked decode + launch_swiglu below 4096 columns,
// within the fp32 accumulation tolerance from 4096 on (where the stacked decode splits the row in two).
bool gu_act_ok(size_t cols, int kind, size_t gs);
hipError_t launch_gu_act(const Ctx &c, int kind, const RbtExpertDev *jobs, const RbtExpertDev &single, int njobs,
                         const int *njobs_dev, const float *x, const int *x_index, long x_stride, int cols, int I,
                         float *h, const RbtAct &act);
// h[p, k] = act(sum of gate parts, sum of up parts) for the stacked producer's output.
hipError_t launch_swiglu(const Ctx &c, const float *gu, long gu_stride, int half, int npairs, const int *npairs_dev,
                         int parts, float *h, const RbtAct &act = RbtAct{});
// One token through one MXFP4 or grouped-int4 (groups of 32) matrix of 2048..8192 columns, x staged
// in LDS per workgroup (a projection); with nw, x is rmsnorm(x) * nw first (DECODE_NORM).
bool proj1_ok(int kind, size_t gs, int cols, int rows, int num_cu);
hipError_t launch_proj1(const Ctx &c, int kind, size_t gs, const void *data, const void *scale, const float *x,
                        int cols, int rows, float *y, const float *nw = nullptr, float eps = 0.0f);
// Column parts the stacked gate/up kernel splits a row of `cols` columns into; its output per job
// is 2 * parts vectors of `half` floats (gate parts, then up parts).
int decode_parts(int cols);
hipError_t launch_pair_generic(const Ctx &c, bool gateup, int kind, size_t gs, const RbtExpertDev *jobs,
                               const RbtExpertDev &single, int njobs, const int *njobs_dev, const float *x,
                               const int *x_index, long x_stride, int cols, int rows, float *y, long y_stride,
                               const RbtAct &act = RbtAct{});

// xgemm.hip: MXFP4 expert products on the matrix cores (decode shapes).
bool xgemm_ok(int kind, size_t d, size_t i, int S, int k, int has_shared);
hipError_t launch_xgateup(const Ctx &c, const RbtExpertDev *jobs, const int *tok, int npairs, const float *x,
                          long x_stride, int K, int I, __bf16 *hp);
// One token (every pair reads x): the same products balanced over num_cu workgroups.
hipError_t launch_xgateup1(const Ctx &c, const RbtExpertDev *jobs, int npairs, const float *x, int K, int I,
                           __bf16 *hp);
// hp: h as three bf16 parts per pair, hp[(p*3 + part)*I + k].
// One token: down + ordered combine balanced over num_cu workgroups, every pair's h in LDS. The
// pairs are the kk winners in slot order (down_job[j], h at pair slot down_slot[j], weight
// tok_w[j]) and, with has_shared, the shared expert (down_job[kk], h at down_slot[kk]).
// accumulate: out += the combined row instead of out = (one rounding, as x[i] += tmp[i]).
// sh_dd/sh_ds: the shared expert's down weights and scales (the same as down_job[kk]'s), or null;
// given, its tiles go first and their first loads are issued before the job table is read.
bool xdown1_ok(int npairs, size_t i);
hipError_t launch_xdown1(const Ctx &c, const RbtExpertDev *down_job, const int *down_slot, int kk, const __bf16 *hp,
                         int I, int H, const float *tok_w, const float *sh_scale, int has_shared, int gated,
                         float *out, bool accumulate = false, const uint8_t *sh_dd = nullptr,
                         const uint8_t *sh_ds = nullptr);
// One token, pair-major: the same pair list's down products as contiguous runs of 4-row tiles per
// wave (a workgroup stages the h of at most two pairs), each pair's rows into yy[j * H + r] (j in
// the pair list's order), then the ordered combine (k_combine1) into out.
bool xdown2_ok(int npairs, size_t i, int H, int num_cu);
hipError_t launch_xdown2(const Ctx &c, const RbtExpertDev *down_job, const int *down_slot, int kk, const __bf16 *hp,
                         int I, int H, const float *tok_w, const float *sh_scale, int has_shared, int gated,
                         float *yy, float *out, bool accumulate, const uint8_t *sh_dd, const uint8_t *sh_ds);
hipError_t launch_xdown(const Ctx &c, const RbtExpertDev *jobs, int npairs, const __bf16 *hp, int I, int H, int S,
                        int k, const int *tok, const int *tok_pair, const float *tok_w, const float *sh_scale,
                        int has_shared, int gated, float *out);

// xgemv1.hip: one token, MXFP4, on the matrix cores with every load issued at entry.
// y[O] = W[O, I] . x (matmul_mxfp4 for s = 1), I a multiple of 512 (4, 7, 8, 14 or 16 steps).
bool xgemv1_ok(size_t cols, size_t rows, int num_cu);
hipError_t launch_xgemv1(const Ctx &c, const uint8_t *data, const uint8_t *scale, const float *x, int I, int O,
                         float *y);
// apply_single_expert for one token (d = 8192 or 7168, i = 2048): when ids[0..k) holds eid, out +=
// w * down(act(gate . x, up . x)) with w its first matching weight; hp: 3 * i bf16 of scratch.
bool xexpert1_ok(size_t d, size_t i, int num_cu);
hipError_t launch_xexpert1(const Ctx &c, const RbtExpertDev &J, const float *x, int d, int i, const int32_t *ids,
                           const float *wts, int k, int eid, __bf16 *hp, float *out, const RbtAct &act);

// prefill.hip: MXFP4 prefill as grouped GEMMs on the matrix cores.
constexpr int PG_MAXE = 2048;  // segments (unique experts + shared) per call
constexpr int PF_TCH = 64;     // tokens per GEMM tile
constexpr int PF_NT = PF_TCH / 16;
struct PSeg {
  int eid;  // expert id, -1 for the shared expert
  int off;  // first pair of the segment
  int cnt;  // tokens (pairs) in the segment
  int pad;
};
struct PTile {
  int seg;  // segment index
  int c0;   // first token of the tile within the segment
};
bool prefill_ok(int kind, size_t d, size_t i, size_t n_experts, size_t k);
long prefill_max_tiles(int S, int k, int E, int has_shared);
hipError_t launch_pgroup(const Ctx &c, const int32_t *ids, const float *wts, int S, int k, int E, int has_shared,
                         const RbtExpertDev *table, uint32_t *bits, uint32_t *pc, PSeg *segs, PTile *tiles,
                         int *ntiles, int *pair_tok, int *tok_pair, float *tok_w, int *err, int *nuniq,
                         int tch = PF_TCH);
// Grouped decode (a few tokens, fp32-accurate): tiles of at most PD_TCH tokens from launch_pgroup
// (tch = PD_TCH), x split into three bf16 parts per token (xb3 [3 S, H]), gate/up -> hb3
// [3 (pairs), I] bf16 parts, down -> y [pairs, H] fp32; then launch_combine.
constexpr int PD_TCH = 10;
bool dgemm_ok(int kind, size_t d, size_t i, size_t n_experts, size_t k);
long dgemm_max_tiles(int S, int k, int E, int has_shared);
hipError_t launch_split3(const Ctx &c, const float *x, int S, int H, __bf16 *xb3);
hipError_t launch_dgateup(const Ctx &c, const PTile *tiles, const int *ntiles, const PSeg *segs,
                          const RbtExpertDev *table, const RbtExpertDev *shared_dev, const int *pair_tok,
                          const __bf16 *xb3, int S, int H, int I, __bf16 *hb3);
hipError_t launch_ddown(const Ctx &c, const PTile *tiles, const int *ntiles, const PSeg *segs,
                        const RbtExpertDev *table, const RbtExpertDev *shared_dev, const __bf16 *hb3, int I, int H,
                        float *y);
hipError_t launch_to_bf16(const Ctx &c, const float *x, long n, __bf16 *xb);
hipError_t launch_pgateup(const Ctx &c, const PTile *tiles, const int *ntiles, long max_tiles, const PSeg *segs,
                          const RbtExpertDev *table, const RbtExpertDev *shared_dev, const int *pair_tok,
                          const __bf16 *xb, int S, int H, int I, __bf16 *hb);
hipError_t launch_pdown(const Ctx &c, const PTile *tiles, const int *ntiles, long max_tiles, const PSeg *segs,
                        const RbtExpertDev *table, const RbtExpertDev *shared_dev, const __bf16 *hb, int I, int H,
                        float *y);

// router.hip
hipError_t launch_router_logits(const Ctx &c, const float *x, int S, int H, const float *W, int E, const float *sgate,
                                double *mid, double *bnd);
// Batched path: the reference's sequential fp32 logits themselves, logits[S, E (+1 with sgate)].
bool router_exact_ok(int S, int H);
hipError_t launch_router_logits_exact(const Ctx &c, const float *x, int S, int H, const float *W, int E,
                                      const float *sgate, float *logits);
// One-token decode on the matrix cores (router launch -> gate/up launch -> down launch). The router
// launch writes mid / bnd and one key record per expert and streams the shared expert's gate/up;
// every workgroup of the gate/up launch then selects the top-k from the key records itself. When
// the certified intervals leave the decision open, the routed pairs are the certain winners in
// midpoint order followed by the undecided candidates (up to D1_KX beyond top-k), and the gate/up
// launch's extra workgroup folds the undecided logits exactly while the pairs stream, then writes
// ids, weights, tok_pair / tok_w and the down launch's job list.
constexpr int D1_KX = 4;   // routed pair slots beyond top-k for undecided candidates
constexpr int D1_NC = 32;  // most routed pairs a deferred decision carries
struct D1Task {
  int nr;       // routed pairs of the call: slots 0 .. nr-1
  int pending;  // 1: the decision waits for exact folds
  int pad[2];
  int id[D1_NC];       // expert of slot c
  uint32_t ku[D1_NC];  // its midpoint order key
  float lm[D1_NC];     // its midpoint logit
  int flag[D1_NC];     // 1: its logit is recomputed as the reference folds it
};

struct GroupArgs {
  const RbtExpertDev *table, *shared_dev;
  RbtExpertDev *pair_job;
  int *pair_tok, *tok_pair;
  float *tok_w;
  int *err;
  // one token (all optional): the down launch's job list and pair slots, the shared expert's slot
  // (default: k)
  RbtExpertDev *down_job = nullptr;
  int *down_slot = nullptr;
  int shared_slot = -1;
  // the shared expert's pointers by value (one token: its gate/up loads go out before the routing
  // is known; all null: not available)
  RbtExpertDev shv{};
};
// The shared expert's gate/up for a one-token call (balanced body of xgemm), run by a router launch
// on the CUs its selection (or its rows) leave free. hp: the shared pair's output parts.
struct SharedGateUp {
  const RbtExpertDev *dev;
  const float *x;
  int K, I;
  __bf16 *hp;
};
// One token of the latent MoE: the selection (with the one-token pair list) on workgroup 0 and the
// latent down projection xl[rows] = proj.dd . x (MXFP4 or grouped int4, 2049..8192 columns) on one
// workgroup per CU, in one launch.
bool router_select_dp_ok(const RouterArgs &a, int kind, int cols, int rows);
hipError_t launch_router_select_dp(const Ctx &c, const RouterArgs &a, const double *mid, const double *bnd,
                                   int32_t *ids, float *wts, float *sh_scale, int *stats, const GroupArgs &grp,
                                   const RbtExpertDev &proj, int kind, int cols, int rows, float *xl);
hipError_t launch_router_select(const Ctx &c, const RouterArgs &a, const double *mid, const double *bnd, int32_t *ids,
                                float *wts, float *sh_scale, int *stats, const GroupArgs *grp = nullptr,
                                const SharedGateUp *sgu = nullptr);
// Router launch of the one-token decode (no cross-workgroup waits): mid / bnd of every router row,
// sh_scale (the shared gate's sigmoid, or 1) and rec (E * ROUTER1_REC_BYTES). With nw, a.x is the
// raw token and the rows use rmsnorm_1p(a.x, nw, eps) (bit-identical to launch_rmsnorm's), which
// the launch also writes to xn.
bool router1_ok(const RouterArgs &a, int num_cu, const SharedGateUp *sgu);
// A decode batch (2+ tokens, hidden a multiple of 1024 up to 8192, up to 1024 experts, no grouped
// routing): certified intervals (mid/bnd as launch_router_logits), one (row, token) per workgroup,
// then one selection workgroup per token (keys formed by the whole workgroup, the one-token fast
// path, the general path where it does not certify). table: the layer's job table (the fast path
// reads winners' entries).
bool router_batch_ok(const RouterArgs &a);
// xb3 (optional, [3 S, H] bf16): the tokens' exact three-part bf16 split, written by the selection
// launch's idle waves (the grouped decode GEMMs' activation)
hipError_t launch_router_batch(const Ctx &c, const RouterArgs &a, const float *sgate, double *mid, double *bnd,
                               const RbtExpertDev *table, int32_t *ids, float *wts, float *sh_scale, int *stats,
                               __bf16 *xb3 = nullptr);
hipError_t launch_router1(const Ctx &c, const RouterArgs &a, const float *sgate, double *mid, double *bnd,
                          float *sh_scale, void *rec, const float *nw = nullptr, float eps = 0.0f,
                          float *xn = nullptr);
// Gate/up launch of the one-token decode (num_cu workgroups): the selection from rec in every
// workgroup, the gate/up of the nr routed pairs (slots 0..nr-1, nr <= k + D1_KX) and, with
// has_shared, of grp.shared_dev at slot nr, into hp (pair slot c at hp + 3 I c), and the routing
// outputs (ids, wts, grp's tok_pair / tok_w / down_job / down_slot, the shared expert last with its
// slot). stats counts exact folds; gup (optional) the pairs streamed.
hipError_t launch_xgateup1s(const Ctx &c, const RouterArgs &a, const void *rec, const double *mid,
                            const double *bnd, const GroupArgs &grp, int32_t *ids, float *wts, int *stats, int *gup,
                            int I, __bf16 *hp, bool has_shared);
// K3's latent MoE, one token: the router rows' key records (one row per workgroup), then, after the
// latent down projection, the selection and the experts' gate/up with act on the matrix cores over
// x_latent (moe_hidden 3584), h in fp32 (pair slot c at h + I c); ga's down job list, slots,
// tok_pair and tok_w as launch_xgateup1s writes them.
bool router1_latent_ok(const RouterArgs &a, int num_cu, int mh, int I);
// One token through the decode GEMVs (grouped int4 and the other non-matrix-core shapes):
// launch_router1_any writes the key records (and the shared gate), launch_gu1s_gemv selects in every
// workgroup and runs the fused gate/up + activation GEMV over the routed pairs and the shared expert
// (h in fp32 at the pair slots; ga's down job list, slots, tok_pair and tok_w as launch_xgateup1s).
bool gu1s_gemv_ok(const RouterArgs &a, int num_cu, int kind, size_t gs, int I);
hipError_t launch_router1_any(const Ctx &c, const RouterArgs &a, double *mid, double *bnd, float *sh_scale,
                              const float *sgate, void *rec);
hipError_t launch_gu1s_gemv(const Ctx &c, const RouterArgs &a, const void *rec, const double *mid,
                            const double *bnd, const GroupArgs &grp, int32_t *ids, float *wts, int *stats, int kind,
                            size_t gs, int I, float *h, bool has_shared);
// The router rows of launch_router1_latent and the latent down projection xl = Dp . x (Dp: mh rows
// of a.H columns, MXFP4 or grouped int4 with groups of 32; launch_proj1's arithmetic) in one launch.
bool router1_proj_ok(const RouterArgs &a, int num_cu, int mh, int I, int kind, size_t gs);
hipError_t launch_router1_proj(const Ctx &c, const RouterArgs &a, double *mid, double *bnd, float *sh_scale,
                               void *rec_buf, int mh, int I, int kind, size_t gs, const void *data, const void *scale,
                               float *xl);
hipError_t launch_router1_latent(const Ctx &c, const RouterArgs &a, double *mid, double *bnd, float *sh_scale,
                                 void *rec, int mh, int I);
hipError_t launch_xgateup1s_latent(const Ctx &c, const RouterArgs &a, const void *rec, const double *mid,
                                   const double *bnd, const GroupArgs &grp, int32_t *ids, float *wts, int *stats,
                                   int *gup, const float *xl, int mh, int I, float *h, const RbtAct &act);
// Device bytes of the key records launch_router1 writes (per router row).
constexpr size_t ROUTER1_REC_BYTES = 16;
hipError_t launch_logits_to_mid(const Ctx &c, const float *logits, size_t n, double *mid, double *bnd);
// Batched router logits on the matrix cores, certified: mid (fp64-accurate) and a rigorous bound on
// the distance to the reference's sequential fp32 fold, for launch_router_select (which folds the
// ambiguous ones exactly). scratch: router_bounded_scratch bytes.
bool router_bounded_ok(const RouterArgs &a);
size_t router_bounded_scratch(const RouterArgs &a, int erows);
hipError_t launch_router_bounded(const Ctx &c, const RouterArgs &a, const float *sgate, double *mid, double *bnd,
                                 void *scratch);
hipError_t launch_group(const Ctx &c, const int32_t *ids, const float *wts, int S, int k, int E,
                        const RbtExpertDev *table, const RbtExpertDev *shared_dev, RbtExpertDev *pair_job,
                        int *pair_tok, int *tok_pair, float *tok_w, int *err, int *nuniq);
hipError_t launch_combine(const Ctx &c, const float *y, int S, int k, int H, const int *tok_pair, const float *tok_w,
                          const float *sh_scale, int has_shared, int gated, float *out);

// moe.hip
hipError_t launch_single_rows(const Ctx &c, const int32_t *ids, const float *w, int S, int k, int eid, int *pair_tok,
                              float *pair_w, int *nr);
hipError_t launch_accumulate(const Ctx &c, const float *y, int S, int H, const int *pair_tok, const float *pair_w,
                             const int *nr, float *out);

// mixers.hip: Qwen 3.8's token mixers for one token.
bool gdn_ok(int n_v, int n_k, int d_k, int d_v);
// act: conv_dim floats of scratch (the conv output after SiLU).
hipError_t launch_gdn(const Ctx &c, float *conv_hist, const float *conv_w, int K, float *states,
                      const float *qkv_pre, const float *z, const float *a, const float *b, const float *a_log,
                      const float *dt_bias, const float *norm_w, float eps, int n_v, int n_k, int d_k, int d_v,
                      float *act, float *out);
bool gqa_ok(int n_heads, int n_kv, int hd, int rope_dim);
// Scratch of the GQA step: qp (n_heads * hd floats) and part (gqa_part_floats).
size_t gqa_part_floats(int n_heads, int n_kv, int hd, int positions);
hipError_t launch_gqa(const Ctx &c, const float *qg, const float *k, const float *v, int n_heads, int n_kv, int hd,
                      const float *qn, const float *kn, float eps, int rope_dim, float theta, float scale, int pos,
                      float *kc, float *vc, float *qp, float *part, float *ctx);

// synth.hip
hipError_t launch_synth_mxfp4(const Ctx &c, uint8_t *data, uint8_t *scale, size_t rows, size_t cols, uint64_t seed,
                              uint32_t lo, uint32_t hi);
hipError_t launch_synth_i4g(const Ctx &c, uint8_t *data, float *scale, size_t rows, size_t cols, size_t gs,
                            uint64_t seed, float lo, float hi);

}  // namespace rbt
