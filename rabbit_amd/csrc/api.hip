// api.hip -- host side of the C ABI declared in include/rabbit_amd.h.
//
// Owns the per-context HIP stream, grow-only device scratch, the HBM-resident expert pool (the
// storage half of ExpertCache, expert_cache.rs) and the per-layer MoE state (router, biases,
// shared expert, device table of resident experts). Orchestrates the decode/prefill pipeline of
// one MoE layer: router logits -> certified top-k -> grouping -> gate/up dequant-GEMV (+SiLU) ->
// down dequant-GEMV -> ordered combine (+ shared expert).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <cstdarg>
#include <initializer_list>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "rbt_internal.h"

#include <mutex>

// Device scratch of the allocation-free entry point (rbt_moe_forward_noalloc_d): one copy per
// device, held until the process ends. On the host this name is only a stand-in for the symbol, not
// a device address: host code uses the address hipGetSymbolAddress returned for the device
// (noalloc_base, resolved once per device by rbt_init) wherever it needs the array's memory.
static __device__ __align__(256) uint8_t noalloc_scratch[RBT_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int NOALLOC_MAX_DEV = 64;
std::mutex g_noalloc_mu;
uint8_t *g_noalloc_ptr[NOALLOC_MAX_DEV];
hipError_t g_noalloc_err[NOALLOC_MAX_DEV];
bool g_noalloc_done[NOALLOC_MAX_DEV];

// The device address of noalloc_scratch on `device`, which must be current: looked up on the
// device's first context, then kept (nullptr when the lookup failed; *err says why).
uint8_t *noalloc_base(int device, hipError_t *err) {
  std::lock_guard<std::mutex> g(g_noalloc_mu);
  if (device < 0 || device >= NOALLOC_MAX_DEV) {
    *err = hipErrorInvalidDevice;
    return nullptr;
  }
  if (!g_noalloc_done[device]) {
    void *p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(noalloc_scratch));
    if (e != hipSuccess) (void)hipGetLastError();
    g_noalloc_err[device] = e;
    g_noalloc_ptr[device] = e == hipSuccess ? static_cast<uint8_t *>(p) : nullptr;
    g_noalloc_done[device] = true;
  }
  *err = g_noalloc_err[device];
  return g_noalloc_ptr[device];
}

enum ScratchSlot {
  SC_X,
  SC_Y,
  SC_W,
  SC_S,
  SC_MID,
  SC_BND,
  SC_IDS,
  SC_WTS,
  SC_SHS,
  SC_PJOB,
  SC_PTOK,
  SC_TPAIR,
  SC_TW,
  SC_H,
  SC_YY,
  SC_FLAGS,
  SC_STAGE,
  SC_OUT,
  SC_IDS_OUT,
  SC_W_OUT,
  SC_GU,
  SC_XB,
  SC_PGRP,
  SC_RLOG,
  SC_RREC,
  SC_DJOB,
  SC_DSLOT,

  SC_NRM,   // sublayer: the normalised rows
  SC_SUB,   // sublayer: the MoE output before the residual add
  SC_PLN,   // sublayer (host call): post_ln staged
  SC_XL,    // latent MoE: x projected down
  SC_ROUTED,  // latent MoE: summed routed rows
  SC_MIXA,    // mixers: the GDN conv output / the GQA prepared queries
  SC_MIXB,    // mixers: the GQA softmax partials
  SC_N
};

struct PoolEntry {
  rbt_expert_slot slot{};  // device pointers
  void *alloc = nullptr;   // owned allocation (nullptr for caller-owned device slots)
  size_t bytes = 0;
};

struct Layer {
  rbt_moe_layer_desc desc{};  // device pointers
  std::vector<void *> owned;
  bool set = false;
  bool dirty = true;
  RbtExpertDev *d_table = nullptr;  // n_experts entries, allocated with the layer
  size_t table_n = 0;
  std::vector<RbtExpertDev> h_table;  // host image of d_table (sized with the layer: refreshing it allocates nothing)
  RbtExpertDev *d_shared = nullptr;
  RbtExpertDev h_shared{};
  int shared_kind = -1;
  size_t shared_gs = 0, shared_inter = 0;
  int routed_kind = -1;
  size_t routed_gs = 0;
  // the latent MoE's view of the pool at (moe_hidden, moe_inter): n_experts jobs, then a zero job
  bool lat_dirty = true;
  RbtExpertDev *d_lat = nullptr;
  size_t lat_cap = 0, lat_mh = 0;
  int lat_kind = -1;
  size_t lat_gs = 0;
};

}  // namespace

struct rbt_ctx : rbt::Ctx {
  std::string err;
  void *scratch[SC_N] = {};
  size_t scratch_cap[SC_N] = {};
  // allocation-free calls: the device's fixed scratch array (its device address, or nullptr when the
  // lookup failed), carved per slot for one call
  uint8_t *noalloc = nullptr;
  hipError_t noalloc_err = hipSuccess;
  uint8_t *arena = nullptr;
  size_t arena_cap = 0, arena_used = 0;
  size_t arena_off[SC_N] = {}, arena_sz[SC_N] = {};
  std::map<uint64_t, PoolEntry> pool;
  std::map<uint32_t, Layer> layers;
  // device: [0] error flag, [1] ambiguity count, [2] unique experts, [4] gate/up pairs; then the
  // arrival counters (d_cnt)
  int *d_flags = nullptr;
  int h_flags[8] = {};
  // profiling: one row of 5 events per recorded moe_forward_d call
  bool prof = false;
  std::vector<hipEvent_t> ev_free;
  std::vector<std::array<hipEvent_t, 7>> ev_rows;
  std::vector<std::array<uint64_t, 2>> ev_experts;  // per recorded call: gate/up and down experts
  rbt_profile acc{};
  // per-kernel profiling: one start/end pair per launch while kprof is on, summed per kernel by
  // rbt_profile_kernels_read
  struct KRec {
    const void *fn;
    hipEvent_t start, stop;
  };
  std::vector<KRec> krecs;
  std::map<const void *, std::pair<uint64_t, double>> kacc;  // kernel -> (launches, ms)
};

namespace rbt {
bool kernel_events(const Ctx &base, const void *fn, hipEvent_t *start, hipEvent_t *stop) {
  // every Ctx the library launches on is the base of an rbt_ctx
  rbt_ctx *c = static_cast<rbt_ctx *>(const_cast<Ctx *>(&base));
  hipEvent_t ev[2] = {nullptr, nullptr};
  for (auto &e : ev) {
    if (!c->ev_free.empty()) {
      e = c->ev_free.back();
      c->ev_free.pop_back();
    } else if (hipEventCreate(&e) != hipSuccess) {
      (void)hipGetLastError();
      if (ev[0]) c->ev_free.push_back(ev[0]);
      return false;
    }
  }
  c->krecs.push_back({fn, ev[0], ev[1]});
  *start = ev[0];
  *stop = ev[1];
  return true;
}
}  // namespace rbt

namespace {

constexpr int FLAG_ERR = 0, FLAG_AMB = 1, FLAG_UNIQ = 2, FLAG_NR = 3, FLAG_GUP = 4, FLAG_N = 8;

int fail(rbt_ctx *c, int code, const char *fmt, ...) __attribute__((format(printf, 3, 4)));
int fail(rbt_ctx *c, int code, const char *fmt, ...) {
  if (c) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    c->err = buf;
  }
  return code;
}

#define HIP_OK(c, expr)                                                                                   \
  do {                                                                                                    \
    hipError_t e_ = (expr);                                                                               \
    if (e_ != hipSuccess) return fail((c), RBT_E_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_),   \
                                      __FILE__, __LINE__);                                                \
  } while (0)

#define RBT_TRY(expr)        \
  do {                       \
    int rc_ = (expr);        \
    if (rc_ != RBT_OK) return rc_; \
  } while (0)

size_t div_ceil(size_t a, size_t b) { return (a + b - 1) / b; }
size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

// Grow-only device scratch. Growth synchronises the stream first, so in-flight work never sees a
// freed buffer. Inside an allocation-free call (c->arena set) the slots are carved out of the
// device's fixed scratch array instead, a slot keeping its region for the rest of the call.
int scratch(rbt_ctx *c, int slot, size_t bytes, void **out) {
  if (bytes == 0) bytes = 256;
  if (c->arena) {
    if (c->arena_sz[slot] == 0) {
      const size_t need = align256(bytes);
      if (need > c->arena_cap - c->arena_used)
        return fail(c, RBT_E_UNSUPPORTED,
                    "the allocation-free call needs more than its %zu bytes of device scratch (slot %d wants %zu "
                    "bytes with %zu already used): fewer tokens per call, or the allocating entry point",
                    c->arena_cap, slot, need, c->arena_used);
      c->arena_off[slot] = c->arena_used;
      c->arena_sz[slot] = need;
      c->arena_used += need;
    } else if (c->arena_sz[slot] < bytes) {
      return fail(c, RBT_E_UNSUPPORTED, "scratch slot %d asked for twice with a larger size in one call", slot);
    }
    *out = c->arena + c->arena_off[slot];
    return RBT_OK;
  }
  if (c->scratch_cap[slot] < bytes) {
    HIP_OK(c, hipStreamSynchronize(c->stream));
    if (c->scratch[slot]) HIP_OK(c, hipFree(c->scratch[slot]));
    c->scratch[slot] = nullptr;
    c->scratch_cap[slot] = 0;
    size_t cap = align256(bytes + bytes / 4);
    if (hipMalloc(&c->scratch[slot], cap) != hipSuccess) {
      (void)hipGetLastError();
      return fail(c, RBT_E_NOMEM, "hipMalloc(%zu) for scratch slot %d failed", cap, slot);
    }
    c->scratch_cap[slot] = cap;
  }
  *out = c->scratch[slot];
  return RBT_OK;
}

template <typename T>
int scratch_t(rbt_ctx *c, int slot, size_t count, T **out) {
  void *p;
  RBT_TRY(scratch(c, slot, count * sizeof(T), &p));
  *out = (T *)p;
  return RBT_OK;
}

// Bytes of a QT's data and scale arrays.
size_t qt_data_bytes(const rbt_qt &w) {
  if (w.kind == RBT_QT_F32) return w.rows * w.cols * 4;
  return w.rows * div_ceil(w.cols, 2);
}
size_t qt_scale_bytes(const rbt_qt &w) {
  if (w.kind == RBT_QT_MXFP4) return w.rows * div_ceil(w.cols, 32);
  if (w.kind == RBT_QT_I4_GROUPED) return w.rows * div_ceil(w.cols, w.group_size) * 4;
  return 0;
}

int check_qt(rbt_ctx *c, const rbt_qt *w, const char *what) {
  if (!w) return fail(c, RBT_E_INVALID, "%s: null rbt_qt", what);
  if (w->kind != RBT_QT_F32 && w->kind != RBT_QT_MXFP4 && w->kind != RBT_QT_I4_GROUPED)
    return fail(c, RBT_E_INVALID, "%s: unknown rbt_qt kind %d", what, (int)w->kind);
  if (w->rows == 0 || w->cols == 0) return fail(c, RBT_E_INVALID, "%s: empty shape", what);
  if (!w->data) return fail(c, RBT_E_INVALID, "%s: null data", what);
  if (w->kind != RBT_QT_F32 && !w->scale) return fail(c, RBT_E_INVALID, "%s: null scale", what);
  if (w->kind == RBT_QT_I4_GROUPED && w->group_size == 0)
    return fail(c, RBT_E_INVALID, "%s: group_size 0", what);
  if (w->rows > (1u << 30) || w->cols > (1u << 30)) return fail(c, RBT_E_INVALID, "%s: dimension too large", what);
  return RBT_OK;
}

// Device view of an expert slot (fused gate_up presented as two halves).
int slot_view(rbt_ctx *c, const rbt_expert_slot *s, size_t d, size_t i, RbtExpertDev *v, int *kind, size_t *gs) {
  const rbt_qt &g = s->fused ? s->gate_up : s->gate;
  RBT_TRY(check_qt(c, &g, s->fused ? "gate_up" : "gate"));
  RBT_TRY(check_qt(c, &s->down, "down"));
  if (!s->fused) RBT_TRY(check_qt(c, &s->up, "up"));
  int k = g.kind;
  if (k == RBT_QT_F32) return fail(c, RBT_E_UNSUPPORTED, "expert %u: f32 expert weights are not on this path", s->eid);
  if (s->down.kind != k || (!s->fused && s->up.kind != k))
    return fail(c, RBT_E_UNSUPPORTED, "expert %u: gate/up/down formats differ", s->eid);
  size_t rows_g = s->fused ? 2 * i : i;
  if (g.rows != rows_g || g.cols != d || s->down.rows != d || s->down.cols != i ||
      (!s->fused && (s->up.rows != i || s->up.cols != d)))
    return fail(c, RBT_E_SHAPE, "expert %u: weight shapes do not match hidden=%zu moe_inter=%zu", s->eid, d, i);
  size_t g_gs = k == RBT_QT_I4_GROUPED ? g.group_size : 32;
  if (k == RBT_QT_I4_GROUPED && (s->down.group_size != g_gs || (!s->fused && s->up.group_size != g_gs)))
    return fail(c, RBT_E_UNSUPPORTED, "expert %u: group sizes differ", s->eid);
  v->gd = (const uint8_t *)g.data;
  v->gs = g.scale;
  if (s->fused) {
    // gate rows first, then up rows (glm52/moe.rs:494-503).
    size_t row_scale = k == RBT_QT_MXFP4 ? div_ceil(d, 32) : div_ceil(d, g_gs) * 4;
    v->ud = (const uint8_t *)g.data + i * div_ceil(d, 2);
    v->us = (const uint8_t *)g.scale + i * row_scale;
  } else {
    v->ud = (const uint8_t *)s->up.data;
    v->us = s->up.scale;
  }
  v->dd = (const uint8_t *)s->down.data;
  v->ds = s->down.scale;
  *kind = k;
  *gs = g_gs;
  return RBT_OK;
}

// Shape of an expert slot: d = hidden (gate cols), i = moe_inter (down cols).
void slot_dims(const rbt_expert_slot *s, size_t *d, size_t *i) {
  *d = s->down.rows;
  *i = s->down.cols;
}

int sync_and_check(rbt_ctx *c) {
  HIP_OK(c, hipStreamSynchronize(c->stream));
  HIP_OK(c, hipMemcpy(c->h_flags, c->d_flags, FLAG_N * sizeof(int), hipMemcpyDeviceToHost));
  if (c->h_flags[FLAG_ERR]) {
    HIP_OK(c, hipMemset(c->d_flags, 0, sizeof(int)));
    return fail(c, RBT_E_NOT_RESIDENT, "a routed expert is not resident in the pool");
  }
  return RBT_OK;
}

// Copies n bytes host -> device scratch slot and returns the device pointer.
int stage_in(rbt_ctx *c, int slot, const void *host, size_t n, void **dev) {
  RBT_TRY(scratch(c, slot, n, dev));
  if (n) HIP_OK(c, hipMemcpyAsync(*dev, host, n, hipMemcpyHostToDevice, c->stream));
  return RBT_OK;
}

// Uploads a host QT into a contiguous staging region at *cursor, returning the device copy.
int upload_qt(rbt_ctx *c, const rbt_qt &h, uint8_t *base, size_t *cursor, rbt_qt *d) {
  *d = h;
  size_t nd = qt_data_bytes(h), ns = qt_scale_bytes(h);
  d->data = base + *cursor;
  HIP_OK(c, hipMemcpyAsync(base + *cursor, h.data, nd, hipMemcpyHostToDevice, c->stream));
  *cursor += align256(nd);
  if (ns) {
    d->scale = base + *cursor;
    HIP_OK(c, hipMemcpyAsync(base + *cursor, h.scale, ns, hipMemcpyHostToDevice, c->stream));
    *cursor += align256(ns);
  } else {
    d->scale = nullptr;
  }
  return RBT_OK;
}

size_t slot_bytes(const rbt_expert_slot *s) {
  size_t n = 0;
  auto add = [&](const rbt_qt &q) { n += align256(qt_data_bytes(q)) + align256(qt_scale_bytes(q)); };
  if (s->fused) add(s->gate_up);
  else {
    add(s->gate);
    add(s->up);
  }
  add(s->down);
  return n;
}

int upload_slot(rbt_ctx *c, const rbt_expert_slot *h, uint8_t *base, rbt_expert_slot *d) {
  size_t cur = 0;
  *d = *h;
  if (h->fused) RBT_TRY(upload_qt(c, h->gate_up, base, &cur, &d->gate_up));
  else {
    RBT_TRY(upload_qt(c, h->gate, base, &cur, &d->gate));
    RBT_TRY(upload_qt(c, h->up, base, &cur, &d->up));
  }
  RBT_TRY(upload_qt(c, h->down, base, &cur, &d->down));
  return RBT_OK;
}

const PoolEntry *find_pool_slot(rbt_ctx *c, const rbt_expert_slot *s) {
  for (auto &kv : c->pool)
    if (&kv.second.slot == s) return &kv.second;
  return nullptr;
}

// y[S,O] = x . W^T for one QT whose pointers are device memory.
int matmul_dev(rbt_ctx *c, float *y, const float *x, const rbt_qt *w, size_t s) {
  RBT_TRY(check_qt(c, w, "matmul"));
  if (s == 0) return RBT_OK;
  if (s > (1u << 24)) return fail(c, RBT_E_INVALID, "token count %zu too large", s);
  const size_t i = w->cols, o = w->rows;
  bool aligned = ((uintptr_t)w->data % 16 == 0) && ((uintptr_t)x % 16 == 0);
  if (w->kind == RBT_QT_MXFP4 && s == 1 && aligned && (uintptr_t)w->scale % 4 == 0 &&
      rbt::xgemv1_ok(i, o, c->num_cu)) {
    // one token on the matrix cores, the whole matrix in flight at once
    HIP_OK(c, rbt::launch_xgemv1(*c, (const uint8_t *)w->data, (const uint8_t *)w->scale, x, (int)i, (int)o, y));
    return RBT_OK;
  }
  if (w->kind != RBT_QT_F32 && aligned && rbt::decode_shape_ok(i, w->kind, w->group_size)) {
    RbtExpertDev one{};
    one.dd = (const uint8_t *)w->data;
    one.ds = w->scale;
    HIP_OK(c, rbt::launch_decode(*c, rbt::DECODE_DOWN, w->kind, nullptr, one, (int)s, nullptr, x, nullptr, (long)i, (int)i,
                                 (int)o, y, (long)o));
    return RBT_OK;
  }
  HIP_OK(c, rbt::launch_generic(*c, w->kind, y, x, w->data, w->scale, w->group_size, s, i, o));
  return RBT_OK;
}

// Runs gate/up (+SiLU) then down for `njobs` (expert, token) pairs.
//   x: [tokens, d], x_index[p] = token of pair p; y: [njobs, d].
//   h: scratch of njobs * 2i floats. The fast path writes the stacked gate|up dot products to a
//   second scratch and a small kernel writes act(g, u) (SiLU, or K3's Situ) to h; the generic path
//   writes the activated [njobs, i] to h directly.
int expert_pairs(rbt_ctx *c, int kind, size_t gs, const RbtExpertDev *jobs, const RbtExpertDev &single, int njobs,
                 const int *njobs_dev, const float *x, const int *x_index, size_t d, size_t i, float *h, float *y,
                 hipEvent_t *mark = nullptr, const RbtAct &act = RbtAct{}) {
  const bool fast_gu = rbt::decode_shape_ok(d, kind, gs) && ((uintptr_t)x % 16 == 0);
  const bool fast_dn = rbt::decode_shape_ok(i, kind, gs);
  if (fast_gu && fast_dn && rbt::gu_act_ok(d, kind, gs)) {
    // gate/up and act(g, u) into h in one launch, down from h
    HIP_OK(c, rbt::launch_gu_act(*c, kind, jobs, single, njobs, njobs_dev, x, x_index, (long)d, (int)d, (int)i, h,
                                 act));
    if (mark) {
      HIP_OK(c, hipEventRecord(mark[0], c->stream));
      HIP_OK(c, hipEventRecord(mark[1], c->stream));
    }
    HIP_OK(c, rbt::launch_decode(*c, rbt::DECODE_DOWN, kind, jobs, single, njobs, njobs_dev, h, nullptr, (long)i,
                                 (int)i, (int)d, y, (long)d));
    return RBT_OK;
  }
  if (fast_gu && fast_dn) {
    // stacked gate|up dot products (column parts) into gu, act(g, u) into h, down from h.
    const int parts = rbt::decode_parts((int)d);
    const long gs_stride = (long)(2 * parts * i);
    float *gu;
    RBT_TRY(scratch_t(c, SC_GU, (size_t)njobs * gs_stride, &gu));
    HIP_OK(c, rbt::launch_decode(*c, rbt::DECODE_STACKED, kind, jobs, single, njobs, njobs_dev, x, x_index, (long)d,
                                 (int)d, (int)(2 * i), gu, gs_stride, parts));
    if (mark) {
      HIP_OK(c, hipEventRecord(mark[0], c->stream));
      HIP_OK(c, hipEventRecord(mark[1], c->stream));
    }
    HIP_OK(c, rbt::launch_swiglu(*c, gu, gs_stride, (int)i, njobs, njobs_dev, parts, h, act));
    HIP_OK(c, rbt::launch_decode(*c, rbt::DECODE_DOWN, kind, jobs, single, njobs, njobs_dev, h, nullptr, (long)i,
                                 (int)i, (int)d, y, (long)d));
    return RBT_OK;
  }
  HIP_OK(c, rbt::launch_pair_generic(*c, true, kind, gs, jobs, single, njobs, njobs_dev, x, x_index, (long)d, (int)d,
                                     (int)i, h, (long)i, act));
  if (mark) {
    HIP_OK(c, hipEventRecord(mark[0], c->stream));
    HIP_OK(c, hipEventRecord(mark[1], c->stream));
  }
  if (fast_dn)
    HIP_OK(c, rbt::launch_decode(*c, rbt::DECODE_DOWN, kind, jobs, single, njobs, njobs_dev, h, nullptr, (long)i,
                                 (int)i, (int)d, y, (long)d));
  else
    HIP_OK(c, rbt::launch_pair_generic(*c, false, kind, gs, jobs, single, njobs, njobs_dev, h, nullptr, (long)i,
                                       (int)i, (int)d, y, (long)d));
  return RBT_OK;
}

// Rebuilds the layer's device table of resident experts after the pool or the layer changed. The
// host image and the device table were sized when the layer was set, so this allocates nothing.
int refresh_table(rbt_ctx *c, uint32_t layer, Layer &L) {
  size_t E = L.desc.n_experts;
  if (!L.dirty && L.table_n == E) return RBT_OK;
  if (L.h_table.size() != E || L.table_n != E || !L.d_table)
    return fail(c, RBT_E_INVALID, "layer %u: expert table not sized", layer);
  RbtExpertDev *t = L.h_table.data();
  memset(t, 0, E * sizeof(RbtExpertDev));
  L.routed_kind = -1;
  for (auto &kv : c->pool) {
    if ((uint32_t)(kv.first >> 32) != layer) continue;
    uint32_t eid = (uint32_t)kv.first;
    if (eid >= E) continue;
    int kind;
    size_t gs;
    RBT_TRY(slot_view(c, &kv.second.slot, L.desc.hidden, L.desc.moe_inter, &t[eid], &kind, &gs));
    if (L.routed_kind >= 0 && (kind != L.routed_kind || gs != L.routed_gs))
      return fail(c, RBT_E_UNSUPPORTED, "layer %u: routed experts mix weight formats", layer);
    L.routed_kind = kind;
    L.routed_gs = gs;
  }
  HIP_OK(c, hipMemcpyAsync(L.d_table, t, E * sizeof(RbtExpertDev), hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  L.dirty = false;
  return RBT_OK;
}

// The latent MoE's table: the layer's pool slots viewed at (mh, moe_inter), rebuilt only after the
// pool or the layer changed or for another width, so a steady-state call copies nothing.
int refresh_latent(rbt_ctx *c, uint32_t layer, Layer &L, size_t mh) {
  const size_t E = L.desc.n_experts;
  if (!L.lat_dirty && L.lat_mh == mh) return RBT_OK;
  std::vector<RbtExpertDev> t(E + 1);
  memset(t.data(), 0, (E + 1) * sizeof(RbtExpertDev));
  int kind = -1;
  size_t gs = 0;
  for (auto it = c->pool.lower_bound((uint64_t)layer << 32); it != c->pool.end() && (uint32_t)(it->first >> 32) == layer;
       ++it) {
    const uint32_t eid = (uint32_t)it->first;
    if (eid >= E) continue;
    int kd;
    size_t g;
    RBT_TRY(slot_view(c, &it->second.slot, mh, L.desc.moe_inter, &t[eid], &kd, &g));
    if (kind >= 0 && (kd != kind || g != gs)) return fail(c, RBT_E_UNSUPPORTED, "layer %u: experts mix formats", layer);
    kind = kd;
    gs = g;
  }
  if (kind < 0) return fail(c, RBT_E_NOT_RESIDENT, "layer %u has no resident experts", layer);
  if (L.lat_cap < E + 1) {
    if (L.d_lat) HIP_OK(c, hipFree(L.d_lat));
    L.d_lat = nullptr;
    L.lat_cap = 0;
    HIP_OK(c, hipMalloc(&L.d_lat, (E + 1) * sizeof(RbtExpertDev)));
    L.lat_cap = E + 1;
  }
  HIP_OK(c, hipMemcpyAsync(L.d_lat, t.data(), (E + 1) * sizeof(RbtExpertDev), hipMemcpyHostToDevice, c->stream));
  HIP_OK(c, hipStreamSynchronize(c->stream));
  L.lat_kind = kind;
  L.lat_gs = gs;
  L.lat_mh = mh;
  L.lat_dirty = false;
  return RBT_OK;
}

void free_layer(Layer &L) {
  for (void *p : L.owned) (void)hipFree(p);
  L.owned.clear();
  if (L.d_table) (void)hipFree(L.d_table);
  L.d_table = nullptr;
  L.table_n = 0;
  if (L.d_shared) (void)hipFree(L.d_shared);
  L.d_shared = nullptr;
  if (L.d_lat) (void)hipFree(L.d_lat);
  L.d_lat = nullptr;
  L.lat_cap = 0;
}

int dev_copy_of(rbt_ctx *c, Layer &L, const void *host, size_t bytes, const void **out) {
  if (!host) {
    *out = nullptr;
    return RBT_OK;
  }
  void *p;
  if (hipMalloc(&p, bytes) != hipSuccess) {
    (void)hipGetLastError();
    return fail(c, RBT_E_NOMEM, "hipMalloc(%zu) failed", bytes);
  }
  L.owned.push_back(p);
  HIP_OK(c, hipMemcpy(p, host, bytes, hipMemcpyHostToDevice));
  *out = p;
  return RBT_OK;
}

int layer_set(rbt_ctx *c, uint32_t layer, const rbt_moe_layer_desc *d, bool device) {
  if (!c || !d) return fail(c, RBT_E_INVALID, "null argument");
  if (d->family < RBT_FAMILY_QWEN38 || d->family > RBT_FAMILY_KIMI_K3)
    return fail(c, RBT_E_INVALID, "unknown family %d", (int)d->family);
  if (d->hidden == 0 || d->moe_inter == 0 || d->n_experts == 0 || d->topk == 0 || !d->router)
    return fail(c, RBT_E_INVALID, "layer %u: empty dimension or null router", layer);
  if (d->n_experts > 2048) return fail(c, RBT_E_UNSUPPORTED, "n_experts > 2048");
  if (std::min(d->topk, d->n_experts) > 64) return fail(c, RBT_E_UNSUPPORTED, "topk > 64");
  if (d->n_group > 1 && (d->n_experts % d->n_group != 0 || d->n_group > 64))
    return fail(c, RBT_E_INVALID, "n_experts %% n_group != 0 or n_group > 64");
  Layer &L = c->layers[layer];
  free_layer(L);
  L = Layer{};
  L.desc = *d;
  size_t E = d->n_experts, H = d->hidden;
  if (!device) {
    const void *p;
    RBT_TRY(dev_copy_of(c, L, d->router, E * H * 4, &p));
    L.desc.router = (const float *)p;
    RBT_TRY(dev_copy_of(c, L, d->router_bias, E * 4, &p));
    L.desc.router_bias = (const float *)p;
    RBT_TRY(dev_copy_of(c, L, d->logit_bias, E * 4, &p));
    L.desc.logit_bias = (const float *)p;
    RBT_TRY(dev_copy_of(c, L, d->shared_gate, H * 4, &p));
    L.desc.shared_gate = (const float *)p;
  }
  if (d->has_shared) {
    size_t sd, si;
    slot_dims(&d->shared, &sd, &si);
    if (sd != H) return fail(c, RBT_E_SHAPE, "shared expert hidden %zu != %zu", sd, H);
    if (!device) {
      void *p;
      size_t nb = slot_bytes(&d->shared);
      if (hipMalloc(&p, nb) != hipSuccess) {
        (void)hipGetLastError();
        return fail(c, RBT_E_NOMEM, "hipMalloc(%zu) failed", nb);
      }
      L.owned.push_back(p);
      RBT_TRY(upload_slot(c, &d->shared, (uint8_t *)p, &L.desc.shared));
      HIP_OK(c, hipStreamSynchronize(c->stream));
    }
    int kind;
    size_t gs;
    RBT_TRY(slot_view(c, &L.desc.shared, H, si, &L.h_shared, &kind, &gs));
    L.shared_kind = kind;
    L.shared_gs = gs;
    L.shared_inter = si;
    HIP_OK(c, hipMalloc(&L.d_shared, sizeof(RbtExpertDev)));
    HIP_OK(c, hipMemcpy(L.d_shared, &L.h_shared, sizeof(RbtExpertDev), hipMemcpyHostToDevice));
  } else {
    HIP_OK(c, hipMalloc(&L.d_shared, sizeof(RbtExpertDev)));
    HIP_OK(c, hipMemset(L.d_shared, 0, sizeof(RbtExpertDev)));
  }
  // the table of resident experts: sized here, refreshed (without allocating) after pool changes
  L.h_table.assign(E, RbtExpertDev{});
  HIP_OK(c, hipMalloc(&L.d_table, E * sizeof(RbtExpertDev)));
  L.table_n = E;
  L.set = true;
  L.dirty = true;
  L.lat_dirty = true;
  return RBT_OK;
}

int pool_insert(rbt_ctx *c, uint32_t layer, const rbt_expert_slot &slot, void *alloc, size_t bytes) {
  uint64_t key = ((uint64_t)layer << 32) | slot.eid;
  auto it = c->pool.find(key);
  if (it != c->pool.end()) {
    HIP_OK(c, hipStreamSynchronize(c->stream));
    if (it->second.alloc) HIP_OK(c, hipFree(it->second.alloc));
    c->pool.erase(it);
  }
  PoolEntry &e = c->pool[key];
  e.slot = slot;
  e.alloc = alloc;
  e.bytes = bytes;
  auto lit = c->layers.find(layer);
  if (lit != c->layers.end()) lit->second.dirty = lit->second.lat_dirty = true;
  return RBT_OK;
}

hipEvent_t take_event(rbt_ctx *c) {
  if (!c->ev_free.empty()) {
    hipEvent_t e = c->ev_free.back();
    c->ev_free.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) {
    (void)hipGetLastError();
    return nullptr;
  }
  return e;
}

// Prefill (several tokens, MXFP4): grouping into per-expert segments, x -> bf16, grouped gate/up
// GEMM with SiLU, grouped down GEMM, ordered combine. ev (profiling): event 1 after the grouping,
// 2..5 recorded by the two GEMM dispatches (start, end each).
int prefill_dev(rbt_ctx *c, Layer &L, const float *x, int S, int k, int E, int H, int I, const int32_t *ids,
                const float *wts, const float *shs, int *ptok, int *tpair, float *tw, float *h, float *yy, bool gated,
                float *out, hipEvent_t *ev) {
  const rbt_moe_layer_desc &D = L.desc;
  const int has_shared = D.has_shared ? 1 : 0;
  const long W = (S + 31) / 32;
  const long max_tiles = rbt::prefill_max_tiles(S, k, E, has_shared);
  // one scratch block: bits [E*W], pc [E*W], segs [PG_MAXE], tiles [max_tiles], ntiles
  const size_t off_pc = align256((size_t)E * W * 4), off_segs = off_pc + align256((size_t)E * W * 4);
  const size_t off_tiles = off_segs + align256(sizeof(rbt::PSeg) * rbt::PG_MAXE);
  const size_t off_nt = off_tiles + align256(sizeof(rbt::PTile) * (size_t)max_tiles);
  void *blk;
  RBT_TRY(scratch(c, SC_PGRP, off_nt + 256, &blk));
  char *b = static_cast<char *>(blk);
  uint32_t *bits = reinterpret_cast<uint32_t *>(b), *pc = reinterpret_cast<uint32_t *>(b + off_pc);
  rbt::PSeg *segs = reinterpret_cast<rbt::PSeg *>(b + off_segs);
  rbt::PTile *tiles = reinterpret_cast<rbt::PTile *>(b + off_tiles);
  int *ntiles = reinterpret_cast<int *>(b + off_nt);
  __bf16 *xb;
  RBT_TRY(scratch_t(c, SC_XB, (size_t)S * H, &xb));
  __bf16 *hb = reinterpret_cast<__bf16 *>(h);  // [S*k + S, I] bf16 fits the fp32 h scratch
  int *dflags = c->d_flags;
  HIP_OK(c, rbt::launch_pgroup(*c, ids, wts, S, k, E, has_shared, L.d_table, bits, pc, segs, tiles, ntiles, ptok,
                               tpair, tw, dflags + FLAG_ERR, dflags + FLAG_UNIQ));
  HIP_OK(c, rbt::launch_to_bf16(*c, x, (long)S * H, xb));
  if (ev) HIP_OK(c, hipEventRecord(ev[1], c->stream));
  if (ev) c->t_start = ev[2], c->t_stop = ev[3];
  const hipError_t e1 = rbt::launch_pgateup(*c, tiles, ntiles, max_tiles, segs, L.d_table, L.d_shared, ptok, xb, S, H,
                                            I, hb);
  c->t_start = c->t_stop = nullptr;
  HIP_OK(c, e1);
  if (ev) c->t_start = ev[4], c->t_stop = ev[5];
  const hipError_t e2 = rbt::launch_pdown(*c, tiles, ntiles, max_tiles, segs, L.d_table, L.d_shared, hb, I, H, yy);
  c->t_start = c->t_stop = nullptr;
  HIP_OK(c, e2);
  HIP_OK(c, rbt::launch_combine(*c, yy, S, k, H, tpair, tw, shs, has_shared, gated ? 1 : 0, out));
  return RBT_OK;
}

constexpr int DECODE_MAX_S = 16;  // tokens per call up to which MXFP4 layers keep fp32 accuracy

// A few tokens (MXFP4, fp32-accurate): grouped by expert as in prefill, every unique expert's
// weights streamed once for all its tokens, each token's activation as three exact bf16 parts.
// xb3: the tokens' three-part split when the router launch already wrote it (else null: split here).
int decode_grouped_dev(rbt_ctx *c, Layer &L, const float *x, int S, int k, int E, int H, int I, const int32_t *ids,
                       const float *wts, const float *shs, int *ptok, int *tpair, float *tw, float *h, float *yy,
                       bool gated, float *out, hipEvent_t *ev, __bf16 *xb3_done = nullptr) {
  const rbt_moe_layer_desc &D = L.desc;
  const int has_shared = D.has_shared ? 1 : 0;
  const long W = (S + 31) / 32;
  const long max_tiles = rbt::dgemm_max_tiles(S, k, E, has_shared);
  const size_t off_pc = align256((size_t)E * W * 4), off_segs = off_pc + align256((size_t)E * W * 4);
  const size_t off_tiles = off_segs + align256(sizeof(rbt::PSeg) * rbt::PG_MAXE);
  const size_t off_nt = off_tiles + align256(sizeof(rbt::PTile) * (size_t)max_tiles);
  void *blk;
  RBT_TRY(scratch(c, SC_PGRP, off_nt + 256, &blk));
  char *b = static_cast<char *>(blk);
  uint32_t *bits = reinterpret_cast<uint32_t *>(b), *pc = reinterpret_cast<uint32_t *>(b + off_pc);
  rbt::PSeg *segs = reinterpret_cast<rbt::PSeg *>(b + off_segs);
  rbt::PTile *tiles = reinterpret_cast<rbt::PTile *>(b + off_tiles);
  int *ntiles = reinterpret_cast<int *>(b + off_nt);
  __bf16 *xb3 = xb3_done;
  if (!xb3) RBT_TRY(scratch_t(c, SC_XB, (size_t)3 * S * H, &xb3));
  __bf16 *hb3 = reinterpret_cast<__bf16 *>(h);  // [3 (S*k + S), I] bf16 fits the fp32 h scratch (2 I floats per pair)
  int *dflags = c->d_flags;
  HIP_OK(c, rbt::launch_pgroup(*c, ids, wts, S, k, E, has_shared, L.d_table, bits, pc, segs, tiles, ntiles, ptok,
                               tpair, tw, dflags + FLAG_ERR, dflags + FLAG_UNIQ, rbt::PD_TCH));
  if (!xb3_done) HIP_OK(c, rbt::launch_split3(*c, x, S, H, xb3));
  if (ev) HIP_OK(c, hipEventRecord(ev[1], c->stream));
  if (ev) c->t_start = ev[2], c->t_stop = ev[3];
  const hipError_t e1 = rbt::launch_dgateup(*c, tiles, ntiles, segs, L.d_table, L.d_shared, ptok, xb3, S, H, I, hb3);
  c->t_start = c->t_stop = nullptr;
  HIP_OK(c, e1);
  if (ev) c->t_start = ev[4], c->t_stop = ev[5];
  const hipError_t e2 = rbt::launch_ddown(*c, tiles, ntiles, segs, L.d_table, L.d_shared, hb3, I, H, yy);
  c->t_start = c->t_stop = nullptr;
  HIP_OK(c, e2);
  HIP_OK(c, rbt::launch_combine(*c, yy, S, k, H, tpair, tw, shs, has_shared, gated ? 1 : 0, out));
  return RBT_OK;
}

// accumulate: out += the layer's output (x and out must not overlap). The one-token down launch adds
// in its own store; the other paths write the output to a scratch and add it after.
// norm_w (the MoE sublayer): the layer's input is rmsnorm_1p(x, norm_w, eps) (qwen38/ops.rs:25-33),
// computed inside the one-token router launch where it runs, else by a norm launch first.
int moe_forward_dev(rbt_ctx *c, uint32_t layer, const float *x, size_t s, float *out, int32_t *ids_out,
                    float *w_out, bool accumulate = false, const float *norm_w = nullptr, float eps = 0.0f) {
  auto lit = c->layers.find(layer);
  if (lit == c->layers.end() || !lit->second.set) return fail(c, RBT_E_INVALID, "layer %u not set", layer);
  Layer &L = lit->second;
  if (s == 0) return RBT_OK;
  if (!x || !out) return fail(c, RBT_E_INVALID, "null x or out");
  if (s > 65536) return fail(c, RBT_E_UNSUPPORTED, "more than 65536 tokens per call");
  RBT_TRY(refresh_table(c, layer, L));
  const rbt_moe_layer_desc &D = L.desc;
  const int S = (int)s, E = (int)D.n_experts, H = (int)D.hidden, I = (int)D.moe_inter;
  const int k = (int)std::min(D.topk, D.n_experts);
  if (L.routed_kind < 0) return fail(c, RBT_E_NOT_RESIDENT, "layer %u has no resident experts", layer);
  const bool qwen = D.family == RBT_FAMILY_QWEN38;
  const bool gated = qwen && D.has_shared && D.shared_gate;
  const int erows = E + (gated ? 1 : 0);
  const int P = S * k;
  const int npairs = P + (D.has_shared ? S : 0);
  const float *xraw = x;
  float *xn = nullptr;
  if (norm_w) {
    RBT_TRY(scratch_t(c, SC_NRM, (size_t)S * H, &xn));
    x = xn;  // the layer's input from here on (written before the first launch that reads it)
  }

  double *mid, *bnd;
  int32_t *ids;
  float *wts, *shs, *tw, *h, *yy;
  RbtExpertDev *pjob;
  int *ptok, *tpair;
  RBT_TRY(scratch_t(c, SC_MID, (size_t)S * erows, &mid));
  RBT_TRY(scratch_t(c, SC_BND, (size_t)S * erows, &bnd));
  RBT_TRY(scratch_t(c, SC_IDS, (size_t)P, &ids));
  RBT_TRY(scratch_t(c, SC_WTS, (size_t)P, &wts));
  RBT_TRY(scratch_t(c, SC_SHS, (size_t)S, &shs));
  // k_group always writes the S shared-expert pair slots after the P routed ones; one token may use
  // k + D1_KX routed slots with the shared expert after them (a deferred router decision)
  const size_t pslots = S == 1 ? std::max((size_t)(P + S), (size_t)(k + rbt::D1_KX + 1)) : (size_t)(P + S);
  RBT_TRY(scratch_t(c, SC_PJOB, pslots, &pjob));
  RBT_TRY(scratch_t(c, SC_PTOK, pslots, &ptok));
  RBT_TRY(scratch_t(c, SC_TPAIR, (size_t)P, &tpair));
  RBT_TRY(scratch_t(c, SC_TW, (size_t)P, &tw));
  size_t hi = std::max((size_t)I, L.shared_inter);
  // 2 * hi floats per pair: fp32 h for the GEMV path, or three bf16 parts (1.5 * I) for the MFMA path
  RBT_TRY(scratch_t(c, SC_H, pslots * hi * 2, &h));
  RBT_TRY(scratch_t(c, SC_YY, (size_t)npairs * H, &yy));
  int *dflags = c->d_flags;

  // profiling events: [0] start, [1] routing done, [2, 3] gate/up kernel, [4, 5] down kernel,
  // [6] end (the MFMA kernels record their own start and end)
  std::array<hipEvent_t, 7> ev{};
  if (c->prof) {
    for (auto &e : ev) e = take_event(c);
    for (auto &e : ev)
      if (!e) return fail(c, RBT_E_HIP, "hipEventCreate failed");
    HIP_OK(c, hipEventRecord(ev[0], c->stream));
  }
  rbt::RouterArgs ra{D.family, E,          erows,          k,     H, S, D.logit_bias, D.router_bias, D.norm_topk,
                     D.routed_scale, (int)D.n_group, (int)D.topk_group, x, D.router};
  // one token: the selection kernel writes the job table itself; several: k_group afterwards
  rbt::GroupArgs ga{L.d_table, L.d_shared, pjob, ptok, tpair, tw, dflags + FLAG_ERR};
  const bool grp_in_select = S == 1 && !(D.n_group > 1 && D.family != RBT_FAMILY_QWEN38);
  const bool merge = D.has_shared && L.shared_kind == L.routed_kind && L.shared_gs == L.routed_gs &&
                     L.shared_inter == (size_t)I;
  if (merge) ga.shv = L.h_shared;
  // MXFP4 decode shapes run on the matrix cores: gate/up with SiLU, then down with the ordered
  // combine fused in (out written directly).
  const bool mfma = (merge || !D.has_shared) && rbt::xgemm_ok(L.routed_kind, H, I, S, k, D.has_shared) &&
                    ((uintptr_t)x % 16 == 0);
  // One token: the balanced gate/up covers the routed pairs, and the shared expert's gate/up runs in
  // the router launch (it does not depend on the routing).
  const bool gu1 = mfma && S == 1 && (long)k * (I / 4) >= 4L * c->num_cu;
  const bool sh_in_select = gu1 && D.has_shared && grp_in_select;
  rbt::SharedGateUp sgu{L.d_shared, x, H, I, nullptr};
  const float *sgate = gated ? D.shared_gate : nullptr;
  // One token on the matrix cores: the down launch takes a compact job list (the winners in rank
  // order, then the shared expert) and fuses the ordered combine.
  const int kk = std::min(k, E);
  const bool dn1 = gu1 && grp_in_select && rbt::xdown1_ok(kk + (D.has_shared ? 1 : 0), (size_t)I);
  // ... and with the three-launch decode, the router launch only computes the logits (and streams
  // the shared expert's gate/up) and every gate/up workgroup selects for itself; a decision that
  // needs exact folds takes up to k + D1_KX routed slots, the shared expert the one after.
  const bool r1 = dn1 && rbt::router1_ok(ra, c->num_cu, sh_in_select ? &sgu : nullptr) &&
                  (uintptr_t)(sgate ? sgate : x) % 16 == 0;
  float *dst = out;
  if (accumulate && !dn1) RBT_TRY(scratch_t(c, SC_SUB, (size_t)S * H, &dst));
  const int sh_slot = r1 ? k + rbt::D1_KX : k;
  sgu.hp = reinterpret_cast<__bf16 *>(h) + (size_t)sh_slot * 3 * I;
  RbtExpertDev *djob = nullptr;
  int *dslot = nullptr;
  if (dn1) {
    RBT_TRY(scratch_t(c, SC_DJOB, (size_t)(kk + 1), &djob));
    RBT_TRY(scratch_t(c, SC_DSLOT, (size_t)(kk + 1), &dslot));
    ga.down_job = djob;
    ga.down_slot = dslot;
    ga.shared_slot = sh_slot;
  }
  float *rec = nullptr;
  // Larger MXFP4 batches (prefill) run as grouped GEMMs on the matrix cores; a few tokens
  // (decode batches) as the fp32-accurate grouped decode GEMMs.
  const bool dgrouped = S > 1 && S <= DECODE_MAX_S && (merge || !D.has_shared) &&
                        rbt::dgemm_ok(L.routed_kind, H, I, (size_t)E, (size_t)k);
  __bf16 *xb3_sel = nullptr;  // the split the batch router's selection writes
  // the sublayer's norm: in the one-token router launch (every workgroup normalises the token for its
  // rows, workgroup 0 writes xn), else as its own launch
  const bool fold_norm = norm_w && r1 && ((uintptr_t)xraw | (uintptr_t)norm_w) % 16 == 0;
  if (norm_w && !fold_norm) HIP_OK(c, rbt::launch_rmsnorm(*c, xraw, norm_w, eps, xn, (size_t)S, (size_t)H, true));
  // One token off the matrix cores (grouped int4, or MXFP4 shapes they do not take): the same three
  // launches with the decode GEMVs. The router rows' key records; the selection in every workgroup of
  // the fused gate/up + activation GEMV (routed pairs, then the shared expert); the down GEMV over the
  // published job list (winners in rank order, then the shared expert) with the ordered combine fused
  // (or the two launches where the fused kernel does not take the shape).
  const bool g1 = S == 1 && !mfma && grp_in_select && (merge || !D.has_shared) && kk == k && !c->prof &&
                  rbt::gu1s_gemv_ok(ra, c->num_cu, L.routed_kind, L.routed_gs, I) &&
                  rbt::decode_shape_ok(I, L.routed_kind, L.routed_gs) && (uintptr_t)(sgate ? sgate : x) % 16 == 0;
  if (g1) {
    RBT_TRY(scratch_t(c, SC_RREC, (size_t)E * rbt::ROUTER1_REC_BYTES / sizeof(float), &rec));
    RBT_TRY(scratch_t(c, SC_DJOB, (size_t)(kk + 1), &djob));
    RBT_TRY(scratch_t(c, SC_DSLOT, (size_t)(kk + 1), &dslot));
    ga.down_job = djob;
    ga.down_slot = dslot;
    ga.shared_slot = k + rbt::D1_KX;
    RbtExpertDev none{};
    HIP_OK(c, rbt::launch_router1_any(*c, ra, mid, bnd, shs, sgate, rec));
    HIP_OK(c, rbt::launch_gu1s_gemv(*c, ra, rec, mid, bnd, ga, ids, wts, dflags + FLAG_AMB, L.routed_kind,
                                    L.routed_gs, I, h, D.has_shared != 0));
    if (rbt::down1c_ok(L.routed_kind, L.routed_gs, kk + (D.has_shared ? 1 : 0), I, H, c->num_cu)) {
      HIP_OK(c, rbt::launch_down1c(*c, L.routed_kind, L.routed_gs, djob, dslot, kk, D.has_shared, h, (long)I, I, H,
                                   tw, shs, gated, dst));
    } else {
      HIP_OK(c, rbt::launch_decode(*c, rbt::DECODE_DOWN, L.routed_kind, djob, none, kk + (D.has_shared ? 1 : 0),
                                   nullptr, h, dslot, (long)I, I, H, yy, (long)H));
      HIP_OK(c, rbt::launch_combine(*c, yy, S, k, H, tpair, tw, shs, D.has_shared, gated, dst));
    }
  } else {
  if (r1) {
    // one token: router logits, key records and the shared gate
    RBT_TRY(scratch_t(c, SC_RREC, (size_t)E * rbt::ROUTER1_REC_BYTES / sizeof(float), &rec));
    rbt::RouterArgs rr = ra;
    if (fold_norm) rr.x = xraw;
    HIP_OK(c, rbt::launch_router1(*c, rr, sgate, mid, bnd, shs, rec, fold_norm ? norm_w : nullptr, eps,
                                  fold_norm ? xn : nullptr));
  } else if (!rbt::router_exact_ok(S, H) && rbt::router_batch_ok(ra) && (uintptr_t)(sgate ? sgate : x) % 16 == 0) {
    // a decode batch: certified intervals for every (row, token), then the per-token selection (whose
    // idle waves split the tokens for the grouped decode GEMMs)
    if (dgrouped && (uintptr_t)x % 16 == 0 && H % 4 == 0) RBT_TRY(scratch_t(c, SC_XB, (size_t)3 * S * H, &xb3_sel));
    HIP_OK(c, rbt::launch_router_batch(*c, ra, sgate, mid, bnd, L.d_table, ids, wts, shs, dflags + FLAG_AMB, xb3_sel));
  } else {
    const bool al16 = ((uintptr_t)x | (uintptr_t)D.router | (uintptr_t)(sgate ? sgate : x)) % 16 == 0;
    if (rbt::router_exact_ok(S, H) && rbt::router_bounded_ok(ra) && al16) {
      // batches: fp64-accurate logits on the matrix cores with a rigorous bound on their distance to
      // the reference's sequential fp32 fold (the selection folds the ambiguous experts exactly)
      void *rs;
      RBT_TRY(scratch(c, SC_RLOG, rbt::router_bounded_scratch(ra, erows), &rs));
      HIP_OK(c, rbt::launch_router_bounded(*c, ra, sgate, mid, bnd, rs));
    } else if (rbt::router_exact_ok(S, H) && al16) {
      // batches: the reference's sequential fp32 logits themselves, then point intervals
      float *lg;
      RBT_TRY(scratch_t(c, SC_RLOG, (size_t)S * erows, &lg));
      HIP_OK(c, rbt::launch_router_logits_exact(*c, x, S, H, D.router, E, sgate, lg));
      HIP_OK(c, rbt::launch_logits_to_mid(*c, lg, (size_t)S * erows, mid, bnd));
    } else {
      HIP_OK(c, rbt::launch_router_logits(*c, x, S, H, D.router, E, sgate, mid, bnd));
    }
    HIP_OK(c, rbt::launch_router_select(*c, ra, mid, bnd, ids, wts, shs, dflags + FLAG_AMB,
                                        grp_in_select ? &ga : nullptr, sh_in_select ? &sgu : nullptr));
  }
  const bool grouped = !dgrouped && !mfma && S > 1 && (merge || !D.has_shared) &&
                       rbt::prefill_ok(L.routed_kind, H, I, (size_t)E, (size_t)k);
  if (dgrouped) {
    RBT_TRY(decode_grouped_dev(c, L, x, S, k, E, H, I, ids, wts, shs, ptok, tpair, tw, h, yy, gated, dst,
                               c->prof ? ev.data() : nullptr, xb3_sel));
  } else if (grouped) {
    RBT_TRY(prefill_dev(c, L, x, S, k, E, H, I, ids, wts, shs, ptok, tpair, tw, h, yy, gated, dst,
                        c->prof ? ev.data() : nullptr));
  } else {
  if (!grp_in_select)
    HIP_OK(c, rbt::launch_group(*c, ids, wts, S, k, E, L.d_table, L.d_shared, pjob, ptok, tpair, tw, dflags + FLAG_ERR,
                                dflags + FLAG_UNIQ));

  RbtExpertDev none{};
  hipEvent_t *mark = c->prof ? &ev[3] : nullptr;
  if (c->prof) HIP_OK(c, hipEventRecord(ev[1], c->stream));
  if (mfma) {
    // h as three bf16 parts per pair (3 * I bf16 = 1.5 * I floats of the h scratch)
    __bf16 *hp = reinterpret_cast<__bf16 *>(h);
    if (c->prof) c->t_start = ev[2], c->t_stop = ev[3];
    // every wave of the balanced grid has work; the shared pair is done when it ran in selection;
    // a deferred router decision is settled by the gate/up launch's extra workgroup
    const hipError_t e2 =
        r1    ? rbt::launch_xgateup1s(*c, ra, rec, mid, bnd, ga, ids, wts, dflags + FLAG_AMB, dflags + FLAG_GUP, I, hp,
                                      D.has_shared != 0)
        : gu1 ? rbt::launch_xgateup1(*c, pjob, sh_in_select ? k : npairs, x, H, I, hp)
              : rbt::launch_xgateup(*c, pjob, ptok, npairs, x, (long)H, H, I, hp);
    c->t_start = c->t_stop = nullptr;
    HIP_OK(c, e2);
    if (c->prof) c->t_start = ev[4], c->t_stop = ev[5];
    // one token: the balanced down over the compact job list (all pairs' h in LDS); batches: a grid
    // of row blocks
    const uint8_t *sh_dd = D.has_shared ? L.h_shared.dd : nullptr;
    const uint8_t *sh_ds = D.has_shared ? (const uint8_t *)L.h_shared.ds : nullptr;
    const hipError_t e3 =
        dn1 && rbt::xdown2_ok(kk + (D.has_shared ? 1 : 0), (size_t)I, H, c->num_cu)
            ? rbt::launch_xdown2(*c, djob, dslot, kk, hp, I, H, tw, shs, D.has_shared, gated, yy, out, accumulate,
                                 sh_dd, sh_ds)
        : dn1 ? rbt::launch_xdown1(*c, djob, dslot, kk, hp, I, H, tw, shs, D.has_shared, gated, out, accumulate,
                                   sh_dd, sh_ds)
              : rbt::launch_xdown(*c, pjob, npairs, hp, I, H, S, k, ptok, tpair, tw, shs, D.has_shared, gated, dst);
    c->t_start = c->t_stop = nullptr;
    HIP_OK(c, e3);
  } else {
    if (c->prof) HIP_OK(c, hipEventRecord(ev[2], c->stream));
    if (merge || !D.has_shared) {
      RBT_TRY(expert_pairs(c, L.routed_kind, L.routed_gs, pjob, none, npairs, nullptr, x, ptok, H, I, h, yy, mark));
    } else {
      RBT_TRY(expert_pairs(c, L.routed_kind, L.routed_gs, pjob, none, P, nullptr, x, ptok, H, I, h, yy, nullptr));
      // shared pairs [P, P+S): h rows at stride shared_inter after the routed block
      float *hs = h + (size_t)P * I;
      RBT_TRY(expert_pairs(c, L.shared_kind, L.shared_gs, pjob + P, none, S, nullptr, x, ptok + P, H, L.shared_inter,
                           hs, yy + (size_t)P * H, nullptr));
      if (c->prof) {
        HIP_OK(c, hipEventRecord(ev[3], c->stream));  // the two expert sets as one gate/up+down phase
        HIP_OK(c, hipEventRecord(ev[4], c->stream));
      }
    }
    if (c->prof) HIP_OK(c, hipEventRecord(ev[5], c->stream));
    HIP_OK(c, rbt::launch_combine(*c, yy, S, k, H, tpair, tw, shs, D.has_shared, gated, dst));
  }
  }
  }
  if (c->prof) {
    HIP_OK(c, hipEventRecord(ev[6], c->stream));
    c->ev_rows.push_back(ev);
    // one-token decode: the experts each phase streamed (the three-launch decode counts its gate/up
    // pairs on the device; prefill: 0, unknown on the host)
    const uint64_t ne = S == 1 ? (uint64_t)npairs : 0;
    c->ev_experts.push_back({S == 1 && !r1 ? ne - (sh_in_select ? 1 : 0) : 0, ne});
  }
  if (dst != out) HIP_OK(c, rbt::launch_add_rows(*c, out, dst, (size_t)S * H));
  if (ids_out)
    HIP_OK(c, hipMemcpyAsync(ids_out, ids, (size_t)P * 4, hipMemcpyDeviceToDevice, c->stream));
  if (w_out) HIP_OK(c, hipMemcpyAsync(w_out, wts, (size_t)P * 4, hipMemcpyDeviceToDevice, c->stream));
  return RBT_OK;
}

int route_dev(rbt_ctx *c, bool softmax, const float *logits, const float *bias, size_t s, size_t n, size_t k,
              int32_t norm_topk, float routed_scale, size_t n_group, size_t topk_group, int32_t *ids, float *w) {
  if (s == 0 || n == 0 || k == 0) return RBT_OK;
  if (!logits || !ids || !w) return fail(c, RBT_E_INVALID, "null argument");
  if (n > 2048) return fail(c, RBT_E_UNSUPPORTED, "more than 2048 experts");
  size_t kk = std::min(k, n);
  if (kk > 64) return fail(c, RBT_E_UNSUPPORTED, "topk > 64");
  if (n_group > 1 && (n % n_group != 0 || n_group > 64)) return fail(c, RBT_E_INVALID, "bad n_group");
  double *mid, *bnd;
  RBT_TRY(scratch_t(c, SC_MID, s * n, &mid));
  RBT_TRY(scratch_t(c, SC_BND, s * n, &bnd));
  HIP_OK(c, rbt::launch_logits_to_mid(*c, logits, s * n, mid, bnd));
  rbt::RouterArgs ra{softmax ? RBT_FAMILY_QWEN38 : RBT_FAMILY_GLM52, (int)n, (int)n, (int)kk, 0, (int)s, nullptr, bias,
                     norm_topk, routed_scale, (int)n_group, (int)topk_group, nullptr, nullptr};
  HIP_OK(c, rbt::launch_router_select(*c, ra, mid, bnd, ids, w, nullptr, nullptr));
  return RBT_OK;
}

// rbt_activation -> the kernels' RbtAct.
int to_act(rbt_ctx *c, const rbt_activation *a, RbtAct *out) {
  *out = RbtAct{};
  if (!a || a->kind == RBT_ACT_SILU) return RBT_OK;
  if (a->kind != RBT_ACT_SITU) return fail(c, RBT_E_INVALID, "activation %d", (int)a->kind);
  // Situ divides by beta (and linear_beta): zero or non-finite values have no defined result
  if (!std::isfinite(a->beta) || a->beta == 0.0f) return fail(c, RBT_E_INVALID, "situ beta %g", (double)a->beta);
  if (a->has_linear_beta && (!std::isfinite(a->linear_beta) || a->linear_beta == 0.0f))
    return fail(c, RBT_E_INVALID, "situ linear_beta %g", (double)a->linear_beta);
  out->kind = 1;
  out->beta = a->beta;
  out->lbeta = a->linear_beta;
  out->has_lb = a->has_linear_beta ? 1 : 0;
  return RBT_OK;
}

int apply_single_dev(rbt_ctx *c, const rbt_expert_slot *slot, const int32_t *ids, const float *w, size_t s, size_t k,
                     const float *x, size_t d, size_t i, const RbtAct &act, float *out) {
  if (!slot || !ids || !w || !x || !out) return fail(c, RBT_E_INVALID, "null argument");
  if (s == 0 || k == 0) return RBT_OK;
  RbtExpertDev v;
  int kind;
  size_t gs;
  RBT_TRY(slot_view(c, slot, d, i, &v, &kind, &gs));
  if (s == 1 && kind == RBT_QT_MXFP4 && k <= 64 && rbt::xexpert1_ok(d, i, c->num_cu) &&
      ((uintptr_t)x | (uintptr_t)v.gd | (uintptr_t)v.ud | (uintptr_t)v.dd) % 16 == 0 &&
      ((uintptr_t)v.gs | (uintptr_t)v.us | (uintptr_t)v.ds) % 4 == 0) {
    // one token: gate/up + act and down + the weighted add, two launches on the matrix cores
    float *hs;
    RBT_TRY(scratch_t(c, SC_H, 2 * i, &hs));  // three bf16 parts of h (1.5 i floats)
    HIP_OK(c, rbt::launch_xexpert1(*c, v, x, (int)d, (int)i, ids, w, (int)k, (int)slot->eid,
                                   reinterpret_cast<__bf16 *>(hs), out, act));
    return RBT_OK;
  }
  int *ptok, *nr;
  float *pw, *h, *yy;
  RBT_TRY(scratch_t(c, SC_PTOK, s, &ptok));
  RBT_TRY(scratch_t(c, SC_TW, s, &pw));
  RBT_TRY(scratch_t(c, SC_FLAGS, 4, &nr));
  RBT_TRY(scratch_t(c, SC_H, s * i, &h));
  RBT_TRY(scratch_t(c, SC_YY, s * d, &yy));
  HIP_OK(c, rbt::launch_single_rows(*c, ids, w, (int)s, (int)k, (int)slot->eid, ptok, pw, nr));
  RBT_TRY(expert_pairs(c, kind, gs, nullptr, v, (int)s, nr, x, ptok, d, i, h, yy, nullptr, act));
  HIP_OK(c, rbt::launch_accumulate(*c, yy, (int)s, (int)d, ptok, pw, nr, out));
  return RBT_OK;
}

// kimi_k3/moe.rs:64-116: route at full width, project down, the routed experts at moe_hidden, the
// optional norm of each summed row, project up.
static int latent_moe_dev(rbt_ctx *c, uint32_t layer, const rbt_latent_moe_desc *lw, const float *x, size_t s,
                          float *out, int32_t *ids_out, float *w_out) {
  auto lit = c->layers.find(layer);
  if (lit == c->layers.end() || !lit->second.set) return fail(c, RBT_E_INVALID, "layer %u not set", layer);
  if (!lw) return fail(c, RBT_E_INVALID, "null latent descriptor");
  if (s == 0) return RBT_OK;
  if (!x || !out) return fail(c, RBT_E_INVALID, "null x or out");
  Layer &Ly = lit->second;
  const rbt_moe_layer_desc &D = Ly.desc;
  const size_t H = D.hidden, MH = lw->moe_hidden, I = D.moe_inter, E = D.n_experts;
  const size_t k = std::min(D.topk, E);
  if (MH == 0 || lw->down_proj.rows != MH || lw->down_proj.cols != H || lw->up_proj.rows != H ||
      lw->up_proj.cols != MH)
    return fail(c, RBT_E_SHAPE, "latent projections must be [moe_hidden, hidden] and [hidden, moe_hidden]");
  if (s > (size_t)INT32_MAX / std::max<size_t>(k, 1)) return fail(c, RBT_E_INVALID, "too many tokens");
  RbtAct act;
  RBT_TRY(to_act(c, &lw->act, &act));
  const int S = (int)s, K = (int)k, P = S * K;
  // the layer's pool slots seen at (moe_hidden, moe_inter), plus a zero job for the shared slots
  RBT_TRY(refresh_latent(c, layer, Ly, MH));
  const int kind = Ly.lat_kind;
  const size_t gs = Ly.lat_gs;
  const RbtExpertDev *table = Ly.d_lat;
  double *mid, *bnd;
  int32_t *ids;
  float *wts, *shs, *tw, *xl, *h, *yy, *routed;
  RbtExpertDev *pjob;
  int *ptok, *tpair;
  RBT_TRY(scratch_t(c, SC_MID, (size_t)S * E, &mid));
  RBT_TRY(scratch_t(c, SC_BND, (size_t)S * E, &bnd));
  RBT_TRY(scratch_t(c, SC_IDS, (size_t)P, &ids));
  RBT_TRY(scratch_t(c, SC_WTS, (size_t)P, &wts));
  RBT_TRY(scratch_t(c, SC_SHS, (size_t)S, &shs));
  // one token may stream k + D1_KX routed pairs (a deferred router decision), each with its h row
  const size_t pslots = S == 1 ? std::max((size_t)(P + S), (size_t)(K + rbt::D1_KX + 1)) : (size_t)(P + S);
  RBT_TRY(scratch_t(c, SC_PJOB, pslots, &pjob));
  RBT_TRY(scratch_t(c, SC_PTOK, pslots, &ptok));
  RBT_TRY(scratch_t(c, SC_TPAIR, (size_t)P, &tpair));
  RBT_TRY(scratch_t(c, SC_TW, (size_t)P, &tw));
  RBT_TRY(scratch_t(c, SC_XL, (size_t)S * MH, &xl));
  RBT_TRY(scratch_t(c, SC_H, pslots * I * 2, &h));
  RBT_TRY(scratch_t(c, SC_YY, (size_t)P * MH, &yy));
  RBT_TRY(scratch_t(c, SC_ROUTED, (size_t)S * MH, &routed));
  int *dflags = c->d_flags;
  // routing of the full-width x (certified logits, exact folds where the order is not certain)
  rbt::RouterArgs ra{D.family, (int)E, (int)E, K, (int)H, S, D.logit_bias, D.router_bias, D.norm_topk,
                     D.routed_scale, (int)D.n_group, (int)D.topk_group, x, D.router};
  const rbt_qt &Dp = lw->down_proj;
  const bool dp_ok = rbt::router_select_dp_ok(ra, Dp.kind, (int)H, (int)MH) &&
                     (Dp.kind != RBT_QT_I4_GROUPED || Dp.group_size == 32) &&
                     ((uintptr_t)Dp.data | (uintptr_t)x) % 16 == 0 && Dp.data && Dp.scale;
  RbtExpertDev none{};
  bool combined = false;  // the down launch wrote the combined rows (routed) itself
  if (kind == RBT_QT_MXFP4 && dp_ok && rbt::router1_latent_ok(ra, c->num_cu, (int)MH, (int)I) &&
      rbt::decode_shape_ok(I, kind, gs)) {
    // One token, MXFP4 experts, as the plain layer's decode: the router rows' key records; the
    // latent down projection; the selection in every workgroup of the gate/up launch (matrix cores,
    // act fused, h in fp32); the down GEMV over the winners' job list (h rows at their pair slots)
    // with the ordered combine fused; then the up projection below.
    RBT_TRY(check_qt(c, &Dp, "matmul"));
    float *rec;
    RbtExpertDev *djob;
    int *dslot;
    RBT_TRY(scratch_t(c, SC_RREC, E * rbt::ROUTER1_REC_BYTES / sizeof(float), &rec));
    RBT_TRY(scratch_t(c, SC_DJOB, (size_t)(K + 1), &djob));
    RBT_TRY(scratch_t(c, SC_DSLOT, (size_t)(K + 1), &dslot));
    rbt::GroupArgs ga{table, table + E, pjob, ptok, tpair, tw, dflags + FLAG_ERR};
    ga.down_job = djob;
    ga.down_slot = dslot;
    if (rbt::router1_proj_ok(ra, c->num_cu, (int)MH, (int)I, Dp.kind, Dp.group_size)) {
      // the router rows and the latent down projection in one launch
      HIP_OK(c, rbt::launch_router1_proj(*c, ra, mid, bnd, shs, rec, (int)MH, (int)I, Dp.kind, Dp.group_size,
                                         Dp.data, Dp.scale, xl));
    } else {
      HIP_OK(c, rbt::launch_router1_latent(*c, ra, mid, bnd, shs, rec, (int)MH, (int)I));
      if (rbt::proj1_ok(Dp.kind, Dp.group_size, (int)H, (int)MH, c->num_cu))
        HIP_OK(c, rbt::launch_proj1(*c, Dp.kind, Dp.group_size, Dp.data, Dp.scale, x, (int)H, (int)MH, xl));
      else
        RBT_TRY(matmul_dev(c, xl, x, &Dp, s));
    }
    HIP_OK(c, rbt::launch_xgateup1s_latent(*c, ra, rec, mid, bnd, ga, ids, wts, dflags + FLAG_AMB, nullptr, xl, (int)MH,
                                           (int)I, h, act));
    if (rbt::down1c_ok(kind, gs, K, (int)I, (int)MH, c->num_cu)) {
      HIP_OK(c, rbt::launch_down1c(*c, kind, gs, djob, dslot, K, 0, h, (long)I, (int)I, (int)MH, tw, nullptr, 0,
                                   routed));
      combined = true;
    } else {
      HIP_OK(c, rbt::launch_decode(*c, rbt::DECODE_DOWN, kind, djob, none, K, nullptr, h, dslot, (long)I, (int)I,
                                   (int)MH, yy, (long)MH));
    }
  } else {
  if (rbt::router_exact_ok(S, (int)H) && ((uintptr_t)x | (uintptr_t)D.router) % 16 == 0) {
    float *lg;
    RBT_TRY(scratch_t(c, SC_RLOG, (size_t)S * E, &lg));
    HIP_OK(c, rbt::launch_router_logits_exact(*c, x, S, (int)H, D.router, (int)E, nullptr, lg));
    HIP_OK(c, rbt::launch_logits_to_mid(*c, lg, (size_t)S * E, mid, bnd));
  } else {
    HIP_OK(c, rbt::launch_router_logits(*c, x, S, (int)H, D.router, (int)E, nullptr, mid, bnd));
  }
  // one token: the selection writes the pair list itself (pair j = slot j)
  const bool grp_in_select = S == 1 && !(D.n_group > 1 && D.family != RBT_FAMILY_QWEN38);
  rbt::GroupArgs ga{table, table + E, pjob, ptok, tpair, tw, dflags + FLAG_ERR};
  const bool dp_fused = grp_in_select && dp_ok;
  if (dp_fused) {
    // one token: the latent down projection streams while the selection runs (one launch)
    RBT_TRY(check_qt(c, &Dp, "matmul"));
    RbtExpertDev pj{};
    pj.dd = (const uint8_t *)Dp.data;
    pj.ds = Dp.scale;
    HIP_OK(c, rbt::launch_router_select_dp(*c, ra, mid, bnd, ids, wts, shs, dflags + FLAG_AMB, ga, pj, Dp.kind,
                                           (int)H, (int)MH, xl));
  } else {
    HIP_OK(c, rbt::launch_router_select(*c, ra, mid, bnd, ids, wts, shs, dflags + FLAG_AMB,
                                        grp_in_select ? &ga : nullptr));
    RBT_TRY(matmul_dev(c, xl, x, &lw->down_proj, s));
  }
  if (!grp_in_select)
    HIP_OK(c, rbt::launch_group(*c, ids, wts, S, K, (int)E, table, table + E, pjob, ptok, tpair, tw,
                                dflags + FLAG_ERR, dflags + FLAG_UNIQ));
  RBT_TRY(expert_pairs(c, kind, gs, pjob, none, P, nullptr, xl, ptok, MH, I, h, yy, nullptr, act));
  }
  if (!combined) HIP_OK(c, rbt::launch_combine(*c, yy, S, K, (int)MH, tpair, tw, shs, 0, 0, routed));
  const rbt_qt &U = lw->up_proj;
  if (S == 1 && rbt::proj1_ok(U.kind, U.group_size, (int)MH, (int)H, c->num_cu) &&
      ((uintptr_t)U.data | (uintptr_t)(lw->norm ? lw->norm : routed)) % 16 == 0) {
    // one token: the up projection with x staged per workgroup (the norm folded in)
    RBT_TRY(check_qt(c, &U, "matmul"));
    HIP_OK(c, rbt::launch_proj1(*c, U.kind, U.group_size, U.data, U.scale, routed, (int)MH, (int)H, out, lw->norm,
                                lw->eps));
  } else if (lw->norm && U.kind != RBT_QT_F32 && rbt::decode_shape_ok(MH, U.kind, U.group_size) &&
      ((uintptr_t)U.data | (uintptr_t)lw->norm) % 16 == 0) {
    // the norm of each summed row inside the up projection's waves, which read the whole row
    RBT_TRY(check_qt(c, &U, "matmul"));
    RbtExpertDev one{};
    one.dd = (const uint8_t *)U.data;
    one.ds = U.scale;
    HIP_OK(c, rbt::launch_decode(*c, rbt::DECODE_NORM, U.kind, nullptr, one, S, nullptr, routed, nullptr, (long)MH,
                                 (int)MH, (int)H, out, (long)H, 1, lw->norm, lw->eps));
  } else {
    if (lw->norm) HIP_OK(c, rbt::launch_rmsnorm(*c, routed, lw->norm, lw->eps, routed, s, MH, false));
    RBT_TRY(matmul_dev(c, out, routed, &lw->up_proj, s));
  }
  if (ids_out) HIP_OK(c, hipMemcpyAsync(ids_out, ids, (size_t)P * 4, hipMemcpyDeviceToDevice, c->stream));
  if (w_out) HIP_OK(c, hipMemcpyAsync(w_out, wts, (size_t)P * 4, hipMemcpyDeviceToDevice, c->stream));
  return RBT_OK;
}

}  // namespace

// ================================================================================================
// C ABI
// ================================================================================================
extern "C" {

int rbt_latent_moe_d(rbt_ctx *c, uint32_t layer, const rbt_latent_moe_desc *lw, const float *x, size_t s,
                     float *out, int32_t *ids_out, float *w_out) {
  if (!c) return RBT_E_INVALID;
  return latent_moe_dev(c, layer, lw, x, s, out, ids_out, w_out);
}

const char *rbt_version(void) { return "rabbit_amd 0.1.0 (gfx950)"; }

// rbt_init has no context to hold its error message; rbt_last_error(NULL) returns this one.
static thread_local std::string g_init_err;

static int init_fail(int code, const char *what, hipError_t e) {
  char buf[256];
  snprintf(buf, sizeof buf, "rbt_init: %s failed: %s (%d)", what, hipGetErrorString(e), (int)e);
  g_init_err = buf;
  (void)hipGetLastError();
  return code;
}

int rbt_init(rbt_ctx **out, int device) {
  if (!out) return RBT_E_INVALID;
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess) return init_fail(RBT_E_HIP, "hipGetDeviceCount", e);
  if (n == 0) return init_fail(RBT_E_HIP, "hipGetDeviceCount (no device)", hipSuccess);
  if (device < 0 || device >= n) return RBT_E_INVALID;
  if ((e = hipSetDevice(device)) != hipSuccess) return init_fail(RBT_E_HIP, "hipSetDevice", e);
  rbt_ctx *c = new rbt_ctx();
  c->device = device;
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) == hipSuccess && prop.multiProcessorCount > 0)
    c->num_cu = prop.multiProcessorCount;
  const char *what = nullptr;
  if ((e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess) what = "hipStreamCreateWithFlags";
  else if ((e = hipMalloc((void **)&c->d_flags, (FLAG_N + rbt::CNT_N) * sizeof(int))) != hipSuccess) what = "hipMalloc";
  else if ((e = hipMemset(c->d_flags, 0, (FLAG_N + rbt::CNT_N) * sizeof(int))) != hipSuccess) what = "hipMemset";
  if (!what) c->d_cnt = reinterpret_cast<unsigned *>(c->d_flags + FLAG_N);
  // the allocation-free entry point's scratch on this device (the device is current)
  if (!what) c->noalloc = noalloc_base(device, &c->noalloc_err);
  if (what) {
    int rc = init_fail(RBT_E_HIP, what, e);
    if (c->d_flags) (void)hipFree(c->d_flags);
    if (c->stream) (void)hipStreamDestroy(c->stream);
    delete c;
    return rc;
  }
  *out = c;
  return RBT_OK;
}

void rbt_destroy(rbt_ctx *c) {
  if (!c) return;
  (void)hipSetDevice(c->device);
  (void)hipStreamSynchronize(c->stream);
  for (auto &kv : c->layers) free_layer(kv.second);
  for (auto &kv : c->pool)
    if (kv.second.alloc) (void)hipFree(kv.second.alloc);
  for (int i = 0; i < SC_N; i++)
    if (c->scratch[i]) (void)hipFree(c->scratch[i]);
  if (c->d_flags) (void)hipFree(c->d_flags);
  for (auto &r : c->ev_rows)
    for (auto e : r) c->ev_free.push_back(e);
  for (auto &r : c->krecs) {
    c->ev_free.push_back(r.start);
    c->ev_free.push_back(r.stop);
  }
  for (auto e : c->ev_free) (void)hipEventDestroy(e);
  (void)hipStreamDestroy(c->stream);
  delete c;
}

const char *rbt_last_error(const rbt_ctx *c) { return c ? c->err.c_str() : g_init_err.c_str(); }

int rbt_sync(rbt_ctx *c) {
  if (!c) return RBT_E_INVALID;
  return sync_and_check(c);
}

void *rbt_stream(rbt_ctx *c) { return c ? (void *)c->stream : nullptr; }

size_t rbt_qt_resident_bytes(const rbt_qt *w) {
  if (!w) return 0;
  // quant.rs:214-228
  switch (w->kind) {
    case RBT_QT_F32: return w->rows * w->cols * 4;
    case RBT_QT_I4_GROUPED:
      return w->group_size ? w->rows * div_ceil(w->cols, 2) + w->rows * div_ceil(w->cols, w->group_size) * 4 : 0;
    case RBT_QT_MXFP4: return w->rows * div_ceil(w->cols, 2) + w->rows * div_ceil(w->cols, 32);
    default: return 0;
  }
}

int rbt_dequant_rows_d(rbt_ctx *c, const rbt_qt *w, size_t row0, size_t nrows, float *out) {
  if (!c) return RBT_E_INVALID;
  RBT_TRY(check_qt(c, w, "dequant"));
  if (row0 + nrows > w->rows) return fail(c, RBT_E_INVALID, "rows [%zu, %zu) out of range", row0, row0 + nrows);
  if (!out) return fail(c, RBT_E_INVALID, "null out");
  HIP_OK(c, rbt::launch_dequant(*c, out, w->kind, w->data, w->scale, w->cols, w->group_size, row0, nrows));
  return RBT_OK;
}

int rbt_dequant_rows(rbt_ctx *c, const rbt_qt *w, size_t row0, size_t nrows, float *out) {
  if (!c) return RBT_E_INVALID;
  RBT_TRY(check_qt(c, w, "dequant"));
  if (row0 + nrows > w->rows) return fail(c, RBT_E_INVALID, "rows [%zu, %zu) out of range", row0, row0 + nrows);
  if (!out) return fail(c, RBT_E_INVALID, "null out");
  void *base;
  size_t nd = qt_data_bytes(*w), ns = qt_scale_bytes(*w);
  RBT_TRY(scratch(c, SC_STAGE, align256(nd) + align256(ns), &base));
  size_t cur = 0;
  rbt_qt d;
  RBT_TRY(upload_qt(c, *w, (uint8_t *)base, &cur, &d));
  float *o;
  RBT_TRY(scratch_t(c, SC_OUT, nrows * w->cols, &o));
  HIP_OK(c, rbt::launch_dequant(*c, o, d.kind, d.data, d.scale, d.cols, d.group_size, row0, nrows));
  HIP_OK(c, hipMemcpyAsync(out, o, nrows * w->cols * 4, hipMemcpyDeviceToHost, c->stream));
  return sync_and_check(c);
}

int rbt_matmul_qt_d(rbt_ctx *c, float *y, const float *x, const rbt_qt *w, size_t s) {
  if (!c) return RBT_E_INVALID;
  if (!y || !x) return fail(c, RBT_E_INVALID, "null y or x");
  return matmul_dev(c, y, x, w, s);
}

int rbt_matmul_qt(rbt_ctx *c, float *y, const float *x, const rbt_qt *w, size_t s) {
  if (!c) return RBT_E_INVALID;
  RBT_TRY(check_qt(c, w, "matmul_qt"));
  if (!y || !x) return fail(c, RBT_E_INVALID, "null y or x");
  if (s == 0) return RBT_OK;
  void *base;
  size_t nd = qt_data_bytes(*w), ns = qt_scale_bytes(*w);
  RBT_TRY(scratch(c, SC_STAGE, align256(nd) + align256(ns), &base));
  size_t cur = 0;
  rbt_qt d;
  RBT_TRY(upload_qt(c, *w, (uint8_t *)base, &cur, &d));
  void *dx;
  float *dy;
  RBT_TRY(stage_in(c, SC_X, x, s * w->cols * 4, &dx));
  RBT_TRY(scratch_t(c, SC_Y, s * w->rows, &dy));
  RBT_TRY(matmul_dev(c, dy, (const float *)dx, &d, s));
  HIP_OK(c, hipMemcpyAsync(y, dy, s * w->rows * 4, hipMemcpyDeviceToHost, c->stream));
  return sync_and_check(c);
}

static rbt_qt make_qt(int kind, size_t rows, size_t cols, const void *data, const void *scale, size_t gs) {
  rbt_qt q;
  q.rows = rows;
  q.cols = cols;
  q.kind = kind;
  q.data = data;
  q.scale = scale;
  q.group_size = gs;
  return q;
}

int rbt_matmul(rbt_ctx *c, float *y, const float *x, const float *w, size_t s, size_t i, size_t o) {
  rbt_qt q = make_qt(RBT_QT_F32, o, i, w, nullptr, 0);
  return rbt_matmul_qt(c, y, x, &q, s);
}
int rbt_matmul_d(rbt_ctx *c, float *y, const float *x, const float *w, size_t s, size_t i, size_t o) {
  rbt_qt q = make_qt(RBT_QT_F32, o, i, w, nullptr, 0);
  return rbt_matmul_qt_d(c, y, x, &q, s);
}
int rbt_matmul_mxfp4(rbt_ctx *c, float *y, const float *x, const uint8_t *data, const uint8_t *bs, size_t s, size_t i,
                     size_t o) {
  rbt_qt q = make_qt(RBT_QT_MXFP4, o, i, data, bs, 32);
  return rbt_matmul_qt(c, y, x, &q, s);
}
int rbt_matmul_mxfp4_d(rbt_ctx *c, float *y, const float *x, const uint8_t *data, const uint8_t *bs, size_t s,
                       size_t i, size_t o) {
  rbt_qt q = make_qt(RBT_QT_MXFP4, o, i, data, bs, 32);
  return rbt_matmul_qt_d(c, y, x, &q, s);
}
int rbt_matmul_i4_grouped(rbt_ctx *c, float *y, const float *x, const uint8_t *q4, const float *scale, size_t gs,
                          size_t s, size_t i, size_t o) {
  rbt_qt q = make_qt(RBT_QT_I4_GROUPED, o, i, q4, scale, gs);
  return rbt_matmul_qt(c, y, x, &q, s);
}
int rbt_matmul_i4_grouped_d(rbt_ctx *c, float *y, const float *x, const uint8_t *q4, const float *scale, size_t gs,
                            size_t s, size_t i, size_t o) {
  rbt_qt q = make_qt(RBT_QT_I4_GROUPED, o, i, q4, scale, gs);
  return rbt_matmul_qt_d(c, y, x, &q, s);
}

int rbt_route_softmax_topk_d(rbt_ctx *c, const float *logits, size_t s, size_t n, size_t k, int32_t *ids, float *w) {
  if (!c) return RBT_E_INVALID;
  return route_dev(c, true, logits, nullptr, s, n, k, 0, 1.0f, 1, 1, ids, w);
}

int rbt_route_sigmoid_topk_d(rbt_ctx *c, const float *logits, const float *bias, size_t s, size_t n, size_t k,
                             int32_t norm_topk, float routed_scale, size_t n_group, size_t topk_group, int32_t *ids,
                             float *w) {
  if (!c) return RBT_E_INVALID;
  return route_dev(c, false, logits, bias, s, n, k, norm_topk, routed_scale, n_group, topk_group, ids, w);
}

static int route_host(rbt_ctx *c, bool softmax, const float *logits, const float *bias, size_t s, size_t n, size_t k,
                      int32_t norm_topk, float routed_scale, size_t n_group, size_t topk_group, int32_t *ids,
                      float *w) {
  if (!c) return RBT_E_INVALID;
  if (s == 0 || n == 0 || k == 0) return RBT_OK;
  if (!logits || !ids || !w) return fail(c, RBT_E_INVALID, "null argument");
  size_t kk = std::min(k, n);
  void *dl, *db = nullptr;
  int32_t *di;
  float *dw;
  RBT_TRY(stage_in(c, SC_X, logits, s * n * 4, &dl));
  if (bias) RBT_TRY(stage_in(c, SC_S, bias, n * 4, &db));
  RBT_TRY(scratch_t(c, SC_IDS_OUT, s * kk, &di));
  RBT_TRY(scratch_t(c, SC_W_OUT, s * kk, &dw));
  RBT_TRY(route_dev(c, softmax, (const float *)dl, (const float *)db, s, n, kk, norm_topk, routed_scale, n_group,
                    topk_group, di, dw));
  HIP_OK(c, hipMemcpyAsync(ids, di, s * kk * 4, hipMemcpyDeviceToHost, c->stream));
  HIP_OK(c, hipMemcpyAsync(w, dw, s * kk * 4, hipMemcpyDeviceToHost, c->stream));
  return sync_and_check(c);
}

int rbt_route_softmax_topk(rbt_ctx *c, const float *logits, size_t s, size_t n, size_t k, int32_t *ids, float *w) {
  return route_host(c, true, logits, nullptr, s, n, k, 0, 1.0f, 1, 1, ids, w);
}

int rbt_route_sigmoid_topk(rbt_ctx *c, const float *logits, const float *bias, size_t s, size_t n, size_t k,
                           int32_t norm_topk, float routed_scale, size_t n_group, size_t topk_group, int32_t *ids,
                           float *w) {
  return route_host(c, false, logits, bias, s, n, k, norm_topk, routed_scale, n_group, topk_group, ids, w);
}

int rbt_unique_experts(const int32_t *ids, size_t s, size_t k, int32_t *uniq) {
  if ((!ids || !uniq) && s * k) return RBT_E_INVALID;
  // glm52/moe.rs:333-344 (host-side; the device pipeline computes the same order in k_group)
  std::vector<int32_t> seen;
  int n = 0;
  for (size_t t = 0; t < s * k; t++) {
    if (std::find(seen.begin(), seen.end(), ids[t]) == seen.end()) {
      seen.push_back(ids[t]);
      uniq[n++] = ids[t];
    }
  }
  return n;
}

int rbt_apply_single_expert_act_d(rbt_ctx *c, const rbt_expert_slot *slot, const int32_t *ids, const float *w,
                                  size_t s, size_t k, const float *x, size_t d, size_t i, const rbt_activation *act,
                                  float *out) {
  if (!c) return RBT_E_INVALID;
  RbtAct a;
  RBT_TRY(to_act(c, act, &a));
  return apply_single_dev(c, slot, ids, w, s, k, x, d, i, a, out);
}

int rbt_apply_single_expert_d(rbt_ctx *c, const rbt_expert_slot *slot, const int32_t *ids, const float *w, size_t s,
                              size_t k, const float *x, size_t d, size_t i, int32_t act, float *out) {
  if (!c) return RBT_E_INVALID;
  if (act != RBT_ACT_SILU) return fail(c, RBT_E_INVALID, "activation %d needs its parameters", (int)act);
  return apply_single_dev(c, slot, ids, w, s, k, x, d, i, RbtAct{}, out);
}

int rbt_apply_single_expert(rbt_ctx *c, const rbt_expert_slot *slot, const int32_t *ids, const float *w, size_t s,
                            size_t k, const float *x, size_t d, size_t i, int32_t act, float *out) {
  if (!c) return RBT_E_INVALID;
  if (act != RBT_ACT_SILU) return fail(c, RBT_E_INVALID, "activation %d needs its parameters", (int)act);
  const rbt_activation silu{RBT_ACT_SILU, 0.0f, 0.0f, 0};
  return rbt_apply_single_expert_act(c, slot, ids, w, s, k, x, d, i, &silu, out);
}

int rbt_apply_single_expert_act(rbt_ctx *c, const rbt_expert_slot *slot, const int32_t *ids, const float *w,
                                size_t s, size_t k, const float *x, size_t d, size_t i, const rbt_activation *act,
                                float *out) {
  if (!c) return RBT_E_INVALID;
  RbtAct a;
  RBT_TRY(to_act(c, act, &a));
  if (!slot || !ids || !w || !x || !out) return fail(c, RBT_E_INVALID, "null argument");
  if (s == 0 || k == 0) return RBT_OK;
  rbt_expert_slot dslot;
  const rbt_expert_slot *use = slot;
  if (!find_pool_slot(c, slot)) {
    RbtExpertDev v;
    int kind;
    size_t gs;
    RBT_TRY(slot_view(c, slot, d, i, &v, &kind, &gs));  // validates before any copy
    void *base;
    RBT_TRY(scratch(c, SC_STAGE, slot_bytes(slot), &base));
    RBT_TRY(upload_slot(c, slot, (uint8_t *)base, &dslot));
    use = &dslot;
  }
  void *dx, *dids, *dw;
  float *dout;
  RBT_TRY(stage_in(c, SC_X, x, s * d * 4, &dx));
  RBT_TRY(stage_in(c, SC_IDS_OUT, ids, s * k * 4, &dids));
  RBT_TRY(stage_in(c, SC_W_OUT, w, s * k * 4, &dw));
  RBT_TRY(scratch_t(c, SC_OUT, s * d, &dout));
  HIP_OK(c, hipMemcpyAsync(dout, out, s * d * 4, hipMemcpyHostToDevice, c->stream));
  RBT_TRY(apply_single_dev(c, use, (const int32_t *)dids, (const float *)dw, s, k, (const float *)dx, d, i, a,
                           dout));
  HIP_OK(c, hipMemcpyAsync(out, dout, s * d * 4, hipMemcpyDeviceToHost, c->stream));
  return sync_and_check(c);
}

int rbt_pool_put(rbt_ctx *c, uint32_t layer, const rbt_expert_slot *h) {
  if (!c) return RBT_E_INVALID;
  if (!h) return fail(c, RBT_E_INVALID, "null slot");
  size_t d, i;
  slot_dims(h, &d, &i);
  RbtExpertDev v;
  int kind;
  size_t gs;
  RBT_TRY(slot_view(c, h, d, i, &v, &kind, &gs));  // byte-length / shape validation
  size_t nb = slot_bytes(h);
  void *p;
  if (hipMalloc(&p, nb) != hipSuccess) {
    (void)hipGetLastError();
    return fail(c, RBT_E_NOMEM, "hipMalloc(%zu) for expert %u failed", nb, h->eid);
  }
  rbt_expert_slot ds;
  int rc = upload_slot(c, h, (uint8_t *)p, &ds);
  if (rc == RBT_OK) rc = hipStreamSynchronize(c->stream) == hipSuccess ? RBT_OK : RBT_E_HIP;
  if (rc != RBT_OK) {
    (void)hipFree(p);
    return rc;
  }
  return pool_insert(c, layer, ds, p, nb);
}

int rbt_pool_put_device(rbt_ctx *c, uint32_t layer, const rbt_expert_slot *s) {
  if (!c) return RBT_E_INVALID;
  if (!s) return fail(c, RBT_E_INVALID, "null slot");
  size_t d, i;
  slot_dims(s, &d, &i);
  RbtExpertDev v;
  int kind;
  size_t gs;
  RBT_TRY(slot_view(c, s, d, i, &v, &kind, &gs));
  for (const void *p : {(const void *)v.gd, (const void *)v.ud, (const void *)v.dd})
    if ((uintptr_t)p % 16) return fail(c, RBT_E_INVALID, "device slot data must be 16-byte aligned");
  return pool_insert(c, layer, *s, nullptr, 0);
}

const rbt_expert_slot *rbt_pool_alloc(rbt_ctx *c, uint32_t layer, uint32_t eid, int32_t kind, size_t d, size_t i,
                                      size_t gs) {
  if (!c) return nullptr;
  if ((kind != RBT_QT_MXFP4 && kind != RBT_QT_I4_GROUPED) || d == 0 || i == 0 ||
      (kind == RBT_QT_I4_GROUPED && gs == 0)) {
    fail(c, RBT_E_INVALID, "rbt_pool_alloc: bad kind or shape");
    return nullptr;
  }
  rbt_expert_slot s{};
  s.eid = eid;
  s.fused = 0;
  s.gate = make_qt(kind, i, d, nullptr, nullptr, kind == RBT_QT_I4_GROUPED ? gs : 0);
  s.up = s.gate;
  s.down = make_qt(kind, d, i, nullptr, nullptr, kind == RBT_QT_I4_GROUPED ? gs : 0);
  size_t nb = slot_bytes(&s);
  void *p;
  if (hipMalloc(&p, nb) != hipSuccess) {
    (void)hipGetLastError();
    fail(c, RBT_E_NOMEM, "hipMalloc(%zu) for expert %u failed", nb, eid);
    return nullptr;
  }
  uint8_t *b = (uint8_t *)p;
  size_t cur = 0;
  for (rbt_qt *q : {&s.gate, &s.up, &s.down}) {
    q->data = b + cur;
    cur += align256(qt_data_bytes(*q));
    q->scale = b + cur;
    cur += align256(qt_scale_bytes(*q));
  }
  if (pool_insert(c, layer, s, p, nb) != RBT_OK) {
    (void)hipFree(p);
    return nullptr;
  }
  return &c->pool[((uint64_t)layer << 32) | eid].slot;
}

// ensure_loaded for MXFP4 experts from safetensors shards (expert_cache.rs:1227-1256): validate all
// six tensors of an expert, allocate its slot, then stream the bytes through two pinned staging
// buffers (pread into one while the other's copy to HBM runs on the context stream).
int rbt_pool_load_mxfp4(rbt_ctx *c, const rbt_shards *sh, int32_t naming, uint32_t layer, const uint32_t *eids,
                        size_t n, size_t hidden, size_t moe_inter) {
  if (!c) return RBT_E_INVALID;
  if (!sh || (!eids && n)) return fail(c, RBT_E_INVALID, "null shards or eids");
  if (naming != RBT_NAMING_QWEN38_MXFP4 && naming != RBT_NAMING_KIMI_K3_MXFP4)
    return fail(c, RBT_E_INVALID, "unknown expert naming %d", naming);
  if (hidden == 0 || moe_inter == 0) return fail(c, RBT_E_INVALID, "zero hidden or moe_inter");
  if (n == 0) return RBT_OK;
  constexpr size_t STAGE = 32u << 20;
  void *stage[2] = {nullptr, nullptr};
  hipEvent_t done[2] = {nullptr, nullptr};
  int rc = RBT_OK;
  auto cleanup = [&]() {
    if (done[0] || done[1]) (void)hipStreamSynchronize(c->stream);
    for (int b = 0; b < 2; b++) {
      if (stage[b]) (void)hipHostFree(stage[b]);
      if (done[b]) (void)hipEventDestroy(done[b]);
    }
  };
  for (int b = 0; b < 2; b++) {
    if (hipHostMalloc(&stage[b], STAGE, hipHostMallocDefault) != hipSuccess ||
        hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess) {
      (void)hipGetLastError();
      cleanup();
      return fail(c, RBT_E_NOMEM, "pinned staging buffers");
    }
  }
  int cur = 0;
  bool pending[2] = {false, false};
  for (size_t j = 0; j < n && rc == RBT_OK; j++) {
    const uint32_t eid = eids[j];
    std::string base[3];
    size_t rows[3], cols[3];
    const char *psuf;
    (void)rbt::mxfp4_specs(naming, layer, eid, hidden, moe_inter, base, rows, cols, &psuf);
    // mxfp4_from_raw's checks on every tensor before anything is allocated
    std::string names[6];
    uint64_t want[6];
    for (int m = 0; m < 3 && rc == RBT_OK; m++) {
      names[2 * m] = base[m] + psuf;
      names[2 * m + 1] = base[m] + ".weight_scale";
      want[2 * m] = (uint64_t)rows[m] * ((cols[m] + 1) / 2);
      want[2 * m + 1] = (uint64_t)rows[m] * ((cols[m] + 31) / 32);
      for (int q = 0; q < 2; q++) {
        rbt_tensor_info ti;
        const int f = rbt_shards_find(sh, names[2 * m + q].c_str(), &ti);
        if (f != RBT_OK) {
          rc = fail(c, f, "%s", rbt_shards_last_error());
          break;
        }
        if (ti.nbytes != want[2 * m + q]) {
          rc = fail(c, RBT_E_SHAPE, "shape mismatch: %s: expected %llu bytes, got %llu", names[2 * m + q].c_str(),
                    (unsigned long long)want[2 * m + q], (unsigned long long)ti.nbytes);
          break;
        }
      }
    }
    if (rc != RBT_OK) break;
    const rbt_expert_slot *slot = rbt_pool_alloc(c, layer, eid, RBT_QT_MXFP4, hidden, moe_inter, 0);
    if (!slot) {
      rc = RBT_E_NOMEM;
      break;
    }
    const rbt_qt *qs[3] = {&slot->gate, &slot->up, &slot->down};
    for (int t = 0; t < 6 && rc == RBT_OK; t++) {
      uint8_t *dst = (uint8_t *)(t % 2 ? qs[t / 2]->scale : qs[t / 2]->data);
      for (uint64_t off = 0; off < want[t] && rc == RBT_OK; off += STAGE) {
        const size_t len = (size_t)std::min<uint64_t>(STAGE, want[t] - off);
        if (pending[cur] && hipEventSynchronize(done[cur]) != hipSuccess) {
          rc = fail(c, RBT_E_HIP, "staging copy failed");
          break;
        }
        const int r = rbt_shards_read_range(sh, names[t].c_str(), off, stage[cur], len);
        if (r != RBT_OK) {
          rc = fail(c, r, "%s", rbt_shards_last_error());
          break;
        }
        if (hipMemcpyAsync(dst + off, stage[cur], len, hipMemcpyHostToDevice, c->stream) != hipSuccess ||
            hipEventRecord(done[cur], c->stream) != hipSuccess) {
          rc = fail(c, RBT_E_HIP, "host-to-device copy of %s", names[t].c_str());
          break;
        }
        pending[cur] = true;
        cur ^= 1;
      }
    }
    if (rc != RBT_OK) {
      // the expert that failed part-way is not left in the pool
      (void)hipStreamSynchronize(c->stream);
      auto it = c->pool.find(((uint64_t)layer << 32) | eid);
      if (it != c->pool.end()) {
        if (it->second.alloc) (void)hipFree(it->second.alloc);
        c->pool.erase(it);
      }
    }
  }
  cleanup();
  if (rc == RBT_OK) HIP_OK(c, hipStreamSynchronize(c->stream));
  return rc;
}

const rbt_expert_slot *rbt_pool_get(rbt_ctx *c, uint32_t layer, uint32_t eid) {
  if (!c) return nullptr;
  auto it = c->pool.find(((uint64_t)layer << 32) | eid);
  return it == c->pool.end() ? nullptr : &it->second.slot;
}

size_t rbt_pool_resident_bytes(rbt_ctx *c) {
  if (!c) return 0;
  size_t n = 0;
  for (auto &kv : c->pool) {
    const rbt_expert_slot &s = kv.second.slot;
    if (s.fused) n += rbt_qt_resident_bytes(&s.gate_up);
    else n += rbt_qt_resident_bytes(&s.gate) + rbt_qt_resident_bytes(&s.up);
    n += rbt_qt_resident_bytes(&s.down);
  }
  return n;
}

int rbt_moe_layer_set(rbt_ctx *c, uint32_t layer, const rbt_moe_layer_desc *d) {
  if (!c) return RBT_E_INVALID;
  return layer_set(c, layer, d, false);
}

int rbt_moe_layer_set_device(rbt_ctx *c, uint32_t layer, const rbt_moe_layer_desc *d) {
  if (!c) return RBT_E_INVALID;
  return layer_set(c, layer, d, true);
}

// ---- token mixers (qwen38/gdn.rs, qwen38/attention.rs) ------------------------------------------
int rbt_gdn_step_d(rbt_ctx *c, const rbt_gdn_desc *d, float *conv_state, float *states, const float *qkv_pre,
                   const float *z, const float *a, const float *b, float *out) {
  if (!c || !d) return RBT_E_INVALID;
  if (!conv_state || !states || !qkv_pre || !z || !a || !b || !out || !d->conv_weight || !d->a_log || !d->dt_bias ||
      !d->norm_weight)
    return fail(c, RBT_E_INVALID, "null GDN buffer");
  const size_t nv = d->n_v_heads, nk = d->n_k_heads, dk = d->head_k_dim, dv = d->head_v_dim, K = d->conv_kernel;
  if (nv == 0 || nk == 0 || dk == 0 || dv == 0 || K == 0 || nv % nk || nv > (1u << 20) || dk > 4096 || dv > 4096 ||
      K > 64)
    return fail(c, RBT_E_INVALID, "bad GDN shape (heads %zu/%zu, dims %zu/%zu, kernel %zu)", nv, nk, dk, dv, K);
  if (!rbt::gdn_ok((int)nv, (int)nk, (int)dk, (int)dv))
    return fail(c, RBT_E_UNSUPPORTED, "GDN head dims %zu x %zu: head_v_dim must be a multiple of 4 dividing 2048 "
                "(at most 512), head_k_dim even and at most 8192 / head_v_dim", dk, dv);
  if ((uintptr_t)states % 16) return fail(c, RBT_E_INVALID, "states must be 16-byte aligned");
  const size_t conv_dim = 2 * nk * dk + nv * dv;
  float *act;
  RBT_TRY(scratch_t(c, SC_MIXA, conv_dim, &act));
  HIP_OK(c, rbt::launch_gdn(*c, conv_state, d->conv_weight, (int)K, states, qkv_pre, z, a, b, d->a_log, d->dt_bias,
                            d->norm_weight, d->eps, (int)nv, (int)nk, (int)dk, (int)dv, act, out));
  return RBT_OK;
}

int rbt_gqa_step_d(rbt_ctx *c, const rbt_gqa_desc *d, float *k_cache, float *v_cache, size_t cap, size_t pos,
                   const float *qg, const float *k, const float *v, float *ctx_out) {
  if (!c || !d) return RBT_E_INVALID;
  if (!k_cache || !v_cache || !qg || !k || !v || !ctx_out || !d->q_norm || !d->k_norm)
    return fail(c, RBT_E_INVALID, "null GQA buffer");
  const size_t nh = d->n_heads, nkv = d->n_kv_heads, hd = d->head_dim;
  if (nh == 0 || nkv == 0 || nh % nkv || hd == 0 || nh > 4096)
    return fail(c, RBT_E_INVALID, "bad GQA shape (heads %zu over %zu kv heads)", nh, nkv);
  if (pos >= cap) return fail(c, RBT_E_INVALID, "position %zu is outside the cache (capacity %zu)", pos, cap);
  if (pos >= (size_t)6144 * 64) return fail(c, RBT_E_UNSUPPORTED, "position %zu (at most 393215)", pos);
  if (!rbt::gqa_ok((int)nh, (int)nkv, (int)hd, (int)d->rope_dim))
    return fail(c, RBT_E_UNSUPPORTED, "GQA shape: head_dim %zu (a multiple of 64, at most 1024), rope_dim %zu, %zu "
                "query heads per kv head (at most 16)", hd, d->rope_dim, nh / nkv);
  if (((uintptr_t)k_cache | (uintptr_t)v_cache) % 16) return fail(c, RBT_E_INVALID, "caches must be 16-byte aligned");
  float *qp, *part;
  RBT_TRY(scratch_t(c, SC_MIXA, nh * hd, &qp));
  RBT_TRY(scratch_t(c, SC_MIXB, rbt::gqa_part_floats((int)nh, (int)nkv, (int)hd, (int)pos + 1), &part));
  HIP_OK(c, rbt::launch_gqa(*c, qg, k, v, (int)nh, (int)nkv, (int)hd, d->q_norm, d->k_norm, d->eps, (int)d->rope_dim,
                            d->theta, d->attn_scale, (int)pos, k_cache, v_cache, qp, part, ctx_out));
  return RBT_OK;
}

int rbt_rmsnorm_d(rbt_ctx *c, float *v, const float *w, size_t s, size_t n, float eps) {
  if (!c) return RBT_E_INVALID;
  if (s == 0 || n == 0) return RBT_OK;
  if (!v || !w) return fail(c, RBT_E_INVALID, "null v or w");
  HIP_OK(c, rbt::launch_rmsnorm(*c, v, w, eps, v, s, n, false));
  return RBT_OK;
}

int rbt_rmsnorm_1p_d(rbt_ctx *c, float *v, const float *w, size_t s, size_t n, float eps) {
  if (!c) return RBT_E_INVALID;
  if (s == 0 || n == 0) return RBT_OK;
  if (!v || !w) return fail(c, RBT_E_INVALID, "null v or w");
  HIP_OK(c, rbt::launch_rmsnorm(*c, v, w, eps, v, s, n, true));
  return RBT_OK;
}

// qwen38/generate.rs:397-413: nrm = rmsnorm_1p(x, post_ln) per row, tmp = moe_forward(nrm), x += tmp.
static int moe_sublayer_dev(rbt_ctx *c, uint32_t layer, float *x, size_t s, const float *post_ln, float eps,
                            int32_t *ids_out, float *w_out) {
  auto lit = c->layers.find(layer);
  if (lit == c->layers.end() || !lit->second.set) return fail(c, RBT_E_INVALID, "layer %u not set", layer);
  if (s == 0) return RBT_OK;
  if (!x || !post_ln) return fail(c, RBT_E_INVALID, "null x or post_ln");
  // x += layer(rmsnorm_1p(x)): the norm rides in the one-token router launch and the residual add
  // in the layer's last store where they can
  RBT_TRY(moe_forward_dev(c, layer, x, s, x, ids_out, w_out, true, post_ln, eps));
  return RBT_OK;
}

int rbt_moe_sublayer_d(rbt_ctx *c, uint32_t layer, float *x, size_t s, const float *post_ln, float eps,
                       int32_t *ids_out, float *w_out) {
  if (!c) return RBT_E_INVALID;
  return moe_sublayer_dev(c, layer, x, s, post_ln, eps, ids_out, w_out);
}

int rbt_moe_sublayer(rbt_ctx *c, uint32_t layer, float *x, size_t s, const float *post_ln, float eps,
                     int32_t *ids_out, float *w_out) {
  if (!c) return RBT_E_INVALID;
  auto lit = c->layers.find(layer);
  if (lit == c->layers.end() || !lit->second.set) return fail(c, RBT_E_INVALID, "layer %u not set", layer);
  if (s == 0) return RBT_OK;
  if (!x || !post_ln) return fail(c, RBT_E_INVALID, "null x or post_ln");
  const rbt_moe_layer_desc &D = lit->second.desc;
  const size_t H = D.hidden, k = std::min(D.topk, D.n_experts);
  void *dx, *dp;
  float *dw;
  int32_t *di;
  RBT_TRY(stage_in(c, SC_X, x, s * H * 4, &dx));
  RBT_TRY(stage_in(c, SC_PLN, post_ln, H * 4, &dp));
  RBT_TRY(scratch_t(c, SC_IDS_OUT, s * k, &di));
  RBT_TRY(scratch_t(c, SC_W_OUT, s * k, &dw));
  RBT_TRY(moe_sublayer_dev(c, layer, (float *)dx, s, (const float *)dp, eps, di, dw));
  HIP_OK(c, hipMemcpyAsync(x, dx, s * H * 4, hipMemcpyDeviceToHost, c->stream));
  if (ids_out) HIP_OK(c, hipMemcpyAsync(ids_out, di, s * k * 4, hipMemcpyDeviceToHost, c->stream));
  if (w_out) HIP_OK(c, hipMemcpyAsync(w_out, dw, s * k * 4, hipMemcpyDeviceToHost, c->stream));
  return sync_and_check(c);
}

int rbt_moe_forward_d(rbt_ctx *c, uint32_t layer, const float *x, size_t s, float *out, int32_t *ids_out,
                      float *w_out) {
  if (!c) return RBT_E_INVALID;
  return moe_forward_dev(c, layer, x, s, out, ids_out, w_out);
}

int rbt_moe_forward_noalloc_d(rbt_ctx *c, uint32_t layer, const float *x, size_t s, float *out, int32_t *ids_out,
                              float *w_out) {
  if (!c) return RBT_E_INVALID;
  if (!c->noalloc)
    return fail(c, RBT_E_HIP, "no allocation-free scratch on device %d: hipGetSymbolAddress: %s", c->device,
                hipGetErrorString(c->noalloc_err));
  // every per-call buffer comes from the device's fixed array; profiling (which creates events) is
  // off for the call
  const bool prof = c->prof, kprof = c->kprof;
  c->prof = c->kprof = false;
  c->arena = c->noalloc;
  c->arena_cap = RBT_NOALLOC_SCRATCH_BYTES;
  c->arena_used = 0;
  memset(c->arena_sz, 0, sizeof c->arena_sz);
  const int rc = moe_forward_dev(c, layer, x, s, out, ids_out, w_out);
  c->arena = nullptr;
  c->arena_cap = c->arena_used = 0;
  c->prof = prof;
  c->kprof = kprof;
  return rc;
}

int rbt_moe_forward(rbt_ctx *c, uint32_t layer, const float *x, size_t s, float *out, int32_t *ids_out,
                    float *w_out) {
  if (!c) return RBT_E_INVALID;
  auto lit = c->layers.find(layer);
  if (lit == c->layers.end() || !lit->second.set) return fail(c, RBT_E_INVALID, "layer %u not set", layer);
  if (s == 0) return RBT_OK;
  if (!x || !out) return fail(c, RBT_E_INVALID, "null x or out");
  const rbt_moe_layer_desc &D = lit->second.desc;
  size_t H = D.hidden, k = std::min(D.topk, D.n_experts);
  void *dx;
  float *dout, *dw;
  int32_t *di;
  RBT_TRY(stage_in(c, SC_X, x, s * H * 4, &dx));
  RBT_TRY(scratch_t(c, SC_OUT, s * H, &dout));
  RBT_TRY(scratch_t(c, SC_IDS_OUT, s * k, &di));
  RBT_TRY(scratch_t(c, SC_W_OUT, s * k, &dw));
  RBT_TRY(moe_forward_dev(c, layer, (const float *)dx, s, dout, di, dw));
  HIP_OK(c, hipMemcpyAsync(out, dout, s * H * 4, hipMemcpyDeviceToHost, c->stream));
  if (ids_out) HIP_OK(c, hipMemcpyAsync(ids_out, di, s * k * 4, hipMemcpyDeviceToHost, c->stream));
  if (w_out) HIP_OK(c, hipMemcpyAsync(w_out, dw, s * k * 4, hipMemcpyDeviceToHost, c->stream));
  return sync_and_check(c);
}

int rbt_profile_enable(rbt_ctx *c, int32_t on) {
  if (!c) return RBT_E_INVALID;
  c->prof = on != 0;
  return RBT_OK;
}

int rbt_profile_read(rbt_ctx *c, rbt_profile *out, int32_t reset) {
  if (!c || !out) return RBT_E_INVALID;
  HIP_OK(c, hipStreamSynchronize(c->stream));
  for (size_t i = 0; i < c->ev_rows.size(); i++) {
    auto &r = c->ev_rows[i];
    float t[4];
    HIP_OK(c, hipEventElapsedTime(&t[0], r[0], r[1]));
    HIP_OK(c, hipEventElapsedTime(&t[1], r[2], r[3]));
    HIP_OK(c, hipEventElapsedTime(&t[2], r[4], r[5]));
    HIP_OK(c, hipEventElapsedTime(&t[3], r[5], r[6]));
    c->acc.router_ms += t[0];
    c->acc.gateup_ms += t[1];
    c->acc.down_ms += t[2];
    c->acc.combine_ms += t[3];
    c->acc.calls += 1;
    c->acc.gateup_experts += c->ev_experts[i][0];
    c->acc.down_experts += c->ev_experts[i][1];
    for (auto e : r) c->ev_free.push_back(e);
  }
  c->ev_rows.clear();
  c->ev_experts.clear();
  HIP_OK(c, hipMemcpy(c->h_flags, c->d_flags, FLAG_N * sizeof(int), hipMemcpyDeviceToHost));
  c->acc.ambiguous = (uint64_t)c->h_flags[FLAG_AMB];
  *out = c->acc;
  out->gateup_experts += (uint64_t)(uint32_t)c->h_flags[FLAG_GUP];  // counted on the device
  if (reset) {
    c->acc = rbt_profile{};
    HIP_OK(c, hipMemset(c->d_flags + FLAG_AMB, 0, sizeof(int)));
    HIP_OK(c, hipMemset(c->d_flags + FLAG_GUP, 0, sizeof(int)));
  }
  return RBT_OK;
}

int rbt_profile_kernels(rbt_ctx *c, int32_t on) {
  if (!c) return RBT_E_INVALID;
  c->kprof = on != 0;
  return RBT_OK;
}

int rbt_profile_kernels_read(rbt_ctx *c, rbt_kernel_stat *out, size_t cap, size_t *n, int32_t reset) {
  if (!c || (cap && !out)) return RBT_E_INVALID;
  HIP_OK(c, hipStreamSynchronize(c->stream));
  for (auto &r : c->krecs) {
    float ms = 0.0f;
    HIP_OK(c, hipEventElapsedTime(&ms, r.start, r.stop));
    auto &a = c->kacc[r.fn];
    a.first += 1;
    a.second += ms;
    c->ev_free.push_back(r.start);
    c->ev_free.push_back(r.stop);
  }
  c->krecs.clear();
  size_t i = 0;
  for (auto &kv : c->kacc) {
    if (i < cap) {
      rbt_kernel_stat &s = out[i];
      s = rbt_kernel_stat{};
      const char *name = hipKernelNameRefByPtr(kv.first, c->stream);
      snprintf(s.name, sizeof s.name, "%s", name ? name : "?");
      s.launches = kv.second.first;
      s.total_ms = kv.second.second;
    }
    i++;
  }
  if (n) *n = i;
  if (reset) c->kacc.clear();
  return RBT_OK;
}

int rbt_synth_mxfp4_d(rbt_ctx *c, uint8_t *data, uint8_t *scale, size_t rows, size_t cols, uint64_t seed,
                      uint32_t lo, uint32_t hi) {
  if (!c) return RBT_E_INVALID;
  if (!data || !scale || lo > hi || hi > 255) return fail(c, RBT_E_INVALID, "bad synth arguments");
  HIP_OK(c, rbt::launch_synth_mxfp4(*c, data, scale, rows, cols, seed, lo, hi));
  return RBT_OK;
}

int rbt_synth_i4g_d(rbt_ctx *c, uint8_t *data, float *scale, size_t rows, size_t cols, size_t gs, uint64_t seed,
                    float lo, float hi) {
  if (!c) return RBT_E_INVALID;
  if (!data || !scale || gs == 0) return fail(c, RBT_E_INVALID, "bad synth arguments");
  HIP_OK(c, rbt::launch_synth_i4g(*c, data, scale, rows, cols, gs, seed, lo, hi));
  return RBT_OK;
}

}  // extern "C"
