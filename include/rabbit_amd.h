/*
 * rabbit_amd.h -- C ABI of the MI355X (gfx950) routed-expert dequant-matmul library.
 *
 * Drop-in boundary for ferrumox/rabbit's routed-expert path: the free functions of
 * src/kernels.rs and src/quant.rs, the routers of src/qwen38/moe.rs and src/glm52/moe.rs,
 * glm52::moe::apply_single_expert, the ExpertCache lookup (src/expert_cache.rs) and the per-family
 * MoE layer (src/qwen38/generate.rs moe_forward, src/glm52/moe.rs moe). Each declaration cites
 * the reference interface it replaces. Citations are path:line inside the reference repository.
 *
 * Conventions (mirroring the reference's slice conventions):
 *  - Plain pointers and sizes; no C++ or torch types cross this boundary.
 *  - Functions without a suffix take HOST buffers borrowed for the call and return after the
 *    result is in the caller's buffer (the reference's &[f32] / &mut [f32] semantics).
 *    Functions with the `_d` suffix take DEVICE pointers, enqueue on the context's stream and
 *    return immediately; rbt_sync() waits.
 *  - matmul-style calls overwrite y; rbt_apply_single_expert accumulates into out;
 *    rbt_moe_forward overwrites out (the reference's moe zeroes out first).
 *  - Nothing aborts or unwinds across the boundary: every call returns RBT_OK (0) or a negative
 *    RBT_E_* status where the reference would panic or return Err; rbt_last_error() describes it.
 *  - A context is not thread-safe (the reference's &mut ExpertCache); use one per host thread.
 *  - Results are deterministic for fixed inputs (no float atomics).
 */
#ifndef RABBIT_AMD_H
#define RABBIT_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes ------------------------------------------------------------------------- */
#define RBT_OK 0
#define RBT_E_INVALID (-1)      /* null pointer, zero/oversized dimension, bad enum */
#define RBT_E_SHAPE (-2)        /* byte length does not match the shape (ModelError::ShapeMismatch,
                                   expert_cache.rs:1245-1256) */
#define RBT_E_HIP (-3)          /* HIP runtime error */
#define RBT_E_NOT_RESIDENT (-4) /* routed expert missing from the pool (ExpertCache::get -> None) */
#define RBT_E_NOMEM (-5)        /* device allocation failed */
#define RBT_E_UNSUPPORTED (-6)  /* valid in the reference but not offered on this path */
#define RBT_E_NOT_FOUND (-7)    /* tensor absent from the checkpoint (SafetensorsError::MissingTensor) */
#define RBT_E_FORMAT (-8)       /* malformed safetensors header or unknown dtype (BadHeader, Json,
                                   UnknownDtype) */
#define RBT_E_IO (-9)           /* file system error (SafetensorsError::Io) */

typedef struct rbt_ctx rbt_ctx;

/* ---- weight containers: QT / QTKind (quant.rs:77-110) --------------------------------------- */
typedef enum {
    RBT_QT_F32 = 0,        /* QTKind::F32:       data f32[rows*cols] */
    RBT_QT_I4_GROUPED = 1, /* QTKind::I4Grouped: data u8[rows*ceil(cols/2)] (value+8, low nibble
                              first), scale f32[rows*ceil(cols/group_size)] (quant.rs:92-100) */
    RBT_QT_MXFP4 = 2       /* QTKind::MxFp4:     data u8[rows*ceil(cols/2)] E2M1 (low nibble first),
                              scale u8[rows*ceil(cols/32)] E8M0 (quant.rs:101-109) */
} rbt_qt_kind;

typedef struct {
    size_t rows, cols;
    int32_t kind;          /* rbt_qt_kind */
    const void *data;
    const void *scale;     /* NULL for RBT_QT_F32 */
    size_t group_size;     /* RBT_QT_I4_GROUPED only */
} rbt_qt;

/* ExpertSlot + GateUp (expert_cache.rs:640-650). fused = 0: gate [i, d] and up [i, d];
 * fused = 1: gate_up [2i, d] (gate rows first). down is [d, i]. */
typedef struct {
    uint32_t eid;
    int32_t fused;
    rbt_qt gate, up, gate_up, down;
} rbt_expert_slot;

/* ---- context ------------------------------------------------------------------------------- */
/* Creates a context on HIP device `device`: its own stream (default priority), scratch, and the
 * HBM-resident expert pool that replaces ExpertCache's storage (expert_cache.rs:1-52). */
int rbt_init(rbt_ctx **out, int device);
void rbt_destroy(rbt_ctx *ctx);
const char *rbt_last_error(const rbt_ctx *ctx);
int rbt_sync(rbt_ctx *ctx);
/* The context's hipStream_t, for callers that enqueue their own work around the `_d` calls. */
void *rbt_stream(rbt_ctx *ctx);
/* Library version string. */
const char *rbt_version(void);

/* ---- quant.rs ------------------------------------------------------------------------------- */
/* QT::resident_bytes (quant.rs:214-228). */
size_t rbt_qt_resident_bytes(const rbt_qt *w);
/* QT::row_f32 (quant.rs:280-341) for rows [row0, row0+nrows): out f32[nrows, cols], the dequantized
 * weights bit-for-bit (e2m1_decode quant.rs:353, e8m0_decode quant.rs:391). */
int rbt_dequant_rows(rbt_ctx *ctx, const rbt_qt *w, size_t row0, size_t nrows, float *out);
int rbt_dequant_rows_d(rbt_ctx *ctx, const rbt_qt *w, size_t row0, size_t nrows, float *out);

/* ---- kernels.rs: y[S,O] = x[S,I] . W^T ---------------------------------------------------- */
/* matmul (kernels.rs:113), f32 weights W[O,I]. */
int rbt_matmul(rbt_ctx *ctx, float *y, const float *x, const float *w, size_t s, size_t i, size_t o);
int rbt_matmul_d(rbt_ctx *ctx, float *y, const float *x, const float *w, size_t s, size_t i, size_t o);
/* matmul_mxfp4 (kernels.rs:233). */
int rbt_matmul_mxfp4(rbt_ctx *ctx, float *y, const float *x, const uint8_t *data,
                     const uint8_t *block_scale, size_t s, size_t i, size_t o);
int rbt_matmul_mxfp4_d(rbt_ctx *ctx, float *y, const float *x, const uint8_t *data,
                       const uint8_t *block_scale, size_t s, size_t i, size_t o);
/* matmul_i4_grouped (kernels.rs:276). */
int rbt_matmul_i4_grouped(rbt_ctx *ctx, float *y, const float *x, const uint8_t *q4, const float *scale,
                          size_t group_size, size_t s, size_t i, size_t o);
int rbt_matmul_i4_grouped_d(rbt_ctx *ctx, float *y, const float *x, const uint8_t *q4, const float *scale,
                            size_t group_size, size_t s, size_t i, size_t o);
/* matmul_qt (kernels.rs:1104): dispatch on w->kind (F32, I4Grouped, MxFp4). The rbt_qt's
 * pointers are host memory for rbt_matmul_qt and device memory for rbt_matmul_qt_d. */
int rbt_matmul_qt(rbt_ctx *ctx, float *y, const float *x, const rbt_qt *w, size_t s);
int rbt_matmul_qt_d(rbt_ctx *ctx, float *y, const float *x, const rbt_qt *w, size_t s);

/* ---- routers -------------------------------------------------------------------------------- */
/* qwen38::moe::route (qwen38/moe.rs:41-76) for s tokens: logits f32[s, n] -> ids i32[s, k'],
 * w f32[s, k'] with k' = min(k, n): top-k by logit (ties -> lower id), softmax over the winners,
 * in descending order. */
int rbt_route_softmax_topk(rbt_ctx *ctx, const float *logits, size_t s, size_t n, size_t k,
                           int32_t *ids, float *w);
int rbt_route_softmax_topk_d(rbt_ctx *ctx, const float *logits, size_t s, size_t n, size_t k,
                             int32_t *ids, float *w);
/* glm52::moe::route (glm52/moe.rs:131-260) for s tokens given router logits: p = sigmoid(logit),
 * select by p + bias (bias may be NULL), lowest id on ties, weight = p, then optional norm_topk
 * (w /= sum + 1e-20) and routed_scale. n_group > 1 selects rank_top_grouped (glm52/moe.rs:214). */
int rbt_route_sigmoid_topk(rbt_ctx *ctx, const float *logits, const float *bias, size_t s, size_t n,
                           size_t k, int32_t norm_topk, float routed_scale, size_t n_group,
                           size_t topk_group, int32_t *ids, float *w);
int rbt_route_sigmoid_topk_d(rbt_ctx *ctx, const float *logits, const float *bias, size_t s, size_t n,
                             size_t k, int32_t norm_topk, float routed_scale, size_t n_group,
                             size_t topk_group, int32_t *ids, float *w);
/* unique_experts (glm52/moe.rs:333-344): ids i32[s, k] -> uniq (first-occurrence order).
 * Returns the count (>= 0) or a negative status. */
int rbt_unique_experts(const int32_t *ids, size_t s, size_t k, int32_t *uniq);

/* ---- one expert ------------------------------------------------------------------------------ */
enum { RBT_ACT_SILU = 0, RBT_ACT_SITU = 1 }; /* Activation::{Silu, Situ} (glm52/moe.rs:49-80) */
/* Activation with its parameters: Situ { beta, linear_beta: Option<f32> } (glm52/moe.rs:49-52). */
typedef struct {
    int32_t kind;            /* RBT_ACT_* */
    float beta;              /* Situ */
    float linear_beta;       /* Situ, when has_linear_beta */
    int32_t has_linear_beta;
} rbt_activation;
/* apply_single_expert (glm52/moe.rs:463-513): the tokens that routed to slot->eid (ids/w are
 * [s, k]) run gate, up, silu(gate)*up, down, and out[t, :] += w * result. Host buffers; the slot's
 * weights may be host (uploaded for the call) or a pool slot from rbt_pool_get (device). */
int rbt_apply_single_expert(rbt_ctx *ctx, const rbt_expert_slot *slot, const int32_t *ids, const float *w,
                            size_t s, size_t k, const float *x, size_t d, size_t i, int32_t activation,
                            float *out);
int rbt_apply_single_expert_d(rbt_ctx *ctx, const rbt_expert_slot *slot, const int32_t *ids,
                              const float *w, size_t s, size_t k, const float *x, size_t d, size_t i,
                              int32_t activation, float *out);
/* The same with a parameterised activation (Situ needs its beta; activation = RBT_ACT_SITU in the
 * two calls above is RBT_E_INVALID). act NULL = SiLU. Situ divides by beta and linear_beta: a zero
 * or non-finite value is RBT_E_INVALID (the reference leaves them unchecked). */
int rbt_apply_single_expert_act(rbt_ctx *ctx, const rbt_expert_slot *slot, const int32_t *ids, const float *w,
                                size_t s, size_t k, const float *x, size_t d, size_t i, const rbt_activation *act,
                                float *out);
int rbt_apply_single_expert_act_d(rbt_ctx *ctx, const rbt_expert_slot *slot, const int32_t *ids, const float *w,
                                  size_t s, size_t k, const float *x, size_t d, size_t i,
                                  const rbt_activation *act, float *out);

/* ---- HBM-resident expert pool (ExpertCache, expert_cache.rs) ---------------------------------- */
/* ensure_loaded (expert_cache.rs:890) for one expert: copies a host slot's bytes into HBM,
 * validating byte lengths as mxfp4_from_raw does (expert_cache.rs:1245-1256). Replaces an
 * existing (layer, eid) entry. */
int rbt_pool_put(rbt_ctx *ctx, uint32_t layer, const rbt_expert_slot *host_slot);
/* Registers a slot whose pointers are already device memory owned by the caller. */
int rbt_pool_put_device(rbt_ctx *ctx, uint32_t layer, const rbt_expert_slot *dev_slot);
/* Allocates an uninitialised device slot of the given shape (MXFP4 or I4G, separate gate/up) in the
 * pool and returns it, so a loader can fill the bytes in place (e.g. straight from a file read or
 * a device-side generator) without a host staging copy. */
const rbt_expert_slot *rbt_pool_alloc(rbt_ctx *ctx, uint32_t layer, uint32_t eid, int32_t kind,
                                      size_t d, size_t i, size_t group_size);
/* ExpertCache::get (expert_cache.rs:1010): the device-resident slot, or NULL when absent. */
const rbt_expert_slot *rbt_pool_get(rbt_ctx *ctx, uint32_t layer, uint32_t eid);
/* Bytes resident in the pool (all layers). */
size_t rbt_pool_resident_bytes(rbt_ctx *ctx);

/* ---- on-disk checkpoints: safetensors shards (safetensors.rs:215-488) ------------------------- */
/* The index of every *.safetensors file in a directory, in file-name order (Shards::open). Host
 * only, no context; the calls below return a status and describe a failure in
 * rbt_shards_last_error() (per thread). */
typedef struct rbt_shards rbt_shards;
typedef struct {
    int32_t file_index;      /* shard (file-name order) */
    uint64_t offset;         /* byte offset of the tensor's data in that file */
    uint64_t nbytes;
    char dtype[16];          /* the header's dtype string */
    int32_t ndim;            /* shape entries kept (at most 8) */
    uint64_t shape[8];
} rbt_tensor_info;
int rbt_shards_open(const char *dir, rbt_shards **out);
void rbt_shards_close(rbt_shards *sh);
const char *rbt_shards_last_error(void);
size_t rbt_shards_count(const rbt_shards *sh);
/* Shards::find / tensor_location: RBT_OK, or RBT_E_NOT_FOUND. */
int rbt_shards_find(const rbt_shards *sh, const char *name, rbt_tensor_info *info);
/* Shards::read_raw: the tensor's bytes into host dst (cap bytes). */
int rbt_shards_read(const rbt_shards *sh, const char *name, void *dst, size_t cap);
/* n bytes from byte `offset` of the tensor. */
int rbt_shards_read_range(const rbt_shards *sh, const char *name, uint64_t offset, void *dst, size_t n);

/* MXFP4 routed experts as the checkpoints name them (ExpertNaming, expert_cache.rs:93-208). */
typedef enum {
    RBT_NAMING_QWEN38_MXFP4 = 0, /* model.layers.{L}.mlp.experts.{E}.{gate,up,down}_proj.weight (+ .weight_scale) */
    RBT_NAMING_KIMI_K3_MXFP4 = 1 /* language_model.model.layers.{L}.block_sparse_moe.experts.{E}.{w1,w3,w2}
                                    .weight_packed (+ .weight_scale) */
} rbt_naming;
/* ensure_loaded (expert_cache.rs:890) for MXFP4 experts: each expert's packed and scale tensors
 * (gate/w1, up/w3 [moe_inter, hidden]; down/w2 [hidden, moe_inter]) are read verbatim into a new
 * pool slot of `layer`, their byte lengths checked as mxfp4_from_raw does (expert_cache.rs:
 * 1245-1256: RBT_E_SHAPE naming the tensor). A missing tensor is RBT_E_NOT_FOUND. Experts before a
 * failing one stay loaded; the failing one is not inserted. Synchronous. */
int rbt_pool_load_mxfp4(rbt_ctx *ctx, const rbt_shards *sh, int32_t naming, uint32_t layer, const uint32_t *eids,
                        size_t n, size_t hidden, size_t moe_inter);

/* ---- MoE layer: family dispatch (model.rs:22-140) and moe_forward / moe ------------------------ */
typedef enum {
    RBT_FAMILY_QWEN38 = 0, /* softmax top-k router, sigmoid-gated shared expert
                              (qwen38/generate.rs:262-351) */
    RBT_FAMILY_GLM52 = 1,  /* sigmoid(+bias) top-k, norm_topk, routed_scale, ungated shared expert
                              (glm52/moe.rs:350-451) */
    RBT_FAMILY_KIMI_K3 = 2 /* K3 routes through glm52::moe::route (kimi_k3/model.rs:426); plain
                              (non-latent) MoE layer, ungated shared expert */
} rbt_family;

typedef struct {
    int32_t family;          /* rbt_family */
    size_t hidden, moe_inter, n_experts, topk;
    const float *router;     /* host f32 [n_experts, hidden] (MoeWeights::router) */
    const float *router_bias;/* host f32 [n_experts] post-sigmoid selection bias, or NULL */
    const float *logit_bias; /* host f32 [n_experts] added to the router logits before the
                                activation (synthetic workload skew; not in the reference), or NULL */
    int32_t norm_topk;
    float routed_scale;
    size_t n_group, topk_group;
    int32_t has_shared;
    rbt_expert_slot shared;  /* host weights of the shared expert (uploaded) */
    const float *shared_gate;/* host f32 [hidden] (Qwen shared_expert_gate) or NULL = ungated */
} rbt_moe_layer_desc;

/* Uploads a layer's router, biases and shared expert to HBM (Model::load_multi's dense part for
 * the MoE block). Routed experts come from the pool (rbt_pool_put / rbt_pool_alloc). */
int rbt_moe_layer_set(rbt_ctx *ctx, uint32_t layer, const rbt_moe_layer_desc *desc);
/* Same, but the descriptor's pointers (router, biases, shared weights, shared gate) are device
 * memory that stays owned by the caller. */
int rbt_moe_layer_set_device(rbt_ctx *ctx, uint32_t layer, const rbt_moe_layer_desc *desc);

/* moe_forward (qwen38/generate.rs:262) / moe (glm52/moe.rs:350): router, top-k, every routed
 * expert in unique_experts order, then the shared expert added last. x f32[s, hidden] ->
 * out f32[s, hidden] (overwritten). ids_out / w_out (optional, [s, topk]) receive the routing. */
int rbt_moe_forward(rbt_ctx *ctx, uint32_t layer, const float *x, size_t s, float *out, int32_t *ids_out,
                    float *w_out);
int rbt_moe_forward_d(rbt_ctx *ctx, uint32_t layer, const float *x, size_t s, float *out,
                      int32_t *ids_out, float *w_out);

/* No counterpart in the reference. For callers that cannot allocate device memory (code under HIP
 * graph capture, tight serving loops, harnesses that forbid hipMalloc): rbt_moe_forward_d with every
 * per-call device buffer carved out of one fixed array of RBT_NOALLOC_SCRATCH_BYTES per device
 * (allocated when the library is loaded and held until the process ends), so the call itself
 * allocates nothing. Same kernels and results as rbt_moe_forward_d. A call whose buffers would not
 * fit returns RBT_E_UNSUPPORTED (e.g. the Qwen3.8-shaped layer fits up to 16 tokens, not a
 * 512-token prefill). Every call on one device shares that device's array: calls that overlap on
 * one GPU (two contexts, two host threads) race. The layer must have been set (rbt_moe_layer_set*),
 * which sizes the layer's own tables. */
#define RBT_NOALLOC_SCRATCH_BYTES (16u << 20)
int rbt_moe_forward_noalloc_d(rbt_ctx *ctx, uint32_t layer, const float *x, size_t s, float *out,
                              int32_t *ids_out, float *w_out);

/* ---- K3 latent MoE (kimi_k3/moe.rs) ----------------------------------------------------------- */
/* LatentMoeWeights (kimi_k3/moe.rs:41-57) plus the layer's expert width and activation. Device
 * memory. */
typedef struct {
    size_t moe_hidden;       /* routed_expert_hidden_size: the width the routed experts run at */
    rbt_qt down_proj;        /* [moe_hidden, hidden] */
    rbt_qt up_proj;          /* [hidden, moe_hidden] */
    const float *norm;       /* f32 [moe_hidden] (latent_moe_use_norm), or NULL */
    float eps;
    rbt_activation act;
} rbt_latent_moe_desc;
/* latent_moe (kimi_k3/moe.rs:64-116): route x[s, hidden] with `layer`'s router at full width,
 * x_latent = matmul_qt(x, down_proj), every routed expert of `layer`'s pool (shaped for moe_hidden:
 * gate/up [moe_inter, moe_hidden], down [moe_hidden, moe_inter]) accumulated at moe_hidden with
 * lw->act, rmsnorm of each summed row when lw->norm, then out[s, hidden] = matmul_qt(routed,
 * up_proj), overwritten; the shared expert is the caller's, as in the reference. Device buffers,
 * asynchronous on the context stream. */
int rbt_latent_moe_d(rbt_ctx *ctx, uint32_t layer, const rbt_latent_moe_desc *lw, const float *x, size_t s,
                     float *out, int32_t *ids_out, float *w_out);

/* ---- norms and the MoE sublayer -------------------------------------------------------------- */
/* rmsnorm (kimi_linear/ops.rs:46-53) of rows v[s, n] in place, device memory:
 * r = 1/sqrt(mean_f64(v^2) as f32 + eps), v *= r * w. */
int rbt_rmsnorm_d(rbt_ctx *ctx, float *v, const float *w, size_t s, size_t n, float eps);
/* rmsnorm_1p (qwen38/ops.rs:25-33): the same r, v *= r * (1 + w) (Qwen3_5MoeRMSNorm). */
int rbt_rmsnorm_1p_d(rbt_ctx *ctx, float *v, const float *w, size_t s, size_t n, float eps);
/* The MoE half of a Qwen 3.8 decoder layer (qwen38/generate.rs:397-413) in one device round trip:
 * x[s, hidden] += moe_forward(rmsnorm_1p(x, post_ln, eps)), in place. post_ln f32[hidden].
 * ids_out / w_out as for rbt_moe_forward. _d: device buffers, asynchronous on the context stream. */
int rbt_moe_sublayer(rbt_ctx *ctx, uint32_t layer, float *x, size_t s, const float *post_ln, float eps,
                     int32_t *ids_out, float *w_out);
int rbt_moe_sublayer_d(rbt_ctx *ctx, uint32_t layer, float *x, size_t s, const float *post_ln, float eps,
                       int32_t *ids_out, float *w_out);

/* ---- token mixers of Qwen 3.8 (one decode token; device buffers) ------------------------------ */
/* Gated DeltaNet (69 of the 92 layers): the part of qwen38/generate.rs:196-219 gdn_step between
 * the input projections (in_proj_qkv -> qkv_pre, in_proj_z/a/b -> z, a, b, each an rbt_matmul_qt_d)
 * and out_proj: ShortConvState::step (kimi_linear/short_conv.rs:58-85) then gdn::step_token
 * (qwen38/gdn.rs:142-196). conv_state [conv_dim, conv_kernel - 1] (conv_dim = 2 n_k_heads
 * head_k_dim + n_v_heads head_v_dim) and states [n_v_heads, head_k_dim, head_v_dim] are the layer's
 * carried state (zero at the start, updated in place: GdnLayerState, KdaState::new kda.rs:99);
 * qkv_pre [conv_dim], z [n_v_heads head_v_dim], a, b [n_v_heads]; out [n_v_heads head_v_dim].
 * head_v_dim must be a multiple of 4 dividing 2048 (at most 512) and head_k_dim even and at most
 * 8192 / head_v_dim (RBT_E_UNSUPPORTED otherwise; Qwen 3.8: 128 x 128); states 16-byte aligned. */
typedef struct {
    size_t n_v_heads, n_k_heads, head_k_dim, head_v_dim, conv_kernel;
    const float *conv_weight;  /* [conv_dim, conv_kernel] (conv1d weight, depthwise, no bias) */
    const float *a_log;        /* [n_v_heads] A_log */
    const float *dt_bias;      /* [n_v_heads] */
    const float *norm_weight;  /* [head_v_dim] the gated RMSNorm's weight */
    float eps;
} rbt_gdn_desc;
int rbt_gdn_step_d(rbt_ctx *ctx, const rbt_gdn_desc *desc, float *conv_state, float *states,
                   const float *qkv_pre, const float *z, const float *a, const float *b, float *out);
/* GQA attention (23 of the 92 layers): the part of qwen38/generate.rs:226-255 attn_step between the
 * projections (q_proj -> qg [n_heads, 2 head_dim] as [query, gate] per head, k_proj -> k, v_proj
 * -> v, each [n_kv_heads head_dim]) and o_proj: split_query_gate (attention.rs:122), norm_heads
 * (:138), rope_half (:160), KvCache::push (:76) at position pos, attend (:190) over positions
 * 0..pos, apply_output_gate (:221). k_cache / v_cache [cap, n_kv_heads, head_dim] hold positions
 * 0..pos-1 (the cache's len is pos; 16-byte aligned). ctx_out [n_heads head_dim]. head_dim a
 * multiple of 64 up to 1024, at most 16 query heads per KV head, pos < 393216 (RBT_E_UNSUPPORTED
 * otherwise; Qwen 3.8: 64 heads over 4, head_dim 256). */
typedef struct {
    size_t n_heads, n_kv_heads, head_dim, rope_dim;
    float theta, attn_scale, eps;
    const float *q_norm, *k_norm;  /* [head_dim] each, (1 + w) RMSNorm weights */
} rbt_gqa_desc;
int rbt_gqa_step_d(rbt_ctx *ctx, const rbt_gqa_desc *desc, float *k_cache, float *v_cache, size_t cap, size_t pos,
                   const float *qg, const float *k, const float *v, float *ctx_out);

/* ---- instrumentation (no counterpart in the reference: benchmark support) -------------------- */
typedef struct {
    double router_ms;    /* router logits + top-k selection + grouping (one-token MXFP4 calls: the
                            router launch; the selection itself runs at the start of gate/up) */
    double gateup_ms;    /* gate/up products + silu(g)*u (the experts this phase streams) */
    double down_ms;      /* down products (with the ordered combine where it is fused in) */
    double combine_ms;   /* the separate weighted combine + shared expert; where the combine is
                            fused into the down kernel, only the time to the call's end */
    uint64_t calls;      /* rbt_moe_forward_d calls recorded */
    uint64_t ambiguous;  /* router logits recomputed exactly because of a near-tie */
    uint64_t gateup_experts; /* one-token calls: experts whose gate/up the gate/up phase streamed
                                (routed pairs, candidates of a deferred decision, the shared expert) */
    uint64_t down_experts;   /* one-token calls: experts whose down the down phase streamed */
} rbt_profile;
/* When on, rbt_moe_forward_d records HIP events on the context stream around each phase. */
int rbt_profile_enable(rbt_ctx *ctx, int32_t on);
/* Synchronises the stream and returns the accumulated phase times; reset != 0 clears them. */
int rbt_profile_read(rbt_ctx *ctx, rbt_profile *out, int32_t reset);
/* Per-kernel timing: while on, every kernel the context launches records HIP events at its own
 * start and end (the dispatch records them, so dispatch gaps are excluded). */
typedef struct {
    char name[160];          /* the kernel's name as the runtime reports it */
    uint64_t launches;
    double total_ms;
} rbt_kernel_stat;
int rbt_profile_kernels(rbt_ctx *ctx, int32_t on);
/* Synchronises, folds the recorded launches into per-kernel sums and copies up to cap of them
 * into out; *n receives the number of kernels recorded. reset != 0 clears the sums. */
int rbt_profile_kernels_read(rbt_ctx *ctx, rbt_kernel_stat *out, size_t cap, size_t *n, int32_t reset);

/* ---- synthetic workload generator (benchmarks and tests; bit-identical to oracle/) ------------ */
/* Fills an MXFP4 [rows, cols] matrix in device memory: nibbles uniform over 0..15, E8M0 bytes
 * uniform over exp_lo..exp_hi, from a counter-based hash of `seed`. */
int rbt_synth_mxfp4_d(rbt_ctx *ctx, uint8_t *data, uint8_t *scale, size_t rows, size_t cols, uint64_t seed,
                      uint32_t exp_lo, uint32_t exp_hi);
/* Fills a grouped-int4 [rows, cols] matrix: nibbles uniform over 0..15 (values -8..7), scales
 * uniform over [s_lo, s_hi). */
int rbt_synth_i4g_d(rbt_ctx *ctx, uint8_t *data, float *scale, size_t rows, size_t cols, size_t group_size,
                    uint64_t seed, float s_lo, float s_hi);

#ifdef __cplusplus
}
#endif
#endif /* RABBIT_AMD_H */
