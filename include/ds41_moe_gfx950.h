/*
 * ds41 speculative-verify MoE path for MI355X (gfx950): C ABI.
 *
 * Drop-in replacements for the reference's components/moe kernel API and its
 * raw C entry points, implemented with hand-written HIP kernels (scaled
 * f8f6f4 MFMA GEMV/GEMM) for gfx950. All buffers are caller-owned DEVICE
 * memory unless stated; `stream` is a hipStream_t passed as void*. Every entry
 * returns a hipError_t value as int (0 == hipSuccess); invalid arguments
 * return hipErrorInvalidValue (1), as the reference returns
 * cudaErrorInvalidValue. No entry point allocates or synchronises unless its
 * comment says so.
 *
 * Reference citations are paths in SSHdotCodes/deepseek-v4.1-flash-pro6000.
 */
#ifndef DS41_MOE_GFX950_H
#define DS41_MOE_GFX950_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* Device ABI types, byte-identical to the reference
 * (components/moe/include/ds41/store.hpp:110-117 DeviceExpert, 64 B;
 *  components/moe/include/ds41/kernels.cuh:8-13 GemmJob, 32 B).
 * ready == NULL: ordering is the caller's (stream/event); otherwise kernels
 * wait until *ready == generation (acquire) before reading the weights. The
 * wait is bounded (about 2 s); when it gives up, status bit 1 is set and the
 * outputs that needed the expert are written as NaN (ds41_take_status). */
typedef struct ds41_device_expert {
  const uint8_t *gate, *gate_scale;
  const uint8_t *up, *up_scale;
  const uint8_t *down, *down_scale;
  const uint32_t *ready;
  uint32_t generation;
  int32_t slot;
} ds41_device_expert;

typedef struct ds41_gemm_job {
  uint32_t expert;          /* index into the DeviceExpert table */
  int32_t tokens;           /* 1..8 rows for this expert (the prefill entry takes up to max_tokens) */
  const uint8_t *x;         /* E4M3 [tokens][k] */
  const uint8_t *x_scale;   /* E8M0 [tokens][k/32] */
  void *output;             /* BF16 [tokens][n] */
} ds41_gemm_job;

enum { DS41_PROJ_GATE = 0, DS41_PROJ_UP = 1, DS41_PROJ_DOWN = 2 };

/* ---- components/moe kernel API (kernels.cuh:14-38) -------------------------- */
/* quantize_mxfp8 (components/moe/src/mxfp4.cu:341-345): bf16 [rows][cols] ->
 * E4M3 q [rows][cols] + E8M0 s [rows][cols/32]. cols % 32 == 0. */
int ds41_quantize_mxfp8(const void *x_bf16, uint8_t *q, uint8_t *scales, int rows, int cols,
                        void *stream);
/* grouped_mxfp4 / _native / _parallel / _native_parallel / _native_tiled
 * (mxfp4.cu:346-381): one launch over `count` jobs of a W4A8 projection,
 * out[t][n] = bf16(sum_k x[t][k] * w[n][k]). All five names run the same
 * gfx950 kernel (fp32 accumulation on the scaled MFMA). k % 32 == 0. */
int ds41_grouped_mxfp4(const ds41_device_expert *table, const ds41_gemm_job *jobs, int count,
                       int projection, int n, int k, void *stream);
int ds41_grouped_mxfp4_native(const ds41_device_expert *table, const ds41_gemm_job *jobs,
                              int count, int projection, int n, int k, void *stream);
int ds41_grouped_mxfp4_parallel(const ds41_device_expert *table, const ds41_gemm_job *jobs,
                                int count, int projection, int n, int k, void *stream);
int ds41_grouped_mxfp4_native_parallel(const ds41_device_expert *table,
                                       const ds41_gemm_job *jobs, int count, int projection,
                                       int n, int k, void *stream);
int ds41_grouped_mxfp4_native_tiled(const ds41_device_expert *table, const ds41_gemm_job *jobs,
                                    int count, int projection, int n, int k, void *stream);
/* swiglu (mxfp4.cu:352-356): g=min(g,L), u=clamp(u,+-L) (L>0), h=silu(g)*u*w[row] -> bf16.
 * route_weight may be NULL. */
int ds41_swiglu(const void *gate_bf16, const void *up_bf16, const float *route_weight,
                void *out_bf16, int rows, int cols, float limit, void *stream);
/* reduce_experts (mxfp4.cu:386-389): per token, routed rows [rows][topk][hidden]
 * summed in ascending expert-id order (fp32), + shared [rows][hidden] (nullable),
 * -> bf16. Duplicate/invalid ids: the token's output row is set to NaN and the
 * call still returns 0 (the reference traps the device instead). topk <= 8. */
int ds41_reduce_experts(const void *routed_bf16, const int32_t *ids, const void *shared_bf16,
                        void *out_bf16, int rows, int topk, int hidden, void *stream);

/* ---- raw C ABI (kernels.cuh:43-62; mxfp4.cu:392-442) ------------------------ */
int ds41_mxfp4_raw(const uint8_t *weight, const uint8_t *weight_scale, const uint8_t *activation,
                   const uint8_t *activation_scale, void *output_bf16, int m, int n, int k,
                   void *stream);
int ds41_mxfp4_native_raw(const uint8_t *weight, const uint8_t *weight_scale,
                          const uint8_t *activation, const uint8_t *activation_scale,
                          void *output_bf16, int m, int n, int k, void *stream);
int ds41_mxfp4_parallel_raw(const uint8_t *weight, const uint8_t *weight_scale,
                            const uint8_t *activation, const uint8_t *activation_scale,
                            void *output_bf16, int m, int n, int k, void *stream);
int ds41_mxfp4_native_parallel_raw(const uint8_t *weight, const uint8_t *weight_scale,
                                   const uint8_t *activation, const uint8_t *activation_scale,
                                   void *output_bf16, int m, int n, int k, void *stream);
int ds41_quantize_mxfp8_raw(const void *input_bf16, uint8_t *q, uint8_t *scales, int rows,
                            int cols, void *stream);
int ds41_swiglu_raw(const void *gate_bf16, const void *up_bf16, const float *route_weight,
                    void *output_bf16, int rows, int cols, float limit, void *stream);

/* ---- pluggable projection backend "xk" v1 (components/moe/include/ds41/decode_backend.hpp:7-22) */
int ds41_xk_projection_abi_version(void); /* returns 1 */
int ds41_xk_grouped_v1(const ds41_device_expert *table, const ds41_gemm_job *jobs, int count,
                       int projection, int n, int k, void *stream);

/* ---- router (components/dense/src/ops.cu:73,107,117; engine/src/ops.cu:59-73,126-130) */
/* u = sqrt(z > 20 ? z : log1p(exp(z))), b = u + bias[col] over logits [M][N]. */
int ds41_dense_router_scores(const float *logits, const float *bias, float *u, float *b, int M,
                             int N, void *stream);
/* w[row][i] = u[row][ids[i]] / (fixed-order sum + 1e-20) * scale, topk in {1..8}. */
int ds41_dense_router_weights(const float *scores, const int32_t *ids, float *w, int M, int N,
                              int topk, float scale, void *stream);
/* engine/src/ops.cu:126-130: one row, scale 1.5. */
int ds41_engine_route_weights(const float *scores, const int *ids, float *out, int k,
                              void *stream);
/* fp32 router GEMV (the reference's cuBLAS fp32 GEMV, batch.inc:23-41,460):
 * logits[t][e] = sum_h bf16 x[t][h] * w[e][h]; M <= 16. */
int ds41_router_logits(const void *x_bf16, const float *w, float *logits, int M, int N, int K,
                       void *stream);
/* Top-k by biased score, descending, ties -> lower id (batch.inc:228-237). M rows of N <= 1024. */
int ds41_router_topk(const float *b, int32_t *ids, int M, int N, int topk, void *stream);

/* ---- fused verify MoE layer (batch.inc:220-335 bmoe + bshared) ------------- */
/* One MoE layer for T = tokens rows (1..8), entirely on the device with no host
 * sync, in five kernels: router GEMV + score + MXFP8 quant of x; top-k + route
 * weights + route plan (one workgroup); fused gate/up MXFP4 GEMV +
 * SwiGLU(limit)*w + MXFP8; down GEMV; ordered reduce (ascending expert id,
 * shared expert last).
 * Routed experts are table[expert_base + id]; the shared expert is
 * table[shared_index] (shared_index < 0: none). hidden % 256 == 0 (<= 8192),
 * inter % 32 == 0, n_experts <= 512, topk <= 8.
 * Calls that share one workspace must be ordered (same stream). */
/* Size and version negotiation of the structs that grow between builds (the reference's C structs
 * carry the same pair, engine/include/ds41/target_shared.h:11-13): ds41_moe_layer_args,
 * ds41_stack_desc, ds41_stack_stats, ds41_cache_stats and ds41_target_experts_desc begin with
 * abi_version and struct_bytes. The caller sets them (DS41_ABI_INIT(T) for the first two
 * initialisers) on the structs it passes in and on those it passes to be filled; the library
 * rejects any other pair with hipErrorInvalidValue before it reads or writes past those two
 * fields. */
#define DS41_GFX950_ABI_VERSION 1u
#define DS41_ABI_INIT(T) DS41_GFX950_ABI_VERSION, (uint32_t)sizeof(T)
typedef struct ds41_moe_layer_args {
  uint32_t abi_version;            /* DS41_GFX950_ABI_VERSION */
  uint32_t struct_bytes;           /* sizeof this struct as the caller was built */
  const void *x_bf16;             /* [tokens][hidden] */
  const float *router_w;          /* [n_experts][hidden] fp32 */
  const float *router_bias;       /* [n_experts] fp32 */
  const ds41_device_expert *table;
  int32_t expert_base, shared_index;
  int32_t tokens, hidden, inter, n_experts, topk;
  int32_t score_mode;             /* 0: sqrt-softplus (reference), 1: sigmoid */
  float route_scale;              /* 1.5 in the reference */
  float swiglu_limit;             /* 10 in the reference */
  void *y_bf16;                   /* [tokens][hidden] */
  void *workspace;                /* ds41_moe_layer_workspace_bytes() device bytes */
  size_t workspace_bytes;
  int32_t *ids_out;               /* optional [tokens][topk] (device) */
  float *weights_out;             /* optional [tokens][topk] (device) */
  float *logits_out;              /* optional [tokens][n_experts] (device) */
  void *const *stage_events;      /* optional: 10 hipEvent_t, the start and stop timestamps of
                                     each of the 5 kernels (router, plan, gate/up/act, down,
                                     reduce) in order (hipExtLaunchKernel) */
  uint32_t stage_mask;            /* 0: every kernel. Otherwise bit i launches kernel i only (for
                                     timing one kernel on a workspace a full call has prepared).
                                     When the activation rows of all jobs fit the fused kernel's
                                     150 KB LDS tile ((tokens*topk + tokens) rows of about inter
                                     bytes: tokens <= 6 at topk 6, inter 2880), kernel 3 is the
                                     fused down projection and reduction and kernel 4 launches
                                     nothing (its two events mark an empty interval). Bit 5 keeps the separate down and
                                     reduce kernels (same output bits); alone it means every kernel. */
  const ds41_device_expert *shared_fp8; /* optional host struct: the shared expert as the checkpoint
                                     stores it, FP8 E4M3 gate/up [inter][hidden] and down
                                     [hidden][inter] with one E8M0 scale per 32 x 32 block
                                     ([rows/32][cols/32]); W8A8 with MXFP8 activations
                                     (components/dense/src/dense.cu:37-91, batch.inc:330-335
                                     bshared). Requires shared_index < 0. */
  int32_t weight_layout;          /* 0: the table's MXFP4 weights are row-major [N][K/2] (the
                                     checkpoint's layout); 1: tiled by ds41_expert_slab_tile (the MFMA
                                     operand order, read as contiguous kilobytes); scales are row-major
                                     either way */
} ds41_moe_layer_args;
size_t ds41_moe_layer_workspace_bytes(int tokens, int hidden, int inter, int n_experts,
                                      int topk);

int ds41_moe_verify_layer(const ds41_moe_layer_args *args, void *stream);
/* No counterpart in the reference. For callers that cannot allocate (code under
 * HIP graph capture, serving loops that forbid hipMalloc): ds41_moe_verify_layer
 * with its workspace in a fixed device array of ds41_moe_layer_noalloc_max_bytes()
 * (1.5 MiB) that each GPU holds until the process ends. args->workspace and
 * workspace_bytes are ignored; shapes whose workspace
 * (ds41_moe_layer_workspace_bytes) exceeds the array return hipErrorInvalidValue.
 * It calls no allocator. Every call on one GPU shares that GPU's array and leaves
 * the last call's plan in it (a stage_mask call reads it); calls that overlap
 * on one GPU (different streams without ordering) race. */
int ds41_moe_verify_layer_noalloc(const ds41_moe_layer_args *args, void *stream);
size_t ds41_moe_layer_noalloc_max_bytes(void);
/* Reads the route plan of the last layer call from its workspace (host copy, synchronous):
 * unique expert count and ids; returns the count or -1. */
int ds41_moe_layer_plan(const void *workspace, int tokens, int hidden, int inter, int n_experts,
                        int topk, int32_t *unique_ids, int max_ids);

/* ---- chunked verify / prefill (T >= 256 rows) on the scaled MFMA ------------- */
/* grouped_mxfp4_prefill (components/moe/src/mxfp4.cu:382-385, prefill.cuh:7-96):
 * jobs of 1..max_tokens (<= 256) rows; grid over 64-channel x 64-row tiles.
 * k % 32 == 0 (the reference requires k % 256 == 0). Job x / x_scale rows must
 * be 16-byte aligned (x: k bytes per row). A job whose token count is outside
 * 1..max_tokens is skipped and sets status bit 2. */
int ds41_grouped_mxfp4_prefill(const ds41_device_expert *table, const ds41_gemm_job *jobs,
                               int count, int projection, int n, int k, int max_tokens,
                               void *stream);
/* ds41_mxfp4_prefill_raw (mxfp4.cu:436-442): one job, m <= 256 rows. */
int ds41_mxfp4_prefill_raw(const uint8_t *weight, const uint8_t *weight_scale,
                           const uint8_t *activation, const uint8_t *activation_scale,
                           void *output_bf16, int m, int n, int k, void *stream);

/* One prefill MoE layer over T = tokens rows (engine/src/prefill/native.inc:240-276
 * with engine/include/ds41/prefill/plan.hpp:39-54): MXFP8 quantisation of x, a
 * device route plan (stable expert-major permutation of the T*topk slots,
 * per-expert offsets; experts with <= 8 rows become GEMV jobs of the decode
 * layer's kernels, the others and the shared expert <= 64-row tiles), fused
 * gate/up + SwiGLU(limit)*w + MXFP8, down, and the ordered reduce (ascending
 * expert id, shared last).
 * ids / weights: device [tokens][topk] routing (the caller's top-k). Invalid or
 * duplicate ids: every output row is NaN and status bit 4 is set.
 * tokens * topk <= 4096, topk <= 8, n_experts <= 1024, hidden % 64 == 0,
 * inter % 32 == 0. */
typedef struct ds41_moe_prefill_args {
  const void *x_bf16;             /* [tokens][hidden] */
  const int32_t *ids;             /* [tokens][topk] */
  const float *weights;           /* [tokens][topk] */
  const ds41_device_expert *table;
  int32_t expert_base, shared_index;
  int32_t tokens, hidden, inter, n_experts, topk;
  float swiglu_limit;
  void *y_bf16;                   /* [tokens][hidden] */
  void *workspace;                /* ds41_moe_prefill_workspace_bytes() device bytes */
  size_t workspace_bytes;
  void *const *stage_events;      /* optional: 18 hipEvent_t, start and stop of each of the 9
                                     kernels: quant, plan, gate/up/act GEMV (<= 4 rows), GEMV
                                     (5..8 rows), tiles, down GEMV (<= 4), GEMV (5..8), tiles,
                                     reduce */
} ds41_moe_prefill_args;
size_t ds41_moe_prefill_workspace_bytes(int tokens, int hidden, int inter, int n_experts,
                                        int topk);
int ds41_moe_prefill_layer(const ds41_moe_prefill_args *args, void *stream);
/* Number of 64-row GEMM tiles the last prefill plan produced (experts with more
 * than 8 rows, and the shared expert; synchronous read; 0 after invalid routes). */
int ds41_moe_prefill_tiles(const void *workspace, int tokens, int hidden, int inter,
                           int n_experts, int topk, int32_t *tiles);
/* The last prefill plan's work split (synchronous read): counts[0] tiles,
 * counts[1] GEMV jobs of experts with <= 4 rows, counts[2] of experts with
 * 5..8 rows. No counterpart in the reference (its sweep batches experts on the host). */
int ds41_moe_prefill_plan_counts(const void *workspace, int tokens, int hidden, int inter,
                                 int n_experts, int topk, int32_t *counts);

/* ---- verify step through a stack of MoE layers with a host expert tier ------ */
/* Canonical expert slab (the reference's 18.8 MB offload slot, store.hpp:32-37,
 * offload.cpp:443-457): gate W [inter][hidden/2] | gate scales [inter][hidden/32]
 * | up W | up scales | down W [hidden][inter/2] | down scales [hidden][inter/32],
 * each tensor 256-byte aligned; `bytes` is the slab size (4 KiB multiple).
 * Returns 0, or hipErrorInvalidValue for hidden/inter not multiples of 32. */
typedef struct ds41_expert_layout {
  uint64_t offset[6];
  uint64_t bytes;
} ds41_expert_layout;
int ds41_expert_slab_layout(int hidden, int inter, ds41_expert_layout *out);
/* No counterpart in the reference. Copies `count` consecutive canonical slabs from `in` to `out`
 * (distinct, 256-byte aligned) with the three weight tensors tiled in the MFMA operand order: the
 * 16-byte piece of row n, K32 group g of a [N][K/2] tensor goes to
 * (n / 16) * (K / 32) * 256 + g * 256 + (n % 16) * 16. The slab size is unchanged. Tiled slabs let
 * each GEMV load instruction read one contiguous kilobyte (weight_layout 1). ds41_expert_slab_tile:
 * device memory, on `stream`; _host: host memory, synchronous. */
int ds41_expert_slab_tile(const void *in, void *out, int hidden, int inter, int count, void *stream);
int ds41_expert_slab_tile_host(const void *in, void *out, int hidden, int inter, int count);

/* One layer of the stack. Routed expert id e is table[expert_base + e]; the
 * shared expert is table[shared_index] (< 0: none). Residency (the reference's
 * OffloadStore placement, components/moe/src/offload.cpp:240-381): host_index (device int32
 * [n_experts]) is -1 for an HBM-resident expert and otherwise the index of the
 * expert's canonical slab in host_slabs (pinned host memory from hipHostMalloc,
 * host_slab_count slabs), whose table entry is then never read.
 * host_index == NULL: all resident. */
typedef struct ds41_stack_layer {
  const float *router_w;           /* device fp32 [n_experts][hidden] */
  const float *router_bias;        /* device fp32 [n_experts] */
  const ds41_device_expert *table; /* device */
  int32_t expert_base, shared_index;
  const int32_t *host_index;       /* device, nullable */
  const uint8_t *host_slabs;       /* pinned host, nullable when host_index is NULL */
  int32_t host_slab_count;
  int32_t reserved;
} ds41_stack_layer;

typedef struct ds41_stack_desc {
  uint32_t abi_version;            /* DS41_GFX950_ABI_VERSION */
  uint32_t struct_bytes;           /* sizeof this struct as the caller was built */
  int32_t layers, max_tokens, hidden, inter, n_experts, topk, score_mode;
  float route_scale, swiglu_limit;
  const ds41_stack_layer *layer;   /* host array [layers], copied at create */
  int32_t weight_layout;           /* as ds41_moe_layer_args.weight_layout, for every table, host and
                                      cached slab of the stack */
} ds41_stack_desc;

/* Cumulative counters of the layers that have a host tier (read back each layer). */
typedef struct ds41_stack_stats {
  uint32_t abi_version;            /* DS41_GFX950_ABI_VERSION */
  uint32_t struct_bytes;           /* sizeof this struct as the caller was built */
  uint64_t steps, layers;          /* layers = layer passes with a host tier */
  uint64_t resident_routed;        /* routed experts served from their table's HBM slabs (shared excluded) */
  uint64_t host_fetched;           /* host-tier experts copied in (on demand or by a prefetch) */
  uint64_t h2d_bytes;
  uint64_t invalid_layers;         /* layer passes whose routes were rejected */
  uint64_t cached_routed;          /* routed host-tier experts served from the HBM cache (held when the
                                      plan ran, or landed by a prefetch before the layer's jobs) */
} ds41_stack_stats;

/* Creates a stack (allocates: the layer workspace, per-layer plan buffers,
 * 2*max_tokens*topk staging slots, two activation buffers, pinned plan
 * read-back mirrors (one per layer), a copy stream at default priority and two
 * events, on the current device). *stack receives
 * an opaque handle. The verify-step counterpart of the MoE part of the
 * reference's Forward::verify (engine/src/forward.cu:769, batched through
 * engine/src/hotpath/batch.inc:220-335), with OffloadStore::order/upload
 * (components/moe/src/offload.cpp:443-457) as the host tier. */
int ds41_verify_stack_create(const ds41_stack_desc *desc, void **stack);
/* One verify step of `tokens` rows (1..max_tokens) through every layer: layer l
 * takes layer l-1's output (layer 0 takes x).
 * Router routing (route_ids NULL), per layer: router + plan on `stream`; a
 * read-back of the plan (one host wait per layer that has a host tier, as the
 * reference's per-layer route-event wait, batch.inc:224); resident gate/up and
 * down run while the host issues hipMemcpyAsync of the routed host-tier slabs
 * on the copy stream; host-tier gate/up and down wait on the copies' event;
 * then the ordered reduce.
 * Caller routing (route_ids: device int32 [layers][tokens][topk] that replaces
 * the router's top-k; the weights still come from the router's scores): every
 * layer is planned in one launch at the start of the step and the host reads
 * all the plans once (one wait per step, while layer 0 runs), then issues every
 * layer's host-tier copies and enqueues every layer without another wait; a
 * layer is then two launches (router + gate/up/act, down + reduce).
 * layer_out (nullable, device bf16 [layers][tokens][hidden]): every layer's
 * output; ids_out / weights_out (nullable, device [layers][tokens][topk]).
 * Steps on one stack must not overlap (one workspace and staging area). */
int ds41_verify_stack_step(void *stack, const void *x_bf16, void *y_bf16, int tokens,
                           const int32_t *route_ids, void *layer_out, int32_t *ids_out,
                           float *weights_out, void *stream);
/* One layer of the same step (layer 0..layers-1), for hosts that run other
 * work (attention) between MoE layers: x [tokens][hidden] -> y, route_ids /
 * ids_out / weights_out [tokens][topk] (nullable). y may alias x (x is read
 * only by the layer's first kernel).
 * The per-layer entry of the reference's bmoe (engine/src/hotpath/batch.inc:220). */
int ds41_verify_stack_layer(void *stack, int layer, const void *x_bf16, void *y_bf16, int tokens,
                            const int32_t *route_ids, int32_t *ids_out, float *weights_out,
                            void *stream);
int ds41_verify_stack_stats(void *stack, ds41_stack_stats *out);

int ds41_verify_stack_destroy(void *stack);
/* Pinned host memory for host-tier slabs (the reference's HostBuffer,
 * components/moe/include/ds41/store.hpp:161-174, which registers an existing
 * mapping; here the pages are allocated pinned with hipHostMalloc, so DMA
 * copies from them run asynchronously). Synchronous; *out is NULL on error. */
int ds41_host_alloc(size_t bytes, void **out);
int ds41_host_free(void *p);

/* ---- FP8 W8A8 shared-expert projections (components/dense/include/ds41/dense.h) ---- */
/* ds41_dense_quant (dense.h:10, dense.cu:8-15): MXFP8 quantisation of BF16 rows, the same rule as
 * ds41_quantize_mxfp8. */
int ds41_dense_quant(const void *x_bf16, void *a_fp8, void *as_ue8m0, int M, int K, void *stream);
/* ds41_dense_fp8 (dense.h:11-17, dense.cu:37-91 and 98-106): y BF16 [M][N] = MXFP8 a [M][K] x E4M3
 * w [N][K] with one E8M0 scale per 32 x 32 block (ws [N/32][K/32]); every K32 block dot times
 * both scales, added in ascending K in fp32. M <= 8, N and K multiples of 32. `variant` (-1, 0..6)
 * is accepted for the reference's signature and ignored: one gfx950 kernel serves all shapes. */
int ds41_dense_fp8(const void *a_fp8, const void *as_ue8m0, const void *w_fp8, const void *ws_ue8m0,
                   void *y_bf16, int M, int N, int K, int variant, void *stream);
/* ds41_dense_shared_act (dense.h:41, ops.cu:103-106): z = BF16(SwiGLU(gate, up) with limit 10)
 * (z may be NULL) and its MXFP8 codes/scales. */
int ds41_dense_shared_act(const void *gate_bf16, const void *up_bf16, void *z_bf16, void *a_fp8,
                          void *as_ue8m0, int M, int K, void *stream);

/* ---- expert slot pool (LFU residency policy) and placement files ------------- */
/* The reference's SlotPool (components/moe/include/ds41/store.hpp:80-157, store.cpp:15-196): a
 * CPU-only, deterministic assignment of experts to HBM slots. Expert ids are flattened layer by
 * layer: layer l owns ids first(l) .. first(l) + layer_experts[l] - 1 (the reference's space is
 * 40 layers of 384 then 3 of 128, store.hpp:16). Errors: -1 capacity (the need set exceeds the
 * usable slots), -2 id out of range, -3 illegal state (bad release, pin of a non-resident
 * expert), -4 invalid argument; ds41_pool_error() gives the text. No call touches the GPU. */
#define DS41_POOL_MAX_LAYERS 64
typedef struct ds41_placement {      /* Placement, store.hpp:39-47 */
  uint32_t recent_window, decay_interval;
  int32_t distinct_lfu, hard_budgets;
  int32_t layers, n_vram, n_host, reserved;
  uint32_t budget[DS41_POOL_MAX_LAYERS];      /* dynamic slots per layer, pins excluded */
  uint32_t host_budget[DS41_POOL_MAX_LAYERS];
  const uint32_t *vram_pins;          /* [n_vram] */
  const uint32_t *host_residents;     /* [n_host] */
} ds41_placement;
/* load_placement (components/moe/src/manifest.cpp:8-34): the text format of the reference's
 * profiles/p80-mtp48.placement. The id lists are written to the caller's arrays. Returns 0 or a
 * negative code with the reason in `error`. */
int ds41_placement_load(const char *path, int layers, const uint32_t *layer_experts,
                        ds41_placement *out, uint32_t *vram_pins, int vram_cap,
                        uint32_t *host_residents, int host_cap, char *error, size_t error_bytes);
typedef struct ds41_pool_allocation { /* SlotPool::Allocation */
  uint32_t id;
  int32_t slot;
  int32_t hit;
  int32_t reserved;
  int64_t evicted;                    /* expert id that lost the slot, -1 for none */
} ds41_pool_allocation;
/* SlotPool(slots, recent_window, decay_interval, distinct_lfu) */
int ds41_pool_create(int slots, int layers, const uint32_t *layer_experts, uint32_t recent_window,
                     uint32_t decay_interval, int distinct_lfu, void **pool);
int ds41_pool_destroy(void *pool);
const char *ds41_pool_error(void *pool);
int ds41_pool_policy(void *pool, const ds41_placement *placement);   /* SlotPool::policy */
/* SlotPool::acquire: one allocation per distinct id in first-seen order (out may be NULL);
 * returns their count. prefetch != 0 leaves the LFU history alone. */
int ds41_pool_acquire(void *pool, const uint32_t *ids, int n, int prefetch,
                      ds41_pool_allocation *out);
int ds41_pool_borrow(void *pool, const uint32_t *ids, int n, ds41_pool_allocation *out);
/* SlotPool::release. A lease listing one slot more often than it is leased is rejected. */
int ds41_pool_release(void *pool, const ds41_pool_allocation *lease, int n);
int ds41_pool_touch(void *pool, const uint32_t *ids, int n);
int ds41_pool_pin(void *pool, uint32_t id);
int ds41_pool_unpin(void *pool, uint32_t id);
int ds41_pool_residency(void *pool, uint32_t id);                     /* slot or -1 */
int ds41_pool_reset_history(void *pool);
/* SlotPool::retain (store.hpp:99-101): a token of the expert's slot contents; while any token of
 * the current occupant lives, the slot is neither evicted nor counted as usable. The token is
 * released with ds41_pool_token_release, which is thread-safe, never calls the pool and stays
 * valid after ds41_pool_destroy. */
int ds41_pool_retain(void *pool, uint32_t id, void **token);
int ds41_pool_token_release(void *token);
/* SlotPool::reserve / drained (store.hpp:102-106, store.cpp:130-152), soft pools only: evicts
 * policy victims (never wanted, pinned, leased or retained) into draining slots until empty +
 * draining slots reach `target`; out (at least `target` entries) gets one allocation per victim
 * with evicted = its id; returns their count. A draining slot has no occupant and is not
 * allocatable until ds41_pool_drained(slot). */
int ds41_pool_reserve(void *pool, int target, const uint32_t *wanted, int n_wanted,
                      ds41_pool_allocation *out);
int ds41_pool_drained(void *pool, int slot);
/* SlotPool::peer / exclusive / decay_interval / fast_minima / switch_target_layer
 * (store.hpp:88-92,107, store.cpp:162-190). The peer (NULL clears it) must share the id space
 * and outlive its use; host != 0 marks this pool as the host tier. Victims are ordered by a score:
 * the LFU count, 0 for an exclusive host pool's peer-resident experts, and in a late target layer
 * halved (host pool, peer-resident) or doubled (VRAM pool, not peer-resident); a late layer's
 * counts decay every 512 (VRAM) or 128 (host) ticks. switch_target_layer turns layer < 40 late
 * once; a VRAM pool unpins that layer's placement pins and adds one budget slot per pin.
 * fast_minima is accepted for the interface: victims are always the full-scan minimum, which is
 * the reference's cached choice too. ds41_pool_late: 1 if the layer is late. */
int ds41_pool_peer(void *pool, void *peer, int host);
int ds41_pool_exclusive(void *pool, int enabled);
int ds41_pool_decay_interval(void *pool, uint32_t interval);
int ds41_pool_fast_minima(void *pool, int enabled);
int ds41_pool_switch_target_layer(void *pool, const ds41_placement *placement, int layer);
int ds41_pool_late(void *pool, int layer);
/* DriftPolicy (store.hpp:161-178, store.cpp:220-255): a width-one token-major controller over a
 * VRAM pool and its RAM pool (it peers them). Each target layer's demand of a token is bracketed
 * by ds41_drift_before / ds41_drift_after in layer order 0..39; after 128 complete tokens whose
 * VRAM-pin hit rate is below one half, the next token's layer 0 turns every target layer of both
 * pools late. The placement must be soft, distinct, recent 2, decay 256. Errors as the pool's. */
int ds41_drift_create(const ds41_placement *placement, void *vram_pool, void *ram_pool, void **drift,
                      char *error, size_t error_bytes);
int ds41_drift_before(void *drift, const uint32_t *ids, int n);
int ds41_drift_after(void *drift, const uint32_t *ids, int n);
int ds41_drift_active(void *drift);                                   /* 1, 0 */
uint64_t ds41_drift_completed_tokens(void *drift);
const char *ds41_drift_error(void *drift);
int ds41_drift_destroy(void *drift);

/* Dynamic HBM cache for the stack's host-tier experts, the reference's VRAM slot pool in front
 * of its host tier (components/moe/src/offload.cpp:240-381 load, SlotPool policy store.cpp).
 * Allocates `slots` expert slabs in HBM (slots <= 0: as many as the free HBM holds less a 2 GiB
 * reserve, at most layers * n_experts; at least max_tokens * topk), a device map of the cached
 * experts, a pinned patch buffer and events; call before the first step or between steps
 * (synchronous; an existing cache is dropped). A routed host-tier expert that the pool holds is
 * read in place with the resident experts (a hit); a miss is copied from its host slab into the
 * slot the policy assigns, after the copy stream has waited for the last layer that read the
 * slot's previous expert. `policy` (nullable: recent 6, decay 32, distinct, soft, no budgets)
 * applies its recent/decay/lfu/pools/budget fields to the stack's layers (policy->layers must
 * equal the stack's); its pin and host lists are not used, because the stack's resident
 * experts come from each layer's table. Expert id of layer l, expert e: l * n_experts + e. */
int ds41_verify_stack_cache(void *stack, int slots, const ds41_placement *policy);
typedef struct ds41_cache_stats {
  uint32_t abi_version;            /* DS41_GFX950_ABI_VERSION */
  uint32_t struct_bytes;           /* sizeof this struct as the caller was built */
  uint64_t requests;                 /* routed host-tier experts served through the cache */
  uint64_t hits, misses, evictions;  /* hits include experts a prefetch brought in */
  uint64_t h2d_bytes;                /* demand and prefetch copies */
  uint64_t slots;                    /* the cache's size in expert slabs */
  uint64_t prefetch_requests;        /* host-tier experts named by prefetches */
  uint64_t prefetch_copies;          /* of which copied in (the others were cached) */
} ds41_cache_stats;
int ds41_verify_stack_cache_stats(void *stack, ds41_cache_stats *out);
/* Prefetch into the HBM cache (the reference's prefetch_experts, engine/src/hotpath/streamed.inc:
 * 89-108, components/moe/src/offload.cpp): host arrays of n (layer, expert) pairs that the caller
 * expects the coming layers to route. Host-tier experts the cache lacks are acquired (one pool
 * call; the LFU history is left alone), copied in on the copy stream and leased until their layer
 * is next processed; HBM-resident experts are skipped. The layer's plan then finds them in the
 * cache: the step waits (on the device) for a layer's prefetch copies before that layer's plan,
 * and no host-tier copy stands between its plan and its down projection. Call between layers or
 * steps, never while another thread uses the stack. Requires a cache. More experts than the
 * unleased slots: hipErrorOutOfMemory and nothing changes. */
int ds41_verify_stack_prefetch(void *stack, const int32_t *layers, const int32_t *experts, int n);

/* ---- on-disk expert format: records manifest over safetensors shards ------------- */
/* load_records (components/moe/src/manifest.cpp:35-55): the manifest written by the reference's
 * scripts/assets/expert_bank.py export_tsv. "R id bytes (offset bytes) x 6" gives a record
 * buffer of `bytes` and six views into it (gate, gate scales, up, up scales, down, down scales =
 * checkpoint w1/w3/w2 .weight/.scale); "E id "path" file_offset bytes dst_offset required
 * expected_file_bytes" lines give the file ranges that fill it. Ids as in store.hpp:16.
 * Calls return 0 or -1 with the reason in `error` (may be NULL). Host code, no device calls. */
typedef struct ds41_record_info {
  uint32_t id;
  int32_t n_extents;
  uint64_t bytes;
  uint64_t view_offset[6], view_bytes[6];
} ds41_record_info;
typedef struct ds41_record_extent {
  char path[4096];
  uint64_t file_offset, bytes, dst_offset;
  uint64_t required_bytes;          /* 0: all of bytes */
  uint64_t expected_file_bytes;
} ds41_record_extent;
int ds41_records_load(const char *manifest, void **records, char *error, size_t error_bytes);
int ds41_records_free(void *records);
int ds41_records_count(void *records);
int ds41_records_find(void *records, uint32_t id);                   /* index or -1 */
int ds41_records_info(void *records, int index, ds41_record_info *out);
int ds41_records_extent(void *records, int index, int extent, ds41_record_extent *out);
/* The engine's checks before any read (engine/src/forward.cu:1781-1832 validate_records with
 * engine/src/store.cpp:79-91 validate_spans and the checkpoint index/shard checks of
 * store.cpp:140-217): every record reads exactly its expert's six tensors of the safetensors
 * checkpoint under checkpoint_root (model.safetensors.index.json), at their own files and
 * offsets, within required extent coverage, with no extraneous extent. complete != 0 also
 * requires every shard file to have its full size. */
int ds41_records_validate(void *records, const char *checkpoint_root, int complete, char *error,
                          size_t error_bytes);
/* Reads a record's extents into dst (>= bytes). A final extent may stop at EOF once its
 * required bytes have arrived; the rest of it is zeroed. */
int ds41_record_read(void *records, int index, void *dst, size_t dst_bytes, char *error,
                     size_t error_bytes);
/* Repacks a read record into the canonical slab of ds41_expert_slab_layout(hidden, inter); the
 * views must have the shape's tensor sizes. ds41_record_load_slab = read + repack. */
int ds41_record_to_slab(void *records, int index, const void *record_buf, int hidden, int inter,
                        void *slab, size_t slab_bytes, char *error, size_t error_bytes);
int ds41_record_load_slab(void *records, int index, int hidden, int inter, void *slab,
                          size_t slab_bytes, char *error, size_t error_bytes);

/* ---- MTP drafter: routed-expert service and router top-3 -------------------- */
/* The reference's ds41_target_experts_fn service (engine/include/ds41/target_shared.h:28-39),
 * bound by Native::services (engine/src/forward.cu:555-566) to routed_spark
 * (forward.cu:1000-1097). The drafter's routed experts of stage s (logical layer 40 + s,
 * components/moe/include/ds41/store.hpp:16) are table[expert_base + 128 * s + id],
 * id 0..127. */
typedef struct ds41_target_experts_desc {
  uint32_t abi_version;            /* DS41_GFX950_ABI_VERSION */
  uint32_t struct_bytes;           /* sizeof this struct as the caller was built */
  const ds41_device_expert *table; /* device; every drafter expert resident in HBM */
  int32_t expert_base;             /* table index of stage 0, expert 0 */
  int32_t hidden, inter;           /* 5120, 2304 for the drafter */
  float swiglu_limit;              /* 10 (forward.cu:1081) */
  int32_t check_routes;            /* 1: read the ids back and reject invalid or duplicate
                                      routes on the host, as the reference does (one stream
                                      sync per call). 0: the device plan checks them: a
                                      rejected call writes NaN to every output slot and sets
                                      status bit 4 (ds41_take_status), without a host wait. */
  void *stream;                    /* every call must pass this stream (forward.cu:1003) */
  void *const *stage_events;       /* optional: 8 hipEvent_t, start/stop of the launch that
                                      quantises x and plans (one kernel), of nothing (the second
                                      pair is recorded back to back), of gate/up/act and of down */
  int32_t weight_layout;           /* 0: the reference's row-major tensors; 1: every entry points
                                      into slabs tiled by ds41_expert_slab_tile (same outputs,
                                      contiguous weight loads). Not in the reference's struct. */
} ds41_target_experts_desc;
/* Allocates the workspace (8 rows x top-3) and, with check_routes, a pinned id buffer. */
int ds41_target_experts_create(const ds41_target_experts_desc *desc, void **user);
int ds41_target_experts_destroy(void *user);
/* ds41_target_experts_fn: x BF16 [rows][hidden] (rows 1..8), ids int32 [rows][3],
 * weights F32 [rows][3] (all device) -> out BF16 [rows][3][hidden] in top-k slot order,
 * routed experts only. Returns 0, or -1 with ds41_target_experts_error() set; a failure
 * poisons the handle and every later call fails (forward.cu:984-998 service_call). */
int ds41_target_experts(void *user, int stage, const void *x_bf16, const int32_t *ids,
                        const float *weights, void *out_bf16, int rows, void *stream);
/* The last call's error, "" after a success; valid until the next call. */
const char *ds41_target_experts_error(void *user);
/* The drafter's default router top-3 (engine/third_party/spark/src/forward.cu:28-40
 * select3, exported at :154 and spark.h:84): scores F32 [rows][128] -> ids int32 [rows][3]
 * in the tie order of CUDA torch.topk(k=3, sorted=True); rows == 1 sorts with the
 * 4-entry network and rows > 1 with the 32-entry one, as the reference does. */
int ds41_spark_topk3_gpu(const float *scores, int32_t *ids, int rows, void *stream);

/* MXFP4 dequantisation: w [n][k/2] + s [n][k/32] -> fp32 [n][k] (bit-exact). */
int ds41_dequant_mxfp4(const uint8_t *w, const uint8_t *s, float *out, int n, int k,
                       void *stream);

/* hipEvent helpers for timing from hosts without HIP bindings. */
int ds41_events_create(void **events, int n);
int ds41_events_destroy(void **events, int n);
int ds41_event_elapsed_ms(void *start, void *stop, float *ms);
int ds41_event_record(void *event, void *stream);

/* Library version string. */
const char *ds41_gfx950_version(void);

/* Measurement utility with no counterpart in the reference: streams `bytes`
 * (a multiple of 16, 16-byte aligned) from device memory with `blocks`
 * workgroups of 256 threads and writes one word per thread to `sink`
 * (device, blocks * 256 * 4 bytes). Timing it gives the practical HBM read
 * ceiling that the HBM-bound kernels' rates are compared against. */
int ds41_hbm_read_probe(const void *buf, size_t bytes, void *sink, int blocks, void *stream);
/* The same probe with loads_in_flight (4, 8 or 16) 16-byte loads in flight per thread and plain
 * (nontemporal 0) or non-temporal (1) loads; sink holds blocks * 256 words. A caller sweeps
 * these and the grid and takes the best rate as the device's read ceiling. */
int ds41_hbm_read_probe_ex(const void *buf, size_t bytes, void *sink, int blocks, int loads_in_flight,
                           int nontemporal, void *stream);
/* Self-check of the device's E4M3 converter (no counterpart in the reference): the MXFP8
 * quantisers convert with the hardware instruction, which must round exactly as the integer
 * formulation of OCP E4M3 (round to nearest even, saturating) on every fp32 in [-448, 448].
 * Adds the number of disagreeing conversions to *mismatches (device, caller-zeroed) on `stream`;
 * 0 is the only acceptable result. About 2.3e9 inputs; well under a second. */
int ds41_e4m3_converter_check(unsigned long long *mismatches, void *stream);
/* Reads and clears the kernels' status bits (synchronous): 1 a residency wait
 * gave up (the rows that needed those weights are written as NaN), 2 a job's
 * row count was outside 1..8, 4 invalid/duplicate routes. */
int ds41_take_status(uint32_t *status);

#ifdef __cplusplus
}
#endif
#endif
