/*
 * ds41 verify-path oracle: a plain-C CPU restatement of the reference's
 * arithmetic for the speculative-decode verify path (MXFP4 routed-expert MoE
 * layer + rejection-sampling accept step).
 *
 * THIS IS TEST INFRASTRUCTURE, NOT PRODUCT CODE. Only tests/, the smoke()
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py may load
 * it, and only as the checker or the timed CPU baseline. The product path
 * (the HIP library under deepseek-v4.1-flash-pro6000_amd/) never calls it.
 *
 * Every function names the reference file:line it restates (paths relative to
 * the reference repository root). Pinning status of each function is listed in
 * the header comments below and in tests/test_oracle_*.py.
 */
#ifndef DS41_ORACLE_H
#define DS41_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar formats ------------------------------------------------------ */
/* bf16 <-> fp32. fp32->bf16 is round-to-nearest-even, NaN kept quiet
 * (the __float2bfloat16_rn boundary used throughout components/moe/src/mxfp4.cu). */
float oracle_bf16_to_f32(uint16_t v);
uint16_t oracle_f32_to_bf16(float v);
/* E2M1 nibble -> value: magnitudes {0,.5,1,1.5,2,3,4,6}, sign = bit 3
 * (components/moe/src/mxfp4.cu:24-29 expand4; OCP MX v1.0 E2M1). */
float oracle_e2m1(uint8_t nibble);
/* E8M0 byte -> 2^(e-127); e==0 -> 2^-127 (0x00400000); e==255 -> NaN
 * (components/moe/src/mxfp4.cu:5-7). */
float oracle_e8m0(uint8_t e);
/* OCP E4M3 (fn) byte -> value (bias 7, subnormals, 0x7f/0xff NaN). */
float oracle_e4m3(uint8_t v);
/* fp32 -> E4M3 with round-to-nearest-even and saturation to +-448
 * (the __nv_cvt_float_to_fp8(.., __NV_SATFINITE, __NV_E4M3) step of
 * components/moe/src/mxfp4.cu:21). NaN -> 0x7f. */
uint8_t oracle_e4m3_from_f32(float v);

/* ---- MX tensors ---------------------------------------------------------- */
/* Dequantise an MXFP4 matrix: w [n][k/2] bytes (low nibble = even k),
 * s [n][k/32] E8M0 -> out [n][k] fp32 = e2m1 * 2^(e-127) (exact). */
void oracle_dequant_mxfp4(const uint8_t *w, const uint8_t *s, int n, int k, float *out);
/* MXFP8 activation quantiser, components/moe/src/mxfp4.cu:8-23 (quant_kernel):
 * per 32-group amax (NaN ignored as fmaxf does), floor 1e-4,
 * e = ceil_pow2_exponent(fp32(amax * (1/448))), q = e4m3_satfinite(clamp(x / 2^(e-127), +-448)).
 * x bf16 [rows][cols] -> q u8 [rows][cols], s u8 [rows][cols/32]. Returns 0 or -1 (cols%32). */
int oracle_quantize_mxfp8(const uint16_t *x, uint8_t *q, uint8_t *s, int rows, int cols);
/* Same quantiser applied to fp32 values that already sit on the bf16 grid. */
void oracle_quantize_mxfp8_f32(const float *x, uint8_t *q, uint8_t *s, int cols);

/* W4A8 projection with the reference's per-K32-group boundary
 * (components/moe/src/mxfp4.cu:46-95 gemm_kernel; the native kernels
 * :113-132/:201-233 keep the same group boundary and serial add):
 *   dot_g  = exact sum over the 32 products e4m3(x) * e2m1(w)   (exact in fp64)
 *   c_g    = fp32(dot_g)
 *   acc    = fp32(acc + fp32(fp32(c_g * sx_g) * sw_g))  for g = 0 .. k/32-1 in order
 *   out    = bf16(acc)
 * w [n][k/2], ws [n][k/32], x [m][k] e4m3, xs [m][k/32]; acc_out [m][n] fp32
 * (may be NULL), out_bf16 [m][n] (may be NULL). Returns 0 or -1 (k%32). */
int oracle_mxfp4_gemm(const uint8_t *w, const uint8_t *ws, const uint8_t *x, const uint8_t *xs,
                      int m, int n, int k, float *acc_out, uint16_t *out_bf16);

/* SwiGLU (+route weight), components/moe/src/mxfp4.cu:323-332 swiglu_kernel:
 * g = min(g, L); u = clamp(u, -L, L) (only when L > 0); h = fp32(fp32(g / fp32(1 + expf(-g))) * u);
 * h = fp32(w[row] * h) when w != NULL; out = bf16(h). expf is evaluated as (float)exp((double)x),
 * the correctly rounded value for practical inputs, in place of CUDA expf (within 2 ulp of it).
 * Pinned by the formula (tests/test_oracle_moe.py swiglu test); bitwise parity with the
 * reference's CUDA expf rounding is unpinned (compared within tolerance only). */
void oracle_swiglu(const uint16_t *g, const uint16_t *u, const float *w, uint16_t *out,
                   int rows, int cols, float limit);

/* ---- router --------------------------------------------------------------- */
/* logits[t][e] = sum_h fp32(x[t][h]) * wg[e][h], summed in fp64 and rounded once
 * to fp32. The reference computes this GEMV with cuBLAS (engine/src/hotpath/batch.inc:23-41,460),
 * whose reduction order is not published: this defines the oracle's value.
 * PARITY UNPINNED against the reference's bits (no reference test or fixture fixes the
 * logits); pinned only to the exact dot product (fp64 check in tests/test_oracle_moe.py). */
void oracle_router_logits(const uint16_t *x, const float *wg, int m, int e, int h, float *logits);
/* components/dense/src/ops.cu:73 router: u = sqrt(z > 20 ? z : log1p(exp(z))), b = u + bias
 * (exp and log1p as the fp32 rounding of the fp64 functions).
 * mode 1 replaces the score by the logistic sigmoid 1/(1+exp(-z)) (a labelled synthetic mode). */
void oracle_router_scores(const float *logits, const float *bias, int m, int n, int mode,
                          float *u, float *b);
/* Top-k per row by biased score, descending, ties -> lower id
 * (engine/src/hotpath/batch.inc:228-237 partial_sort comparator). ids [m][k]. */
void oracle_topk(const float *b, int m, int n, int k, int32_t *ids);
/* The MTP drafter's router top-3 (engine/third_party/spark/src/forward.cu:28-40 select3):
 * scores [m][128] -> ids [m][3]. Pick 3 ids by an upward scan that keeps the first strict
 * maximum; gather the scores above the third pick's score in id order, then the equal ones
 * in id order (3 at most); sort with the bitonic network of 4 entries (m == 1) or 32
 * (m > 1) whose comparator exchanges equal valid pairs.
 * Pinning: distinct scores give the descending top-3 (closed form); the tie order is pinned
 * to the reference's own statement that the 32-entry network reverses a tied pair above
 * the threshold (forward.cu:30-33) and otherwise restated (parity unpinned against torch). */
void oracle_spark_topk3(const float *scores, int m, int32_t *ids);
/* engine/src/ops.cu:59-73 route (== components/dense/src/ops.cu:107 routerweights):
 * k=6: sum = ((s0+s4)+s2) + ((s1+s5)+s3); k=3: sum = (s0+s2)+s1; other k: the same
 * four-accumulator rule. w_i = fp32(fp32(s_i / fp32(sum + 1e-20)) * scale). */
void oracle_route_weights(const float *u, const int32_t *ids, int m, int n, int k, float scale,
                          float *w);

/* ---- route plan / reduce -------------------------------------------------- */
/* engine/include/ds41/hotpath/route_plan.hpp:23-51 plan_routes (without the layer offset):
 * stable sort of the rows*topk slots by expert id. Outputs: n_unique, ids[n_unique]
 * ascending, begin[n_unique], count[n_unique], source[rows*topk] = slot/topk,
 * destination[rows*topk] = slot. Returns -1 on an id outside [0,n_experts) or a
 * duplicate id within one token's routes (the reference throws), else n_unique. */
int oracle_plan_routes(const int32_t *selected, int rows, int topk, int n_experts,
                       int32_t *ids, int32_t *begin, int32_t *count, int32_t *source,
                       int32_t *destination);
/* components/moe/src/mxfp4.cu:333-340 reduce_kernel: per token, add routed rows in
 * ascending expert-id order (fp32 serial), then + shared, -> bf16. routed [rows][topk][h],
 * ids [rows][topk], shared [rows][h] or NULL. Returns -1 on duplicate ids. */
int oracle_reduce_experts(const uint16_t *routed, const int32_t *ids, const uint16_t *shared,
                          uint16_t *out, int rows, int topk, int hidden);

/* ---- one MoE layer (batch.inc:220-335 bmoe + bshared, non-streamed order) ----- */
typedef struct {
  const uint8_t *gate, *gate_scale, *up, *up_scale, *down, *down_scale;
} oracle_expert;
typedef struct {
  int hidden, inter, n_experts, topk;
  int score_mode;      /* 0 sqrt-softplus (reference), 1 sigmoid */
  float route_scale;   /* 1.5 in the reference */
  float swiglu_limit;  /* 10 in the reference */
} oracle_moe_config;
/* x bf16 [m][hidden] -> y bf16 [m][hidden]. Optional outputs (NULL to skip):
 * ids [m][topk], weights [m][topk], logits [m][n_experts]. shared may be NULL.
 * threads: worker threads for the expert projections (<=0: all online cores).
 * Returns 0, or -1 on invalid routes. */
int oracle_moe_layer(const oracle_moe_config *cfg, const uint16_t *x, const float *router_w,
                     const float *router_bias, const oracle_expert *experts,
                     const oracle_expert *shared, int m, uint16_t *y, int32_t *ids_out,
                     float *weights_out, float *logits_out, int threads);
/* The same layer with the routing given: ids [m][topk], route weights [m][topk]
 * (everything after batch.inc:237). Experts with a NULL gate pointer must not be routed. */
int oracle_moe_layer_routed(const oracle_moe_config *cfg, const uint16_t *x, const int32_t *ids,
                            const float *w, const oracle_expert *experts, const oracle_expert *shared,
                            int m, uint16_t *y, int threads);
/* components/dense/src/dense.cu:37-91 W8A8 (basic / parallel kernels): E4M3 weights w [n][k] with one
 * E8M0 scale per 32 x 32 block ws [n/32][k/32], MXFP8 x [m][k] + xs [m][k/32]; per K32 group the exact
 * dot (fp64, exact: products of two E4M3 values span < 2^49) rounded once to fp32, times sx then sw
 * (fp32), added in ascending K into an fp32 accumulator; bf16 out. n % 32 == 0.
 * Pinning: the shared per-group rule is pinned with the MXFP4 GEMM (Python brute force, one-hot and
 * scale-linearity tests); the E4M3 weight decode and 32 x 32 block indexing by a Python brute force
 * over random codes in tests/test_oracle_moe.py. */
int oracle_dense_fp8(const uint8_t *w, const uint8_t *ws, const uint8_t *x, const uint8_t *xs, int m, int n,
                     int k, float *acc_out, uint16_t *out_bf16);
/* The FP8 shared expert (engine/src/hotpath/batch.inc:330-335 bshared): gate/up = dense_fp8 (bf16),
 * components/dense/src/ops.cu:103-106 shared_act (SwiGLU limit 10, bf16, MXFP8), down = dense_fp8. */
int oracle_shared_fp8_ffn(const oracle_expert *e, const uint8_t *xq, const uint8_t *xs, int m, int hidden,
                          int inter, uint16_t *out_bf16);
/* Worker threads used by oracle_mxfp4_gemm and oracle_expert_ffn (default 1). */
void oracle_set_threads(int n);
/* One routed/shared expert FFN on already-quantised input rows (the inner part of
 * oracle_moe_layer): gate/up -> swiglu(w) -> MXFP8 -> down -> bf16 [m][hidden]. */
int oracle_expert_ffn(const oracle_expert *e, const uint8_t *xq, const uint8_t *xs,
                      const float *route_w, int m, int hidden, int inter, float limit,
                      uint16_t *out_bf16, float *down_acc);

/* ---- acceptance sampling (engine/third_party/spark) ------------------------ */
/* Philox4x32-10 v2, engine/third_party/spark/include/ds41/spark_rng.h:23-36. */
uint32_t oracle_philox_word_v2(uint64_t seed, uint64_t step, uint32_t slot, uint32_t purpose,
                               uint64_t draw);
double oracle_uniform_v2(uint64_t seed, uint64_t step, uint32_t slot, uint32_t purpose,
                         uint64_t draw);
/* engine/third_party/spark/src/sampling.cpp:30-38 ds41_spark_probabilities, with the
 * engine adapter's temperature floor max(T, 1e-5) applied by the caller
 * (engine/src/sampling.cpp:208-210). Returns 0 or -1. */
int oracle_probabilities(const float *x, double *p, int n, double t, double top_p);
typedef struct {
  int32_t tokens[6];
  int emitted, accepted_drafts, accepted_input_rows, rejected;
} oracle_spark_result;
/* engine/third_party/spark/src/sampling.cpp:39-56 verify_impl (v2 uniforms). Returns 0 or -1. */
int oracle_verify_v2(const int32_t *d, const double *q, const double *p, int count, int n,
                     int greedy, uint64_t seed, uint64_t step, oracle_spark_result *out);
/* engine/third_party/spark/src/sampling.cpp:59 ds41_spark_sample_v2. Returns 0 or -1. */
int oracle_sample_v2(const double *p, int n, uint64_t seed, uint64_t step, uint32_t slot,
                     uint32_t purpose, int32_t *out);
/* Full accept step from logits (engine/src/speculation.cpp:163-182 after drafting):
 * q_k = probabilities(draft_logits[k]), p_k = probabilities(target_logits[k]) for
 * k <= drafts, then verify_v2. temperature 0 -> greedy. q may be NULL when greedy.
 * p_out/q_out (may be NULL) receive the measures. Returns 0 or -1. */
int oracle_accept_logits(const float *target_logits, const float *draft_logits,
                         const int32_t *drafts, int count, int n, double temperature,
                         double top_p, uint64_t seed, uint64_t step, oracle_spark_result *out,
                         double *p_out, double *q_out);
/* The reference's GPU sampler over fp32 measures, normalised in fp64
 * (engine/third_party/spark/src/sampling.cu:6-39,48-49 verify_kernel / sample_kernel with v2
 * uniforms): the kernel's fp64 summation orders (256 strided sums + halving tree for a row's
 * mass; 256 contiguous chunk sums + serial prefix + in-chunk scan for a draw). Pinned against the
 * compiled reference host sampler where every sum is exact (integer measures over a power-of-two
 * mass), by closed forms and by the distribution test of tests/test_oracle_sampler.py; the
 * summation order itself, where sums round, is restated from the kernel and otherwise unpinned.
 * Invalid rows or ids give emitted = -1 (the kernel's convention). Returns 0, or -1 for bad
 * arguments. */
int oracle_spark_verify_gpu_v2(const int32_t *d, const float *q, const float *p, int count, int n,
                               int greedy, uint64_t seed, uint64_t step, oracle_spark_result *out);
int oracle_spark_sample_gpu_v2(const float *p, int n, uint64_t seed, uint64_t step, uint32_t slot,
                               uint32_t purpose, int32_t *out);
const char *oracle_error(void);

#ifdef __cplusplus
}
#endif
#endif
