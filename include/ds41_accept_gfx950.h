/*
 * ds41 speculative-decode acceptance sampler for MI355X (gfx950): C ABI.
 *
 * GPU replacement of the host fp64 accept step the engine runs after verify
 * (engine/src/speculation.cpp:179-182 -> engine/src/sampling.cpp:142-275 ->
 * engine/third_party/spark/src/sampling.cpp:30-56 ds41_spark_probabilities +
 * ds41_spark_verify_v2). All pointers are device memory; `stream` is a
 * hipStream_t passed as void*; returns a hipError_t value as int.
 */
#ifndef DS41_ACCEPT_GFX950_H
#define DS41_ACCEPT_GFX950_H
#include <stddef.h>
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* engine/third_party/spark/include/ds41/spark.h ds41_spark_result. emitted == -1
 * marks an invalid input (non-finite logits, draft id out of range, q[d] == 0),
 * where the host sampler throws. */
typedef struct ds41_spark_result {
  int32_t tokens[6];
  int emitted, accepted_drafts, accepted_input_rows, rejected;
} ds41_spark_result;

/* Device workspace for ds41_spark_verify_logits_gpu_v2 (drafts <= 5). */
size_t ds41_spark_accept_workspace_bytes(int drafts, int vocab);

/* The whole accept step from fp32 logits: probabilities of every target row
 * [drafts+1][vocab] and draft row [drafts][vocab] with temperature floor
 * max(T, 1e-5) (T == 0: greedy, draft_logits may be NULL), then verify_v2 with
 * Philox v2 uniforms (seed, step). Decisions and tokens equal the host
 * sampler's: a decision whose margin is within the bound on the difference
 * between parallel and sequential fp64 sums is recomputed with sequential sums.
 * flags bit 0 forces that sequential path for every decision (testing).
 * top_p < 1 with T > 0 returns hipErrorNotSupported in this version. */
int ds41_spark_verify_logits_gpu_v2(const float *target_logits, const float *draft_logits,
                                    const int32_t *drafts_dev, int drafts, int vocab,
                                    double temperature, double top_p, uint64_t seed, uint64_t step,
                                    ds41_spark_result *out, void *workspace, size_t workspace_bytes,
                                    int flags, void *stream);
/* The spark GPU sampler over fp32 measures (engine/third_party/spark/src/sampling.cu:25-49,
 * declared in spark.h:133-134): p [drafts+1][vocab] and q [drafts][vocab] (q may be NULL when
 * greedy) are unnormalised non-negative fp32 measures; each row is normalised by its fp64
 * mass, with the reference kernel's summation orders, so decisions and tokens equal its.
 * Writes a device ds41_spark_result; an invalid row or draft id gives emitted == -1.
 * One workgroup; no workspace. Returns the launch error (hipErrorInvalidValue for bad
 * arguments, as the reference). */
int ds41_spark_verify_gpu_v2(const int32_t *drafts_dev, const float *q, const float *p,
                             int drafts, int vocab, int greedy, uint64_t seed, uint64_t step,
                             ds41_spark_result *out, void *stream);
/* sample_kernel (sampling.cu:23,48): one token of measure p with the v2 uniform of
 * (seed, step, slot, purpose); -1 for an invalid row. out: device int32. */
int ds41_spark_sample_gpu_v2(const float *p, int vocab, uint64_t seed, uint64_t step, uint32_t slot,
                             uint32_t purpose, int32_t *out, void *stream);
/* Number of accept steps that took the sequential path since the workspace was
 * zeroed (synchronous read). */
int ds41_spark_accept_fallbacks(const void *workspace, int drafts, int vocab, uint32_t *count);

/* Philox v2 purposes (spark.h:109). */
enum ds41_spark_purpose { DS41_SPARK_TARGET = 0, DS41_SPARK_DRAFT = 1, DS41_SPARK_ACCEPT = 2, DS41_SPARK_RESIDUAL = 3 };

/* Token sampling from fp32 logits on the device: for each row r of logits [rows][vocab], the
 * engine's sample(probabilities(x_r, T, top_p), rng, step, first_slot + r, purpose)
 * (engine/src/sampling.cpp:205-226), which SpeculativeStep uses to draw draft token k from q_k
 * with (step, k, DS41_SPARK_DRAFT) (engine/src/speculation.cpp:147-155); T == 0 gives the first
 * argmax (speculation.cpp:149). tokens: device int32 [rows], -1 for a row with a non-finite
 * logit. Tokens equal the host sampler's: a draw whose margin is within the bound on the
 * difference between parallel and sequential fp64 sums is redone with sequential sums.
 * rows 1..6 with first_slot + rows - 1 <= 5, purpose 0..3; flags bit 0 forces the sequential
 * path (testing). Workspace: ds41_spark_sample_workspace_bytes(rows, vocab) device bytes; calls
 * sharing one workspace must be ordered. No counterpart entry in the reference (its drafts are
 * sampled on the host). */
size_t ds41_spark_sample_workspace_bytes(int rows, int vocab);
int ds41_spark_sample_logits_gpu_v2(const float *logits, int rows, int vocab, double temperature,
                                    double top_p, uint64_t seed, uint64_t step, uint32_t first_slot,
                                    uint32_t purpose, int32_t *tokens, void *workspace,
                                    size_t workspace_bytes, int flags, void *stream);

/* ---- host sampler C ABI (engine/third_party/spark/include/ds41/spark.h:115-132), host memory.
 * Each returns 0 (or the value) on success and -1 (a word: 0, a uniform: NaN) on invalid input,
 * with the reason in ds41_spark_error(), a thread-local string valid until the thread's next
 * failing call. The results equal libds41_spark's bit for bit. */
const char *ds41_spark_error(void);
/* p [vocab] = exp((x - x_b) / t) / z in fp64 (b = first argmax, z summed in index order), T == 0
 * one-hot at b; top_p < 1 keeps the shortest prefix in (p desc, index asc) order whose
 * sequential mass reaches top_p and divides by that mass. */
int ds41_spark_probabilities(const float *logits, double *p, int vocab, double temperature,
                             double top_p);
uint32_t ds41_spark_rng_word_v2(uint64_t seed, uint64_t step, uint32_t slot, uint32_t purpose,
                                uint64_t draw);
double ds41_spark_uniform_v2(uint64_t seed, uint64_t step, uint32_t slot, uint32_t purpose,
                             uint64_t draw);
/* One token of the normalised row p with uniform 0 of (seed, step, slot, purpose). */
int ds41_spark_sample_v2(const double *p, int vocab, uint64_t seed, uint64_t step, uint32_t slot,
                         uint32_t purpose, int32_t *token);
/* The accept/reject/residual/bonus decisions over p [(drafts+1)][vocab] and q [drafts][vocab]
 * (q may be NULL when greedy), drafts <= 5. */
int ds41_spark_verify_v2(const int32_t *drafts_ids, const double *q, const double *p, int drafts,
                         int vocab, int greedy, uint64_t seed, uint64_t step,
                         ds41_spark_result *out);

#ifdef __cplusplus
}
#endif
#endif
