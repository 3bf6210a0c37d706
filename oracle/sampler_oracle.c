/*
 * Acceptance-sampling restatement: Philox4x32-10 v2 uniforms, fp64 logits ->
 * measure transform with temperature and top-p, and the rejection-sampling
 * verify of engine/third_party/spark/src/sampling.cpp. TEST INFRASTRUCTURE ONLY
 * (see ds41_oracle.h). Sequential fp64 sums in index order, glibc exp.
 */
#include "ds41_oracle.h"
#include <math.h>
#include <stdlib.h>
#include <string.h>

static __thread const char *last_error = "";
const char *oracle_error(void) { return last_error; }
static int fail(const char *msg) { last_error = msg; return -1; }

/* spark_rng.h:23-31. Philox4x32-10 (Salmon et al., SC'11) with the v2 counter
 * {step lo, step hi, draw/4, 0x53500000 | purpose<<3 | slot} and key = seed. */
uint32_t oracle_philox_word_v2(uint64_t seed, uint64_t step, uint32_t slot, uint32_t purpose,
                               uint64_t draw) {
  uint32_t c0 = (uint32_t)step, c1 = (uint32_t)(step >> 32), c2 = (uint32_t)(draw / 4),
           c3 = 0x53500000u | (purpose << 3) | slot;
  uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  for (int r = 0; r < 10; ++r) {
    uint64_t a = (uint64_t)0xD2511F53u * c0, b = (uint64_t)0xCD9E8D57u * c2;
    uint32_t n0 = (uint32_t)(b >> 32) ^ c1 ^ k0, n1 = (uint32_t)b;
    uint32_t n2 = (uint32_t)(a >> 32) ^ c3 ^ k1, n3 = (uint32_t)a;
    c0 = n0; c1 = n1; c2 = n2; c3 = n3;
    k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
  }
  switch (draw % 4) { case 0: return c0; case 1: return c1; case 2: return c2; default: return c3; }
}

/* spark_rng.h:32-36: 27 + 26 random bits -> [0,1) with 2^-53 resolution. */
double oracle_uniform_v2(uint64_t seed, uint64_t step, uint32_t slot, uint32_t purpose, uint64_t draw) {
  uint64_t a = oracle_philox_word_v2(seed, step, slot, purpose, draw * 2) >> 5;
  uint64_t b = oracle_philox_word_v2(seed, step, slot, purpose, draw * 2 + 1) >> 6;
  return (double)((a << 26) | b) * 0x1p-53;
}

/* Stable order by p descending (ties keep the lower index first): bottom-up merge sort. */
static void sort_desc_stable(const double *p, int *idx, int n) {
  int *tmp = (int *)malloc(sizeof(int) * (size_t)n);
  for (int width = 1; width < n; width *= 2) {
    for (int lo = 0; lo < n; lo += 2 * width) {
      int mid = lo + width < n ? lo + width : n, hi = lo + 2 * width < n ? lo + 2 * width : n;
      int i = lo, j = mid, o = lo;
      while (i < mid && j < hi) tmp[o++] = (p[idx[j]] > p[idx[i]]) ? idx[j++] : idx[i++];
      while (i < mid) tmp[o++] = idx[i++];
      while (j < hi) tmp[o++] = idx[j++];
    }
    memcpy(idx, tmp, sizeof(int) * (size_t)n);
  }
  free(tmp);
}

/* sampling.cpp:30-38 ds41_spark_probabilities. */
int oracle_probabilities(const float *x, double *p, int n, double t, double top) {
  if (!x || !p || n < 1 || !isfinite(t) || t < 0 || !isfinite(top) || top <= 0 || top > 1)
    return fail("temperature/top_p/logits");
  int b = 0;
  for (int i = 0; i < n; ++i) {
    if (!isfinite(x[i])) return fail("nonfinite logits");
    if (x[i] > x[b]) b = i;
  }
  for (int i = 0; i < n; ++i) p[i] = 0;
  if (t == 0) { p[b] = 1; return 0; }
  double z = 0;
  for (int i = 0; i < n; ++i) { p[i] = exp(((double)x[i] - x[b]) / t); z += p[i]; }
  for (int i = 0; i < n; ++i) p[i] /= z;
  if (top < 1) {
    int *idx = (int *)malloc(sizeof(int) * (size_t)n);
    if (!idx) return fail("allocation");
    for (int i = 0; i < n; ++i) idx[i] = i;
    sort_desc_stable(p, idx, n);
    double mass = 0;
    int k = 0;
    do { mass += p[idx[k++]]; } while (k < n && mass < top);
    for (int i = k; i < n; ++i) p[idx[i]] = 0;
    for (int i = 0; i < n; ++i) p[i] /= mass;
    free(idx);
  }
  return 0;
}

/* sampling.cpp:12-17 validate: finite, >= 0, |sum - 1| <= 1e-8. */
static int validate(const double *p, int n) {
  if (!p || n < 1) return fail("null/empty probability row");
  double z = 0;
  for (int i = 0; i < n; ++i) {
    if (!isfinite(p[i]) || p[i] < 0) return fail("invalid probability");
    z += p[i];
  }
  if (fabs(z - 1) > 1e-8) return fail("probabilities must be normalized");
  return 0;
}

/* sampling.cpp:18-21 draw: inverse CDF over the sequential running sum. */
static int draw(const double *p, int n, double u, int *out) {
  double z = 0;
  for (int i = 0; i < n; ++i) z += p[i];
  if (!(z > 0)) return fail("empty residual support");
  double t = u * z, c = 0;
  int last = -1;
  for (int i = 0; i < n; ++i) {
    c += p[i];
    if (p[i] > 0) last = i;
    if (t < c) { *out = i; return 0; }
  }
  *out = last;
  return 0;
}

/* sampling.cpp:22 best: first maximum. */
static int best(const double *p, int n) {
  int b = 0;
  for (int i = 1; i < n; ++i) if (p[i] > p[b]) b = i;
  return b;
}

enum { PURPOSE_TARGET = 0, PURPOSE_DRAFT = 1, PURPOSE_ACCEPT = 2, PURPOSE_RESIDUAL = 3 };

/* sampling.cpp:39-53 verify_impl with v2 uniforms. */
int oracle_verify_v2(const int32_t *d, const double *q, const double *p, int count, int n, int greedy,
                     uint64_t seed, uint64_t step, oracle_spark_result *out) {
  if (!out || count < 0 || count > 5 || n < 1 || !p || (count && (!d || (!q && !greedy))))
    return fail("verify arguments");
  oracle_spark_result r;
  memset(&r, 0, sizeof r);
  for (int k = 0; k <= count; ++k)
    if (validate(p + (size_t)k * n, n)) return -1;
  for (int k = 0; k < count; ++k) {
    if (d[k] < 0 || d[k] >= n) return fail("draft id");
    const double *pk = p + (size_t)k * n, *qk = q ? q + (size_t)k * n : NULL;
    int accept;
    if (greedy) accept = d[k] == best(pk, n);
    else {
      if (validate(qk, n)) return -1;
      if (qk[d[k]] <= 0) return fail("draft impossible under logged q");
      double ratio = pk[d[k]] / qk[d[k]];
      accept = oracle_uniform_v2(seed, step, (uint32_t)k, PURPOSE_ACCEPT, 0) < (ratio < 1. ? ratio : 1.);
    }
    if (accept) { r.tokens[r.emitted++] = d[k]; ++r.accepted_drafts; }
    else {
      if (greedy) r.tokens[r.emitted++] = best(pk, n);
      else {
        double *res = (double *)malloc(sizeof(double) * (size_t)n);
        if (!res) return fail("allocation");
        for (int i = 0; i < n; ++i) { double v = pk[i] - qk[i]; res[i] = v > 0. ? v : 0.; }
        int tok, rc = draw(res, n, oracle_uniform_v2(seed, step, (uint32_t)k, PURPOSE_RESIDUAL, 0), &tok);
        free(res);
        if (rc) return -1;
        r.tokens[r.emitted++] = tok;
      }
      r.rejected = 1;
      break;
    }
  }
  if (!r.rejected) {
    const double *last = p + (size_t)count * n;
    int tok;
    if (greedy) tok = best(last, n);
    else if (draw(last, n, oracle_uniform_v2(seed, step, (uint32_t)count, PURPOSE_TARGET, 0), &tok)) return -1;
    r.tokens[r.emitted++] = tok;
  }
  r.accepted_input_rows = r.accepted_drafts + 1;
  *out = r;
  return 0;
}

int oracle_sample_v2(const double *p, int n, uint64_t seed, uint64_t step, uint32_t slot,
                     uint32_t purpose, int32_t *out) {
  if (!out || slot > 5 || purpose > 3) return fail("sample v2 arguments");
  if (validate(p, n)) return -1;
  int tok;
  if (draw(p, n, oracle_uniform_v2(seed, step, slot, purpose, 0), &tok)) return -1;
  *out = tok;
  return 0;
}

int oracle_accept_logits(const float *target_logits, const float *draft_logits, const int32_t *drafts,
                         int count, int n, double temperature, double top_p, uint64_t seed, uint64_t step,
                         oracle_spark_result *out, double *p_out, double *q_out) {
  if (!isfinite(temperature) || temperature < 0 || count < 0 || count > 5) return fail("accept arguments");
  const int greedy = temperature == 0;
  const double t = temperature > 0 ? (temperature > 1e-5 ? temperature : 1e-5) : temperature;
  double *p = p_out ? p_out : (double *)malloc(sizeof(double) * (size_t)(count + 1) * n);
  double *q = NULL;
  int rc = -1;
  if (!p) return fail("allocation");
  if (!greedy && count) {
    q = q_out ? q_out : (double *)malloc(sizeof(double) * (size_t)count * n);
    if (!q) goto done;
    for (int k = 0; k < count; ++k)
      if (oracle_probabilities(draft_logits + (size_t)k * n, q + (size_t)k * n, n, t, top_p)) goto done;
  }
  for (int k = 0; k <= count; ++k)
    if (oracle_probabilities(target_logits + (size_t)k * n, p + (size_t)k * n, n, t, top_p)) goto done;
  rc = oracle_verify_v2(drafts, q, p, count, n, greedy, seed, step, out);
done:
  if (p != p_out) free(p);
  if (q && q != q_out) free(q);
  return rc;
}

/* ---- the reference's GPU sampler over fp32 measures -------------------------------------------
 * engine/third_party/spark/src/sampling.cu, restated for one block of 256 threads executed in
 * order. The fp64 summation orders are those of the kernel: mass = 256 strided per-thread sums
 * then a halving tree (sampling.cu:6-7); draw = 256 contiguous chunk sums, a serial exclusive
 * prefix over the chunks, and an in-chunk scan (sampling.cu:12-22). */
#define GPU_THREADS 256

/* sampling.cu:7 mass: non-finite or negative entries make the sum NaN. */
static double gpu_mass(const float *p, int n) {
  double sh[GPU_THREADS];
  for (int t = 0; t < GPU_THREADS; ++t) {
    double z = 0;
    for (int i = t; i < n; i += GPU_THREADS) {
      double x = p[i];
      if (!isfinite(x) || x < 0) x = NAN;
      z += x;
    }
    sh[t] = z;
  }
  for (int d = GPU_THREADS / 2; d; d >>= 1)
    for (int t = 0; t < d; ++t) sh[t] += sh[t + d];
  return sh[0];
}

/* sampling.cu:8 argmax of a row of finite values: the first maximum. */
static int gpu_argmax(const float *p, int n) {
  int b = 0;
  for (int i = 1; i < n; ++i)
    if (p[i] > p[b]) b = i;
  return b;
}

static double gpu_value(const float *p, const float *q, int i, double pz, double qz) {
  if (!q) return (double)p[i] / pz;
  const double v = (double)p[i] / pz - (double)q[i] / qz;
  return v > 0. ? v : 0.;  /* fmax(0., v); v is never NaN for valid rows */
}

/* sampling.cu:12-22 draw: -1 when no index is selected. */
static int gpu_draw(const float *p, const float *q, int n, double pz, double qz, double u) {
  const int chunk = (n + GPU_THREADS - 1) / GPU_THREADS;
  double pre[GPU_THREADS + 1], sh[GPU_THREADS];
  for (int t = 0; t < GPU_THREADS; ++t) {
    const int begin = t * chunk, end = begin + chunk < n ? begin + chunk : n;
    double z = 0;
    for (int i = begin; i < end; ++i) z += gpu_value(p, q, i, pz, qz);
    sh[t] = z;
  }
  double sum = 0;
  for (int j = 0; j < GPU_THREADS; ++j) {
    pre[j] = sum;
    sum += sh[j];
  }
  pre[GPU_THREADS] = sum;
  const double total = pre[GPU_THREADS], target = u * total;
  int answer = n;
  for (int t = 0; t < GPU_THREADS; ++t) {
    if (!(total > 0 && target >= pre[t] && (t == GPU_THREADS - 1 || target < pre[t + 1]))) continue;
    const int begin = t * chunk, end = begin + chunk < n ? begin + chunk : n;
    double c = pre[t];
    int last = -1;
    for (int i = begin; i < end; ++i) {
      const double v = gpu_value(p, q, i, pz, qz);
      if (v > 0) last = i;
      c += v;
      if (target < c) {
        if (i < answer) answer = i;
        break;
      }
    }
    if (answer == n && last >= 0) answer = last;
  }
  return answer == n ? -1 : answer;
}

/* sampling.cu:25-39 verify_kernel with v2 uniforms (ds41_spark_verify_gpu_v2, sampling.cu:49).
 * Invalid rows or draft ids end the step with emitted = -1 and the fields gathered so far. */
int oracle_spark_verify_gpu_v2(const int32_t *d, const float *q, const float *p, int count, int n, int greedy,
                               uint64_t seed, uint64_t step, oracle_spark_result *out) {
  if (!out || !p || count < 0 || count > 5 || n < 1 || (count && (!d || (!q && !greedy))))
    return fail("verify_gpu_v2 arguments");
  oracle_spark_result r;
  memset(&r, 0, sizeof r);
  for (int k = 0; k <= count; ++k) {
    const float *pk = p + (size_t)k * n;
    const double pz = gpu_mass(pk, n);
    if (!(pz > 0) || !isfinite(pz)) { r.emitted = -1; *out = r; return 0; }
    if (k == count) {
      r.tokens[r.emitted++] = greedy ? gpu_argmax(pk, n)
                                     : gpu_draw(pk, NULL, n, pz, 1, oracle_uniform_v2(seed, step, (uint32_t)k,
                                                                                     PURPOSE_TARGET, 0));
      break;
    }
    const int token = d[k];
    if (token < 0 || token >= n) { r.emitted = -1; *out = r; return 0; }
    const float *qk = q ? q + (size_t)k * n : NULL;
    const double qz = greedy ? 1 : gpu_mass(qk, n);
    if (!greedy && (!(qz > 0) || !isfinite(qz) || !(qk[token] > 0))) { r.emitted = -1; *out = r; return 0; }
    int accept;
    if (greedy) accept = token == gpu_argmax(pk, n);
    else {
      const double ratio = ((double)pk[token] / pz) / ((double)qk[token] / qz);
      accept = oracle_uniform_v2(seed, step, (uint32_t)k, PURPOSE_ACCEPT, 0) < (ratio < 1. ? ratio : 1.);
    }
    if (accept) {
      r.tokens[r.emitted++] = token;
      ++r.accepted_drafts;
    } else {
      r.tokens[r.emitted++] = greedy ? gpu_argmax(pk, n)
                                     : gpu_draw(pk, qk, n, pz, qz,
                                                oracle_uniform_v2(seed, step, (uint32_t)k, PURPOSE_RESIDUAL, 0));
      r.rejected = 1;
      break;
    }
  }
  r.accepted_input_rows = r.accepted_drafts + 1;
  *out = r;
  return 0;
}

/* sampling.cu:23,48 sample_kernel / ds41_spark_sample_gpu_v2: -1 for an invalid row. */
int oracle_spark_sample_gpu_v2(const float *p, int n, uint64_t seed, uint64_t step, uint32_t slot, uint32_t purpose,
                               int32_t *out) {
  if (!p || !out || n < 1 || purpose > 3 || slot > 5) return fail("sample_gpu_v2 arguments");
  const double z = gpu_mass(p, n);
  *out = (!(z > 0) || !isfinite(z)) ? -1 : gpu_draw(p, NULL, n, z, 1, oracle_uniform_v2(seed, step, slot, purpose, 0));
  return 0;
}
