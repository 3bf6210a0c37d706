/*
 * MXFP4 / MXFP8 / router / route-plan / reduce restatement of the reference's
 * MoE verify arithmetic. TEST INFRASTRUCTURE ONLY (see ds41_oracle.h).
 * Built with -ffp-contract=off and without fast-math so every float operation
 * rounds to fp32 exactly once, as the reference's __fadd_rn/__fmul_rn do.
 */
#define _GNU_SOURCE
#include "ds41_oracle.h"
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

static float f32_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static uint32_t bits_from_f32(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

float oracle_bf16_to_f32(uint16_t v) { return f32_from_bits((uint32_t)v << 16); }

uint16_t oracle_f32_to_bf16(float v) {
  uint32_t u = bits_from_f32(v);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40); /* quiet NaN */
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* OCP MX E2M1: 1 sign, 2 exponent (bias 1), 1 mantissa bit. */
float oracle_e2m1(uint8_t nibble) {
  static const float mag[8] = {0.0f, 0.5f, 1.0f, 1.5f, 2.0f, 3.0f, 4.0f, 6.0f};
  float v = mag[nibble & 7];
  return (nibble & 8) ? -v : v;
}

float oracle_e8m0(uint8_t e) {
  if (e == 0) return f32_from_bits(0x00400000u);
  if (e == 255) return f32_from_bits(0x7fffffffu);
  return f32_from_bits((uint32_t)e << 23);
}

float oracle_e4m3(uint8_t v) {
  int s = v >> 7, e = (v >> 3) & 15, m = v & 7;
  float x;
  if (e == 15 && m == 7) return f32_from_bits(s ? 0xffc00000u : 0x7fc00000u);
  if (e == 0) x = ldexpf((float)m, -9);
  else x = ldexpf((float)(8 + m), e - 10);
  return s ? -x : x;
}

uint8_t oracle_e4m3_from_f32(float v) {
  if (isnan(v)) return 0x7f;
  uint8_t sign = signbit(v) ? 0x80 : 0x00;
  float a = fabsf(v);
  if (a >= 448.0f) return sign | 0x7e;
  if (a < 0.015625f) {               /* below 2^-6: subnormal grid of 2^-9 */
    float m = rintf(a * 512.0f);     /* exact scaling, ties to even */
    return sign | (uint8_t)m;        /* m == 8 is the smallest normal 0x08 */
  }
  uint32_t u = bits_from_f32(a);
  int e = (int)(u >> 23) - 127;
  uint32_t mant = u & 0x7fffffu, r = mant >> 20, rem = mant & 0xfffffu;
  if (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) ++r;
  if (r == 8) { r = 0; ++e; }
  if (e > 8 || (e == 8 && r > 6)) return sign | 0x7e;
  return sign | (uint8_t)(((e + 7) << 3) | (int)r);
}

void oracle_dequant_mxfp4(const uint8_t *w, const uint8_t *s, int n, int k, float *out) {
  for (int r = 0; r < n; ++r)
    for (int c = 0; c < k; ++c) {
      uint8_t byte = w[(size_t)r * (k / 2) + c / 2];
      uint8_t nib = (c & 1) ? (byte >> 4) : (byte & 15);
      out[(size_t)r * k + c] = oracle_e2m1(nib) * oracle_e8m0(s[(size_t)r * (k / 32) + c / 32]);
    }
}

/* One 32-group of mxfp4.cu:12-22. v holds 32 fp32 values (bf16-representable). */
static void quant_group(const float *v, uint8_t *q, uint8_t *s) {
  float amax = NAN;
  for (int i = 0; i < 32; ++i) amax = fmaxf(amax, fabsf(v[i])); /* fmaxf drops NaN */
  amax = fmaxf(amax, 1e-4f);
  uint32_t b = bits_from_f32(amax * (1.0f / 448.0f));
  uint32_t e = (b >> 23) + ((b & 0x7fffffu) != 0);
  float scale = f32_from_bits(e << 23);
  for (int i = 0; i < 32; ++i) q[i] = oracle_e4m3_from_f32(fminf(448.0f, fmaxf(-448.0f, v[i] / scale)));
  *s = (uint8_t)e;
}

void oracle_quantize_mxfp8_f32(const float *x, uint8_t *q, uint8_t *s, int cols) {
  for (int g = 0; g < cols / 32; ++g) quant_group(x + g * 32, q + g * 32, s + g);
}

int oracle_quantize_mxfp8(const uint16_t *x, uint8_t *q, uint8_t *s, int rows, int cols) {
  if (rows < 1 || cols < 1 || cols % 32) return -1;
  float v[32];
  for (int r = 0; r < rows; ++r)
    for (int g = 0; g < cols / 32; ++g) {
      for (int i = 0; i < 32; ++i) v[i] = oracle_bf16_to_f32(x[(size_t)r * cols + g * 32 + i]);
      quant_group(v, q + (size_t)r * cols + g * 32, s + (size_t)r * (cols / 32) + g);
    }
  return 0;
}

/* ---- thread helper -------------------------------------------------------- */
typedef void (*range_fn)(void *ctx, int begin, int end);
typedef struct { range_fn fn; void *ctx; int begin, end; } range_job;
static void *range_main(void *p) { range_job *j = (range_job *)p; j->fn(j->ctx, j->begin, j->end); return NULL; }
static int online_cores(void) { long n = sysconf(_SC_NPROCESSORS_ONLN); return n > 0 ? (int)n : 1; }
static void parallel_range(int n, int threads, range_fn fn, void *ctx) {
  if (threads <= 0) threads = online_cores();
  if (threads > n) threads = n;
  if (threads <= 1) { fn(ctx, 0, n); return; }
  pthread_t tid[256];
  range_job jobs[256];
  if (threads > 256) threads = 256;
  for (int t = 0; t < threads; ++t) {
    jobs[t].fn = fn; jobs[t].ctx = ctx;
    jobs[t].begin = (int)((long)n * t / threads);
    jobs[t].end = (int)((long)n * (t + 1) / threads);
  }
  int started = 1;
  for (int t = 1; t < threads; ++t, ++started)
    if (pthread_create(&tid[t], NULL, range_main, &jobs[t])) break;
  for (int t = started; t < threads; ++t) fn(ctx, jobs[t].begin, jobs[t].end);
  fn(ctx, jobs[0].begin, jobs[0].end);
  for (int t = 1; t < started; ++t) pthread_join(tid[t], NULL);
}

/* ---- W4A8 projection -------------------------------------------------------- */
typedef struct {
  const uint8_t *w, *ws;
  const double *xd;  /* [m][k] decoded e4m3 */
  const float *sx;   /* [m][k/32] decoded e8m0 */
  int m, n, k;
  float *acc_out;
  uint16_t *out;
  int fp8; /* 1: E4M3 weights [n][k], one E8M0 scale per 32 x 32 block [n/32][k/32] */
} gemm_ctx;

static void gemm_rows(void *p, int begin, int end) {
  gemm_ctx *c = (gemm_ctx *)p;
  const int ng = c->k / 32;
  double wd[32];
  float acc[64];
  for (int row = begin; row < end; ++row) {
    for (int t0 = 0; t0 < c->m; t0 += 64) {
      int tn = c->m - t0 < 64 ? c->m - t0 : 64;
      for (int t = 0; t < tn; ++t) acc[t] = 0.0f;
      for (int g = 0; g < ng; ++g) {
        float sw;
        if (c->fp8) {
          const uint8_t *src = c->w + (size_t)row * c->k + g * 32;
          for (int i = 0; i < 32; ++i) wd[i] = oracle_e4m3(src[i]);
          sw = oracle_e8m0(c->ws[(size_t)(row / 32) * ng + g]);
        } else {
          const uint8_t *src = c->w + (size_t)row * (c->k / 2) + g * 16;
          for (int i = 0; i < 16; ++i) {
            wd[2 * i] = oracle_e2m1(src[i] & 15);
            wd[2 * i + 1] = oracle_e2m1(src[i] >> 4);
          }
          sw = oracle_e8m0(c->ws[(size_t)row * ng + g]);
        }
        for (int t = 0; t < tn; ++t) {
          const double *x = c->xd + (size_t)(t0 + t) * c->k + g * 32;
          double dot = 0.0;
          for (int i = 0; i < 32; ++i) dot += x[i] * wd[i]; /* exact: the products span < 2^49 */
          float cg = (float)dot;
          float term = (cg * c->sx[(size_t)(t0 + t) * ng + g]) * sw;
          acc[t] = acc[t] + term;
        }
      }
      for (int t = 0; t < tn; ++t) {
        size_t o = (size_t)(t0 + t) * c->n + row;
        if (c->acc_out) c->acc_out[o] = acc[t];
        if (c->out) c->out[o] = oracle_f32_to_bf16(acc[t]);
      }
    }
  }
}

static int gemm_threads = 1;
static int gemm_any(const uint8_t *w, const uint8_t *ws, const uint8_t *x, const uint8_t *xs, int m, int n,
                    int k, float *acc_out, uint16_t *out_bf16, int threads, int fp8) {
  if (m < 1 || n < 1 || k < 32 || k % 32 || (fp8 && n % 32)) return -1;
  double *xd = (double *)malloc(sizeof(double) * (size_t)m * k);
  float *sx = (float *)malloc(sizeof(float) * (size_t)m * (k / 32));
  if (!xd || !sx) { free(xd); free(sx); return -1; }
  for (size_t i = 0; i < (size_t)m * k; ++i) xd[i] = oracle_e4m3(x[i]);
  for (size_t i = 0; i < (size_t)m * (k / 32); ++i) sx[i] = oracle_e8m0(xs[i]);
  gemm_ctx c = {w, ws, xd, sx, m, n, k, acc_out, out_bf16, fp8};
  parallel_range(n, threads, gemm_rows, &c);
  free(xd);
  free(sx);
  return 0;
}
static int gemm_impl(const uint8_t *w, const uint8_t *ws, const uint8_t *x, const uint8_t *xs, int m,
                     int n, int k, float *acc_out, uint16_t *out_bf16, int threads) {
  return gemm_any(w, ws, x, xs, m, n, k, acc_out, out_bf16, threads, 0);
}

int oracle_mxfp4_gemm(const uint8_t *w, const uint8_t *ws, const uint8_t *x, const uint8_t *xs,
                      int m, int n, int k, float *acc_out, uint16_t *out_bf16) {
  return gemm_impl(w, ws, x, xs, m, n, k, acc_out, out_bf16, gemm_threads);
}

/* exp / log1p as the fp32 rounding of the fp64 function (the correctly rounded fp32 value for all
 * practical inputs); the GPU kernels evaluate the same expression. */
static float exp_f32(float x) { return (float)exp((double)x); }
static float log1p_f32(float x) { return (float)log1p((double)x); }

void oracle_swiglu(const uint16_t *g, const uint16_t *u, const float *w, uint16_t *out, int rows,
                   int cols, float limit) {
  for (int r = 0; r < rows; ++r)
    for (int c = 0; c < cols; ++c) {
      size_t i = (size_t)r * cols + c;
      float gv = oracle_bf16_to_f32(g[i]), uv = oracle_bf16_to_f32(u[i]);
      if (limit > 0) { gv = fminf(gv, limit); uv = fminf(limit, fmaxf(-limit, uv)); }
      float den = 1.0f + exp_f32(-gv);
      float h = (gv / den) * uv;
      if (w) h = w[r] * h;
      out[i] = oracle_f32_to_bf16(h);
    }
}

/* ---- router ----------------------------------------------------------------- */
void oracle_router_logits(const uint16_t *x, const float *wg, int m, int e, int h, float *logits) {
  for (int t = 0; t < m; ++t)
    for (int j = 0; j < e; ++j) {
      double s = 0.0;
      for (int i = 0; i < h; ++i) s += (double)oracle_bf16_to_f32(x[(size_t)t * h + i]) * (double)wg[(size_t)j * h + i];
      logits[(size_t)t * e + j] = (float)s;
    }
}

void oracle_router_scores(const float *logits, const float *bias, int m, int n, int mode, float *u,
                          float *b) {
  for (int i = 0; i < m * n; ++i) {
    float z = logits[i], v;
    if (mode == 1) v = 1.0f / (1.0f + exp_f32(-z));
    else v = sqrtf(z > 20.0f ? z : log1p_f32(exp_f32(z)));
    u[i] = v;
    b[i] = v + bias[i % n];
  }
}

static int better(const float *s, int a, int c) { return s[a] == s[c] ? a < c : s[a] > s[c]; }

void oracle_topk(const float *b, int m, int n, int k, int32_t *ids) {
  for (int r = 0; r < m; ++r) {
    const float *s = b + (size_t)r * n;
    int32_t *out = ids + (size_t)r * k;
    int have = 0;
    for (int i = 0; i < n; ++i) { /* insertion into a sorted list of the best k */
      if (have == k && !better(s, i, out[k - 1])) continue;
      int pos = have < k ? have++ : k - 1;
      while (pos > 0 && better(s, i, out[pos - 1])) { out[pos] = out[pos - 1]; --pos; }
      out[pos] = i;
    }
  }
}

/* Compare-exchange of the drafter's top-3 network: the test is "a is a valid
 * entry with a strictly larger value, or b is padding"; the pair is exchanged
 * when the test equals the stage direction. */
static void top3_cex(float *v, int32_t *id, int *ok, int a, int b, int dir) {
  const int test = (v[a] > v[b] && ok[a]) || !ok[b];
  if (test != dir) return;
  float fv = v[a]; v[a] = v[b]; v[b] = fv;
  int32_t fi = id[a]; id[a] = id[b]; id[b] = fi;
  int fo = ok[a]; ok[a] = ok[b]; ok[b] = fo;
}

void oracle_spark_topk3(const float *scores, int m, int32_t *ids) {
  const int n = 128, width = m == 1 ? 4 : 32;
  for (int r = 0; r < m; ++r) {
    const float *s = scores + (size_t)r * n;
    int pick[3];
    for (int k = 0; k < 3; ++k) { /* scan upward; replace only by a strictly larger score */
      int best = -1;
      for (int i = 0; i < n; ++i) {
        int taken = 0;
        for (int j = 0; j < k; ++j) taken |= pick[j] == i;
        if (taken) continue;
        if (best < 0 || s[i] > s[best]) best = i;
      }
      pick[k] = best;
    }
    const float thr = s[pick[2]];
    float v[32];
    int32_t id[32];
    int ok[32];
    for (int i = 0; i < 32; ++i) { v[i] = 0.0f; id[i] = 0; ok[i] = i < 3; }
    int got = 0;
    for (int i = 0; i < n; ++i)
      if (s[i] > thr) { v[got] = s[i]; id[got++] = i; }
    for (int i = 0; i < n && got < 3; ++i)
      if (s[i] == thr) { v[got] = s[i]; id[got++] = i; }
    /* bitonic network over `width` entries: pair p of a stage with half-span h
     * joins entries lo = 2p - (p mod h) and lo + h */
    for (int size = 2; size < width; size *= 2)
      for (int h = size / 2; h >= 1; h /= 2)
        for (int p = 0; p < width / 2; ++p) {
          const int lo = 2 * p - (p & (h - 1));
          top3_cex(v, id, ok, lo, lo + h, (p & (size / 2)) != 0);
        }
    for (int h = width / 2; h >= 1; h /= 2)
      for (int p = 0; p < width / 2; ++p) {
        const int lo = 2 * p - (p & (h - 1));
        top3_cex(v, id, ok, lo, lo + h, 0);
      }
    for (int k = 0; k < 3; ++k) ids[(size_t)r * 3 + k] = id[k];
  }
}

void oracle_route_weights(const float *u, const int32_t *ids, int m, int n, int k, float scale,
                          float *w) {
  for (int r = 0; r < m; ++r) {
    const float *s = u + (size_t)r * n;
    const int32_t *id = ids + (size_t)r * k;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < k; ++i) v[i % 4] = v[i % 4] + s[id[i]];
    float sum = k == 3 ? (v[0] + v[2]) + v[1] : (v[0] + v[2]) + (v[1] + v[3]);
    sum = sum + 1e-20f;
    for (int i = 0; i < k; ++i) w[(size_t)r * k + i] = (s[id[i]] / sum) * scale;
  }
}

/* ---- route plan / reduce -------------------------------------------------- */
int oracle_plan_routes(const int32_t *selected, int rows, int topk, int n_experts, int32_t *ids,
                       int32_t *begin, int32_t *count, int32_t *source, int32_t *destination) {
  int total = rows * topk;
  if (rows < 1 || topk < 1) return -1;
  int *order = (int *)malloc(sizeof(int) * (size_t)total);
  if (!order) return -1;
  for (int i = 0; i < total; ++i) {
    if (selected[i] < 0 || selected[i] >= n_experts) { free(order); return -1; }
    for (int j = i / topk * topk; j < i; ++j)
      if (selected[i] == selected[j]) { free(order); return -1; }
    order[i] = i;
  }
  for (int i = 1; i < total; ++i) { /* stable insertion sort by expert id */
    int v = order[i], j = i;
    while (j > 0 && selected[order[j - 1]] > selected[v]) { order[j] = order[j - 1]; --j; }
    order[j] = v;
  }
  int u = 0;
  for (int i = 0; i < total; ++i) {
    int slot = order[i];
    if (u == 0 || ids[u - 1] != selected[slot]) { ids[u] = selected[slot]; begin[u] = i; count[u] = 0; ++u; }
    ++count[u - 1];
    source[i] = slot / topk;
    destination[i] = slot;
  }
  free(order);
  return u;
}

int oracle_reduce_experts(const uint16_t *routed, const int32_t *ids, const uint16_t *shared,
                          uint16_t *out, int rows, int topk, int hidden) {
  for (int t = 0; t < rows; ++t) {
    int chosen[16];
    int last = -1;
    for (int i = 0; i < topk; ++i) {
      int pick = -1, smallest = 0x7fffffff;
      for (int j = 0; j < topk; ++j) {
        int id = ids[t * topk + j];
        if (id > last && id < smallest) { pick = j; smallest = id; }
      }
      if (pick < 0) return -1;
      chosen[i] = pick;
      last = smallest;
    }
    for (int h = 0; h < hidden; ++h) {
      float acc = 0.0f;
      for (int i = 0; i < topk; ++i)
        acc = acc + oracle_bf16_to_f32(routed[((size_t)t * topk + chosen[i]) * hidden + h]);
      if (shared) acc = acc + oracle_bf16_to_f32(shared[(size_t)t * hidden + h]);
      out[(size_t)t * hidden + h] = oracle_f32_to_bf16(acc);
    }
  }
  return 0;
}

/* ---- expert FFN and full layer -------------------------------------------- */
static int expert_ffn_threads(const oracle_expert *e, const uint8_t *xq, const uint8_t *xs,
                              const float *route_w, int m, int hidden, int inter, float limit,
                              uint16_t *out_bf16, float *down_acc, int threads) {
  size_t mi = (size_t)m * inter;
  uint16_t *g = (uint16_t *)malloc(mi * 2), *u = (uint16_t *)malloc(mi * 2), *h = (uint16_t *)malloc(mi * 2);
  uint8_t *hq = (uint8_t *)malloc(mi), *hs = (uint8_t *)malloc(mi / 32 + 1);
  int rc = -1;
  if (!g || !u || !h || !hq || !hs) goto done;
  if (gemm_impl(e->gate, e->gate_scale, xq, xs, m, inter, hidden, NULL, g, threads)) goto done;
  if (gemm_impl(e->up, e->up_scale, xq, xs, m, inter, hidden, NULL, u, threads)) goto done;
  oracle_swiglu(g, u, route_w, h, m, inter, limit);
  if (oracle_quantize_mxfp8(h, hq, hs, m, inter)) goto done;
  if (gemm_impl(e->down, e->down_scale, hq, hs, m, hidden, inter, down_acc, out_bf16, threads)) goto done;
  rc = 0;
done:
  free(g); free(u); free(h); free(hq); free(hs);
  return rc;
}

int oracle_expert_ffn(const oracle_expert *e, const uint8_t *xq, const uint8_t *xs,
                      const float *route_w, int m, int hidden, int inter, float limit,
                      uint16_t *out_bf16, float *down_acc) {
  return expert_ffn_threads(e, xq, xs, route_w, m, hidden, inter, limit, out_bf16, down_acc, gemm_threads);
}

int oracle_moe_layer_routed(const oracle_moe_config *cfg, const uint16_t *x, const int32_t *ids,
                            const float *w, const oracle_expert *experts, const oracle_expert *shared,
                            int m, uint16_t *y, int threads) {
  const int H = cfg->hidden, I = cfg->inter, E = cfg->n_experts, K = cfg->topk;
  const int total = m * K;
  int rc = -1, u;
  int32_t *uid = (int32_t *)malloc(sizeof(int32_t) * total), *beg = (int32_t *)malloc(sizeof(int32_t) * total);
  int32_t *cnt = (int32_t *)malloc(sizeof(int32_t) * total), *src = (int32_t *)malloc(sizeof(int32_t) * total);
  int32_t *dst = (int32_t *)malloc(sizeof(int32_t) * total);
  uint8_t *xq = (uint8_t *)malloc((size_t)m * H), *xs = (uint8_t *)malloc((size_t)m * H / 32);
  uint8_t *gq = (uint8_t *)malloc((size_t)total * H), *gs = (uint8_t *)malloc((size_t)total * H / 32);
  float *gw = (float *)malloc(sizeof(float) * total);
  uint16_t *compact = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)total * H);
  uint16_t *routed = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)total * H);
  uint16_t *sh = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)m * H);
  if (!uid || !beg || !cnt || !src || !dst || !xq || !xs || !gq || !gs || !gw || !compact || !routed || !sh)
    goto done;
  u = oracle_plan_routes(ids, m, K, E, uid, beg, cnt, src, dst);
  if (u < 0) goto done;
  oracle_quantize_mxfp8(x, xq, xs, m, H);
  for (int r = 0; r < total; ++r) { /* hotpath/kernels.cu:13-20 gather */
    memcpy(gq + (size_t)r * H, xq + (size_t)src[r] * H, H);
    memcpy(gs + (size_t)r * H / 32, xs + (size_t)src[r] * H / 32, H / 32);
    gw[r] = w[dst[r]];
  }
  for (int e = 0; e < u; ++e) {
    int b0 = beg[e];
    if (!experts[uid[e]].gate) goto done; /* routed to an expert the caller did not provide */
    if (expert_ffn_threads(&experts[uid[e]], gq + (size_t)b0 * H, gs + (size_t)b0 * H / 32, gw + b0,
                           cnt[e], H, I, cfg->swiglu_limit, compact + (size_t)b0 * H, NULL, threads))
      goto done;
  }
  for (int r = 0; r < total; ++r) /* hotpath/kernels.cu:28-31 scatter */
    memcpy(routed + (size_t)dst[r] * H, compact + (size_t)r * H, sizeof(uint16_t) * H);
  if (shared && expert_ffn_threads(shared, xq, xs, NULL, m, H, I, cfg->swiglu_limit, sh, NULL, threads))
    goto done;
  if (oracle_reduce_experts(routed, ids, shared ? sh : NULL, y, m, K, H)) goto done;
  rc = 0;
done:
  free(uid); free(beg); free(cnt); free(src); free(dst); free(xq); free(xs); free(gq); free(gs);
  free(gw); free(compact); free(routed); free(sh);
  return rc;
}

int oracle_moe_layer(const oracle_moe_config *cfg, const uint16_t *x, const float *router_w,
                     const float *router_bias, const oracle_expert *experts,
                     const oracle_expert *shared, int m, uint16_t *y, int32_t *ids_out,
                     float *weights_out, float *logits_out, int threads) {
  const int H = cfg->hidden, E = cfg->n_experts, K = cfg->topk;
  int rc = -1;
  float *logits = (float *)malloc(sizeof(float) * (size_t)m * E);
  float *su = (float *)malloc(sizeof(float) * (size_t)m * E), *sb = (float *)malloc(sizeof(float) * (size_t)m * E);
  int32_t *ids = (int32_t *)malloc(sizeof(int32_t) * (size_t)m * K);
  float *w = (float *)malloc(sizeof(float) * (size_t)m * K);
  if (!logits || !su || !sb || !ids || !w) goto done;
  oracle_router_logits(x, router_w, m, E, H, logits);
  oracle_router_scores(logits, router_bias, m, E, cfg->score_mode, su, sb);
  oracle_topk(sb, m, E, K, ids);
  oracle_route_weights(su, ids, m, E, K, cfg->route_scale, w);
  if (oracle_moe_layer_routed(cfg, x, ids, w, experts, shared, m, y, threads)) goto done;
  if (ids_out) memcpy(ids_out, ids, sizeof(int32_t) * (size_t)m * K);
  if (weights_out) memcpy(weights_out, w, sizeof(float) * (size_t)m * K);
  if (logits_out) memcpy(logits_out, logits, sizeof(float) * (size_t)m * E);
  rc = 0;
done:
  free(logits); free(su); free(sb); free(ids); free(w);
  return rc;
}

int oracle_dense_fp8(const uint8_t *w, const uint8_t *ws, const uint8_t *x, const uint8_t *xs, int m, int n,
                     int k, float *acc_out, uint16_t *out_bf16) {
  return gemm_any(w, ws, x, xs, m, n, k, acc_out, out_bf16, gemm_threads, 1);
}

int oracle_shared_fp8_ffn(const oracle_expert *e, const uint8_t *xq, const uint8_t *xs, int m, int hidden,
                          int inter, uint16_t *out_bf16) {
  int rc = -1;
  uint16_t *g = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)m * inter);
  uint16_t *u = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)m * inter);
  uint16_t *h = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)m * inter);
  uint8_t *hq = (uint8_t *)malloc((size_t)m * inter);
  uint8_t *hs = (uint8_t *)malloc((size_t)m * inter / 32);
  if (!g || !u || !h || !hq || !hs) goto done;
  if (gemm_any(e->gate, e->gate_scale, xq, xs, m, inter, hidden, NULL, g, gemm_threads, 1)) goto done;
  if (gemm_any(e->up, e->up_scale, xq, xs, m, inter, hidden, NULL, u, gemm_threads, 1)) goto done;
  oracle_swiglu(g, u, NULL, h, m, inter, 10.0f);
  if (oracle_quantize_mxfp8(h, hq, hs, m, inter)) goto done;
  if (gemm_any(e->down, e->down_scale, hq, hs, m, hidden, inter, NULL, out_bf16, gemm_threads, 1)) goto done;
  rc = 0;
done:
  free(g); free(u); free(h); free(hq); free(hs);
  return rc;
}

/* Threads used by oracle_mxfp4_gemm / oracle_expert_ffn (1 by default). */
void oracle_set_threads(int n) { gemm_threads = n; }
