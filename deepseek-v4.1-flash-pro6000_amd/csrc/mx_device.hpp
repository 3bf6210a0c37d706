// Device-side building blocks shared by the gfx950 MoE kernels: MX scalar
// formats, bf16 rounding, and the 16-channel MXFP4 x MXFP8 GEMV tile on the
// CDNA4 scaled MFMA (V_MFMA_SCALE_F32_16X16X128_F8F6F4).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "ds41_moe_gfx950.h"
#include "ds41_accept_gfx950.h"

namespace ds41g {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef const u32x4 __attribute__((address_space(1))) *global_u4;
typedef const u32x2 __attribute__((address_space(1))) *global_u2;
typedef u32x4 __attribute__((aligned(1))) u32x4_u;
typedef const u32x4_u __attribute__((address_space(1))) *global_u4u;

static_assert(sizeof(ds41_device_expert) == 64, "DeviceExpert must stay 64 bytes");
static_assert(sizeof(ds41_gemm_job) == 32, "GemmJob must stay 32 bytes");

constexpr int kMaxJobTokens = 8;   // rows per expert job (reference GemmJob: 1..8)
constexpr int kWave = 64;

// Kernel-visible status bits (ds41_status): a bounded wait that gave up, or a
// job descriptor whose row count is outside 1..kMaxJobTokens.
enum : uint32_t { kStatusReadyTimeout = 1u, kStatusBadJob = 2u, kStatusBadRoute = 4u };
extern __device__ uint32_t ds41_status;

__device__ __forceinline__ float bf16_to_f32(uint16_t v) { return __uint_as_float((uint32_t)v << 16); }

// Round-to-nearest-even to bf16; NaN stays a quiet NaN.
__device__ __forceinline__ uint16_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}
__device__ __forceinline__ float bf16_round(float f) { return bf16_to_f32(f32_to_bf16(f)); }

// E8M0 -> fp32: 2^(e-127), e == 0 -> 2^-127, e == 255 -> NaN.
__device__ __forceinline__ float e8m0_to_f32(uint32_t e) {
  return e == 0 ? __uint_as_float(0x00400000u) : e == 255 ? __uint_as_float(0x7fffffffu)
                                                            : __uint_as_float(e << 23);
}

// fp32 -> OCP E4M3 (fn), round-to-nearest-even, saturating at +-448, NaN -> 0x7f.
// Integer formulation: the result never depends on the hardware converter's
// rounding or NaN conventions.
__device__ __forceinline__ uint32_t e4m3_from_f32(float v) {
  uint32_t u = __float_as_uint(v);
  uint32_t sign = (u >> 24) & 0x80u;
  uint32_t a = u & 0x7fffffffu;
  if (a > 0x7f800000u) return 0x7fu;
  if (a >= 0x43e00000u) return sign | 0x7eu;                 // |v| >= 448
  if (a < 0x3c800000u) {                                     // |v| < 2^-6: grid of 2^-9
    float m = __builtin_rintf(__uint_as_float(a) * 512.0f);  // exact scaling, ties-to-even
    return sign | (uint32_t)m;
  }
  int e = (int)(a >> 23) - 127;
  uint32_t mant = a & 0x7fffffu, r = mant >> 20, rem = mant & 0xfffffu;
  r += (rem > 0x80000u || (rem == 0x80000u && (r & 1u))) ? 1u : 0u;
  if (r == 8u) { r = 0u; ++e; }
  if (e > 8 || (e == 8 && r > 6u)) return sign | 0x7eu;
  return sign | (uint32_t)(((e + 7) << 3) | (int)r);
}

// E4M3 code of v clamped to [-448, 448] (fminf / fmaxf return the number, so a NaN v gives the
// code of -448): the hardware converter, round to nearest even. On gfx950 it equals
// e4m3_from_f32 for every fp32 in [-448, 448] (all 2^31-odd of them are compared by
// ds41_e4m3_converter_check), so the quantisers keep the integer formulation's bits.
__device__ __forceinline__ float e4m3_clamp(float v) { return fminf(448.f, fmaxf(-448.f, v)); }
__device__ __forceinline__ uint32_t e4m3_sat(float v) {
  const float c = e4m3_clamp(v);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(c, c, 0, false) & 0xffu;
}
// Four codes in one dword, value i in byte i.
__device__ __forceinline__ uint32_t e4m3_sat4(float a, float b, float c, float d) {
  const int lo = __builtin_amdgcn_cvt_pk_fp8_f32(e4m3_clamp(a), e4m3_clamp(b), 0, false);
  return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(e4m3_clamp(c), e4m3_clamp(d), lo, true);
}

// MXFP8 scale exponent of a 32-group from its amax (mxfp4.cu:16-19):
// e = ceil-to-power-of-two exponent of fp32(max(amax, 1e-4) * (1/448)).
__device__ __forceinline__ uint32_t mxfp8_exponent(float amax) {
  amax = fmaxf(amax, 1e-4f);
  uint32_t b = __float_as_uint(amax * (1.0f / 448.0f));
  return (b >> 23) + ((b & 0x7fffffu) != 0u);
}

// E4M3 code of v in a 32-group whose MXFP8 scale exponent is e (mxfp4.cu:16-19 scaling).
__device__ __forceinline__ uint8_t mx8_code(float v, uint32_t e) {
  return (uint8_t)e4m3_sat(v / __uint_as_float(e << 23));
}

// Bounded acquire-wait on a residency flag (mxfp4.cu:36-43 semantics): relaxed
// device-coherent polls, then one acquire fence once the expected generation is
// seen. Gives up after kReadyWaitTicks of the 100 MHz constant wall clock
// (2 s), so no wave can spin forever.
constexpr uint64_t kReadyWaitTicks = 200000000ull;
__device__ __forceinline__ bool wait_ready(const ds41_device_expert &e) {
  if (!e.ready) return true;
  const uint64_t t0 = wall_clock64();
  for (;;) {
    const uint32_t v = __hip_atomic_load(e.ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (v == e.generation) {
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
      return true;
    }
    if (wall_clock64() - t0 > kReadyWaitTicks) break;
    __builtin_amdgcn_s_sleep(8);
  }
  atomicOr(&ds41_status, kStatusReadyTimeout);
  return false;
}

__device__ __forceinline__ const uint8_t *proj_weight(const ds41_device_expert &e, int p) {
  return p == 0 ? e.gate : p == 1 ? e.up : e.down;
}
__device__ __forceinline__ const uint8_t *proj_scale(const ds41_device_expert &e, int p) {
  return p == 0 ? e.gate_scale : p == 1 ? e.up_scale : e.down_scale;
}

// LDS image of the activation rows of one job: rows of `stride` bytes holding
// E4M3 values zero-padded to a multiple of 128, and rows of `sstride` E8M0
// scale bytes padded with 127 (both strides multiples of 16 bytes).
struct XTile {
  const uint8_t *q, *s;
  int stride, sstride, tokens;
  int split;  // 1: the GEMV feeds every row twice, as its |v| >= 1 and its |v| < 1 bytes
};

// One extra all-zero 128-k chunk (scales 127) follows the padded row, so a GEMV
// may run whole batches past the last chunk and add exact zeros.
__device__ __host__ __forceinline__ int xtile_stride(int k) { return ((k + 127) / 128 + 1) * 128 + 16; }
__device__ __host__ __forceinline__ int xtile_sstride(int k) { return (((k + 127) / 128 + 1) * 4 + 15) & ~15; }

// Byte mask (0xff per byte) of the E4M3 bytes with |v| >= 1 (exponent field >= 7):
// (b & 0x78) + 0x48 has bit 7 set exactly when the exponent field is >= 7 (no
// carry leaves the byte), and v_perm's selectors 8..11 replicate bit 7 of
// bytes 1, 3, 5, 7 of its 8-byte operand {t, t << 8}, i.e. of t's bytes 0, 2, 1, 3.
__device__ __forceinline__ uint32_t e4m3_big_mask(uint32_t v) {
  const uint32_t t = (v & 0x78787878u) + 0x48484848u;
  return __builtin_amdgcn_perm(t, t << 8, 0x0B090A08u);
}

// Magnitude split of the activation rows. The scaled MFMA forms each K32 block
// dot with a window of about 14 bits below the block's largest product
// (measured on gfx950: with a 2688 product in the block a lone 2^-4 product is
// dropped, 2^-3 kept), so MXFP8 rows, whose largest byte in every block has
// exponent field 14 or 15, lose their smallest products. Split, a row becomes
// two rows: its bytes with |v| >= 1 and its bytes with |v| < 1; each half fits
// the window, and the two results are added in fp32. With T <= 8 tokens the
// halves fill rows 0..T4-1 and T4..2*T4-1 (T4 = T rounded up to 4) of the
// 16-row MFMA, so the split costs no extra MFMA: split_combine() adds each
// token's two rows, which sit 4*T4 lanes apart. LDS holds each row once; a
// lane masks its row's bytes to its half as it reads them (split_lane), so the
// split costs no LDS either.
__device__ __host__ __forceinline__ int split_rows(int tokens) { return 2 * ((tokens + 3) & ~3); }
// MFMA row i (= lane & 15) of a split XTile: source row, and the mask flip
// (0: |v| >= 1 bytes, ~0: |v| < 1 bytes). Rows past 2*T4 read a finite row and
// their outputs are dropped (an MFMA output row depends on its own A row only).
struct SplitLane {
  int src;
  uint32_t flip;
};
__device__ __forceinline__ SplitLane split_lane(int i, int tokens, bool split) {
  const int T4 = (tokens + 3) & ~3;
  SplitLane r{i, 0u};
  if (split) {
    r.src = i < T4 ? i : i - T4;
    r.flip = i < T4 ? 0u : 0xffffffffu;
  }
  if (r.src >= tokens) r.src = 0;  // padding rows: any finite row, outputs dropped
  return r;
}
// The split half of 16 activation bytes: 6 vector operations per dword (the v_perm mask).
__device__ __forceinline__ uint4 split_bytes(uint4 v, const SplitLane &l) {
  v.x &= e4m3_big_mask(v.x) ^ l.flip;
  v.y &= e4m3_big_mask(v.y) ^ l.flip;
  v.z &= e4m3_big_mask(v.z) ^ l.flip;
  v.w &= e4m3_big_mask(v.w) ^ l.flip;
  return v;
}
__device__ __forceinline__ v4f split_combine(v4f acc, int tokens) {
  const int shift = 4 * ((tokens + 3) & ~3);
  v4f o;
#pragma unroll
  for (int r = 0; r < 4; ++r) o[r] = acc[r] + __shfl_down(acc[r], shift);
  return o;
}

// Stage `tokens` activation rows into LDS: LDS row r is source row row_idx(r) of
// the E4M3 matrix x [*][k] and its scales xs [*][k/32], each row zero-padded
// to its trailing zero chunk. Returns the number of rows. Caller syncs.
// Each thread issues the global loads of up to four 16-byte pieces (or four
// scale bytes) before it stores any of them, so a workgroup's staging costs
// about one memory round trip instead of one per loop trip.
template <class RowIdx>
__device__ __forceinline__ int stage_xtile(uint8_t *lq, uint8_t *ls, const uint8_t *x,
                                           const uint8_t *xs, int k, int tokens, RowIdx row_idx) {
  const int stride = xtile_stride(k), sstride = xtile_sstride(k);
  const int pieces = (stride - 16) >> 4;  // includes the trailing zero chunk
  const int kp = k >> 4;                  // pieces holding data (k % 32 == 0)
  const bool aligned = (((uintptr_t)x) & 15u) == 0;
  const int nsrc = tokens * kp;
  for (int p0 = threadIdx.x; p0 < nsrc; p0 += 4 * blockDim.x) {
    uint4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j * (int)blockDim.x;
      v[j] = make_uint4(0, 0, 0, 0);
      if (p < nsrc) {
        const int t = p / kp, off = (p - t * kp) << 4;
        const uint8_t *src = x + (size_t)row_idx(t) * k + off;
        if (aligned) {
          v[j] = *reinterpret_cast<const uint4 *>(src);
        } else {
          const u32x4 u = *(const u32x4_u *)(src);
          v[j] = make_uint4(u.x, u.y, u.z, u.w);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j * (int)blockDim.x;
      if (p >= nsrc) break;
      const int t = p / kp, off = (p - t * kp) << 4;
      *reinterpret_cast<uint4 *>(lq + t * stride + off) = v[j];
    }
  }
  for (int p = threadIdx.x; p < tokens * (pieces - kp); p += blockDim.x) {  // trailing zeros
    const int r = p / (pieces - kp), pc = kp + (p - r * (pieces - kp));
    *reinterpret_cast<uint4 *>(lq + r * stride + (pc << 4)) = make_uint4(0, 0, 0, 0);
  }
  const int ng = k >> 5;
  for (int p0 = threadIdx.x; p0 < tokens * sstride; p0 += 4 * blockDim.x) {
    uint8_t b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j * (int)blockDim.x, t = p / sstride, g = p - t * sstride;
      b[j] = p < tokens * sstride && g < ng ? xs[(size_t)row_idx(t) * ng + g] : (uint8_t)127;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j * (int)blockDim.x;
      if (p >= tokens * sstride) break;
      ls[p] = b[j];
    }
  }
  return tokens;
}

// stage_xtile of rows 0..tokens-1 of x in one memory round trip, for a big
// workgroup whose tile is a few pieces per thread: issue() loads each thread's
// up to NP 16-byte pieces and NS scale bytes (addresses clamped into the tile,
// so every load is unconditional), hold() waits for all of them once, and
// store() writes them and the trailing zero chunks to LDS. The caller may issue
// loads of its own between issue() and hold(). A tile of more than NP * blockDim
// pieces or NS * blockDim scale bytes, or an x not 16-byte aligned, is not
// loaded (ok false) and store() stages it with stage_xtile. Caller syncs.
// Quotient by a divisor 2 <= d < 2^16 fixed for the launch, as one multiply-high:
// m = ceil(2^32 / d) gives floor(p / d) exactly for 0 <= p < 2^32 / d (the
// rounding error of m is below 1 / d per unit of p).
struct UDiv {
  uint32_t d, m;
  __device__ __forceinline__ explicit UDiv(uint32_t dd) : d(dd), m(0xffffffffu / dd + 1u) {}
  __device__ __forceinline__ uint32_t q(uint32_t p) const { return __umulhi(p, m); }
};

template <int NP, int NS>
struct XTileRound {
  uint4 v[NP];
  uint32_t b[NS];
  bool ok;
  __device__ __forceinline__ void issue(const uint8_t *x, const uint8_t *xs, int k, int tokens) {
    const int kp = k >> 4, nsrc = tokens * kp, ng = k >> 5, sstride = xtile_sstride(k), bd = (int)blockDim.x;
    ok = (((uintptr_t)x) & 15u) == 0 && tokens > 0 && nsrc <= NP * bd && tokens * sstride <= NS * bd &&
         k < (1 << 20);
    // Loaded whatever ok says (a branch or a value select here makes the compiler wait on each
    // load); the clamped addresses stay inside rows 0..max(tokens, 1)-1.
    const UDiv dkp((uint32_t)kp), dss((uint32_t)sstride);
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int q = (int)threadIdx.x + j * bd, p = q < nsrc ? q : (nsrc > 0 ? nsrc - 1 : 0);
      const int t = (int)dkp.q((uint32_t)p), off = (p - t * kp) << 4;
      const u32x4 u = *(global_u4u)(x + (size_t)t * k + off);
      v[j] = make_uint4(u.x, u.y, u.z, u.w);
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int p = (int)threadIdx.x + j * bd, t = (int)dss.q((uint32_t)p), g = p - t * sstride;
      const int tc = t < tokens ? t : (tokens > 0 ? tokens - 1 : 0), gc = g < ng ? g : ng - 1;
      b[j] = xs[(size_t)tc * ng + gc];
    }
  }
  __device__ __forceinline__ void hold() {
#pragma unroll
    for (int j = 0; j < NP; ++j) asm volatile("" : "+v"(v[j].x), "+v"(v[j].y), "+v"(v[j].z), "+v"(v[j].w));
#pragma unroll
    for (int j = 0; j < NS; ++j) asm volatile("" : "+v"(b[j]));
  }
  __device__ __forceinline__ void store_presplit(uint8_t *lq, uint8_t *ls, const uint8_t *x, const uint8_t *xs, int k,
                                                 int tokens) const;
  // Presplit: the layout of stage_xtile_presplit (2 * T4 rows), else that of stage_xtile.
  template <bool Presplit = false>
  __device__ __forceinline__ void store(uint8_t *lq, uint8_t *ls, const uint8_t *x, const uint8_t *xs, int k,
                                        int tokens) const {
    if constexpr (Presplit) {
      store_presplit(lq, ls, x, xs, k, tokens);
      return;
    }
    if (!ok) {
      stage_xtile(lq, ls, x, xs, k, tokens, [](int r) { return (size_t)r; });
      return;
    }
    const int stride = xtile_stride(k), sstride = xtile_sstride(k), pieces = (stride - 16) >> 4;
    const int kp = k >> 4, nsrc = tokens * kp, ng = k >> 5, bd = (int)blockDim.x;
    const UDiv dkp((uint32_t)kp), dss((uint32_t)sstride);
#pragma unroll
    for (int j = 0; j < NP; ++j) {
      const int p = (int)threadIdx.x + j * bd;
      if (p >= nsrc) break;
      const int t = (int)dkp.q((uint32_t)p), off = (p - t * kp) << 4;
      *reinterpret_cast<uint4 *>(lq + t * stride + off) = v[j];
    }
    for (int p = threadIdx.x; p < tokens * (pieces - kp); p += bd) {  // trailing zeros
      const int r = p / (pieces - kp), pc = kp + (p - r * (pieces - kp));
      *reinterpret_cast<uint4 *>(lq + r * stride + (pc << 4)) = make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < NS; ++j) {
      const int p = (int)threadIdx.x + j * bd;
      if (p >= tokens * sstride) break;
      ls[p] = p - (int)dss.q((uint32_t)p) * sstride < ng ? (uint8_t)b[j] : (uint8_t)127;
    }
  }
};

template <int NP, int NS>
__device__ __forceinline__ void XTileRound<NP, NS>::store_presplit(uint8_t *lq, uint8_t *ls, const uint8_t *x,
                                                                  const uint8_t *xs, int k, int tokens) const {
  if (!ok) {
    stage_xtile_presplit(lq, ls, x, xs, k, tokens, [](int r) { return (size_t)r; });
    return;
  }
  const int stride = xtile_stride(k), sstride = xtile_sstride(k), pieces = (stride - 16) >> 4;
  const int T4 = (tokens + 3) & ~3, nrows = 2 * T4, kp = k >> 4, nsrc = tokens * kp, ng = k >> 5;
  const int bd = (int)blockDim.x;
  const UDiv dkp((uint32_t)kp), dss((uint32_t)sstride);
#pragma unroll
  for (int j = 0; j < NP; ++j) {
    const int p = (int)threadIdx.x + j * bd;
    if (p >= nsrc) break;
    const int t = (int)dkp.q((uint32_t)p), off = (p - t * kp) << 4;
    const SplitLane big{t, 0u}, small{t, 0xffffffffu};
    *reinterpret_cast<uint4 *>(lq + t * stride + off) = split_bytes(v[j], big);
    *reinterpret_cast<uint4 *>(lq + (T4 + t) * stride + off) = split_bytes(v[j], small);
  }
  for (int p = threadIdx.x; p < nrows * pieces; p += bd) {  // trailing chunk, padding rows
    const int r = p / pieces, pc = p - r * pieces, t = r < T4 ? r : r - T4;
    if (pc >= kp || t >= tokens) *reinterpret_cast<uint4 *>(lq + r * stride + (pc << 4)) = make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int j = 0; j < NS; ++j) {  // rows tokens..T4-1 of the scales (never loaded) are 127 too
    const int p = (int)threadIdx.x + j * bd;
    if (p >= T4 * sstride) break;
    const int t = (int)dss.q((uint32_t)p), g = p - t * sstride;
    const uint8_t e = g < ng && t < tokens ? (uint8_t)b[j] : (uint8_t)127;
    ls[p] = e;
    ls[T4 * sstride + p] = e;
  }
  for (int p = (int)threadIdx.x + NS * bd; p < T4 * sstride; p += bd) {  // past the loaded rows
    ls[p] = (uint8_t)127;
    ls[T4 * sstride + p] = (uint8_t)127;
  }
}

// Pre-split staging: split_rows(tokens) LDS rows, row t = the |v| >= 1 bytes of
// source row t and row T4 + t its |v| < 1 bytes (padding rows zero, scales
// 127), read by a GEMV with XTile.split = 0. It costs twice the LDS of
// stage_xtile and saves the per-chunk masks of the read-time split; the
// kernels take it where the doubled tile does not lower their occupancy.
template <class RowIdx>
__device__ __forceinline__ int stage_xtile_presplit(uint8_t *lq, uint8_t *ls, const uint8_t *x,
                                                    const uint8_t *xs, int k, int tokens, RowIdx row_idx) {
  const int stride = xtile_stride(k), sstride = xtile_sstride(k);
  const int T4 = (tokens + 3) & ~3, nrows = 2 * T4;
  const int pieces = (stride - 16) >> 4, kp = k >> 4;
  const bool aligned = (((uintptr_t)x) & 15u) == 0;
  const int nsrc = tokens * kp;
  for (int p0 = threadIdx.x; p0 < nsrc; p0 += 4 * blockDim.x) {
    uint4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j * (int)blockDim.x;
      v[j] = make_uint4(0, 0, 0, 0);
      if (p < nsrc) {
        const int t = p / kp, off = (p - t * kp) << 4;
        const uint8_t *src = x + (size_t)row_idx(t) * k + off;
        if (aligned) {
          v[j] = *reinterpret_cast<const uint4 *>(src);
        } else {
          const u32x4 u = *(const u32x4_u *)(src);
          v[j] = make_uint4(u.x, u.y, u.z, u.w);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j * (int)blockDim.x;
      if (p >= nsrc) break;
      const int t = p / kp, off = (p - t * kp) << 4;
      const SplitLane big{t, 0u}, small{t, 0xffffffffu};
      *reinterpret_cast<uint4 *>(lq + t * stride + off) = split_bytes(v[j], big);
      *reinterpret_cast<uint4 *>(lq + (T4 + t) * stride + off) = split_bytes(v[j], small);
    }
  }
  for (int p = threadIdx.x; p < nrows * pieces; p += blockDim.x) {  // trailing chunk, padding rows
    const int r = p / pieces, pc = p - r * pieces, t = r < T4 ? r : r - T4;
    if (pc >= kp || t >= tokens) *reinterpret_cast<uint4 *>(lq + r * stride + (pc << 4)) = make_uint4(0, 0, 0, 0);
  }
  const int ng = k >> 5;
  for (int p0 = threadIdx.x; p0 < T4 * sstride; p0 += 4 * blockDim.x) {
    uint8_t b[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j * (int)blockDim.x, t = p / sstride, g = p - t * sstride;
      b[j] = p < T4 * sstride && g < ng && t < tokens ? xs[(size_t)row_idx(t) * ng + g] : (uint8_t)127;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int p = p0 + j * (int)blockDim.x;
      if (p >= T4 * sstride) break;
      ls[p] = b[j];
      ls[T4 * sstride + p] = b[j];
    }
  }
  return nrows;
}
// MXFP8 codes of 16 consecutive values of a 32-group whose other 16 values sit in the
// neighbouring lane (lane ^ 1): the group's exponent from both halves' amax, then the codes of
// mx8_code. For 1 <= e <= 253 the power-of-two divisor's reciprocal is a normal float, so the
// product rounds exactly as the quotient does; other exponents (an infinite or NaN amax) take the
// quotient itself.
__device__ __forceinline__ uint4 mx8_codes16(const float *f, uint32_t *e_out) {
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(f[i]));
  amax = fmaxf(amax, __shfl_xor(amax, 1));
  const uint32_t e = mxfp8_exponent(amax);
  *e_out = e;
  uint32_t w[4];
  if (e - 1u <= 252u) {
    const float inv = __uint_as_float((254u - e) << 23);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = e4m3_sat4(f[4 * i] * inv, f[4 * i + 1] * inv, f[4 * i + 2] * inv, f[4 * i + 3] * inv);
  } else {
    const float d = __uint_as_float(e << 23);
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = e4m3_sat4(f[4 * i] / d, f[4 * i + 1] / d, f[4 * i + 2] / d, f[4 * i + 3] / d);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// stage_xtile (Presplit false) or stage_xtile_presplit (Presplit true) of `tokens` rows of the
// bf16 matrix x [*][k], quantised to MXFP8 on the way (the codes and exponents the MXFP8
// quantiser writes for the same rows). A thread takes one 16-value half of a 32-group per trip;
// the group's halves are neighbouring lanes, so every lane runs every trip (loads clamped into
// the tile, stores skipped past its end). Returns the LDS row count. Caller syncs.
template <bool Presplit, class RowIdx>
__device__ __forceinline__ int stage_xtile_bf16(uint8_t *lq, uint8_t *ls, const uint16_t *x, int k, int tokens,
                                                RowIdx row_idx) {
  const int stride = xtile_stride(k), sstride = xtile_sstride(k);
  const int T4 = (tokens + 3) & ~3, nrows = Presplit ? 2 * T4 : tokens, srows = Presplit ? T4 : tokens;
  const int pieces = (stride - 16) >> 4, kp = k >> 4, ng = k >> 5, bd = (int)blockDim.x;
  const int nsrc = tokens * kp;
  const bool aligned = (((uintptr_t)x) & 15u) == 0;
  for (int p0 = 0; p0 < nsrc; p0 += 2 * bd) {
    u32x4 v[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = p0 + (int)threadIdx.x + j * bd, p = q < nsrc ? q : nsrc - 1;
      const int t = p / kp, pc = p - t * kp;
      const uint16_t *src = x + (size_t)row_idx(t) * k + 16 * pc;
      if (aligned) {
        v[j][0] = *(global_u4)(src);
        v[j][1] = *(global_u4)(src + 8);
      } else {
        v[j][0] = *(global_u4u)(src);
        v[j][1] = *(global_u4u)(src + 8);
      }
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const int q = p0 + (int)threadIdx.x + j * bd, p = q < nsrc ? q : nsrc - 1;
      const int t = p / kp, pc = p - t * kp;
      const uint32_t wd[8] = {v[j][0].x, v[j][0].y, v[j][0].z, v[j][0].w, v[j][1].x, v[j][1].y, v[j][1].z, v[j][1].w};
      float f[16];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        f[2 * i] = __uint_as_float(wd[i] << 16);
        f[2 * i + 1] = __uint_as_float(wd[i] & 0xffff0000u);
      }
      uint32_t e;
      const uint4 c = mx8_codes16(f, &e);  // every lane: its neighbour needs its amax
      if (q < nsrc) {
        if (Presplit) {
          const SplitLane big{t, 0u}, small{t, 0xffffffffu};
          *reinterpret_cast<uint4 *>(lq + t * stride + 16 * pc) = split_bytes(c, big);
          *reinterpret_cast<uint4 *>(lq + (T4 + t) * stride + 16 * pc) = split_bytes(c, small);
        } else {
          *reinterpret_cast<uint4 *>(lq + t * stride + 16 * pc) = c;
        }
        if (!(pc & 1)) {
          ls[t * sstride + (pc >> 1)] = (uint8_t)e;
          if (Presplit) ls[(T4 + t) * sstride + (pc >> 1)] = (uint8_t)e;
        }
      }
    }
  }
  for (int p = threadIdx.x; p < nrows * pieces; p += bd) {  // trailing chunk, padding rows
    const int r = p / pieces, pc = p - r * pieces, t = r < srows ? r : r - T4;
    if (pc >= kp || t >= tokens) *reinterpret_cast<uint4 *>(lq + r * stride + (pc << 4)) = make_uint4(0, 0, 0, 0);
  }
  for (int p = threadIdx.x; p < nrows * sstride; p += bd) {  // scale padding, padding rows
    const int r = p / sstride, g = p - r * sstride, t = r < srows ? r : r - T4;
    if (g >= ng || t >= tokens) ls[p] = (uint8_t)127;
  }
  return nrows;
}

// The pre-split tile when it fits `budget` bytes of LDS.
__host__ __device__ __forceinline__ bool presplit_fits(int tokens, int k, int budget) {
  return (size_t)split_rows(tokens) * (xtile_stride(k) + xtile_sstride(k)) <= (size_t)budget;
}

// Operand layout of V_MFMA_SCALE_F32_16X16X128_F8F6F4 (measured on gfx950):
//   B (fp4 weights, 128 x 16): lane l holds 32 consecutive k = 32*(l>>4) .. +31 of
//     column l&15, low nibble first -> one 16-byte load of the weight row;
//   A (fp8 activations, 16 x 128): lane l holds row l&15, bytes 0..15 = k 16q..16q+15
//     and bytes 16..31 = k 64+16q..64+16q+15 with q = l>>4;
//   scales: lane l carries the E8M0 of row/column l&15 for k-block l>>4 (byte 0);
//   D (16 x 16 fp32): lane l holds column l&15, rows 4*(l>>4) + r in register r.
// A = activations (tokens as rows), B = weights (channels as columns), so lane l
// ends with channel l&15 for tokens 4*(l>>4) .. +3.
//
// Gemv16 streams the 16 weight rows of one wave (row l&15 at `wrow`, K bytes/2)
// through the MFMA, 128 k per chunk. The constructor issues the first U chunk
// loads so they are in flight while the caller stages LDS; run() then keeps two
// register batches in flight (ping-pong, no register copies) so each wait covers
// only the older batch. All weight loads are unconditional: lanes past the last
// K32 group re-read a valid group and get scale 127 against zero activations,
// and a partial last batch re-reads the last chunk without computing it.
// One 128-k chunk of the scaled MFMA (A = 16 activation rows, lo/hi = this
// lane's two 16-byte pieces of k 16q..16q+15 and 64+16q..64+16q+15, q = l>>4;
// B = weights) accumulated into acc. Measured on gfx950: the result equals four
// single-K32-group MFMAs into fresh accumulators added to acc in k order in
// fp32 (the reference's one block-scaled MMA per k32 plus serial fp32 add,
// components/moe/src/mxfp4.cu:113-132), bit for bit, so one instruction does it.
__device__ __forceinline__ v4f mfma_chunk(const uint4 &lo, const uint4 &hi, const v8i &bv, v4f acc, int sa, int sw) {
  const v8i a = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
  return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, bv, acc, 0, 4, 0, sa, 0, sw);
}
// The same chunk as two operands: its bytes with |v| >= 1 and its bytes with |v| < 1.
__device__ __forceinline__ void split_chunk(const uint4 &lo, const uint4 &hi, v8i &big, v8i &small) {
  const uint32_t w[8] = {lo.x, lo.y, lo.z, lo.w, hi.x, hi.y, hi.z, hi.w};
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const uint32_t m = e4m3_big_mask(w[i]);
    big[i] = (int)(w[i] & m);
    small[i] = (int)(w[i] & ~m);
  }
}


// Tiled weights (ds41_expert_slab_tile): the 16-byte K32 pieces of an MXFP4
// matrix [N][K/2] stored in the MFMA B-operand order, piece (row n, group g) at
// (n / 16) * (K / 32) * 256 + g * 256 + (n % 16) * 16. A wave's chunk load (16
// rows x 4 groups) is then one contiguous kilobyte, read once, with
// non-temporal loads. N % 16 == 0. The row-major reference layout has the
// piece at n * K / 2 + g * 16.
template <bool Tiled>
__device__ __forceinline__ const uint8_t *weight_row(const uint8_t *w, int row, int K) {
  return Tiled ? w + (size_t)(row >> 4) * ((size_t)K << 3) + (size_t)(row & 15) * 16 : w + (size_t)row * (size_t)(K >> 1);
}

// GScale: the weight scales come from global memory instead of an LDS row.
// With each batch's weights a lane loads its channel's 32 scale bytes of that
// batch (8 chunks x 4 groups; dword u holds chunk u's four groups) and takes
// byte kb of each dword. Requires U == 8 and k % 1024 == 0 (whole batches).
// Frees the workgroup's LDS of the weight scales.
// Tiled: `wrow` from weight_row<true>; pieces are 256 bytes apart.
template <int U, bool Aligned16, bool GScale = false, bool Tiled = false>
struct Gemv16 {
  const uint8_t *w;  // weight row
  const uint8_t *gs; // GScale: this lane's channel's scale row
  int kb, ng, nch, nb;
  uint4 A[U], B[U];
  uint4 SA[2], SB[2];

  // 16 bytes of K32 group min(4c + kb, ng - 1) through a global-address-space
  // pointer (global_load, counted by vmcnt only, never by lgkmcnt). Plain (not
  // non-temporal) loads: each 128-byte row line is consumed by two consecutive
  // chunk loads, and the second one must still find the line in L2.
  __device__ __forceinline__ uint4 ld(int c) const {
    const int cc = c < nch ? c : nch - 1;
    int g = 4 * cc + kb;
    g = g < ng ? g : ng - 1;
    if (Tiled) {  // each kilobyte block is read by this one instruction: no reuse to keep in the caches
      const u32x4 v = __builtin_nontemporal_load((global_u4)(w + 256 * g));
      return make_uint4(v.x, v.y, v.z, v.w);
    }
    const uint8_t *p = w + 16 * g;
    if (Aligned16) {
      const u32x4 v = *(global_u4)(p);
      return make_uint4(v.x, v.y, v.z, v.w);
    }
    const u32x2 lo = *(global_u2)(p), hi = *(global_u2)(p + 8);
    return make_uint4(lo.x, lo.y, hi.x, hi.y);
  }
  __device__ __forceinline__ void load(uint4 *buf, int b) const {
#pragma unroll
    for (int u = 0; u < U; ++u) buf[u] = ld(b * U + u);
  }
  __device__ __forceinline__ void ld_scales(uint4 *S, int b) const {
    // any alignment: gfx950 global loads take unaligned addresses (one dwordx4 either way)
    const uint8_t *p = gs + 32 * b;
    const u32x4 v0 = *(global_u4u)(p), v1 = *(global_u4u)(p + 16);
    S[0] = make_uint4(v0.x, v0.y, v0.z, v0.w);
    S[1] = make_uint4(v1.x, v1.y, v1.z, v1.w);
  }
  __device__ __forceinline__ Gemv16(const uint8_t *wrow, int k, const uint8_t *gscale_row = nullptr) {
    begin(wrow, k, gscale_row);
  }
  // Unbound: begin() names the row and issues its first batch (for a caller that
  // starts the stream before it knows the row is needed, or across a branch).
  __device__ __forceinline__ Gemv16() {}
  __device__ __forceinline__ void begin(const uint8_t *wrow, int k, const uint8_t *gscale_row = nullptr) {
    kb = (threadIdx.x & 63) >> 4;
    w = wrow;
    gs = gscale_row;
    ng = k >> 5;
    nch = (ng + 3) >> 2;
    nb = (nch + U - 1) / U;
    load(A, 0);
    if (GScale) ld_scales(SA, 0);
  }
  // xt: activation rows in LDS; lsw: this lane's weight-scale row in LDS (ng bytes).
  // Chunks past the end read the zero chunk of the activation rows (exact zero
  // products against a finite weight scale), so no MFMA sits behind a branch.
  // acc: the sum so far (a chain's carry), continued chunk by chunk in k order.
  template <bool Split = false>
  __device__ __forceinline__ v4f run(const XTile &xt, const uint8_t *lsw, v4f acc = v4f{0.f, 0.f, 0.f, 0.f}) {
    const int lane = threadIdx.x & 63, q = lane >> 4, i = lane & 15;
    const SplitLane sl = split_lane(i, xt.tokens, Split);  // padded rows repeat row 0; outputs dropped
    const uint8_t *xa = xt.q + sl.src * xt.stride + 16 * q;
    const uint8_t *sa = xt.s + sl.src * xt.sstride + q;
    auto mma = [&](const uint4 &wv, int c, int sw) {
      const int cx = c < nch ? c : nch;  // nch is the zero chunk
      uint4 lo = *reinterpret_cast<const uint4 *>(xa + 128 * cx);
      uint4 hi = *reinterpret_cast<const uint4 *>(xa + 128 * cx + 64);
      if (Split) {
        lo = split_bytes(lo, sl);
        hi = split_bytes(hi, sl);
      }
      const v8i bv = v8i{(int)wv.x, (int)wv.y, (int)wv.z, (int)wv.w, 0, 0, 0, 0};
      acc = mfma_chunk(lo, hi, bv, acc, (int)sa[4 * cx], sw);
    };
    auto compute = [&](const uint4 *buf, const uint4 *S, int b) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = b * U + u;
        int sw;
        if (GScale) {  // byte kb of dword u of the batch's scale window
          const uint4 &w4 = S[u >> 2];
          const uint32_t d = (u & 3) == 0 ? w4.x : (u & 3) == 1 ? w4.y : (u & 3) == 2 ? w4.z : w4.w;
          sw = (int)((d >> (8 * kb)) & 0xffu);
        } else {
          int g = 4 * c + kb;
          g = g < ng ? g : ng - 1;
          sw = (int)lsw[g];
        }
        mma(buf[u], c, sw);
      }
    };
    int b = 0;
    for (; b + 2 < nb; b += 2) {
      load(B, b + 1);
      if (GScale) ld_scales(SB, b + 1);
      compute(A, SA, b);
      load(A, b + 2);
      if (GScale) ld_scales(SA, b + 2);
      compute(B, SB, b + 1);
    }
    if (b + 2 == nb) {
      load(B, b + 1);
      if (GScale) ld_scales(SB, b + 1);
      compute(A, SA, b);
      compute(B, SB, b + 1);
    } else {
      compute(A, SA, b);
    }
    return acc;
  }
};

// FP8 (E4M3) weights with one E8M0 scale per 32 x 32 block (row block n/32,
// K32 group g at scale[(n/32) * (k/32) + g]; components/dense/src/dense.cu:37-91),
// against MXFP8 activation rows from an XTile. B operand of the scaled MFMA in
// FP8 form (format code 0) has A's layout: lane l holds column l&15, bytes
// 0..15 = k 16q..16q+15 and 16..31 = k 64+16q..64+16q+15 of the 128-k chunk,
// q = l>>4, and the E8M0 of K32 block q. All 16 channels of a wave sit in one
// 32-row scale block, so a lane's scales are bytes q, 4+q, 8+q, ... of that
// block's scale row: one 16-byte load per batch of 4 chunks gives byte q of
// its dwords. Pieces at k >= K (the partial last chunk) are zero; their
// activations are zero too.
//
// A wave streams the chunk range [c0, c1) of its 16 weight rows in batches of
// U = 4 chunks, two batches in flight (ping-pong), both issued by the
// constructor. A serial-carry chain of
// waves (f8_chain) splits K into contiguous ranges: every wave's loads are in
// flight from the start, and the accumulator passes from wave to wave in K
// order, so the sum is the same serial K-order sum one wave would form (the
// reference's serial carry, dense.cu:38-91), with up to all of the tile's
// weight bytes in flight at once.
struct Gemv16F8 {
  static constexpr int U = 4;
  const uint8_t *w;   // weight row of this lane's channel
  const uint8_t *sr;  // scale row of the channel's 32-row block
  int q, k, ng, c0, c1, nb;
  uint4 A[U][2], B[U][2];
  uint4 SA, SB;
  // activation operands and scales of batches 0 / 1 (prefetch_x), with the tile row of this lane
  uint4 XA[U][2], XB[U][2];
  int XSA[U], XSB[U];
  const uint8_t *xa_, *sa_;
  SplitLane sl_;

  // 16 weight bytes at `off`; a piece past the row (the partial last chunk) reads the row's last
  // 16 bytes instead. Its activations are zero, so it adds nothing: 0 x a finite code is 0, and a
  // NaN code there already makes the row's true sum NaN. The load is unconditional, so the wait
  // counts of the loads issued before it (the activation tile's) stay exact.
  __device__ __forceinline__ uint4 piece(int off) const {
    const u32x4 v = *(global_u4u)(w + (off < k ? off : k - 16));
    return make_uint4(v.x, v.y, v.z, v.w);
  }
  // first K32 group of the 16-group scale window loaded for batch b
  __device__ __forceinline__ int window(int b) const {
    const int g0 = 4 * (c0 + b * U);
    return g0 + 16 <= ng ? g0 : (ng >= 16 ? ng - 16 : 0);
  }
  __device__ __forceinline__ void load(uint4 (*buf)[2], uint4 &S, int b) const {
    load_w(buf, b);
    load_scales(S, b);
  }
  __device__ __forceinline__ void load_w(uint4 (*buf)[2], int b) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int c = c0 + b * U + u;
      c = c < c1 ? c : (c1 > c0 ? c1 - 1 : 0);
      buf[u][0] = piece(128 * c + 16 * q);
      buf[u][1] = piece(128 * c + 64 + 16 * q);
    }
  }
  __device__ __forceinline__ void load_scales(uint4 &S, int b) const {
    if (ng >= 16) {
      const u32x4 v = *(global_u4u)(sr + window(b));
      S = make_uint4(v.x, v.y, v.z, v.w);
    } else {  // short rows (k < 512): bytes clamped to the row, packed four to a dword
      uint32_t d[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int i = 0; i < 16; ++i) d[i >> 2] |= (uint32_t)sr[i < ng ? i : ng - 1] << (8 * (i & 3));
      S = make_uint4(d[0], d[1], d[2], d[3]);
    }
  }
  __device__ __forceinline__ Gemv16F8(const uint8_t *wrow, const uint8_t *srow, int kk, int cbegin, int cend) {
    q = (threadIdx.x & 63) >> 4;
    w = wrow;
    sr = srow;
    k = kk;
    ng = kk >> 5;
    // the chunk range is the same for the whole wave: scalar registers, scalar branches
    c0 = __builtin_amdgcn_readfirstlane(cbegin);
    c1 = __builtin_amdgcn_readfirstlane(cend);
    nb = (c1 - c0 + U - 1) / U;
    // both batches in flight before the wave's turn in a chain: the scales first (their short-row
    // form is a branch), then the weights unconditionally (a one-batch range reloads its last
    // chunk), so that the wait counts of loads issued before these stay exact
    load_scales(SA, 0);
    load_scales(SB, 1);
    load_w(A, 0);
    load_w(B, 1);
  }
  __device__ __forceinline__ int scale_of(const uint4 &S, int b, int c) const {
    const int g = 4 * c + q, gc = g < ng ? g : ng - 1, idx = gc - window(b);
    // byte idx (0..15) of S with selects of values (not of member addresses, which would put the
    // object in scratch) and a bit-field extract: no branches
    const uint32_t sx = S.x, sy = S.y, sz = S.z, sw = S.w;
    const uint32_t lo = (idx & 4) ? sy : sx, hi = (idx & 4) ? sw : sz, d = (idx & 8) ? hi : lo;
    return (int)__builtin_amdgcn_ubfe(d, 8u * (uint32_t)(idx & 3), 8u);
  }
  // A operands and activation scales of batch b from the tile (chunks clamped as load() does).
  template <bool Split>
  __device__ __forceinline__ void xload(uint4 (*X)[2], int *XS, int b) const {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      int c = c0 + b * U + u;
      c = c < c1 ? c : (c1 > c0 ? c1 - 1 : 0);
      uint4 lo = *reinterpret_cast<const uint4 *>(xa_ + 128 * c);
      uint4 hi = *reinterpret_cast<const uint4 *>(xa_ + 128 * c + 64);
      if (Split) {
        lo = split_bytes(lo, sl_);
        hi = split_bytes(hi, sl_);
      }
      X[u][0] = lo;
      X[u][1] = hi;
      XS[u] = sa_[4 * c];
    }
  }
  // Reads the activation operands of the first two batches from the staged tile into registers
  // (after the tile's barrier), for dots().
  template <bool Split>
  __device__ __forceinline__ void prefetch_x(const XTile &xt) {
    sl_ = split_lane(threadIdx.x & 15, xt.tokens, Split);
    xa_ = xt.q + sl_.src * xt.stride + 16 * q;
    sa_ = xt.s + sl_.src * xt.sstride + q;
    xload<Split>(XA, XSA, 0);
    if (nb > 1) xload<Split>(XB, XSB, 1);
  }
  // With at most two batches (nb <= 2) and the operands prefetched: each chunk's scaled dot on its
  // own (no accumulator chained through the MFMAs, so they issue back to back as soon as the
  // weights land), for add_dots to add in ascending K during the wave's turn.
  __device__ __forceinline__ void dots(v4f (&d)[2 * U]) const {
    const v4f z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const v8i av = v8i{(int)XA[u][0].x, (int)XA[u][0].y, (int)XA[u][0].z, (int)XA[u][0].w,
                         (int)XA[u][1].x, (int)XA[u][1].y, (int)XA[u][1].z, (int)XA[u][1].w};
      const v8i bv = v8i{(int)A[u][0].x, (int)A[u][0].y, (int)A[u][0].z, (int)A[u][0].w,
                         (int)A[u][1].x, (int)A[u][1].y, (int)A[u][1].z, (int)A[u][1].w};
      d[u] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, z, 0, 0, 0, XSA[u], 0, scale_of(SA, 0, c0 + u));
    }
    if (nb < 2) return;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const v8i av = v8i{(int)XB[u][0].x, (int)XB[u][0].y, (int)XB[u][0].z, (int)XB[u][0].w,
                         (int)XB[u][1].x, (int)XB[u][1].y, (int)XB[u][1].z, (int)XB[u][1].w};
      const v8i bv = v8i{(int)B[u][0].x, (int)B[u][0].y, (int)B[u][0].z, (int)B[u][0].w,
                         (int)B[u][1].x, (int)B[u][1].y, (int)B[u][1].z, (int)B[u][1].w};
      d[U + u] =
          __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, z, 0, 0, 0, XSB[u], 0, scale_of(SB, 1, c0 + U + u));
    }
  }
  // Chunks past the wave's range (the clamped reloads of its last chunk) as +0, which leaves a
  // sum unchanged, so the chain adds all 2U slots of every wave without a branch.
  __device__ __forceinline__ void clear_past_range(v4f (&d)[2 * U]) const {
    const v4f z = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 2 * U; ++i)
      if (c0 + i >= c1) d[i] = z;  // uniform
  }
  // acc plus the wave's chunk dots, one chunk after another in ascending K (after
  // clear_past_range the slots past the range add +0).
  __device__ __forceinline__ v4f add_dots(const v4f (&d)[2 * U], v4f acc) const {
#pragma unroll
    for (int i = 0; i < 2 * U; ++i) {
#pragma unroll
      for (int r = 0; r < 4; ++r) acc[r] = __fadd_rn(acc[r], d[i][r]);
    }
    return acc;
  }
  // Continues acc over the wave's chunk range.
  template <bool Split = false>
  __device__ __forceinline__ v4f run(const XTile &xt, v4f acc) {
    const int lane = threadIdx.x & 63, i = lane & 15;
    const SplitLane sl = split_lane(i, xt.tokens, Split);
    const uint8_t *xa = xt.q + sl.src * xt.stride + 16 * q;
    const uint8_t *sa = xt.s + sl.src * xt.sstride + q;
    auto compute = [&](const uint4 (*buf)[2], const uint4 &S, int b) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int c = c0 + b * U + u;
        if (c >= c1) break;  // uniform: the rest belongs to the next wave of the chain
        uint4 lo = *reinterpret_cast<const uint4 *>(xa + 128 * c);
        uint4 hi = *reinterpret_cast<const uint4 *>(xa + 128 * c + 64);
        if (Split) {
          lo = split_bytes(lo, sl);
          hi = split_bytes(hi, sl);
        }
        const v8i av = v8i{(int)lo.x, (int)lo.y, (int)lo.z, (int)lo.w, (int)hi.x, (int)hi.y, (int)hi.z, (int)hi.w};
        const v8i bv = v8i{(int)buf[u][0].x, (int)buf[u][0].y, (int)buf[u][0].z, (int)buf[u][0].w,
                           (int)buf[u][1].x, (int)buf[u][1].y, (int)buf[u][1].z, (int)buf[u][1].w};
        acc = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(av, bv, acc, 0, 0, 0, (int)sa[4 * c], 0,
                                                                scale_of(S, b, c));
      }
    };
    if (nb <= 0) return acc;
    // at entry A holds batch 0 and B batch 1; each buffer is refilled right after its compute
    int b = 0;
    for (; b + 2 < nb; b += 2) {
      compute(A, SA, b);
      load(A, SA, b + 2);
      compute(B, SB, b + 1);
      if (b + 3 < nb) load(B, SB, b + 3);
    }
    if (b + 2 == nb) {
      compute(A, SA, b);
      compute(B, SB, b + 1);
    } else {
      compute(A, SA, b);
    }
    return acc;
  }
};

// Chunk range of wave j of a Wc-wave chain over a k-long row.
__device__ __forceinline__ void f8_chain_range(int k, int Wc, int j, int &c0, int &c1) {
  const int nch = ((k >> 5) + 3) >> 2, per = (nch + Wc - 1) / Wc;
  c0 = j * per < nch ? j * per : nch;
  c1 = c0 + per < nch ? c0 + per : nch;
}
// Runs a Wc-wave serial-carry chain: in turn t, wave j == t continues the
// accumulator the previous wave left in `carry` (LDS, 64 lanes x 4 floats of
// this chain). Every wave of the workgroup calls it (the turns synchronise the
// workgroup); the returned value is valid in the chain's last wave. Wave j
// passes j barriers, runs its turn, then passes the other Wc - j: barrier t
// (1-based) separates turn t-1 from turn t, and the GEMV's code exists once.
// Dots: every wave has at most two batches (f8_dots_fit) and the caller prefetched its operands
// (prefetch_x). Each wave forms its chunk dots as soon as its weights land (Gemv16F8::dots);
// waves 0..Wc-2 leave theirs in `carry` ([Wc-1][8 chunks][64 lanes] x 4 floats), and after one
// barrier the last wave adds every chunk dot in ascending K: every 128-k chunk's dot is kept
// apart and the chunks are added serially (the reference keeps every K32 dot apart and adds them
// serially, components/dense/src/dense.cu:36-82; a chunk here is four K32 dots summed by the
// MFMA). Otherwise (carry: 64 lanes x 4 floats) the turns run the MFMAs on the carried sum.
template <int Wc, bool Split, bool Dots = false>
__device__ __forceinline__ v4f f8_chain(Gemv16F8 &g, const XTile &xt, float *carry, int j) {
  constexpr int D = 2 * Gemv16F8::U;
  const int lane = threadIdx.x & 63, jj = __builtin_amdgcn_readfirstlane(j);
  v4f acc = {0.f, 0.f, 0.f, 0.f};
  if constexpr (Dots) {
    v4f d[D];
    g.dots(d);
    g.clear_past_range(d);
    if (jj + 1 < Wc) {
#pragma unroll
      for (int i = 0; i < D; ++i) *reinterpret_cast<v4f *>(carry + 4 * ((jj * D + i) * 64 + lane)) = d[i];
    }
    __syncthreads();
    if (jj + 1 == Wc) {
      v4f p[(Wc - 1) * D];  // every slot read at once, then added in order (+0 past a range)
#pragma unroll
      for (int i = 0; i < (Wc - 1) * D; ++i) p[i] = *reinterpret_cast<const v4f *>(carry + 4 * (i * 64 + lane));
#pragma unroll
      for (int i = 0; i < (Wc - 1) * D; ++i) {
#pragma unroll
        for (int r = 0; r < 4; ++r) acc[r] = __fadd_rn(acc[r], p[i][r]);
      }
      acc = g.add_dots(d, acc);
    }
    return acc;
  } else {
    for (int t = 0; t < jj; ++t) __syncthreads();
    if (jj) acc = *reinterpret_cast<const v4f *>(carry + 4 * lane);
    acc = g.template run<Split>(xt, acc);
    if (jj + 1 < Wc) *reinterpret_cast<v4f *>(carry + 4 * lane) = acc;
    for (int t = jj; t < Wc; ++t) __syncthreads();
    return acc;
  }
}
// LDS bytes of f8_chain's carry for one chain.
__host__ __device__ __forceinline__ constexpr size_t f8_carry_bytes(int Wc, bool dots) {
  return dots ? (size_t)(Wc - 1) * 8 * 64 * 16 : (size_t)64 * 16;
}
// Whether every wave of a Wc-wave chain over a k-long row has at most two batches of chunks.
__host__ __device__ __forceinline__ bool f8_dots_fit(int k, int Wc) {
  const int nch = ((k >> 5) + 3) >> 2;
  return (nch + Wc - 1) / Wc <= 2 * Gemv16F8::U;
}

// Workgroup barrier that orders LDS accesses only. __syncthreads() also
// fences global memory, which makes every wave wait (s_waitcnt vmcnt(0)) for
// all of its outstanding global loads, including prefetches meant to stay in
// flight across the barrier; this fence waits for LDS operations only.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Copy `bytes` contiguous bytes global -> LDS with the whole workgroup
// (16-byte pieces when both ends allow it). Caller syncs.
__device__ __forceinline__ void stage_bytes(uint8_t *dst, const uint8_t *src, int bytes) {
  if (((((uintptr_t)src) | (uintptr_t)bytes) & 15u) == 0) {
    for (int p = threadIdx.x; p < (bytes >> 4); p += blockDim.x)
      reinterpret_cast<uint4 *>(dst)[p] = reinterpret_cast<const uint4 *>(src)[p];
  } else {
    for (int p = threadIdx.x; p < bytes; p += blockDim.x) dst[p] = src[p];
  }
}

}  // namespace ds41g
