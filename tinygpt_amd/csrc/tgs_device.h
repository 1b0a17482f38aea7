// tgs_device.h -- device-side numerics and block primitives of the gfx950
// sampler.  Everything here follows the canonical rules of the sampling
// contract bit for bit:
//   * tg_expf: Cody-Waite reduction x = n ln2 + r and the degree-7 Taylor
//     polynomial of e^r (Horner, fused multiply-adds), scaled by 2^n through
//     the exponent field; 0 below -32.
//   * masses are exact integers q = floor(e * 2^40), so any summation order
//     (atomics, trees, split rows) gives the same result;
//   * order keys map floats to uint32 monotonically (-0 folded onto +0);
//     composite keys (key(y) << 32 | ~id) order by (y desc, id asc).
// Wavefronts are 64 lanes.  Most kernels run NT = 256 threads (4 waves); the
// block primitives take the block size as a template parameter (BS, at most
// 1024 threads).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Dynamic LDS of a kernel (a CPU simulation of the kernels for debugging
// defines its own form).
#ifndef TGS_DYN_SMEM
#define TGS_DYN_SMEM(name) extern __shared__ __align__(16) unsigned char name[]
#endif
// A kernel's static LDS gathered in one object (the CPU simulation gives
// each workgroup its own copy, so that workgroups can run concurrently).
#ifndef TGS_STATIC_SMEM
#define TGS_STATIC_SMEM(type, name) __shared__ type name
#endif

namespace tgs {

constexpr int NT = 256;        // threads per workgroup
constexpr int NW = NT / 64;    // waves per workgroup
constexpr int KMAX = 1024;     // largest top-k served by the candidate path
constexpr int CAPB = 2048;     // candidate buffer entries (before history)
constexpr int SPEC_BLOCK = 1024;

typedef unsigned long long u64;

// ------------------------------------------------------------------ numerics

__device__ __forceinline__ float tg_u2f(uint32_t u) { return __uint_as_float(u); }
__device__ __forceinline__ uint32_t tg_f2u(float f) { return __float_as_uint(f); }

__device__ __forceinline__ float tg_expf(float x) {
  if (!(x >= -32.0f)) return 0.0f;
  if (x > 88.0f) return __builtin_inff();
  const float log2e = 0x1.715476p+0f;
  const float ln2_hi = 0x1.62ep-1f;
  const float ln2_lo = 0x1.0bfbe8p-15f;
  const float shifter = 12582912.0f;
  float t = x * log2e;
  float n = (t + shifter) - shifter;
  float r = __builtin_fmaf(n, -ln2_hi, x);
  r = __builtin_fmaf(n, -ln2_lo, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  int ni = (int)n;
  return p * tg_u2f((uint32_t)(ni + 127) << 23);
}

// tg_expf(x) for x <= 0, -inf or NaN (the range of y - m with m the maximum
// of the y's): the same value bit for bit.  The overflow test cannot fire,
// and 2^n (n >= -47 once x >= -32) scales p exactly through ldexp.
// Branch free: the polynomial runs on max(x, -32) (x itself wherever the
// result is used) and x < -32, -inf and NaN select 0 at the end.
__device__ __forceinline__ float tg_expf_nonpos(float x_in) {
  const float x = fmaxf(x_in, -32.0f);
  const float log2e = 0x1.715476p+0f;
  const float ln2_hi = 0x1.62ep-1f;
  const float ln2_lo = 0x1.0bfbe8p-15f;
  const float shifter = 12582912.0f;
  float t = x * log2e;
  float n = (t + shifter) - shifter;
  float r = __builtin_fmaf(n, -ln2_hi, x);
  r = __builtin_fmaf(n, -ln2_lo, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const float e = __builtin_ldexpf(p, (int)n);
  return (x_in >= -32.0f) ? e : 0.0f;
}

// tg_expf_nonpos(x) for -32 < x <= 0 (a caller that has tested the range):
// the same operations without the clamp to -32 and the final select, which
// are the identity there.
__device__ __forceinline__ float tg_expf_nonpos_in(float x) {
  const float log2e = 0x1.715476p+0f;
  const float ln2_hi = 0x1.62ep-1f;
  const float ln2_lo = 0x1.0bfbe8p-15f;
  const float shifter = 12582912.0f;
  float t = x * log2e;
  float n = (t + shifter) - shifter;
  float r = __builtin_fmaf(n, -ln2_hi, x);
  r = __builtin_fmaf(n, -ln2_lo, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

// floor(e * 2^40) of a weight e in [0, 1] as an integer-valued double: the
// per-lane sums of a few dozen such terms stay exact (below 2^53) and
// convert to the same u64 as summing tg_q40 terms.
__device__ __forceinline__ double tg_q40d(float e) { return (double)__builtin_floorf(e * 0x1p40f); }

// tg_q40d(tg_expf_nonpos(x)) bit for bit, in four operations fewer, for the
// passes that sum a mass for every element:
//   * the scaling by 2^40 joins the scaling by 2^n: e = p 2^n is exact for
//     n >= -47, so e 2^40 = p 2^(n + 40), and n + 40 is read from the bits
//     of s = t + 1.5 2^23, an integer in [2^23, 2^24) whose last mantissa
//     bits are n (one integer subtraction instead of a conversion);
//   * no final select: below -32 (and for -inf and NaN, which fmaxf maps to
//     -32) the polynomial runs on -32, where e 2^40 = 0.014, and floor gives
//     the same 0 as the select did (every x < -27.73 floors to 0).
// Checked against the two-step form in tests/cpu_sim/numerics.cpp, mode q40exp.
__device__ __forceinline__ double tg_q40d_exp_nonpos(float x_in) {
  const float x = fmaxf(x_in, -32.0f);
  const float log2e = 0x1.715476p+0f;
  const float ln2_hi = 0x1.62ep-1f;
  const float ln2_lo = 0x1.0bfbe8p-15f;
  const float shifter = 12582912.0f;  // 1.5 2^23, bits 0x4B400000
  const float t = x * log2e;
  const float s = t + shifter;
  const float n = s - shifter;
  float r = __builtin_fmaf(n, -ln2_hi, x);
  r = __builtin_fmaf(n, -ln2_lo, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  const int n40 = (int)(tg_f2u(s) - (0x4B400000u - 40u));
  return (double)__builtin_floorf(__builtin_ldexpf(p, n40));
}

// a / b correctly rounded from rb = RN(1 / b): q = RN(a * rb) is within one
// ulp of a / b, the residual a - b q is exact through a fused multiply-add,
// and one correction q + (a - b q) rb rounds to RN(a / b) (Markstein's
// theorem; a, b and a / b normal or a == 0).  Used for weights a in [0, 1]
// over softmax denominators b >= 1.
__device__ __forceinline__ float tg_div_rcp(float a, float b, float rb) {
  const float q = a * rb;
  const float r = __builtin_fmaf(-q, b, a);
  return __builtin_fmaf(r, rb, q);
}

// z / T correctly rounded (the temperature divide of Serve.swift:1499 and
// wasm/src/model.cpp:499), from the row's rT = RN(1 / T), by a mode fixed
// once per row (tg_div_t_mode):
//   TDIV_POW2  T a power of two: z rT is the same real number as z / T,
//              so one multiply rounds it the same way;
//   TDIV_FAST  T in [2^-20, 2^20]: q0 = RN(z rT) lies within 1.5 ulp of
//              z / T; one residual correction q1 = q0 + (z - T q0) rT makes
//              it faithful, and a second, with the residual z - T q1 exact
//              by a fused multiply-add, rounds to RN(z / T) (Markstein's
//              theorem).  The residuals stay exactly representable while
//              |z| is in [2^-30, 2^30]; any other z (0, tiny, huge, inf,
//              NaN) takes the IEEE division;
//   TDIV_IEEE  any other T: the IEEE division.
// Bit-equal to z / T: tests/cpu_sim/numerics.cpp, mode divt.
constexpr int TDIV_POW2 = 0, TDIV_FAST = 1, TDIV_IEEE = 2;
__device__ __forceinline__ int tg_div_t_mode(float T) {
  if (T >= 0x1p-126f && (tg_f2u(T) & 0x7FFFFFu) == 0u) return TDIV_POW2;
  return (T >= 0x1p-20f && T <= 0x1p20f) ? TDIV_FAST : TDIV_IEEE;
}
__device__ __forceinline__ float tg_div_t(float z, float T, float rT, int mode) {
  if (mode == TDIV_POW2) return z * rT;
  const float az = __builtin_fabsf(z);
  if (mode == TDIV_FAST && az >= 0x1p-30f && az <= 0x1p30f) {
    const float q0 = z * rT;
    const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, T, z), rT, q0);
    return __builtin_fmaf(__builtin_fmaf(-q1, T, z), rT, q1);
  }
  return z / T;
}

__device__ __forceinline__ float tg_weight(float y, float m) {
  return (y == m) ? 1.0f : tg_expf(y - m);
}

__device__ __forceinline__ u64 tg_q40(float e) { return (u64)(e * 0x1p40f); }

// Weight of a kept id for its reported probability only (masses and draws
// never use it): tg_weight's formula continued below -32 down to
// y - m = -86 instead of returning 0 there (2^n with n >= -124 is still a
// normal scale and p 2^n a normal result), so that ids far below the
// maximum keep their relative accuracy.  Equal to tg_weight wherever
// y - m >= -32.
__device__ __forceinline__ float tg_weight_wide(float y, float m) {
  if (y == m) return 1.0f;
  const float x = y - m;
  if (!(x >= -86.0f)) return 0.0f;
  const float log2e = 0x1.715476p+0f;
  const float ln2_hi = 0x1.62ep-1f;
  const float ln2_lo = 0x1.0bfbe8p-15f;
  const float shifter = 12582912.0f;
  float t = x * log2e;
  float n = (t + shifter) - shifter;
  float r = __builtin_fmaf(n, -ln2_hi, x);
  r = __builtin_fmaf(n, -ln2_lo, r);
  float p = 0x1.a01a02p-13f;
  p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
  p = __builtin_fmaf(p, r, 0x1.111112p-7f);
  p = __builtin_fmaf(p, r, 0x1.555556p-5f);
  p = __builtin_fmaf(p, r, 0x1.555556p-3f);
  p = __builtin_fmaf(p, r, 0.5f);
  p = __builtin_fmaf(p, r, 1.0f);
  p = __builtin_fmaf(p, r, 1.0f);
  return __builtin_ldexpf(p, (int)n);
}

__device__ __forceinline__ float tg_u64_to_f32(u64 x) {
  if (x < (1ull << 24)) return (float)(uint32_t)x;
  int lz = __clzll((long long)x);
  int sh = 40 - lz;
  u64 m = x >> sh;
  u64 rem = x & ((1ull << sh) - 1);
  u64 half = 1ull << (sh - 1);
  if (rem > half || (rem == half && (m & 1))) m += 1;
  float f = (float)(uint32_t)m;
  return f * tg_u2f((uint32_t)(sh + 127) << 23);
}

__device__ __forceinline__ uint32_t tg_key(float f) {
  uint32_t u = tg_f2u(f);
  if (u == 0x80000000u) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float tg_unkey(uint32_t k) {
  return tg_u2f((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}
__device__ __forceinline__ u64 comp_key(uint32_t key, int v) {
  return ((u64)key << 32) | (u64)(0xFFFFFFFFu - (uint32_t)v);
}
__device__ __forceinline__ int comp_id(u64 c) { return (int)(0xFFFFFFFFu - (uint32_t)c); }
__device__ __forceinline__ float comp_y(u64 c) { return tg_unkey((uint32_t)(c >> 32)); }

// floor(a * b / 2^24) for a < 2^64, b < 2^24 (the product fits in 88 bits).
__device__ __forceinline__ u64 mul_shr24(u64 a, uint32_t b) {
  u64 lo = a * (u64)b;
  u64 hi = __umul64hi(a, (u64)b);
  return (hi << 40) | (lo >> 24);
}

// A 16-byte load that is not expected to be reused (streamed logits):
// marked non-temporal so it does not displace cache lines that are.
__device__ __forceinline__ uint4 tg_load_nt(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef unsigned v4u __attribute__((ext_vector_type(4)));
  const v4u t = __builtin_nontemporal_load((const v4u*)p);
  return make_uint4(t.x, t.y, t.z, t.w);
#else
  return *(const uint4*)p;
#endif
}

// Per-half signed 16-bit maxima of two words (one packed max).
__device__ __forceinline__ uint32_t pk_max_i16(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_max(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b)));
#else
  const short al = (short)(a & 0xFFFFu), bl = (short)(b & 0xFFFFu);
  const short ah = (short)(a >> 16), bh = (short)(b >> 16);
  return (uint32_t)(uint16_t)(al > bl ? al : bl) | ((uint32_t)(uint16_t)(ah > bh ? ah : bh) << 16);
#endif
}

// Per-half signed 16-bit minima of two words (one packed min).
__device__ __forceinline__ uint32_t pk_min_i16(uint32_t a, uint32_t b) {
#if defined(__HIP_DEVICE_COMPILE__)
  typedef short s16x2 __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t,
                            __builtin_elementwise_min(__builtin_bit_cast(s16x2, a), __builtin_bit_cast(s16x2, b)));
#else
  const short al = (short)(a & 0xFFFFu), bl = (short)(b & 0xFFFFu);
  const short ah = (short)(a >> 16), bh = (short)(b >> 16);
  return (uint32_t)(uint16_t)(al < bl ? al : bl) | ((uint32_t)(uint16_t)(ah < bh ? ah : bh) << 16);
#endif
}

// ------------------------------------------------------------------ waves

__device__ __forceinline__ int lane_id() { return __lane_id(); }

// Lane l's value (l wave-uniform) through the scalar unit, bit for bit.
__device__ __forceinline__ uint32_t readlane_u32(uint32_t x, int l) {
  return (uint32_t)__builtin_amdgcn_readlane((int)x, l);
}
__device__ __forceinline__ u64 readlane_u64(u64 x, int l) {
  return ((u64)readlane_u32((uint32_t)(x >> 32), l) << 32) | readlane_u32((uint32_t)x, l);
}
__device__ __forceinline__ float readlane_f32(float x, int l) { return tg_u2f(readlane_u32(tg_f2u(x), l)); }

// Butterfly wave reductions (defined with the lane permutes below).
template <typename T>
__device__ __forceinline__ T wave_sum(T x);
template <typename T>
__device__ __forceinline__ T wave_max(T x);
__device__ __forceinline__ float wave_maxf(float x);

// Inclusive wave scan with DPP lane moves (no trip through LDS): Kogge-Stone
// within rows of 16 lanes (row_shr 1, 2, 4, 8; a lane with no source adds
// 0), then the row totals: row_bcast:15 adds lane 15 of rows 0 and 2 to
// rows 1 and 3, row_bcast:31 adds lane 31 to rows 2 and 3.  Exact for
// integer sums (32- or 64-bit lanes).
template <int CTRL, int ROWS>
__device__ __forceinline__ uint32_t dpp_or0(uint32_t x) {
  return __builtin_amdgcn_update_dpp(0u, x, CTRL, ROWS, 0xF, false);
}
template <int CTRL, int ROWS, typename T>
__device__ __forceinline__ T dpp_or0_t(T x) {
  if constexpr (sizeof(T) == 8) {
    const u64 v = (u64)x;
    return (T)(((u64)dpp_or0<CTRL, ROWS>((uint32_t)(v >> 32)) << 32) | dpp_or0<CTRL, ROWS>((uint32_t)v));
  } else {
    return (T)dpp_or0<CTRL, ROWS>((uint32_t)x);
  }
}
template <typename T>
__device__ __forceinline__ T wave_incl_scan(T x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "integer lanes");
  x += dpp_or0_t<0x111, 0xF>(x);  // row_shr:1
  x += dpp_or0_t<0x112, 0xF>(x);  // row_shr:2
  x += dpp_or0_t<0x114, 0xF>(x);  // row_shr:4
  x += dpp_or0_t<0x118, 0xF>(x);  // row_shr:8
  x += dpp_or0_t<0x142, 0xA>(x);  // row_bcast:15 into rows 1, 3
  x += dpp_or0_t<0x143, 0xC>(x);  // row_bcast:31 into rows 2, 3
  return x;
}

// ------------------------------------------------------------------ shared

// Static shared scratch used by the block primitives.
struct BlockScratch {
  unsigned hc[256];        // radix histogram: counts
  u64 hm[256];             // radix histogram: masses
  u64 red64[16];
  unsigned red32[16];
  int sel, binc_i;
  unsigned need;
  u64 mass_above, found;
  unsigned cnt_above;
  int imin0, imin1;
  unsigned nbuf;
  int last;
};

template <typename T, int BS = NT>
__device__ __forceinline__ T block_sum(T x, T* red) {
  x = wave_sum(x);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if (lane_id() == 0) red[w] = x;
  __syncthreads();
  T t = 0;
#pragma unroll
  for (int i = 0; i < BS / 64; i++) t += red[i];
  return t;
}

template <typename T, int BS = NT>
__device__ __forceinline__ T block_max(T x, T* red) {
  x = wave_max(x);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if (lane_id() == 0) red[w] = x;
  __syncthreads();
  T t = red[0];
#pragma unroll
  for (int i = 1; i < BS / 64; i++) t = red[i] > t ? red[i] : t;
  return t;
}

// Count-based MSB radix select over a multiset of keys (8-bit digits).
// `en(f)` calls f(key) for every key this thread owns.  Returns a value T
// with #{key >= T} >= kth and #{key > T'} < kth for the exact kth key T'; T
// equals the kth largest key, or a prefix of it with zeroed low bits when
// the keys of that prefix number exactly what is needed (then
// #{key >= T} == kth).  kth >= 1 and the multiset holds >= kth keys.
template <typename K, int NBITS, int BS = NT, class Enum>
__device__ __forceinline__ K block_select_kth(Enum en, unsigned kth, BlockScratch& s) {
  K prefix = 0, pmask = 0;
  unsigned need = kth;
#pragma unroll 1  // one pass live at a time: callers hold large register state across
  for (int shift = NBITS - 8; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += BS) s.hc[i] = 0;
    __syncthreads();
    en([&](K x) {
      if ((x & pmask) == prefix) atomicAdd(&s.hc[(unsigned)(x >> shift) & 255u], 1u);
    });
    __syncthreads();
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      unsigned cs[4];
#pragma unroll
      for (int j = 0; j < 4; j++) cs[j] = s.hc[255 - 4 * lane - j];
      unsigned lsum = cs[0] + cs[1] + cs[2] + cs[3];
      unsigned cum = wave_incl_scan(lsum) - lsum;
      int found = -1;
      unsigned above = 0, bc = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if (found < 0 && cs[j] > 0 && cum + cs[j] >= need) {
          found = 255 - 4 * lane - j;
          above = cum;
          bc = cs[j];
        }
        cum += cs[j];
      }
      u64 bal = __ballot(found >= 0);
      int first = __ffsll((long long)bal) - 1;
      if (lane == first) {
        s.sel = found;
        s.need = need - above;
        s.binc_i = (int)bc;
      }
    }
    __syncthreads();
    const int d = s.sel;
    need = s.need;
    const unsigned bc = (unsigned)s.binc_i;
    prefix |= (K)d << shift;
    pmask |= (K)255 << shift;
    if (bc == need) break;
  }
  return prefix;
}

// Mass-based MSB radix select over unique 64-bit composite keys, each with
// an integer mass.  Finds the element i (in descending key order) that is
// the first with C_i >= target, where C_i is the inclusive mass prefix.
// `en(f)` calls f(key, mass) for every key this thread owns.  Returns the
// element's key; *before gets the mass strictly ahead of it, *rank the
// number of elements strictly ahead of it.
template <int BS = NT, class Enum>
__device__ __forceinline__ u64 block_mass_select(Enum en, u64 target, BlockScratch& s, u64* before,
                                 unsigned* rank) {
  u64 prefix = 0, pmask = 0;
  u64 mass_above = 0;
  unsigned cnt_above = 0;
  bool single = false;
#pragma unroll 1
  for (int shift = 56; shift >= 0; shift -= 8) {
    for (int i = threadIdx.x; i < 256; i += BS) {
      s.hc[i] = 0;
      s.hm[i] = 0;
    }
    __syncthreads();
    en([&](u64 x, u64 q) {
      if ((x & pmask) == prefix) {
        const unsigned d = (unsigned)(x >> shift) & 255u;
        atomicAdd(&s.hc[d], 1u);
        if (q) atomicAdd(&s.hm[d], q);
      }
    });
    __syncthreads();
    if (threadIdx.x < 64) {
      const int lane = threadIdx.x;
      unsigned cs[4];
      u64 ms[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        cs[j] = s.hc[255 - 4 * lane - j];
        ms[j] = s.hm[255 - 4 * lane - j];
      }
      u64 lm = ms[0] + ms[1] + ms[2] + ms[3];
      unsigned lc = cs[0] + cs[1] + cs[2] + cs[3];
      u64 cm = wave_incl_scan(lm) - lm + mass_above;
      unsigned cc = wave_incl_scan(lc) - lc + cnt_above;
      int found = -1;
      u64 ab = 0;
      unsigned ca = 0, bc = 0;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        if (found < 0 && cs[j] > 0 && cm + ms[j] >= target) {
          found = 255 - 4 * lane - j;
          ab = cm;
          ca = cc;
          bc = cs[j];
        }
        cm += ms[j];
        cc += cs[j];
      }
      u64 bal = __ballot(found >= 0);
      int first = __ffsll((long long)bal) - 1;
      if (lane == first) {
        s.sel = found;
        s.mass_above = ab;
        s.cnt_above = ca;
        s.binc_i = (int)bc;
      }
    }
    __syncthreads();
    const int d = s.sel;
    mass_above = s.mass_above;
    cnt_above = s.cnt_above;
    const int bc = s.binc_i;
    prefix |= (u64)d << shift;
    pmask |= (u64)255 << shift;
    if (bc == 1) {
      single = shift > 0;
      break;
    }
  }
  if (single) { // one element carries this prefix: fetch its full key
    __syncthreads();
    en([&](u64 x, u64) {
      if ((x & pmask) == prefix) s.found = x;
    });
    __syncthreads();
    prefix = s.found;
  }
  *before = mass_above;
  *rank = cnt_above;
  return prefix;
}

// In-place descending bitonic sort of n2 (power of two) keys in LDS.
__device__ __forceinline__ void block_bitonic_desc(u64* buf, int n2) {
  for (int size = 2; size <= n2; size <<= 1) {
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      for (int i = threadIdx.x; i < (n2 >> 1); i += NT) {
        const int pos = 2 * i - (i & (stride - 1));
        const int q = pos + stride;
        const bool desc = (pos & size) == 0;
        u64 a = buf[pos], b = buf[q];
        if (desc ? (a < b) : (a > b)) {
          buf[pos] = b;
          buf[q] = a;
        }
      }
      __syncthreads();
    }
  }
}

// Inclusive prefix sum of n <= 4*NT u64 values in LDS (in place).
__device__ __forceinline__ void block_incl_scan_u64(u64* c, int n, u64* red) {
  const int base = threadIdx.x * 4;
  u64 v[4];
  u64 run = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    v[j] = (base + j < n) ? c[base + j] : 0;
    run += v[j];
    v[j] = run;
  }
  u64 incl = wave_incl_scan(run);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if (lane_id() == 63) red[w] = incl;
  __syncthreads();
  u64 off = incl - run;
  for (int i = 0; i < w; i++) off += red[i];
#pragma unroll
  for (int j = 0; j < 4; j++)
    if (base + j < n) c[base + j] = v[j] + off;
  __syncthreads();
}

}  // namespace tgs

namespace tgs {

// ------------------------------------------------------------------ wave sorts
// One value per lane; "sorted" means descending with lane 0 holding the max.

template <typename T>
__device__ __forceinline__ T tmax(T a, T b) { return a > b ? a : b; }
template <typename T>
__device__ __forceinline__ T tmin(T a, T b) { return a < b ? a : b; }

// ------------------------------------------------------------------ lane permutes
// The value of lane (lane ^ S), S a power of two below 64, by VALU lane
// moves only (no trip through the LDS crossbar):
//   S = 1, 2   DPP quad_perm [1,0,3,2] / [2,3,0,1]
//   S = 4      DPP row_shl:4 and row_shr:4, picked by lane bit 2
//   S = 8      DPP row_ror:8 (rotation by half a 16-lane row)
//   S = 16/32  v_permlane16_swap / v_permlane32_swap of x with itself: the
//              two results hold the rows (halves) moved each way, picked by
//              the lane bit.
template <int S>
__device__ __forceinline__ uint32_t xor_lane32(uint32_t x) {
  static_assert(S == 1 || S == 2 || S == 4 || S == 8 || S == 16 || S == 32, "lane xor");
  if constexpr (S == 1) {
    return __builtin_amdgcn_update_dpp(0u, x, 0xB1, 0xF, 0xF, false);
  } else if constexpr (S == 2) {
    return __builtin_amdgcn_update_dpp(0u, x, 0x4E, 0xF, 0xF, false);
  } else if constexpr (S == 4) {
    const uint32_t up = __builtin_amdgcn_update_dpp(0u, x, 0x104, 0xF, 0xF, false);  // lane + 4
    const uint32_t dn = __builtin_amdgcn_update_dpp(0u, x, 0x114, 0xF, 0xF, false);  // lane - 4
    return (lane_id() & 4) ? dn : up;
  } else if constexpr (S == 8) {
    return __builtin_amdgcn_update_dpp(0u, x, 0x128, 0xF, 0xF, false);
  } else if constexpr (S == 16) {
    const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
    return (lane_id() & 16) ? r[0] : r[1];
  } else {
    const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
    return (lane_id() & 32) ? r[0] : r[1];
  }
}

// lane 63 - lane: DPP row_mirror (xor 15 inside a row), then xor 16 and 32
__device__ __forceinline__ uint32_t rev_lanes32(uint32_t x) {
  return xor_lane32<32>(xor_lane32<16>(__builtin_amdgcn_update_dpp(0u, x, 0x140, 0xF, 0xF, false)));
}

template <int S, typename T>
__device__ __forceinline__ T xor_lane(T x) {
  static_assert(sizeof(T) == 4 || sizeof(T) == 8, "32- or 64-bit lanes");
  if constexpr (sizeof(T) == 8) {
    const u64 v = (u64)x;
    return (T)(((u64)xor_lane32<S>((uint32_t)(v >> 32)) << 32) | xor_lane32<S>((uint32_t)v));
  } else if constexpr (__is_same(T, float)) {
    return tg_u2f(xor_lane32<S>(tg_f2u(x)));  // the bits, not the value
  } else {
    return (T)xor_lane32<S>((uint32_t)x);
  }
}

template <typename T>
__device__ __forceinline__ T rev_lanes(T x) {
  if constexpr (sizeof(T) == 8) {
    const u64 v = (u64)x;
    return (T)(((u64)rev_lanes32((uint32_t)(v >> 32)) << 32) | rev_lanes32((uint32_t)v));
  } else {
    return (T)rev_lanes32((uint32_t)x);
  }
}

// xor_lane for a stride known after unrolling
template <typename T>
__device__ __forceinline__ T xor_lane_s(T x, int s) {
  switch (s) {
    case 1: return xor_lane<1>(x);
    case 2: return xor_lane<2>(x);
    case 4: return xor_lane<4>(x);
    case 8: return xor_lane<8>(x);
    case 16: return xor_lane<16>(x);
    default: return xor_lane<32>(x);
  }
}

// Butterfly reductions over the wave with the lane moves above (every lane
// gets the result).  Exact for maxima and integer sums.
template <typename T>
__device__ __forceinline__ T wave_sum(T x) {
  x += xor_lane<32>(x);
  x += xor_lane<16>(x);
  x += xor_lane<8>(x);
  x += xor_lane<4>(x);
  x += xor_lane<2>(x);
  x += xor_lane<1>(x);
  return x;
}

// G (2 or 4) sums at once, x[g] summed over the wave: lane l ends with the
// sum for group l / (64 / G).  Each step halves the values a lane carries
// (the lane keeps one half, sends the other to its partner at lane ^ 32,
// then ^ 16) before the plain butterfly: one sum's cost instead of G.
// Exact for integer sums.
template <int G, typename T>
__device__ __forceinline__ T wave_sum_groups(const T (&x)[G]) {
  static_assert(G == 2 || G == 4, "groups");
  const int lane = lane_id();
  const bool h32 = (lane & 32) != 0;
  T k;
  if constexpr (G == 4) {
    T k0 = h32 ? x[2] : x[0], k1 = h32 ? x[3] : x[1];
    const T s0 = h32 ? x[0] : x[2], s1 = h32 ? x[1] : x[3];
    k0 += xor_lane<32>(s0);
    k1 += xor_lane<32>(s1);
    const bool h16 = (lane & 16) != 0;
    k = h16 ? k1 : k0;
    k += xor_lane<16>(h16 ? k0 : k1);
  } else {
    k = h32 ? x[1] : x[0];
    k += xor_lane<32>(h32 ? x[0] : x[1]);
    k += xor_lane<16>(k);
  }
  k += xor_lane<8>(k);
  k += xor_lane<4>(k);
  k += xor_lane<2>(k);
  k += xor_lane<1>(k);
  return k;
}

template <typename T>
__device__ __forceinline__ T wave_max(T x) {
  T y;
  y = xor_lane<32>(x); x = y > x ? y : x;
  y = xor_lane<16>(x); x = y > x ? y : x;
  y = xor_lane<8>(x); x = y > x ? y : x;
  y = xor_lane<4>(x); x = y > x ? y : x;
  y = xor_lane<2>(x); x = y > x ? y : x;
  y = xor_lane<1>(x); x = y > x ? y : x;
  return x;
}

__device__ __forceinline__ float wave_maxf(float x) {
  x = fmaxf(x, tg_u2f(xor_lane32<32>(tg_f2u(x))));
  x = fmaxf(x, tg_u2f(xor_lane32<16>(tg_f2u(x))));
  x = fmaxf(x, tg_u2f(xor_lane32<8>(tg_f2u(x))));
  x = fmaxf(x, tg_u2f(xor_lane32<4>(tg_f2u(x))));
  x = fmaxf(x, tg_u2f(xor_lane32<2>(tg_f2u(x))));
  x = fmaxf(x, tg_u2f(xor_lane32<1>(tg_f2u(x))));
  return x;
}

// Bitwise OR over the wave, as a wave-uniform (scalar) value.
__device__ __forceinline__ uint32_t wave_or(uint32_t x) {
  x |= xor_lane32<32>(x);
  x |= xor_lane32<16>(x);
  x |= xor_lane32<8>(x);
  x |= xor_lane32<4>(x);
  x |= xor_lane32<2>(x);
  x |= xor_lane32<1>(x);
  return (uint32_t)__builtin_amdgcn_readfirstlane((int)x);
}

// Number of set bits of a wave mask below this lane.
__device__ __forceinline__ unsigned lanes_below(u64 mask) {
  return __builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// Orders a wave's LDS accesses before and after it (LDS operations of one
// wave execute in issue order, so this only restrains the compiler).
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Bitonic sort of 64 values across the lanes of a wave (descending).  The
// strides are template arguments, so every lane move is one fixed DPP or
// permlane instruction (a loop over a runtime stride compiles to branches).
template <int SIZE, int STRIDE, typename T>
__device__ __forceinline__ T sort_stage(T x, int lane) {
  if constexpr (STRIDE == 0) {
    return x;
  } else {
    const T y = xor_lane<STRIDE>(x);
    const bool lower = (lane & STRIDE) == 0;
    const bool desc = (lane & SIZE) == 0;
    x = (lower == desc) ? tmax(x, y) : tmin(x, y);
    return sort_stage<SIZE, STRIDE / 2>(x, lane);
  }
}
template <int SIZE, typename T>
__device__ __forceinline__ T sort_sizes(T x, int lane) {
  if constexpr (SIZE > 64) {
    return x;
  } else {
    x = sort_stage<SIZE, SIZE / 2>(x, lane);
    return sort_sizes<SIZE * 2>(x, lane);
  }
}
template <typename T>
__device__ __forceinline__ T wave_sort_desc(T x) {
  return sort_sizes<2>(x, lane_id());
}

// Half-cleaner steps of a bitonic merge (descending), strides STRIDE..1.
template <int STRIDE, typename T>
__device__ __forceinline__ T merge_stage(T c, int lane) {
  if constexpr (STRIDE == 0) {
    return c;
  } else {
    const T y = xor_lane<STRIDE>(c);
    c = ((lane & STRIDE) == 0) ? tmax(c, y) : tmin(c, y);
    return merge_stage<STRIDE / 2>(c, lane);
  }
}

// a and b sorted descending across lanes: the 64 largest of their union,
// sorted descending (max with the reversed b is bitonic, then 6 merge steps).
template <typename T>
__device__ __forceinline__ T wave_merge_top64(T a, T b) {
  return merge_stage<32>(tmax(a, rev_lanes(b)), lane_id());
}

}  // namespace tgs
