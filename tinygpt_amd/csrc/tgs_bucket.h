// tgs_bucket.h -- the count and exact-mass histogram over buckets below the
// row maximum that the top-k and top-p kernels place their cut and draw
// with (one workgroup of 1024 threads per row).
//
// A composite with canonical logit y under the row maximum m lands in
// bucket floor((m - y) * 32) (0 at y == m); y - m <= -32 (mass 0) lands in
// bucket NB.  A larger y never lands in a later bucket, so the bucket order
// is the composite order (logit desc, id asc) and prefixes over the buckets
// locate the bucket holding the element at a given count or mass; only that
// bucket's members are then ranked.  Width 1/32 keeps a bucket to one or two
// distinct bf16 values (a wave sort of at most 64 members in the common case).
#pragma once

#include "tgs_device.h"

namespace tgs {
namespace bucket {

constexpr int NB = 1024;  // buckets of width 1/32 below the maximum (+1 for mass 0)

struct alignas(16) u64x2 {
  u64 x, y;
};

__device__ __forceinline__ int of(float y, float m) {
  if (y == m) return 0;
  const float x = y - m;
  if (!(x > -32.0f)) return NB;
  return (int)(-x * 32.0f);
}

// Exact mass floor(exp(y - m) 2^40) of a canonical logit y <= m.
__device__ __forceinline__ u64 mass(float y, float m) { return tg_q40(y == m ? 1.0f : tg_expf_nonpos(y - m)); }

__device__ __forceinline__ u64 mass_c(u64 c, float m) { return mass(comp_y(c), m); }

// In place: CI[0..NB] bucket counts become inclusive prefixes, MI[0..NB)
// bucket masses inclusive prefixes with MI[NB] = MI[NB - 1] (the last bucket
// holds mass 0).  BT threads (NB a multiple of BT), thread t owns buckets
// [t NB/BT, (t + 1) NB/BT); red32 / red64 hold BT / 64 entries.  The
// histogram must be complete (a barrier) before the call; ends with a
// barrier.
template <int BT>
__device__ __forceinline__ void prefix(unsigned* CI, u64* MI, unsigned* red32, u64* red64) {
  static_assert(NB % BT == 0, "whole buckets per thread");
  constexpr int PER = NB / BT;
  const int t = threadIdx.x, w = t >> 6, lane = lane_id();
  unsigned cc[PER];
  u64 cm[PER];
  unsigned ct = 0;
  u64 mt = 0;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    cc[i] = CI[t * PER + i];
    cm[i] = MI[t * PER + i];
    ct += cc[i];
    mt += cm[i];
  }
  const unsigned tailc = (t == BT - 1) ? CI[NB] : 0u;
  unsigned ci = wave_incl_scan(ct);
  u64 mi = wave_incl_scan(mt);
  if (lane == 63) {
    red32[w] = ci;
    red64[w] = mi;
  }
  __syncthreads();
  unsigned oc = ci - ct;
  u64 om = mi - mt;
  for (int v = 0; v < w; v++) {
    oc += red32[v];
    om += red64[v];
  }
#pragma unroll
  for (int i = 0; i < PER; i++) {
    oc += cc[i];
    om += cm[i];
    CI[t * PER + i] = oc;
    MI[t * PER + i] = om;
  }
  if (t == BT - 1) {
    CI[NB] = oc + tailc;
    MI[NB] = om;
  }
  __syncthreads();
}

__device__ __forceinline__ unsigned count_before(const unsigned* CI, int bq) { return bq ? CI[bq - 1] : 0u; }
__device__ __forceinline__ u64 mass_before(const u64* MI, int bq) { return bq ? MI[bq - 1] : 0ull; }

// The bucket whose inclusive count first reaches target (1 <= target <=
// CI[NB]).  Every thread calls it; one barrier; *sel is scratch that no
// thread reads again before the next barrier.
template <int BT>
__device__ __forceinline__ int find_count(const unsigned* CI, unsigned target, int* sel) {
  constexpr int PER = NB / BT;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int t = threadIdx.x * PER + i;
    if (CI[t] >= target && (t == 0 || CI[t - 1] < target)) *sel = t;
  }
  if (threadIdx.x == 0 && CI[NB] >= target && CI[NB - 1] < target) *sel = NB;
  __syncthreads();
  return *sel;
}

// The bucket whose inclusive mass first reaches target (1 <= target <=
// MI[NB - 1]); as find_count.
template <int BT>
__device__ __forceinline__ int find_mass(const u64* MI, u64 target, int* sel) {
  constexpr int PER = NB / BT;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int t = threadIdx.x * PER + i;
    if (MI[t] >= target && (t == 0 || MI[t - 1] < target)) *sel = t;
  }
  __syncthreads();
  return *sel;
}

// Ranks the n (<= BT, uniform) distinct composites L[0, n) gathered into
// LDS (a barrier after the gather; L[n] == 0 when n is odd): R[0, n) in
// descending order, Q[0, n) the inclusive masses under m.  At most 64: one
// wave's bitonic sort; more: the rank of each is the number of larger
// composites, counted by the waves that hold members (two per 16-byte
// broadcast read).  red64: BT / 64 entries.  Ends with a barrier.
template <int BT>
__device__ __forceinline__ void rank_list(const u64* L, unsigned n, float m, u64* R, u64* Q, u64* red64) {
  const int i = threadIdx.x, w = i >> 6, lane = lane_id();
  if (n <= 64) {
    if (w == 0) {
      u64 x = lane < (int)n ? L[lane] : 0ull;
      x = wave_sort_desc(x);
      const u64 q = lane < (int)n ? mass_c(x, m) : 0ull;
      const u64 ci = wave_incl_scan(q);
      if (lane < (int)n) {
        R[lane] = x;
        Q[lane] = ci;
      }
    }
    __syncthreads();
    return;
  }
  if (w * 64 < (int)n) {
    const u64 x = i < (int)n ? L[i] : ~0ull;
    int rk = 0;
    const int np = ((int)n + 1) / 2;
    const u64x2* L2 = (const u64x2*)L;
#pragma unroll 4
    for (int p = 0; p < np; p++) {
      const u64x2 e = L2[p];
      rk += (e.x > x) + (e.y > x);
    }
    if (i < (int)n) R[rk] = x;
  }
  __syncthreads();
  const u64 q = i < (int)n ? mass_c(R[i], m) : 0ull;
  const u64 wi = wave_incl_scan(q);
  if (lane == 63) red64[w] = wi;
  __syncthreads();
  u64 off = 0;
  for (int v = 0; v < w; v++) off += red64[v];
  if (i < (int)n) Q[i] = off + wi;
  __syncthreads();
}

// First rank of a ranked list whose inclusive mass reaches target (>= 1 and
// at most Q[n - 1]).  Every thread calls it; two barriers.
template <int BT>
__device__ __forceinline__ int first_rank(const u64* Q, unsigned n, u64 target, int* slot) {
  const int i = threadIdx.x;
  if (i < (int)n && Q[i] >= target && (i == 0 || Q[i - 1] < target)) *slot = i;
  __syncthreads();
  const int f = *slot;
  __syncthreads();
  return f;
}

// One wave ranks L[0, n) (n <= 64) into R (descending) and Q (inclusive
// masses under m); no barrier.
__device__ __forceinline__ void wave_rank64(const u64* L, unsigned n, float m, u64* R, u64* Q) {
  const int lane = lane_id();
  u64 x = lane < (int)n ? L[lane] : 0ull;
  x = wave_sort_desc(x);
  const u64 q = lane < (int)n ? mass_c(x, m) : 0ull;
  const u64 ci = wave_incl_scan(q);
  if (lane < (int)n) {
    R[lane] = x;
    Q[lane] = ci;
  }
}

// The buckets whose inclusive masses first reach t1 and t2 (both in
// [1, MI[NB - 1]]), in one pass and one barrier.
template <int BT>
__device__ __forceinline__ void find_mass2(const u64* MI, u64 t1, u64 t2, int* s1, int* s2) {
  constexpr int PER = NB / BT;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int t = threadIdx.x * PER + i;
    const u64 lo = t ? MI[t - 1] : 0ull, hi = MI[t];
    if (hi >= t1 && lo < t1) *s1 = t;
    if (hi >= t2 && lo < t2) *s2 = t;
  }
  __syncthreads();
}

// First rank of a ranked list whose inclusive mass reaches target (>= 1, at
// most Q[n - 1]); one barrier, so each call needs a slot of its own.
__device__ __forceinline__ int first_rank_once(const u64* Q, unsigned n, u64 target, int* slot) {
  const int i = threadIdx.x;
  if (i < (int)n && Q[i] >= target && (i == 0 || Q[i - 1] < target)) *slot = i;
  __syncthreads();
  return *slot;
}

}  // namespace bucket
}  // namespace tgs
