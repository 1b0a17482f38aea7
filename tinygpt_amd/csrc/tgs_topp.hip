// tgs_topp.hip -- rows that sample with top-p over the whole vocabulary (top_k
// disabled: k <= 0 or k >= V), one workgroup of 1024 threads per row.
//
// The contract keeps the smallest prefix of the allowed ids in (y desc,
// id asc) order whose exact mass reaches P = floor(S p24 / 2^24) and draws
// the first id whose inclusive prefix exceeds t = floor(S' u24 / 2^24);
// masses are q = floor(exp(y - m) 2^40).  Only ids with q > 0 can be the cut
// or the draw (both are where the prefix grows), and those lie within 32 of
// the maximum.  So:
//
//   pass 1  stream the row: y (mask, penalties, 1/T), the maximum m, the
//           allowed count, the largest and smallest composite (diagnostics);
//   pass 2  stream the row: per allowed id with y - m > -32 its mass q,
//           added to bucket floor((m - y) * 8) of a 256-bucket histogram
//           (mass and count).  Bucket order follows the sorted order (a
//           larger y never lands in a later bucket), so the prefix over
//           buckets locates the bucket of the cut and then of the draw;
//   pass 3  stream the row: gather that bucket's ids (composites) into LDS,
//           rank them exactly by counting, scan their masses in rank order
//           and pick the element.  The draw's bucket reuses the ranked list
//           when it is the cut's bucket; otherwise one more gather.
//
// A bucket of more than CAPG ids (a flat row: ties, tiny temperature
// spreads) is resolved by a mass-weighted radix selection restricted to the
// bucket instead (a few more passes).  The row stays in L2 / MALL between
// passes; exp runs once per id.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace topp {

constexpr int BT = TOPP_NT;    // threads per workgroup
constexpr int WT = BT / 64;    // waves
constexpr int NBKT = 256;      // histogram buckets of width 1/8 in y below m
constexpr int CAPG = TOPP_CAP; // ids of one bucket ranked in LDS

struct Scratch {
  u64 hm[NBKT];
  unsigned hc[NBKT];
  u64 red64[WT];
  u64 red64b[WT];
  unsigned red32[WT];
  float redf[WT];
  unsigned ng;    // gathered ids
  int first;      // first rank meeting the target
  int bsel;       // selected bucket
  u64 bbefore;    // mass of the buckets ahead of it
  unsigned bcnt;  // ids ahead of it
};

// Calls f(id, y, allowed) for every id of the row (y: canonical logit after
// penalties and temperature; allowed: the mask bit is set and y > -inf).
template <typename Tin, class F>
__device__ __forceinline__ void stream(const SampleArgs& a, const Row& r, const int2* hash, const uint32_t* hbits,
                                       const Tin* rowp, F f) {
  constexpr int EPV = Elem<Tin>::EPV;
  const int nvec = (a.V + EPV - 1) / EPV;
  for (int vi = threadIdx.x; vi < nvec; vi += BT) {
    const int v = vi * EPV;
    const uint4 raw = load_vec<Tin>(rowp, v, a.V, a.aligned);
    const uint32_t mw = r.mrow ? r.mrow[v >> 5] : 0xFFFFFFFFu;
    const uint32_t hw = r.use_pen ? hbits[v >> 5] : 0u;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      const int id = v + e;
      if (id >= a.V) break;
      float z = Elem<Tin>::get(raw, e);
      if ((hw >> (id & 31)) & 1u) z = penalise(z, hash_count(hash, a.TS, a.ts_shift, id), r);
      const float y = z * r.invT;
      const bool ok = ((mw >> (id & 31)) & 1u) && (y > -__builtin_inff());
      f(id, y, ok);
    }
  }
}

// Weight of y under the row maximum m (y <= m): exp(y - m), 1 at y == m.
__device__ __forceinline__ float weight_le(float y, float m) {
  return (y == m) ? 1.0f : tg_expf_nonpos(y - m);
}

// Histogram bucket of an allowed y with positive-or-boundary weight, -1 when
// y - m <= -32 (mass 0: never the cut or the draw).
__device__ __forceinline__ int bucket_of(float y, float m) {
  if (y == m) return 0;
  const float x = y - m;
  if (!(x > -32.0f)) return -1;
  return (int)(-x * 8.0f);
}

template <typename T>
__device__ __forceinline__ T block_reduce_sum(T x, T* red) {
  x = wave_sum(x);
  if (lane_id() == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  T t = 0;
#pragma unroll
  for (int i = 0; i < WT; i++) t += red[i];
  __syncthreads();
  return t;
}

template <typename T>
__device__ __forceinline__ T block_reduce_max(T x, T* red) {
  x = wave_max(x);
  if (lane_id() == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  T t = red[0];
#pragma unroll
  for (int i = 1; i < WT; i++) t = red[i] > t ? red[i] : t;
  __syncthreads();
  return t;
}

// Bucket scan (wave 0): the first bucket whose inclusive mass reaches
// `target` (>= 1), with the mass and count ahead of it, into ts.
__device__ __forceinline__ void pick_bucket(Scratch& ts, u64 target) {
  const int lane = lane_id();
  u64 ms[4];
  unsigned cs[4];
  u64 lm = 0;
  unsigned lc = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    ms[j] = ts.hm[4 * lane + j];
    cs[j] = ts.hc[4 * lane + j];
    lm += ms[j];
    lc += cs[j];
  }
  u64 cm = wave_incl_scan(lm) - lm;
  unsigned cc = wave_incl_scan(lc) - lc;
  int found = -1;
  u64 ab = 0;
  unsigned ca = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (found < 0 && cm + ms[j] >= target) {
      found = 4 * lane + j;
      ab = cm;
      ca = cc;
    }
    cm += ms[j];
    cc += cs[j];
  }
  // one lane writes the result (the first lane that found the bucket)
  const u64 bal = __ballot(found >= 0);
  const int first = bal ? __ffsll((long long)bal) - 1 : 0;
  const int fb = __shfl(found, first, 64);
  const u64 fab = __shfl(ab, first, 64);
  const unsigned fca = __shfl(ca, first, 64);
  if (lane == 0) {
    ts.bsel = fb;
    ts.bbefore = fab;
    ts.bcnt = fca;
  }
}

// The bucket's ids ranked in LDS: R[0, n) holds their composites in
// descending order and Q[0, n) their inclusive mass prefix.  Returns n, or
// -1 when the bucket holds more than CAPG ids (nothing ranked).
template <typename Tin>
__device__ __forceinline__ int rank_bucket(const SampleArgs& a, const Row& r, const int2* hash, const uint32_t* hbits,
                                           const Tin* rowp, float m, int bkt, u64* L, u64* R, u64* Q, Scratch& ts) {
  if (threadIdx.x == 0) ts.ng = 0;
  __syncthreads();
  stream<Tin>(a, r, hash, hbits, rowp, [&](int id, float y, bool ok) {
    if (ok && bucket_of(y, m) == bkt) {
      const unsigned slot = atomicAdd(&ts.ng, 1u);
      if (slot < (unsigned)CAPG) L[slot] = comp_key(tg_key(y), id);
    }
  });
  __syncthreads();
  const int n = (int)ts.ng;
  if (n > CAPG) return -1;
  // rank = number of larger composites (composites are distinct)
  const int j0 = threadIdx.x, j1 = threadIdx.x + BT;
  const u64 x0 = j0 < n ? L[j0] : ~0ull, x1 = j1 < n ? L[j1] : ~0ull;
  int r0 = 0, r1 = 0;
  for (int i = 0; i < n; i++) {
    const u64 li = L[i];
    r0 += li > x0;
    r1 += li > x1;
  }
  if (j0 < n) R[r0] = x0;
  if (j1 < n) R[r1] = x1;
  __syncthreads();
  // masses in rank order, inclusive prefix (two ranks per thread)
  const int k0 = 2 * threadIdx.x, k1 = k0 + 1;
  const u64 q0 = k0 < n ? tg_q40(weight_le(comp_y(R[k0]), m)) : 0ull;
  const u64 q1 = k1 < n ? tg_q40(weight_le(comp_y(R[k1]), m)) : 0ull;
  const u64 ls = q0 + q1;
  const u64 wi = wave_incl_scan(ls);
  if (lane_id() == 63) ts.red64b[threadIdx.x >> 6] = wi;
  __syncthreads();
  u64 off = 0;
  for (int i = 0; i < (int)(threadIdx.x >> 6); i++) off += ts.red64b[i];
  const u64 c0 = off + wi - ls + q0;
  if (k0 < n) Q[k0] = c0;
  if (k1 < n) Q[k1] = c0 + q1;
  __syncthreads();
  return n;
}

// First rank of the ranked bucket whose within-bucket inclusive prefix
// reaches target (>= 1).
__device__ __forceinline__ int first_rank(const u64* Q, int n, u64 target, Scratch& ts) {
  if (threadIdx.x == 0) ts.first = 0x7FFFFFFF;
  __syncthreads();
  int mine = 0x7FFFFFFF;
  for (int i = threadIdx.x; i < n; i += BT)
    if (Q[i] >= target && (i == 0 || Q[i - 1] < target)) mine = i;
  if (mine != 0x7FFFFFFF) atomicMin(&ts.first, mine);
  __syncthreads();
  return ts.first;
}

// The element of bucket bkt whose inclusive prefix (from the bucket start)
// first reaches target: its composite, the mass strictly ahead of it within
// the bucket and its rank within the bucket.  `ranked` says whether R/Q
// already hold this bucket (n ids).
template <typename Tin>
__device__ __forceinline__ u64 select_in_bucket(const SampleArgs& a, const Row& r, const int2* hash,
                                                const uint32_t* hbits, const Tin* rowp, float m, int bkt,
                                                u64 target, int n, u64* R, u64* Q, Scratch& ts, BlockScratch& bs,
                                                u64* before, unsigned* rank) {
  if (n >= 0) {
    const int i = first_rank(Q, n, target, ts);
    *before = i > 0 ? Q[i - 1] : 0ull;
    *rank = (unsigned)i;
    return R[i];
  }
  // more ids than CAPG: mass-weighted radix selection over the bucket
  auto en = [&](auto f) {
    stream<Tin>(a, r, hash, hbits, rowp, [&](int id, float y, bool ok) {
      if (ok && bucket_of(y, m) == bkt) f(comp_key(tg_key(y), id), tg_q40(weight_le(y, m)));
    });
  };
  return block_mass_select<BT>(en, target, bs, before, rank);
}

template <typename Tin>
__global__ __launch_bounds__(BT) void topp_kernel(SampleArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ Scratch ts;
  __shared__ BlockScratch bs;
  const int b = blockIdx.x;
  if (b >= a.B) return;
  Row r;
  if (!row_setup(a, b, 0, r) || r.mode != 2 || (r.k >= 1 && r.k < a.V)) return;  // other kernels' rows
  const int bw = a.TS > 0 ? (a.V + 31) / 32 : 0;
  uint32_t* hbits = (uint32_t*)smem;
  int2* hash = (int2*)(smem + ((bw * 4 + 15) / 16) * 16);
  u64* L = (u64*)((unsigned char*)hash + (size_t)a.TS * 8);
  u64* R = L + CAPG;
  u64* Q = R + CAPG;
  r.v0 = 0;
  r.v1 = a.V;
  if (r.use_pen) hash_build<BT>(a, r, hash, hbits, bw);
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  float* post = a.dbg.post_logits ? a.dbg.post_logits + (long long)b * a.V : nullptr;

  // pass 1: maximum, allowed count, largest and smallest composite
  u64 best = 0, minc = ~0ull;
  unsigned nv = 0;
  stream<Tin>(a, r, hash, hbits, rowp, [&](int id, float y, bool ok) {
    if (post) post[id] = ok ? y : -__builtin_inff();
    if (ok) {
      const u64 c = comp_key(tg_key(y), id);
      best = c > best ? c : best;
      minc = c < minc ? c : minc;
      nv++;
    }
  });
  best = block_reduce_max(best, ts.red64);
  minc = ~block_reduce_max(~minc, ts.red64);
  nv = block_reduce_sum(nv, ts.red32);
  if (nv == 0) {
    if (threadIdx.x == 0) {
      a.out[b] = -1;
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
  } else {
    const float m = comp_y(best);
    // pass 2: mass histogram over buckets below m
    for (int i = threadIdx.x; i < NBKT; i += BT) {
      ts.hm[i] = 0;
      ts.hc[i] = 0;
    }
    __syncthreads();
    u64 Sl = 0;
    stream<Tin>(a, r, hash, hbits, rowp, [&](int id, float y, bool ok) {
      if (!ok) return;
      const int bk = bucket_of(y, m);
      if (bk < 0) return;
      const u64 q = tg_q40(weight_le(y, m));
      Sl += q;
      atomicAdd(&ts.hc[bk], 1u);
      if (q) atomicAdd(&ts.hm[bk], q);
    });
    const u64 S = block_reduce_sum(Sl, ts.red64);  // also orders the histogram atomics
    // the cut (top-p): element i* with inclusive prefix >= P
    u64 cutc = minc, Sp = S;
    unsigned ntopp = nv;
    int nr = -2, rb = -1;  // ids ranked in R/Q (-2: none), their bucket
    if (r.top_p < 1.0f) {
      const uint32_t pq = (uint32_t)(r.top_p * 16777216.0f);
      const u64 P = mul_shr24(S, pq);
      if (P == 0) {
        cutc = best;
        Sp = tg_q40(1.0f);
        ntopp = 1;
      } else {
        if (threadIdx.x < 64) pick_bucket(ts, P);
        __syncthreads();
        const int bk = ts.bsel;
        const u64 bb = ts.bbefore;
        const unsigned bc = ts.bcnt;
        __syncthreads();
        nr = rank_bucket<Tin>(a, r, hash, hbits, rowp, m, bk, L, R, Q, ts);
        rb = bk;
        u64 before;
        unsigned rank;
        cutc = select_in_bucket<Tin>(a, r, hash, hbits, rowp, m, bk, P - bb, nr, R, Q, ts, bs, &before, &rank);
        Sp = bb + before + tg_q40(weight_le(comp_y(cutc), m));
        ntopp = bc + rank + 1;
      }
    }
    // the draw: first element with inclusive prefix > t
    const uint32_t uq = (uint32_t)(r.u * 16777216.0f);
    const u64 t = mul_shr24(Sp, uq);
    __syncthreads();
    if (threadIdx.x < 64) pick_bucket(ts, t + 1);
    __syncthreads();
    const int bk = ts.bsel;
    const u64 bb = ts.bbefore;
    __syncthreads();
    if (bk != rb) nr = rank_bucket<Tin>(a, r, hash, hbits, rowp, m, bk, L, R, Q, ts);
    u64 before;
    unsigned rank;
    const u64 pick = select_in_bucket<Tin>(a, r, hash, hbits, rowp, m, bk, t + 1 - bb, nr, R, Q, ts, bs, &before,
                                           &rank);
    if (threadIdx.x == 0) {
      a.out[b] = comp_id(pick);
      write_row_diag(a, b, (int)nv, (int)ntopp, S, Sp, comp_id(cutc));
    }
  }
  if (a.dbg.kept_ids)
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) a.dbg.kept_ids[(long long)b * a.dbg.kept_cap + i] = -1;
  if (a.dbg.kept_probs)
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) a.dbg.kept_probs[(long long)b * a.dbg.kept_cap + i] = 0.0f;
}

}  // namespace topp

size_t topp_lds_bytes(int V, int TS) {
  const int bw = TS > 0 ? (V + 31) / 32 : 0;
  return (size_t)((bw * 4 + 15) / 16) * 16 + (size_t)TS * 8 + (size_t)3 * TOPP_CAP * 8;
}

hipError_t launch_topp(const SampleArgs& a, int dtype, size_t lds, hipStream_t st) {
  if (dtype == 1) hipLaunchKernelGGL(topp::topp_kernel<uint16_t>, dim3(a.B), dim3(TOPP_NT), lds, st, a);
  else hipLaunchKernelGGL(topp::topp_kernel<float>, dim3(a.B), dim3(TOPP_NT), lds, st, a);
  return hipGetLastError();
}

hipError_t set_topp_lds_limit(size_t bytes) {
  const void* fns[] = {(const void*)topp::topp_kernel<float>, (const void*)topp::topp_kernel<uint16_t>};
  hipError_t e = hipSuccess;
  for (const void* f : fns) {
    hipError_t e2 = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e2 != hipSuccess) e = e2;
  }
  return e;
}

}  // namespace tgs
