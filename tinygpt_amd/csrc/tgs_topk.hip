// tgs_topk.hip -- batches whose rows are greedy or sample with 1 <= top_k <=
// KMAX (1024), for rows that fit in the registers of one workgroup (bf16 rows
// up to 163840 ids, fp32 rows up to 81920; 16-byte aligned, a whole number of
// 16-byte vectors): one workgroup of 1024 threads per row, the row read from
// HBM exactly once.
//
//   load    every thread issues its NVR 16-byte vectors (ids tid*EPV +
//           j*1024*EPV) and keeps them; the row's history (ids -> counts)
//           goes into an LDS hash and a bitmap while they are in flight.
//   bound   four slot values per thread, each the largest logit of a
//           disjoint group of its ids (packed 16-bit integer maxima and
//           minima of the raw bf16 words, 32-bit ones of fp32 words; -inf
//           where that lands on a NaN).  So at least k' distinct ids lie at
//           or above the k'-th largest slot value.  History ids may
//           still be penalised downward, so k' = k + (distinct history ids
//           of the row).  The k'-th slot is found to 16 key bits by one
//           histogram of the slots' distance below the largest one (a radix
//           pass only when it lies more than 254 bf16 steps below).
//           Temperature is applied after the bound: 16 representable values
//           of slack keep every id whose scaled logit could round to the
//           bound's.
//   collect one test per vector (a packed 16-bit maximum of its bf16
//           patterns against the bound) into a per-thread bit mask; the
//           passing vectors' indexes go to LDS (block offsets from a wave
//           scan); each is read again (16 bytes, a scattered gather), its
//           ids tested one by one, and the passing ids turned into
//           composites (logit desc, id asc), history ids skipped there and
//           added with their penalised logits instead.
//   tail    over the candidates (at most 4096, four per thread): the maximum
//           m, then a count and exact-mass histogram over 1024 buckets of
//           width 1/32 below m (y - m <= -32, mass 0, in one more bucket).
//           Bucket order follows the composite order, so prefixes over the
//           buckets find the bucket of the k-th composite, of the top-p cut
//           and of the draw; only those buckets are ranked (a wave sort of
//           at most 64, else counting ranks) to place the element inside.
//           The cut's and the draw's buckets share one gather when the
//           draw's bucket is fixed before the cut is resolved.
//
// A candidate list beyond its capacity (massive ties at the bound) falls
// back to a radix selection over all ids of the row, read again from
// L2 / MALL; a bucket beyond the ranking capacity to radix selections
// restricted to it.
#include "tgs_bucket.h"
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace topk {

constexpr int BT = TOPK_NT;    // threads per workgroup
constexpr int WT = BT / 64;    // waves
constexpr int CAPK = TOPK_CAP; // candidates
constexpr int CPT = CAPK / BT; // candidates per thread in the tail
constexpr int NB = bucket::NB; // mass buckets below the maximum (+1 for mass 0)
constexpr int LCAP = KMAX;     // ids of one bucket ranked in LDS
static_assert(NB == BT, "one bucket per thread in the prefix");
static_assert(2 * LCAP * 8 >= CAPK * 4, "candidate ids alias the ranking lists");

struct Scratch {
  u64 red64[WT];
  u64 red64b[WT];
  unsigned red32[WT];
  unsigned nc;    // candidates written
  unsigned ng;    // bucket members gathered
  unsigned na;    // collection: candidates appended
  unsigned need;  // bound: slots still needed below the histogram range
  int dsel;       // bound: histogram bin of the k'-th slot
  int sel[3];     // tail: buckets of the k-th, of the cut and of the draw
  int first;      // tail: first rank meeting a mass target
  unsigned ng2;   // tail: members of the draw's bucket gathered with the cut's
  int first2;     // tail: the draw's rank in the one-gather tail
};

template <typename T>
__device__ __forceinline__ T bsum(T x, T* red) {
  x = wave_sum(x);
  if (lane_id() == 0) red[threadIdx.x >> 6] = x;
  __syncthreads();
  T t = 0;
#pragma unroll
  for (int i = 0; i < WT; i++) t += red[i];
  __syncthreads();
  return t;
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
  return i == 0 ? v.x : i == 1 ? v.y : i == 2 ? v.z : v.w;
}

template <typename Tin, int NVR>
struct Regs {
  static constexpr int EPV = Elem<Tin>::EPV;
  uint4 raw[NVR];  // the row, packed as loaded
  __device__ __forceinline__ static int vec_id(int j) { return ((int)threadIdx.x + j * BT) * EPV; }
  // every vector, from addresses clamped into the row (the row is 16-byte
  // aligned and a whole number of vectors)
  __device__ __forceinline__ void load(const Tin* rowp, int V) {
#pragma unroll
    for (int j = 0; j < NVR; j++) {
      const int v = vec_id(j);
      raw[j] = *(const uint4*)(rowp + (v < V ? v : V - EPV));
    }
  }
  // vectors past the end become all-ones words: NaN in every element, below
  // every logit as a signed integer and never at or above a bound.  Apart
  // from load, so that the work between them does not wait for the row.
  __device__ __forceinline__ void past_end(int V) {
#pragma unroll
    for (int j = 0; j < NVR; j++)
      if (vec_id(j) >= V) raw[j] = make_uint4(~0u, ~0u, ~0u, ~0u);
  }
  // a masked-out element becomes the all-ones pattern (as past the row end)
  __device__ __forceinline__ void apply_mask(const Row& r, int V) {
#pragma unroll
    for (int j = 0; j < NVR; j++) {
      const int v = vec_id(j);
      const uint32_t bits = (r.mrow[(v < V ? v : V - 1) >> 5] >> (v & 31)) & ((1u << EPV) - 1u);
      uint32_t wd[4] = {raw[j].x, raw[j].y, raw[j].z, raw[j].w};
#pragma unroll
      for (int w = 0; w < 4; w++) {
        if constexpr (EPV == 8) {
          const uint32_t lo = ((bits >> (2 * w)) & 1u) ? 0u : 0x0000FFFFu;
          const uint32_t hi = ((bits >> (2 * w + 1)) & 1u) ? 0u : 0xFFFF0000u;
          wd[w] |= lo | hi;
        } else {
          wd[w] |= ((bits >> w) & 1u) ? 0u : 0xFFFFFFFFu;
        }
      }
      raw[j] = make_uint4(wd[0], wd[1], wd[2], wd[3]);
    }
  }
};

__device__ __forceinline__ bool hist_bit(const uint32_t* hbits, int id) { return (hbits[id >> 5] >> (id & 31)) & 1u; }

// Canonical logit of a (non-history) id from its raw logit: y = z / T when
// allowed, else the composite 0.
__device__ __forceinline__ u64 comp_of(float z, bool allowed, const Row& r, int id) {
  const float y = row_y(r, z);
  return (allowed && y > -__builtin_inff()) ? comp_key(tg_key(y), id) : 0ull;
}

__device__ __forceinline__ float nan_to_ninf(float x) { return x == x ? x : -__builtin_inff(); }

// Four slot values of this thread: the largest logit of each of four
// disjoint groups of its ids, from signed-integer maxima and minima of the
// raw patterns (a group with a non-negative logit: its largest pattern; an
// all-negative group: its smallest pattern, the negative logit nearest 0).
// A NaN pattern there (NaN logits, masked-out ids, vectors past the end hold
// all-ones) gives -inf: still at most the group's largest logit.
template <typename Tin, int NVR>
__device__ __forceinline__ void slot_values(const Regs<Tin, NVR>& g, float (&s)[4]) {
  if constexpr (sizeof(Tin) == 2) {
    uint32_t hi[2] = {0x80008000u, 0x80008000u}, lo[2] = {0x7FFF7FFFu, 0x7FFF7FFFu};
#pragma unroll
    for (int j = 0; j < NVR; j++)
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const int h = (j * 2) / NVR;
        hi[h] = pk_max_i16(hi[h], word_of(g.raw[j], w));
        lo[h] = pk_min_i16(lo[h], word_of(g.raw[j], w));
      }
#pragma unroll
    for (int h = 0; h < 2; h++) {
      const uint32_t b0 = (hi[h] & 0x8000u) ? (lo[h] & 0xFFFFu) : (hi[h] & 0xFFFFu);
      const uint32_t b1 = (hi[h] & 0x80000000u) ? (lo[h] >> 16) : (hi[h] >> 16);
      s[2 * h] = nan_to_ninf(tg_u2f(b0 << 16));
      s[2 * h + 1] = nan_to_ninf(tg_u2f(b1 << 16));
    }
  } else {
    int hi[4], lo[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      hi[i] = (int)0x80000000u;
      lo[i] = 0x7FFFFFFF;
    }
#pragma unroll
    for (int j = 0; j < NVR; j++)
#pragma unroll
      for (int w = 0; w < 4; w++) {
        const int i = (j * 4) / NVR;
        const int x = (int)word_of(g.raw[j], w);
        hi[i] = x > hi[i] ? x : hi[i];
        lo[i] = x < lo[i] ? x : lo[i];
      }
#pragma unroll
    for (int i = 0; i < 4; i++) s[i] = nan_to_ninf(tg_u2f((uint32_t)(hi[i] >= 0 ? hi[i] : lo[i])));
  }
}

// 16-bit key prefix T16 with at least kp slots whose key >> 16 is >= T16
// (kp <= 4 * BT).  One histogram of each slot's distance (in 16-bit key
// steps) below the largest slot, bins 0..254 exact, 255 for the rest; a
// radix selection restricted to that last bin when the k'-th lies there.
__device__ __forceinline__ uint32_t bound_key16(const float (&s)[4], unsigned kp, Scratch& ts, BlockScratch& bs) {
  uint32_t k16[4];
#pragma unroll
  for (int i = 0; i < 4; i++) k16[i] = tg_key(s[i]) >> 16;
  uint32_t mx = k16[0];
#pragma unroll
  for (int i = 1; i < 4; i++) mx = k16[i] > mx ? k16[i] : mx;
  mx = wave_max(mx);
  if (lane_id() == 0) ts.red32[threadIdx.x >> 6] = mx;
  if (threadIdx.x < 256) bs.hc[threadIdx.x] = 0;
  __syncthreads();
  uint32_t K0 = ts.red32[0];
#pragma unroll
  for (int i = 1; i < WT; i++) K0 = ts.red32[i] > K0 ? ts.red32[i] : K0;
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const uint32_t d = K0 - k16[i];
    atomicAdd(&bs.hc[d < 255u ? d : 255u], 1u);
  }
  __syncthreads();
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    unsigned cs[4];
#pragma unroll
    for (int j = 0; j < 4; j++) cs[j] = bs.hc[4 * lane + j];
    const unsigned lsum = cs[0] + cs[1] + cs[2] + cs[3];
    unsigned cum = wave_incl_scan(lsum) - lsum;
    int found = -1;
    unsigned above = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      if (found < 0 && cs[j] > 0 && cum + cs[j] >= kp) {
        found = 4 * lane + j;
        above = cum;
      }
      cum += cs[j];
    }
    const u64 bal = __ballot(found >= 0);
    const int first = bal ? __ffsll((long long)bal) - 1 : 0;
    const int fd = __shfl(found, first, 64);
    const unsigned fa = __shfl(above, first, 64);
    if (lane == 0) {
      ts.dsel = fd;
      ts.need = kp - fa;
    }
  }
  __syncthreads();
  const int d = ts.dsel;
  const unsigned need = ts.need;
  if (d < 255) return K0 - (uint32_t)d;
  return block_select_kth<uint32_t, 16, BT>(
      [&](auto f) {
#pragma unroll
        for (int i = 0; i < 4; i++)
          if (K0 - k16[i] >= 255u) f(k16[i]);
      },
      need, bs);
}

__device__ __forceinline__ void finish_greedy(const SampleArgs& a, int b, u64 best) {
  const int id = best ? comp_id(best) : -1;
  if (threadIdx.x == 0) {
    a.out[b] = id;
    write_row_diag(a, b, id >= 0, id >= 0, 0, 0, id);
  }
  if (a.dbg.kept_ids) {
    int32_t* kid = a.dbg.kept_ids + (long long)b * a.dbg.kept_cap;
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) kid[i] = (i == 0) ? id : -1;
  }
  if (a.dbg.kept_probs) {
    float* kp = a.dbg.kept_probs + (long long)b * a.dbg.kept_cap;
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) kp[i] = (i == 0 && id >= 0) ? 1.0f : 0.0f;
  }
}

// Block bitonic sort, descending, of BT values, one per thread (thread i
// holds element i).  Partners within a wave move through lane permutes,
// wider strides through LDS (buf: BT entries).  Every thread calls it.
__device__ __forceinline__ u64 block_sort_desc(u64 x, u64* buf) {
  const int i = threadIdx.x;
#pragma unroll 1
  for (int k = 2; k <= BT; k <<= 1) {
#pragma unroll 1
    for (int j = k >> 1; j > 0; j >>= 1) {
      u64 y;
      if (j >= 64) {
        buf[i] = x;
        __syncthreads();
        y = buf[i ^ j];
        __syncthreads();
      } else {
        y = xor_lane_s(x, j);
      }
      const bool keep_max = ((i & j) == 0) == ((i & k) == 0);
      x = keep_max ? (y > x ? y : x) : (y < x ? y : x);
    }
  }
  return x;
}

// The candidates of one row, four per thread, and their buckets.
struct Cands {
  u64 c[CPT];
  int bk[CPT];  // -1: no candidate
};

// Ranks the members of bucket bq (n of them, n uniform) into R / Q (see
// bucket::rank_list).  Returns false (nothing ranked) when n > LCAP.
// ts.ng is 0 on entry and on return.
__device__ __forceinline__ bool rank_bucket(const Cands& cd, int bq, unsigned n, float m, u64* L, u64* R, u64* Q,
                                            Scratch& ts) {
  if (n > (unsigned)LCAP) return false;
  if (threadIdx.x == 0 && (n & 1)) L[n] = 0ull;  // pad below every composite
#pragma unroll
  for (int j = 0; j < CPT; j++)
    if (cd.bk[j] == bq) L[atomicAdd(&ts.ng, 1u)] = cd.c[j];
  __syncthreads();
  if (threadIdx.x == 0) ts.ng = 0;  // read again only after rank_list's barriers
  bucket::rank_list<BT>(L, n, m, R, Q, ts.red64b);
  return true;
}

// The row's tail over nc candidates in cand[] (composites, 0 = none).
template <bool DIAG>
__device__ __forceinline__ void tail(const SampleArgs& a, const Row& r, int nc, u64* cand, u64* L, u64* R, u64* Q,
                                     unsigned* CI, u64* MI, Scratch& ts, BlockScratch& bs) {
  const int b = r.b;
  const int k = r.mode == 0 ? 1 : r.k;
  const int lane = lane_id(), w = threadIdx.x >> 6;
  Cands cd;
  u64 mx = 0;
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    const int i = threadIdx.x + j * BT;
    cd.c[j] = i < nc ? cand[i] : 0ull;
    mx = cd.c[j] > mx ? cd.c[j] : mx;
  }
  mx = wave_max(mx);
  if (lane == 0) ts.red64[w] = mx;
  __syncthreads();
  if (threadIdx.x == 0) {
    ts.ng = 0;  // every thread has read the candidate count
    ts.ng2 = 0;
  }
  u64* L2 = MI + NB + 1;  // the draw's bucket when gathered with the cut's: 64 (+ pad)
  u64* R2 = L2 + 66;      // 64
  u64* Q2 = R2 + 64;      // 64
  u64 M = ts.red64[0];
#pragma unroll
  for (int i = 1; i < WT; i++) M = ts.red64[i] > M ? ts.red64[i] : M;
  if (r.mode == 0) {  // greedy: the largest composite
    finish_greedy(a, b, M);
    return;
  }
  if (M == 0ull) {  // no allowed id
    if (threadIdx.x == 0) {
      a.out[b] = -1;
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    if (a.dbg.kept_ids)
      for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) a.dbg.kept_ids[(long long)b * a.dbg.kept_cap + i] = -1;
    if (a.dbg.kept_probs)
      for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) a.dbg.kept_probs[(long long)b * a.dbg.kept_cap + i] = 0.0f;
    return;
  }
  const float m = comp_y(M);

  // count and mass histogram over the buckets (CI, MI cleared by the caller)
#pragma unroll
  for (int j = 0; j < CPT; j++) {
    cd.bk[j] = -1;
    if (cd.c[j]) {
      const int bq = bucket::of(comp_y(cd.c[j]), m);
      cd.bk[j] = bq;
      atomicAdd(&CI[bq], 1u);
      if (bq < NB) {
        const u64 q = bucket::mass_c(cd.c[j], m);
        if (q) atomicAdd(&MI[bq], q);
      }
    }
  }
  __syncthreads();
  bucket::prefix<BT>(CI, MI, ts.red32, ts.red64);
  auto cex = [&](int bq) -> unsigned { return bq ? CI[bq - 1] : 0u; };
  auto mex = [&](int bq) -> u64 { return bq ? MI[bq - 1] : 0ull; };
  // the bucket whose inclusive count (mass) first reaches target
  auto find_count = [&](unsigned target, int slot) -> int { return bucket::find_count<BT>(CI, target, &ts.sel[slot]); };
  auto find_mass = [&](u64 target, int slot) -> int { return bucket::find_mass<BT>(MI, target, &ts.sel[slot]); };
  // the ranked bucket (-1: none) and its size
  int rb = -1;
  unsigned rn = 0;
  auto ensure_ranked = [&](int bq) -> bool {
    if (rb == bq) return true;
    const unsigned n = CI[bq] - cex(bq);
    if (!rank_bucket(cd, bq, n, m, L, R, Q, ts)) return false;
    rb = bq;
    rn = n;
    return true;
  };
  // element of bucket bq whose within-bucket inclusive prefix first reaches
  // target (>= 1): its composite, the mass ahead of it in the bucket, its rank
  auto resolve_mass = [&](int bq, u64 target, u64* before, unsigned* rank) -> u64 {
    if (ensure_ranked(bq)) {
      const int i = bucket::first_rank<BT>(Q, rn, target, &ts.first);
      *before = i > 0 ? Q[i - 1] : 0ull;
      *rank = (unsigned)i;
      return R[i];
    }
    auto en = [&](auto f) {
#pragma unroll
      for (int j = 0; j < CPT; j++)
        if (cd.bk[j] == bq) f(cd.c[j], bucket::mass_c(cd.c[j], m));
    };
    return block_mass_select<BT>(en, target, bs, before, rank);
  };
  // the rr-th largest member of bucket bq (1-based) and the mass of the rr
  // largest
  auto resolve_count = [&](int bq, unsigned rr, u64* mass) -> u64 {
    if (ensure_ranked(bq)) {
      *mass = Q[rr - 1];
      return R[rr - 1];
    }
    auto en = [&](auto f) {
#pragma unroll
      for (int j = 0; j < CPT; j++)
        if (cd.bk[j] == bq) f(cd.c[j]);
    };
    const u64 T = block_select_kth<u64, 64, BT>(en, rr, bs);
    u64 lo = ~0ull, ms = 0;
#pragma unroll
    for (int j = 0; j < CPT; j++)
      if (cd.bk[j] == bq && cd.c[j] >= T) {
        lo = cd.c[j] < lo ? cd.c[j] : lo;
        ms += bucket::mass_c(cd.c[j], m);
      }
    lo = ~wave_max(~lo);
    ms = wave_sum(ms);
    if (lane == 0) {
      ts.red64[w] = lo;
      ts.red64b[w] = ms;
    }
    __syncthreads();
    u64 x = ~0ull, s = 0;
    for (int v = 0; v < WT; v++) {
      x = ts.red64[v] < x ? ts.red64[v] : x;
      s += ts.red64b[v];
    }
    __syncthreads();
    *mass = s;
    return x;
  };

  // top-k: the bucket of the k-th composite and the kept mass S
  const unsigned nz = CI[NB];
  const unsigned nk = (unsigned)k < nz ? (unsigned)k : nz;
  const int bk = find_count(nk, 0);
  const unsigned rr = nk - cex(bk);  // kept members of bucket bk (its largest)
  const unsigned nbk = CI[bk] - cex(bk);
  u64 S;
  u64 lastc = 0;  // smallest kept composite, when known
  if (bk == NB) {
    S = MI[NB - 1];
  } else if (rr == nbk) {
    S = MI[bk];
  } else {
    u64 mb;
    lastc = resolve_count(bk, rr, &mb);
    S = mex(bk) + mb;
  }
  // top-p: the cut, the first element whose inclusive prefix reaches P
  const uint32_t uq = (uint32_t)(r.u * 16777216.0f);
  unsigned istar;
  u64 Sp, cutc = 0, pick = 0;
  bool drawn = false;  // the draw resolved with the cut
  if (r.top_p < 1.0f) {
    const uint32_t pq = (uint32_t)(r.top_p * 16777216.0f);
    const u64 P = mul_shr24(S, pq);
    if (P == 0) {
      istar = 0;
      cutc = M;
      Sp = tg_q40(1.0f);
    } else {
      // The draw's bucket while the cut is open: S' lies in [P, MI[bp]] (the
      // cut's inclusive prefix reaches P and ends in bucket bp), so t lies in
      // [floor(P u24 / 2^24), floor(MI[bp] u24 / 2^24)]; when one bucket holds
      // every draw target of that range, the cut's and the draw's buckets are
      // gathered in one pass over the candidates and ranked side by side.
      const u64 tlo = mul_shr24(P, uq);
      bucket::find_mass2<BT>(MI, P, tlo + 1, &ts.sel[1], &ts.sel[2]);
      const int bp = ts.sel[1], btl = ts.sel[2];
      const unsigned na = CI[bp] - cex(bp);
      const unsigned nb2 = btl != bp ? CI[btl] - cex(btl) : 0u;
      const bool one = MI[btl] >= mul_shr24(MI[bp], uq) + 1 && nb2 <= 64u && (rb == bp || na <= (unsigned)LCAP);
      if (one) {
        const bool gather_a = rb != bp;  // the cut's bucket not ranked yet
        const int bb = btl != bp ? btl : -1;
        if (gather_a && threadIdx.x == 0 && (na & 1)) L[na] = 0ull;  // pad below every composite
#pragma unroll
        for (int j = 0; j < CPT; j++) {
          if (gather_a && cd.bk[j] == bp) L[atomicAdd(&ts.ng, 1u)] = cd.c[j];
          else if (bb >= 0 && cd.bk[j] == bb) L2[atomicAdd(&ts.ng2, 1u)] = cd.c[j];  // (bk -1: no candidate)
        }
        __syncthreads();
        if (threadIdx.x == 0) {
          ts.ng = 0;  // read again only after the barriers below
          ts.ng2 = 0;
        }
        if (bb >= 0 && w == 1) bucket::wave_rank64(L2, nb2, m, R2, Q2);
        if (gather_a) {
          bucket::rank_list<BT>(L, na, m, R, Q, ts.red64b);  // ends with a barrier
          rb = bp;
          rn = na;
        } else {
          __syncthreads();
        }
        const int i = bucket::first_rank_once(Q, rn, P - mex(bp), &ts.first);
        cutc = R[i];
        istar = cex(bp) + (unsigned)i;
        Sp = mex(bp) + (i > 0 ? Q[i - 1] : 0ull) + bucket::mass_c(cutc, m);
        const u64 tb = mul_shr24(Sp, uq) + 1 - mex(btl);
        pick = bb >= 0 ? R2[bucket::first_rank_once(Q2, nb2, tb, &ts.first2)]
                       : R[bucket::first_rank_once(Q, rn, tb, &ts.first2)];
        drawn = true;
      } else {
        u64 before;
        unsigned rank;
        cutc = resolve_mass(bp, P - mex(bp), &before, &rank);
        istar = cex(bp) + rank;
        Sp = mex(bp) + before + bucket::mass_c(cutc, m);
      }
    }
  } else {
    istar = nk - 1;
    Sp = S;
    if (DIAG) {
      if (lastc == 0) {
        u64 mb;
        lastc = resolve_count(bk, rr, &mb);
      }
      cutc = lastc;
    }
  }
  // the draw: the first element whose inclusive prefix exceeds t
  if (!drawn) {
    const u64 t = mul_shr24(Sp, uq);
    const int bt = find_mass(t + 1, 2);
    u64 before;
    unsigned rank;
    pick = resolve_mass(bt, t + 1 - mex(bt), &before, &rank);
  }
  if (threadIdx.x == 0) {
    a.out[b] = comp_id(pick);
    write_row_diag(a, b, (int)nk, (int)istar + 1, S, Sp, comp_id(cutc));
  }
  if (a.dbg.kept_ids || a.dbg.kept_probs) {
    // the kept set in order (diagnostics only): the exact k-th composite,
    // the composites at or above it, a bitonic sort
    u64 Tk = 1;
    if (nz > (unsigned)k)
      Tk = block_select_kth<u64, 64, BT>(
          [&](auto f) {
#pragma unroll
            for (int j = 0; j < CPT; j++)
              if (cd.c[j]) f(cd.c[j]);
          },
          (unsigned)k, bs);
    if (threadIdx.x == 0) ts.nc = 0;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < CPT; j++)
      if (cd.c[j] && cd.c[j] >= Tk) cand[atomicAdd(&ts.nc, 1u)] = cd.c[j];
    __syncthreads();
    u64 x = (int)threadIdx.x < (int)nk ? cand[threadIdx.x] : 0ull;
    __syncthreads();
    x = block_sort_desc(x, cand);
    cand[threadIdx.x] = x;
    __syncthreads();
    if (a.dbg.kept_ids) {
      int32_t* kid = a.dbg.kept_ids + (long long)b * a.dbg.kept_cap;
      for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) kid[i] = i < (int)nk ? comp_id(cand[i]) : -1;
    }
    if (a.dbg.kept_probs) {
      float* kp = a.dbg.kept_probs + (long long)b * a.dbg.kept_cap;
      const float fs = tg_u64_to_f32(Sp);
      for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT)
        kp[i] = i <= (int)istar ? kept_prob(comp_y(cand[i]), m, fs) : 0.0f;
    }
  }
}

template <typename Tin, int NVR, bool MASK>
__device__ __forceinline__ void topk_row(const SampleArgs& a, Row& r, unsigned char* smem, Scratch& ts,
                                         BlockScratch& bs, Regs<Tin, NVR>& g, const int (&hpre)[1]) {
  using RG = Regs<Tin, NVR>;
  constexpr int EPV = RG::EPV;
  const int b = r.b;
  const int V = a.V;
  const int bw = a.TS > 0 ? (V + 31) / 32 : 0;
  uint32_t* hbits = (uint32_t*)smem;
  int2* hash = (int2*)(smem + ((bw * 4 + 15) / 16) * 16);
  u64* cand = (u64*)((unsigned char*)hash + (size_t)a.TS * 8);  // CAPK
  u64* L = cand + CAPK;                                           // LCAP (+ pad)
  u64* R = L + LCAP + 2;                                          // LCAP
  u64* Q = R + LCAP;                                              // LCAP
  unsigned* CI = (unsigned*)(Q + LCAP);                           // NB + 1 (+ pad)
  u64* MI = (u64*)(CI + NB + 4);                                  // NB + 1
  uint32_t* cid = (uint32_t*)L;                                   // CAPK ids, over L and R
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  const int k = r.mode == 0 ? 1 : r.k;

  // the row's vectors (g) and history entries (hpre) were requested at entry
  // history: id -> count hash and the row's bitmap; distinct ids
  r.v0 = 0;
  r.v1 = V;
  unsigned nh = 0;
  if (r.use_pen) {
    hash_build_pre<BT, 1>(a, r, hpre, hash, hbits, bw);
    unsigned c = 0;
    for (int i = threadIdx.x; i < a.TS; i += BT) c += hash[i].x != -1;
    nh = bsum(c, ts.red32);
  }
  g.past_end(V);
  if (MASK && r.mrow != nullptr) g.apply_mask(r, V);

  // bound
  float s[4];
  slot_values<Tin, NVR>(g, s);
  const unsigned kp = (unsigned)k + nh;  // <= 2 * KMAX (top_k and history capped at KMAX)
  const uint32_t tkey = bound_key16(s, kp, ts, bs) << 16;
  // raw-logit bound, 16 representable values lower: a raw logit below it
  // scales (x / T, correctly rounded and monotone) strictly below the
  // scaled bound, also across a binade edge
  const uint32_t kneg = 0x007FFFFFu;  // key of -inf
  const float thz = tkey > kneg + 16u ? tg_unkey(tkey - 16u) : -__builtin_inff();
  const float thf = fmaxf(thz, -3.40282347e38f);  // -inf never qualifies

  // collect: the vectors holding an id at or above the bound (bit j of vb:
  // this thread's vector j), from packed maxima of the patterns held in
  // registers; the per-id test runs afterwards on those vectors only, read
  // again from memory.  bf16 x >= thf exactly on the 16-bit patterns: for
  // thf > 0 a signed compare with ceil(thf bits / 2^16); otherwise (sign
  // set, or +0) an unsigned compare with the truncated pattern (every
  // non-negative pattern lies below it).  Masked-out ids and ids past the
  // row end hold the all-ones pattern and never pass.
  const uint32_t tb = tg_f2u(thf);
  const bool pos = !(tb >> 31) && tb != 0u;
  const int ts16 = (int)((tb + 0xFFFFu) >> 16);
  const uint32_t tu16 = tb == 0u ? 0x8000u : (tb >> 16);
  auto id_passes = [&](uint32_t w, int e) -> bool {  // element e of a vector word w (its word e / (EPV / 4))
    if constexpr (sizeof(Tin) == 2) {
      const uint32_t h = (e & 1) ? (w >> 16) : (w & 0xFFFFu);
      return pos ? ((int)(short)h >= ts16) : (h <= tu16);
    } else {
      return tg_u2f(w) >= thf;
    }
  };
  uint32_t vb = 0;
  if constexpr (sizeof(Tin) == 2) {
    if (pos) {
#pragma unroll
      for (int j = 0; j < NVR; j++) {
        const uint4 v = g.raw[j];
        const uint32_t mx = pk_max_i16(pk_max_i16(v.x, v.y), pk_max_i16(v.z, v.w));
        const int lo = (int)(short)(mx & 0xFFFFu), hi = (int)mx >> 16;
        vb |= ((hi > lo ? hi : lo) >= ts16 ? 1u : 0u) << j;
      }
    } else {
      // per-half unsigned minima: signed minima of the patterns with their
      // top bits flipped
      constexpr uint32_t F = 0x80008000u;
#pragma unroll
      for (int j = 0; j < NVR; j++) {
        const uint4 v = g.raw[j];
        const uint32_t mn = pk_min_i16(pk_min_i16(v.x ^ F, v.y ^ F), pk_min_i16(v.z ^ F, v.w ^ F)) ^ F;
        const uint32_t lo = mn & 0xFFFFu, hi = mn >> 16;
        vb |= ((lo < hi ? lo : hi) <= tu16 ? 1u : 0u) << j;
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < NVR; j++) {
      const uint4 v = g.raw[j];
      const bool p = tg_u2f(v.x) >= thf || tg_u2f(v.y) >= thf || tg_u2f(v.z) >= thf || tg_u2f(v.w) >= thf;
      vb |= (p ? 1u : 0u) << j;
    }
  }
  const unsigned cnt = (unsigned)__builtin_popcount(vb);
  if (threadIdx.x == 0) {
    ts.nc = 0;
    ts.ng = 0;
    ts.na = 0;
  }
  for (int i = threadIdx.x; i < NB + 1; i += BT) {
    CI[i] = 0u;
    MI[i] = 0ull;
  }
  __syncthreads();
  {
    // the vectors' indexes in the row, in cid
    const unsigned wincl = wave_incl_scan(cnt);
    unsigned wbase = 0;
    if (lane_id() == 63 && wincl) wbase = atomicAdd(&ts.nc, wincl);
    wbase = __shfl(wbase, 63, 64);
    unsigned slot = wbase + wincl - cnt;
    uint32_t m = vb;
    while (m) {
      const int j = __builtin_ctz(m);
      m &= m - 1u;
      if (slot < (unsigned)CAPK) cid[slot] = (uint32_t)((int)threadIdx.x + j * BT);
      slot++;
    }
  }
  __syncthreads();
  const unsigned ncv = ts.nc;  // vectors holding an id at or above the bound
  unsigned ncb = (unsigned)CAPK + 1u;  // candidates in cand[0, ncb) (beyond CAPK: overflow)
  if (ncv <= (unsigned)CAPK) {
    // each vector read again from memory (with its mask word); its ids that
    // pass (history ids: composite 0, added below with their penalised
    // logits) into cand by a wave-aggregated append
#pragma unroll
    for (int q = 0; q < CPT; q++) {
      if (q * BT >= (int)ncv) break;  // (uniform)
      const int i = (int)threadIdx.x + q * BT;
      const bool act = i < (int)ncv;
      const int vid = act ? (int)cid[i] * EPV : 0;
      const uint4 v = *(const uint4*)(rowp + vid);
      const uint32_t mw = (MASK && r.mrow != nullptr) ? r.mrow[vid >> 5] >> (vid & 31) : 0xFFFFFFFFu;
      uint32_t on = 0;
#pragma unroll
      for (int e = 0; e < EPV; e++)
        on |= (act && ((mw >> e) & 1u) && id_passes(word_of(v, e / (EPV / 4)), e) ? 1u : 0u) << e;
      const unsigned c = (unsigned)__builtin_popcount(on);
      const unsigned incl = wave_incl_scan(c);
      const unsigned tot = readlane_u32(incl, 63);
      unsigned base = 0;
      if (lane_id() == 63 && tot) base = atomicAdd(&ts.na, tot);
      unsigned sl = readlane_u32(base, 63) + incl - c;
      while (on) {
        const int e = __builtin_ctz(on);
        on &= on - 1u;
        const int id = vid + e;
        const u64 x = (r.use_pen && hist_bit(hbits, id)) ? 0ull : comp_of(Elem<Tin>::get(v, e), true, r, id);
        if (sl < (unsigned)CAPK) cand[sl] = x;
        sl++;
      }
    }
    __syncthreads();
    ncb = ts.na;
  }
  if (ncb <= (unsigned)CAPK) {
    if (r.use_pen) {
      for (int i = threadIdx.x; i < a.TS; i += BT) {
        const int2 h = hash[i];
        if (h.x == -1) continue;
        const int hid = h.x;
        const float z = penalise(Elem<Tin>::scalar(rowp, hid), h.y, r);
        const u64 c = comp_of(z, mask_allows(r, hid), r, hid);
        if (c) {
          const unsigned sl = ncb + atomicAdd(&ts.ng, 1u);
          if (sl < (unsigned)CAPK) cand[sl] = c;
        }
      }
    }
  }
  __syncthreads();
  int nc = (int)(ncb + ts.ng);  // ts.ng is cleared in the tail, past its first barrier
  if (nc > CAPK) {
    // candidate overflow: radix selection over every id of the row, read
    // again from L2 / MALL (rare: massive ties at the bound); the kept set
    // becomes the candidate list
    auto en = [&](auto f) {
      const int nvec = (V + EPV - 1) / EPV;
#pragma unroll 1
      for (int vi = threadIdx.x; vi < nvec; vi += BT) {
        const uint4 raw = load_vec<Tin>(rowp, vi * EPV, V, a.aligned);
#pragma unroll
        for (int e = 0; e < EPV; e++) {
          const int id = vi * EPV + e;
          if (id >= V) continue;
          float z = Elem<Tin>::get(raw, e);
          if (r.use_pen && hist_bit(hbits, id)) z = penalise(z, hash_count(hash, a.TS, a.ts_shift, id), r);
          const u64 c = comp_of(z, mask_allows(r, id), r, id);
          if (c) f(c);
        }
      }
    };
    unsigned na = 0;
    en([&](u64) { na++; });
    na = bsum(na, ts.red32);
    u64 T = 1;
    if ((int)na > k) T = block_select_kth<u64, 64, BT>(en, (unsigned)k, bs);
    if (threadIdx.x == 0) ts.nc = 0;
    __syncthreads();
    en([&](u64 c) {
      if (c >= T) cand[atomicAdd(&ts.nc, 1u)] = c;  // at most k (distinct composites)
    });
    __syncthreads();
    nc = (int)ts.nc;
  }
  if (a.dbg.post_logits) {
    float* post = a.dbg.post_logits + (long long)b * V;
    const int nvec = (V + EPV - 1) / EPV;
#pragma unroll 1
    for (int vi = threadIdx.x; vi < nvec; vi += BT) {
      const uint4 raw = load_vec<Tin>(rowp, vi * EPV, V, a.aligned);
#pragma unroll
      for (int e = 0; e < EPV; e++) {
        const int id = vi * EPV + e;
        if (id >= V) continue;
        float z = Elem<Tin>::get(raw, e);
        if (r.use_pen && hist_bit(hbits, id)) z = penalise(z, hash_count(hash, a.TS, a.ts_shift, id), r);
        const float y = row_y(r, z);
        post[id] = (mask_allows(r, id) && y > -__builtin_inff()) ? y : -__builtin_inff();
      }
    }
  }
  if (a.dbg.cut_ids) tail<true>(a, r, nc, cand, L, R, Q, CI, MI, ts, bs);
  else tail<false>(a, r, nc, cand, L, R, Q, CI, MI, ts, bs);
}

template <typename Tin, int NVR, bool MASK>
__global__ __launch_bounds__(BT) void topk_kernel(SampleArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ Scratch ts;
  __shared__ BlockScratch bs;
  const int b = blockIdx.x;
  if (b >= a.B) return;
  // everything requested first, in the order it is needed (a wave's loads
  // return in order): the row's parameters (scalar loads), its history
  // entries (one per thread: the history is at most KMAX ids), its vectors
  const tgs_row_params p = a.params[b];
  const float ub = a.u[b];
  const int hl = a.hist_len ? a.hist_len[b] : a.hist_cap;
  int hid[1];
  hist_prefetch<BT, 1>(a, b, hid);
  Regs<Tin, NVR> g;
  g.load((const Tin*)a.logits + (long long)b * a.row_stride, a.V);
  Row r;
  const bool valid = row_setup_from(a, b, 0, p, ub, hl, r);
  if (!valid || outside_hint(a, r) || r.mode == 2) {
    if (threadIdx.x == 0) {
      a.out[b] = valid ? -3 : -2;  // -3: row outside the launch hint
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    return;
  }
  topk_row<Tin, NVR, MASK>(a, r, smem, ts, bs, g, hid);
}

template <typename Tin, int NVR>
hipError_t launch_nvr(const SampleArgs& a, size_t lds, hipStream_t st) {
  const bool mask = a.mask_table != nullptr && a.n_states > 0;
  if (mask) hipLaunchKernelGGL((topk_kernel<Tin, NVR, true>), dim3(a.B), dim3(BT), lds, st, a);
  else hipLaunchKernelGGL((topk_kernel<Tin, NVR, false>), dim3(a.B), dim3(BT), lds, st, a);
  return hipGetLastError();
}

template <typename Tin>
hipError_t launch_t(const SampleArgs& a, size_t lds, hipStream_t st) {
  constexpr int EPV = Elem<Tin>::EPV;
  const int nvr = (a.V + BT * EPV - 1) / (BT * EPV);
  if (nvr <= 8) return launch_nvr<Tin, 8>(a, lds, st);
  return launch_nvr<Tin, 20>(a, lds, st);
}

template <typename Tin, int NVR>
void collect_fns(const void** f) {
  f[0] = (const void*)topk_kernel<Tin, NVR, true>;
  f[1] = (const void*)topk_kernel<Tin, NVR, false>;
}

}  // namespace topk

int topk_max_vocab(int dtype) { return topk::BT * 20 * (dtype == 1 ? 8 : 4); }

size_t topk_lds_bytes(int V, int TS) {
  const int bw = TS > 0 ? (V + 31) / 32 : 0;
  return (size_t)((bw * 4 + 15) / 16) * 16 + (size_t)TS * 8 + (size_t)(TOPK_CAP + 3 * topk::LCAP + 2) * 8 +
         (size_t)(topk::NB + 4) * 4 + (size_t)(topk::NB + 1) * 8 + (size_t)(66 + 64 + 64) * 8;
}

hipError_t launch_topk(const SampleArgs& a, int dtype, size_t lds, hipStream_t st) {
  return dtype == 1 ? topk::launch_t<uint16_t>(a, lds, st) : topk::launch_t<float>(a, lds, st);
}

hipError_t set_topk_lds_limit(size_t bytes) {
  const void* fns[8];
  topk::collect_fns<float, 8>(fns + 0);
  topk::collect_fns<float, 20>(fns + 2);
  topk::collect_fns<uint16_t, 8>(fns + 4);
  topk::collect_fns<uint16_t, 20>(fns + 6);
  hipError_t e = hipSuccess;
  for (const void* f : fns) {
    hipError_t e2 = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e2 != hipSuccess) e = e2;
  }
  return e;
}

}  // namespace tgs
