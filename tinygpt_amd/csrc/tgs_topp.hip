// tgs_topp.hip -- rows that sample with top-p over the whole vocabulary (top_k
// disabled: k <= 0 or k >= V), one workgroup of 1024 threads per row; in a
// launch that serves the whole batch (every sampling row without a top-k),
// the greedy rows too.
//
// The contract keeps the smallest prefix of the allowed ids in (y desc,
// id asc) order whose exact mass reaches P = floor(S p24 / 2^24) and draws
// the first id whose inclusive prefix exceeds t = floor(S' u24 / 2^24);
// masses are q = floor(exp(y - m) 2^40).  Only ids with q > 0 can be the cut
// or the draw (both are where the prefix grows), and those lie within 32 of
// the maximum.  So:
//
//   pass 1  y (mask, penalties, 1/T): the largest composite (its y is the
//           maximum m; it is the answer of a greedy row) and the allowed
//           count;
//   pass 2  per allowed id its bucket below m (width 1/32, tgs_bucket.h)
//           and mass q, into a count and mass histogram; block prefixes
//           over the buckets locate the bucket of the cut and then of the
//           draw;
//   pass 3  gather that bucket's ids (composites) into LDS, rank them (a
//           wave sort for at most 64), scan their masses in rank order and
//           pick the element.  The draw's bucket is known before the cut is
//           resolved whenever every S' the cut can leave draws from one
//           bucket (nearly always: S' lies in the cut's bucket); then one
//           gather collects both buckets and two waves rank them side by
//           side.  Otherwise the cut is resolved first and the draw's
//           bucket gathered after it.
//
// A row of at most 32768 ids is held in registers (32 per thread) after one
// read; a longer row is streamed again from L2 / MALL by every pass.
//
// A bucket of more than CAPG ids (a flat row: ties, tiny temperature
// spreads) is resolved by a mass-weighted radix selection restricted to the
// bucket instead (a few more passes).  exp runs once per id (plus once per
// ranked id).
#include "tgs_bucket.h"
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace topp {

constexpr int BT = TOPP_NT;    // threads per workgroup
constexpr int WT = BT / 64;    // waves
constexpr int NB = bucket::NB; // mass buckets below the maximum
constexpr int CAPG = TOPP_CAP; // ids of one bucket ranked in LDS
constexpr int RES_EPT = 32;    // ids per thread kept in registers when the row fits (V <= 32768)

struct Scratch {
  u64 red64[WT];
  u64 red64b[WT];
  unsigned red32[WT];
  unsigned ng;    // gathered ids
  unsigned ng2;   // gathered ids of the draw's bucket (list B)
  int sel[2];     // buckets of the cut and of the draw
  int first;      // first rank meeting a mass target
  int first2;     // the same for the draw, in the one-gather tail
};

// The row's canonical logits: y after penalties and temperature, -inf where
// the id is not allowed (mask bit clear, -inf or NaN).  RES: the row fits in
// registers (RES_EPT ids per thread, loaded once); otherwise every walk
// streams the row again from L2 / MALL.
template <typename Tin, bool RES>
struct RowView {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int NV = RES ? RES_EPT / EPV : 1;  // vectors per thread held
  const SampleArgs& a;
  const Row& r;
  const int2* hash;
  const uint32_t* hbits;
  const Tin* rowp;
  float y[RES ? RES_EPT : 1];
  unsigned nallowed = 0;  // this thread's allowed ids among y (set by load)

  __device__ __forceinline__ RowView(const SampleArgs& a_, const Row& r_, const int2* h_, const uint32_t* hb_,
                                     const Tin* p_)
      : a(a_), r(r_), hash(h_), hbits(hb_), rowp(p_) {}

  // y of the EPV ids of vector v from its loaded bits
  __device__ __forceinline__ void vec_y(int v, const uint4& raw, float (&yv)[EPV]) const {
    const bool in = v < a.V;  // a vector past the row end reads no mask or history word
    const uint32_t mw = !in ? 0u : r.mrow ? r.mrow[v >> 5] : 0xFFFFFFFFu;
    const uint32_t hw = (in && r.use_pen) ? hbits[v >> 5] : 0u;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      const int id = v + e;
      float z = Elem<Tin>::get(raw, e);
      if ((hw >> (id & 31)) & 1u) z = penalise(z, hash_count(hash, a.TS, a.ts_shift, id), r);
      const float yy = row_y(r, z);
      yv[e] = (((mw >> (id & 31)) & 1u) && yy > -__builtin_inff() && id < a.V) ? yy : -__builtin_inff();
    }
  }

  // the row's vectors J0 .. J1 - 1 of this thread.  Rows of whole aligned
  // vectors read every vector with one unconditional load (a vector past
  // the row end reads the last one again; vec_y drops its ids), so no load
  // waits for an earlier one: a divergent fallback beside the loads makes
  // the compiler wait for the loads already issued before reusing their
  // registers.
  template <int J0, int J1>
  __device__ __forceinline__ static void fetch(const SampleArgs& a, const Tin* p, uint4 (&raw)[NV]) {
    if constexpr (RES) {
      if (a.aligned && a.V >= EPV && a.V % EPV == 0) {
        const int last = a.V / EPV - 1;
#pragma unroll
        for (int j = J0; j < J1; j++) {
          const int vi = (int)threadIdx.x + j * BT;
          raw[j] = tg_load_nt(p + (vi < last ? vi : last) * EPV);
        }
      } else {
#pragma unroll
        for (int j = J0; j < J1; j++) raw[j] = load_vec<Tin>(p, (threadIdx.x + j * BT) * EPV, a.V, a.aligned);
      }
    }
  }

  // the mask word of each of this thread's register-resident vectors (all
  // ones without a mask row, 0 past the row end)
  __device__ __forceinline__ static void mask_words(const SampleArgs& a, const Row& r, uint32_t (&mw)[NV]) {
    if constexpr (RES) {
#pragma unroll
      for (int j = 0; j < NV; j++) {
        const int v = ((int)threadIdx.x + j * BT) * EPV;
        mw[j] = v >= a.V ? 0u : r.mrow ? r.mrow[v >> 5] : 0xFFFFFFFFu;
      }
    }
  }

  // y of the register-resident vectors, specialised on what is uniform over
  // the row (penalties present, a power-of-two temperature, T = 1: y = z
  // exactly) so that the per-element code carries no branch or operation for
  // the cases the row does not have
  template <bool PEN, bool POW2, bool ONE = false>
  __device__ __forceinline__ void load_t(const uint4 (&raw)[NV], const uint32_t (&mw)[NV]) {
#pragma unroll
    for (int j = 0; j < NV; j++) {
      const int v = ((int)threadIdx.x + j * BT) * EPV;
      const uint32_t hw = (PEN && v < a.V) ? hbits[v >> 5] : 0u;
#pragma unroll
      for (int e = 0; e < EPV; e++) {
        const int id = v + e;
        float z = Elem<Tin>::get(raw[j], e);
        if constexpr (PEN) {
          if ((hw >> (id & 31)) & 1u) z = penalise(z, hash_count(hash, a.TS, a.ts_shift, id), r);
        }
        // (an id past the row end needs no test: its vector's mask word is
        // 0, or, in a vector that straddles the end, load_vec read it as NaN)
        const float yy = ONE ? z : POW2 ? z * r.rT : row_y(r, z);
        const bool ok = ((mw[j] >> (id & 31)) & 1u) && yy > -__builtin_inff();
        y[j * EPV + e] = ok ? yy : -__builtin_inff();
        nallowed += ok ? 1u : 0u;
      }
    }
  }

  __device__ __forceinline__ void load(const uint4 (&raw)[NV], const uint32_t (&mw)[NV]) {
    if constexpr (RES) {
      if (r.use_pen) load_t<true, false>(raw, mw);
      else if (r.tdiv == TDIV_POW2 && r.rT == 1.0f) load_t<false, true, true>(raw, mw);
      else if (r.tdiv == TDIV_POW2) load_t<false, true>(raw, mw);
      else load_t<false, false>(raw, mw);
    }
  }

  // f(id, y) for every allowed id of the row, read again from L2 / MALL
  // (a rolled loop: no register-held state besides the caller's)
  template <class F>
  __device__ __forceinline__ void each_stream(F f) const {
    const int nvec = (a.V + EPV - 1) / EPV;
#pragma unroll 1
    for (int vi = threadIdx.x; vi < nvec; vi += BT) {
      const int v = vi * EPV;
      const uint4 raw = load_vec<Tin>(rowp, v, a.V, a.aligned);
      float yv[EPV];
      vec_y(v, raw, yv);
#pragma unroll
      for (int e = 0; e < EPV; e++)
        if (yv[e] > -__builtin_inff()) f(v + e, yv[e]);
    }
  }

  // f(id, y) for every allowed id of the row
  template <class F>
  __device__ __forceinline__ void each(F f) const {
    if constexpr (RES) {
#pragma unroll
      for (int j = 0; j < NV; j++)
#pragma unroll
        for (int e = 0; e < EPV; e++) {
          const float yy = y[j * EPV + e];
          if (yy > -__builtin_inff()) f((threadIdx.x + j * BT) * EPV + e, yy);
        }
    } else {
      const int nvec = (a.V + EPV - 1) / EPV;
      for (int vi = threadIdx.x; vi < nvec; vi += BT) {
        const int v = vi * EPV;
        const uint4 raw = load_vec<Tin>(rowp, v, a.V, a.aligned);
        float yv[EPV];
        vec_y(v, raw, yv);
#pragma unroll
        for (int e = 0; e < EPV; e++)
          if (yv[e] > -__builtin_inff()) f(v + e, yv[e]);
      }
    }
  }
};

// One allowed id and its canonical logit, packed in LDS.
struct alignas(8) Packed {
  float y;
  int id;
};

// The allowed ids of a row packed in LDS: E[0, n).
struct CompactView {
  const Packed* E;
  int n;
  template <class F>
  __device__ __forceinline__ void each(F f) const {
#pragma unroll 2
    for (int i = threadIdx.x; i < n; i += BT) {
      const Packed e = E[i];
      f(e.id, e.y);
    }
  }
  template <class F>
  __device__ __forceinline__ void each_stream(F f) const {
    each(f);
  }
};

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

// The row's tail state: the bucket prefixes and the one ranked bucket.
struct Tail {
  unsigned* CI;  // NB + 1 inclusive counts
  u64* MI;       // NB + 1 inclusive masses
  u64 *L, *R, *Q;     // list A: CAPG gathered, ranked, inclusive masses
  u64 *L2, *R2, *Q2;  // list B: the same for at most 64 ids
  Packed* E;     // a.topp_cap packed allowed ids
  float m;
  int rb = -1;   // ranked bucket (-1: none)
  unsigned rn = 0;
};

// The element of bucket bq whose within-bucket inclusive prefix first
// reaches target (>= 1): its composite, the mass ahead of it in the bucket
// and its rank there.  The bucket's members are gathered from the row and
// ranked in LDS (kept for a later call on the same bucket); a bucket of more
// than CAPG ids is resolved by a mass-weighted radix selection over the row
// restricted to it instead.
template <class View>
__device__ __forceinline__ u64 resolve_mass(const View& rv, Tail& tl, int bq, u64 target, u64* before,
                                            unsigned* rank, Scratch& ts, BlockScratch& bs) {
  const float m = tl.m;
  if (tl.rb != bq) {
    const unsigned n = tl.CI[bq] - bucket::count_before(tl.CI, bq);
    if (n <= (unsigned)CAPG) {
      if (threadIdx.x == 0) {
        ts.ng = 0;
        if (n & 1) tl.L[n] = 0ull;  // pad below every composite
      }
      __syncthreads();
      u64* L = tl.L;
      rv.each([&](int id, float y) {
        if (bucket::of(y, m) == bq) L[atomicAdd(&ts.ng, 1u)] = comp_key(tg_key(y), id);
      });
      __syncthreads();
      bucket::rank_list<BT>(tl.L, n, m, tl.R, tl.Q, ts.red64b);
      tl.rb = bq;
      tl.rn = n;
    }
  }
  if (tl.rb == bq) {
    const int i = bucket::first_rank<BT>(tl.Q, tl.rn, target, &ts.first);
    *before = i > 0 ? tl.Q[i - 1] : 0ull;
    *rank = (unsigned)i;
    return tl.R[i];
  }
  auto en = [&](auto f) {
    rv.each_stream([&](int id, float y) {
      if (bucket::of(y, m) == bq) f(comp_key(tg_key(y), id), bucket::mass(y, m));
    });
  };
  return block_mass_select<BT>(en, target, bs, before, rank);
}

// The row after pass 1 (m, the largest composite Mc, nv allowed ids): the
// mass histogram, the cut and the draw over the allowed ids of view v.
template <class View>
__device__ __forceinline__ void topp_rest(const SampleArgs& a, const Row& r, const View& rv, Tail& tl, u64 Mc,
                                          unsigned nv, Scratch& ts, BlockScratch& bs) {
  const int b = r.b;
  const float m = tl.m;
  // pass 2: count and exact-mass histogram over the buckets below m.  With
  // a finite maximum, x = y - m is +-0 exactly at y == m, where bucket 0 and
  // weight 1 follow from x itself (tg_expf_nonpos(+-0) = 1), so the test for
  // y == m that an infinite maximum needs is left out.
  if (m < __builtin_inff()) {
    rv.each([&](int, float y) {
      const float x = y - m;
      const int bq = !(x > -32.0f) ? NB : (int)(-x * 32.0f);
      atomicAdd(&tl.CI[bq], 1u);
      if (bq < NB) {  // -32 < x <= 0
        const u64 q = tg_q40(tg_expf_nonpos_in(x));
        if (q) atomicAdd(&tl.MI[bq], q);
      }
    });
  } else {
    rv.each([&](int, float y) {
      const int bq = bucket::of(y, m);
      atomicAdd(&tl.CI[bq], 1u);
      if (bq < NB) {
        const u64 q = bucket::mass(y, m);
        if (q) atomicAdd(&tl.MI[bq], q);
      }
    });
  }
  __syncthreads();
  bucket::prefix<BT>(tl.CI, tl.MI, ts.red32, ts.red64);
  const u64 S = tl.MI[NB - 1];

  // the cut (top-p): element i* with inclusive prefix >= P
  u64 cutc = 0, Sp = S, P = 0;
  unsigned ntopp = nv;
  bool cut_last = false, cut_search = false;
  if (r.top_p < 1.0f) {
    const uint32_t pq = (uint32_t)(r.top_p * 16777216.0f);
    P = mul_shr24(S, pq);
    if (P == 0) {
      cutc = Mc;
      Sp = tg_q40(1.0f);
      ntopp = 1;
    } else {
      cut_search = true;
    }
  } else {
    cut_last = true;
  }
  // the draw: first element with inclusive prefix > t = floor(S' u24 / 2^24).
  // While the cut is open, S' lies in [P, MI[bp]] (the cut's inclusive
  // prefix reaches P and ends inside bucket bp), so t lies in [tlo, thi];
  // when bucket bt holds every target in [tlo + 1, thi + 1], the cut's and
  // the draw's buckets are gathered in one pass and ranked side by side.
  const uint32_t uq = (uint32_t)(r.u * 16777216.0f);
  const u64 tlo = mul_shr24(cut_search ? P : Sp, uq);
  if (threadIdx.x == 0) {
    ts.ng = 0;
    ts.ng2 = 0;
  }
  bucket::find_mass2<BT>(tl.MI, cut_search ? P : tlo + 1, tlo + 1, &ts.sel[0], &ts.sel[1]);
  const int bp = ts.sel[0], btl = ts.sel[1];
  const int ba = cut_search ? bp : btl;               // list A: the cut's bucket (else the draw's)
  const int bb = (cut_search && btl != bp) ? btl : -1;  // list B: the draw's bucket when it differs
  const unsigned na = tl.CI[ba] - bucket::count_before(tl.CI, ba);
  const unsigned nb2 = bb >= 0 ? tl.CI[bb] - bucket::count_before(tl.CI, bb) : 0u;
  bool one = na <= (unsigned)CAPG && nb2 <= 64u;
  if (cut_search) one = one && tl.MI[btl] >= mul_shr24(tl.MI[bp], uq) + 1;
  u64 pick;
  if (one) {
    if (threadIdx.x == 0 && (na & 1)) tl.L[na] = 0ull;  // pad below every composite
    rv.each([&](int id, float y) {
      const int q = bucket::of(y, m);
      if (q == ba) tl.L[atomicAdd(&ts.ng, 1u)] = comp_key(tg_key(y), id);
      else if (q == bb) tl.L2[atomicAdd(&ts.ng2, 1u)] = comp_key(tg_key(y), id);
    });
    __syncthreads();
    if (bb >= 0 && (threadIdx.x >> 6) == 1) bucket::wave_rank64(tl.L2, nb2, m, tl.R2, tl.Q2);
    if (na > 64u) {
      bucket::rank_list<BT>(tl.L, na, m, tl.R, tl.Q, ts.red64b);  // ends with a barrier
    } else {
      if ((threadIdx.x >> 6) == 0) bucket::wave_rank64(tl.L, na, m, tl.R, tl.Q);
      __syncthreads();
    }
    if (cut_search) {
      const int i = bucket::first_rank_once(tl.Q, na, P - bucket::mass_before(tl.MI, bp), &ts.first);
      cutc = tl.R[i];
      Sp = bucket::mass_before(tl.MI, bp) + (i > 0 ? tl.Q[i - 1] : 0ull) + bucket::mass_c(cutc, m);
      ntopp = bucket::count_before(tl.CI, bp) + (unsigned)i + 1u;
    }
    const u64 t = mul_shr24(Sp, uq);
    const u64 tb = t + 1 - bucket::mass_before(tl.MI, btl);
    if (bb >= 0) pick = tl.R2[bucket::first_rank_once(tl.Q2, nb2, tb, &ts.first2)];
    else pick = tl.R[bucket::first_rank_once(tl.Q, na, tb, &ts.first2)];
  } else {
    if (cut_search) {
      u64 before;
      unsigned rank;
      cutc = resolve_mass(rv, tl, bp, P - bucket::mass_before(tl.MI, bp), &before, &rank, ts, bs);
      Sp = bucket::mass_before(tl.MI, bp) + before + bucket::mass_c(cutc, m);
      ntopp = bucket::count_before(tl.CI, bp) + rank + 1;
    }
    const u64 t = mul_shr24(Sp, uq);
    const int bt = bucket::find_mass<BT>(tl.MI, t + 1, &ts.sel[1]);
    u64 before;
    unsigned rank;
    pick = resolve_mass(rv, tl, bt, t + 1 - bucket::mass_before(tl.MI, bt), &before, &rank, ts, bs);
  }
  // diagnostics: with top-p disabled the cut is the smallest allowed composite
  if (cut_last && a.dbg.cut_ids) {
    u64 x = 0;
    rv.each([&](int id, float y) {
      const u64 v = ~comp_key(tg_key(y), id);
      x = v > x ? v : x;
    });
    cutc = ~block_reduce_max(x, ts.red64);
  }
  if (threadIdx.x == 0) {
    a.out[b] = comp_id(pick);
    write_row_diag(a, b, (int)nv, (int)ntopp, S, Sp, comp_id(cutc));
  }
  if (a.dbg.kept_ids)
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) a.dbg.kept_ids[(long long)b * a.dbg.kept_cap + i] = -1;
  if (a.dbg.kept_probs)
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) a.dbg.kept_probs[(long long)b * a.dbg.kept_cap + i] = 0.0f;
}

template <typename Tin, bool RES>
__device__ __forceinline__ void topp_row(const SampleArgs& a, Row& r, unsigned char* smem, Scratch& ts,
                                         BlockScratch& bs, const uint4 (&raw)[RowView<Tin, RES>::NV],
                                         const uint32_t (&mw)[RowView<Tin, RES>::NV]) {
  const int b = r.b;
  const int bw = a.TS > 0 ? (a.V + 31) / 32 : 0;
  uint32_t* hbits = (uint32_t*)smem;
  int2* hash = (int2*)(smem + ((bw * 4 + 15) / 16) * 16);
  Tail tl;
  tl.L = (u64*)((unsigned char*)hash + (size_t)a.TS * 8);  // CAPG (+ pad)
  tl.R = tl.L + CAPG + 2;                                   // CAPG
  tl.Q = tl.R + CAPG;                                       // CAPG
  tl.CI = (unsigned*)(tl.Q + CAPG);                         // NB + 1 (+ pad)
  tl.MI = (u64*)(tl.CI + NB + 4);                           // NB + 1
  tl.L2 = tl.MI + NB + 1;                                   // 64 (+ pad)
  tl.R2 = tl.L2 + 66;                                       // 64
  tl.Q2 = tl.R2 + 64;                                       // 64
  tl.E = (Packed*)(tl.Q2 + 64);                             // a.topp_cap
  r.v0 = 0;
  r.v1 = a.V;
  if (r.use_pen) hash_build<BT>(a, r, hash, hbits, bw);
  RowView<Tin, RES> rv(a, r, hash, hbits, (const Tin*)a.logits + (long long)b * a.row_stride);
  rv.load(raw, mw);
  if (a.dbg.post_logits) {
    float* post = a.dbg.post_logits + (long long)b * a.V;
    for (int v = threadIdx.x; v < a.V; v += BT) post[v] = -__builtin_inff();
    __syncthreads();
    rv.each([&](int id, float y) { post[id] = y; });
  }

  // pass 1: the largest composite (the greedy answer; its y is the maximum m)
  // and the allowed count
  u64 mcl = 0;
  unsigned nvl = 0;
  if constexpr (RES) {
    // branch free over the registers: a thread's ids rise with the index,
    // so a strict > keeps the smallest id among its equal maxima (the slot
    // is tracked, and its id formed once)
    constexpr int EPV = RowView<Tin, RES>::EPV;
    float mx = -__builtin_inff();
    int mq = 0;
#pragma unroll
    for (int q = 0; q < RES_EPT; q++) {
      const float y = rv.y[q];
      const bool gt = y > mx;
      mq = gt ? q : mq;
      mx = gt ? y : mx;
    }
    nvl = rv.nallowed;
    const int mid = ((int)threadIdx.x + (mq / EPV) * BT) * EPV + mq % EPV;
    mcl = mx > -__builtin_inff() ? comp_key(tg_key(mx), mid) : 0ull;
  } else {
    rv.each([&](int id, float y) {
      const u64 c = comp_key(tg_key(y), id);
      mcl = c > mcl ? c : mcl;
      nvl++;
    });
  }
  for (int i = threadIdx.x; i < NB + 1; i += BT) {
    tl.CI[i] = 0u;
    tl.MI[i] = 0ull;
  }
  const unsigned nown = nvl;  // this thread's allowed ids
  const unsigned wincl = wave_incl_scan(nown);  // lane 63: the wave's allowed ids
  mcl = wave_max(mcl);
  if (lane_id() == 63) {
    ts.red64[threadIdx.x >> 6] = mcl;
    ts.red32[threadIdx.x >> 6] = wincl;
  }
  __syncthreads();
  u64 Mc = 0;
  unsigned nv = 0, wbase = 0;  // wbase: allowed ids of the waves before this one
#pragma unroll
  for (int i = 0; i < WT; i++) {
    Mc = ts.red64[i] > Mc ? ts.red64[i] : Mc;
    wbase += i < (int)(threadIdx.x >> 6) ? ts.red32[i] : 0u;
    nv += ts.red32[i];
  }
  if (nv == 0 || r.mode == 0) {
    // nothing allowed (-1), or a greedy row (the largest composite)
    const int id = nv ? comp_id(Mc) : -1;
    if (threadIdx.x == 0) {
      a.out[b] = id;
      write_row_diag(a, b, id >= 0, id >= 0, 0, 0, id);
    }
    if (a.dbg.kept_ids)
      for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT)
        a.dbg.kept_ids[(long long)b * a.dbg.kept_cap + i] = (i == 0 && r.mode == 0) ? id : -1;
    if (a.dbg.kept_probs)
      for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT)
        a.dbg.kept_probs[(long long)b * a.dbg.kept_cap + i] = (i == 0 && r.mode == 0 && id >= 0) ? 1.0f : 0.0f;
    return;
  }
  tl.m = comp_y(Mc);
  if constexpr (RES) {
    if (nv <= (unsigned)a.topp_cap) {
      // few allowed ids (a grammar mask): they alone, packed into LDS, feed
      // every later pass (the exact exp and the bucket gathers run on
      // allowed ids only)
      // (in wave order: a thread's slots follow the allowed ids of the
      // waves and lanes before it)
      Packed* dst = tl.E + (wbase + wincl - nown);
      rv.each([&](int id, float y) { *dst++ = Packed{y, id}; });
      __syncthreads();
      topp_rest(a, r, CompactView{tl.E, (int)nv}, tl, Mc, nv, ts, bs);
      return;
    }
  }
  topp_rest(a, r, rv, tl, Mc, nv, ts, bs);
}

template <typename Tin, bool RES>
__global__ __launch_bounds__(BT) void topp_kernel(SampleArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ Scratch ts;
  __shared__ BlockScratch bs;
  const int b = blockIdx.x;
  if (b >= a.B) return;
  // the row's parameters (scalar loads) requested before its vectors, so
  // that they arrive first.  The mask words wait for them (the first request
  // takes about a microsecond): the row's first NPRE vectors go out before
  // the words, the rest after them, so that neither the row's stream waits
  // for the parameters nor the words for the whole row (the vectors are
  // evaluated in order, each with its word).
  using RV = RowView<Tin, RES>;
  constexpr int NPRE = RV::NV < TOPP_MASK_PRE ? RV::NV : TOPP_MASK_PRE;
  const tgs_row_params p = a.params[b];
  const float ub = a.u[b];
  const int hl = a.hist_len ? a.hist_len[b] : a.hist_cap;
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  uint4 raw[RV::NV];
  RV::template fetch<0, NPRE>(a, rowp, raw);
  Row r;
  const bool valid = row_setup_from(a, b, 0, p, ub, hl, r);
  const bool mine = valid && (r.mode == 2 ? !(r.k >= 1 && r.k < a.V) : (r.mode == 0 && a.topp_all));
  if (!mine) {
    // other kernels' rows; in a launch that serves the whole batch, invalid
    // rows (-2) and rows outside the hint (-3)
    if (a.topp_all && threadIdx.x == 0) {
      a.out[b] = valid ? -3 : -2;
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    return;
  }
  uint32_t mw[RV::NV];
  RV::mask_words(a, r, mw);
  RV::template fetch<NPRE, RV::NV>(a, rowp, raw);
  topp_row<Tin, RES>(a, r, smem, ts, bs, raw, mw);
}

}  // namespace topp

size_t topp_lds_bytes(int V, int TS) {
  const int bw = TS > 0 ? (V + 31) / 32 : 0;
  return (size_t)((bw * 4 + 15) / 16) * 16 + (size_t)TS * 8 + (size_t)(3 * TOPP_CAP + 2) * 8 +
         (size_t)(bucket::NB + 4) * 4 + (size_t)(bucket::NB + 1) * 8 + (size_t)(66 + 64 + 64) * 8;
}

int topp_pack_cap(int V, int TS, size_t lds_avail) {
  const size_t base = topp_lds_bytes(V, TS);
  if (lds_avail <= base) return 0;
  const size_t n = (lds_avail - base) / sizeof(topp::Packed);
  return (int)(n < (size_t)V ? n : (size_t)V);
}

hipError_t launch_topp(const SampleArgs& a, int dtype, hipStream_t st) {
  const size_t lds = topp_lds_bytes(a.V, a.TS) + (size_t)a.topp_cap * sizeof(topp::Packed);
  const bool res = a.V <= TOPP_NT * topp::RES_EPT;  // the row fits in registers
  const dim3 g(a.B), blk(TOPP_NT);
  if (dtype == 1) {
    if (res) hipLaunchKernelGGL((topp::topp_kernel<uint16_t, true>), g, blk, lds, st, a);
    else hipLaunchKernelGGL((topp::topp_kernel<uint16_t, false>), g, blk, lds, st, a);
  } else {
    if (res) hipLaunchKernelGGL((topp::topp_kernel<float, true>), g, blk, lds, st, a);
    else hipLaunchKernelGGL((topp::topp_kernel<float, false>), g, blk, lds, st, a);
  }
  return hipGetLastError();
}

hipError_t set_topp_lds_limit(size_t bytes) {
  const void* fns[] = {(const void*)topp::topp_kernel<float, true>, (const void*)topp::topp_kernel<float, false>,
                       (const void*)topp::topp_kernel<uint16_t, true>, (const void*)topp::topp_kernel<uint16_t, false>};
  hipError_t e = hipSuccess;
  for (const void* f : fns) {
    hipError_t e2 = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e2 != hipSuccess) e = e2;
  }
  return e;
}

}  // namespace tgs
