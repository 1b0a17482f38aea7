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
//   pass 1  y (mask, penalties, 1/T): the maximum m and the allowed count;
//   pass 2  per allowed id with y - m > -32 its mass q, added to bucket
//           floor((m - y) * 8) of a 256-bucket mass histogram.  Bucket
//           order follows the sorted order (a larger y never lands in a
//           later bucket), so the prefix over buckets locates the bucket of
//           the cut and then of the draw;
//   pass 3  gather that bucket's ids (composites) into LDS, rank them
//           exactly by counting, scan their masses in rank order and pick
//           the element.  The draw's bucket reuses the ranked list when it
//           is the cut's bucket; otherwise one more gather.
//
// A row of at most 32768 ids is held in registers (32 per thread) after one
// read; a longer row is streamed again from L2 / MALL by every pass.
//
// A bucket of more than CAPG ids (a flat row: ties, tiny temperature
// spreads) is resolved by a mass-weighted radix selection restricted to the
// bucket instead (a few more passes).  exp runs once per id (plus once per
// ranked id).
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace topp {

constexpr int BT = TOPP_NT;    // threads per workgroup
constexpr int WT = BT / 64;    // waves
constexpr int NBKT = 256;      // histogram buckets of width 1/8 in y below m
constexpr int CAPG = TOPP_CAP; // ids of one bucket ranked in LDS

struct alignas(16) u64x2 {
  u64 x, y;
};

constexpr int NCOPY = 4;       // histogram copies (lane & 3) to spread atomic contention
constexpr int RES_EPT = 32;    // ids per thread kept in registers when the row fits (V <= 32768)

struct Scratch {
  u64 hm[NCOPY][NBKT];
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
      const float yy = z * r.invT;
      yv[e] = (((mw >> (id & 31)) & 1u) && yy > -__builtin_inff() && id < a.V) ? yy : -__builtin_inff();
    }
  }

  __device__ __forceinline__ void load() {
    if constexpr (RES) {
      uint4 raw[NV];
#pragma unroll
      for (int j = 0; j < NV; j++) raw[j] = load_vec<Tin>(rowp, (threadIdx.x + j * BT) * EPV, a.V, a.aligned);
#pragma unroll
      for (int j = 0; j < NV; j++) {
        float yv[EPV];
        vec_y((threadIdx.x + j * BT) * EPV, raw[j], yv);
#pragma unroll
        for (int e = 0; e < EPV; e++) y[j * EPV + e] = yv[e];
      }
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
// `target` (>= 1) and the mass of the buckets ahead of it, into ts.
__device__ __forceinline__ void pick_bucket(Scratch& ts, u64 target) {
  const int lane = lane_id();
  u64 ms[4];
  u64 lm = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    u64 x = 0;
#pragma unroll
    for (int c = 0; c < NCOPY; c++) x += ts.hm[c][4 * lane + j];
    ms[j] = x;
    lm += x;
  }
  u64 cm = wave_incl_scan(lm) - lm;
  int found = -1;
  u64 ab = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (found < 0 && cm + ms[j] >= target) {
      found = 4 * lane + j;
      ab = cm;
    }
    cm += ms[j];
  }
  // one lane writes the result (the first lane that found the bucket)
  const u64 bal = __ballot(found >= 0);
  const int first = bal ? __ffsll((long long)bal) - 1 : 0;
  const int fb = __shfl(found, first, 64);
  const u64 fab = __shfl(ab, first, 64);
  if (lane == 0) {
    ts.bsel = fb;
    ts.bbefore = fab;
  }
}

// The bucket's ids ranked in LDS: R[0, n) holds their composites in
// descending order and Q[0, n) their inclusive mass prefix; *ahead gets the
// number of allowed ids in earlier buckets.  Returns n, or -1 when the
// bucket holds more than CAPG ids (nothing ranked).
template <class View>
__device__ __forceinline__ int rank_bucket(const View& rv, float m, int bkt, u64* L, u64* R, u64* Q, Scratch& ts,
                                           unsigned* ahead) {
  if (threadIdx.x == 0) ts.ng = 0;
  __syncthreads();
  unsigned na = 0;
  rv.each([&](int id, float y) {
    const int bk = bucket_of(y, m);
    na += (bk >= 0 && bk < bkt);
    if (bk == bkt) {
      const unsigned slot = atomicAdd(&ts.ng, 1u);
      if (slot < (unsigned)CAPG) L[slot] = comp_key(tg_key(y), id);
    }
  });
  *ahead = block_reduce_sum(na, ts.red32);  // also publishes L and ts.ng
  const int n = (int)ts.ng;
  if (n > CAPG) return -1;
  const int w = threadIdx.x >> 6;
  if (n <= 64) {
    // one wave: bitonic sort in registers (0 pads below every composite)
    if (w == 0) {
      const int lane = lane_id();
      const u64 x = wave_sort_desc(lane < n ? L[lane] : 0ull);
      if (lane < n) R[lane] = x;
    }
  } else {
    // rank = number of larger composites (composites are distinct), counted
    // by the waves that hold ids, two entries per 16-byte broadcast read
    if (threadIdx.x == 0 && (n & 1)) L[n] = 0ull;  // pad below every composite
    __syncthreads();
    const int j0 = threadIdx.x, j1 = threadIdx.x + BT;
    if (w * 64 < n) {
      const u64 x0 = j0 < n ? L[j0] : ~0ull, x1 = j1 < n ? L[j1] : ~0ull;
      int r0 = 0, r1 = 0;
      const int np = (n + 1) / 2;
      const u64x2* L2 = (const u64x2*)L;
      if (j1 - threadIdx.x + w * 64 < n) {  // this wave holds a second id too
#pragma unroll 4
        for (int i = 0; i < np; i++) {
          const u64x2 e = L2[i];
          r0 += (e.x > x0) + (e.y > x0);
          r1 += (e.x > x1) + (e.y > x1);
        }
      } else {
#pragma unroll 4
        for (int i = 0; i < np; i++) {
          const u64x2 e = L2[i];
          r0 += (e.x > x0) + (e.y > x0);
        }
      }
      if (j0 < n) R[r0] = x0;
      if (j1 < n) R[r1] = x1;
    }
  }
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
// the bucket and its rank within the bucket.  n: ids ranked in R/Q for this
// bucket (-1: more than CAPG, resolved by a mass-weighted radix selection
// restricted to the bucket).
template <class View>
__device__ __forceinline__ u64 select_in_bucket(const View& rv, float m, int bkt, u64 target, int n, const u64* R,
                                                const u64* Q, Scratch& ts, BlockScratch& bs, u64* before,
                                                unsigned* rank) {
  if (n >= 0) {
    const int i = first_rank(Q, n, target, ts);
    *before = i > 0 ? Q[i - 1] : 0ull;
    *rank = (unsigned)i;
    return R[i];
  }
  auto en = [&](auto f) {
    rv.each_stream([&](int id, float y) {
      if (bucket_of(y, m) == bkt) f(comp_key(tg_key(y), id), tg_q40(weight_le(y, m)));
    });
  };
  return block_mass_select<BT>(en, target, bs, before, rank);
}

template <typename Tin, bool RES>
__device__ __forceinline__ void topp_row(const SampleArgs& a, Row& r, unsigned char* smem, Scratch& ts,
                                         BlockScratch& bs) {
  const int b = r.b;
  const int bw = a.TS > 0 ? (a.V + 31) / 32 : 0;
  uint32_t* hbits = (uint32_t*)smem;
  int2* hash = (int2*)(smem + ((bw * 4 + 15) / 16) * 16);
  u64* L = (u64*)((unsigned char*)hash + (size_t)a.TS * 8);
  u64* R = L + CAPG;
  u64* Q = R + CAPG;
  r.v0 = 0;
  r.v1 = a.V;
  if (r.use_pen) hash_build<BT>(a, r, hash, hbits, bw);
  RowView<Tin, RES> rv(a, r, hash, hbits, (const Tin*)a.logits + (long long)b * a.row_stride);
  rv.load();
  if (a.dbg.post_logits) {
    float* post = a.dbg.post_logits + (long long)b * a.V;
    for (int v = threadIdx.x; v < a.V; v += BT) post[v] = -__builtin_inff();
    __syncthreads();
    rv.each([&](int id, float y) { post[id] = y; });
  }

  // pass 1: maximum and allowed count
  float mxl = -__builtin_inff();
  unsigned nvl = 0;
  rv.each([&](int, float y) {
    mxl = fmaxf(mxl, y);
    nvl++;
  });
  const float m = block_reduce_max(mxl, ts.redf);
  const unsigned nv = block_reduce_sum(nvl, ts.red32);
  if (nv == 0) {
    if (threadIdx.x == 0) {
      a.out[b] = -1;
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    return;
  }
  // pass 2: mass histogram over buckets below m (4 copies, by lane)
  for (int i = threadIdx.x; i < NCOPY * NBKT; i += BT) (&ts.hm[0][0])[i] = 0;
  __syncthreads();
  u64 Sl = 0;
  u64* hcopy = ts.hm[lane_id() & (NCOPY - 1)];
  rv.each([&](int, float y) {
    const int bk = bucket_of(y, m);
    if (bk < 0) return;
    const u64 q = tg_q40(weight_le(y, m));
    Sl += q;
    if (q) atomicAdd(&hcopy[bk], q);
  });
  const u64 S = block_reduce_sum(Sl, ts.red64);  // also orders the histogram atomics
  // the cut (top-p): element i* with inclusive prefix >= P
  u64 cutc = 0, Sp = S;
  unsigned ntopp = nv;
  bool cut_best = false, cut_last = false;
  int nr = -2, rb = -1;  // ids ranked in R/Q (-2: none), their bucket
  if (r.top_p < 1.0f) {
    const uint32_t pq = (uint32_t)(r.top_p * 16777216.0f);
    const u64 P = mul_shr24(S, pq);
    if (P == 0) {
      cut_best = true;
      Sp = tg_q40(1.0f);
      ntopp = 1;
    } else {
      if (threadIdx.x < 64) pick_bucket(ts, P);
      __syncthreads();
      const int bk = ts.bsel;
      const u64 bb = ts.bbefore;
      __syncthreads();
      unsigned ahead;
      nr = rank_bucket(rv, m, bk, L, R, Q, ts, &ahead);
      rb = bk;
      u64 before;
      unsigned rank;
      cutc = select_in_bucket(rv, m, bk, P - bb, nr, R, Q, ts, bs, &before, &rank);
      Sp = bb + before + tg_q40(weight_le(comp_y(cutc), m));
      ntopp = ahead + rank + 1;
    }
  } else {
    cut_last = true;
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
  unsigned ahead;
  if (bk != rb) nr = rank_bucket(rv, m, bk, L, R, Q, ts, &ahead);
  u64 before;
  unsigned rank;
  const u64 pick = select_in_bucket(rv, m, bk, t + 1 - bb, nr, R, Q, ts, bs, &before, &rank);
  // diagnostics: the cut is the largest composite (P == 0) or the smallest
  // allowed one (top-p disabled)
  if (cut_best || cut_last) {
    u64 x = 0;
    rv.each([&](int id, float y) {
      const u64 c = comp_key(tg_key(y), id);
      const u64 v = cut_best ? c : ~c;
      x = v > x ? v : x;
    });
    x = block_reduce_max(x, ts.red64);
    cutc = cut_best ? x : ~x;
  }
  if (threadIdx.x == 0) {
    a.out[b] = comp_id(pick);
    write_row_diag(a, b, (int)nv, (int)ntopp, S, Sp, comp_id(cutc));
  }
}

template <typename Tin, bool RES>
__global__ __launch_bounds__(BT) void topp_kernel(SampleArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ Scratch ts;
  __shared__ BlockScratch bs;
  const int b = blockIdx.x;
  if (b >= a.B) return;
  Row r;
  if (!row_setup(a, b, 0, r) || r.mode != 2 || (r.k >= 1 && r.k < a.V)) return;  // other kernels' rows
  topp_row<Tin, RES>(a, r, smem, ts, bs);
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
