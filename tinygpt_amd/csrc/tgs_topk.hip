// tgs_topk.hip -- batches whose rows are greedy or sample with 1 <= top_k <=
// KMAX (1024), for rows that fit in the registers of one workgroup (bf16 rows
// up to 163840 ids, fp32 rows up to 81920; 16-byte aligned, a whole number of
// 16-byte vectors): one workgroup of 1024 threads per row, the row read from
// HBM exactly once.
//
//   load    every thread issues its NVR 16-byte vectors (ids tid*EPV +
//           j*1024*EPV) and keeps them; the row's history (ids -> counts)
//           goes into an LDS hash and a bitmap while they are in flight.
//   bound   each thread keeps the two largest allowed logits among its ids
//           (NaN and masked ids count as -inf; three min/max per id).  Any k'
//           of the 2048 values are distinct ids, so the k'-th largest is a
//           logit with at least k' ids at or above it.  History ids may
//           still be penalised downward, so k' = k + (distinct history ids
//           of the row): at least k ids that are not history ids lie at or
//           above the bound.  Temperature is applied after the bound: 16
//           representable values of slack keep every id whose scaled logit
//           could round to the bound's.
//   collect every non-history id at or above the bound (registers, counted
//           then written), plus every history id with its penalised logit,
//           as composites (logit desc, id asc) into LDS.
//   select  the exact k-th composite (radix select over the candidates),
//           the k kept in order by a block bitonic sort (one per thread),
//           then masses, top-p and the draw.
//
// A candidate list beyond its capacity (massive ties at the bound) falls
// back to a radix selection over all ids of the row, still in registers.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace topk {

constexpr int BT = TOPK_NT;   // threads per workgroup
constexpr int WT = BT / 64;   // waves
constexpr int CAPK = TOPK_CAP;

struct alignas(16) u64x2 {
  u64 x, y;
};

struct Scratch {
  u64 red64[WT];
  unsigned red32[WT];
  unsigned nc;    // candidates written
  int imin0, imin1;
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

template <typename Tin, int NVR>
struct Regs {
  static constexpr int EPV = Elem<Tin>::EPV;
  uint4 raw[NVR];  // the row, packed as loaded
  __device__ __forceinline__ static int vec_id(int j) { return ((int)threadIdx.x + j * BT) * EPV; }
  // mask word of vector j (vectors past the row end hold NaN already)
  __device__ __forceinline__ static uint32_t mword(const Row& r, int V, int j) {
    const int v = vec_id(j);
    return r.mrow[(v < V ? v : V - 1) >> 5];
  }
  // every vector, from addresses clamped into the row (the row is 16-byte
  // aligned and a whole number of vectors); vectors past the end become NaN
  __device__ __forceinline__ void load(const Tin* rowp, int V) {
#pragma unroll
    for (int j = 0; j < NVR; j++) {
      const int v = vec_id(j);
      raw[j] = *(const uint4*)(rowp + (v < V ? v : V - EPV));
    }
#pragma unroll
    for (int j = 0; j < NVR; j++)
      if (vec_id(j) >= V) raw[j] = make_uint4(Elem<Tin>::NAN_BITS, Elem<Tin>::NAN_BITS, Elem<Tin>::NAN_BITS, Elem<Tin>::NAN_BITS);
  }
  // logit of element e of vector j mapped for the bound: -inf when NaN,
  // -inf or masked out (and for ids past the row end)
  template <bool MASK>
  __device__ __forceinline__ float xval(int j, int e, uint32_t mw) const {
    const float x = fmaxf(Elem<Tin>::get(raw[j], e), -__builtin_inff());
    if constexpr (!MASK) return x;
    return ((mw >> ((vec_id(j) + e) & 31)) & 1u) ? x : -__builtin_inff();
  }
  // Each pass over the row unpacks it again: an empty asm on the packed
  // registers keeps the compiler from holding every unpacked logit live from
  // one pass to the next (they do not fit the register budget).
  __device__ __forceinline__ void fence() {
#if defined(__HIP_DEVICE_COMPILE__)
#pragma unroll
    for (int j = 0; j < NVR; j++) asm volatile("" : "+v"(raw[j].x), "+v"(raw[j].y), "+v"(raw[j].z), "+v"(raw[j].w));
#endif
  }
};

__device__ __forceinline__ bool hist_bit(const uint32_t* hbits, int id) { return (hbits[id >> 5] >> (id & 31)) & 1u; }

// Canonical logit of a (non-history) id from its raw logit: y = z / T when
// allowed, else the composite 0.
__device__ __forceinline__ u64 comp_of(float z, bool allowed, float invT, int id) {
  const float y = z * invT;
  return (allowed && y > -__builtin_inff()) ? comp_key(tg_key(y), id) : 0ull;
}

// Block bitonic sort, descending, of BT * RG values, RG per thread: element
// (w * RG + h) * 64 + lane is x[h] of lane `lane` of wave w.  Partners in the
// same 64-block move through lane permutes; stride 64 (RG == 2) swaps the
// thread's two registers; wider strides go through LDS (buf: BT * RG
// entries).  Every thread calls it.
template <int RG, typename T>
__device__ __forceinline__ void block_sort_desc(T (&x)[RG], T* buf) {
  const int lane = lane_id(), w = threadIdx.x >> 6;
  constexpr int N = BT * RG;
#pragma unroll
  for (int k = 2; k <= N; k <<= 1) {
#pragma unroll
    for (int j = k >> 1; j > 0; j >>= 1) {
      if (j >= 64 * RG) {
#pragma unroll
        for (int h = 0; h < RG; h++) buf[(w * RG + h) * 64 + lane] = x[h];
        __syncthreads();
#pragma unroll
        for (int h = 0; h < RG; h++) {
          const int i = (w * RG + h) * 64 + lane;
          const T y = buf[i ^ j];
          const bool keep_max = ((i & j) == 0) == ((i & k) == 0);
          x[h] = keep_max ? (y > x[h] ? y : x[h]) : (y < x[h] ? y : x[h]);
        }
        __syncthreads();
      } else if (j >= 64) {
        if constexpr (RG == 2) {
          const bool desc = (((w * 2) * 64 + lane) & k) == 0;
          const T hi = x[0] > x[1] ? x[0] : x[1], lo = x[0] > x[1] ? x[1] : x[0];
          x[0] = desc ? hi : lo;
          x[1] = desc ? lo : hi;
        }
      } else {
#pragma unroll
        for (int h = 0; h < RG; h++) {
          const int i = (w * RG + h) * 64 + lane;
          const T y = xor_lane_s(x[h], j);
          const bool keep_max = ((lane & j) == 0) == ((i & k) == 0);
          x[h] = keep_max ? (y > x[h] ? y : x[h]) : (y < x[h] ? y : x[h]);
        }
      }
    }
  }
}

// Softmax masses of the n sorted kept composites R, top-p cut, draw and the
// outputs (row b, sampling mode).  C gets the inclusive mass prefix.
__device__ __forceinline__ void finish(const SampleArgs& a, const Row& r, const u64* R, u64* C, int n, Scratch& ts) {
  const int b = r.b;
  const float m = comp_y(R[0]);
  const u64 q = (int)threadIdx.x < n ? tg_q40(tg_weight(comp_y(R[threadIdx.x]), m)) : 0ull;
  const u64 wi = wave_incl_scan(q);
  if (lane_id() == 63) ts.red64[threadIdx.x >> 6] = wi;
  if (threadIdx.x == 0) {
    ts.imin0 = n - 1;
    ts.imin1 = 0x7FFFFFFF;
  }
  __syncthreads();
  u64 off = 0;
  for (int i = 0; i < (int)(threadIdx.x >> 6); i++) off += ts.red64[i];
  if ((int)threadIdx.x < n) C[threadIdx.x] = off + wi;
  __syncthreads();
  const u64 S = C[n - 1];
  if (r.top_p < 1.0f) {
    const uint32_t pq = (uint32_t)(r.top_p * 16777216.0f);
    const u64 P = mul_shr24(S, pq);
    const int i = threadIdx.x;
    if (i < n && C[i] >= P && (i == 0 || C[i - 1] < P)) atomicMin(&ts.imin0, i);
    __syncthreads();
  }
  const int istar = ts.imin0;
  const u64 Sp = C[istar];
  const uint32_t uq = (uint32_t)(r.u * 16777216.0f);
  const u64 t = mul_shr24(Sp, uq);
  {
    const int i = threadIdx.x;
    if (i <= istar && C[i] > t && (i == 0 || C[i - 1] <= t)) atomicMin(&ts.imin1, i);
  }
  __syncthreads();
  int pick = ts.imin1;
  if (pick > istar) pick = istar;
  if (threadIdx.x == 0) {
    a.out[b] = comp_id(R[pick]);
    write_row_diag(a, b, n, istar + 1, S, Sp, comp_id(R[istar]));
  }
  if (a.dbg.kept_ids) {
    int32_t* kid = a.dbg.kept_ids + (long long)b * a.dbg.kept_cap;
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) kid[i] = i < n ? comp_id(R[i]) : -1;
  }
  if (a.dbg.kept_probs) {
    float* kp = a.dbg.kept_probs + (long long)b * a.dbg.kept_cap;
    const float fs = tg_u64_to_f32(Sp);
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) {
      float pv = 0.0f;
      if (i <= istar) pv = tg_u64_to_f32(C[i] - (i ? C[i - 1] : 0ull)) / fs;
      kp[i] = pv;
    }
  }
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

template <typename Tin, int NVR, bool MASK>
__device__ __forceinline__ void topk_row(const SampleArgs& a, Row& r, unsigned char* smem, Scratch& ts,
                                         BlockScratch& bs) {
  using RG = Regs<Tin, NVR>;
  constexpr int EPV = RG::EPV;
  const int b = r.b;
  const int V = a.V;
  const int bw = a.TS > 0 ? (V + 31) / 32 : 0;
  uint32_t* hbits = (uint32_t*)smem;
  int2* hash = (int2*)(smem + ((bw * 4 + 15) / 16) * 16);
  u64* cand = (u64*)((unsigned char*)hash + (size_t)a.TS * 8);  // CAPK (+ pad)
  u64* K = cand + CAPK + 2;                                      // KMAX (+ pad)
  u64* R = K + KMAX + 2;                                         // KMAX
  u64* C = R + KMAX;                                             // KMAX
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  const int k = r.mode == 0 ? 1 : r.k;

  // load: every vector of the row, once
  RG g;
  g.load(rowp, V);
  // history: id -> count hash and the row's bitmap; distinct ids
  r.v0 = 0;
  r.v1 = V;
  unsigned nh = 0;
  if (r.use_pen) {
    hash_build<BT>(a, r, hash, hbits, bw);
    unsigned c = 0;
    for (int i = threadIdx.x; i < a.TS; i += BT) c += hash[i].x != -1;
    nh = bsum(c, ts.red32);
  }
  const bool mask = MASK && r.mrow != nullptr;

  // bound: the two largest x of this thread
  float a1 = -__builtin_inff(), a2 = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < NVR; j++) {
    const uint32_t mw = MASK && mask ? RG::mword(r, V, j) : 0xFFFFFFFFu;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      const float x = g.template xval<MASK>(j, e, mw);
      a2 = fmaxf(a2, fminf(a1, x));
      a1 = fmaxf(a1, x);
    }
  }
  g.fence();
  const unsigned kp = (unsigned)k + nh;
  // (kp <= 2 * BT: the dispatch keeps top_k <= KMAX and the history to
  // at most KMAX ids)
  const uint32_t tkey = block_select_kth<uint32_t, 32, BT>(
      [&](auto f) {
        f(tg_key(a1));
        f(tg_key(a2));
      },
      kp, bs);
  // raw-logit bound, 16 representable values lower: a raw logit below it
  // scales (x / T, correctly rounded and monotone) strictly below the
  // scaled bound, also across a binade edge
  const uint32_t kneg = 0x007FFFFFu;  // key of -inf
  const float thz = tkey > kneg + 16u ? tg_unkey(tkey - 16u) : -__builtin_inff();

  // collect: every non-history id at or above the bound (counted, placed by
  // a wave scan, written), then every history id with its penalised logit
  const float thf = fmaxf(thz, -3.40282347e38f);  // -inf never qualifies
  unsigned cnt = 0;
#pragma unroll
  for (int j = 0; j < NVR; j++) {
    const uint32_t mw = MASK && mask ? RG::mword(r, V, j) : 0xFFFFFFFFu;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      const float x = g.template xval<MASK>(j, e, mw);
      if (x >= thf && !(r.use_pen && hist_bit(hbits, RG::vec_id(j) + e))) cnt++;
    }
  }
  g.fence();
  if (threadIdx.x == 0) ts.nc = 0;
  __syncthreads();
  const unsigned wincl = wave_incl_scan(cnt);
  unsigned wbase = 0;
  if (lane_id() == 63 && wincl) wbase = atomicAdd(&ts.nc, wincl);
  wbase = __shfl(wbase, 63, 64);
  unsigned slot = wbase + wincl - cnt;
  if (cnt) {
#pragma unroll
    for (int j = 0; j < NVR; j++) {
      const uint32_t mw = MASK && mask ? RG::mword(r, V, j) : 0xFFFFFFFFu;
#pragma unroll
      for (int e = 0; e < EPV; e++) {
        const float x = g.template xval<MASK>(j, e, mw);
        const int id = RG::vec_id(j) + e;
        if (x >= thf && !(r.use_pen && hist_bit(hbits, id))) {
          if (slot < (unsigned)CAPK) cand[slot] = comp_of(x, true, r.invT, id);
          slot++;  // a composite 0 (scaled to -inf) drops out below
        }
      }
    }
  }
  if (r.use_pen) {
    for (int i = threadIdx.x; i < a.TS; i += BT) {
      const int2 h = hash[i];
      if (h.x == -1) continue;
      const int id = h.x;
      const float z = penalise(Elem<Tin>::scalar(rowp, id), h.y, r);
      const u64 c = comp_of(z, mask_allows(r, id), r.invT, id);
      if (c) {
        const unsigned sl = atomicAdd(&ts.nc, 1u);
        if (sl < (unsigned)CAPK) cand[sl] = c;
      }
    }
  }
  __syncthreads();
  const int nc = (int)ts.nc;
  int nk;
  if (nc <= CAPK) {
    // exact k-th composite of the candidates, then exactly those >= it
    int nz = 0;
    for (int i = threadIdx.x; i < nc; i += BT) nz += cand[i] != 0ull;
    nz = (int)bsum((unsigned)nz, ts.red32);
    u64 T = 1;
    if (nz > k)
      T = block_select_kth<u64, 64, BT>(
          [&](auto f) {
            for (int i = threadIdx.x; i < nc; i += BT)
              if (cand[i]) f(cand[i]);
          },
          (unsigned)k, bs);
    if (threadIdx.x == 0) ts.nc = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < nc; i += BT) {
      const u64 c = cand[i];
      if (c && c >= T) K[atomicAdd(&ts.nc, 1u)] = c;
    }
    __syncthreads();
    nk = (int)ts.nc;
  } else {
    // candidate overflow: radix selection over every id of the row, read
    // again from L2 (rare: massive ties at the bound)
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
          const u64 c = comp_of(z, mask_allows(r, id), r.invT, id);
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
      if (c >= T) K[atomicAdd(&ts.nc, 1u)] = c;
    });
    __syncthreads();
    nk = (int)ts.nc;
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
        const float y = z * r.invT;
        post[id] = (mask_allows(r, id) && y > -__builtin_inff()) ? y : -__builtin_inff();
      }
    }
  }
  if (nk == 0) {
    if (r.mode == 0) {
      finish_greedy(a, b, 0ull);
    } else {
      if (threadIdx.x == 0) {
        a.out[b] = -1;
        write_row_diag(a, b, 0, 0, 0, 0, -1);
      }
      if (a.dbg.kept_ids)
        for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) a.dbg.kept_ids[(long long)b * a.dbg.kept_cap + i] = -1;
      if (a.dbg.kept_probs)
        for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BT) a.dbg.kept_probs[(long long)b * a.dbg.kept_cap + i] = 0.0f;
    }
    return;
  }
  {
    // the kept set in order: a bitonic sort of one entry per thread (0 pads last)
    u64 xs[1] = {(int)threadIdx.x < nk ? K[threadIdx.x] : 0ull};
    __syncthreads();
    block_sort_desc<1>(xs, K);
    if ((int)threadIdx.x < nk) R[threadIdx.x] = xs[0];
    __syncthreads();
  }
  if (r.mode == 0) finish_greedy(a, b, R[0]);
  else finish(a, r, R, C, nk, ts);
}

template <typename Tin, int NVR, bool MASK>
__global__ __launch_bounds__(BT) void topk_kernel(SampleArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ Scratch ts;
  __shared__ BlockScratch bs;
  const int b = blockIdx.x;
  if (b >= a.B) return;
  Row r;
  const bool valid = row_setup(a, b, 0, r);
  if (!valid || outside_hint(a, r) || r.mode == 2) {
    if (threadIdx.x == 0) {
      a.out[b] = valid ? -3 : -2;  // -3: row outside the launch hint
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    return;
  }
  topk_row<Tin, NVR, MASK>(a, r, smem, ts, bs);
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
  return (size_t)((bw * 4 + 15) / 16) * 16 + (size_t)TS * 8 + (size_t)(TOPK_CAP + 2 + 3 * KMAX + 2) * 8;
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
