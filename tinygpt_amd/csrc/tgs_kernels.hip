// tgs_kernels.hip -- gfx950 kernels of the decode-time sampler.
//
// Sampling a [B, V] batch takes one to three launches on the caller's
// stream:
//
//   chunk_kernel  workgroup (b, c) owns chunk c of row b (S chunks per row).
//                 It issues all 16-byte loads of its first tile up front,
//                 builds the row's history hash (id -> count) and chunk bitmap
//                 in LDS while they are in flight, then keys every id
//                 (penalised ids are skipped and re-added with their
//                 penalised logit), keeps a threshold-filtered candidate
//                 buffer in LDS and reduces it to the chunk's exact top-k
//                 (sorted) or its argmax.  With S == 1 the same workgroup
//                 finishes the row: softmax masses, top-p scan and draw.
//   merge_kernel  (S > 1 only) one workgroup per row merges the S sorted
//                 chunk lists -- for k <= 64 entirely in wave registers
//                 (bitonic top-64 merges) -- and finishes the row.
//
// Rows sampling top-p without a top-k run in tgs_topp.hip.
//
// The kernel boundary is the handoff between chunks: cross-workgroup
// fences cost a full L2 writeback per workgroup on this part, a second
// launch costs one dispatch.
//
//   full_kernel   (only when the batch may hold them) rows that sample
//                 without a usable top-k (k disabled or above KMAX): one
//                 workgroup per row makes several passes over the row with
//                 radix selections on exact integer masses.
//
// Every device function is inlined into its kernel: no kernel makes calls,
// so none needs a call stack or passes pointers to private memory.
//
// Speculative verification lives in tgs_spec.hip.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {

// kept candidates in cand[0, n) (unsorted, unique composites, n <= KMAX):
// sort, masses, top-p, draw.  cand must hold 2*KMAX entries.
__device__ __forceinline__ void finalize_topk(const SampleArgs& a, const Row& r, u64* cand, int n,
                                              BlockScratch& s) {
  const int b = r.b;
  u64* C = cand + KMAX;
  if (n > KMAX) n = KMAX;  // never taken: callers pass exact top-k sets (k <= KMAX)
  if (n <= 0) {
    if (threadIdx.x == 0) {
      a.out[b] = -1;
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    if (a.dbg.kept_ids)
      for (int i = threadIdx.x; i < a.dbg.kept_cap; i += NT) a.dbg.kept_ids[(long long)b * a.dbg.kept_cap + i] = -1;
    if (a.dbg.kept_probs)
      for (int i = threadIdx.x; i < a.dbg.kept_cap; i += NT) a.dbg.kept_probs[(long long)b * a.dbg.kept_cap + i] = 0.0f;
    return;
  }
  int n2 = 1;
  while (n2 < n) n2 <<= 1;
  for (int i = n + threadIdx.x; i < n2; i += NT) cand[i] = 0ull;
  __syncthreads();
  block_bitonic_desc(cand, n2);
  const float m = comp_y(cand[0]);
  for (int i = threadIdx.x; i < n; i += NT) C[i] = tg_q40(tg_weight(comp_y(cand[i]), m));
  __syncthreads();
  block_incl_scan_u64(C, n, s.red64);
  const u64 S = C[n - 1];
  if (threadIdx.x == 0) {
    s.imin0 = n - 1;
    s.imin1 = 0x7FFFFFFF;
  }
  __syncthreads();
  if (r.top_p < 1.0f) {
    const uint32_t pq = (uint32_t)(r.top_p * 16777216.0f);
    const u64 P = mul_shr24(S, pq);
    int best = 0x7FFFFFFF;
    for (int i = threadIdx.x; i < n; i += NT)
      if (C[i] >= P && i < best) best = i;
    if (best != 0x7FFFFFFF) atomicMin(&s.imin0, best);
    __syncthreads();
  }
  const int istar = s.imin0;
  const u64 Sp = C[istar];
  const uint32_t uq = (uint32_t)(r.u * 16777216.0f);
  const u64 t = mul_shr24(Sp, uq);
  {
    int best = 0x7FFFFFFF;
    for (int i = threadIdx.x; i <= istar; i += NT)
      if (C[i] > t && i < best) best = i;
    if (best != 0x7FFFFFFF) atomicMin(&s.imin1, best);
  }
  __syncthreads();
  int pick = s.imin1;
  if (pick > istar) pick = istar;
  if (threadIdx.x == 0) {
    a.out[b] = comp_id(cand[pick]);
    write_row_diag(a, b, n, istar + 1, S, Sp, comp_id(cand[istar]));
  }
  if (a.dbg.kept_ids) {
    int32_t* kid = a.dbg.kept_ids + (long long)b * a.dbg.kept_cap;
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += NT) kid[i] = i < n ? comp_id(cand[i]) : -1;
  }
  if (a.dbg.kept_probs) {
    float* kp = a.dbg.kept_probs + (long long)b * a.dbg.kept_cap;
    const float fs = tg_u64_to_f32(Sp);
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += NT) {
      float pv = 0.0f;
      if (i <= istar) pv = kept_prob(comp_y(cand[i]), m, fs);
      kp[i] = pv;
    }
  }
  __syncthreads();
}


// Keep the entries >= T of buf[0, n) in place (order not preserved); returns
// the new count.  Batches of 4*NT entries: a batch is read completely before
// its survivors are written, and survivors only land below the batch end
// (the output count never exceeds the number of entries read so far).
__device__ __forceinline__ int compact_ge(u64* buf, int n, u64 T, BlockScratch& s) {
  __syncthreads();
  if (threadIdx.x == 0) s.nbuf = 0;
  __syncthreads();
  for (int base = 0; base < n; base += 4 * NT) {
    u64 x[4];
    unsigned cnt = 0;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = base + j * NT + (int)threadIdx.x;
      x[j] = (i < n) ? buf[i] : 0ull;
      cnt += (i < n && x[j] >= T);
    }
    __syncthreads();
    unsigned pos = cnt ? atomicAdd(&s.nbuf, cnt) : 0u;
#pragma unroll
    for (int j = 0; j < 4; j++) {
      const int i = base + j * NT + (int)threadIdx.x;
      if (i < n && x[j] >= T) buf[pos++] = x[j];
    }
  }
  __syncthreads();
  return (int)s.nbuf;
}

// ------------------------------------------------------------------ full path

// Streams row b once, calling f(v, key, y) for every id.  Keys are
// recomputed from global memory (the row stays hot in L2 / MALL).
template <typename Tin, class F>
__device__ __forceinline__ void full_stream(const SampleArgs& a, const Row& r, const int2* hash,
                                            const Tin* rowp, F f) {
  constexpr int EPV = Elem<Tin>::EPV;
  const int nvec = (a.V + EPV - 1) / EPV;
  for (int vi = threadIdx.x; vi < nvec; vi += NT) {
    const int v = vi * EPV;
    const uint4 raw = load_vec<Tin>(rowp, v, a.V, a.aligned);
    const uint32_t mw = r.mrow ? r.mrow[v >> 5] : 0xFFFFFFFFu;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      const int id = v + e;
      float z = Elem<Tin>::get(raw, e);
      if (r.use_pen && id < a.V) {
        const int cnt = hash_count(hash, a.TS, a.ts_shift, id);
        if (cnt > 0) z = penalise(z, cnt, r);
      }
      float y;
      const uint32_t key = elem_key(z, ((mw >> (id & 31)) & 1u) != 0, r, &y);
      if (id < a.V) f(id, key, y);
    }
  }
}

template <typename Tin>
__device__ __forceinline__ void full_path(const SampleArgs& a, const Row& r, const int2* hash, u64* cand, BlockScratch& s) {
  const int b = r.b;
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  float* post = a.dbg.post_logits ? a.dbg.post_logits + (long long)b * a.V : nullptr;
  // pass A: maximum composite and allowed count
  u64 best = 0;
  unsigned nv = 0;
  full_stream<Tin>(a, r, hash, rowp, [&](int v, uint32_t key, float y) {
    if (post) post[v] = y;
    if (key) {
      nv++;
      const u64 c = comp_key(key, v);
      best = c > best ? c : best;
    }
  });
  best = block_max(best, s.red64);
  nv = block_sum(nv, s.red32);
  if (nv == 0) {
    finalize_topk(a, r, cand, 0, s);
    return;
  }
  const unsigned kk = (r.k >= 1 && r.k < a.V) ? ((unsigned)r.k < nv ? (unsigned)r.k : nv) : nv;
  // pass B: top-k threshold (exact count of kk entries)
  u64 T = 1;
  if (kk < nv) {
    T = block_select_kth<u64, 64>(
        [&](auto f) {
          full_stream<Tin>(a, r, hash, rowp, [&](int v, uint32_t key, float) {
            if (key) f(comp_key(key, v));
          });
        },
        kk, s);
  }
  const float m = comp_y(best);
  // pass C: total mass of the kept set and its last element
  u64 S = 0, minc = ~0ull;
  full_stream<Tin>(a, r, hash, rowp, [&](int v, uint32_t key, float y) {
    if (!key) return;
    const u64 c = comp_key(key, v);
    if (c < T) return;
    S += tg_q40(tg_weight(y, m));
    minc = c < minc ? c : minc;
  });
  S = block_sum(S, s.red64);
  minc = ~block_max(~minc, s.red64);
  auto kept_enum = [&](auto f) {
    full_stream<Tin>(a, r, hash, rowp, [&](int v, uint32_t key, float y) {
      if (!key) return;
      const u64 c = comp_key(key, v);
      if (c >= T) f(c, tg_q40(tg_weight(y, m)));
    });
  };
  // pass D: top-p cut
  u64 cutc = minc, Sp = S;
  unsigned ntopp = kk;
  if (r.top_p < 1.0f) {
    const uint32_t pq = (uint32_t)(r.top_p * 16777216.0f);
    const u64 P = mul_shr24(S, pq);
    if (P == 0) {
      cutc = best;
      Sp = tg_q40(1.0f);
      ntopp = 1;
    } else {
      u64 before;
      unsigned rank;
      cutc = block_mass_select(kept_enum, P, s, &before, &rank);
      Sp = before + tg_q40(tg_weight(comp_y(cutc), m));
      ntopp = rank + 1;
    }
  }
  // pass E: draw
  const uint32_t uq = (uint32_t)(r.u * 16777216.0f);
  const u64 t = mul_shr24(Sp, uq);
  u64 before;
  unsigned rank;
  const u64 pick = block_mass_select(kept_enum, t + 1, s, &before, &rank);
  if (threadIdx.x == 0) {
    a.out[b] = comp_id(pick);
    write_row_diag(a, b, (int)kk, (int)ntopp, S, Sp, comp_id(cutc));
  }
  if (a.dbg.kept_ids)
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += NT) a.dbg.kept_ids[(long long)b * a.dbg.kept_cap + i] = -1;
  if (a.dbg.kept_probs)
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += NT) a.dbg.kept_probs[(long long)b * a.dbg.kept_cap + i] = 0.0f;
}

// ------------------------------------------------------------------ chunk paths

template <typename Tin>
struct Tile {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int EPT = 32;          // elements per thread per tile
  static constexpr int U = EPT / EPV;     // 16-byte vectors per thread per tile
  static constexpr int SIZE = NT * EPT;   // ids per tile (8192)
};

__device__ __forceinline__ int tile_id(int t0, int j, int EPV) {
  const int u = j / EPV, e = j % EPV;
  return t0 + (u * NT + (int)threadIdx.x) * EPV + e;
}

template <typename Tin>
__device__ __forceinline__ void tile_load(const Tin* rowp, const Row& r, int t0, bool aligned,
                                          uint4 (&raw)[Tile<Tin>::U], uint32_t (&mw)[Tile<Tin>::U]) {
  constexpr int EPV = Tile<Tin>::EPV;
  constexpr int U = Tile<Tin>::U;
  if (aligned && t0 + Tile<Tin>::SIZE <= r.v1) {  // whole tile inside the chunk: plain vector loads
#pragma unroll
    for (int u = 0; u < U; u++) raw[u] = *(const uint4*)(rowp + t0 + (u * NT + (int)threadIdx.x) * EPV);
  } else {
#pragma unroll
    for (int u = 0; u < U; u++) raw[u] = load_vec<Tin>(rowp, t0 + (u * NT + (int)threadIdx.x) * EPV, r.v1, aligned);
  }
  if (r.mrow) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int v = t0 + (u * NT + (int)threadIdx.x) * EPV;
      mw[u] = r.mrow[(v < r.v1 ? v : r.v1 - 1) >> 5];
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; u++) mw[u] = 0xFFFFFFFFu;
  }
}

// Keys of a loaded tile; history ids (bitmap) and disallowed ids get key 0.
// Ids past the chunk end were loaded as NaN and get key 0 as well.
template <typename Tin>
__device__ __forceinline__ void tile_keys(const Row& r, const uint32_t* bitmap, int bw, int t0,
                                          const uint4 (&raw)[Tile<Tin>::U],
                                          const uint32_t (&mw)[Tile<Tin>::U],
                                          uint32_t (&key)[Tile<Tin>::EPT], float* post) {
  constexpr int EPV = Tile<Tin>::EPV;
  constexpr int U = Tile<Tin>::U;
  uint32_t hb[U];
  if (r.use_pen) {
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int v = t0 + (u * NT + (int)threadIdx.x) * EPV;
      const int w = (v - r.v0) >> 5;
      hb[u] = bitmap[w < bw ? w : bw - 1];
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; u++) hb[u] = 0u;
  }
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int v = t0 + (u * NT + (int)threadIdx.x) * EPV;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      const int id = v + e;
      const bool hist = (hb[u] >> ((id - r.v0) & 31)) & 1u;
      float y;
      const bool allowed = ((mw[u] >> (id & 31)) & 1u) && !hist;
      key[u * EPV + e] = elem_key(Elem<Tin>::get(raw[u], e), allowed, r, &y);
      if (post && id < r.v1 && !hist) post[id] = y;
    }
  }
}

// History ids of the chunk with their penalised logits: calls f(v, key, y).
template <typename Tin, class F>
__device__ __forceinline__ void history_pass(const SampleArgs& a, const Row& r, const int2* hash,
                                             const Tin* rowp, F f) {
  for (int i = threadIdx.x; i < a.TS; i += NT) {
    const int2 e = hash[i];
    if (e.x < 0) continue;
    const int v = e.x;
    const float z = penalise(Elem<Tin>::scalar(rowp, v), e.y, r);
    float y;
    const uint32_t key = elem_key(z, mask_allows(r, v), r, &y);
    f(v, key, y);
  }
}

// Lower bound T0 (a key) with at least k stream keys >= T0 in this tile.
template <int EPT>
__device__ __forceinline__ uint32_t first_threshold(const uint32_t (&key)[EPT], int k, BlockScratch& s) {
  if (k <= 64) {
    uint32_t mx = 0;
#pragma unroll
    for (int j = 0; j < EPT; j++) mx = key[j] > mx ? key[j] : mx;
    // the k-th largest thread maximum of a wave has k keys above it
    const uint32_t srt = wave_sort_desc(mx);
    const uint32_t wk = __shfl(srt, k - 1, 64);
    return block_max(wk, s.red32);
  }
  // per-thread j-th largest (j = ceil(k / NT) <= 4), then the ceil(k/j)-th
  // largest of those over the block
  const int jj = (k + NT - 1) / NT;
  uint32_t t4[4] = {0, 0, 0, 0};
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    uint32_t x = key[j];
#pragma unroll
    for (int q = 0; q < 4; q++) {
      const uint32_t hi = x > t4[q] ? x : t4[q];
      const uint32_t lo = x > t4[q] ? t4[q] : x;
      t4[q] = hi;
      x = lo;
    }
  }
  const uint32_t aj = jj == 1 ? t4[0] : jj == 2 ? t4[1] : jj == 3 ? t4[2] : t4[3];
  const unsigned rk = (unsigned)((k + jj - 1) / jj);
  return block_select_kth<uint32_t, 32>([&](auto f) { f(aj); }, rk, s);
}

// Bit j set <=> element j of this thread's tile is a candidate: allowed and
// composite (key, id) >= thr, tested on 32-bit halves.
template <int EPT, int EPV>
__device__ __forceinline__ uint32_t cand_mask(const uint32_t (&key)[EPT], int t0, u64 thr) {
  const uint32_t tk = (uint32_t)(thr >> 32), tl = (uint32_t)thr;
  uint32_t cm = 0;
#pragma unroll
  for (int j = 0; j < EPT; j++) {
    const uint32_t lo = 0xFFFFFFFFu - (uint32_t)tile_id(t0, j, EPV);
    const bool c = key[j] != 0u && (key[j] > tk || (key[j] == tk && lo >= tl));
    cm |= (uint32_t)c << j;
  }
  return cm;
}

template <typename Tin>
__device__ __forceinline__ void greedy_chunk(const SampleArgs& a, const Row& r, const int2* hash,
                                             const uint32_t* bitmap, BlockScratch& s,
                                             uint4 (&raw)[Tile<Tin>::U], uint32_t (&mw)[Tile<Tin>::U]) {
  using TL = Tile<Tin>;
  const Tin* rowp = (const Tin*)a.logits + (long long)r.b * a.row_stride;
  float* post = a.dbg.post_logits ? a.dbg.post_logits + (long long)r.b * a.V : nullptr;
  u64 best = 0;
  uint32_t key[TL::EPT];
  for (int t0 = r.v0; t0 < r.v1; t0 += TL::SIZE) {
    tile_keys<Tin>(r, bitmap, a.BW, t0, raw, mw, key, post);
    if (t0 + TL::SIZE < r.v1) tile_load<Tin>(rowp, r, t0 + TL::SIZE, a.aligned, raw, mw);
#pragma unroll
    for (int j = 0; j < TL::EPT; j++)
      if (key[j]) {
        const u64 c = comp_key(key[j], tile_id(t0, j, TL::EPV));
        best = c > best ? c : best;
      }
  }
  if (r.use_pen)
    history_pass<Tin>(a, r, hash, rowp, [&](int v, uint32_t k, float y) {
      if (post) post[v] = y;
      if (k) {
        const u64 c = comp_key(k, v);
        best = c > best ? c : best;
      }
    });
  best = block_max(best, s.red64);
  if (a.S == 1) {
    finalize_greedy(a, r.b, best);
    return;
  }
  if (threadIdx.x == 0) {
    a.ws[((long long)r.b * a.S + r.c) * a.ws_stride] = best;
    a.ws_cnt[r.b * a.S + r.c] = best ? 1 : 0;
  }
}

template <typename Tin>
__device__ __forceinline__ void topk_chunk(const SampleArgs& a, const Row& r, const int2* hash,
                                           const uint32_t* bitmap, u64* cand, BlockScratch& s,
                                           uint4 (&raw)[Tile<Tin>::U], uint32_t (&mw)[Tile<Tin>::U]) {
  using TL = Tile<Tin>;
  const Tin* rowp = (const Tin*)a.logits + (long long)r.b * a.row_stride;
  float* post = a.dbg.post_logits ? a.dbg.post_logits + (long long)r.b * a.V : nullptr;
  const int k = r.k;
  if (threadIdx.x == 0) s.nbuf = 0;
  u64 thr = 0;  // candidates: composite >= thr and key != 0
  uint32_t key[TL::EPT];
  bool first = true;
  for (int t0 = r.v0; t0 < r.v1; t0 += TL::SIZE) {
    tile_keys<Tin>(r, bitmap, a.BW, t0, raw, mw, key, post);
    if (t0 + TL::SIZE < r.v1) tile_load<Tin>(rowp, r, t0 + TL::SIZE, a.aligned, raw, mw);
    if (first) {
      thr = (u64)first_threshold<TL::EPT>(key, k, s) << 32;
      first = false;
    }
    uint32_t cm = cand_mask<TL::EPT, TL::EPV>(key, t0, thr);
    const unsigned total = block_sum((unsigned)__popc(cm), s.red32);
    const unsigned nbuf = s.nbuf;
    if (nbuf + total > (unsigned)CAPB) {
      // shrink: exact k-th composite over the buffer and this tile's candidates
      const uint32_t cm_old = cm;
      const u64 T = block_select_kth<u64, 64>(
          [&](auto f) {
            for (unsigned i = threadIdx.x; i < nbuf; i += NT) f(cand[i]);
#pragma unroll
            for (int j = 0; j < TL::EPT; j++)
              if ((cm_old >> j) & 1u) f(comp_key(key[j], tile_id(t0, j, TL::EPV)));
          },
          (unsigned)k, s);
      compact_ge(cand, (int)nbuf, T, s);
      thr = T;
      cm = cand_mask<TL::EPT, TL::EPV>(key, t0, thr);
    }
    {
      const unsigned mine = (unsigned)__popc(cm);
      const unsigned incl = wave_incl_scan(mine);
      unsigned base = 0;
      if (lane_id() == 63 && incl) base = atomicAdd(&s.nbuf, incl);
      base = __shfl(base, 63, 64) + incl - mine;
#pragma unroll
      for (int j = 0; j < TL::EPT; j++)
        if ((cm >> j) & 1u) {
          if (base < (unsigned)a.capt) cand[base] = comp_key(key[j], tile_id(t0, j, TL::EPV));
          base++;
        }
    }
    __syncthreads();
  }
  if (r.use_pen) {
    history_pass<Tin>(a, r, hash, rowp, [&](int v, uint32_t kk, float y) {
      if (post) post[v] = y;
      if (kk) {
        const u64 c = comp_key(kk, v);
        if (c >= thr) {
          const unsigned p = atomicAdd(&s.nbuf, 1u);
          if (p < (unsigned)a.capt) cand[p] = c;
        }
      }
    });
    __syncthreads();
  }
  int n = min((int)s.nbuf, a.capt);
  if (k <= 64) {
    if (n > 64) {
      const u64 T = block_select_kth<u64, 64>(
          [&](auto f) {
            for (int i = threadIdx.x; i < n; i += NT) f(cand[i]);
          },
          (unsigned)k, s);
      n = compact_ge(cand, n, T, s);  // exactly k <= 64
    }
    if (threadIdx.x < 64) {
      const int lane = lane_id();
      u64 x = lane < n ? cand[lane] : 0ull;
      x = wave_sort_desc(x);
      const int nk = n < k ? n : k;
      if (a.S == 1) {
        if (nk > 0) wave_finalize(a, r, x, nk);
      } else {
        if (lane < nk) a.ws[((long long)r.b * a.S + r.c) * a.ws_stride + lane] = x;
        if (lane == 0) a.ws_cnt[r.b * a.S + r.c] = nk;
      }
    }
    if (a.S == 1 && n == 0) finalize_topk(a, r, cand, 0, s);
    return;
  }
  // k > 64: exact top-k via radix selection in LDS
  if (n > k) {
    const u64 T = block_select_kth<u64, 64>(
        [&](auto f) {
          for (int i = threadIdx.x; i < n; i += NT) f(cand[i]);
        },
        (unsigned)k, s);
    n = compact_ge(cand, n, T, s);
  }
  if (a.S == 1) {
    finalize_topk(a, r, cand, n, s);
    return;
  }
  u64* dst = a.ws + ((long long)r.b * a.S + r.c) * a.ws_stride;
  for (int i = threadIdx.x; i < n; i += NT) dst[i] = cand[i];
  if (threadIdx.x == 0) a.ws_cnt[r.b * a.S + r.c] = n;
}

// ------------------------------------------------------------------ kernels

// Greedy rows and rows with 1 <= top_k <= KMAX, one workgroup per (row,
// chunk).  Rows that need the full path are left to full_kernel when
// a.full_rows is set and get id -3 (outside the launch hint) otherwise.
template <typename Tin>
__global__ __launch_bounds__(NT) void chunk_kernel(SampleArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ BlockScratch s;
  int2* hash = (int2*)(smem + a.off_hash);
  uint32_t* bitmap = (uint32_t*)(smem + a.off_bitmap);
  u64* cand = (u64*)(smem + a.off_cand);
  const int b = blockIdx.x / a.S, c = blockIdx.x % a.S;
  if (b >= a.B) return;
  Row r;
  if (!row_setup(a, b, c, r)) {
    if (c == 0 && threadIdx.x == 0) {
      a.out[b] = -2;
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    return;
  }
  if (outside_hint(a, r)) {
    if (c == 0 && threadIdx.x == 0) {
      a.out[b] = -3;
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    return;
  }
  if (r.mode == 2) return;  // full_kernel
  r.v0 = c * a.L;
  r.v1 = min(a.V, r.v0 + a.L);
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  uint4 raw[Tile<Tin>::U];
  uint32_t mw[Tile<Tin>::U];
  tile_load<Tin>(rowp, r, r.v0, a.aligned, raw, mw);  // in flight during the history build
  if (r.use_pen) hash_build(a, r, hash, bitmap, a.BW);
  if (r.mode == 0) greedy_chunk<Tin>(a, r, hash, bitmap, s, raw, mw);
  else topk_chunk<Tin>(a, r, hash, bitmap, cand, s, raw, mw);
}

// Rows with KMAX < top_k < V, one workgroup per row; every other row
// returns at once (rows without a top-k go to the top-p kernel).
template <typename Tin>
__global__ __launch_bounds__(NT) void full_kernel(SampleArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ BlockScratch s;
  int2* hash = (int2*)(smem + a.off_hash);
  u64* cand = (u64*)(smem + a.off_cand);
  const int b = blockIdx.x;
  if (b >= a.B) return;
  Row r;
  if (!row_setup(a, b, 0, r) || r.mode != 2 || !(r.k >= 1 && r.k < a.V)) return;
  if (r.use_pen) hash_build(a, r, hash, nullptr, 0);  // whole row, lookups per id
  full_path<Tin>(a, r, hash, cand, s);
}

// One workgroup per row: merge the S chunk results of greedy and candidate
// rows and finish them.
__global__ __launch_bounds__(NT) void merge_kernel(SampleArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ BlockScratch s;
  __shared__ u64 wl[NW][64];
  u64* cand = (u64*)(smem + a.off_cand);
  const int b = blockIdx.x;
  if (b >= a.B) return;
  Row r;
  if (!row_setup(a, b, 0, r) || r.mode == 2 || outside_hint(a, r)) return;
  const int S = a.S;
  const int WS = a.ws_stride;
  const u64* src = a.ws + (long long)b * S * WS;
  const int* cnt = a.ws_cnt + (long long)b * S;
  if (r.mode == 0) {
    u64 m = 0;
    for (int c = threadIdx.x; c < S; c += NT) {
      const u64 x = src[(long long)c * WS];
      m = x > m ? x : m;
    }
    m = block_max(m, s.red64);
    finalize_greedy(a, b, m);
    return;
  }
  const int k = r.k;
  int total = 0;
  for (int c = 0; c < S; c++) total += cnt[c];
  const int kk = total < k ? total : k;
  if (k <= 64) {
    const int w = threadIdx.x >> 6, lane = lane_id();
    u64 acc = 0;
    for (int c = w; c < S; c += NW) {
      const int nc = cnt[c];
      const u64 x = lane < nc ? src[(long long)c * WS + lane] : 0ull;
      acc = wave_merge_top64(acc, x);
    }
    wl[w][lane] = acc;
    __syncthreads();
    if (w == 0) {
      acc = wl[0][lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; w2++) acc = wave_merge_top64(acc, wl[w2][lane]);
      if (kk > 0) wave_finalize(a, r, acc, kk);
    }
    if (kk == 0) finalize_topk(a, r, cand, 0, s);
    return;
  }
  int n;
  if (total <= a.capt) {
    int off = 0;
    for (int c = 0; c < S; c++) {
      const int nc = cnt[c];
      for (int i = threadIdx.x; i < nc; i += NT) cand[off + i] = src[(long long)c * WS + i];
      off += nc;
    }
    __syncthreads();
    n = total;
    if (n > kk) {
      const u64 T = block_select_kth<u64, 64>(
          [&](auto f) {
            for (int i = threadIdx.x; i < n; i += NT) f(cand[i]);
          },
          (unsigned)kk, s);
      n = compact_ge(cand, n, T, s);
    }
  } else {
    const u64 T = block_select_kth<u64, 64>(
        [&](auto f) {
          for (int c = 0; c < S; c++) {
            const int nc = cnt[c];
            for (int i = threadIdx.x; i < nc; i += NT) f(src[(long long)c * WS + i]);
          }
        },
        (unsigned)kk, s);
    if (threadIdx.x == 0) s.nbuf = 0;
    __syncthreads();
    for (int c = 0; c < S; c++) {
      const int nc = cnt[c];
      for (int i = threadIdx.x; i < nc; i += NT) {
        const u64 x = src[(long long)c * WS + i];
        if (x >= T) {
          const unsigned p = atomicAdd(&s.nbuf, 1u);
          if (p < (unsigned)a.capt) cand[p] = x;
        }
      }
    }
    __syncthreads();
    n = min((int)s.nbuf, a.capt);
  }
  finalize_topk(a, r, cand, n, s);
}

// ------------------------------------------------------------------ launchers

hipError_t launch_sample(const SampleArgs& a, int dtype, size_t lds, hipStream_t st) {
  const dim3 g(a.B * a.S), blk(NT);
  if (dtype == 1) hipLaunchKernelGGL(chunk_kernel<uint16_t>, g, blk, lds, st, a);
  else hipLaunchKernelGGL(chunk_kernel<float>, g, blk, lds, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (a.S > 1) {
    hipLaunchKernelGGL(merge_kernel, dim3(a.B), blk, lds, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  if (a.full_rows) {
    if (dtype == 1) hipLaunchKernelGGL(full_kernel<uint16_t>, dim3(a.B), blk, lds, st, a);
    else hipLaunchKernelGGL(full_kernel<float>, dim3(a.B), blk, lds, st, a);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = launch_topp(a, dtype, st);
  }
  return e;
}

hipError_t set_sample_lds_limit(size_t bytes) {
  const void* fns[] = {(const void*)chunk_kernel<float>, (const void*)chunk_kernel<uint16_t>,
                       (const void*)full_kernel<float>,  (const void*)full_kernel<uint16_t>,
                       (const void*)merge_kernel};
  hipError_t e = hipSuccess;
  for (const void* f : fns) {
    hipError_t e2 = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e2 != hipSuccess) e = e2;
  }
  return e;
}

}  // namespace tgs
