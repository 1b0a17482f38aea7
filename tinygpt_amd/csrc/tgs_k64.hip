// tgs_k64.hip -- one fused kernel for batches whose rows are greedy or sample
// with 1 <= top_k <= 64 (the launch's batch hint promises it).
//
// Workgroup (b, c) of K64_NT = 256 threads (4 waves) owns chunk c of row b:
// S chunks per row, each one tile of at most 16384 ids (64 per thread:
// sixteen 16-byte vectors of fp32 or eight of bf16).  At entry it requests
// everything it reads first in one go -- two history ids per thread, the
// tile, the row's parameters, uniform and history length -- so that one
// memory latency covers them all.  Then:
//   * the history ids that fall in the chunk go to an LDS table
//     (id -> count) and to a 64-bit mask per thread of its history
//     elements, and the logit of every table slot is fetched again (an L2
//     hit);
//   * one pass scales the tile by 1/T (masked ids: -inf) and takes thread
//     maxima, leaving the history ids out (-inf); their penalised values
//     are computed per table slot afterwards;
//   * every wave sorts its thread maxima (bitonic, in registers); their
//     k-th and ceil(k/4)-th entries give a threshold with at least k
//     elements above it (first_threshold);
//   * every thread writes its elements at or above the threshold to its own
//     eight LDS slots (history candidates go to a compact region), then the
//     slots are compacted (a wave prefix sum, one LDS atomic per wave); when
//     ties or a skewed tile overflow them, a radix selection finds the
//     exact k-th composite first;
//   * ranks by counting (every candidate counts the entries above it,
//     several threads per candidate, 16-byte broadcast LDS reads) give the
//     chunk's top k, sorted.
// With S == 1 the workgroup finishes its row.  Otherwise wave 0 publishes
// the chunk's sorted list with agent-coherent stores (sc1: written through
// to memory past the per-XCD L2s, which are not coherent with each other),
// waits for them to complete and counts the chunk in the row's arrival
// counter with a relaxed device atomic.  The workgroup that arrives last
// reads the S lists back with agent-coherent loads, merges them the same
// way and finishes the row (masses, top-p, draw); it then clears the
// counter.  No agent-scope release/acquire fence is issued: on this part
// such a fence writes back or invalidates the whole L2 of the XCD.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace k64 {

constexpr int BS = K64_NT;
constexpr int NWB = BS / 64;
constexpr int KM = 64;  // largest top_k served

// A tile gives every thread 64 elements: 16384 ids.
template <typename Tin>
struct TileK {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int EPT = 64;
  static constexpr int U = EPT / EPV;  // 16-byte vectors per thread
  static constexpr int SIZE = BS * EPT;
};
constexpr int BITMAP_WORDS = K64_BITMAP_WORDS;  // one bit per id of a tile
static_assert(BITMAP_WORDS * 32 == BS * 64, "bitmap covers a tile");

// id of element j of this thread in the tile starting at t0
template <int EPV>
__device__ __forceinline__ int id_of(int t0, int j) {
  return t0 + ((j / EPV) * BS + (int)threadIdx.x) * EPV + (j % EPV);
}

// The tile's 16-byte vectors; ids at or past v1 read as NaN (never
// allowed).  A chunk that fills the tile is read without checks; with
// whole_vec a vector is wholly before or after v1 (chunk ends are multiples
// of 64 ids, and so is the row end's vector boundary).
template <typename Tin, int U = TileK<Tin>::U>
__device__ __forceinline__ void load_data(const Tin* rowp, int t0, int v1, bool aligned, bool whole_vec,
                                          uint4 (&raw)[U]) {
  constexpr int EPV = TileK<Tin>::EPV;
  if (whole_vec && t0 + TileK<Tin>::SIZE <= v1) {
#pragma unroll
    for (int u = 0; u < U; u++) raw[u] = *(const uint4*)(rowp + t0 + (u * BS + (int)threadIdx.x) * EPV);
  } else if (whole_vec) {
    const uint4 nan4 = make_uint4(Elem<Tin>::NAN_BITS, Elem<Tin>::NAN_BITS, Elem<Tin>::NAN_BITS, Elem<Tin>::NAN_BITS);
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int v = t0 + (u * BS + (int)threadIdx.x) * EPV;
      raw[u] = v < v1 ? *(const uint4*)(rowp + v) : nan4;
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; u++) raw[u] = load_vec<Tin>(rowp, t0 + (u * BS + (int)threadIdx.x) * EPV, v1, aligned);
  }
}

template <typename Tin, int U = TileK<Tin>::U>
__device__ __forceinline__ void load_mask(const Row& r, int t0, uint32_t (&mw)[U]) {
  constexpr int EPV = TileK<Tin>::EPV;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int v = t0 + (u * BS + (int)threadIdx.x) * EPV;
    mw[u] = r.mrow[(v < r.v1 ? v : r.v1 - 1) >> 5];
  }
}

// y = logit / T over a tile with no mask and no history ids.  NaN and -inf
// (ids at or past the chunk end were loaded as NaN) never pass a threshold
// test or raise a maximum, so they are left as they are.  Returns the
// thread maximum.
template <typename Tin, int U = TileK<Tin>::U>
__device__ __forceinline__ float values_plain(const Row& r, const uint4 (&raw)[U], float (&y)[TileK<Tin>::EPT]) {
  constexpr int EPV = TileK<Tin>::EPV;
  float mx = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < U; u++)
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      y[u * EPV + e] = Elem<Tin>::get(raw[u], e) * r.invT;
      mx = fmaxf(mx, y[u * EPV + e]);
    }
  return mx;
}

// The same with the grammar mask (masked ids: -inf) and/or the history ids
// of the tile left out (-inf; they are penalised separately).  hb: this
// thread's history elements, bit j for element j (from the LDS table
// build); masked ids are gathered into the same kind of mask first.
template <typename Tin, int U = TileK<Tin>::U>
__device__ __forceinline__ float values_general(const Row& r, u64 hb, int t0, const uint4 (&raw)[U],
                                                const uint32_t (&mw)[U], float (&y)[TileK<Tin>::EPT]) {
  constexpr int EPV = TileK<Tin>::EPV;
  constexpr uint32_t GM = (1u << EPV) - 1u;
  const float ninf = -__builtin_inff();
  const uint32_t hlo = (uint32_t)hb, hhi = (uint32_t)(hb >> 32);
  float mx = ninf;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int v = t0 + (u * BS + (int)threadIdx.x) * EPV;
    uint32_t d = ((u * EPV < 32 ? hlo : hhi) >> ((u * EPV) & 31)) & GM;
    if (r.mrow) d |= ~(mw[u] >> (v & 31)) & GM;
#pragma unroll
    for (int e = 0; e < EPV; e++) y[u * EPV + e] = Elem<Tin>::get(raw[u], e) * r.invT;
    if (d) {
#pragma unroll
      for (int e = 0; e < EPV; e++) y[u * EPV + e] = (d & (1u << e)) ? ninf : y[u * EPV + e];
    }
#pragma unroll
    for (int e = 0; e < EPV; e++) mx = fmaxf(mx, y[u * EPV + e]);
  }
  return mx;
}

// An order key T with at least k allowed elements of key >= T in the tile:
// the larger of (max over waves of the wave's k-th largest thread maximum)
// and (min over waves of the wave's ceil(k / waves)-th largest thread
// maximum), read from each wave's sorted thread maxima.  mx: this thread's
// maximum y.  Ends with a barrier.
__device__ __forceinline__ uint32_t first_threshold(float mx, int k, uint32_t* thr_w) {
  const uint32_t key = mx > -__builtin_inff() ? tg_key(mx) : 0u;
  const uint32_t srt = wave_sort_desc(key);  // lane i: the (i+1)-th largest
  const uint32_t tk = __shfl(srt, k - 1, 64);
  const uint32_t tj = __shfl(srt, (k + NWB - 1) / NWB - 1, 64);
  const int w = threadIdx.x >> 6;
  if (lane_id() == 0) {
    thr_w[w] = tk;
    thr_w[NWB + w] = tj;
  }
  __syncthreads();
  uint32_t hi = 0, lo = 0xFFFFFFFFu;
#pragma unroll
  for (int i = 0; i < NWB; i++) {
    hi = thr_w[i] > hi ? thr_w[i] : hi;
    lo = thr_w[NWB + i] < lo ? thr_w[NWB + i] : lo;
  }
  return hi > lo ? hi : lo;
}

// Smallest y whose key is at least the key part of composite threshold thr
// (-FLT_MAX when that admits every allowed value).
__device__ __forceinline__ float thr_value(u64 thr) {
  const uint32_t tk = (uint32_t)(thr >> 32);
  const uint32_t kmin = 0x00800000u;  // key of -FLT_MAX
  return tk <= kmin ? -3.40282347e38f : tg_unkey(tk);
}

// Candidate buffer: ES slots per thread for its tile elements, slot-major
// (slot q of thread t at q * BS + t), a compact region of HCAP entries for
// history table slots, and the compacted candidates (CCAP + 16 pad).  Tile candidates (y >= tf; tf is the value of a
// threshold whose low, id part is 1, so this is the composite test for any
// id) are written as (y bits << 32 | id) pairs and turned into composite
// keys by their thread afterwards; unused slots hold 0.  Returns this
// thread's number of tile candidates (more than ES: overflow).
constexpr int ES = 8;
constexpr int HCAP = 512;
constexpr int CCAP = K64_CAP;  // compacted candidates (rank selection input), + 16 pad entries
static_assert(ES * BS + HCAP + CCAP + 16 == K64_CAND_ENTRIES, "candidate buffer");

template <int EPT, int EPV>
__device__ __forceinline__ int emit_lane_slots(u64* cand, const float (&y)[EPT], float tf, int t0) {
  const int idb = t0 + (int)threadIdx.x * EPV;
  u64* my = cand + threadIdx.x;
  int pos = 0;
#pragma unroll
  for (int j = 0; j < EPT; j++)
    if (y[j] >= tf) {
      if (pos < ES) my[pos * BS] = ((u64)tg_f2u(y[j]) << 32) | (uint32_t)(idb + (j / EPV) * BS * EPV + (j % EPV));
      pos++;
    }
#pragma unroll
  for (int q = 0; q < ES; q++) {
    if (q >= pos) {
      my[q * BS] = 0ull;
    } else {
      const u64 e = my[q * BS];
      my[q * BS] = comp_key(tg_key(tg_u2f((uint32_t)(e >> 32))), (int)(uint32_t)e);
    }
  }
  return pos;
}

// cmp[0, n) holds unique composites (published by a barrier; room for 16
// pad entries).  Writes the min(n, k) largest to top[rank] (rank 0 = the
// largest).  The rank of an entry is the number of entries above it; P
// adjacent threads (P a power of two, P * n <= BS where possible) each count
// over one segment of the buffer with 16-byte broadcast reads and sum with
// lane shuffles.  Ends with a barrier.
struct alignas(16) u64x2 {
  u64 x, y;
};

__device__ __forceinline__ void rank_into(u64* cmp, u64* top, int n, int k) {
  int P = 1;
  while (P < 8 && n * P * 2 <= BS) P <<= 1;
  const int seg = (n + 2 * P - 1) / (2 * P) * 2;  // even, seg * P >= n
  for (int i = n + (int)threadIdx.x; i < seg * P; i += BS) cmp[i] = 0ull;  // never above a key
  __syncthreads();
  const int groups = n * P;
  for (int t0 = 0; t0 < groups; t0 += BS) {
    const int t = t0 + (int)threadIdx.x;
    const bool act = t < groups;
    const int i = act ? t / P : 0, part = act ? t % P : 0;
    const u64 x = cmp[i];
    int rk = 0;
    if (act) {
      const u64x2* q = (const u64x2*)(cmp + part * seg);
#pragma unroll 4
      for (int j = 0; j < seg / 2; j++) {
        const u64x2 e = q[j];
        rk += (e.x > x) + (e.y > x);
      }
    }
    for (int d = 1; d < P; d <<= 1) rk += __shfl_xor(rk, d, 64);
    if (act && part == 0 && rk < k) top[rk] = x;
  }
  __syncthreads();
}

// Calls f(x) for every candidate composite x of this thread, re-reading the
// tile (the overflow path: a rolled loop keeps registers free).
template <typename Tin, class F>
__device__ __forceinline__ void each_cand(const Row& r, bool has_hist, const uint32_t* bitmap, const Tin* rowp,
                                          int t0, float tf, const u64* hcomp, int TS, u64 thr, F f) {
  constexpr int EPV = TileK<Tin>::EPV;
#pragma unroll 1
  for (int j = 0; j < TileK<Tin>::EPT; j++) {
    const int id = id_of<EPV>(t0, j);
    if (id >= r.v1) continue;
    if (has_hist && ((bitmap[2 * threadIdx.x + (j >> 5)] >> (j & 31)) & 1u)) continue;
    const float yy = Elem<Tin>::scalar(rowp, id) * r.invT;
    if (yy >= tf && mask_allows(r, id)) f(comp_key(tg_key(yy), id));
  }
  for (int i = threadIdx.x; i < TS; i += BS)
    if (hcomp[i] >= thr) f(hcomp[i]);
}

// Tree merge of the waves' sorted top-64 lists (lane i = rank i) held in
// tops[w]: after it, wave 0 returns the top 64 of their union, sorted.
// Called by all waves; ends with a barrier; only wave 0's result counts.
__device__ __forceinline__ u64 merge_waves(u64 acc, u64 (*tops)[64]) {
  const int w = threadIdx.x >> 6, lane = lane_id();
  tops[w][lane] = acc;
  __syncthreads();
#pragma unroll
  for (int step = 1; step < NWB; step <<= 1) {
    if ((w & (2 * step - 1)) == 0 && w + step < NWB) {
      acc = wave_merge_top64(acc, tops[w + step][lane]);
      tops[w][lane] = acc;
    }
    __syncthreads();
  }
  return acc;
}

// Row finish by one wave; x: lane i holds the row's i-th kept composite
// (descending), n of them (n <= k <= 64).
__device__ __forceinline__ void wave_finish_row(const SampleArgs& a, const Row& r, u64 x, int n) {
  const int lane = lane_id();
  const int b = r.b;
  if (r.mode == 1 && n > 0) {
    wave_finalize(a, r, x, n);
    return;
  }
  // greedy (the top entry) or no allowed token
  const int id = n > 0 ? comp_id(__shfl(x, 0, 64)) : -1;
  if (lane == 0) {
    a.out[b] = id;
    if (r.mode == 0) write_row_diag(a, b, id >= 0, id >= 0, 0, 0, id);
    else write_row_diag(a, b, 0, 0, 0, 0, -1);
  }
  if (a.dbg.kept_ids) {
    int32_t* kid = a.dbg.kept_ids + (long long)b * a.dbg.kept_cap;
    for (int i = lane; i < a.dbg.kept_cap; i += 64) kid[i] = (i == 0) ? id : -1;
  }
  if (a.dbg.kept_probs) {
    float* kp = a.dbg.kept_probs + (long long)b * a.dbg.kept_cap;
    for (int i = lane; i < a.dbg.kept_cap; i += 64) kp[i] = (i == 0 && id >= 0) ? 1.0f : 0.0f;
  }
}

template <typename Tin>
__global__ __launch_bounds__(BS) void k64_kernel(SampleArgs a) {
  using TL = TileK<Tin>;
  TGS_DYN_SMEM(smem);
  __shared__ uint32_t thr_w[2 * NWB];
  __shared__ u64 tops[NWB][64];
  __shared__ unsigned nbuf, nhist, nhc;
  __shared__ int ovf;
  __shared__ int last_s;
  __shared__ BlockScratch bs;
  int2* hash = (int2*)(smem + a.off_hash);
  uint32_t* bitmap = (uint32_t*)(smem + a.off_bitmap);
  u64* cand = (u64*)(smem + a.off_cand);
  const int w = threadIdx.x >> 6, lane = lane_id();

  const int b = blockIdx.x / a.S, c = blockIdx.x % a.S;
  if (b >= a.B) return;
  const int v0 = c * a.L, v1 = min(a.V, v0 + a.L);
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;

  // one round trip for the history ids, the tile and the row's parameters
  // (history ids first: a wave's loads return in order)
  const int* hrow = a.hist ? a.hist + (long long)b * a.hist_cap : nullptr;
  const int hid0 = (hrow && (int)threadIdx.x < a.hist_cap) ? hrow[threadIdx.x] : -1;
  const int hid1 = (hrow && (int)threadIdx.x + BS < a.hist_cap) ? hrow[threadIdx.x + BS] : -1;
  uint4 raw[TL::U];
  load_data<Tin>(rowp, v0, v1, a.aligned, a.whole_vec, raw);
  const tgs_row_params p = a.params[b];
  const float ub = a.u[b];
  const int hl = a.hist_len ? a.hist_len[b] : a.hist_cap;

  Row r;
  const bool valid = row_setup_from(a, b, c, p, ub, hl, r);
  if (!valid || outside_hint(a, r) || r.mode == 2) {
    if (c == 0 && threadIdx.x == 0) {
      a.out[b] = valid ? -3 : -2;  // -3: row outside the launch hint
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    return;
  }
  const int k = r.mode == 0 ? 1 : r.k;
  r.v0 = v0;
  r.v1 = v1;
  float* post = a.dbg.post_logits ? a.dbg.post_logits + (long long)b * a.V : nullptr;
  uint32_t mw[TL::U];
  if (r.mrow) load_mask<Tin>(r, v0, mw);

  if (threadIdx.x == 0) {
    nbuf = 0;
    nhist = 0;
    nhc = 0;
    ovf = 0;
  }
  // history: id -> count table, and per thread a 64-bit mask of its
  // elements that are history ids (two words per thread; bitmap[2t + h])
  if (r.use_pen) {
    for (int i = threadIdx.x; i < a.TS; i += BS) hash[i] = make_int2(-1, 0);
    for (int i = threadIdx.x; i < BITMAP_WORDS; i += BS) bitmap[i] = 0u;
    __syncthreads();
    unsigned mine = 0;
    for (int j = threadIdx.x; j < r.H; j += BS) {
      const int id = j == (int)threadIdx.x ? hid0 : j == (int)threadIdx.x + BS ? hid1 : r.hrow[j];
      if (id < v0 || id >= v1) continue;
      hash_insert(hash, a.TS, a.ts_shift, id);
      const int loc = id - v0;                              // < TileK::SIZE
      const int u = loc / (BS * TL::EPV), rr = loc % (BS * TL::EPV);
      const int t = rr / TL::EPV, el = u * TL::EPV + rr % TL::EPV;  // owner thread, its element
      atomicOr(&bitmap[2 * t + (el >> 5)], 1u << (el & 31));
      mine++;
    }
    if (mine) atomicAdd(&nhist, mine);
  }
  __syncthreads();
  const bool has_hist = r.use_pen && nhist > 0;
  u64 hb = 0;
  if (has_hist) hb = ((u64)bitmap[2 * threadIdx.x + 1] << 32) | bitmap[2 * threadIdx.x];

  // history slots: their logits are fetched now (an L2 hit: the tile was
  // just read) and penalised after the threshold
  const int TS = has_hist ? a.TS : 0;
  constexpr int PRE = 4;
  float zs[PRE];
#pragma unroll
  for (int q = 0; q < PRE; q++) {
    const int i = (int)threadIdx.x + q * BS;
    zs[q] = 0.0f;
    if (i < TS && hash[i].x >= 0) zs[q] = Elem<Tin>::scalar(rowp, hash[i].x);
  }

  // the chunk is one tile (L <= TileK::SIZE)
  float y[TL::EPT];
  const float mx = (!r.mrow && !has_hist) ? values_plain<Tin>(r, raw, y)
                                          : values_general<Tin>(r, hb, v0, raw, mw, y);
  if (post) {
#pragma unroll
    for (int j = 0; j < TL::EPT; j++) {
      const int id = id_of<TL::EPV>(v0, j);
      if (id < v1) post[id] = y[j] > -__builtin_inff() ? y[j] : -__builtin_inff();
    }
  }
  // candidates are >= thr; thr >= 1 keeps empty history slots (composite 0)
  // out, every allowed composite is far above it
  const u64 thr = ((u64)first_threshold(mx, k, thr_w) << 32) | 1ull;
  const float tf = thr_value(thr);
  // history slots: penalised value, mask, composite (0 if not allowed or
  // empty), written over the slot (each slot is read and written by one
  // thread; the table is not probed again)
  u64* hcomp = (u64*)hash;
#pragma unroll
  for (int q = 0; q < PRE; q++) {
    const int i = (int)threadIdx.x + q * BS;
    if (i < TS) {
      const int2 e = hash[i];
      u64 x = 0ull;
      if (e.x >= 0) {
        const float yy = penalise(zs[q], e.y, r) * r.invT;
        const bool ok = yy > -__builtin_inff() && mask_allows(r, e.x);
        if (ok) x = comp_key(tg_key(yy), e.x);
        if (post) post[e.x] = ok ? yy : -__builtin_inff();
      }
      hcomp[i] = x;
    }
  }
  for (int i = (int)threadIdx.x + PRE * BS; i < TS; i += BS) {
    const int2 e = hash[i];
    u64 x = 0ull;
    if (e.x >= 0) {
      const float yy = penalise(Elem<Tin>::scalar(rowp, e.x), e.y, r) * r.invT;
      const bool ok = yy > -__builtin_inff() && mask_allows(r, e.x);
      if (ok) x = comp_key(tg_key(yy), e.x);
      if (post) post[e.x] = ok ? yy : -__builtin_inff();
    }
    hcomp[i] = x;
  }
  // tile candidates into this thread's slots, history candidates into the
  // compact region
  u64* hreg = cand + ES * BS;
  u64* cmp = hreg + HCAP;
  const int mine_c = emit_lane_slots<TL::EPT, TL::EPV>(cand, y, tf, v0);
  for (int i = threadIdx.x; i < TS; i += BS)
    if (hcomp[i] >= thr) {
      const unsigned pp = atomicAdd(&nhc, 1u);
      if (pp < (unsigned)HCAP) hreg[pp] = hcomp[i];
    }
  if (mine_c > ES) ovf = 1;
  __syncthreads();
  if (!ovf && nhc <= (unsigned)HCAP) {
    // compact: a wave prefix sum of the per-thread counts, one LDS atomic
    // per wave, then the history entries
    const unsigned incl = wave_incl_scan((unsigned)mine_c);
    unsigned wb = 0;
    if (lane == 63 && incl) wb = atomicAdd(&nbuf, incl);
    unsigned pos = __shfl(wb, 63, 64) + incl - (unsigned)mine_c;
#pragma unroll
    for (int q = 0; q < ES; q++)
      if (q < mine_c && pos + q < (unsigned)CCAP) cmp[pos + q] = cand[q * BS + threadIdx.x];
    __syncthreads();
    const unsigned ne = nbuf, nh = nhc;
    for (unsigned i = threadIdx.x; i < nh; i += BS)
      if (ne + i < (unsigned)CCAP) cmp[ne + i] = hreg[i];
    if (ne + nh > (unsigned)CCAP) ovf = 1;
    __syncthreads();
    if (threadIdx.x == 0) nbuf = ne + nh;
  }
  __syncthreads();
  if (ovf || nhc > (unsigned)HCAP) {
    // more candidates than the slots hold (ties, or a skewed tile): the
    // exact k-th composite among them, then exactly the k candidates >= it
    auto en = [&](auto f) { each_cand<Tin>(r, has_hist, bitmap, rowp, v0, tf, hcomp, TS, thr, f); };
    const u64 T = block_select_kth<u64, 64, BS>(en, (unsigned)k, bs);
    __syncthreads();
    if (threadIdx.x == 0) nbuf = 0;
    __syncthreads();
    int c2 = 0;
    en([&](u64 x) { c2 += x >= T ? 1 : 0; });
    unsigned p2 = c2 ? atomicAdd(&nbuf, (unsigned)c2) : 0u;
    en([&](u64 x) {
      if (x >= T) cmp[p2++] = x;
    });
    __syncthreads();
  }
  // the chunk's top k, sorted, by ranks
  const int nc = (int)nbuf;
  rank_into(cmp, tops[0], nc, k);
  const int n = nc < k ? nc : k;
  const u64 acc = lane < n ? tops[0][lane] : 0ull;

  if (a.S == 1) {
    if (w == 0) wave_finish_row(a, r, lane < n ? acc : 0ull, n);
    return;
  }
  // publish the chunk's list; the last workgroup of the row merges
  if (w == 0) {
    const u64 x = lane < n ? acc : 0ull;
    __hip_atomic_store(a.ws + ((long long)b * a.S + c) * KM + lane, x, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the list is written through before it is counted
    unsigned prev = 0;
    if (lane == 0)
      prev = __hip_atomic_fetch_add(a.cnt + (long long)b * K64_CNT_STRIDE, 1u, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0, 64);
    if (lane == 0) last_s = prev == (unsigned)(a.S - 1);
  }
  __syncthreads();
  if (!last_s) return;

  // last arrival: merge the S sorted, zero-padded lists
  const u64* lists = a.ws + (long long)b * a.S * KM;
  u64 racc = 0ull;
  for (int cc = w; cc < a.S; cc += NWB) {
    const u64 x = __hip_atomic_load(lists + (long long)cc * KM + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    racc = cc == w ? x : wave_merge_top64(racc, x);
  }
  racc = merge_waves(racc, tops);
  if (w == 0) {
    const int nr = __popcll(__ballot(racc != 0ull));
    const int nk = nr < k ? nr : k;
    wave_finish_row(a, r, lane < nk ? racc : 0ull, nk);
    if (lane == 0)
      __hip_atomic_store(a.cnt + (long long)b * K64_CNT_STRIDE, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace k64

hipError_t launch_k64(const SampleArgs& a, int dtype, size_t lds, hipStream_t st) {
  const dim3 g(a.B * a.S), blk(K64_NT);
  if (dtype == 1) hipLaunchKernelGGL(k64::k64_kernel<uint16_t>, g, blk, lds, st, a);
  else hipLaunchKernelGGL(k64::k64_kernel<float>, g, blk, lds, st, a);
  return hipGetLastError();
}

hipError_t set_k64_lds_limit(size_t bytes) {
  const void* fns[] = {(const void*)k64::k64_kernel<float>, (const void*)k64::k64_kernel<uint16_t>};
  hipError_t e = hipSuccess;
  for (const void* f : fns) {
    hipError_t e2 = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e2 != hipSuccess) e = e2;
  }
  return e;
}

}  // namespace tgs
