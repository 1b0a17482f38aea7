// tgs_k64.hip -- one fused kernel for batches whose rows are greedy or sample
// with 1 <= top_k <= 64 (the launch's batch hint promises it).
//
// Workgroup (b, c) of K64_NT = 256 threads (4 waves) owns chunk c of row b:
// S chunks per row, each one tile of at most 16384 ids (64 per thread:
// sixteen 16-byte vectors of fp32 or eight of bf16).
//
// Loads.  At entry a thread requests everything it reads: four history ids,
// the tile and (with a mask table) the mask word of each of its vectors; the
// row's parameters come through the scalar cache.  In the vector variant
// every load is issued unconditionally (addresses clamped into the chunk,
// values past its end replaced afterwards), so the same number of loads is
// in flight on every path and each use waits for exactly the loads it needs:
// the history counts are built while the tile streams in, and the values of
// a vector are computed as soon as it arrives.
//
// History.  The row's history ids that fall in the chunk are counted in LDS
// (a 16-bit count per id of the tile, two per word) and marked in a bitmap
// of the tile by owner thread.  The value pass leaves marked elements out
// (-inf); the thread whose insertion of an id came first (its producer)
// loads that id's logit once, penalises it and adds it to its wave's
// candidates, so history ids cost one lane each, not a pass over the tile.
//
// Candidates.  Every wave sorts its threads' maxima (bitonic, in registers);
// the k-th and ceil(k/4)-th entries of all waves give a threshold T with at
// least k elements of the tile at or above it.  Each wave stages the vectors
// whose maximum reaches T (placed by ballot prefix counts), tests their
// elements one per lane, sorts its candidates in registers (64 at a time),
// and wave 0 merges the four waves' top 64.  A wave with more candidates
// than its staging holds (ties, skewed tiles) sends the workgroup down an
// exact path: radix selection of the k-th composite, then ranking of the k
// candidates at or above it.
//
// Rows split over S > 1 chunks.  Each workgroup counts itself in the row's
// arrival counter at entry (a relaxed device atomic issued with the loads).
// The workgroup that arrives last merges the row: every other workgroup of
// the row has started by then and will store its chunk's sorted list with
// agent-coherent stores (written through past the per-XCD L2s, which are not
// coherent with each other) without waiting for anything, so the merging
// workgroup polls those lists with agent-coherent loads until no entry holds
// the empty marker, merges them with its own, finishes the row (masses,
// top-p, draw) and resets the lists to the marker and the counter to zero
// for the next call.  The wait is bounded: one that runs out (it cannot
// while every workgroup runs) writes id -4 for the row.  No fence is issued:
// on this part an agent-scope release or acquire fence writes back or
// invalidates the whole L2 of the XCD.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace k64 {

constexpr int BS = K64_NT;
constexpr int NWB = BS / 64;
constexpr int KM = 64;                   // largest top_k served
constexpr int NHID = K64_MAX_HIST / BS;  // history ids per thread
constexpr u64 EMPTY = ~0ull;             // list entry not written yet: above every composite
constexpr int SPIN_LIMIT = 1 << 18;      // polls of one list before the wait gives up
constexpr int KM_PRE = 2;                // lists per wave the merging workgroup requests early (S <= 8)

// A tile gives every thread 64 elements: 16384 ids.
template <typename Tin>
struct TileK {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int EPT = 64;
  static constexpr int U = EPT / EPV;  // 16-byte vectors per thread
  static constexpr int SIZE = BS * EPT;
  static_assert(SIZE == K64_TILE, "tile size");
};
constexpr int BITMAP_WORDS = K64_BITMAP_WORDS;  // one bit per id of a tile
constexpr int CNT_WORDS = K64_TILE / 2;         // 16-bit history counts, two per word
static_assert(BITMAP_WORDS * 32 == K64_TILE, "bitmap covers a tile");

// id of element j of this thread in the tile starting at t0
template <int EPV>
__device__ __forceinline__ int id_of(int t0, int j) {
  return t0 + ((j / EPV) * BS + (int)threadIdx.x) * EPV + (j % EPV);
}

// The tile's 16-byte vectors.  VEC: the chunk holds whole vectors (rows
// aligned, chunk ends multiples of the vector); a vector past the chunk end
// is read at the chunk's last vector and replaced by NaN in the value pass.
// Otherwise ids at or past v1 read as NaN here (checked loads).
template <typename Tin, bool VEC, int U = TileK<Tin>::U>
__device__ __forceinline__ void load_tile(const Tin* rowp, int t0, int v1, bool aligned, uint4 (&raw)[U]) {
  constexpr int EPV = TileK<Tin>::EPV;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int v = t0 + (u * BS + (int)threadIdx.x) * EPV;
    if constexpr (VEC) raw[u] = tg_load_nt(rowp + (v < v1 ? v : v1 - EPV));
    else raw[u] = load_vec<Tin>(rowp, v, v1, aligned);
  }
}

// Mask word of each vector (unconditional; rows without a mask read a valid
// table row and ignore it).
template <typename Tin, int U = TileK<Tin>::U>
__device__ __forceinline__ void load_mask(const uint32_t* mrow, int t0, int v1, uint32_t (&mw)[U]) {
  constexpr int EPV = TileK<Tin>::EPV;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int v = t0 + (u * BS + (int)threadIdx.x) * EPV;
    mw[u] = mrow[(v < v1 ? v : v1 - 1) >> 5];
  }
}

// Logit of element e of a vector; NaN for a vector past the chunk end.
template <typename Tin>
__device__ __forceinline__ float elem_z(const uint4& raw, int e, bool past) {
  const float z = Elem<Tin>::get(raw, e);
  return past ? __builtin_nanf("") : z;
}

// y = logit / T over a tile with no mask and no history ids.  NaN and -inf
// (ids past the chunk end read as NaN) never pass a threshold test or raise
// a maximum.  vm[u]: the maximum of vector u.  Returns the thread maximum.
// tail: vectors past the chunk end were read at a clamped address.
template <typename Tin, int U = TileK<Tin>::U>
__device__ __forceinline__ float values_plain(const Row& r, int t0, bool tail, const uint4 (&raw)[U],
                                              float (&y)[TileK<Tin>::EPT], float (&vm)[U]) {
  constexpr int EPV = TileK<Tin>::EPV;
  float mx = -__builtin_inff();
#pragma unroll
  for (int u = 0; u < U; u++) {
    const bool past = tail && t0 + (u * BS + (int)threadIdx.x) * EPV >= r.v1;
    float m = -__builtin_inff();
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      y[u * EPV + e] = row_y(r, elem_z<Tin>(raw[u], e, past));
      m = fmaxf(m, y[u * EPV + e]);
    }
    vm[u] = m;
    mx = fmaxf(mx, m);
  }
  return mx;
}

// The same with the grammar mask and the history ids of the tile left out
// (-inf; their penalised values join the candidates separately).  hb: this
// thread's history elements, bit j for element j.
template <typename Tin, bool MASK, int U = TileK<Tin>::U>
__device__ __forceinline__ float values_general(const Row& r, u64 hb, int t0, bool tail, const uint4 (&raw)[U],
                                                const uint32_t (&mw)[U], float (&y)[TileK<Tin>::EPT],
                                                float (&vm)[U]) {
  constexpr int EPV = TileK<Tin>::EPV;
  constexpr uint32_t GM = (1u << EPV) - 1u;
  const float ninf = -__builtin_inff();
  const uint32_t hlo = (uint32_t)hb, hhi = (uint32_t)(hb >> 32);
  float mx = ninf;
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int v = t0 + (u * BS + (int)threadIdx.x) * EPV;
    const bool past = tail && v >= r.v1;
    uint32_t d = ((u * EPV < 32 ? hlo : hhi) >> ((u * EPV) & 31)) & GM;
    if constexpr (MASK) {
      if (r.mrow) d |= ~(mw[u] >> (v & 31)) & GM;
    }
#pragma unroll
    for (int e = 0; e < EPV; e++) y[u * EPV + e] = row_y(r, elem_z<Tin>(raw[u], e, past));
    if (d) {
#pragma unroll
      for (int e = 0; e < EPV; e++) y[u * EPV + e] = ((d >> e) & 1u) ? ninf : y[u * EPV + e];
    }
    float m = ninf;
#pragma unroll
    for (int e = 0; e < EPV; e++) m = fmaxf(m, y[u * EPV + e]);
    vm[u] = m;
    mx = fmaxf(mx, m);
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
  const uint32_t tk = __builtin_amdgcn_readlane(srt, k - 1);
  const uint32_t tj = __builtin_amdgcn_readlane(srt, (k + NWB - 1) / NWB - 1);
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

// Candidate buffer (LDS).  Common path, per wave: up to VCAP candidate
// vectors (a vector whose maximum reaches the threshold value tf; tf is the
// value of a threshold whose low, id part is 1, so y >= tf is the composite
// test for any id) as EPV floats each plus the id of their first element,
// and a list of up to LCAP candidate composites.  The exact path (a wave
// with more candidate vectors or candidates than that) reuses the same
// memory for up to CCAP compacted candidates (+ 16 pad entries for the rank
// counting).
constexpr int VCAP = 64;
constexpr int LCAP = 256;
constexpr int CCAP = K64_CAP;
static_assert(CCAP + 16 <= K64_CAND_ENTRIES, "candidate buffer");

template <typename Tin>
struct Stage {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int VALS = NWB * VCAP * EPV;  // floats
  static constexpr int IDS = NWB * VCAP;         // ints
  static constexpr int BYTES = VALS * 4 + IDS * 4 + NWB * LCAP * 8;
  static_assert(BYTES <= K64_CAND_ENTRIES * 8, "stage fits the candidate buffer");
};

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
// tile (the exact path: a rolled loop keeps registers free).
template <typename Tin, bool MASK, class F>
__device__ __forceinline__ void each_cand(const Row& r, bool has_hist, const uint32_t* bitmap, const uint32_t* hcnt,
                                          const Tin* rowp, int t0, float tf, F f) {
  constexpr int EPV = TileK<Tin>::EPV;
#pragma unroll 1
  for (int j = 0; j < TileK<Tin>::EPT; j++) {
    const int id = id_of<EPV>(t0, j);
    if (id >= r.v1) continue;
    const float z = Elem<Tin>::scalar(rowp, id);
    float yy = row_y(r, z);
    if (has_hist && ((bitmap[2 * threadIdx.x + (j >> 5)] >> (j & 31)) & 1u)) {
      const int loc = id - t0;
      yy = row_y(r, penalise(z, (int)((hcnt[loc >> 1] >> ((loc & 1) * 16)) & 0xFFFFu), r));
    }
    if (yy >= tf && (!MASK || mask_allows(r, id))) f(comp_key(tg_key(yy), id));
  }
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

template <typename Tin, bool VEC, bool MASK>
__global__ __launch_bounds__(BS) void k64_kernel(SampleArgs a) {
  using TL = TileK<Tin>;
  TGS_DYN_SMEM(smem);
  __shared__ uint32_t thr_w[2 * NWB];
  __shared__ u64 tops[NWB][64];
  __shared__ u64 own[64];
  __shared__ unsigned nbuf, nhist;
  __shared__ int ovf, elect, tmo;
  __shared__ BlockScratch bs;
  uint32_t* hcnt = (uint32_t*)(smem + a.off_hash);
  uint32_t* bitmap = (uint32_t*)(smem + a.off_bitmap);
  u64* cand = (u64*)(smem + a.off_cand);
  const int w = threadIdx.x >> 6, lane = lane_id();

  const int b = blockIdx.x / a.S, c = blockIdx.x % a.S;
  if (b >= a.B) return;
  const int v0 = c * a.L, v1 = min(a.V, v0 + a.L);
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  const bool full = v0 + TL::SIZE <= v1;
  unsigned* cnt = a.cnt + (long long)b * K64_CNT_STRIDE;

  // everything read first, in one round trip, in the order it is needed (a
  // wave's loads return in order): the row's parameters, its history length
  // and ids, the arrival count, the tile
  const tgs_row_params p = a.params[b];
  const float ub = a.u[b];
  const int hlr = *(a.hist_len ? a.hist_len + b : (const int*)a.params);
  const bool hv = a.hist && a.hist_cap > 0;
  const int* hp = hv ? a.hist + (long long)b * a.hist_cap : (const int*)a.params;
  const int hlast = hv ? a.hist_cap - 1 : 0;
  int hid[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) {
    const int j = (int)threadIdx.x + q * BS;
    hid[q] = hp[j < hlast ? j : hlast];
  }
  unsigned arrived = 0;
  if (a.S > 1 && threadIdx.x == 0)
    arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint4 raw[TL::U];
  load_tile<Tin, VEC>(rowp, v0, v1, a.aligned, raw);
  const int hl = a.hist_len ? hlr : a.hist_cap;

  Row r;
  const bool valid = row_setup_from(a, b, c, p, ub, hl, r);
  if (!valid || outside_hint(a, r) || r.mode == 2) {
    if (c == 0 && threadIdx.x == 0) {
      a.out[b] = valid ? -3 : -2;  // -3: row outside the launch hint
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    // the row's last arrival clears the counter (no lists were written)
    if (a.S > 1 && threadIdx.x == 0 && arrived == (unsigned)(a.S - 1))
      __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  const int k = r.mode == 0 ? 1 : r.k;
  r.v0 = v0;
  r.v1 = v1;
  float* post = a.dbg.post_logits ? a.dbg.post_logits + (long long)b * a.V : nullptr;
  uint32_t mw[TL::U];
  if constexpr (MASK) load_mask<Tin>(r.mrow ? r.mrow : a.mask_table, v0, v1, mw);

  if (threadIdx.x == 0) {
    nbuf = 0;
    nhist = 0;
    ovf = 0;
    tmo = 0;
  }
  // history: count of every id of the tile, and per thread a 64-bit mask of
  // its elements that are history ids (two words per thread; bitmap[2t + h]);
  // the first insertion of each id makes its thread the id's producer
  bool prod[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) prod[q] = false;
  if (r.use_pen) {
#pragma unroll
    for (int i = 0; i < CNT_WORDS / 4 / BS; i++) ((uint4*)hcnt)[threadIdx.x + i * BS] = make_uint4(0u, 0u, 0u, 0u);
    for (int i = threadIdx.x; i < BITMAP_WORDS; i += BS) bitmap[i] = 0u;
    __syncthreads();
    unsigned mine = 0;
#pragma unroll
    for (int q = 0; q < NHID; q++) {
      const int id = hid[q];
      if ((int)threadIdx.x + q * BS < r.H && id >= v0 && id < v1) {
        const int loc = id - v0;                              // < TileK::SIZE
        const unsigned old = atomicAdd(&hcnt[loc >> 1], 1u << ((loc & 1) * 16));
        prod[q] = ((old >> ((loc & 1) * 16)) & 0xFFFFu) == 0u;  // first occurrence: this id's producer
        const int u = loc / (BS * TL::EPV), rr = loc % (BS * TL::EPV);
        const int t = rr / TL::EPV, el = u * TL::EPV + rr % TL::EPV;  // owner thread, its element
        atomicOr(&bitmap[2 * t + (el >> 5)], 1u << (el & 31));
        mine++;
      }
    }
    if (mine) atomicAdd(&nhist, mine);
  }
  __syncthreads();
  const bool has_hist = r.use_pen && nhist > 0;
  u64 hb = 0;
  if (has_hist) hb = ((u64)bitmap[2 * threadIdx.x + 1] << 32) | bitmap[2 * threadIdx.x];
  // producers' logits (and mask words): one load per history id of this
  // thread, issued behind the tile and first needed after the threshold;
  // the loads are unconditional (others read id v0) to keep the count fixed
  float zq[NHID];
  uint32_t mq[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) {
    const int id = prod[q] ? hid[q] : v0;
    zq[q] = Elem<Tin>::scalar(rowp, id);
    if constexpr (MASK) mq[q] = (r.mrow ? r.mrow : a.mask_table)[id >> 5];
  }

  // values, per-vector maxima, thread maximum
  float y[TL::EPT];
  float vm[TL::U];
  const bool tail = VEC && !full;
  bool gen = has_hist;
  if constexpr (MASK) gen = gen || r.mrow != nullptr;
  const float mx = gen ? values_general<Tin, MASK>(r, hb, v0, tail, raw, mw, y, vm)
                       : values_plain<Tin>(r, v0, tail, raw, y, vm);
  if (post) {
#pragma unroll
    for (int j = 0; j < TL::EPT; j++) {
      const int id = id_of<TL::EPV>(v0, j);
      if (id < v1) post[id] = y[j] > -__builtin_inff() ? y[j] : -__builtin_inff();
    }
  }
  // candidates are >= thr; every allowed composite is far above the id part
  if (threadIdx.x == 0) elect = a.S > 1 && arrived == (unsigned)(a.S - 1);  // published by the next barrier
  const u64 thr = ((u64)first_threshold(mx, k, thr_w) << 32) | 1ull;
  // the merging workgroup requests the other chunks' lists now, so that
  // their load overlaps its own candidate work; entries still empty are
  // polled again at the merge
  u64 pre[KM_PRE];
  const bool elected = elect != 0;
  u64* lists = a.lists + (long long)b * a.S * KM;
#pragma unroll
  for (int q = 0; q < KM_PRE; q++) {
    const int cc = w + q * NWB;
    pre[q] = (elected && cc < a.S && cc != c)
                 ? __hip_atomic_load(lists + (long long)cc * KM + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                 : EMPTY;
  }
  const float tf = thr_value(thr);

  // Every element >= tf, wave by wave.  A vector whose maximum reaches tf
  // is staged whole (lanes placed by a ballot prefix count); the staged
  // elements are then tested one per lane and listed with the wave's history
  // candidates; the list is sorted in registers and the four waves' top 64
  // are merged.
  using ST = Stage<Tin>;
  float* svals = (float*)cand + w * VCAP * TL::EPV;
  int* sids = (int*)((float*)cand + ST::VALS) + w * VCAP;
  u64* wl = (u64*)((int*)((float*)cand + ST::VALS) + ST::IDS) + w * LCAP;
  unsigned nv = 0;  // candidate vectors of the wave
#pragma unroll
  for (int u = 0; u < TL::U; u++) {
    const bool pv = vm[u] >= tf;
    const u64 bal = __ballot(pv);
    if (bal) {
      const unsigned sl = nv + lanes_below(bal);
      if (pv && sl < (unsigned)VCAP) {
        uint4* dst = (uint4*)(svals + sl * TL::EPV);
#pragma unroll
        for (int q = 0; q < TL::EPV / 4; q++)
          dst[q] = make_uint4(tg_f2u(y[u * TL::EPV + 4 * q]), tg_f2u(y[u * TL::EPV + 4 * q + 1]),
                              tg_f2u(y[u * TL::EPV + 4 * q + 2]), tg_f2u(y[u * TL::EPV + 4 * q + 3]));
        sids[sl] = id_of<TL::EPV>(v0, u * TL::EPV);
      }
      nv += (unsigned)__popcll(bal);
    }
  }
  wave_lds_sync();
  const unsigned nel = (nv < (unsigned)VCAP ? nv : (unsigned)VCAP) * TL::EPV;
  unsigned nl = 0;  // list entries of the wave
  for (unsigned e0 = 0; e0 < nel; e0 += 64) {
    const unsigned e = e0 + (unsigned)lane;
    const float yy = e < nel ? svals[e] : -__builtin_inff();
    const bool pc = yy >= tf;
    const u64 bal = __ballot(pc);
    const unsigned sl = nl + lanes_below(bal);
    if (pc && sl < (unsigned)LCAP) wl[sl] = comp_key(tg_key(yy), sids[e / TL::EPV] + (int)(e % TL::EPV));
    nl += (unsigned)__popcll(bal);
  }
  // history candidates: the penalised logit of each history id of the
  // chunk, computed by its producer (counts are final since the barrier)
#pragma unroll
  for (int q = 0; q < NHID; q++) {
    u64 x = 0ull;
    if (prod[q]) {
      const int id = hid[q], loc = id - v0;
      const int hc = (int)((hcnt[loc >> 1] >> ((loc & 1) * 16)) & 0xFFFFu);
      const float yy = row_y(r, penalise(zq[q], hc, r));
      bool ok = yy > -__builtin_inff();
      if constexpr (MASK) ok = ok && (!r.mrow || ((mq[q] >> (id & 31)) & 1u));
      if (post) post[id] = ok ? yy : -__builtin_inff();
      if (ok) x = comp_key(tg_key(yy), id);
    }
    const bool pc = x >= thr;
    const u64 bal = __ballot(pc);
    const unsigned sl = nl + lanes_below(bal);
    if (pc && sl < (unsigned)LCAP) wl[sl] = x;
    nl += (unsigned)__popcll(bal);
  }
  wave_lds_sync();
  const bool wovf = nv > (unsigned)VCAP || nl > (unsigned)LCAP;
  // the wave's top 64: its list sorted 64 at a time, merged
  u64 xs = 0ull;
  if (!wovf) {
#pragma unroll 1
    for (unsigned c0 = 0; c0 < nl; c0 += 64) {
      u64 x = c0 + (unsigned)lane < nl ? wl[c0 + lane] : 0ull;
      x = wave_sort_desc(x);
      xs = c0 == 0 ? x : wave_merge_top64(xs, x);
    }
  }
  if (wovf && lane == 0) ovf = 1;
  tops[w][lane] = xs;
  __syncthreads();
  u64 acc = 0ull;  // wave 0: the chunk's top 64 candidates, sorted
  if (!ovf) {
    if (w == 0) {
      acc = xs;
#pragma unroll
      for (int i = 1; i < NWB; i++) acc = wave_merge_top64(acc, tops[i][lane]);
    }
  } else {
    // the exact k-th composite among all candidates, then exactly the k
    // candidates >= it, ranked
    u64* cmp = cand;
    auto en = [&](auto f) { each_cand<Tin, MASK>(r, has_hist, bitmap, hcnt, rowp, v0, tf, f); };
    const u64 T = block_select_kth<u64, 64, BS>(en, (unsigned)k, bs);
    __syncthreads();
    int c2 = 0;
    en([&](u64 x) { c2 += x >= T ? 1 : 0; });
    unsigned p2 = c2 ? atomicAdd(&nbuf, (unsigned)c2) : 0u;
    en([&](u64 x) {
      if (x >= T) cmp[p2++] = x;
    });
    __syncthreads();
    const int nc = (int)nbuf;
    rank_into(cmp, tops[0], nc, k);
    const int n = nc < k ? nc : k;
    acc = lane < n ? tops[0][lane] : 0ull;
  }

  if (a.S == 1) {
    if (w == 0) {
      const int n = __popcll(__ballot(acc != 0ull));
      const int nk = n < k ? n : k;
      wave_finish_row(a, r, lane < nk ? acc : 0ull, nk);
    }
    return;
  }
  if (!elected) {
    // publish the chunk's list for the row's merging workgroup
    if (w == 0) __hip_atomic_store(lists + (long long)c * KM + lane, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }

  // the row's last arrival: merge the S sorted, zero-padded lists
  if (w == 0) own[lane] = acc;
  __syncthreads();
  u64 racc = 0ull;
  bool first = true;
  for (int cc = w; cc < a.S; cc += NWB) {
    u64 x;
    if (cc == c) {
      x = own[lane];
    } else {
      const u64* lp = lists + (long long)cc * KM + lane;
      const int q = (cc - w) / NWB;
      x = q < KM_PRE ? pre[q] : __hip_atomic_load(lp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int spins = 0;
      while (__ballot(x == EMPTY) != 0ull) {
        if (++spins > SPIN_LIMIT) {
          if (lane == 0) tmo = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(2);
        x = __hip_atomic_load(lp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
    racc = first ? x : wave_merge_top64(racc, x);
    first = false;
  }
  racc = merge_waves(racc, tops);
  if (w == 0) {
    if (tmo) {
      if (lane == 0) {
        a.out[b] = -4;
        write_row_diag(a, b, 0, 0, 0, 0, -1);
      }
    } else {
      const int nr = __popcll(__ballot(racc != 0ull));
      const int nk = nr < k ? nr : k;
      wave_finish_row(a, r, lane < nk ? racc : 0ull, nk);
    }
  }
  // ready for the next call: lists empty, counter zero
  for (int cc = w; cc < a.S; cc += NWB)
    if (cc != c) __hip_atomic_store(lists + (long long)cc * KM + lane, EMPTY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

template <typename Tin>
hipError_t launch_t(const SampleArgs& a, size_t lds, hipStream_t st) {
  const dim3 g(a.B * a.S), blk(K64_NT);
  const bool vec = a.whole_vec != 0, mask = a.mask_table != nullptr && a.n_states > 0;
  if (vec && mask) hipLaunchKernelGGL((k64_kernel<Tin, true, true>), g, blk, lds, st, a);
  else if (vec) hipLaunchKernelGGL((k64_kernel<Tin, true, false>), g, blk, lds, st, a);
  else if (mask) hipLaunchKernelGGL((k64_kernel<Tin, false, true>), g, blk, lds, st, a);
  else hipLaunchKernelGGL((k64_kernel<Tin, false, false>), g, blk, lds, st, a);
  return hipGetLastError();
}

}  // namespace k64

hipError_t launch_k64(const SampleArgs& a, int dtype, size_t lds, hipStream_t st) {
  return dtype == 1 ? k64::launch_t<uint16_t>(a, lds, st) : k64::launch_t<float>(a, lds, st);
}

hipError_t set_k64_lds_limit(size_t bytes) {
  const void* fns[] = {
      (const void*)k64::k64_kernel<float, true, true>,     (const void*)k64::k64_kernel<float, true, false>,
      (const void*)k64::k64_kernel<float, false, true>,    (const void*)k64::k64_kernel<float, false, false>,
      (const void*)k64::k64_kernel<uint16_t, true, true>,  (const void*)k64::k64_kernel<uint16_t, true, false>,
      (const void*)k64::k64_kernel<uint16_t, false, true>, (const void*)k64::k64_kernel<uint16_t, false, false>,
  };
  hipError_t e = hipSuccess;
  for (const void* f : fns) {
    hipError_t e2 = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e2 != hipSuccess) e = e2;
  }
  return e;
}

}  // namespace tgs
