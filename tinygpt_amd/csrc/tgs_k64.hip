// tgs_k64.hip -- one fused kernel for batches whose rows are greedy or sample
// with 1 <= top_k <= 64 (the launch's batch hint promises it).
//
// Workgroup (b, c) of K64_NT threads owns chunk c of row b: S chunks per
// row, each at most K64_NT * K64_NVT sixteen-byte vectors (thread t holding
// chunk vectors t, t + K64_NT, ...).  Rows that fit one chunk of
// K64_SMALL_NT threads (one wave) run on that instantiation instead.
// Everything a thread reads is requested at entry: the row's parameters,
// its history ids, its vectors and (with a mask table) their mask words, so
// the whole chunk is in flight at once.  Under a full-chip stream the
// chunk's data lands in one burst near the end of the stream, so the steps
// after it are kept short:
//   1. Vector maxima and thread maxima of the raw logits (ids the mask
//      forbids and ids past the chunk left out).
//   2. A bound B: a raw logit such that at least k distinct ids of the row
//      that are neither masked nor history ids lie at or above it.
//        * The chunk's own bound: for m = 1 .. waves, the m-th largest over
//          waves of the wave's ceil(k / m)-th largest thread maximum (m
//          waves hold that many at or above it each), read from one wave
//          sort each.  In the sort a thread whose maximum lies in a vector
//          holding a history id of the chunk takes the lowest key (in the
//          one-wave instantiation a thread's key is the largest of its ids
//          that are neither history ids nor masked).
//        * Split rows whose whole grid is resident at once (the launch's
//          exchange flag) also share a row-wide bound: each wave publishes
//          the kq largest keys of its sort, tagged with the call's epoch,
//          and wave 0 polls the row's S * waves * kq keys and takes their
//          k-th largest (to 20 key bits).  Those keys belong to
//          distinct threads, so k of them are k distinct qualifying ids.
//          The row's k-th largest thread maximum lies close to its k-th
//          largest logit, so a chunk collects a few ids instead of its own
//          top k.  A wave whose poll does not complete in the launch's
//          key_spins rounds keeps the chunk's bound.
//      A wave collects from cz, 16 representable values below its bound
//      (the larger of the two).
//   3. Every vector whose maximum reaches cz is staged whole in its wave's
//      LDS list (a one-wave row of at most two vectors per thread skips the
//      staging: each lane tests its own vectors in step 4).
//   4. One staged vector per lane: every allowed element whose raw logit z
//      reaches cz becomes a composite of z and its id, history ids left to
//      their producers (the lane whose insertion created the id's LDS hash
//      slot loads its logit at entry and appends its penalised value), the
//      mask test, and a wave-aggregated append to the LDS candidate buffer.
//      The temperature applies to candidates only: each composite becomes
//      one of the canonical y = z / T (correctly rounded, tg_div_t) before
//      any selection in the chunk, or, in an unsorted published list, in
//      the merging workgroup (at most 64 divisions per row).
//   5. An id left out is not a history id and has z < cz, so its y is at
//      most yc = cz / T, while the k ids behind the bound have y at least
//      y(B): when y(B) > yc, every id of the row's top k that lies in this
//      chunk is a candidate.  When the quotients collide (a temperature so
//      small that z / T overflows, say) or a wave stages more vectors than
//      its list holds, the chunk's exact top k comes from a radix selection
//      over the chunk read again from memory instead.
//
// Rows split over S > 1 chunks.  Each workgroup reads the row's epoch word
// at entry (the call's tag is that word plus one) and counts itself in the
// row's arrival counter (a relaxed device atomic) once its keys are out:
// the last wave issues it after its history logits have landed, so that
// no wait for a load queues behind it.  The workgroup that arrives last
// merges the row: every other workgroup of the row is past its loads by
// then.  The others publish their list with
// agent-coherent stores (written through past the per-XCD L2s, which are
// not coherent with each other) and exit: their candidates unsorted when
// the row-wide bound left at most 64, else their sorted top k, then a count
// word tagged with the epoch.  A list entry is the candidate's composite
// with the epoch's low 14 bits between its key and its 18-bit id, so that
// entries of one call order as their composites.  The merging workgroup
// polls the count words, then the entries (until each holds the call's
// tag), sorts the union in one wave when it holds at most 64 entries (a
// tree of wave merges otherwise), finishes the row (masses, top-p, draw),
// clears the entries it read (0: not written), and resets the counter and
// advances the epoch for the next call.  Stale entries of an earlier call
// carry another tag.  Every wait is bounded: a merge wait that runs out
// after the launch's merge_spins polls (it cannot while every workgroup
// runs; tests force it from the host) writes id -4 for the row, and lists
// published after it stay behind under their call's tag.  No fence is
// issued: on this part an agent-scope release or acquire fence writes back
// or invalidates the whole L2 of the XCD.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace k64 {

constexpr int NVT = K64_NVT;         // 16-byte vectors per thread
constexpr int KM = 64;               // largest top_k served; longest published list
constexpr int CAP = K64_CAP;         // candidate buffer entries
constexpr u64 EMPTY = 0ull;          // list entry not written: a published entry never is 0
constexpr uint32_t KEY_MIN = 0x00800000u;  // key of -FLT_MAX: below it only -inf and NaN
constexpr uint32_t TAG_MASK = 0x3FFFu;     // epoch bits a list entry carries
constexpr uint32_t ID_MASK = 0x3FFFFu;     // list entry id bits (V <= 2^18)

template <typename Tin, int NTT>
struct Geo {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int NW = NTT / 64;
  static constexpr int CH = NTT * NVT * EPV;  // ids of a chunk at most
  static constexpr int MAXH = NTT >= K64_NT ? K64_MAX_HIST : K64_SMALL_MAX_HIST;  // longest history
  static constexpr int NHID = (MAXH + NTT - 1) / NTT;  // history ids per thread (its share of the row's)
  static constexpr uint32_t GM = (1u << EPV) - 1u;
};

// The static LDS of one workgroup.
template <int NW>
struct Shared {
  u64 slots[NW][64];      // wave lists (merges, the ranked top k)
  uint4 svec[NW][64];     // per wave: vectors whose maximum reaches the collection threshold
  int sidx[NW][64];       // their vector index in the chunk (with a mask: forbidden-id bits above bit 16)
  u64 own[64];            // merging workgroup: its own sorted top k
  uint32_t wkey[NW][NW];  // [m - 1][wave]: the wave's ceil(k / m)-th largest thread maximum key
  unsigned nbuf;          // candidates appended
  int elect, tmo, spill;
  int lcnt[K64_MAX_SPLIT];     // merging workgroup: entries of each chunk's list
  int lsort[K64_MAX_SPLIT];    // 1: that list is sorted
  int lz[K64_MAX_SPLIT];       // 1: that list holds logits before the temperature
  int fast;                    // merging workgroup: entries laid out in mer (-1: the merge tree)
  uint32_t rkey;               // the row-wide bound key (0: none)
  alignas(16) u64 mer[66];     // merging workgroup: the lists end to end (+ a pad entry)
  BlockScratch bs;
};

// The chunk's history bits in LDS, packed per thread: the EPV bits of chunk
// vector j (bit e for its element e) lie in the HPW words of thread
// j mod NTT, at bit (j div NTT) * EPV, so that a thread reads the bits of
// all its vectors with one load.
template <typename Tin, int NTT>
struct HBits {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int HPW = NVT * EPV / 32;  // words per thread
  static constexpr int WORDS = NTT * HPW;
  static constexpr uint32_t GM = (1u << EPV) - 1u;
  __device__ static int word(int j) { return (j % NTT) * HPW + (j / NTT) * EPV / 32; }
  __device__ static int shift(int j) { return (j / NTT) * EPV % 32; }
  __device__ static uint32_t of(const uint32_t* bits, int j) { return (bits[word(j)] >> shift(j)) & GM; }
};

// max over m = 1 .. NW of the m-th largest of wkey[m - 1][0, NW) (NW one,
// four or eight), in every lane.  Four waves: lanes 4 (m - 1) + i load
// wkey[m - 1][i], each group of four lanes sorts itself descending
// (comparators (0,1) (2,3), (0,2) (1,3), (1,2) as lane exchanges), and lane
// 5 (m - 1) then holds the m-th largest of group m - 1 (the exchanges are
// DPP quad permutes).  Eight waves: lanes 8 (m - 1) + i load wkey[m - 1][i],
// each lane counts the entries of its group that rank above it (larger, or
// equal at a lower index), and the lane of rank m - 1 in group m - 1 offers
// its key to a wave maximum.
template <int NW>
__device__ __forceinline__ uint32_t bound_key(const uint32_t (*wkey)[NW], int lane) {
  static_assert(NW == 1 || NW == 4 || NW == 8, "waves per workgroup");
  if constexpr (NW == 1) {
    return wkey[0][0];
  } else if constexpr (NW == 8) {
    const int g = lane >> 3, i = lane & 7;
    const uint32_t x = wkey[g][i];
    int rank = 0;
#pragma unroll
    for (int d = 1; d < 8; d++) {
      const int j = (i + d) & 7;
      const uint32_t y = __shfl(x, (g << 3) | j, 64);
      rank += (y > x || (y == x && j < i)) ? 1 : 0;
    }
    return wave_max(rank == g ? x : 0u);
  } else {
    const int pos = lane & 3;
    uint32_t x = wkey[(lane >> 2) & 3][pos];
    uint32_t y = xor_lane32<1>(x);
    x = (pos & 1) ? min(x, y) : max(x, y);
    y = xor_lane32<2>(x);
    x = (pos & 2) ? min(x, y) : max(x, y);
    y = __builtin_amdgcn_update_dpp(0u, x, 0x1B, 0xF, 0xF, false);  // quad_perm [3,2,1,0]: lane ^ 3
    x = pos == 1 ? max(x, y) : pos == 2 ? min(x, y) : x;
    return max(max(readlane_u32(x, 0), readlane_u32(x, 5)), max(readlane_u32(x, 10), readlane_u32(x, 15)));
  }
}

// The row's published keys as one wave polls them: lane l holds keys l,
// l + 64, ... (NJ = ceil(nk / 64) <= 4 of them); keys of this call carry its
// epoch ep in their high word.  Every slot is loaded (a slot past nk reads
// the last key) and slots past nk count as current keys of value 0, so that
// the loops carry no branch (a branch per slot made each step of the k-th
// key search a chain of scalar branches).
template <int NJ>
struct RowKeys {
  u64 e[NJ];
};
template <int NJ>
__device__ __forceinline__ void keys_issue(RowKeys<NJ>& K, const u64* keys, int nk) {
  const int lane = lane_id();
#pragma unroll
  for (int j = 0; j < NJ; j++) {
    const int i = lane + 64 * j;
    K.e[j] = __hip_atomic_load(keys + (i < nk ? i : nk - 1), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}
template <int NJ>
__device__ __forceinline__ bool keys_current(const RowKeys<NJ>& K, int nk, uint32_t ep) {
  const int lane = lane_id();
  bool stale = false;
#pragma unroll
  for (int j = 0; j < NJ; j++) stale = stale || (lane + 64 * j < nk && (uint32_t)(K.e[j] >> 32) != ep);
  return __ballot(stale) == 0ull;
}

// One wave polls the row's nk keys K (requested earlier by the caller)
// until every key holds the call's tag; false when max_spins polls did not
// see every key.
__device__ __forceinline__ bool keys_wait(RowKeys<4>& K, const u64* keys, int nk, uint32_t ep, int max_spins) {
  for (int spins = 0;; spins++) {
    if (keys_current(K, nk, ep)) return true;
    if (spins >= max_spins) return false;
    __builtin_amdgcn_s_sleep(1);
    keys_issue(K, keys, nk);
  }
}

// The k-th largest of the row's keys (NJ = ceil(nk / 64) slots per lane), to
// 20 bits: the largest multiple of 2^12 that at least k of them reach, one
// wave-wide count per bit (2^-11 of relative slack).
template <int NJ>
__device__ __forceinline__ uint32_t keys_kth(const RowKeys<4>& K, int nk, int k) {
  const int lane = lane_id();
  uint32_t kk[NJ];
#pragma unroll
  for (int j = 0; j < NJ; j++) kk[j] = lane + 64 * j < nk ? (uint32_t)K.e[j] : 0u;
  uint32_t X = 0u;
#pragma unroll
  for (int bit = 31; bit >= 12; bit--) {
    const uint32_t t = X | (1u << bit);
    int n = 0;
#pragma unroll
    for (int j = 0; j < NJ; j++) n += __popcll(__ballot(kk[j] >= t));
    X = n >= k ? t : X;
  }
  return X;
}

// The candidate buffer holds composites of the logits before the
// temperature (z, or the penalised z of a history id): z / T is monotone in
// z, so the collection threshold applies to them exactly, and only a
// selection needs the canonical logit's order (distinct z can share one
// y = z / T, whose ties go to the lower id).  y-composite of a z-composite
// (0: none, or y = -inf, which is not allowed).
__device__ __forceinline__ u64 z_to_y(u64 x, const Row& r) {
  if (x == 0ull) return 0ull;
  const float y = row_y(r, tg_unkey((uint32_t)(x >> 32)));
  return y > -__builtin_inff() ? comp_key(tg_key(y), comp_id(x)) : 0ull;
}

// A list entry: composite x with the epoch's low bits between its key and
// its id (entries of one call order as their composites; never 0, since a
// candidate's key is above that of -inf).
__device__ __forceinline__ u64 tag_entry(u64 x, uint32_t ep) {
  const uint32_t id = (uint32_t)comp_id(x);
  return (x & 0xFFFFFFFF00000000ull) | ((u64)(ep & TAG_MASK) << 18) | (u64)(ID_MASK - id);
}
__device__ __forceinline__ bool entry_ok(u64 e, uint32_t ep) {
  return e != EMPTY && (uint32_t)((e >> 18) & TAG_MASK) == (ep & TAG_MASK);
}
__device__ __forceinline__ u64 untag_entry(u64 e) {
  return comp_key((uint32_t)(e >> 32), (int)(ID_MASK - (uint32_t)(e & ID_MASK)));
}

// One list entry of another chunk for each lane with act (entry p of list
// lp), polled until it holds the call's tag (bounded), then cleared for the
// next call.  Returns the composite (0 without act or after a timeout, which
// sets *tmo).
__device__ __forceinline__ u64 take_entry(u64* lp, bool act, uint32_t ep, bool* tmo, int max_spins) {
  u64 e = act ? __hip_atomic_load(lp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : EMPTY;
  int spins = 0;
  while (__ballot(act && !entry_ok(e, ep)) != 0ull) {
    if (++spins > max_spins) {
      *tmo = true;
      break;
    }
    __builtin_amdgcn_s_sleep(1);
    if (act && !entry_ok(e, ep)) e = __hip_atomic_load(lp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  if (!act) return 0ull;
  __hip_atomic_store(lp, EMPTY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return entry_ok(e, ep) ? untag_entry(e) : 0ull;
}

struct alignas(16) u64x2 {
  u64 x, y;
};

// The min(n, k) largest of the unique composites cmp[0, n) (published by a
// barrier; room for 16 pad entries past n) into top[rank], rank 0 the
// largest.  The rank of an entry is the number of entries above it; P
// adjacent threads (P a power of two, P n <= BS where possible) each count
// over one segment of the buffer with 16-byte broadcast reads and sum with
// lane moves.  Ends with a barrier.
template <int BS>
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

// Tree merge of the waves' sorted top-64 lists (lane i = rank i): after it,
// wave 0 holds the top 64 of their union, sorted.  Each slot is written once
// (by its wave, at the level it sends), so one barrier per level suffices.
// Called by all waves; ends with a barrier.
template <int NW, typename T>
__device__ __forceinline__ T merge_waves(T acc, T (*slots)[64]) {
  const int w = threadIdx.x >> 6, lane = lane_id();
#pragma unroll
  for (int step = 1; step < NW; step <<= 1) {
    if ((w & (2 * step - 1)) == step) slots[w][lane] = acc;
    __syncthreads();
    if ((w & (2 * step - 1)) == 0) acc = wave_merge_top64(acc, slots[w + step][lane]);
  }
  __syncthreads();
  return acc;
}

// The sorted top k of buf[0, n) (n <= CAP, unique composites) in wave 0's
// lanes: ranking for short buffers (n^2 <= 16 NTT: one round, at most 8
// entry pairs read per thread), wave sorts of 64-entry slices merged as a
// tree otherwise (ranking 256 entries in one wave took 13 us).  Ends with a
// barrier.
template <int NTT>
__device__ __forceinline__ u64 select_top(u64* buf, int n, int k, u64 (*slots)[64]) {
  constexpr int NW = NTT / 64;
  const int w = threadIdx.x >> 6, lane = lane_id();
  if (n * n <= 16 * NTT) {
    u64* top = slots[NW - 1];
    if (threadIdx.x < 64) top[threadIdx.x] = 0ull;
    __syncthreads();
    rank_into<NTT>(buf, top, n, k);
    return lane < k ? top[lane] : 0ull;
  }
  u64 acc = 0ull;
  bool first = true;
  for (int s0 = w * 64; s0 < n; s0 += NTT) {
    u64 x = s0 + lane < n ? buf[s0 + lane] : 0ull;
    x = wave_sort_desc(x);
    acc = first ? x : wave_merge_top64(acc, x);
    first = false;
  }
  acc = merge_waves<NW>(acc, slots);
  return lane < k ? acc : 0ull;
}

// Wave-aggregated append of up to N composites per lane (entry q when
// ok[q]) to the LDS buffer: one LDS atomic per wave on the counter, slots
// from a wave prefix sum of the lanes' counts.
template <int N>
__device__ __forceinline__ void append_n(const u64 (&x)[N], const bool (&ok)[N], u64* buf, unsigned* count) {
  unsigned cnt = 0;
#pragma unroll
  for (int q = 0; q < N; q++) cnt += ok[q] ? 1u : 0u;
  const unsigned incl = wave_incl_scan(cnt);
  const unsigned tot = readlane_u32(incl, 63);
  if (tot == 0u) return;
  unsigned base = 0;
  if (lane_id() == 0) base = atomicAdd(count, tot);
  base = readlane_u32(base, 0);
  unsigned sl = base + (incl - cnt);
#pragma unroll
  for (int q = 0; q < N; q++)
    if (ok[q]) {
      if (sl < (unsigned)CAP) buf[sl] = x[q];
      sl++;
    }
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

// Finish of a merged row (wave 0): x sorted descending, id -4 after a wait
// that gave up.
__device__ __forceinline__ void finish_merged(const SampleArgs& a, const Row& r, u64 x, int k, bool tmo) {
  if (tmo) {
    if (lane_id() == 0) {
      a.out[r.b] = -4;
      write_row_diag(a, r.b, 0, 0, 0, 0, -1);
    }
    return;
  }
  const int n = __popcll(__ballot(x != 0ull));
  wave_finish_row(a, r, lane_id() < k ? x : 0ull, n < k ? n : k);
}

// Calls f(composite) for every allowed, non-history id of the chunk (and
// each history composite of this thread), reading the chunk again from
// memory in a rolled loop (the exact path keeps the registers free).
template <typename Tin, int NTT, int NHID, class F>
__device__ __forceinline__ void each_allowed(const SampleArgs& a, const Row& r, const Tin* rowp, int nvec, bool pen,
                                             const uint32_t* bitmap, bool masked, const u64 (&hcomp)[NHID], F f) {
  constexpr int EPV = Elem<Tin>::EPV;
#pragma unroll 1
  for (int j = threadIdx.x; j < nvec; j += NTT) {
    const int vid = r.v0 + j * EPV;
    const uint4 v = load_vec<Tin>(rowp, vid, r.v1, a.aligned);
    const uint32_t hw = pen ? HBits<Tin, NTT>::of(bitmap, j) : 0u;
    const uint32_t mwv = masked ? r.mrow[vid >> 5] >> (vid & 31) : 0xFFFFFFFFu;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      if (((hw >> e) & 1u) || !((mwv >> e) & 1u)) continue;
      const float y = row_y(r, Elem<Tin>::get(v, e));  // ids past the chunk read as NaN
      if (y > -__builtin_inff()) f(comp_key(tg_key(y), vid + e));
    }
  }
#pragma unroll
  for (int q = 0; q < NHID; q++)
    if (hcomp[q] != 0ull) f(hcomp[q]);
}

// The exact path: the k-th composite of the chunk by radix selection, the k
// entries at or above it (composites are unique), ranked into wave 0.
template <typename Tin, int NTT, bool MASK, int NHID>
__device__ __forceinline__ u64 exact_top(const SampleArgs& a, const Row& r, const Tin* rowp, int nvec, bool pen,
                                      const uint32_t* bitmap, bool masked, const u64 (&hcomp)[NHID], int k, u64* buf,
                                      unsigned* nbuf, u64 (*slots)[64], BlockScratch& bs) {
  auto en = [&](auto f) { each_allowed<Tin, NTT, NHID>(a, r, rowp, nvec, pen, bitmap, masked, hcomp, f); };
  const u64 T = block_select_kth<u64, 64, NTT>(en, (unsigned)k, bs);
  if (threadIdx.x == 0) *nbuf = 0;
  __syncthreads();
  en([&](u64 x) {
    if (x >= T) buf[atomicAdd(nbuf, 1u)] = x;  // exactly k entries
  });
  __syncthreads();
  const int n2 = (int)*nbuf;
  return select_top<NTT>(buf, n2 < CAP ? n2 : CAP, k, slots);
}

// Debug output: the canonical logit of every non-history id of the chunk
// (history ids are written by their producers), -inf where not allowed.
template <typename Tin, int NTT>
__device__ __forceinline__ void post_logits_chunk(const SampleArgs& a, const Row& r, const Tin* rowp, int nvec, bool pen,
                                               const uint32_t* bitmap, bool masked) {
  constexpr int EPV = Elem<Tin>::EPV;
  float* post = a.dbg.post_logits + (long long)r.b * a.V;
#pragma unroll 1
  for (int j = threadIdx.x; j < nvec; j += NTT) {
    const int vid = r.v0 + j * EPV;
    const uint4 v = load_vec<Tin>(rowp, vid, r.v1, a.aligned);
    const uint32_t hw = pen ? HBits<Tin, NTT>::of(bitmap, j) : 0u;
    const uint32_t mwv = masked ? r.mrow[vid >> 5] >> (vid & 31) : 0xFFFFFFFFu;
#pragma unroll
    for (int e = 0; e < EPV; e++) {
      const int id = vid + e;
      if (id >= r.v1 || ((hw >> e) & 1u)) continue;
      const float y = row_y(r, Elem<Tin>::get(v, e));
      post[id] = (((mwv >> e) & 1u) && y > -__builtin_inff()) ? y : -__builtin_inff();
    }
  }
}

// Vector i of this thread's share of the chunk [v0, v1) (nvec vectors).
template <typename Tin, int NTT, bool VEC>
__device__ __forceinline__ uint4 chunk_vec(const Tin* rowp, int i, int v0, int v1, int nvec, bool aligned) {
  constexpr int EPV = Elem<Tin>::EPV;
  const int j = (int)threadIdx.x + i * NTT;
  if constexpr (VEC) {
    return tg_load_nt(rowp + v0 + (j < nvec ? j : nvec - 1) * EPV);
  } else if (i * NTT < nvec) {  // whole-workgroup test: vectors wholly past the chunk are not read
    return load_vec<Tin>(rowp, v0 + j * EPV, v1, aligned);
  } else {
    return make_uint4(0x7FC00000u, 0x7FC00000u, 0x7FC00000u, 0x7FC00000u);  // NaN: never counted
  }
}

template <typename Tin, int NTT, bool VEC, bool MASK>
__global__ __launch_bounds__(NTT) void k64_kernel(SampleArgs a) {
  using G = Geo<Tin, NTT>;
  constexpr int EPV = G::EPV, NW = G::NW, NHID = G::NHID;
  constexpr uint32_t GM = G::GM;
  constexpr int SCAP = 64;   // staged vectors per wave
  TGS_DYN_SMEM(smem);
  TGS_STATIC_SMEM(Shared<NW>, sh);
  int2* hash = (int2*)(smem + a.off_hash);
  uint32_t* bitmap = (uint32_t*)(smem + a.off_bitmap);
  u64* buf = (u64*)(smem + a.off_cand);
  const int w = threadIdx.x >> 6, lane = lane_id();

  // workgroup -> (row, chunk); with xmap (B a multiple of 8) the S chunks of
  // a row are workgroups g = x (mod 8), which the dispatcher places on one
  // XCD when it deals workgroups out to the eight XCDs in turn
  int b, c;
  if (a.xmap) {
    const int g = (int)blockIdx.x, j = g >> 3;
    b = (g & 7) + 8 * (j / a.S);
    c = j % a.S;
  } else {
    b = (int)blockIdx.x / a.S;
    c = (int)blockIdx.x % a.S;
  }
  if (b >= a.B) return;
  const int v0 = c * a.L, v1 = min(a.V, v0 + a.L);  // a.L is a multiple of EPV
  const int nvec = (v1 - v0 + EPV - 1) / EPV;
  const int nfull = nvec / NTT;  // vectors every thread holds
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  unsigned* cnt = a.cnt + (long long)b * K64_CNT_STRIDE;

  // ---- everything read first, in the order it is needed (a wave's loads
  // return in order): the row's parameters, its epoch word, its history
  // length and ids, the chunk; with a mask table, its words between the
  // chunk's first NPRE vectors and the rest
  const tgs_row_params p = a.params[b];
  const float ub = a.u[b];
  const int hlr = *(a.hist_len ? a.hist_len + b : (const int*)a.params);
  const bool hv = a.hist && a.hist_cap > 0;
  const int* hp = hv ? a.hist + (long long)b * a.hist_cap : (const int*)a.params;
  const int hlast = hv ? a.hist_cap - 1 : 0;
  // the row's epoch word (every wave reads it: one request per wave)
  const uint32_t epw = __hip_atomic_load(cnt + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  int hid[NHID];  // this thread's share of the history: entries threadIdx.x + q NTT
#pragma unroll
  for (int q = 0; q < NHID; q++) {
    const int j = (int)threadIdx.x + q * NTT;
    hid[q] = hp[j < hlast ? j : hlast];
  }
  // Whole vectors: one unconditional load each (a vector past the chunk
  // reads its last one again and is left out in step 1).  With no branch
  // among the loads the compiler waits exactly for the history ids, so the
  // history hash is built while the chunk streams in.
  uint4 raw[NVT];
  // The mask words depend on the parameters, whose first request takes
  // about a microsecond to return: the chunk's first NPRE vectors go out
  // before the words, so that the chunk's stream does not wait for the
  // parameters, and the rest after them, so that the words do not queue
  // behind the whole chunk (step 1 takes the vectors in order, each with its
  // word).  A state out of range reads the first row, and the row is
  // rejected below.
  constexpr int NPRE = MASK ? K64_MASK_PRE : 0;
  static_assert(NPRE >= 0 && NPRE <= NVT, "chunk vectors before the mask words");
#pragma unroll
  for (int i = 0; i < NPRE; i++) raw[i] = chunk_vec<Tin, NTT, VEC>(rowp, i, v0, v1, nvec, a.aligned);
  uint32_t mw[MASK ? NVT : 1];
  const uint32_t* mrow_any = a.mask_table;  // the row's mask row (the first row for a state out of range)
  if constexpr (MASK) {
    const uint32_t* mrow = a.mask_table;
    if (p.mask_state >= 0 && p.mask_state < a.n_states) mrow += (long long)p.mask_state * a.mask_words;
    mrow_any = mrow;
#pragma unroll
    for (int i = 0; i < NVT; i++) {
      const int j = (int)threadIdx.x + i * NTT;
      mw[i] = mrow[(v0 + (j < nvec ? j : nvec - 1) * EPV) >> 5];
    }
  }
#pragma unroll
  for (int i = NPRE; i < NVT; i++) raw[i] = chunk_vec<Tin, NTT, VEC>(rowp, i, v0, v1, nvec, a.aligned);
  const int hl = a.hist_len ? hlr : a.hist_cap;

  Row r;
  const bool valid = row_setup_from(a, b, c, p, ub, hl, r);
  if (!valid || outside_hint(a, r) || r.mode == 2) {
    if (c == 0 && threadIdx.x == 0) {
      a.out[b] = valid ? -3 : -2;  // -3: row outside the launch hint
      write_row_diag(a, b, 0, 0, 0, 0, -1);
    }
    return;  // no workgroup of the row counts itself in or publishes anything
  }
  const int k = r.mode == 0 ? 1 : r.k;
  r.v0 = v0;
  r.v1 = v1;
  const bool masked = MASK && r.mrow != nullptr;

  // ---- history, first its bits: each id of the chunk marked in the packed
  // history bits (HBits), all the bound needs.  The id -> count table is
  // cleared here and filled once the bound's keys have gone out.
  if (threadIdx.x == 0) {
    sh.nbuf = 0;
    sh.tmo = 0;
    sh.spill = 0;
  }
  const bool pen = r.use_pen;
  using HB = HBits<Tin, NTT>;
  constexpr int HPW = HB::HPW;
  if (pen) {
    for (int i = threadIdx.x; i < a.TS; i += NTT) hash[i] = make_int2(-1, 0);
#pragma unroll
    for (int q = 0; q < HPW; q++) bitmap[threadIdx.x * HPW + q] = 0u;
    __syncthreads();
#pragma unroll
    for (int q = 0; q < NHID; q++) {
      const int id = hid[q];
      if ((int)threadIdx.x + q * NTT < r.H && id >= v0 && id < v1) {
        const int j = (id - v0) / EPV;
        atomicOr(&bitmap[HB::word(j)], 1u << (HB::shift(j) + (id - v0) % EPV));
      }
    }
  }
  __syncthreads();
  int hslot[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) hslot[q] = -1;
  // The logits (and mask words) of this thread's history entries, read now,
  // right behind the chunk, so that they have landed when the penalties are
  // applied after the bound.  Every lane loads (an entry outside the chunk
  // reads the chunk's first id), so that the loads carry no branch: a branch
  // would leave the compiler to wait for them wherever the chunk is waited
  // for.
  float zq[NHID];
  uint32_t mq[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) {
    const int id = hid[q];
    const bool in = (int)threadIdx.x + q * NTT < r.H && id >= v0 && id < v1;
    const int lid = in ? id : v0;
    zq[q] = Elem<Tin>::scalar(rowp, lid);
    mq[q] = 0xFFFFFFFFu;
    if constexpr (MASK) mq[q] = mrow_any[lid >> 5];
  }
  // the history bits of this thread's vectors (vector i at bit i * EPV), one
  // load while the chunk is still in flight
  uint32_t hpk[HPW];
  if (pen) {
    if constexpr (HPW == 2) {
      const uint2 t = *(const uint2*)(bitmap + threadIdx.x * HPW);
      hpk[0] = t.x;
      hpk[1] = t.y;
    } else {
      static_assert(HPW == 4, "history words per thread");
      const uint4 t = *(const uint4*)(bitmap + threadIdx.x * HPW);
      hpk[0] = t.x;
      hpk[1] = t.y;
      hpk[2] = t.z;
      hpk[3] = t.w;
    }
  } else {
#pragma unroll
    for (int q = 0; q < HPW; q++) hpk[q] = 0u;
  }

  // ---- 1. vector maxima and thread maximum of the raw logits (ids the
  // mask forbids and vectors past the chunk left out; history ids included)
  // and the first vector that holds the thread maximum
  float vm[NVT];
  float tm = -__builtin_inff();
  int im = 0;
  uint32_t xpk[MASK ? HPW : 1] = {};  // forbidden-id bits of the thread's vectors (vector i at bit i * EPV)
#pragma unroll
  for (int i = 0; i < NVT; i++) {
    float m;
    if constexpr (MASK) {
      // an id the mask forbids becomes a quiet NaN (its bits ORed with
      // 0xFFC00000, through the sign-extended bit of x), which the maximum
      // ignores: two operations per id instead of a test and a select
      const uint32_t x = masked ? ~(mw[i] >> ((v0 + ((int)threadIdx.x + i * NTT) * EPV) & 31)) : 0u;
      xpk[(i * EPV) >> 5] |= (x & GM) << ((i * EPV) & 31);
      m = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < EPV; e++) {
        const uint32_t off = (uint32_t)((int)(x << (31 - e)) >> 31) & 0xFFC00000u;
        m = fmaxf(m, tg_u2f(tg_f2u(Elem<Tin>::get(raw[i], e)) | off));
      }
    } else {
      m = Elem<Tin>::get(raw[i], 0);
#pragma unroll
      for (int e = 1; e < EPV; e++) m = fmaxf(m, Elem<Tin>::get(raw[i], e));
    }
    if (i >= nfull) m = ((int)threadIdx.x + i * NTT < nvec) ? m : -__builtin_inff();  // vectors past the chunk
    vm[i] = m;
    im = m > tm ? i : im;
    tm = fmaxf(tm, m);
  }

  uint32_t ep;
  // ---- 2. the bound.  A thread whose maximum lies in a vector holding a
  // history id sorts as the lowest key, so every thread maximum behind a
  // bound is an id that is not a history id.  The chunk's bound: for
  // m = 1 .. NW, the m-th largest over waves of the wave's ceil(k / m)-th
  // largest key (m waves hold ceil(k / m) keys at or above it each), all
  // read from one sort per wave.  With the exchange, the wave's kq largest
  // keys go out to the row first.
  {
    uint32_t tk;
    if constexpr (NTT == 64) {
      // one wave: a thread's key is the largest logit of its own ids that
      // are neither history ids nor masked out (with few threads, leaving
      // out every thread whose maximum shares a vector with a history id
      // left a byte-level row with 64 history ids too few keys for a bound,
      // and every id became a candidate)
      float t2 = -__builtin_inff();
#pragma unroll
      for (int i = 0; i < NVT; i++) {
        if (i * NTT >= nvec) break;  // (uniform) no thread holds vector i
        const bool live = i < nfull || (int)threadIdx.x + i * NTT < nvec;
        uint32_t x = 0u;
        if constexpr (MASK) x = masked ? ~(mw[i] >> ((v0 + ((int)threadIdx.x + i * NTT) * EPV) & 31)) & GM : 0u;
#pragma unroll
        for (int e = 0; e < EPV; e++) {
          const int bit = i * EPV + e;
          const bool out = ((hpk[bit >> 5] >> (bit & 31)) & 1u) || ((x >> e) & 1u) || !live;
          t2 = out ? t2 : fmaxf(t2, Elem<Tin>::get(raw[i], e));
        }
      }
      tk = t2 > -__builtin_inff() ? tg_key(t2) : 0u;
    } else {
      uint32_t hw = hpk[0];
#pragma unroll
      for (int q = 1; q < HPW; q++) hw = im * EPV / 32 == q ? hpk[q] : hw;
      const bool hmax = ((hw >> (im * EPV % 32)) & GM) != 0u;
      tk = (tm > -__builtin_inff() && !hmax) ? tg_key(tm) : 0u;
    }
    const uint32_t srt = wave_sort_desc(tk);  // lane i: the (i+1)-th largest
    // the call's tag: never 0 (the exchange memory starts zeroed, and the
    // epoch word never holds ~0)
    ep = epw + 1u;
    if (a.xchg) {
      if (lane < a.kq)
        __hip_atomic_store(a.keys + (long long)b * K64_KEYS + (c * NW + w) * a.kq + lane, ((u64)ep << 32) | srt,
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int m = 1; m <= NW; m++) {
      const uint32_t v = readlane_u32(srt, (k + m - 1) / m - 1);
      if (lane == 0) sh.wkey[m - 1][w] = v;
    }
  }
  // The row's arrival count, issued by the last wave (which polls nothing)
  // once its keys are out: the workgroup whose arrival is the row's last
  // merges it, and every other workgroup of the row is past its loads by
  // then.  Its result is first needed after the collection.  The history
  // logits are taken first, so that no wait for them lands behind the
  // atomic (a wave's memory operations return in order).
  unsigned arrived = 0;
  if (a.S > 1 && w == NW - 1) {
#pragma unroll
    for (int q = 0; q < NHID; q++) asm volatile("" ::"v"(zq[q]), "v"(mq[q]));
    if (lane == 63) arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();  // the table clear and the wave keys
  // ---- history counts: each id of the chunk counted in the LDS hash (its
  // producer is the lane that created its slot)
  if (pen) {
    const unsigned tmask = (unsigned)a.TS - 1u;
#pragma unroll
    for (int q = 0; q < NHID; q++) {
      const int id = hid[q];
      if ((int)threadIdx.x + q * NTT < r.H && id >= v0 && id < v1) {
        unsigned h = hash_slot(id, a.ts_shift);
        for (;;) {  // the table has at least twice as many slots as history entries
          const int old = atomicCAS(&hash[h].x, -1, id);
          if (old == -1 || old == id) {
            atomicAdd(&hash[h].y, 1);
            if (old == -1) hslot[q] = (int)h;
            break;
          }
          h = (h + 1) & tmask;
        }
      }
    }
  }
  uint32_t bkey = bound_key<NW>(sh.wkey, lane);
  if (a.xchg) {
    if (w == 0) {
      // wave 0 polls for the workgroup
      const int nk = a.S * NW * a.kq;
      RowKeys<4> rkeys;
      uint32_t rk = 0u;
      // (a first poll issued as soon as the keys went out measured slower:
      // it mostly returns before the row's other keys are out; issued after
      // the barrier, with the history counts in its shadow, 0.03 us slower)
      keys_issue(rkeys, a.keys + (long long)b * K64_KEYS, nk);
      if (keys_wait(rkeys, a.keys + (long long)b * K64_KEYS, nk, ep, a.key_spins))
        rk = nk <= 64 ? keys_kth<1>(rkeys, nk, k) : nk <= 128 ? keys_kth<2>(rkeys, nk, k) : keys_kth<4>(rkeys, nk, k);
      if (lane == 0) sh.rkey = rk;
    }
    __syncthreads();  // also publishes the table
    const uint32_t rk = sh.rkey;
    bkey = rk > bkey ? rk : bkey;
  } else if (pen) {
    __syncthreads();  // the table
  }
  // the collection threshold: 16 representable values below the bound, so
  // that the ids that set the bound land strictly above its canonical value
  const bool all = bkey < KEY_MIN + 32u;  // no usable bound: collect every allowed id
  const float cz = all ? -__builtin_inff() : tg_unkey(bkey - 16u);
  const float yc = all ? -__builtin_inff() : row_y(r, cz);
  const uint32_t kcz = tg_key(cz);  // z-composites at or above it are candidates
  // quotients that collide at the bound: the exact path
  if (!all && !(row_y(r, tg_unkey(bkey)) > yc) && lane == 0) sh.spill = 1;
  // the producers' composites (their penalised logits; the loads went out
  // before the bound)
  u64 hcomp[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) {
    u64 x = 0ull;
    if (hslot[q] >= 0) {
      const int id = hid[q];
      const float zp = penalise(zq[q], hash[hslot[q]].y, r);
      const bool okm = !masked || ((mq[q] >> (id & 31)) & 1u);
      if (okm && zp > -__builtin_inff()) x = comp_key(tg_key(zp), id);  // (NaN fails the compare)
      if (a.dbg.post_logits) {
        const float y = row_y(r, zp);
        a.dbg.post_logits[(long long)b * a.V + id] = (okm && y > -__builtin_inff()) ? y : -__builtin_inff();
      }
    }
    hcomp[q] = x;
  }

  // ---- 3. collection: the vectors whose maximum reaches cz, staged whole
  // (their bits and their chunk index) in the wave's LDS list.  Each lane
  // marks its own (one bit per vector, plain compares), and the wave's union
  // of those marks skips the empty vector slots with a scalar bit test (a
  // ballot per slot cost more than the staging itself).
  uint32_t pm = 0u;
#pragma unroll
  for (int i = 0; i < NVT; i++)
    pm |= (vm[i] >= cz && vm[i] > -__builtin_inff()) ? (1u << i) : 0u;  // (cz may be -inf)
  const uint32_t PM = wave_or(pm);
  bool direct = false;  // (uniform)
  if constexpr (NTT == 64) {
    // one wave over at most two vectors per thread: each lane tests its own
    // vectors from its registers (no staging round trip through LDS)
    if (nvec <= 2 * NTT) {
      direct = true;
#pragma unroll
      for (int i = 0; i < 2; i++) {
        if (!(PM & (1u << i))) continue;  // uniform
        const int j = (int)threadIdx.x + i * NTT, o = j * EPV;
        const bool pass = ((pm >> i) & 1u) && j < nvec;
        const uint32_t hw = (hpk[(i * EPV) >> 5] >> ((i * EPV) & 31)) & GM;
        uint32_t xm = 0u;
        if constexpr (MASK) xm = masked ? ~(mw[i] >> ((v0 + o) & 31)) & GM : 0u;
        u64 x[EPV];
        bool ok[EPV];
#pragma unroll
        for (int e = 0; e < EPV; e++) {
          const float z = Elem<Tin>::get(raw[i], e);
          ok[e] = pass && z >= cz && z > -__builtin_inff() && !((hw >> e) & 1u) && !((xm >> e) & 1u);
          x[e] = comp_key(tg_key(z), v0 + o + e);
        }
        append_n<EPV>(x, ok, buf, &sh.nbuf);
      }
    }
  }
  if (!direct) {
    unsigned ns = 0;  // staged vectors of the wave (uniform)
#pragma unroll
    for (int i = 0; i < NVT; i++) {
      if (!(PM & (1u << i))) continue;  // uniform
      const bool pass = (pm >> i) & 1u;
      const u64 bal = __ballot(pass);
      const unsigned sl = ns + lanes_below(bal);
      if (pass && sl < (unsigned)SCAP) {
        sh.svec[w][sl] = raw[i];
        // the vector index, with its forbidden-id bits above bit 16
        int sx = (int)threadIdx.x + i * NTT;
        if constexpr (MASK) sx |= (int)(((xpk[(i * EPV) >> 5] >> ((i * EPV) & 31)) & GM) << 16);
        sh.sidx[w][sl] = sx;
      }
      ns += (unsigned)__popcll(bal);
    }
    if (ns > (unsigned)SCAP && lane == 0) sh.spill = 1;
    wave_lds_sync();

    // ---- 4. the staged vectors (one per lane): exact canonical logits,
    // history ids left to their producers, into the candidate buffer
    const unsigned nst = ns < (unsigned)SCAP ? ns : (unsigned)SCAP;
    for (unsigned s0 = 0; s0 < nst; s0 += 64) {
      const unsigned si = s0 + (unsigned)lane;
      u64 x[EPV];
      bool ok[EPV];
      uint4 v = make_uint4(0x7FC00000u, 0x7FC00000u, 0x7FC00000u, 0x7FC00000u);
      int sx = 0;
      if (si < nst) {
        v = sh.svec[w][si];
        sx = sh.sidx[w][si];
      }
      const int j = MASK ? sx & 0xFFFF : sx;
      const int o = j * EPV;
      const uint32_t hw = (pen && si < nst) ? HB::of(bitmap, j) : 0u;
      const uint32_t xm = MASK ? (uint32_t)sx >> 16 : 0u;  // the forbidden-id bits staged with the index
#pragma unroll
      for (int e = 0; e < EPV; e++) {
        const float z = Elem<Tin>::get(v, e);
        ok[e] = si < nst && z >= cz && z > -__builtin_inff() && !((hw >> e) & 1u) && !((xm >> e) & 1u) &&
                j < nvec;
        x[e] = comp_key(tg_key(z), v0 + o + e);
      }
      append_n<EPV>(x, ok, buf, &sh.nbuf);
    }
  }
  {
    bool hok[NHID];
#pragma unroll
    for (int q = 0; q < NHID; q++) hok[q] = hcomp[q] != 0ull && (uint32_t)(hcomp[q] >> 32) >= kcz;
    append_n<NHID>(hcomp, hok, buf, &sh.nbuf);
  }
  if (threadIdx.x == NTT - 1) sh.elect = a.S > 1 && arrived == (unsigned)(a.S - 1);
  __syncthreads();

  // ---- 5. the chunk's list: its candidates as they stand when a split row
  // shares the row-wide bound and they number at most 64, else its sorted
  // top k (from the candidates, or from the exact path)
  const int nb = (int)sh.nbuf;
  const bool exact = sh.spill || nb > CAP;
  const bool raw_list = a.S > 1 && a.xchg && !exact && nb <= KM;
  u64 acc = 0ull;
  if (!raw_list) {
    // a selection orders by the canonical logit: the candidates (and the
    // producers' composites, which the exact path enumerates) become
    // y-composites first
#pragma unroll
    for (int q = 0; q < NHID; q++) hcomp[q] = z_to_y(hcomp[q], r);
    if (!exact) {
      for (int t = threadIdx.x; t < nb; t += NTT) buf[t] = z_to_y(buf[t], r);
      __syncthreads();
      acc = select_top<NTT>(buf, nb, k, sh.slots);
    } else {
      // exact path (rare: quotients that collide, skewed chunks): the k-th
      // composite of the chunk by radix selection over the chunk read again
      // (L2 / MALL hits), then the k entries at or above it
      acc = exact_top<Tin, NTT, MASK>(a, r, rowp, nvec, pen, bitmap, masked, hcomp, k, buf, &sh.nbuf, sh.slots, sh.bs);
    }
  }
  if (a.dbg.post_logits) post_logits_chunk<Tin, NTT>(a, r, rowp, nvec, pen, bitmap, masked);

  // ---- 6. the row
  if (a.S == 1) {
    if (w == 0) {
      const int n = __popcll(__ballot(acc != 0ull));
      wave_finish_row(a, r, acc, n < k ? n : k);
    }
    return;
  }
  u64* lists = a.lists + (long long)b * K64_MAX_SPLIT * KM;
  u64* cw = (u64*)(cnt + K64_CNT_WORDS);  // the row's count words, one per chunk
  if (!sh.elect) {
    // publish the chunk's list (entries, then its count word) and leave
    if (raw_list) {
      for (int t = threadIdx.x; t < nb; t += NTT)
        __hip_atomic_store(lists + (long long)c * KM + t, tag_entry(buf[t], ep), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      if (threadIdx.x == 0)  // 0x200: entries hold logits before the temperature
        __hip_atomic_store(cw + c, ((u64)ep << 32) | 0x200u | (u64)nb, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else if (w == 0) {
      const int n = __popcll(__ballot(acc != 0ull));
      if (lane < n)
        __hip_atomic_store(lists + (long long)c * KM + lane, tag_entry(acc, ep), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
      if (lane == 0)
        __hip_atomic_store(cw + c, ((u64)ep << 32) | 0x100u | (u64)n, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    return;
  }

  // ---- the row's last arrival: its own list stays in LDS.  Wave 0 reads
  // every other chunk's count word and the first E = 128 / S entries of its
  // list in one round of requests (two entries per lane), polled until each
  // count word and each entry below its count holds the call's tag.  When
  // the lists hold at most 64 entries, none beyond its first E, they are
  // laid end to end in LDS and sorted by one wave; otherwise every wave
  // takes part in a tree of wave merges over the lists read again.
  if (w == 0) {
    const int own_n = raw_list ? nb : __popcll(__ballot(acc != 0ull));
    if (!raw_list) sh.own[lane] = acc;
    const int E = 128 / a.S;  // S <= 16: E >= 8
    const bool cl = lane < a.S && lane != c;  // this lane polls list `lane`'s count word
    int ec[2], epo[2];
#pragma unroll
    for (int j = 0; j < 2; j++) {
      const int idx = lane + 64 * j;
      ec[j] = idx < a.S * E ? idx / E : -1;
      epo[j] = idx % E;
      if (ec[j] == c) ec[j] = -1;  // the own list is in LDS
    }
    u64 cwv = cl ? __hip_atomic_load(cw + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : ((u64)ep << 32);
    u64 ent[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
      ent[j] = ec[j] >= 0 ? __hip_atomic_load(lists + (long long)ec[j] * KM + epo[j], __ATOMIC_RELAXED,
                                              __HIP_MEMORY_SCOPE_AGENT)
                          : EMPTY;
    bool tmo = false;
    int ncl = 0;  // lanes below S: that list's entries
    int nce[2] = {0, 0};  // entries of the list of each slot
    for (int spins = 0;; spins++) {
      const bool cok = (uint32_t)(cwv >> 32) == ep;
      ncl = cok ? (int)(cwv & 0xFFu) : 0;
      bool pend = cl && !cok;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int src = ec[j] >= 0 ? ec[j] : 0;
        const int okc = __shfl((int)cok, src, 64);
        nce[j] = __shfl(ncl, src, 64);
        if (ec[j] >= 0) pend = pend || !okc || (epo[j] < nce[j] && !entry_ok(ent[j], ep));
      }
      if (__ballot(pend) == 0ull) break;
      if (spins >= a.merge_spins) {
        tmo = true;
        break;
      }
      __builtin_amdgcn_s_sleep(1);
      if (cl && !cok) cwv = __hip_atomic_load(cw + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
      for (int j = 0; j < 2; j++)
        if (ec[j] >= 0 && !entry_ok(ent[j], ep))
          ent[j] = __hip_atomic_load(lists + (long long)ec[j] * KM + epo[j], __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
    }
    ncl = ncl < KM ? ncl : KM;
    if (lane == c) ncl = own_n;
    if (lane >= a.S) ncl = 0;
    if (lane < a.S) {
      sh.lcnt[lane] = ncl;
      sh.lsort[lane] = lane == c ? (raw_list ? 0 : 1) : (int)((cwv >> 8) & 1u);
      sh.lz[lane] = lane == c ? (raw_list ? 1 : 0) : (int)((cwv >> 9) & 1u);
    }
    const int incl = (int)wave_incl_scan((uint32_t)ncl);
    const int total = (int)readlane_u32((uint32_t)incl, 63);
    const int maxn = (int)wave_max((uint32_t)(lane == c ? 0 : ncl));
    const bool fast = !tmo && total <= KM && maxn <= E;
    if (fast) {
      // the lists end to end: list q from the sum of the counts before it
      const int off = incl - ncl;
#pragma unroll
      for (int j = 0; j < 2; j++) {
        const int src = ec[j] >= 0 ? ec[j] : 0;
        const int o = __shfl(off, src, 64);
        const int zl = __shfl((int)((cwv >> 9) & 1u), src, 64);
        if (ec[j] >= 0 && epo[j] < nce[j]) {
          const u64 xe = untag_entry(ent[j]);
          sh.mer[o + epo[j]] = zl ? z_to_y(xe, r) : xe;
          __hip_atomic_store(lists + (long long)ec[j] * KM + epo[j], EMPTY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
      }
      const int oo = __shfl(off, c, 64);
      if (lane < own_n) sh.mer[oo + lane] = raw_list ? z_to_y(buf[lane], r) : sh.own[lane];
      if (lane >= total) sh.mer[lane] = 0ull;  // pads: never above an entry
    }
    if (lane == 0) {
      sh.fast = fast ? total : -1;
      if (tmo) sh.tmo = 1;
    }
  }
  __syncthreads();
  const int nfast = sh.fast;
  if (nfast >= 0) {
    if (w == 0) {
      // the entries are distinct composites and the pads (and entries that
      // z / T leaves out) are 0, below every one: one wave sort ranks them
      finish_merged(a, r, wave_sort_desc(sh.mer[lane]), k, false);
    }
  } else {
    // a tree of wave merges: wave w takes lists w, w + NW, ...
    u64 racc = 0ull;
    bool first = true, tmo = false;
    for (int cc = w; cc < a.S; cc += NW) {
      const int n = sh.lcnt[cc];
      u64 x;
      if (cc == c) {
        x = lane < n ? (raw_list ? buf[lane] : sh.own[lane]) : 0ull;
      } else {
        x = take_entry(lists + (long long)cc * KM + lane, lane < n, ep, &tmo, a.merge_spins);
      }
      if (sh.lz[cc]) x = z_to_y(x, r);
      if (!sh.lsort[cc]) x = wave_sort_desc(x);
      racc = first ? x : wave_merge_top64(racc, x);
      first = false;
    }
    if (tmo && lane == 0) sh.tmo = 1;
    racc = merge_waves<NW>(racc, sh.slots);
    if (w == 0) finish_merged(a, r, racc, k, sh.tmo != 0);
  }
  // ready for the next call: counter zero, epoch advanced (entries were
  // cleared as they were read)
  if (threadIdx.x == 0) {
    __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(cnt + 1, ep == 0xFFFFFFFFu ? 0u : ep, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

template <typename Tin, int NTT>
hipError_t launch_n(const SampleArgs& a, size_t lds, hipStream_t st) {
  const dim3 g(a.B * a.S), blk(NTT);
  const bool vec = a.whole_vec != 0, mask = a.mask_table != nullptr && a.n_states > 0;
  if (vec && mask) hipLaunchKernelGGL((k64_kernel<Tin, NTT, true, true>), g, blk, lds, st, a);
  else if (vec) hipLaunchKernelGGL((k64_kernel<Tin, NTT, true, false>), g, blk, lds, st, a);
  else if (mask) hipLaunchKernelGGL((k64_kernel<Tin, NTT, false, true>), g, blk, lds, st, a);
  else hipLaunchKernelGGL((k64_kernel<Tin, NTT, false, false>), g, blk, lds, st, a);
  return hipGetLastError();
}

// Workgroups of the K64_NT instantiation one CU holds at once with lds bytes
// of dynamic LDS (0 when the runtime cannot say).
template <typename Tin>
int resident_n(bool vec, bool mask, size_t lds) {
  const void* f = vec && mask ? (const void*)k64_kernel<Tin, K64_NT, true, true>
                  : vec       ? (const void*)k64_kernel<Tin, K64_NT, true, false>
                  : mask      ? (const void*)k64_kernel<Tin, K64_NT, false, true>
                              : (const void*)k64_kernel<Tin, K64_NT, false, false>;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, f, K64_NT, lds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  return n;
}

template <typename Tin, int NTT>
hipError_t set_lds(size_t bytes) {
  const void* fns[] = {
      (const void*)k64_kernel<Tin, NTT, true, true>,
      (const void*)k64_kernel<Tin, NTT, true, false>,
      (const void*)k64_kernel<Tin, NTT, false, true>,
      (const void*)k64_kernel<Tin, NTT, false, false>,
  };
  hipError_t e = hipSuccess;
  for (const void* f : fns) {
    hipError_t e2 = hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e2 != hipSuccess) e = e2;
  }
  return e;
}

}  // namespace k64

int k64_chunk_ids(int dtype) { return K64_NT * K64_NVT * (dtype == 1 ? 8 : 4); }

int k64_small_ids(int dtype) { return K64_SMALL_NT * K64_NVT * (dtype == 1 ? 8 : 4); }

size_t k64_static_lds() { return sizeof(k64::Shared<K64_NT / 64>); }

int k64_resident_per_cu(int dtype, bool whole_vec, bool mask, size_t lds) {
  return dtype == 1 ? k64::resident_n<uint16_t>(whole_vec, mask, lds) : k64::resident_n<float>(whole_vec, mask, lds);
}

hipError_t launch_k64(const SampleArgs& a, int dtype, size_t lds, hipStream_t st, bool small) {
  if (small)
    return dtype == 1 ? k64::launch_n<uint16_t, K64_SMALL_NT>(a, lds, st) : k64::launch_n<float, K64_SMALL_NT>(a, lds, st);
  return dtype == 1 ? k64::launch_n<uint16_t, K64_NT>(a, lds, st) : k64::launch_n<float, K64_NT>(a, lds, st);
}

hipError_t set_k64_lds_limit(size_t bytes) {
  hipError_t e = hipSuccess, e2;
  if ((e2 = k64::set_lds<float, K64_NT>(bytes)) != hipSuccess) e = e2;
  if ((e2 = k64::set_lds<uint16_t, K64_NT>(bytes)) != hipSuccess) e = e2;
  if ((e2 = k64::set_lds<float, K64_SMALL_NT>(bytes)) != hipSuccess) e = e2;
  if ((e2 = k64::set_lds<uint16_t, K64_SMALL_NT>(bytes)) != hipSuccess) e = e2;
  return e;
}

}  // namespace tgs
