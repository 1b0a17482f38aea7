// tgs_k64.hip -- one fused kernel for batches whose rows are greedy or sample
// with 1 <= top_k <= 64 (the launch's batch hint promises it).
//
// Workgroup (b, c) of K64_NT threads owns chunk c of row b: S chunks per
// row, each at most K64_NT * K64_NVT sixteen-byte vectors (thread t holding
// chunk vectors t, t + K64_NT, ...).  Rows that fit one chunk of
// K64_SMALL_NT threads (one wave) run on that instantiation instead.  Everything a thread reads is requested
// at entry: the row's parameters, its history ids, its vectors and (with a
// mask table) their mask words, so the whole chunk is in flight at once.
// Under a full-chip stream the chunk's data lands in one burst near the end
// of the stream, so the steps after it are kept short:
//   1. Vector maxima and thread maxima of the raw logits (ids the mask
//      forbids and ids past the chunk left out).
//   2. A bound: for m = 1 .. waves, the m-th largest over waves of the
//      wave's ceil(k / m)-th largest thread maximum qualifies (m waves hold
//      that many at or above it each); the bound is the largest of them,
//      read from one wave sort each.  In the sort a thread whose maximum
//      lies in a vector holding a history id of the chunk (the bits are in
//      LDS before the chunk lands) takes the lowest key, so at least k
//      distinct ids that are neither masked nor history ids have a raw
//      logit at or above the bound.  The collection threshold cz lies 16
//      representable values below it.
//   3. Every vector whose maximum reaches cz is staged whole in its wave's
//      LDS list.
//   4. One staged vector per lane: the canonical logit y = z / T of each
//      element (correctly rounded, tg_div_t), history ids left to their
//      producers (the lane whose insertion created the id's LDS hash slot
//      loads its logit at entry and adds its penalised value), the mask
//      test, and a wave-aggregated append to the LDS candidate buffer that
//      also counts the candidates strictly above yc = cz / T.
//   5. An id left out is not a history id and has z < cz, so its y is at
//      most yc: with at least k candidates strictly above yc the chunk's top
//      k are among the candidates and are ranked into wave 0.  The ids
//      behind the bound make that count at least k unless their quotients
//      by T collide (a temperature so small that z / T overflows, say);
//      then, and when a wave stages more vectors than its list holds (a
//      skewed chunk), an exact radix selection runs over the chunk read
//      again from memory.
//
// Rows split over S > 1 chunks.  Each workgroup counts itself in the row's
// arrival counter at entry (a relaxed device atomic issued with the loads).
// The workgroup that arrives last merges the row: every other workgroup of
// the row has started by then and stores its sorted list with agent-coherent
// stores (written through past the per-XCD L2s, which are not coherent with
// each other) without waiting for anything.  The merging workgroup polls
// those lists with agent-coherent loads, one list per wave, until no entry
// holds the empty marker, merges them with its own (a tree of wave merges),
// finishes the row (masses, top-p, draw) and resets the lists to the marker
// and the counter to zero for the next call.  The wait is bounded: one that
// runs out (it cannot while every workgroup runs) writes id -4 for the row.
// No fence is issued: on this part an agent-scope release or acquire fence
// writes back or invalidates the whole L2 of the XCD.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace k64 {

constexpr int NVT = K64_NVT;         // 16-byte vectors per thread
constexpr int P1 = NVT / 2;          // vectors behind the bound
constexpr int KM = 64;               // largest top_k served
constexpr int CAP = K64_CAP;         // candidate buffer entries
constexpr u64 EMPTY = ~0ull;         // list entry not written yet: above every composite
constexpr int SPIN_LIMIT = 1 << 18;  // polls of one list before the wait gives up
constexpr uint32_t KEY_MIN = 0x00800000u;  // key of -FLT_MAX: below it only -inf and NaN

template <typename Tin, int NTT>
struct Geo {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int NW = NTT / 64;
  static constexpr int CH = NTT * NVT * EPV;  // ids of a chunk at most
  static constexpr int MAXH = NTT >= K64_NT ? K64_MAX_HIST : K64_SMALL_MAX_HIST;  // longest history
  static constexpr int NHID = (MAXH + NTT - 1) / NTT;  // history ids per thread
  static constexpr uint32_t GM = (1u << EPV) - 1u;
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

// max over m = 1 .. NW of the m-th largest of wkey[m - 1][0, NW) (NW one or
// four), in every lane: lanes 4 (m - 1) + i load wkey[m - 1][i], each group
// of four lanes sorts itself descending (comparators (0,1) (2,3), (0,2)
// (1,3), (1,2) as lane exchanges), and lane 5 (m - 1) then holds the m-th
// largest of group m - 1.  The exchanges are DPP quad permutes.
template <int NW>
__device__ __forceinline__ uint32_t bound_key(const uint32_t (*wkey)[NW], int lane) {
  static_assert(NW == 1 || NW == 4, "waves per workgroup");
  if constexpr (NW == 1) {
    return wkey[0][0];
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
// lanes: ranking for short buffers, wave sorts of 64-entry slices merged
// as a tree otherwise.  Ends with a barrier.
template <int NTT>
__device__ __forceinline__ u64 select_top(u64* buf, int n, int k, u64 (*slots)[64]) {
  constexpr int NW = NTT / 64;
  const int w = threadIdx.x >> 6, lane = lane_id();
  if (n <= 256) {
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

// Wave-aggregated append of composite x (when ok) to the LDS buffer.
__device__ __forceinline__ void append(bool ok, u64 x, u64* buf, unsigned* nbuf) {
  const u64 bal = __ballot(ok);
  if (bal == 0ull) return;
  unsigned base = 0;
  if (lane_id() == 0) base = atomicAdd(nbuf, (unsigned)__popcll(bal));
  base = (unsigned)__shfl((int)base, 0, 64);
  const unsigned sl = base + lanes_below(bal);
  if (ok && sl < (unsigned)CAP) buf[sl] = x;
}

// Wave-aggregated append of up to N composites per lane (entry q when
// ok[q]) to the LDS buffer, counting the appended entries whose key is above
// kc: one LDS atomic per wave on a packed counter (appended entries in the
// low 16 bits, entries above kc in the high 16), slots from a wave prefix
// sum of the lanes' counts.
template <int N>
__device__ __forceinline__ void append_n(const u64 (&x)[N], const bool (&ok)[N], uint32_t kc, u64* buf,
                                         unsigned* packed) {
  unsigned cnt = 0, abv = 0;
#pragma unroll
  for (int q = 0; q < N; q++) {
    cnt += ok[q] ? 1u : 0u;
    abv += (ok[q] && (uint32_t)(x[q] >> 32) > kc) ? 1u : 0u;
  }
  const unsigned v = cnt | (abv << 16);
  const unsigned incl = wave_incl_scan(v);
  const unsigned tot = readlane_u32(incl, 63);
  if (tot == 0u) return;
  unsigned base = 0;
  if (lane_id() == 0) base = atomicAdd(packed, tot);
  base = readlane_u32(base, 0) & 0xFFFFu;
  unsigned sl = base + ((incl - v) & 0xFFFFu);
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

template <typename Tin, int NTT, bool VEC, bool MASK>
__global__ __launch_bounds__(NTT) void k64_kernel(SampleArgs a) {
  using G = Geo<Tin, NTT>;
  constexpr int EPV = G::EPV, NW = G::NW, NHID = G::NHID;
  constexpr uint32_t GM = G::GM;
  constexpr int SCAP = 64;   // staged vectors per wave
  TGS_DYN_SMEM(smem);
  __shared__ u64 slots[NW][64];      // wave lists (merges, the ranked top k)
  __shared__ uint4 svec[NW][SCAP];   // per wave: vectors whose maximum reaches the collection threshold
  __shared__ int sidx[NW][SCAP];     // their vector index in the chunk
  __shared__ uint32_t wkey[NW][NW];  // [m - 1][wave]: the wave's ceil(k / m)-th largest thread maximum key
  __shared__ unsigned nbuf;          // candidates appended (low 16 bits), of them above yc (high 16)
  __shared__ int elect, tmo, spill;
  __shared__ BlockScratch bs;
  int2* hash = (int2*)(smem + a.off_hash);
  uint32_t* bitmap = (uint32_t*)(smem + a.off_bitmap);
  u64* buf = (u64*)(smem + a.off_cand);
  const int w = threadIdx.x >> 6, lane = lane_id();

  const int b = blockIdx.x / a.S, c = blockIdx.x % a.S;
  if (b >= a.B) return;
  const int v0 = c * a.L, v1 = min(a.V, v0 + a.L);  // a.L is a multiple of EPV
  const int nvec = (v1 - v0 + EPV - 1) / EPV;
  const int nfull = nvec / NTT;  // vectors every thread holds
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  unsigned* cnt = a.cnt + (long long)b * K64_CNT_STRIDE;

  // ---- everything read first, in the order it is needed (a wave's loads
  // return in order): the row's parameters, its history length and ids, the
  // arrival count, the chunk, the mask words
  const tgs_row_params p = a.params[b];
  const float ub = a.u[b];
  const int hlr = *(a.hist_len ? a.hist_len + b : (const int*)a.params);
  const bool hv = a.hist && a.hist_cap > 0;
  const int* hp = hv ? a.hist + (long long)b * a.hist_cap : (const int*)a.params;
  const int hlast = hv ? a.hist_cap - 1 : 0;
  int hid[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) {
    const int j = (int)threadIdx.x + q * NTT;
    hid[q] = hp[j < hlast ? j : hlast];
  }
  unsigned arrived = 0;
  if (a.S > 1 && threadIdx.x == 0)
    arrived = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // the mask words depend on the parameters: requested before the chunk so
  // that they do not queue behind it (a state out of range reads the first
  // row, and the row is rejected below)
  uint32_t mw[MASK ? NVT : 1];
  if constexpr (MASK) {
    const uint32_t* mrow = a.mask_table;
    if (p.mask_state >= 0 && p.mask_state < a.n_states) mrow += (long long)p.mask_state * a.mask_words;
#pragma unroll
    for (int i = 0; i < NVT; i++) {
      const int j = (int)threadIdx.x + i * NTT;
      mw[i] = mrow[(v0 + (j < nvec ? j : nvec - 1) * EPV) >> 5];
    }
  }
  // Whole vectors: one unconditional load each (a vector past the chunk
  // reads its last one again and is left out in step 1).  With no branch
  // among the loads the compiler waits exactly for the history ids and the
  // arrival count, so the history hash is built while the chunk streams in.
  uint4 raw[NVT];
#pragma unroll
  for (int i = 0; i < NVT; i++) {
    const int j = (int)threadIdx.x + i * NTT;
    if constexpr (VEC) {
      raw[i] = tg_load_nt(rowp + v0 + (j < nvec ? j : nvec - 1) * EPV);
    } else if (i * NTT < nvec) {  // whole-workgroup test: vectors wholly past the chunk are not read
      raw[i] = load_vec<Tin>(rowp, v0 + j * EPV, v1, a.aligned);
    } else {
      raw[i] = make_uint4(0x7FC00000u, 0x7FC00000u, 0x7FC00000u, 0x7FC00000u);  // NaN: never counted
    }
  }
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
  const bool masked = MASK && r.mrow != nullptr;

  // ---- history: each id of the chunk counted in the LDS hash (its
  // producer is the lane that created its slot) and marked in the packed
  // history bits (HBits)
  if (threadIdx.x == 0) {
    nbuf = 0;
    tmo = 0;
    spill = 0;
    elect = a.S > 1 && arrived == (unsigned)(a.S - 1);
  }
  const bool pen = r.use_pen;
  using HB = HBits<Tin, NTT>;
  constexpr int HPW = HB::HPW;
  int hslot[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) hslot[q] = -1;
  if (pen) {
    for (int i = threadIdx.x; i < a.TS; i += NTT) hash[i] = make_int2(-1, 0);
#pragma unroll
    for (int q = 0; q < HPW; q++) bitmap[threadIdx.x * HPW + q] = 0u;
    __syncthreads();
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
        const int j = (id - v0) / EPV;
        atomicOr(&bitmap[HB::word(j)], 1u << (HB::shift(j) + (id - v0) % EPV));
      }
    }
  }
  __syncthreads();
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
  // producers' logits (and mask words): one load per history id of the
  // chunk, first needed after the bound
  float zq[NHID];
  uint32_t mq[NHID];
#pragma unroll
  for (int q = 0; q < NHID; q++) {
    zq[q] = 0.0f;
    mq[q] = 0xFFFFFFFFu;
    if (hslot[q] >= 0) {
      zq[q] = Elem<Tin>::scalar(rowp, hid[q]);
      if (masked) mq[q] = r.mrow[hid[q] >> 5];
    }
  }

  // ---- 1. vector maxima and thread maximum of the raw logits (ids the
  // mask forbids and vectors past the chunk left out; history ids included)
  // and the first vector that holds the thread maximum
  float vm[NVT];
  float tm = -__builtin_inff();
  int im = 0;
#pragma unroll
  for (int i = 0; i < NVT; i++) {
    float m;
    if constexpr (MASK) {
      const uint32_t x = masked ? ~(mw[i] >> ((v0 + ((int)threadIdx.x + i * NTT) * EPV) & 31)) & GM : 0u;
      m = -__builtin_inff();
#pragma unroll
      for (int e = 0; e < EPV; e++) m = ((x >> e) & 1u) ? m : fmaxf(m, Elem<Tin>::get(raw[i], e));
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

  // ---- 2. the bound: at least k thread maxima (distinct ids) are >= it.
  // For m = 1 .. NW, the m-th largest over waves of the wave's ceil(k / m)-th
  // largest key qualifies (m waves hold ceil(k / m) keys at or above it
  // each); the bound is the largest of them, all read from one sort per
  // wave.  A thread whose maximum lies in a vector holding a history id
  // sorts as the lowest key, so every thread maximum behind the bound is an
  // id that is not a history id.
  {
    uint32_t hw = hpk[0];
#pragma unroll
    for (int q = 1; q < HPW; q++) hw = im * EPV / 32 == q ? hpk[q] : hw;
    const bool hmax = ((hw >> (im * EPV % 32)) & GM) != 0u;
    const uint32_t tk = (tm > -__builtin_inff() && !hmax) ? tg_key(tm) : 0u;
    const uint32_t srt = wave_sort_desc(tk);  // lane i: the (i+1)-th largest
#pragma unroll
    for (int m = 1; m <= NW; m++) {
      const uint32_t v = readlane_u32(srt, (k + m - 1) / m - 1);
      if (lane == 0) wkey[m - 1][w] = v;
    }
  }
  __syncthreads();
  const uint32_t bkey = bound_key<NW>(wkey, lane);
  // the collection threshold: 16 representable values below the bound, so
  // that the ids that set the bound land strictly above its canonical value
  const bool all = bkey < KEY_MIN + 32u;  // no usable bound: collect every allowed id
  const float cz = all ? -__builtin_inff() : tg_unkey(bkey - 16u);
  const float yc = all ? -__builtin_inff() : row_y(r, cz);
  const uint32_t kc = tg_key(yc);

  // ---- 3. collection: every vector whose maximum reaches cz is staged
  // whole (its bits and its chunk index) in its wave's list
  unsigned ns = 0;  // staged vectors of the wave (uniform)
#pragma unroll
  for (int i = 0; i < NVT; i++) {
    const bool pass = vm[i] >= cz && vm[i] > -__builtin_inff();  // (cz may be -inf)
    const u64 bal = __ballot(pass);
    if (bal != 0ull) {
      const unsigned sl = ns + lanes_below(bal);
      if (pass && sl < (unsigned)SCAP) {
        svec[w][sl] = raw[i];
        sidx[w][sl] = (int)threadIdx.x + i * NTT;
      }
      ns += (unsigned)__popcll(bal);
    }
  }
  if (ns > (unsigned)SCAP && lane == 0) spill = 1;
  wave_lds_sync();

  // ---- 4. the staged vectors (one per lane) and the history ids: exact
  // canonical logits, history ids left to their producers, into the
  // candidate buffer; the high half of the packed counter counts candidates
  // strictly above yc
  {
    const unsigned nst = ns < (unsigned)SCAP ? ns : (unsigned)SCAP;
    for (unsigned s0 = 0; s0 < nst; s0 += 64) {
      const unsigned si = s0 + (unsigned)lane;
      u64 x[EPV];
      bool ok[EPV];
      uint4 v = make_uint4(0x7FC00000u, 0x7FC00000u, 0x7FC00000u, 0x7FC00000u);
      int j = 0;
      if (si < nst) {
        v = svec[w][si];
        j = sidx[w][si];
      }
      const int o = j * EPV;
      const uint32_t hw = (pen && si < nst) ? HB::of(bitmap, j) : 0u;
      uint32_t xm = 0u;
      if constexpr (MASK) xm = (masked && si < nst) ? ~(r.mrow[(v0 + o) >> 5] >> ((v0 + o) & 31)) : 0u;
#pragma unroll
      for (int e = 0; e < EPV; e++) {
        const float z = Elem<Tin>::get(v, e);
        const float y = row_y(r, z);
        ok[e] = si < nst && z >= cz && !((hw >> e) & 1u) && !((xm >> e) & 1u) && y > -__builtin_inff() &&
                j < nvec;
        x[e] = comp_key(tg_key(y), v0 + o + e);
      }
      append_n<EPV>(x, ok, kc, buf, &nbuf);
    }
  }
  u64 hcomp[NHID];
  {
    bool hok[NHID];
#pragma unroll
    for (int q = 0; q < NHID; q++) {
      u64 x = 0ull;
      if (hslot[q] >= 0) {
        const int id = hid[q];
        const float y = row_y(r, penalise(zq[q], hash[hslot[q]].y, r));
        const bool ok = y > -__builtin_inff() && (!masked || ((mq[q] >> (id & 31)) & 1u));
        if (ok) x = comp_key(tg_key(y), id);
        if (a.dbg.post_logits) a.dbg.post_logits[(long long)b * a.V + id] = ok ? y : -__builtin_inff();
      }
      hcomp[q] = x;
      hok[q] = x != 0ull && (uint32_t)(x >> 32) >= kc;
    }
    append_n<NHID>(hcomp, hok, kc, buf, &nbuf);
  }
  __syncthreads();

  // ---- 5. the chunk's sorted top k: from the candidates when they hold at
  // least k entries strictly above yc (then no id left out can be among the
  // top k) or every allowed id; otherwise the exact path
  u64 acc;
  const int nb = (int)(nbuf & 0xFFFFu), nab = (int)(nbuf >> 16);
  if (!spill && nb <= CAP && (all || nab >= k)) {
    acc = select_top<NTT>(buf, nb, k, slots);
  } else {
    // exact path (rare: quotients that collide, skewed chunks): the k-th
    // composite of the chunk by radix selection over the
    // chunk read again (L2 / MALL hits), then the k entries at or above it
    acc = exact_top<Tin, NTT, MASK>(a, r, rowp, nvec, pen, bitmap, masked, hcomp, k, buf, &nbuf, slots, bs);
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
  u64* lists = a.lists + (long long)b * a.S * KM;
  if (!elect) {
    // publish the chunk's list for the row's merging workgroup
    if (w == 0) __hip_atomic_store(lists + (long long)c * KM + lane, acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return;
  }
  // the row's last arrival: one list per wave (own list from wave 0's
  // registers through LDS), polled in parallel, then a tree of merges
  u64* own = slots[NW - 1];
  if (w == 0) own[lane] = acc;
  __syncthreads();
  u64 racc = 0ull;
  bool first = true;
  for (int cc = w; cc < a.S; cc += NW) {
    u64 x;
    if (cc == c) {
      x = own[lane];
    } else {
      const u64* lp = lists + (long long)cc * KM + lane;
      x = __hip_atomic_load(lp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      int spins = 0;
      while (__ballot(x == EMPTY) != 0ull) {
        if (++spins > SPIN_LIMIT) {
          if (lane == 0) tmo = 1;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
        x = __hip_atomic_load(lp, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      if (x == EMPTY) x = 0ull;
    }
    racc = first ? x : wave_merge_top64(racc, x);
    first = false;
  }
  __syncthreads();  // own[] (a slot of the merge tree) read by its wave
  racc = merge_waves<NW>(racc, slots);
  if (w == 0) {
    if (tmo) {
      if (lane == 0) {
        a.out[b] = -4;
        write_row_diag(a, b, 0, 0, 0, 0, -1);
      }
    } else {
      const int nr = __popcll(__ballot(racc != 0ull));
      wave_finish_row(a, r, lane < k ? racc : 0ull, nr < k ? nr : k);
    }
  }
  // ready for the next call: lists empty, counter zero
  for (int cc = w; cc < a.S; cc += NW)
    if (cc != c) __hip_atomic_store(lists + (long long)cc * KM + lane, EMPTY, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (threadIdx.x == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
