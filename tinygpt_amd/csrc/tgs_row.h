// tgs_row.h -- per-row state shared by the sampling kernels: element
// access for fp32 / bf16 rows, row parameter validation (the same rules as
// the CPU restatement), the LDS history table (id -> count) and penalties,
// keys of one element, and the single-wave finish of a row whose kept list
// (at most 64 entries, sorted) sits one entry per lane.
#pragma once

#include "tgs_device.h"
#include "tgs_kernels.h"

namespace tgs {

// ------------------------------------------------------------------ loads

template <typename Tin>
struct Elem;
template <>
struct Elem<float> {
  static constexpr int EPV = 4;
  static constexpr uint32_t NAN_BITS = 0x7FC00000u;
  __device__ static __forceinline__ float get(const uint4& r, int e) {
    const uint32_t w = e == 0 ? r.x : e == 1 ? r.y : e == 2 ? r.z : r.w;
    return tg_u2f(w);
  }
  __device__ static __forceinline__ float scalar(const void* p, long long i) {
    return ((const float*)p)[i];
  }
};
template <>
struct Elem<uint16_t> {  // bf16 bits
  static constexpr int EPV = 8;
  static constexpr uint32_t NAN_BITS = 0x7FC07FC0u;
  __device__ static __forceinline__ float get(const uint4& r, int e) {
    const uint32_t w = (e >> 1) == 0 ? r.x : (e >> 1) == 1 ? r.y : (e >> 1) == 2 ? r.z : r.w;
    return tg_u2f((e & 1) ? (w & 0xFFFF0000u) : (w << 16));
  }
  __device__ static __forceinline__ float scalar(const void* p, long long i) {
    return tg_u2f((uint32_t)((const uint16_t*)p)[i] << 16);
  }
};

// Load EPV consecutive logits starting at id v (v a multiple of EPV) from
// row pointer rowp; ids >= vend read as NaN (never allowed).
template <typename Tin>
__device__ __forceinline__ uint4 load_vec(const Tin* rowp, int v, int vend, bool aligned) {
  constexpr int EPV = Elem<Tin>::EPV;
  if (aligned && v + EPV <= vend) return *(const uint4*)(rowp + v);
  uint32_t w[4];
#pragma unroll
  for (int i = 0; i < 4; i++) w[i] = Elem<Tin>::NAN_BITS;
  if (sizeof(Tin) == 4) {
#pragma unroll
    for (int e = 0; e < 4; e++)
      if (v + e < vend) w[e] = ((const uint32_t*)rowp)[v + e];
  } else {
#pragma unroll
    for (int e = 0; e < 8; e++)
      if (v + e < vend) {
        const uint32_t h = ((const uint16_t*)rowp)[v + e];
        w[e >> 1] = (e & 1) ? ((w[e >> 1] & 0xFFFFu) | (h << 16)) : ((w[e >> 1] & 0xFFFF0000u) | h);
      }
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// ------------------------------------------------------------------ row state

struct Row {
  int b, c;
  int mode;  // 0 greedy, 1 candidate top-k, 2 full
  float T, rT;  // temperature (1 for greedy rows) and RN(1 / T)
  int tdiv;     // tg_div_t mode of T
  int k;
  float top_p, rep, pres, freq, u;
  bool use_pen;
  int H;
  const int* hrow;
  const uint32_t* mrow;  // nullptr: no mask
  int v0, v1;            // chunk id range [v0, v1)
};

// Validates row b's parameters (p, its uniform u and history length H are
// passed in so that callers can issue those loads early) and fills r.
__device__ __forceinline__ bool row_setup_from(const SampleArgs& a, int b, int c, const tgs_row_params& p,
                                               float u, int H, Row& r) {
  r.b = b;
  r.c = c;
  const float T = p.temperature;
  if (__builtin_isnan(T)) return false;
  const bool greedy = (p.flags & TGS_FLAG_GREEDY) || T <= 0.0f;
  r.T = 1.0f;
  r.rT = 1.0f;
  r.tdiv = TDIV_POW2;
  r.u = 0.0f;
  if (!greedy) {
    if (!__builtin_isfinite(T)) return false;
    r.T = T;
    r.rT = 1.0f / T;
    if (!__builtin_isfinite(r.rT)) return false;
    r.tdiv = tg_div_t_mode(T);
    if (__builtin_isnan(p.top_p) || p.top_p <= 0.0f) return false;
    r.u = u;
    if (__builtin_isnan(r.u) || r.u < 0.0f || r.u >= 1.0f) return false;
  }
  if (!(p.repetition > 0.0f) || !__builtin_isfinite(p.repetition)) return false;
  if (!__builtin_isfinite(p.presence) || !__builtin_isfinite(p.frequency)) return false;
  r.H = H;
  if (r.H < 0 || r.H > a.hist_cap) return false;
  r.hrow = a.hist ? a.hist + (long long)b * a.hist_cap : nullptr;
  r.mrow = nullptr;
  if (p.mask_state >= 0) {
    if (p.mask_state >= a.n_states) return false;
    r.mrow = a.mask_table + (long long)p.mask_state * a.mask_words;
  }
  r.k = p.top_k;
  r.top_p = p.top_p;
  r.rep = p.repetition;
  r.pres = p.presence;
  r.freq = p.frequency;
  const bool neutral = (p.repetition == 1.0f && p.presence == 0.0f && p.frequency == 0.0f);
  r.use_pen = (r.H > 0 && !neutral && r.hrow != nullptr);
  if (greedy) r.mode = 0;
  else if (p.top_k >= 1 && p.top_k <= KMAX && p.top_k < a.V) r.mode = 1;
  else r.mode = 2;
  r.v0 = 0;
  r.v1 = a.V;
  return true;
}

__device__ __forceinline__ bool row_setup(const SampleArgs& a, int b, int c, Row& r) {
  const tgs_row_params p = a.params[b];
  const bool greedy = (p.flags & TGS_FLAG_GREEDY) || p.temperature <= 0.0f;
  const float u = greedy ? 0.0f : a.u[b];
  return row_setup_from(a, b, c, p, u, a.hist_len ? a.hist_len[b] : a.hist_cap, r);
}

// A sampling row outside the launch hint: top-k above hint_k, or no usable
// top-k while the full-path kernel is not launched.  Such rows get id -3.
__device__ __forceinline__ bool outside_hint(const SampleArgs& a, const Row& r) {
  return (r.mode == 1 && r.k > a.hint_k) || (r.mode == 2 && !a.full_rows);
}

// ------------------------------------------------------------------ history

__device__ __forceinline__ unsigned hash_slot(int id, int shift) {
  return ((unsigned)id * 2654435761u) >> shift;
}

// Counts one occurrence of id in the LDS hash (open addressing, linear
// probing; the table has at least twice as many slots as history entries,
// so a free slot always exists).
__device__ __forceinline__ void hash_insert(int2* hash, int TS, int shift, int id) {
  const unsigned tmask = (unsigned)TS - 1u;
  unsigned h = hash_slot(id, shift);
  for (;;) {
    const int old = atomicCAS(&hash[h].x, -1, id);
    if (old == -1 || old == id) {
      atomicAdd(&hash[h].y, 1);
      break;
    }
    h = (h + 1) & tmask;
  }
}

// Insert the row's history ids that fall in [r.v0, r.v1) into the LDS hash
// (id -> count) and, when BW > 0, the chunk bitmap.
template <int BS = NT>
__device__ __forceinline__ void hash_build(const SampleArgs& a, const Row& r, int2* hash,
                                           uint32_t* bitmap, int BW) {
  for (int i = threadIdx.x; i < a.TS; i += BS) hash[i] = make_int2(-1, 0);
  for (int i = threadIdx.x; i < BW; i += BS) bitmap[i] = 0u;
  __syncthreads();
  for (int j = threadIdx.x; j < r.H; j += BS) {
    const int id = r.hrow[j];
    if (id < r.v0 || id >= r.v1 || id >= a.V) continue;
    hash_insert(hash, a.TS, a.ts_shift, id);
    if (BW) atomicOr(&bitmap[(id - r.v0) >> 5], 1u << ((id - r.v0) & 31));
  }
  __syncthreads();
}

// The history entries of this thread, read before the row's logits so that
// building the hash does not wait for them (a wave's loads return in
// order): entry threadIdx.x + q * BS in hid[q] (clamped reads; entries at
// or past the row's history length are ignored by hash_build_pre).
template <int BS, int NPRE>
__device__ __forceinline__ void hist_prefetch(const SampleArgs& a, int b, int (&hid)[NPRE]) {
  const bool hv = a.hist && a.hist_cap > 0;
  const int* hp = hv ? a.hist + (long long)b * a.hist_cap : (const int*)a.params;
  const int hlast = hv ? a.hist_cap - 1 : 0;
#pragma unroll
  for (int q = 0; q < NPRE; q++) {
    const int j = (int)threadIdx.x + q * BS;
    hid[q] = hp[j < hlast ? j : hlast];
  }
}

// hash_build over the entries hist_prefetch read (r.H <= NPRE * BS).
template <int BS, int NPRE>
__device__ __forceinline__ void hash_build_pre(const SampleArgs& a, const Row& r, const int (&hid)[NPRE],
                                               int2* hash, uint32_t* bitmap, int BW) {
  for (int i = threadIdx.x; i < a.TS; i += BS) hash[i] = make_int2(-1, 0);
  for (int i = threadIdx.x; i < BW; i += BS) bitmap[i] = 0u;
  __syncthreads();
#pragma unroll
  for (int q = 0; q < NPRE; q++) {
    const int id = hid[q];
    if ((int)threadIdx.x + q * BS >= r.H || id < r.v0 || id >= r.v1 || id >= a.V) continue;
    hash_insert(hash, a.TS, a.ts_shift, id);
    if (BW) atomicOr(&bitmap[(id - r.v0) >> 5], 1u << ((id - r.v0) & 31));
  }
  __syncthreads();
}

__device__ __forceinline__ int hash_count(const int2* hash, int TS, int shift, int id) {
  const unsigned tmask = (unsigned)TS - 1u;
  unsigned h = hash_slot(id, shift);
  for (;;) {
    const int2 e = hash[h];
    if (e.x == id) return e.y;
    if (e.x == -1) return 0;
    h = (h + 1) & tmask;
  }
}

// Penalised logit of a history id (count c > 0): CTRL repetition, then
// frequency per occurrence, then presence.
__device__ __forceinline__ float penalise(float z, int c, const Row& r) {
  if (r.rep != 1.0f) z = (z > 0.0f) ? z / r.rep : z * r.rep;
  z = z - r.freq * (float)c;
  z = z - r.pres;
  return z;
}

__device__ __forceinline__ bool mask_allows(const Row& r, int v) {
  return r.mrow == nullptr || ((r.mrow[v >> 5] >> (v & 31)) & 1u);
}

// The canonical logit of a (penalised) logit z: z / T correctly rounded
// (z itself on greedy rows, whose T is 1).
__device__ __forceinline__ float row_y(const Row& r, float z) { return tg_div_t(z, r.T, r.rT, r.tdiv); }

// Key of one element (0 when not allowed); *y_out gets the canonical logit.
__device__ __forceinline__ uint32_t elem_key(float z, bool allowed, const Row& r, float* y_out) {
  const float y = row_y(r, z);
  const bool ok = allowed && (y > -__builtin_inff());
  *y_out = ok ? y : -__builtin_inff();
  return ok ? tg_key(y) : 0u;
}

// ------------------------------------------------------------------ finalize

__device__ __forceinline__ void write_row_diag(const SampleArgs& a, int b, int n1, int n2, u64 S, u64 Sp, int cut) {
  if (a.dbg.counts) { a.dbg.counts[2 * b] = n1; a.dbg.counts[2 * b + 1] = n2; }
  if (a.dbg.mass) { a.dbg.mass[2 * b] = S; a.dbg.mass[2 * b + 1] = Sp; }
  if (a.dbg.cut_ids) a.dbg.cut_ids[b] = cut;
}

// Reported probability of a kept id: its float weight (tg_weight_wide) over
// the top-p mass (fs = f32(S'), 2^-40 units).  S' differs from the exact sum
// of the weights by at most one unit per kept id (plus the weights below
// 2^-40 it leaves out) and is at least 2^40, so the ratio carries only float
// roundings, not the floor of the integer masses.
__device__ __forceinline__ float kept_prob(float y, float m, float fs) {
  return (tg_weight_wide(y, m) * 0x1p40f) / fs;
}

// Called by one whole wave: x is this lane's entry of the kept list sorted
// by (logit desc, id asc) (lane i = rank i), n in [1, 64] valid entries.
__device__ __forceinline__ void wave_finalize(const SampleArgs& a, const Row& r, u64 x, int n) {
  const int lane = lane_id();
  const int b = r.b;
  const float y = comp_y(x);
  const float m = readlane_f32(y, 0);
  const u64 q = lane < n ? tg_q40(tg_weight(y, m)) : 0ull;
  const u64 C = wave_incl_scan(q);
  const u64 S = readlane_u64(C, n - 1);
  int istar = n - 1;
  if (r.top_p < 1.0f) {
    const uint32_t pq = (uint32_t)(r.top_p * 16777216.0f);
    const u64 P = mul_shr24(S, pq);
    const u64 bal = __ballot(lane < n && C >= P);
    istar = __ffsll((long long)bal) - 1;
  }
  const u64 Sp = readlane_u64(C, istar);
  const uint32_t uq = (uint32_t)(r.u * 16777216.0f);
  const u64 t = mul_shr24(Sp, uq);
  const u64 bal2 = __ballot(lane <= istar && C > t);
  const int pick = bal2 ? __ffsll((long long)bal2) - 1 : istar;
  const u64 xp = readlane_u64(x, pick);
  const u64 xc = readlane_u64(x, istar);
  if (lane == 0) {
    a.out[b] = comp_id(xp);
    write_row_diag(a, b, n, istar + 1, S, Sp, comp_id(xc));
  }
  if (a.dbg.kept_ids) {
    int32_t* kid = a.dbg.kept_ids + (long long)b * a.dbg.kept_cap;
    for (int i = lane; i < a.dbg.kept_cap; i += 64) kid[i] = (i < n) ? comp_id(x) : -1;
  }
  if (a.dbg.kept_probs) {
    float* kp = a.dbg.kept_probs + (long long)b * a.dbg.kept_cap;
    const float fs = tg_u64_to_f32(Sp);
    for (int i = lane; i < a.dbg.kept_cap; i += 64) kp[i] = (i <= istar) ? kept_prob(y, m, fs) : 0.0f;
  }
}


template <int BS = NT>
__device__ __forceinline__ void finalize_greedy(const SampleArgs& a, int b, u64 best) {
  const int id = best ? comp_id(best) : -1;
  if (threadIdx.x == 0) {
    a.out[b] = id;
    write_row_diag(a, b, id >= 0, id >= 0, 0, 0, id);
  }
  if (a.dbg.kept_ids) {
    int32_t* kid = a.dbg.kept_ids + (long long)b * a.dbg.kept_cap;
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BS) kid[i] = (i == 0) ? id : -1;
  }
  if (a.dbg.kept_probs) {
    float* kp = a.dbg.kept_probs + (long long)b * a.dbg.kept_cap;
    for (int i = threadIdx.x; i < a.dbg.kept_cap; i += BS) kp[i] = (i == 0 && id >= 0) ? 1.0f : 0.0f;
  }
}

}  // namespace tgs
