// tgs_spec.hip -- speculative-decoding verification on gfx950.
//
// One call verifies B sequences, each with k draft tokens: target logits
// [B, k+1, V] and draft logits [B, k, V].  The row statistics of the
// contract are built from aligned blocks of SPEC_BLOCK ids -- block maximum
// m_b and exact block mass Q_b = sum q40(weight(y, m_b)) -- so every block
// is independent work.  Four launches on the caller's stream:
//
//   spec_block_kernel   one wave per (sequence, row, block): m_b and Q_b
//                       (stochastic rows), or the block's argmax composite
//                       (greedy sequences, target rows only).  This is the
//                       pass over all (2k+1) V logits of a sequence: the
//                       bandwidth of the call.
//   spec_decide_kernel  one workgroup per sequence: row maxima and softmax
//                       denominators from the block terms (pairwise fp32
//                       tree), the accept/reject scan with every draft
//                       position evaluated at once, and the outputs of
//                       greedy, invalid and empty sequences.  Leaves the
//                       row to draw from (residual at the rejected position
//                       or the bonus target row) in the workspace.
//   spec_mass_kernel    one wave per (sequence, block) of that row: the
//                       block's exact draw mass (residual max(pT - pD, 0) or
//                       target weight, as 2^-40 integers).
//   spec_draw_kernel    one workgroup per sequence: id-order scan of the
//                       block masses, then of the chosen block's ids; the
//                       draw.  A residual of mass <= 1e-10 (Q < 110) falls
//                       back to the target row at that position, summed
//                       here by the whole workgroup (p_target <= p_draft
//                       everywhere: rare).
//
// The kernel boundaries order the workspace handoffs; nothing waits on
// another workgroup.  Semantics follow SpeculativeDecode.stepStochastic /
// .step (native-mac/Sources/TinyGPT/SpeculativeDecode.swift:121-210, :41-98)
// with the contract's strict u < pT/pD accept rule and id-order draws.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace spec {

constexpr int WPB = NT / 64;  // waves per workgroup

template <typename Tin>
struct Tile {
  static constexpr int EPV = Elem<Tin>::EPV;
  static constexpr int NV = SPEC_BLOCK / (64 * EPV);  // vectors per lane per block
  static constexpr int EPL = NV * EPV;                // elements per lane per block
};

// id of (vector i, element e) of this lane within block blk
template <typename Tin>
__device__ __forceinline__ int blk_id(int blk, int i, int e) {
  constexpr int EPV = Elem<Tin>::EPV;
  return blk * SPEC_BLOCK + i * 64 * EPV + lane_id() * EPV + e;
}

template <typename Tin>
__device__ __forceinline__ const Tin* row_ptr(const SpecArgs& a, int b, int r) {
  const int k = a.k;
  if (r <= k) return (const Tin*)a.target + ((long long)b * (k + 1) + r) * a.V;
  return (const Tin*)a.draft + ((long long)b * k + (r - k - 1)) * a.V;
}

template <typename Tin>
__device__ __forceinline__ void load_block(const Tin* rowp, int blk, int V, bool aligned,
                                           uint4 (&raw)[Tile<Tin>::NV]) {
#pragma unroll
  for (int i = 0; i < Tile<Tin>::NV; i++) raw[i] = load_vec<Tin>(rowp, blk_id<Tin>(blk, i, 0), V, aligned);
}

// y = z * invT with NaN and -inf mapped to -inf (ids past V were loaded as NaN)
__device__ __forceinline__ float scaled(float z, float invT) {
  const float t = z * invT;
  return (t > -__builtin_inff()) ? t : -__builtin_inff();
}

// Sequence temperature: greedy (T <= 0), the clamped T = max(T, 1e-5) and
// its reciprocal.  NaN T is reported by the decide kernel.
struct SeqT {
  bool greedy;
  float invT;
};
__device__ __forceinline__ SeqT seq_temp(float T) {
  SeqT s;
  s.greedy = !(T > 0.0f);
  const float Tc = T > 1e-5f ? T : 1e-5f;
  s.invT = s.greedy ? 1.0f : 1.0f / Tc;
  return s;
}

// ------------------------------------------------------------------ K1

template <typename Tin>
__global__ __launch_bounds__(NT) void spec_block_kernel(SpecArgs a) {
  using TL = Tile<Tin>;
  const int R = 2 * a.k + 1;
  const long long nwork = (long long)a.B * R * a.nb;
  const long long f = (long long)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (f >= nwork) return;
  const int blk = (int)(f % a.nb);
  const int br = (int)(f / a.nb);
  const int b = br / R, r = br % R;
  const float T = a.T[b];
  if (__builtin_isnan(T)) return;
  const SeqT st = seq_temp(T);
  if (st.greedy && r > a.k) return;  // draft rows unused by greedy verification
  const Tin* rowp = row_ptr<Tin>(a, b, r);
  uint4 raw[TL::NV];
  load_block<Tin>(rowp, blk, a.V, a.aligned, raw);
  const long long o = (long long)br * a.nbs + blk;
  if (st.greedy) {
    u64 arg = 0;
#pragma unroll
    for (int i = 0; i < TL::NV; i++)
#pragma unroll
      for (int e = 0; e < TL::EPV; e++) {
        const float y = scaled(Elem<Tin>::get(raw[i], e), 1.0f);
        if (y > -__builtin_inff()) {
          const u64 c = comp_key(tg_key(y), blk_id<Tin>(blk, i, e));
          arg = c > arg ? c : arg;
        }
      }
    arg = wave_max(arg);
    if (lane_id() == 0) a.blk_q[o] = arg;
    return;
  }
  float y[TL::EPL];
  float mx = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < TL::NV; i++)
#pragma unroll
    for (int e = 0; e < TL::EPV; e++) {
      y[i * TL::EPV + e] = scaled(Elem<Tin>::get(raw[i], e), st.invT);
      mx = fmaxf(mx, y[i * TL::EPV + e]);
    }
  mx = wave_maxf(mx);
  u64 q = 0;
  if (mx > -__builtin_inff()) {
#pragma unroll
    for (int j = 0; j < TL::EPL; j++)
      if (y[j] > -__builtin_inff()) q += tg_q40(tg_weight(y[j], mx));
  }
  q = wave_sum(q);
  if (lane_id() == 0) {
    a.blk_m[o] = mx;
    a.blk_q[o] = q;
  }
}

// ------------------------------------------------------------------ K2

// Sequence state left for the draw kernels.
//   status: 0 all accepted (bonus draw from target row k), 1 rejected at j
//   (residual draw), 2 nothing to draw (outputs complete).
struct alignas(16) SeqState {
  int status, j, pad0, pad1;
  float mt, St, md, Sd;
};
static_assert(sizeof(SeqState) == 32, "state layout");

// Row statistics (m, S) of row r of sequence b from its block terms, by one
// wave: m = max m_b; S = pairwise tree over term_b = (f32(Q_b) 2^-40)
// weight(m_b, m), zero padded to 256 leaves (four per lane).
__device__ __forceinline__ void row_stats(const SpecArgs& a, long long br, float* m_out, float* S_out) {
  const int lane = lane_id();
  float mb[4];
  u64 qb[4];
  float m = -__builtin_inff();
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int i = 4 * lane + j;
    mb[j] = i < a.nb ? a.blk_m[br * a.nbs + i] : -__builtin_inff();
    qb[j] = i < a.nb ? a.blk_q[br * a.nbs + i] : 0ull;
    m = fmaxf(m, mb[j]);
  }
  m = wave_maxf(m);
  float S = 0.0f;
  if (m > -__builtin_inff()) {
    float t[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
      t[j] = (mb[j] > -__builtin_inff()) ? (tg_u64_to_f32(qb[j]) * 0x1p-40f) * tg_weight(mb[j], m) : 0.0f;
    float x = (t[0] + t[1]) + (t[2] + t[3]);
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) x = x + __shfl_xor(x, d, 64);
    S = x;
  }
  *m_out = m;
  *S_out = S;
}

template <typename Tin>
__global__ __launch_bounds__(NT) void spec_decide_kernel(SpecArgs a) {
  __shared__ float sm[2 * SPEC_MAX_K + 1], sS[2 * SPEC_MAX_K + 1];
  __shared__ u64 sarg[SPEC_MAX_K + 1];
  __shared__ unsigned sbad;
  const int b = blockIdx.x;
  if (b >= a.B) return;
  const int k = a.k, R = 2 * k + 1;
  const int w = threadIdx.x >> 6, lane = lane_id();
  const float T = a.T[b];
  const SeqT st = seq_temp(T);
  int* out = a.out + (long long)b * (k + 1);
  SeqState* state = (SeqState*)a.seq_state + b;
  // validation (the CPU restatement's rules): T, draft ids, uniforms
  if (threadIdx.x == 0) sbad = 0u;
  __syncthreads();
  {
    bool bad = __builtin_isnan(T) || (!st.greedy && !(st.invT > 0.0f && __builtin_isfinite(st.invT)));
    for (int j = threadIdx.x; j < k; j += NT) {
      const int d = a.dtok[(long long)b * k + j];
      if (d < 0 || d >= a.V) bad = true;
      if (!st.greedy) {
        const float ua = a.u_acc[(long long)b * k + j];
        if (__builtin_isnan(ua) || ua < 0.0f || ua >= 1.0f) bad = true;
      }
    }
    if (threadIdx.x == 0 && !st.greedy) {
      const float ur = a.u_res[b];
      if (__builtin_isnan(ur) || ur < 0.0f || ur >= 1.0f) bad = true;
    }
    if (bad) atomicOr(&sbad, 1u);
  }
  __syncthreads();
  if (sbad) {
    for (int j = threadIdx.x; j <= k; j += NT) out[j] = j == 0 ? -2 : -1;
    if (threadIdx.x == 0) {
      a.n_acc[b] = -1;
      state->status = 2;
    }
    return;
  }
  const long long br0 = (long long)b * R;
  if (st.greedy) {
    // argmax of target rows 0..k: the largest block composite
    for (int r = w; r <= k; r += WPB) {
      u64 x = 0;
      for (int i = lane; i < a.nb; i += 64) {
        const u64 c = a.blk_q[(br0 + r) * a.nbs + i];
        x = c > x ? c : x;
      }
      x = wave_max(x);
      if (lane == 0) sarg[r] = x;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      int j;
      for (j = 0; j <= k; j++) out[j] = -1;
      for (j = 0; j < k; j++) {
        const u64 c = sarg[j];
        const int am = c ? comp_id(c) : -1;
        out[j] = am;
        if (am != a.dtok[(long long)b * k + j]) break;
      }
      if (j == k) out[k] = sarg[k] ? comp_id(sarg[k]) : -1;
      a.n_acc[b] = j;
      state->status = 2;
    }
    return;
  }
  for (int r = w; r < R; r += WPB) {
    float m, S;
    row_stats(a, br0 + r, &m, &S);
    if (lane == 0) {
      sm[r] = m;
      sS[r] = S;
    }
  }
  __syncthreads();
  if (w != 0) return;
  // every draft position at once (lane j), then the first rejection
  bool acc = true, empty = false;
  float yt = 0.0f, yd = 0.0f;
  int d = 0;
  if (lane < k) {
    d = a.dtok[(long long)b * k + lane];
    yt = scaled(Elem<Tin>::scalar(row_ptr<Tin>(a, b, lane), d), st.invT);
    yd = scaled(Elem<Tin>::scalar(row_ptr<Tin>(a, b, k + 1 + lane), d), st.invT);
  }
  if (lane < k) {
    const float mt = sm[lane], St = sS[lane];
    const float md = sm[k + 1 + lane], Sd = sS[k + 1 + lane];
    if (!(St > 0.0f) || !(Sd > 0.0f)) {
      empty = true;
      acc = false;
    } else {
      const float pt = tg_weight(yt, mt) / St;
      const float pd = tg_weight(yd, md) / Sd;
      const float ratio = pt / fmaxf(pd, 1e-10f);
      acc = a.u_acc[(long long)b * k + lane] < ratio;
    }
  }
  const u64 stop = __ballot(lane < k && !acc);
  const int j = stop ? __ffsll((long long)stop) - 1 : k;
  const bool empty_j = __shfl(empty ? 1 : 0, j < k ? j : 0, 64) != 0 && j < k;
  // i < j <= k <= 64 only for i == lane (this lane's draft token d)
  for (int i = lane; i <= k; i += 64) out[i] = (i < j) ? d : -1;
  if (lane == 0) {
    SeqState s;
    s.pad0 = s.pad1 = 0;
    s.j = j;
    if (empty_j || (j == k && !(sS[k] > 0.0f))) {
      s.status = 2;
      a.n_acc[b] = -1;
    } else if (j < k) {
      s.status = 1;
    } else {
      s.status = 0;
    }
    s.mt = sm[j];
    s.St = sS[j];
    s.md = j < k ? sm[k + 1 + j] : 0.0f;
    s.Sd = j < k ? sS[k + 1 + j] : 0.0f;
    *state = s;
  }
  // an empty row at the stop: every output -1 (the rows after the stop are
  // never examined, as in the serial scan)
  if (empty_j || (j == k && !(sS[k] > 0.0f)))
    for (int i = lane; i <= k; i += 64) out[i] = -1;
}

// ------------------------------------------------------------------ K3 / K4

// Mass of id v of the draw row (0 past V): residual or target weight.
template <typename Tin>
struct DrawRow {
  const Tin* tr;
  const Tin* dr;
  float invT, mt, St, md, Sd;
  int V;
  bool resid;
  __device__ __forceinline__ u64 mass(float zt, float zd) const {
    const float yt = scaled(zt, invT);
    if (!resid) return tg_q40(tg_weight(yt, mt));
    const float yd = scaled(zd, invT);
    const float pa = tg_weight(yt, mt) / St;
    const float pb = tg_weight(yd, md) / Sd;
    return tg_q40(fmaxf(pa - pb, 0.0f));
  }
};

template <typename Tin>
__device__ __forceinline__ DrawRow<Tin> draw_row(const SpecArgs& a, int b, const SeqState& s, bool resid) {
  DrawRow<Tin> d;
  d.invT = seq_temp(a.T[b]).invT;
  d.V = a.V;
  d.resid = resid;
  d.mt = s.mt;
  d.St = s.St;
  d.md = s.md;
  d.Sd = s.Sd;
  d.tr = row_ptr<Tin>(a, b, s.status == 0 ? a.k : s.j);
  d.dr = resid ? row_ptr<Tin>(a, b, a.k + 1 + s.j) : d.tr;
  return d;
}

// Masses of this lane's elements of block blk; ws[i * EPV + e].
template <typename Tin>
__device__ __forceinline__ void block_masses(const SpecArgs& a, const DrawRow<Tin>& dw, int blk,
                                             u64 (&ws)[Tile<Tin>::EPL]) {
  using TL = Tile<Tin>;
  uint4 rt[TL::NV], rd[TL::NV];
  load_block<Tin>(dw.tr, blk, dw.V, a.aligned, rt);
  if (dw.resid) load_block<Tin>(dw.dr, blk, dw.V, a.aligned, rd);
#pragma unroll
  for (int i = 0; i < TL::NV; i++)
#pragma unroll
    for (int e = 0; e < TL::EPV; e++) {
      const float zt = Elem<Tin>::get(rt[i], e);
      const float zd = dw.resid ? Elem<Tin>::get(rd[i], e) : 0.0f;
      ws[i * TL::EPV + e] = dw.mass(zt, zd);  // ids past V were loaded as NaN: mass 0
    }
}

template <typename Tin>
__global__ __launch_bounds__(NT) void spec_mass_kernel(SpecArgs a) {
  using TL = Tile<Tin>;
  const long long f = (long long)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (f >= (long long)a.B * a.nb) return;
  const int b = (int)(f / a.nb), blk = (int)(f % a.nb);
  const SeqState s = ((const SeqState*)a.seq_state)[b];
  if (s.status > 1) return;
  const DrawRow<Tin> dw = draw_row<Tin>(a, b, s, s.status == 1);
  u64 ws[TL::EPL];
  block_masses<Tin>(a, dw, blk, ws);
  u64 q = 0;
#pragma unroll
  for (int j = 0; j < TL::EPL; j++) q += ws[j];
  q = wave_sum(q);
  if (lane_id() == 0) a.blk_w[(long long)b * a.nbs + blk] = q;
}

struct DrawScratch {
  u64 wsum[256];
  u64 t, before;
  int blk, pick;
  u64 total;
};

// Block of the first id whose inclusive prefix (id order) exceeds
// floor(total * uq / 2^24), from the block masses bw[0, nb) (wave 0).
__device__ __forceinline__ void pick_block(const u64* bw, int nb, uint32_t uq, DrawScratch& ds) {
  const int lane = lane_id();
  u64 vals[4];
  u64 ls = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int i = 4 * lane + j;
    vals[j] = i < nb ? bw[i] : 0ull;
    ls += vals[j];
  }
  const u64 incl = wave_incl_scan(ls);
  const u64 total = __shfl(incl, 63, 64);
  const u64 t = mul_shr24(total, uq);
  u64 cum = incl - ls;
  int found = -1;
  u64 before = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    if (found < 0 && cum + vals[j] > t) {
      found = 4 * lane + j;
      before = cum;
    }
    cum += vals[j];
  }
  const u64 bal = __ballot(found >= 0);
  const int first = bal ? __ffsll((long long)bal) - 1 : -1;
  if (lane == 0) {
    ds.blk = -1;
    ds.total = total;
    ds.t = t;
  }
  if (first >= 0 && lane == first) {
    ds.blk = found;
    ds.before = before;
  }
}

// Within block blk (wave 0): the first id whose inclusive prefix exceeds t,
// given the mass `before` of the blocks ahead of it.
template <typename Tin>
__device__ __forceinline__ int pick_in_block(const SpecArgs& a, const DrawRow<Tin>& dw, int blk, u64 t, u64 before) {
  using TL = Tile<Tin>;
  u64 ws[TL::EPL];
  block_masses<Tin>(a, dw, blk, ws);
  u64 run = before;
  int pick = -1;
#pragma unroll
  for (int i = 0; i < TL::NV; i++) {
    u64 ls = 0;
#pragma unroll
    for (int e = 0; e < TL::EPV; e++) ls += ws[i * TL::EPV + e];
    const u64 incl = wave_incl_scan(ls);
    u64 cum = run + incl - ls;
    int mine = -1;
#pragma unroll
    for (int e = 0; e < TL::EPV; e++) {
      if (mine < 0 && cum + ws[i * TL::EPV + e] > t) mine = blk_id<Tin>(blk, i, e);
      cum += ws[i * TL::EPV + e];
    }
    const u64 bal = __ballot(mine >= 0);
    if (pick < 0 && bal) pick = __shfl(mine, __ffsll((long long)bal) - 1, 64);
    run += __shfl(incl, 63, 64);
  }
  return pick;
}

template <typename Tin>
__global__ __launch_bounds__(NT) void spec_draw_kernel(SpecArgs a) {
  __shared__ DrawScratch ds;
  const int b = blockIdx.x;
  if (b >= a.B) return;
  const SeqState s = ((const SeqState*)a.seq_state)[b];
  if (s.status > 1) return;
  const uint32_t uq = (uint32_t)(a.u_res[b] * 16777216.0f);
  const int w = threadIdx.x >> 6;
  const u64* bw = a.blk_w + (long long)b * a.nbs;
  bool resid = s.status == 1;
  if (w == 0) pick_block(bw, a.nb, uq, ds);
  __syncthreads();
  if (resid && ds.total < 110ull) {
    // residual mass <= 1e-10: draw from the target row at the rejected
    // position instead (its block masses summed here)
    resid = false;
    const DrawRow<Tin> dw = draw_row<Tin>(a, b, s, false);
    for (int blk = w; blk < a.nb; blk += WPB) {
      u64 ws[Tile<Tin>::EPL];
      block_masses<Tin>(a, dw, blk, ws);
      u64 q = 0;
#pragma unroll
      for (int j = 0; j < Tile<Tin>::EPL; j++) q += ws[j];
      q = wave_sum(q);
      if (lane_id() == 0) ds.wsum[blk] = q;
    }
    __syncthreads();
    if (w == 0) pick_block(ds.wsum, a.nb, uq, ds);
    __syncthreads();
  }
  if (w != 0) return;
  const DrawRow<Tin> dw = draw_row<Tin>(a, b, s, resid);
  const int pick = ds.blk >= 0 ? pick_in_block<Tin>(a, dw, ds.blk, ds.t, ds.before) : -1;
  if (lane_id() == 0) {
    a.out[(long long)b * (a.k + 1) + s.j] = pick;
    a.n_acc[b] = s.j;
  }
}

template <typename Tin>
hipError_t launch_t(const SpecArgs& a, hipStream_t st) {
  const long long nblk = (long long)a.B * (2 * a.k + 1) * a.nb;
  hipLaunchKernelGGL(spec_block_kernel<Tin>, dim3((unsigned)((nblk + WPB - 1) / WPB)), dim3(NT), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(spec_decide_kernel<Tin>, dim3(a.B), dim3(NT), 0, st, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  const long long nm = (long long)a.B * a.nb;
  hipLaunchKernelGGL(spec_mass_kernel<Tin>, dim3((unsigned)((nm + WPB - 1) / WPB)), dim3(NT), 0, st, a);
  e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(spec_draw_kernel<Tin>, dim3(a.B), dim3(NT), 0, st, a);
  return hipGetLastError();
}

}  // namespace spec

hipError_t launch_spec(const SpecArgs& a, int dtype, hipStream_t st) {
  return dtype == 1 ? spec::launch_t<uint16_t>(a, st) : spec::launch_t<float>(a, st);
}

}  // namespace tgs
