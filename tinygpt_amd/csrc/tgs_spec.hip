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
#include <algorithm>

#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace spec {

constexpr int WPB = NT / 64;  // waves per workgroup
constexpr int K1_WG_PER_CU = 8;  // most resident workgroups per CU of the block kernel's grid

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

// A block wholly inside the row of an aligned row (every block but a row's
// last when V is not a multiple of the block) takes plain 16-byte loads
// behind one wave-uniform test; the others test each vector.
template <typename Tin>
__device__ __forceinline__ void load_block(const Tin* rowp, int blk, int V, bool aligned,
                                           uint4 (&raw)[Tile<Tin>::NV]) {
  if (aligned && (blk + 1) * SPEC_BLOCK <= V) {
#pragma unroll
    for (int i = 0; i < Tile<Tin>::NV; i++) raw[i] = *(const uint4*)(rowp + blk_id<Tin>(blk, i, 0));
    return;
  }
#pragma unroll
  for (int i = 0; i < Tile<Tin>::NV; i++) raw[i] = load_vec<Tin>(rowp, blk_id<Tin>(blk, i, 0), V, aligned);
}

// Sequence temperature: greedy (T <= 0), the clamped T = max(T, 1e-5), its
// reciprocal and the mode of the exact divide (greedy: T = 1).  NaN T is
// reported by the decide kernel.
struct SeqT {
  bool greedy, tnan;
  float T, rT;
  int tdiv;
};
__device__ __forceinline__ SeqT seq_temp(float T) {
  SeqT s;
  s.tnan = __builtin_isnan(T);
  s.greedy = !(T > 0.0f);
  const float Tc = T > 1e-5f ? T : 1e-5f;
  s.T = s.greedy ? 1.0f : Tc;
  s.rT = 1.0f / s.T;
  s.tdiv = tg_div_t_mode(s.T);
  return s;
}

// y = z / T (correctly rounded) with NaN and -inf mapped to -inf (ids past V
// were loaded as NaN)
__device__ __forceinline__ float scaled(float z, const SeqT& st) {
  const float t = tg_div_t(z, st.T, st.rT, st.tdiv);
  return (t > -__builtin_inff()) ? t : -__builtin_inff();
}

// ------------------------------------------------------------------ K1

// Block (b, r, blk) of the flat index, with the sequence's temperature;
// live: computed (NaN T is reported by the decide kernel, greedy sequences
// skip their draft rows).  A wave walks consecutive blocks and updates the
// cursor incrementally (wave-uniform scalar arithmetic; the temperature is
// read only when the sequence changes, so that no load in the walk waits
// for the blocks in flight).
struct BlockRef {
  int b, r, blk;
  bool live, greedy;
  SeqT st;
};
__device__ __forceinline__ void block_ref_temp(const SpecArgs& a, BlockRef& x) {
  const float T = a.T[x.b];
  x.st = seq_temp(T);
  x.greedy = x.st.greedy;
}
__device__ __forceinline__ bool block_live(const SpecArgs& a, const BlockRef& x) {
  return !x.st.tnan && !(x.greedy && x.r > a.k);
}
__device__ __forceinline__ BlockRef block_ref(const SpecArgs& a, int f) {
  const int R = 2 * a.k + 1;
  BlockRef x;
  x.blk = f % a.nb;
  const int br = f / a.nb;
  x.b = br / R;
  x.r = br % R;
  block_ref_temp(a, x);
  x.live = block_live(a, x);
  return x;
}
__device__ __forceinline__ BlockRef block_next(const SpecArgs& a, const BlockRef& x) {
  BlockRef y = x;
  if (++y.blk == a.nb) {
    y.blk = 0;
    if (++y.r == 2 * a.k + 1) {
      y.r = 0;
      y.b++;
      block_ref_temp(a, y);
    }
  }
  y.live = block_live(a, y);
  return y;
}

// A block of finite maximum whose exact mass waits, as per-lane partial
// sums, to be reduced together with the wave's next such block: one grouped
// reduction per pair of blocks instead of one per block (exact: integers).
struct PendingMass {
  u64 q;        // this lane's partial sum
  float m;      // the block's maximum
  long long o;  // its slot; -1: none (wave-uniform)
};
__device__ __forceinline__ void flush_pending(const SpecArgs& a, PendingMass& p) {
  if (p.o < 0) return;
  const u64 q = wave_sum(p.q);
  if (lane_id() == 0) {
    a.blk_m[p.o] = p.m;
    a.blk_q[p.o] = q;
  }
  p.o = -1;
}

// One block's statistics from its loaded vectors; lane 0 stores them (lane
// 32 too when a pending block is reduced with this one).
template <typename Tin>
__device__ __forceinline__ void block_stats(const SpecArgs& a, const BlockRef& x, const uint4 (&raw)[Tile<Tin>::NV],
                                            PendingMass& pend) {
  using TL = Tile<Tin>;
  const long long o = ((long long)x.b * (2 * a.k + 1) + x.r) * a.nbs + x.blk;
  if (x.greedy) {
    u64 arg = 0;
#pragma unroll
    for (int i = 0; i < TL::NV; i++)
#pragma unroll
      for (int e = 0; e < TL::EPV; e++) {
        const float y = scaled(Elem<Tin>::get(raw[i], e), x.st);
        if (y > -__builtin_inff()) {
          const u64 c = comp_key(tg_key(y), blk_id<Tin>(x.blk, i, e));
          arg = c > arg ? c : arg;
        }
      }
    arg = wave_max(arg);
    if (lane_id() == 0) a.blk_q[o] = arg;
    return;
  }
  // y = z / T; NaN and -inf never raise the maximum and weigh 0 (y - m is
  // NaN or -inf there), so they need no mapping.  With a power-of-two T
  // (C5's T = 1) v holds the logits z themselves: y = z rT is monotone in
  // z, so m = RN(max z rT), and the mass term of y - m is that of the fused
  // fma(z, rT, -m) (z rT is exact, or below the normal range where both
  // forms weigh the same; tests/cpu_sim/numerics.cpp, mode pow2fma).
  const bool pow2 = x.st.tdiv == TDIV_POW2;
  float v[TL::EPL];
  float mx = -__builtin_inff();
#pragma unroll
  for (int i = 0; i < TL::NV; i++)
#pragma unroll
    for (int e = 0; e < TL::EPV; e++) {
      const float z = Elem<Tin>::get(raw[i], e);
      v[i * TL::EPV + e] = pow2 ? z : tg_div_t(z, x.st.T, x.st.rT, x.st.tdiv);
      mx = fmaxf(mx, v[i * TL::EPV + e]);
    }
  mx = wave_maxf(mx);
  if (pow2) mx = mx * x.st.rT;
  u64 q = 0;
  if (mx > -__builtin_inff() && mx < __builtin_inff()) {
    // y - m <= 0 (y == m gives +-0 and weight 1): the non-positive exp, and
    // exact masses summed per lane in f64
    double qd = 0.0;
    if (pow2) {
#pragma unroll
      for (int j = 0; j < TL::EPL; j++) qd += tg_q40d_exp_nonpos(__builtin_fmaf(v[j], x.st.rT, -mx));
    } else {
#pragma unroll
      for (int j = 0; j < TL::EPL; j++) qd += tg_q40d_exp_nonpos(v[j] - mx);
    }
    q = (u64)qd;
    if (pend.o < 0) {
      pend.q = q;
      pend.m = mx;
      pend.o = o;
      return;
    }
    // lanes 0-31 end with the pending block's sum, lanes 32-63 with this one's
    const u64 pair[2] = {pend.q, q};
    const u64 s2 = wave_sum_groups<2>(pair);
    const int lane = lane_id();
    if (lane == 0) {
      a.blk_m[pend.o] = pend.m;
      a.blk_q[pend.o] = s2;
    }
    if (lane == 32) {
      a.blk_m[o] = mx;
      a.blk_q[o] = s2;
    }
    pend.o = -1;
    return;
  } else if (mx > -__builtin_inff()) {
    // a +inf logit in the block (weight(inf, inf) = 1, everything else 0)
#pragma unroll
    for (int j = 0; j < TL::EPL; j++) {
      const float y = pow2 ? v[j] * x.st.rT : v[j];
      const float yy = (y > -__builtin_inff()) ? y : -__builtin_inff();
      if (yy > -__builtin_inff()) q += tg_q40(tg_weight(yy, mx));
    }
  }
  q = wave_sum(q);
  if (lane_id() == 0) {
    a.blk_m[o] = mx;
    a.blk_q[o] = q;
  }
}

// K1: every wave takes a run of consecutive blocks (about eight at C5's
// size), the loads of its next block issued before the current block is
// reduced.
template <typename Tin>
__global__ __launch_bounds__(NT) void spec_block_kernel(SpecArgs a) {
  using TL = Tile<Tin>;
  const int nwork = a.B * (2 * a.k + 1) * a.nb;
  const int nwaves = (int)gridDim.x * WPB;
  const int gw = __builtin_amdgcn_readfirstlane((int)blockIdx.x * WPB + (int)(threadIdx.x >> 6));
  const int per = (nwork + nwaves - 1) / nwaves;
  const int f0 = gw * per;
  const int n = min(per, nwork - f0);
  if (n <= 0) return;
  BlockRef x = block_ref(a, f0);
  PendingMass pend;
  pend.q = 0;
  pend.m = 0.0f;
  pend.o = -1;
  uint4 cur[TL::NV];
  if (x.live) load_block<Tin>(row_ptr<Tin>(a, x.b, x.r), x.blk, a.V, a.aligned, cur);
  for (int i = 0; i < n; i++) {
    const bool more = i + 1 < n;
    BlockRef xn = x;
    uint4 nxt[TL::NV];
    if (more) {
      xn = block_next(a, x);
      if (xn.live) load_block<Tin>(row_ptr<Tin>(a, xn.b, xn.r), xn.blk, a.V, a.aligned, nxt);
    }
    if (x.live) block_stats<Tin>(a, x, cur, pend);
    if (!more) break;
#pragma unroll
    for (int v = 0; v < TL::NV; v++) cur[v] = nxt[v];
    x = xn;
  }
  flush_pending(a, pend);
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
static_assert(Tile<float>::NV <= SPEC_GROUPS && Tile<uint16_t>::NV <= SPEC_GROUPS, "group sums per block");

// Block terms of one row, four per lane (blocks 4 lane + j; -inf / 0 past
// the row's blocks).
struct RowTerms {
  float mb[4];
  u64 qb[4];
};
__device__ __forceinline__ RowTerms row_terms(const SpecArgs& a, long long br) {
  const int lane = lane_id();
  RowTerms t;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int i = 4 * lane + j;
    t.mb[j] = i < a.nb ? a.blk_m[br * a.nbs + i] : -__builtin_inff();
    t.qb[j] = i < a.nb ? a.blk_q[br * a.nbs + i] : 0ull;
  }
  return t;
}

// Row statistics (m, S) of a row from its block terms, by one wave:
// m = max m_b; S = pairwise tree over term_b = (f32(Q_b) 2^-40)
// weight(m_b, m), zero padded to 256 leaves (four per lane).
__device__ __forceinline__ void row_stats(const RowTerms& tt, float* m_out, float* S_out) {
  const float (&mb)[4] = tt.mb;
  const u64 (&qb)[4] = tt.qb;
  float m = fmaxf(fmaxf(mb[0], mb[1]), fmaxf(mb[2], mb[3]));
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

constexpr int DT = 1024;        // decide kernel: threads per workgroup
constexpr int DW = DT / 64;    // its waves

template <typename Tin>
__global__ __launch_bounds__(DT) void spec_decide_kernel(SpecArgs a) {
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
  // wave 0, lane j < k: draft token j, its uniform and its two logits (the
  // id clamped into the row for the load; an invalid id fails validation)
  int d = 0;
  float ua = 0.0f, zt = 0.0f, zd = 0.0f;
  if (w == 0 && lane < k) {
    d = a.dtok[(long long)b * k + lane];
    ua = a.u_acc[(long long)b * k + lane];
    const int dc = d < 0 ? 0 : (d >= a.V ? a.V - 1 : d);
    zt = Elem<Tin>::scalar(row_ptr<Tin>(a, b, lane), dc);
    zd = Elem<Tin>::scalar(row_ptr<Tin>(a, b, k + 1 + lane), dc);
  }
  // validation (the CPU restatement's rules): T, draft ids, uniforms
  if (w == 0) {
    bool bad = __builtin_isnan(T) || (!st.greedy && !(st.rT > 0.0f && __builtin_isfinite(st.rT)));
    if (lane < k) {
      if (d < 0 || d >= a.V) bad = true;
      if (!st.greedy && (__builtin_isnan(ua) || ua < 0.0f || ua >= 1.0f)) bad = true;
    }
    if (lane == 0 && !st.greedy) {
      const float ur = a.u_res[b];
      if (__builtin_isnan(ur) || ur < 0.0f || ur >= 1.0f) bad = true;
    }
    const u64 bb = __ballot(bad);
    if (lane == 0) sbad = bb ? 1u : 0u;
  }
  // row statistics (stochastic) or argmax (greedy), one row per wave
  const long long br0 = (long long)b * R;
  if (st.greedy) {
    for (int r = w; r <= k; r += DW) {
      u64 x = 0;
      for (int i = lane; i < a.nb; i += 64) {
        const u64 c = a.blk_q[(br0 + r) * a.nbs + i];
        x = c > x ? c : x;
      }
      x = wave_max(x);
      if (lane == 0) sarg[r] = x;
    }
  } else if (!__builtin_isnan(T)) {
    // a wave's rows r and r + DW in pairs: both rows' terms requested
    // before either is reduced (C5's 17 rows: one pair for wave 0)
    for (int r = w; r < R; r += 2 * DW) {
      const bool two = r + DW < R;
      const RowTerms t0 = row_terms(a, br0 + r);
      RowTerms t1 = {};
      if (two) t1 = row_terms(a, br0 + r + DW);
      float m, S;
      row_stats(t0, &m, &S);
      if (lane == 0) {
        sm[r] = m;
        sS[r] = S;
      }
      if (two) {
        row_stats(t1, &m, &S);
        if (lane == 0) {
          sm[r + DW] = m;
          sS[r + DW] = S;
        }
      }
    }
  }
  __syncthreads();
  if (w != 0) return;
  if (sbad) {
    for (int i = lane; i <= k; i += 64) out[i] = i == 0 ? -2 : -1;
    if (lane == 0) {
      a.n_acc[b] = -1;
      state->status = 2;
    }
    return;
  }
  if (st.greedy) {
    // accept while the target argmax equals the draft token (lane j: position j)
    const int am = lane < k ? (sarg[lane] ? comp_id(sarg[lane]) : -1) : -1;
    const u64 miss = __ballot(lane < k && am != d);
    const int j = miss ? __ffsll((long long)miss) - 1 : k;  // first mismatch, or k
    // accepted tokens, then the correction (or the bonus argmax at k)
    for (int i = lane; i <= k; i += 64) out[i] = i <= j ? (sarg[i] ? comp_id(sarg[i]) : -1) : -1;
    if (lane == 0) {
      a.n_acc[b] = j;
      state->status = 2;
    }
    return;
  }
  // every draft position at once (lane j), then the first rejection
  bool acc = true, empty = false;
  if (lane < k) {
    const float yt = scaled(zt, st), yd = scaled(zd, st);
    const float mt = sm[lane], St = sS[lane];
    const float md = sm[k + 1 + lane], Sd = sS[k + 1 + lane];
    if (!(St > 0.0f) || !(Sd > 0.0f)) {
      empty = true;
      acc = false;
    } else {
      const float pt = tg_weight(yt, mt) / St;
      const float pd = tg_weight(yd, md) / Sd;
      const float ratio = pt / fmaxf(pd, 1e-10f);
      acc = ua < ratio;
    }
  }
  const u64 stop = __ballot(lane < k && !acc);
  const int j = stop ? __ffsll((long long)stop) - 1 : k;
  const bool empty_j = j < k && __shfl(empty ? 1 : 0, j < k ? j : 0, 64) != 0;
  const bool none = empty_j || (j == k && !(sS[k] > 0.0f));
  // i < j <= k <= 64 only for i == lane (this lane's draft token d); an empty
  // row at the stop makes every output -1 (the rows after the stop are never
  // examined, as in the serial scan)
  for (int i = lane; i <= k; i += 64) out[i] = (!none && i < j) ? d : -1;
  if (lane == 0) {
    SeqState s;
    s.pad0 = s.pad1 = 0;
    s.j = j;
    if (none) {
      s.status = 2;
      a.n_acc[b] = -1;
    } else {
      s.status = j < k ? 1 : 0;
    }
    s.mt = sm[j];
    s.St = sS[j];
    s.md = j < k ? sm[k + 1 + j] : 0.0f;
    s.Sd = j < k ? sS[k + 1 + j] : 0.0f;
    *state = s;
  }
}

// ------------------------------------------------------------------ K3 / K4

// Mass of one id of the draw row: the residual q40(max(pT - pD, 0)) or the
// target weight q40(weight(yt, mt)), both as exact integer-valued doubles.
// With finite row maxima (the common case) the weights use the non-positive
// exp and the divisions by the softmax denominators (>= 1) the reciprocal
// with one correction; both equal the canonical operations bit for bit.
template <typename Tin>
struct DrawRow {
  const Tin* tr;
  const Tin* dr;
  SeqT st;
  float mt, St, md, Sd, rSt, rSd;
  int V;
  bool resid, fast;
  __device__ __forceinline__ double mass(float zt, float zd) const {
    if (fast) {
      // a power-of-two T: y - m as one fma (the block kernel's form; the
      // weight, and so every mass below, is the same bit for bit)
      const bool p2 = st.tdiv == TDIV_POW2;
      const float xt = p2 ? __builtin_fmaf(zt, st.rT, -mt) : tg_div_t(zt, st.T, st.rT, st.tdiv) - mt;
      if (!resid) return tg_q40d_exp_nonpos(xt);
      const float wt = tg_expf_nonpos(xt);
      const float xd = p2 ? __builtin_fmaf(zd, st.rT, -md) : tg_div_t(zd, st.T, st.rT, st.tdiv) - md;
      const float wd = tg_expf_nonpos(xd);
      const float pa = tg_div_rcp(wt, St, rSt);
      const float pb = tg_div_rcp(wd, Sd, rSd);
      return tg_q40d(fmaxf(pa - pb, 0.0f));
    }
    const float yt = scaled(zt, st);
    if (!resid) return tg_q40d(tg_weight(yt, mt));
    const float yd = scaled(zd, st);
    const float pa = tg_weight(yt, mt) / St;
    const float pb = tg_weight(yd, md) / Sd;
    return tg_q40d(fmaxf(pa - pb, 0.0f));
  }
};

template <typename Tin>
__device__ __forceinline__ DrawRow<Tin> draw_row(const SpecArgs& a, int b, const SeqState& s, bool resid) {
  DrawRow<Tin> d;
  d.st = seq_temp(a.T[b]);
  d.V = a.V;
  d.resid = resid;
  d.mt = s.mt;
  d.St = s.St;
  d.md = s.md;
  d.Sd = s.Sd;
  d.rSt = 1.0f / s.St;
  d.rSd = resid ? 1.0f / s.Sd : 1.0f;
  d.fast = s.mt < __builtin_inff() && (!resid || s.md < __builtin_inff());
  d.tr = row_ptr<Tin>(a, b, s.status == 0 ? a.k : s.j);
  d.dr = resid ? row_ptr<Tin>(a, b, a.k + 1 + s.j) : d.tr;
  return d;
}

// Masses of this lane's EPV ids of vector group i of block blk (ids past V
// were loaded as NaN: mass 0).
template <typename Tin>
__device__ __forceinline__ void group_masses(const DrawRow<Tin>& dw, const uint4& rt, const uint4& rd,
                                             double (&ws)[Elem<Tin>::EPV]) {
#pragma unroll
  for (int e = 0; e < Elem<Tin>::EPV; e++)
    ws[e] = dw.mass(Elem<Tin>::get(rt, e), dw.resid ? Elem<Tin>::get(rd, e) : 0.0f);
}

// K3: per (sequence, block) the draw mass of each vector group of the block
// (group i: ids blk*SPEC_BLOCK + i*64*EPV + [0, 64*EPV)).
template <typename Tin>
__global__ __launch_bounds__(NT) void spec_mass_kernel(SpecArgs a) {
  using TL = Tile<Tin>;
  const long long f = (long long)blockIdx.x * WPB + (threadIdx.x >> 6);
  if (f >= (long long)a.B * a.nb) return;
  const int b = (int)(f / a.nb), blk = (int)(f % a.nb);
  const SeqState s = ((const SeqState*)a.seq_state)[b];
  if (s.status > 1) return;
  const DrawRow<Tin> dw = draw_row<Tin>(a, b, s, s.status == 1);
  uint4 rt[TL::NV], rd[TL::NV];
  load_block<Tin>(dw.tr, blk, dw.V, a.aligned, rt);
  if (dw.resid) load_block<Tin>(dw.dr, blk, dw.V, a.aligned, rd);
  u64* gw = a.blk_w + ((long long)b * a.nbs + blk) * SPEC_GROUPS;
  u64 gq[TL::NV];
#pragma unroll
  for (int i = 0; i < TL::NV; i++) {
    double ws[TL::EPV];
    group_masses<Tin>(dw, rt[i], dw.resid ? rd[i] : rt[i], ws);
    double ls = 0.0;
#pragma unroll
    for (int e = 0; e < TL::EPV; e++) ls += ws[e];
    gq[i] = (u64)ls;
  }
  // the groups' sums in one reduction: lane 64 / NV * i holds group i's
  const u64 q = wave_sum_groups<TL::NV>(gq);
  constexpr int LPG = 64 / TL::NV;
  if ((lane_id() & (LPG - 1)) == 0) gw[lane_id() / LPG] = q;
}

struct DrawScratch {
  u64 wsum[256];
  u64 t, before;
  int blk, pick;
  u64 total;
};

// Block of the first id whose inclusive prefix (id order) exceeds
// floor(total * uq / 2^24), from the block masses bw(i), i < nb (wave 0).
template <class BW>
__device__ __forceinline__ void pick_block(BW bw, int nb, uint32_t uq, DrawScratch& ds) {
  const int lane = lane_id();
  u64 vals[4];
  u64 ls = 0;
#pragma unroll
  for (int j = 0; j < 4; j++) {
    const int i = 4 * lane + j;
    vals[j] = i < nb ? bw(i) : 0ull;
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
  // one lane writes the result (the first lane that found the block)
  const u64 bal = __ballot(found >= 0);
  const int first = bal ? __ffsll((long long)bal) - 1 : 0;
  const int fb = __shfl(found, first, 64);
  const u64 fbefore = __shfl(before, first, 64);
  if (lane == 0) {
    ds.blk = fb;
    ds.before = fbefore;
    ds.total = total;
    ds.t = t;
  }
}

// Within vector group i of block blk (wave 0): the first id whose inclusive
// prefix exceeds t, given the mass `run` of everything ahead of the group;
// -1 when the group does not reach t.
template <typename Tin>
__device__ __forceinline__ int pick_in_group(const SpecArgs& a, const DrawRow<Tin>& dw, int blk, int i, u64 t,
                                             u64 run) {
  constexpr int EPV = Elem<Tin>::EPV;
  const int v = blk_id<Tin>(blk, i, 0);
  const uint4 rt = load_vec<Tin>(dw.tr, v, dw.V, a.aligned);
  const uint4 rd = dw.resid ? load_vec<Tin>(dw.dr, v, dw.V, a.aligned) : rt;
  double ws[EPV];
  group_masses<Tin>(dw, rt, rd, ws);
  u64 ls = 0;
#pragma unroll
  for (int e = 0; e < EPV; e++) ls += (u64)ws[e];
  const u64 incl = wave_incl_scan(ls);
  u64 cum = run + incl - ls;
  int mine = -1;
#pragma unroll
  for (int e = 0; e < EPV; e++) {
    if (mine < 0 && cum + (u64)ws[e] > t) mine = v + e;
    cum += (u64)ws[e];
  }
  const u64 bal = __ballot(mine >= 0);
  return bal ? __shfl(mine, __ffsll((long long)bal) - 1, 64) : -1;
}

// Within block blk (wave 0), group by group.
template <typename Tin>
__device__ __forceinline__ int pick_in_block(const SpecArgs& a, const DrawRow<Tin>& dw, int blk, u64 t, u64 before) {
  u64 run = before;
  for (int i = 0; i < Tile<Tin>::NV; i++) {
    const int p = pick_in_group<Tin>(a, dw, blk, i, t, run);
    if (p >= 0) return p;
    // mass of the group, for the next one
    constexpr int EPV = Elem<Tin>::EPV;
    const int v = blk_id<Tin>(blk, i, 0);
    const uint4 rt = load_vec<Tin>(dw.tr, v, dw.V, a.aligned);
    const uint4 rd = dw.resid ? load_vec<Tin>(dw.dr, v, dw.V, a.aligned) : rt;
    double ws[EPV];
    group_masses<Tin>(dw, rt, rd, ws);
    double ls = 0.0;
#pragma unroll
    for (int e = 0; e < EPV; e++) ls += ws[e];
    run += wave_sum((u64)ls);
  }
  return -1;
}

template <typename Tin>
__global__ __launch_bounds__(NT) void spec_draw_kernel(SpecArgs a) {
  using TL = Tile<Tin>;
  __shared__ DrawScratch ds;
  const int b = blockIdx.x;
  if (b >= a.B) return;
  const SeqState s = ((const SeqState*)a.seq_state)[b];
  if (s.status > 1) return;
  const uint32_t uq = (uint32_t)(a.u_res[b] * 16777216.0f);
  const int w = threadIdx.x >> 6;
  const u64* gw = a.blk_w + (long long)b * a.nbs * SPEC_GROUPS;
  bool resid = s.status == 1;
  if (w == 0)
    pick_block([&](int i) {
      u64 x = 0;
#pragma unroll
      for (int g = 0; g < TL::NV; g++) x += gw[i * SPEC_GROUPS + g];
      return x;
    }, a.nb, uq, ds);
  __syncthreads();
  if (resid && ds.total < 110ull) {
    // residual mass <= 1e-10: draw from the target row at the rejected
    // position instead (its block masses summed here, id order within the
    // chosen block group by group)
    resid = false;
    const DrawRow<Tin> dw = draw_row<Tin>(a, b, s, false);
    for (int blk = w; blk < a.nb; blk += WPB) {
      uint4 rt[TL::NV];
      load_block<Tin>(dw.tr, blk, dw.V, a.aligned, rt);
      double ls = 0.0;
#pragma unroll
      for (int i = 0; i < TL::NV; i++) {
        double ws[TL::EPV];
        group_masses<Tin>(dw, rt[i], rt[i], ws);
#pragma unroll
        for (int e = 0; e < TL::EPV; e++) ls += ws[e];
      }
      const u64 q = wave_sum((u64)ls);
      if (lane_id() == 0) ds.wsum[blk] = q;
    }
    __syncthreads();
    if (w == 0) pick_block([&](int i) { return ds.wsum[i]; }, a.nb, uq, ds);
    __syncthreads();
    if (w != 0) return;
    const int pick = ds.blk >= 0 ? pick_in_block<Tin>(a, dw, ds.blk, ds.t, ds.before) : -1;
    if (lane_id() == 0) {
      a.out[(long long)b * (a.k + 1) + s.j] = pick;
      a.n_acc[b] = s.j;
    }
    return;
  }
  if (w != 0) return;
  int pick = -1;
  if (ds.blk >= 0) {
    // the group of the chosen block that holds the draw, from its stored
    // group masses, then the id within the group
    const u64* g = gw + (long long)ds.blk * SPEC_GROUPS;
    u64 run = ds.before;
    int gi = TL::NV - 1;
    for (int i = 0; i < TL::NV; i++) {
      if (run + g[i] > ds.t) {
        gi = i;
        break;
      }
      run += g[i];
    }
    const DrawRow<Tin> dw = draw_row<Tin>(a, b, s, resid);
    pick = pick_in_group<Tin>(a, dw, ds.blk, gi, ds.t, run);
  }
  if (lane_id() == 0) {
    a.out[(long long)b * (a.k + 1) + s.j] = pick;
    a.n_acc[b] = s.j;
  }
}

template <typename Tin>
hipError_t launch_t(const SpecArgs& a, hipStream_t st) {
  // the block kernel's grid: as many workgroups per CU as its registers let
  // stay resident (asked once per element type), at most K1_WG_PER_CU, so
  // that every wave's run of blocks starts at once
  static int per_cu = 0;
  if (per_cu == 0) {
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, spec_block_kernel<Tin>, NT, 0) != hipSuccess || n < 1) n = 1;
    per_cu = std::min(n, K1_WG_PER_CU);
  }
  const long long nblk = (long long)a.B * (2 * a.k + 1) * a.nb;
  const long long g1 = std::min<long long>((nblk + WPB - 1) / WPB, (long long)a.ncu * per_cu);
  hipLaunchKernelGGL(spec_block_kernel<Tin>, dim3((unsigned)g1), dim3(NT), 0, st, a);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(spec_decide_kernel<Tin>, dim3(a.B), dim3(DT), 0, st, a);
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
