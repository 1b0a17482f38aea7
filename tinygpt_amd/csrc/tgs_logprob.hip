// tgs_logprob.hip -- log-probability of a given token under the softmax of a
// row of raw logits (teacher-forced scoring: log(softmax(x))[tok] =
// x[tok] - logsumexp(x)), for B rows.
//
// HBM-bound: one read of every logit, 2 or 4 bytes, against about six VALU
// operations.  Workgroups of 256 threads stream 16-byte vectors (four issued
// per thread before any is used) and keep an online pair (m, s): the running
// maximum and sum of exp(x - m), rescaled when m grows; exp is exp2 of
// x * log2(e) - m * log2(e) (one fused multiply-add and one v_exp_f32).
// A batch of fewer rows than the chip holds workgroups splits each row into
// S chunks whose (m, s) pairs a second, one-wave-per-row kernel combines.
//
// IEEE behaviour: -inf logits add nothing; a NaN logit, a +inf logit or a
// row of only -inf gives NaN; a token outside [0, V) gives NaN.
#include "tgs_device.h"
#include "tgs_kernels.h"
#include "tgs_row.h"

namespace tgs {
namespace lp {

constexpr int LT = LP_NT;  // threads per workgroup
constexpr int UNR = 4;     // vectors in flight per thread
constexpr float LOG2E = 1.4426950408889634f;

struct Pair {
  float m, s;
};

// (m, s) of the union of two parts: the larger maximum, the other sum scaled
// onto it (exp2 of the difference, exactly 1 when the maxima are equal).
__device__ __forceinline__ Pair merge(Pair a, Pair b) {
  const float m = fmaxf(a.m, b.m);
  const float sa = a.m == m ? a.s : a.s * exp2f((a.m - m) * LOG2E);
  const float sb = b.m == m ? b.s : b.s * exp2f((b.m - m) * LOG2E);
  return Pair{m, sa + sb};
}

// Adds n logits of one batch to (m, s).  A NaN logit makes s NaN; a row
// maximum of -inf keeps s at 0.
template <int N>
__device__ __forceinline__ void accumulate(Pair& p, const float (&x)[N]) {
  float bm = x[0];
#pragma unroll
  for (int i = 1; i < N; i++) bm = fmaxf(bm, x[i]);
  const float m = fmaxf(p.m, bm);
  if (m == -__builtin_inff()) {
#pragma unroll
    for (int i = 0; i < N; i++) p.s += (x[i] == x[i]) ? 0.0f : x[i];  // NaN propagates
    return;
  }
  p.s = (p.m == m) ? p.s : p.s * exp2f((p.m - m) * LOG2E);
  const float mL = m * LOG2E;
  float acc = 0.0f;
#pragma unroll
  for (int i = 0; i < N; i++) acc += exp2f(__builtin_fmaf(x[i], LOG2E, -mL));
  p.s += acc;
  p.m = m;
}

// logsumexp of a row from its pair; NaN for a row of only -inf (and, through
// s, for a row holding NaN or +inf).
__device__ __forceinline__ float row_lse(Pair p) {
  return p.m == -__builtin_inff() ? __builtin_nanf("") : p.m + logf(p.s);
}

__device__ __forceinline__ Pair wave_merge(Pair p) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    Pair q;
    q.m = tg_u2f(__shfl_xor(tg_f2u(p.m), o, 64));
    q.s = tg_u2f(__shfl_xor(tg_f2u(p.s), o, 64));
    p = merge(p, q);
  }
  return p;
}

// Workgroup (row b, chunk c) over ids [c L, min(V, (c + 1) L)).
template <typename Tin>
__global__ __launch_bounds__(LT) void chunk_kernel(LogprobArgs a) {
  constexpr int EPV = Elem<Tin>::EPV;
  __shared__ Pair red[LT / 64];
  const int b = blockIdx.x / a.S, c = blockIdx.x % a.S;
  if (b >= a.B) return;
  const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
  // the token's logit, requested at entry (used at the end when S == 1)
  float xtok = __builtin_nanf("");
  if (a.S == 1 && threadIdx.x == 0) {
    const int tok = a.tokens[b];
    if (tok >= 0 && tok < a.V) xtok = Elem<Tin>::scalar(rowp, tok);
  }
  const int v0 = c * a.L;
  const int v1 = v0 + a.L < a.V ? v0 + a.L : a.V;
  Pair p{-__builtin_inff(), 0.0f};
  // whole vectors: [v0, vend) when rows are 16-byte aligned, else none
  const int vend = a.aligned ? v0 + (v1 - v0) / EPV * EPV : v0;
  const int nvec = (vend - v0) / EPV;
  int i = threadIdx.x;
  for (; i + (UNR - 1) * LT < nvec; i += UNR * LT) {
    uint4 raw[UNR];
#pragma unroll
    for (int u = 0; u < UNR; u++) raw[u] = tg_load_nt(rowp + v0 + (i + u * LT) * EPV);
    float x[UNR * EPV];
#pragma unroll
    for (int u = 0; u < UNR; u++)
#pragma unroll
      for (int e = 0; e < EPV; e++) x[u * EPV + e] = Elem<Tin>::get(raw[u], e);
    accumulate(p, x);
  }
  for (; i < nvec; i += LT) {
    const uint4 raw = tg_load_nt(rowp + v0 + i * EPV);
    float x[EPV];
#pragma unroll
    for (int e = 0; e < EPV; e++) x[e] = Elem<Tin>::get(raw, e);
    accumulate(p, x);
  }
  for (int v = vend + (int)threadIdx.x; v < v1; v += LT) {  // unaligned rows, the row's tail
    float x[1] = {Elem<Tin>::scalar(rowp, v)};
    accumulate(p, x);
  }
  p = wave_merge(p);
  if (lane_id() == 0) red[threadIdx.x >> 6] = p;
  __syncthreads();
  if (threadIdx.x == 0) {
    Pair q = red[0];
#pragma unroll
    for (int w = 1; w < LT / 64; w++) q = merge(q, red[w]);
    if (a.S == 1) {
      const float lse = row_lse(q);
      a.out_lp[b] = xtok - lse;
      if (a.out_lse) a.out_lse[b] = lse;
    } else {
      float* pp = a.part + 2 * ((long long)b * a.S + c);
      pp[0] = q.m;
      pp[1] = q.s;
    }
  }
}

// One wave per row: the S chunk pairs of row b, merged in chunk order.
template <typename Tin>
__global__ __launch_bounds__(64) void combine_kernel(LogprobArgs a) {
  const int b = blockIdx.x;
  if (b >= a.B) return;
  const int lane = lane_id();
  Pair p{-__builtin_inff(), 0.0f};
  for (int c = lane; c < a.S; c += 64) {
    const float* pp = a.part + 2 * ((long long)b * a.S + c);
    p = merge(p, Pair{pp[0], pp[1]});
  }
  p = wave_merge(p);
  if (lane == 0) {
    const float lse = row_lse(p);
    const int tok = a.tokens[b];
    const Tin* rowp = (const Tin*)a.logits + (long long)b * a.row_stride;
    const float x = (tok >= 0 && tok < a.V) ? Elem<Tin>::scalar(rowp, tok) : __builtin_nanf("");
    a.out_lp[b] = x - lse;
    if (a.out_lse) a.out_lse[b] = lse;
  }
}

template <typename Tin>
hipError_t launch_t(const LogprobArgs& a, hipStream_t st) {
  hipLaunchKernelGGL(chunk_kernel<Tin>, dim3(a.B * a.S), dim3(LT), 0, st, a);
  if (a.S > 1) hipLaunchKernelGGL(combine_kernel<Tin>, dim3(a.B), dim3(64), 0, st, a);
  return hipGetLastError();
}

}  // namespace lp

hipError_t launch_logprob(const LogprobArgs& a, int dtype, hipStream_t st) {
  return dtype == 1 ? lp::launch_t<uint16_t>(a, st) : lp::launch_t<float>(a, st);
}

}  // namespace tgs
