// tgs_mask.hip -- rows of the handle's mask table computed on the device
// from a byte-level DFA (a grammar compiled on the host): bit v of the row
// for DFA state s is set when token v is non-empty and each of its bytes has
// a transition walking from s.  This is the reference's per-token byte replay
// (ServeTokenMasker.mask(for:), native-mac/Sources/TinyGPTServe/
// Serve.swift:2005-2025; LogitsMasker.mask(forFSM:), ConstrainedGen.swift:
// 805-822) for every token of every requested state at once.  A state that
// is complete (accepting, no way on) allows only the EOS token given (none
// for -1).
//
// One lane per token per state (grid y = the requested states): the token's
// first 16 bytes are read up front, so only the transition lookups (an
// L2-resident table of 1 KiB per state) form a dependent chain; a ballot
// gives two mask words per wave, written straight into the table row.
// Malformed input cannot read out of bounds: a next state outside the
// table rejects, rows outside the table are skipped.
#include "tgs_device.h"
#include "tgs_kernels.h"

namespace tgs {
namespace maskb {

constexpr int MT = MASK_NT;
constexpr int PRE = 16;  // token bytes read before the walk

__global__ __launch_bounds__(MT) void build_kernel(MaskBuildArgs a) {
  const int i = blockIdx.y;
  const int row = a.rows[i];
  if (row < 0 || row >= a.n_rows) return;
  const int s = a.states[i];
  const int v = blockIdx.x * MT + (int)threadIdx.x;
  bool ok = false;
  if (s >= 0 && s < a.n_dfa && v < a.n_tokens) {
    if (a.complete[s]) {
      ok = v == a.eos;
    } else {
      const int p0 = a.tok_off[v], p1 = a.tok_off[v + 1];
      const int len = p1 - p0;
      uint32_t pre[PRE];
#pragma unroll
      for (int k = 0; k < PRE; k++) pre[k] = k < len ? a.tok_bytes[p0 + k] : 0u;
      int cur = s;
#pragma unroll
      for (int k = 0; k < PRE; k++) {
        if (k < len && cur >= 0) {
          cur = a.trans[(long long)cur * 256 + pre[k]];
          if (cur >= a.n_dfa) cur = -1;
        }
      }
      for (int p = p0 + PRE; p < p1 && cur >= 0; p++) {
        cur = a.trans[(long long)cur * 256 + a.tok_bytes[p]];
        if (cur >= a.n_dfa) cur = -1;
      }
      ok = len > 0 && cur >= 0;
    }
  }
  const u64 bal = __ballot(ok);
  const int lane = lane_id();
  const int w0 = (blockIdx.x * MT + ((int)threadIdx.x & ~63)) >> 5;  // this wave's first word
  uint32_t* dst = a.table + (long long)row * a.words;
  if (lane == 0 && w0 < a.words) dst[w0] = (uint32_t)bal;
  if (lane == 32 && w0 + 1 < a.words) dst[w0 + 1] = (uint32_t)(bal >> 32);
}

}  // namespace maskb

hipError_t launch_mask_build(const MaskBuildArgs& a, hipStream_t st) {
  const dim3 g((a.words * 32 + maskb::MT - 1) / maskb::MT, a.n);
  hipLaunchKernelGGL(maskb::build_kernel, g, dim3(maskb::MT), 0, st, a);
  return hipGetLastError();
}

}  // namespace tgs
