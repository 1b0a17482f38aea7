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
// One lane per token; each workgroup walks its tokens from eight requested
// states side by side (eight independent lookup chains per lane), reading
// each token's first 16 bytes once, so the token table is read once per
// eight rows and only the transition lookups (an L2-resident table of 1 KiB
// per state) form dependent chains; a ballot per state gives two mask words
// per wave, written straight into the table row.
// Malformed input cannot read out of bounds: a next state outside the
// table rejects, rows outside the table are skipped.
#include "tgs_device.h"
#include "tgs_kernels.h"

namespace tgs {
namespace maskb {

constexpr int MT = MASK_NT;
constexpr int PRE = 16;  // token bytes read before the walks
constexpr int SG = 8;    // states walked together per lane (independent lookup chains)

// Workgroup (token chunk, group of SG requested states): each lane reads its
// token's first PRE bytes once and walks them from the SG states side by
// side, then one ballot per state gives the lane's wave two mask words.
__global__ __launch_bounds__(MT) void build_kernel(MaskBuildArgs a) {
  const int v = blockIdx.x * MT + (int)threadIdx.x;
  const int i0 = blockIdx.y * SG;
  int p0 = 0, len = 0;
  if (v < a.n_tokens) {
    p0 = a.tok_off[v];
    len = a.tok_off[v + 1] - p0;
  }
  uint32_t pre[PRE];
#pragma unroll
  for (int k = 0; k < PRE; k++) pre[k] = k < len ? a.tok_bytes[p0 + k] : 0u;
  int cur[SG];
  bool eos_ok[SG];
#pragma unroll
  for (int g = 0; g < SG; g++) {
    const int i = i0 + g;
    const int s = i < a.n ? a.states[i] : -1;
    const bool in = s >= 0 && s < a.n_dfa && v < a.n_tokens;
    const bool comp = in && a.complete[s];
    eos_ok[g] = comp && v == a.eos;
    cur[g] = (in && !comp && len > 0) ? s : -1;
  }
#pragma unroll
  for (int k = 0; k < PRE; k++) {
    if (k < len) {
#pragma unroll
      for (int g = 0; g < SG; g++) {
        if (cur[g] >= 0) {
          const int nx = a.trans[(long long)cur[g] * 256 + pre[k]];
          cur[g] = nx < a.n_dfa ? nx : -1;
        }
      }
    }
  }
  for (int p = p0 + PRE; p < p0 + len; p++) {  // tokens longer than PRE bytes
    const uint32_t byte = a.tok_bytes[p];
#pragma unroll
    for (int g = 0; g < SG; g++) {
      if (cur[g] >= 0) {
        const int nx = a.trans[(long long)cur[g] * 256 + byte];
        cur[g] = nx < a.n_dfa ? nx : -1;
      }
    }
  }
  const int lane = lane_id();
  const int w0 = (blockIdx.x * MT + ((int)threadIdx.x & ~63)) >> 5;  // this wave's first word
#pragma unroll
  for (int g = 0; g < SG; g++) {
    const int i = i0 + g;
    const u64 bal = __ballot(cur[g] >= 0 || eos_ok[g]);
    if (i >= a.n) continue;
    const int row = a.rows[i];
    if (row < 0 || row >= a.n_rows) continue;
    uint32_t* dst = a.table + (long long)row * a.words;
    if (lane == 0 && w0 < a.words) dst[w0] = (uint32_t)bal;
    if (lane == 32 && w0 + 1 < a.words) dst[w0 + 1] = (uint32_t)(bal >> 32);
  }
}

}  // namespace maskb

hipError_t launch_mask_build(const MaskBuildArgs& a, hipStream_t st) {
  const dim3 g((a.words * 32 + maskb::MT - 1) / maskb::MT, (a.n + maskb::SG - 1) / maskb::SG);
  hipLaunchKernelGGL(maskb::build_kernel, g, dim3(maskb::MT), 0, st, a);
  return hipGetLastError();
}

}  // namespace tgs
