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
// The DFA comes as a byte-class map and a [n_dfa][n_cls] transition table
// (bytes of one class move every state alike).  One lane per token; a
// workgroup takes 256 tokens and up to MASK_SPW requested states, a group at
// a time: each lane reads its token's first 16 bytes once (as classes) and
// walks them from several states side by side (independent lookup chains).
// A ballot per state gives two mask words per wave; the LDS kernel stages
// the workgroup's words and stores each row's eight consecutive words from
// adjacent lanes, the global kernel stores them straight into the rows.
//
// When the table is small enough (16-bit entries, MASK_LDS_TABLE bytes) the
// workgroup first copies it into LDS with an extra dead state and extra
// reject and stay columns, so every invalid move lands in the dead state and
// a walk is a chain of branch-free LDS reads.  Otherwise the walk reads the
// table from global memory (L2).
// A class or next state outside the table rejects and rows outside the
// table are skipped.  A token whose offsets do not give a range inside the
// byte buffer (negative, decreasing, or past its length) is read as empty,
// so it is never allowed and no offset leads a read outside the buffer.
#include "tgs_device.h"
#include "tgs_kernels.h"

namespace tgs {
namespace maskb {

constexpr int MT = MASK_NT;
constexpr int PRE = 16;  // token bytes read before the walks
constexpr int SG = 8;    // states walked together per lane (independent lookup chains)
constexpr int SPW = MASK_SPW;
static_assert(SPW % SG == 0, "whole groups per workgroup");

// Writes the row bits of one group of G states (i0 .. i0 + G - 1); row(i)
// gives the table row of requested state i.
template <int G, class RowOf>
__device__ __forceinline__ void store_rows(const MaskBuildArgs& a, int i0, const bool (&ok)[G], RowOf row_of) {
  const int lane = lane_id();
  const int w0 = (blockIdx.x * MT + ((int)threadIdx.x & ~63)) >> 5;  // this wave's first word
#pragma unroll
  for (int g = 0; g < G; g++) {
    const int i = i0 + g;
    const u64 bal = __ballot(ok[g]);
    if (i >= a.n) continue;
    const int row = row_of(i);
    if (row < 0 || row >= a.n_rows) continue;
    uint32_t* dst = a.table + (long long)row * a.words;
    if (lane == 0 && w0 < a.words) dst[w0] = (uint32_t)bal;
    if (lane == 32 && w0 + 1 < a.words) dst[w0 + 1] = (uint32_t)(bal >> 32);
  }
}

// Start of each requested state of group i0 for this lane's token: eos_ok
// for a complete state's EOS token; live walks start at the state, others
// at `none`.  state_of(i) gives requested state i and complete_of(i, s)
// whether its DFA state s (in range) is complete.
template <int G, class StateOf, class CompleteOf>
__device__ __forceinline__ void group_start(const MaskBuildArgs& a, int i0, int v, int len, int none,
                                            int (&st)[G], bool (&eos_ok)[G], StateOf state_of,
                                            CompleteOf complete_of) {
#pragma unroll
  for (int g = 0; g < G; g++) {
    const int i = i0 + g;
    const int s = i < a.n ? state_of(i) : -1;
    const bool in = s >= 0 && s < a.n_dfa && v < a.n_tokens;
    const bool comp = in && complete_of(i, s);
    eos_ok[g] = comp && v == a.eos;
    st[g] = (in && !comp && len > 0) ? s : none;
  }
}

// LDS table.  Columns: the n_cls classes, then `reject` (every state to the
// dead state) and `stay` (every state to itself, for the steps past a
// token's end); rows: the n_dfa states, then the dead state (every column
// back to it).  Entries are byte offsets of the next state's row, so a step
// is one add and one 16-bit LDS read; the table is at most MASK_LDS_TABLE
// bytes, so offsets fit 16 bits.  The class map holds byte offsets of
// columns.  Workgroup (token chunk, SPW requested states).
constexpr int SGL = 16;         // states walked together in the LDS kernel
constexpr int NSUB = MASK_NSUB; // 256-token sub-chunks per LDS-kernel workgroup
constexpr int SPWL = MASK_SPW_LDS;
static_assert(SPWL % SGL == 0, "whole groups per workgroup");

// A token's byte range and its first PRE bytes (0 past the end).
struct Tok {
  int p0, len;
  uint32_t raw[PRE];
};
// Token v's byte range [p0, p0 + len): empty for ids past n_tokens and for
// offsets that do not lie in order inside the byte buffer.
__device__ __forceinline__ void tok_span(const MaskBuildArgs& a, int v, int& p0, int& len) {
  p0 = 0;
  len = 0;
  if (v < a.n_tokens) {
    const int s = a.tok_off[v], e = a.tok_off[v + 1];
    if (s >= 0 && e > s && e <= a.n_bytes) {
      p0 = s;
      len = e - s;
    }
  }
}
__device__ __forceinline__ void tok_range(const MaskBuildArgs& a, int v, Tok& k) { tok_span(a, v, k.p0, k.len); }
__device__ __forceinline__ void tok_bytes(const MaskBuildArgs& a, Tok& k) {
#pragma unroll
  for (int j = 0; j < PRE; j++) k.raw[j] = j < k.len ? a.tok_bytes[k.p0 + j] : 0u;
}

// The LDS image, once per call: entry i < 256 is the column offset of byte
// i's class (the reject column for a class outside the table), entry
// 256 + s W + c the byte offset of the row of state s's successor under
// column c (the dead row for a rejection; s itself for `stay`).
__global__ __launch_bounds__(MT) void prep_image(MaskBuildArgs a) {
  const int W = a.n_cls + 2, dead = a.n_dfa;
  const int i = blockIdx.x * MT + (int)threadIdx.x;
  const int n = 256 + (a.n_dfa + 1) * W;
  if (i >= n) return;
  if (i < 256) {
    const int c = a.byte_class[i];
    a.image[i] = (uint16_t)(2 * (c < a.n_cls ? c : a.n_cls));
    return;
  }
  const int j = i - 256, s = j / W, c = j - s * W;
  int nx = dead;
  if (s < a.n_dfa) {
    if (c < a.n_cls) {
      const int q = a.trans[(long long)s * a.n_cls + c];
      nx = (q >= 0 && q < a.n_dfa) ? q : dead;
    } else if (c == a.n_cls + 1) {
      nx = s;
    }
  }
  a.image[i] = (uint16_t)(nx * W * 2);
}

// Workgroup (NSUB * MT tokens, SPWL requested states): every row it writes
// gets NSUB * MT / 32 consecutive words (64-byte segments), staged in
// LDS and stored by adjacent lanes.
__global__ __launch_bounds__(MT) void build_lds(MaskBuildArgs a) {
  TGS_DYN_SMEM(smem);
  __shared__ uint32_t req_start2[SPWL];  // byte offset of the state's row; the dead row if it has no walk
  __shared__ int req_row[SPWL];
  __shared__ uint8_t req_complete[SPWL];
  __shared__ u64 words[SPWL][NSUB * MT / 64];  // [state][sub-chunk wave]
  uint16_t* cls2 = (uint16_t*)smem;             // [256] column byte offsets
  unsigned char* tab = smem + 512;              // [(n_dfa + 1)][W] uint16
  const int W = a.n_cls + 2, dead = a.n_dfa;
  const int t = threadIdx.x;
  const int vb = blockIdx.x * NSUB * MT + t;    // this lane's token in sub-chunk 0
  Tok cur_tok, next_tok;
  tok_range(a, vb, cur_tok);
  tok_bytes(a, cur_tok);
  const int ib = blockIdx.y * SPWL;
  if (t < SPWL) {  // this workgroup's requested states: walk start, row, completeness
    const int i = ib + t;
    const int s = i < a.n ? a.states[i] : -1;
    const bool in = s >= 0 && s < a.n_dfa;
    const bool comp = in && a.complete[s];
    req_start2[t] = (uint32_t)((in && !comp ? s : dead) * W * 2);
    req_row[t] = i < a.n ? a.rows[i] : -1;
    req_complete[t] = comp;
  }
  {  // the LDS image (class offsets, then the table), four 16-byte loads in flight per thread
    const int nvec = (int)(mask_image_bytes(a.n_dfa, a.n_cls) / 16);
    const uint4* src = (const uint4*)a.image;
    uint4* dst = (uint4*)smem;
    for (int i0 = t; i0 < nvec; i0 += 4 * MT) {
      uint4 x[4];
#pragma unroll
      for (int u = 0; u < 4; u++) x[u] = i0 + u * MT < nvec ? src[i0 + u * MT] : make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (i0 + u * MT < nvec) dst[i0 + u * MT] = x[u];
    }
  }
  __syncthreads();
  const uint32_t stay2 = 2u * (uint32_t)(a.n_cls + 1);
  const uint32_t dead2 = (uint32_t)(dead * W * 2);

#pragma unroll 1
  for (int sub = 0; sub < NSUB; sub++) {
    const int v = vb + sub * MT;
    if (sub + 1 < NSUB) {  // the next sub-chunk's bytes load under this one's walks
      tok_range(a, v + MT, next_tok);
      tok_bytes(a, next_tok);
    }
    const int p0 = cur_tok.p0, len = cur_tok.len;
    uint32_t pc[PRE];  // column offsets of the first PRE bytes; `stay` past the end
#pragma unroll
    for (int k = 0; k < PRE; k++) pc[k] = k < len ? (uint32_t)cls2[cur_tok.raw[k]] : stay2;
    const int lmax = __builtin_amdgcn_readfirstlane(wave_max(len < PRE ? len : PRE));  // steps this wave needs
    const bool walks = v < a.n_tokens && len > 0;
    const bool is_eos = v == a.eos;  // eos < n_tokens
#pragma unroll 1
    for (int i0 = ib; i0 < ib + SPWL && i0 < a.n; i0 += SGL) {
      uint32_t cur[SGL];
      bool eos_ok[SGL];
#pragma unroll
      for (int g = 0; g < SGL; g++) {  // slots past the request count start dead, not complete
        cur[g] = walks ? req_start2[i0 - ib + g] : dead2;
        eos_ok[g] = is_eos && req_complete[i0 - ib + g];
      }
#pragma unroll
      for (int k = 0; k < PRE; k++) {
        if (k < lmax) {
#pragma unroll
          for (int g = 0; g < SGL; g++) cur[g] = *(const uint16_t*)(tab + cur[g] + pc[k]);
        }
      }
      for (int p = p0 + PRE; p < p0 + len; p++) {  // tokens longer than PRE bytes
        const uint32_t c2 = cls2[a.tok_bytes[p]];
#pragma unroll
        for (int g = 0; g < SGL; g++) cur[g] = *(const uint16_t*)(tab + cur[g] + c2);
      }
#pragma unroll
      for (int g = 0; g < SGL; g++) {
        const u64 bal = __ballot(cur[g] != dead2 || eos_ok[g]);
        if (lane_id() == 0) words[i0 - ib + g][sub * (MT / 64) + (t >> 6)] = bal;
      }
    }
    if (sub + 1 < NSUB) cur_tok = next_tok;
  }
  // the rows' words of this token range, stored coalesced: each row gets
  // its NSUB * MT / 32 consecutive words from adjacent lanes
  __syncthreads();
  constexpr int WPB = NSUB * MT / 32;  // words per row per workgroup
  const int nst = (a.n - ib) < SPWL ? (a.n - ib) : SPWL;
  const uint32_t* wsrc = (const uint32_t*)&words[0][0];
  for (int j = t; j < nst * WPB; j += MT) {
    const int r = j / WPB, q = j - r * WPB;
    const int row = req_row[r];
    const int word = blockIdx.x * WPB + q;
    if (row >= 0 && row < a.n_rows && word < a.words) a.table[(long long)row * a.words + word] = wsrc[r * WPB + q];
  }
}

// Global table (too large for LDS): the class map in LDS, transitions read
// from memory with every index checked.
__global__ __launch_bounds__(MT) void build_global(MaskBuildArgs a) {
  __shared__ uint8_t cls[256];
  const int v = blockIdx.x * MT + (int)threadIdx.x;
  int p0, len;
  tok_span(a, v, p0, len);
  uint32_t raw[PRE];
#pragma unroll
  for (int k = 0; k < PRE; k++) raw[k] = k < len ? a.tok_bytes[p0 + k] : 0u;
  for (int i = threadIdx.x; i < 256; i += MT) {
    const int c = a.byte_class[i];
    cls[i] = (uint8_t)(c < a.n_cls ? c : 255);
  }
  __syncthreads();
  uint32_t pre[PRE];
#pragma unroll
  for (int k = 0; k < PRE; k++) pre[k] = cls[raw[k]];
  const int ib = blockIdx.y * SPW;
#pragma unroll 1
  for (int i0 = ib; i0 < ib + SPW && i0 < a.n; i0 += SG) {
    int cur[SG];
    bool eos_ok[SG];
    group_start<SG>(a, i0, v, len, -1, cur, eos_ok, [&](int i) { return a.states[i]; },
                    [&](int, int s) { return a.complete[s] != 0; });
    auto step = [&](int c) {
#pragma unroll
      for (int g = 0; g < SG; g++) {
        if (cur[g] >= 0) {
          const int nx = c < a.n_cls ? a.trans[(long long)cur[g] * a.n_cls + c] : -1;
          cur[g] = nx < a.n_dfa ? nx : -1;
        }
      }
    };
#pragma unroll
    for (int k = 0; k < PRE; k++)
      if (k < len) step((int)pre[k]);
    for (int p = p0 + PRE; p < p0 + len; p++) step((int)cls[a.tok_bytes[p]]);
    bool ok[SG];
#pragma unroll
    for (int g = 0; g < SG; g++) ok[g] = cur[g] >= 0 || eos_ok[g];
    store_rows<SG>(a, i0, ok, [&](int i) { return a.rows[i]; });
  }
}

// Mask-table rows from a staging upload: packed [n dst rows][n src rows]
// ints, then the source rows' words; workgroup (x, y) copies one stretch
// of MT words of rows y, y + gridDim.y, ...
__global__ __launch_bounds__(MT) void scatter_rows(const int* packed, const uint32_t* src, int n, int words,
                                                   uint32_t* table) {
  const int w = blockIdx.x * MT + (int)threadIdx.x;
  if (w >= words) return;
  for (int r = blockIdx.y; r < n; r += gridDim.y)
    table[(size_t)packed[r] * words + w] = src[(size_t)packed[n + r] * words + w];
}

}  // namespace maskb

hipError_t launch_mask_scatter(const int* packed, const uint32_t* src, int n, int words, uint32_t* table,
                               hipStream_t st) {
  if (n <= 0) return hipSuccess;
  const dim3 g((words + maskb::MT - 1) / maskb::MT, n < 65535 ? n : 65535);
  hipLaunchKernelGGL(maskb::scatter_rows, g, dim3(maskb::MT), 0, st, packed, src, n, words, table);
  return hipGetLastError();
}

hipError_t launch_mask_build(const MaskBuildArgs& a, hipStream_t st) {
  if (a.lds) {
    constexpr int TPW = maskb::NSUB * maskb::MT;  // tokens per workgroup
    const dim3 g((a.words * 32 + TPW - 1) / TPW, (a.n + maskb::SPWL - 1) / maskb::SPWL);
    const int n_img = 256 + (a.n_dfa + 1) * (a.n_cls + 2);
    hipLaunchKernelGGL(maskb::prep_image, dim3((n_img + maskb::MT - 1) / maskb::MT), dim3(maskb::MT), 0, st, a);
    hipLaunchKernelGGL(maskb::build_lds, g, dim3(maskb::MT), mask_image_bytes(a.n_dfa, a.n_cls), st, a);
  } else {
    const dim3 g((a.words * 32 + maskb::MT - 1) / maskb::MT, (a.n + maskb::SPW - 1) / maskb::SPW);
    hipLaunchKernelGGL(maskb::build_global, g, dim3(maskb::MT), 0, st, a);
  }
  return hipGetLastError();
}

}  // namespace tgs
