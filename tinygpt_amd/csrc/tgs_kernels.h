// tgs_kernels.h -- argument blocks shared by the host C ABI and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/tgs_sampler.h"

namespace tgs {

// Fused top_k <= 64 kernel: threads per workgroup, 16-byte vectors per
// thread (a chunk is at most K64_NT x K64_NVT vectors), longest history it
// takes, candidate buffer entries (u64; 16 more are reserved for ranking
// pads), chunks per row at most, the stride (in unsigned words) between the
// per-row exchange lines (word 0 the arrival counter, word 1 the epoch word,
// from word K64_CNT_WORDS on one 64-bit count word per chunk), and the
// bound-exchange keys per row.
constexpr int K64_NT = 512;
constexpr int K64_NVT = 16;
constexpr int K64_MASK_PRE = 2;  // with a mask table: chunk vectors requested before the mask words
constexpr int K64_MAX_HIST = 1024;
constexpr int K64_SMALL_NT = 64;        // one-wave variant for rows of one small chunk
constexpr int K64_SMALL_MAX_HIST = 256;  // its longest history
constexpr int K64_CAP = 2048;
constexpr int K64_MAX_SPLIT = 16;
constexpr int K64_CNT_STRIDE = 64;
constexpr int K64_CNT_WORDS = 32;
constexpr int K64_KEYS = 256;

// Top-p kernel (rows without a top-k): threads per workgroup and the most
// ids of one histogram bucket ranked in LDS.
constexpr int TOPP_NT = 1024;
constexpr int TOPP_CAP = 1024;
constexpr int TOPP_MASK_PRE = 2;  // register-resident row vectors requested before the mask words

// Top-k kernel (1 <= top_k <= KMAX, the row held in registers): threads per
// workgroup and candidate capacity.
constexpr int TOPK_NT = 1024;
constexpr int TOPK_CAP = 4096;

struct SampleArgs {
  const void* logits;
  long long row_stride;  // elements
  int B, V;
  int aligned;           // rows start 16-byte aligned: vector loads
  int whole_vec;         // aligned and V a multiple of the 16-byte vector: a vector lies wholly inside or outside a row
  const int* hist;
  const int* hist_len;
  int hist_cap;
  const tgs_row_params* params;
  const float* u;
  int* out;
  const uint32_t* mask_table;
  int n_states, mask_words;
  int S, L;              // chunks per row, chunk length in ids
  int TS, ts_shift;      // history hash slots (power of two), 32 - log2(TS)
  int BW;                // history bitmap words per chunk
  int capt;              // candidate buffer entries
  int off_hash, off_bitmap, off_cand;  // dynamic LDS byte offsets
  unsigned long long* ws;  // [B*S][ws_stride] chunk candidate lists
  int ws_stride;         // entries per chunk list (64 fast variant, KMAX otherwise)
  int* ws_cnt;           // [B*S]
  unsigned* cnt;         // fused kernel: [B * K64_CNT_STRIDE] exchange lines (counter zero between calls)
  unsigned long long* lists;  // fused kernel: [B][K64_MAX_SPLIT][64] chunk lists (entries 0 between calls)
  unsigned long long* keys;   // fused kernel: [B][K64_KEYS] bound-exchange keys
  int xchg;              // fused kernel: split rows share a row-wide bound (the grid is resident at once)
  int kq;                // fused kernel: keys each wave publishes (S * waves * kq <= K64_KEYS, >= 64)
  int xmap;              // fused kernel: a row's chunks are workgroups congruent mod 8 (B a multiple of 8)
  int key_spins;         // fused kernel: polls of the row's keys before a wave keeps its chunk's bound
  int merge_spins;       // fused kernel: polls of the row's lists before the merge gives up (id -4)
  int full_rows;         // 1: full_kernel runs after the chunk kernels
  int hint_k;            // the launch hint's max_top_k (INT_MAX without a hint)
  int topp_all;          // 1: the top-p kernel alone serves the batch (its greedy rows too)
  int topp_cap;          // top-p kernel: allowed ids packed into LDS (beyond topp_lds_bytes)
  tgs_debug dbg;
};

// Mask-table rows from a byte-level DFA (tgs_mask.hip).
constexpr int MASK_NT = 256;
constexpr int MASK_SPW = 64;             // requested states per workgroup (global-table kernel)
constexpr int MASK_SPW_LDS = 16;         // requested states per workgroup (LDS-table kernel)
constexpr int MASK_NSUB = 2;             // 256-token sub-chunks per LDS-table workgroup (64-byte row segments)
constexpr int MASK_LDS_TABLE = 60 * 1024;  // largest transition table held in LDS (16-bit row offsets)
struct MaskBuildArgs {
  const uint8_t* byte_class;  // [256] class of each byte (>= n_cls rejects)
  const int* trans;           // [n_dfa][n_cls] next state, -1 rejects
  int n_cls;
  const uint8_t* complete;    // [n_dfa] accepting with no way on
  int n_dfa;
  int lds;                    // 1: the table fits LDS (16-bit row offsets, dead state, reject and stay columns)
  uint16_t* image;            // with lds: the LDS image (class offsets, then the table), written per call
  const int* tok_off;        // [n_tokens + 1]
  const uint8_t* tok_bytes;  // [n_bytes]
  int n_bytes;               // a token's range outside [0, n_bytes) reads as empty
  int n_tokens;
  int eos;                   // token allowed in a complete state (-1: none)
  const int* states;         // [n]
  const int* rows;           // [n]
  int n;
  uint32_t* table;           // the handle's mask table
  int n_rows, words;         // its rows and words per row
};
hipError_t launch_mask_build(const MaskBuildArgs& a, hipStream_t st);
// Rows packed[i] of table (rows of `words` words) from rows packed[n + i] of
// src, i < n (distinct destinations).
hipError_t launch_mask_scatter(const int* packed, const uint32_t* src, int n, int words, uint32_t* table,
                               hipStream_t st);
// The 16-bit table with the dead state, reject and stay columns, and the LDS
// image (512 bytes of class offsets, then the table, in whole 16 bytes).
__host__ __device__ inline size_t mask_lds_table_bytes(int n_dfa, int n_cls) {
  return (size_t)(n_dfa + 1) * (size_t)(n_cls + 2) * 2;
}
__host__ __device__ inline size_t mask_image_bytes(int n_dfa, int n_cls) {
  return (512 + mask_lds_table_bytes(n_dfa, n_cls) + 15) / 16 * 16;
}

// Token log-probabilities (tgs_logprob.hip).
constexpr int LP_NT = 256;
struct LogprobArgs {
  const void* logits;
  long long row_stride;  // elements
  int B, V;
  int aligned;           // rows start 16-byte aligned: vector loads
  const int* tokens;     // [B]
  float* out_lp;         // [B]
  float* out_lse;        // [B] or nullptr
  float* part;           // [B * S][2] chunk (max, sum of exp) pairs when S > 1
  int S, L;              // chunks per row, chunk length in ids (whole vectors)
};
hipError_t launch_logprob(const LogprobArgs& a, int dtype, hipStream_t st);

struct SpecArgs {
  const void* target;
  const void* draft;
  int B, k, V;
  int aligned;
  const int* dtok;
  const float* T;
  const float* u_acc;
  const float* u_res;
  int* n_acc;
  int* out;
  int nb;                      // blocks of SPEC_BLOCK ids per row
  int nbs;                     // block stride of the per-row workspace arrays (>= nb)
  float* blk_m;                // [B][2k+1][nbs] block maxima
  unsigned long long* blk_q;   // [B][2k+1][nbs] exact block masses (greedy: block argmax composite)
  unsigned long long* blk_w;   // [B][nbs][SPEC_GROUPS] draw mass per vector group of each block of the row drawn from
  void* seq_state;             // [B] 32-byte per-sequence decision
  int ncu;                     // compute units of the device (grid sizing)
};

constexpr int SPEC_MAX_K = 64;  // most draft tokens per sequence
constexpr int SPEC_GROUPS = 4;  // 16-byte vector groups per block of 1024 ids (fp32: 4, bf16: 2)

// Launches the chunk kernel, the merge kernel when rows are split (a.S > 1)
// and, when a.full_rows is set, the full-path kernel (rows with
// KMAX < top_k < V) and the top-p kernel (rows without a top-k), in that
// order on st.
hipError_t launch_sample(const SampleArgs& a, int dtype, size_t lds, hipStream_t st);
hipError_t set_sample_lds_limit(size_t bytes);
// The fused kernel for batches of greedy rows and rows with top_k <= 64:
// K64_NT threads per workgroup, chunks of at most k64_chunk_ids(dtype) ids.
int k64_chunk_ids(int dtype);
// small: the one-wave variant (K64_SMALL_NT threads, one chunk per row of at
// most k64_small_ids(dtype) ids, history <= K64_SMALL_MAX_HIST).
int k64_small_ids(int dtype);
hipError_t launch_k64(const SampleArgs& a, int dtype, size_t lds, hipStream_t st, bool small = false);
// Workgroups of the K64_NT instantiation that one CU holds at once with lds
// bytes of dynamic LDS (0 when the runtime cannot tell).
int k64_resident_per_cu(int dtype, bool whole_vec, bool mask, size_t lds);
// Static LDS of the K64_NT instantiation.
size_t k64_static_lds();
hipError_t set_k64_lds_limit(size_t bytes);
hipError_t launch_spec(const SpecArgs& a, int dtype, hipStream_t st);
// Rows sampling top-p over the whole vocabulary (top_k disabled).
size_t topp_lds_bytes(int V, int TS);
// Packed-id capacity of the top-p kernel given lds_avail bytes of dynamic LDS.
int topp_pack_cap(int V, int TS, size_t lds_avail);
// Dynamic LDS: topp_lds_bytes + a.topp_cap packed ids.
hipError_t launch_topp(const SampleArgs& a, int dtype, hipStream_t st);
hipError_t set_topp_lds_limit(size_t bytes);
// Batches of greedy rows and rows with 1 <= top_k <= KMAX whose rows fit the
// top-k kernel's registers (V <= topk_max_vocab(dtype)).
int topk_max_vocab(int dtype);
size_t topk_lds_bytes(int V, int TS);
hipError_t launch_topk(const SampleArgs& a, int dtype, size_t lds, hipStream_t st);
hipError_t set_topk_lds_limit(size_t bytes);

}  // namespace tgs
