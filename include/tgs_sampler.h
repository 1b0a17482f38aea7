/*
 * tgs_sampler.h -- C ABI of the MI355X (gfx950) decode-time sampler.
 *
 * One call samples a [B, V] batch of logits rows on the GPU: repetition /
 * presence / frequency penalties from a per-row token history, per-row
 * temperature, a grammar mask read from a per-state vocab bitmask table
 * resident in HBM, top-k, top-p, and a categorical draw from a
 * caller-supplied uniform.  A second entry point runs speculative-decoding
 * verification (accept/reject plus residual resample).
 *
 * Plain C: no HIP or torch types.  Streams are passed as `tgs_stream`,
 * which is HIP's hipStream_t (a pointer to struct ihipStream_t); NULL means
 * the default stream of the handle's device.
 *
 * Ownership: the caller owns every input and output buffer (device
 * pointers on the handle's device).  The handle owns its workspace and the
 * mask table.  Calls are asynchronous on `stream`; synchronise before
 * reading outputs.  One handle serves one host thread at a time, and calls
 * on one handle must be ordered on one stream (they share workspace).
 *
 * Errors are status codes (never exceptions).  Argument errors the host can
 * see are returned by the call; per-row conditions found on the device are
 * written into the row's output id:
 *     id >= 0   sampled token
 *     id == -1  no token is allowed (all masked / -inf / NaN)   [TGS_EALLMASKED]
 *               (NaN logits are expected quiet, as arithmetic makes them; a
 *               signaling-NaN logit may hide the other ids of its 16-byte
 *               vector, since the kernels' maxima follow fmaxf)
 *     id == -2  invalid row parameters (see tgs_row_params)
 *     id == -3  row outside the tgs_batch_hint given to the call
 *     id == -4  a device-side wait between the workgroups of a row ran out
 *               (cannot happen while the GPU runs every workgroup; the
 *               handle should then be destroyed)
 *
 * Reference interfaces replaced (paths under the reference repository):
 *   tgs_sample       <- Server.sampleToken(from:temperature:constraint:)
 *                       native-mac/Sources/TinyGPTServe/Serve.swift:1483-1506;
 *                       Sample.sampleWithSchema native-mac/Sources/TinyGPT/Sample.swift:812-836;
 *                       ModelController.runGenerate penalty + top-k
 *                       native-mac/Sources/TinyGPTApp/ModelController.swift:262-304;
 *                       the tg_generate sampler wasm/src/model.cpp:486-516 (C ABI precedent:
 *                       WASM_EXPORT extern "C" + opaque handle, wasm/src/model.h:17-56)
 *   tgs_mask_table_* <- LogitsMasker.mask(forFSM:) native-mac/Sources/TinyGPTModel/ConstrainedGen.swift:805-822
 *                       and ServeTokenMasker.mask(for:) Serve.swift:2005-2025 (the per-step
 *                       host-built float mask becomes a per-state bit row kept in HBM)
 *   tgs_spec_verify  <- SpeculativeDecode.stepStochastic native-mac/Sources/TinyGPT/SpeculativeDecode.swift:121-210
 *                       and the greedy SpeculativeDecode.step :41-98
 */
#ifndef TGS_SAMPLER_H
#define TGS_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TGS_ABI_VERSION 4

struct ihipStream_t;
typedef struct ihipStream_t* tgs_stream;

typedef struct tgs_ctx* tgs_handle; /* opaque, cf. TgModel in wasm/src/model.h:17-18 */

typedef enum {
  TGS_OK = 0,
  TGS_EINVAL = -1,     /* bad argument                                    */
  TGS_ENOMEM = -2,     /* device allocation failed                        */
  TGS_EHIP = -3,       /* HIP runtime error (no device, launch failure)   */
  TGS_EALLMASKED = -4, /* used by host wrappers for rows whose id is -1   */
  TGS_ETOOBIG = -5     /* size beyond what the handle was created for     */
} tgs_status;

typedef enum { TGS_F32 = 0, TGS_BF16 = 1 } tgs_dtype;

#define TGS_FLAG_GREEDY 1 /* decode this row by argmax regardless of T */

/* Per-row parameters (32 bytes, device memory, one per row). */
typedef struct {
  float temperature;  /* <= 0 (or TGS_FLAG_GREEDY): greedy argmax; else finite > 0     */
  int32_t top_k;      /* <= 0 or >= V: disabled                                         */
  float top_p;        /* >= 1: disabled; must be > 0                                    */
  float repetition;   /* CTRL penalty over distinct history ids; 1 = off; must be > 0   */
  float presence;     /* subtracted once from every id present in the history           */
  float frequency;    /* subtracted per occurrence of the id in the history             */
  int32_t mask_state; /* < 0: no grammar mask; else row of the mask table               */
  int32_t flags;      /* TGS_FLAG_GREEDY                                                */
} tgs_row_params;

/* Optional per-row diagnostics (host struct of nullable device pointers). */
typedef struct {
  int32_t* kept_ids;   /* [B][kept_cap] top-k set, (logit desc, id asc) order, -1 padded.
                          Written for rows with 1 <= top_k <= 1024; other rows: -1.      */
  float* kept_probs;   /* [B][kept_cap] normalised probability of each top-p survivor    */
  int32_t kept_cap;
  int32_t* counts;     /* [B][2] size of the top-k set, size of the top-p set            */
  uint64_t* mass;      /* [B][2] S and S' in 2^-40 units (exact integer masses)           */
  int32_t* cut_ids;    /* [B] id of the last top-p survivor                               */
  float* post_logits;  /* [B][V] logit after penalties, mask (-inf) and temperature       */
} tgs_debug;

/* Host-side summary of a batch's row parameters.  It selects kernels
 * specialised for the batch: max_top_k <= 64 -> one-tile chunks merged in
 * wave registers (one launch); <= 1024 -> one workgroup per row holding the
 * row in registers (16-byte aligned rows of whole vectors: bf16 V <= 163840,
 * fp32 V <= 81920, history <= 1024 ids), else the candidate path; otherwise
 * (or no hint) the candidate path, the full-path kernel for rows with
 * 1024 < top_k < V and the top-p kernel for rows without a top-k.  The hint
 * is a promise: a sampling row whose top_k exceeds max_top_k (a row without
 * a usable top-k counts as V) gets id -3.  Greedy rows are served under any
 * hint.  min_top_k == V (every sampling row without a usable top-k, as in
 * grammar-constrained top-p decoding) lets the top-p kernel serve the whole
 * batch, its greedy rows included, in one launch. */
typedef struct {
  int32_t max_top_k; /* max over sampling rows of top_k when 1 <= top_k < V, else V;
                        0 when every row is greedy */
  int32_t min_top_k; /* min over sampling rows of the same; V when every row is greedy.
                        0 (unknown) is always safe */
} tgs_batch_hint;

/* Library / status helpers (no device work). */
int tgs_abi_version(void);
const char* tgs_status_string(int status);

/* Fill *out from host copies of the row parameters (greedy rows: flag set or
 * temperature <= 0 or NaN). */
int tgs_hint_from_params(const tgs_row_params* host_params, int B, int V, tgs_batch_hint* out);

/* Create a sampler on `device`.  max_batch, max_vocab and max_hist bound
 * every later call (workspace is sized once here; calls never allocate). */
int tgs_create(tgs_handle* out, int device, int max_batch, int max_vocab, int max_hist);
void tgs_destroy(tgs_handle h);
/* Message of the handle's last error; NULL: the calling thread's last
 * tgs_sample_noalloc error ("null handle" when there is none). */
const char* tgs_last_error(tgs_handle h);

/* Grammar mask table: n_states rows of ceil(vocab/32) uint32 words; bit v
 * of row s (word v>>5, bit v&31) is 1 <=> token v is allowed in state s.
 * _set replaces the table (synchronous upload); _update overwrites n rows
 * (states[i] < current n_states, all checked before anything is written;
 * the last of repeated states wins): one upload of every row, then (states
 * not consecutive) one scatter launch; synchronous. */
int tgs_mask_table_set(tgs_handle h, const uint32_t* host_words, int n_states, int vocab);
int tgs_mask_table_update(tgs_handle h, const int32_t* host_states, const uint32_t* host_words,
                          int n);
/* Rows [first, first + n) of the table copied to host_words (n rows of
 * ceil(vocab/32) words), after all work queued on the handle's device has
 * finished: the rows as tgs_mask_table_set / _update and
 * tgs_mask_rows_from_dfa left them.  A readback for checks and
 * diagnostics, not for the decode loop (it synchronises the device).  No
 * reference counterpart: the reference's mask rows live in host arrays. */
int tgs_mask_table_get(tgs_handle h, int first, int n, uint32_t* host_words);

/* Sample one token per row.
 *   d_logits    [B] rows of V logits, row_stride elements apart (fp32 or bf16)
 *   d_hist      [B][hist_cap] token history (ids outside [0,V) ignored), nullable if hist_cap == 0
 *   d_hist_len  [B] valid history entries per row (nullable: hist_cap for every row)
 *   d_params    [B] tgs_row_params
 *   d_u         [B] uniforms in [0,1) (ignored by greedy rows)
 *   d_out_ids   [B] output ids (see the id codes above)
 *   hint        nullable host struct (see tgs_batch_hint)
 *   dbg         nullable diagnostics */
int tgs_sample(tgs_handle h, const void* d_logits, tgs_dtype dt, int B, int V, int64_t row_stride,
               const int32_t* d_hist, const int32_t* d_hist_len, int hist_cap,
               const tgs_row_params* d_params, const float* d_u, int32_t* d_out_ids,
               const tgs_batch_hint* hint, const tgs_debug* dbg, tgs_stream stream);

/* tgs_sample without a handle, for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  It has no counterpart in the reference: the reference
 * samples inline in Swift/MLX.  Same arguments, kernels and results as
 * tgs_sample; the mask table is passed in (d_mask_table: n_states rows of
 * ceil(mask_vocab / 32) words, mask_vocab >= V; NULL / 0 for none).  Its
 * workspace is a static device array of about 6 MiB that every GPU the
 * library runs on holds until the process ends; the first call on a device
 * also prepares that array (and synchronises the device once), so it must
 * not be made under graph capture (it then returns TGS_EINVAL): make it
 * before capturing, with B = 0 if there is nothing to sample yet; every
 * later call can be captured.  Limits:
 * B <= 256, V <= 262144, hist_cap <= 1024; beyond them it returns
 * TGS_ETOOBIG.  It calls no hipMalloc or hipFree.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (several streams,
 * several threads) race and must be ordered by the caller.  Errors:
 * tgs_last_error(NULL) gives the calling thread's last message. */
int tgs_sample_noalloc(int device, const void* d_logits, tgs_dtype dt, int B, int V, int64_t row_stride,
                       const int32_t* d_hist, const int32_t* d_hist_len, int hist_cap,
                       const tgs_row_params* d_params, const float* d_u, int32_t* d_out_ids,
                       const uint32_t* d_mask_table, int n_states, int mask_vocab, const tgs_batch_hint* hint,
                       const tgs_debug* dbg, tgs_stream stream);

/* Size the speculative-verification workspace for up to max_batch sequences
 * of up to max_k draft tokens (allocates; call once before capturing
 * tgs_spec_verify in a graph).  tgs_spec_verify grows the workspace itself
 * (allocating, hence synchronising) when a call exceeds the reservation. */
int tgs_reserve_spec(tgs_handle h, int max_batch, int max_k);

/* Speculative verification for B sequences with k draft tokens each.
 *   d_target [B][k+1][V], d_draft [B][k][V] contiguous logits (fp32 or bf16)
 *   d_draft_tok [B][k]; d_T [B] temperature (<= 0: greedy verify, else max(T,1e-5));
 *   d_u_acc [B][k] accept uniforms; d_u_res [B] resample / bonus uniform.
 * Outputs: d_n_acc [B] accepted draft count (-1 error), d_out [B][k+1]
 * accepted drafts followed by the resampled or bonus token, -1 padded. */
int tgs_spec_verify(tgs_handle h, const void* d_target, const void* d_draft, tgs_dtype dt,
                    const int32_t* d_draft_tok, int B, int k, int V, const float* d_T,
                    const float* d_u_acc, const float* d_u_res, int32_t* d_n_acc, int32_t* d_out,
                    tgs_stream stream);

/* Rows of the handle's mask table computed on the device from a byte-level
 * DFA (a grammar compiled on the host, e.g. tinygpt_amd/grammar.py): row
 * rows[i] gets bit v set when token v is non-empty and each of its bytes has
 * a transition walking from DFA state states[i]; a complete state allows
 * only eos_id (-1: no token).  Replaces the per-token byte replay of
 * ServeTokenMasker.mask(for:), native-mac/Sources/TinyGPTServe/
 * Serve.swift:2005-2025 (and LogitsMasker.mask(forFSM:),
 * ConstrainedGen.swift:805-822), one row per FSM state, and the upload of
 * that row: the table is written in place on the stream.
 *   d_byte_class [256] class of each byte (a class >= n_cls rejects)
 *   d_trans      [n_dfa][n_cls] next state per class (-1 rejects)
 *   d_complete   [n_dfa] 1 for accepting states with no transition
 *   d_tok_off    [n_tokens + 1] offsets of each token's bytes in d_tok_bytes
 *   d_tok_bytes  [n_bytes] the tokens' bytes (nullable when n_bytes = 0)
 *   d_states, d_rows [n] DFA states and the table rows to fill
 * Token v's bytes are d_tok_bytes[off[v] .. off[v+1]); offsets are checked
 * against the buffer on the device: a token whose range starts below 0,
 * ends before it starts or ends past n_bytes is read as empty (never
 * allowed), so no offset can make the kernels read outside d_tok_bytes.
 * d_tok_off itself must hold n_tokens + 1 entries.
 * (the identity class map with n_cls = 256 passes a plain [n_dfa][256]
 * table).  The table (tgs_mask_table_set) must hold at least n_tokens ids;
 * bits of ids at or past n_tokens are cleared.  Rows outside the table are
 * skipped; a next state outside [0, n_dfa) rejects.  At most 1,048,560 pairs
 * per call; the inputs must stay alive until the stream reaches the call.
 * Uses the handle's workspace (like every call on the handle: order calls on
 * one stream); allocates nothing. */
int tgs_mask_rows_from_dfa(tgs_handle h, const uint8_t* d_byte_class, const int32_t* d_trans, int n_cls,
                           const uint8_t* d_complete, int n_dfa, const int32_t* d_tok_off,
                           const uint8_t* d_tok_bytes, int64_t n_bytes, int n_tokens, int eos_id,
                           const int32_t* d_states, const int32_t* d_rows, int n, tgs_stream stream);

/* Log-probability of one given token per row under the softmax of the raw
 * logits: out_logprob[b] = x[b][tok[b]] - logsumexp(x[b]) (teacher-forced
 * scoring; replaces `MLX.log(MLX.softmax(logits))[0, i, next]` in
 * scoreLogprobs, native-mac/Sources/TinyGPTServe/Serve.swift:983-993, computed
 * here in fp32 from fp32 or bf16 logits).  No penalty, temperature or mask
 * applies.
 *   d_logits      [B] rows of V logits, row_stride elements apart
 *   d_tokens      [B] token ids (outside [0,V): NaN)
 *   d_out_logprob [B] log-probabilities
 *   d_out_lse     [B] logsumexp of each row (nullable)
 * A row holding NaN or +inf, or only -inf, gives NaN.  B and V are not
 * bounded by the handle's limits (no per-row workspace beyond a few bytes). */
int tgs_token_logprobs(tgs_handle h, const void* d_logits, tgs_dtype dt, int B, int V, int64_t row_stride,
                       const int32_t* d_tokens, float* d_out_logprob, float* d_out_lse, tgs_stream stream);

#ifdef __cplusplus
}
#endif
#endif /* TGS_SAMPLER_H */
