/*
 * tgs_oracle.h -- CPU restatement of TinyGPT's decode-time sampling path.
 *
 * TEST INFRASTRUCTURE ONLY.  This oracle is the checker for the HIP
 * sampler in tinygpt_amd/: only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it.  The product never links it.
 *
 * It restates, in plain C, the sampler the reference spreads over Swift,
 * C++ and JS (citations are to /root/reference):
 *   - repetition penalty (CTRL, set of history ids, divide positive /
 *     multiply non-positive):  native-mac/Sources/TinyGPTApp/ModelController.swift:262-283
 *   - temperature, greedy argmax (strict >, lowest id wins ties):
 *     native-mac/Sources/TinyGPTServe/Serve.swift:1496-1500, wasm/src/model.cpp:489-493
 *   - grammar mask (allowed <=> mask value 0; others -inf):
 *     native-mac/Sources/TinyGPTModel/ConstrainedGen.swift:805-822, Serve.swift:2005-2025
 *   - top-k by value threshold: ModelController.swift:292-302, python_ref/model.py:219-222,
 *     wasm/src/model.cpp:500-506
 *   - softmax + categorical draw: wasm/src/model.cpp:495-516, Serve.swift:1498-1500
 *   - stochastic speculative verify (Leviathan): native-mac/Sources/TinyGPT/SpeculativeDecode.swift:121-210
 *   - greedy speculative verify: SpeculativeDecode.swift:41-98
 * and fixes the points the reference leaves open the way the north-star
 * contract requires (exact top-k tie-break, host-supplied uniforms,
 * presence/frequency penalties, top-p).  The canonical rules, one per
 * function, are in the comments of tgs_oracle.c.
 */
#ifndef TGS_ORACLE_H
#define TGS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TGO_FLAG_GREEDY 1

/* Same layout as tgs_row_params in include/tgs_sampler.h (32 bytes). */
typedef struct {
  float temperature;  /* <= 0 (or TGO_FLAG_GREEDY): greedy argmax           */
  int32_t top_k;      /* <= 0 or >= V: disabled                               */
  float top_p;        /* >= 1: disabled; must be > 0                          */
  float repetition;   /* CTRL penalty; 1: off; must be > 0                    */
  float presence;     /* OpenAI presence penalty                              */
  float frequency;    /* OpenAI frequency penalty                             */
  int32_t mask_state; /* < 0: no grammar mask; else row of the bitmask table  */
  int32_t flags;      /* TGO_FLAG_GREEDY                                      */
} tgo_params;

typedef struct {
  int32_t token;         /* >= 0 token id; -1 no allowed token; -2 invalid row */
  int32_t n_topk;        /* size of the kept set after top-k                   */
  int32_t n_topp;        /* size of the kept set after top-p                   */
  int32_t cut_id;        /* id of the last (lowest-ranked) top-p survivor      */
  uint64_t mass_k;       /* S : sum of q over the top-k set (2^-40 units)      */
  uint64_t mass_p;       /* S': sum of q over the top-p set                    */
  int32_t draw_boundary; /* 1 if u*S' lies within 1e-6*S' of a CDF step        */
  int32_t topp_boundary; /* 1 if the top-p cut lies within 1e-6*S of p*S       */
  int32_t ref_tie_extra; /* ids the reference's keep-all-ties top-k would add  */
  int32_t greedy;        /* 1 if the row was decoded greedily                  */
} tgo_row_result;

/* ---- canonical numerics (exposed so tests can pin them) ---------------- */
float tgo_expf(float x);            /* e^x for x in [-32, 88]; 0 below -32   */
float tgo_weight(float y, float m); /* y == m ? 1 : tgo_expf(y - m)          */
float tgo_weight_wide(float y, float m);           /* as tgo_weight, down to y - m = -86 (reported probabilities) */
float tgo_kept_prob(float y, float m, float fs);   /* reported probability: wide weight 2^40 / fs */
uint64_t tgo_q40(float e);          /* floor(e * 2^40), e in [0, 1]          */
float tgo_u64_to_f32(uint64_t x);   /* round-to-nearest-even conversion      */
uint32_t tgo_key(float f);          /* order-preserving key, -0 -> +0        */
float tgo_unkey(uint32_t k);

/* One row of the sampler.  x: fp32 logits [V].  hist: H ids (ids outside
 * [0,V) ignored).  mask_row: V/32 words of the grammar table row, or NULL.
 * kept_ids / kept_probs (nullable, kept_cap entries): the top-k set in
 * (logit desc, id asc) order and q_i/S' for the top-p survivors.
 * post_logits (nullable, V): canonical post-penalty/mask/temperature logit,
 * -inf where not allowed. */
int tgo_sample_row(const float* x, int V, const int32_t* hist, int H, const tgo_params* p,
                   const uint32_t* mask_row, float u, tgo_row_result* r, int32_t* kept_ids,
                   float* kept_probs, int kept_cap, float* post_logits);

/* Batched wrapper over rows, nthreads POSIX threads (contiguous row ranges).
 * dtype 0: fp32 logits, 1: bf16 (upcast exactly).  hist is [B][hist_cap],
 * hist_len [B] (NULL: every row uses hist_cap).  mask_table is
 * [n_states][ceil(V/32)] (NULL if n_states == 0).  results / debug arrays
 * are nullable. */
int tgo_sample_batch(const void* logits, int dtype, int B, int V, int64_t row_stride,
                     const int32_t* hist, const int32_t* hist_len, int hist_cap,
                     const tgo_params* params, const uint32_t* mask_table, int n_states,
                     const float* u, int32_t* out_ids, tgo_row_result* results,
                     int32_t* kept_ids, float* kept_probs, int kept_cap, float* post_logits,
                     int nthreads);

/* ---- speculative verification ----------------------------------------- */
#define TGO_SPEC_BLOCK 1024

typedef struct {
  int32_t n_acc;          /* accepted draft tokens (0..k); -1 on error        */
  int32_t n_out;          /* tokens written to out (n_acc + 1)                */
  int32_t resampled;      /* 1 residual draw, 2 fallback-to-target, 3 bonus   */
  int32_t accept_boundary;/* 1 if some |u_acc - ratio| <= 1e-6                */
  int32_t draw_boundary;  /* 1 if the final draw lies within 1e-6 of a step   */
  float ratio_last;       /* ratio at the last examined position              */
  uint64_t resid_mass;    /* R (2^-40 units) when a residual was formed       */
  float s_target[16];     /* canonical softmax denominators of the first rows */
  float s_draft[16];
} tgo_spec_info;

/* target: k+1 rows, draft: k rows, each row_stride elements apart, fp32 (or
 * bf16 when dtype == 1).  dtok: k draft tokens.  T <= 0: greedy verify.
 * out: k+1 ids (-1 padded).  Returns 0, or -2 for invalid inputs (out[0]=-2). */
int tgo_spec_verify_row(const void* target, const void* draft, int dtype, int64_t row_stride,
                        const int32_t* dtok, int k, int V, float T, const float* u_acc,
                        float u_res, int32_t* out, tgo_spec_info* info);

int tgo_spec_verify_batch(const void* target, const void* draft, int dtype, const int32_t* dtok,
                          int B, int k, int V, const float* T, const float* u_acc,
                          const float* u_res, int32_t* n_acc, int32_t* out,
                          tgo_spec_info* infos, int nthreads);

/* Softmax helpers used by the speculative path, exposed for tests:
 * canonical row maximum and denominator (block sums in 2^-40 fixed point,
 * combined by a pairwise fp32 tree over 1024-id blocks). */
float tgo_spec_row_stats(const float* y, int V, float* m_out);

#ifdef __cplusplus
}
#endif
#endif /* TGS_ORACLE_H */
