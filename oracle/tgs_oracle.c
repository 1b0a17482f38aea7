/*
 * tgs_oracle.c -- CPU restatement of TinyGPT's decode-time sampler.
 *
 * TEST INFRASTRUCTURE ONLY (see tgs_oracle.h).  Built with
 * -ffp-contract=off so every float operation is the single IEEE operation
 * written here; the HIP kernels follow the same canonical rules.
 *
 * Canonical row semantics (one sampling row, logits x[0..V)):
 *  1. z = x.  Penalties apply when the row has history and is not neutral
 *     (repetition != 1 or presence != 0 or frequency != 0).  For every id v
 *     with count c > 0 in the history:
 *        z = z > 0 ? z / r : z * r          (ModelController.swift:276-279)
 *        z = z - frequency * c              (OpenAI definition; the reference
 *        z = z - presence                    has no presence/frequency term)
 *  2. Grammar mask: bit v of the state's table row == 0  ->  not allowed
 *     (ConstrainedGen.swift:816-819 sets 0 for accepted ids, -inf otherwise).
 *  3. Greedy (T <= 0 or flag): argmax z, ties -> lowest id
 *     (model.cpp:491-493 strict '>').
 *  4. y = z / T, the IEEE (correctly rounded) division, as the reference
 *     divides (Serve.swift:1499, wasm/src/model.cpp:499).  A row whose 1/T
 *     is not finite is invalid.  Allowed <=> y > -inf.
 *  5. Order allowed ids by (y desc, id asc).  Top-k keeps the first
 *     min(k, n_allowed) (the reference keeps all ties at the k-th value,
 *     model.py:222; ref_tie_extra counts the difference).
 *  6. m = y of the first kept id.  e_i = tgo_weight(y_i, m),
 *     q_i = floor(e_i * 2^40)  (exact integer masses).
 *     C_i = q_0 + ... + q_i (exact), S = C_last.
 *  7. Top-p (p < 1): P = floor(S * floor(p * 2^24) / 2^24); keep 0..i* with
 *     i* = first i such that C_i >= P.  S' = C_i*.
 *  8. Draw: t = floor(S' * floor(u * 2^24) / 2^24); token = first i with
 *     C_i > t.  (model.cpp:507-516 walks a CDF the same way, in id order and
 *     with its own RNG; here the walk is in sorted order with host u.)
 */
#define _GNU_SOURCE
#include "tgs_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

/* ---------------------------------------------------------------- numerics */

static inline uint32_t f2u(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  return u;
}
static inline float u2f(uint32_t u) {
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* e^x by Cody-Waite reduction x = n*ln2 + r, |r| <= ln2/2, and the degree-7
 * Taylor polynomial of e^r (coefficients 1/j!, truncation error < 1e-8
 * relative), evaluated by Horner with fused multiply-adds, then scaled by
 * 2^n through the exponent field.  Results below e^-32 are returned as 0
 * (they are below the 2^-40 mass resolution). */
float tgo_expf(float x) {
  if (!(x >= -32.0f)) return 0.0f; /* also NaN and -inf */
  if (x > 88.0f) return INFINITY;
  const float log2e = 0x1.715476p+0f;
  const float ln2_hi = 0x1.62ep-1f;
  const float ln2_lo = 0x1.0bfbe8p-15f;
  const float shifter = 12582912.0f; /* 1.5 * 2^23: adds round to integer */
  float t = x * log2e;
  float n = (t + shifter) - shifter;
  float r = fmaf(n, -ln2_hi, x);
  r = fmaf(n, -ln2_lo, r);
  float p = 0x1.a01a02p-13f;       /* 1/5040 */
  p = fmaf(p, r, 0x1.6c16c2p-10f); /* 1/720  */
  p = fmaf(p, r, 0x1.111112p-7f);  /* 1/120  */
  p = fmaf(p, r, 0x1.555556p-5f);  /* 1/24   */
  p = fmaf(p, r, 0x1.555556p-3f);  /* 1/6    */
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  int ni = (int)n;
  float scale = u2f((uint32_t)(ni + 127) << 23);
  return p * scale;
}

float tgo_weight(float y, float m) { return (y == m) ? 1.0f : tgo_expf(y - m); }

uint64_t tgo_q40(float e) { return (uint64_t)(e * 0x1p40f); }

/* Weight for reported probabilities only: tgo_weight's formula continued
 * below -32 down to y - m = -86 (2^n, n >= -124, a normal scale) instead of
 * 0; equal to tgo_weight wherever y - m >= -32. */
float tgo_weight_wide(float y, float m) {
  if (y == m) return 1.0f;
  const float x = y - m;
  if (!(x >= -86.0f)) return 0.0f;
  const float log2e = 0x1.715476p+0f;
  const float ln2_hi = 0x1.62ep-1f;
  const float ln2_lo = 0x1.0bfbe8p-15f;
  const float shifter = 12582912.0f;
  float t = x * log2e;
  float n = (t + shifter) - shifter;
  float r = fmaf(n, -ln2_hi, x);
  r = fmaf(n, -ln2_lo, r);
  float p = 0x1.a01a02p-13f;
  p = fmaf(p, r, 0x1.6c16c2p-10f);
  p = fmaf(p, r, 0x1.111112p-7f);
  p = fmaf(p, r, 0x1.555556p-5f);
  p = fmaf(p, r, 0x1.555556p-3f);
  p = fmaf(p, r, 0.5f);
  p = fmaf(p, r, 1.0f);
  p = fmaf(p, r, 1.0f);
  return ldexpf(p, (int)n);
}

/* Reported probability of a kept id: its wide weight over the top-p mass S'
 * (2^-40 units).  S' differs from the exact sum of the weights by at most
 * one unit per kept id (plus the weights below 2^-40 it leaves out) and is
 * at least 2^40, so the ratio carries only the float roundings of the
 * weight, of f32(S') and of the quotient. */
float tgo_kept_prob(float y, float m, float fs) { return (tgo_weight_wide(y, m) * 0x1p40f) / fs; }

float tgo_u64_to_f32(uint64_t x) {
  if (x < (1ull << 24)) return (float)(uint32_t)x;
  int lz = __builtin_clzll(x);
  int sh = 40 - lz; /* bits below the 24-bit significand */
  uint64_t m = x >> sh;
  uint64_t rem = x & ((1ull << sh) - 1);
  uint64_t half = 1ull << (sh - 1);
  if (rem > half || (rem == half && (m & 1))) m += 1;
  float f = (float)(uint32_t)m; /* m <= 2^24: exact */
  return f * u2f((uint32_t)(sh + 127) << 23);
}

uint32_t tgo_key(float f) {
  uint32_t u = f2u(f);
  if (u == 0x80000000u) u = 0;
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

float tgo_unkey(uint32_t k) { return u2f((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k); }

static inline uint64_t comp_key(float y, int v) {
  return ((uint64_t)tgo_key(y) << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)v);
}
static inline int comp_id(uint64_t c) { return (int)(0xFFFFFFFFu - (uint32_t)c); }
static inline float comp_y(uint64_t c) { return tgo_unkey((uint32_t)(c >> 32)); }

static inline float bf16_to_f32(uint16_t h) { return u2f((uint32_t)h << 16); }

/* -------------------------------------------------------------- selection */

/* Rearrange a[0..n) so its kk largest values occupy a[0..kk) (any order).
 * Quickselect with a median-of-three pivot (the reference uses
 * std::nth_element for the same job, model.cpp:502-503). */
static void select_top(uint64_t* a, long n, long kk) {
  long lo = 0, hi = n - 1;
  if (kk <= 0 || kk >= n) return;
  long target = kk - 1; /* position of the kk-th largest in desc order */
  while (hi > lo) {
    long mid = lo + (hi - lo) / 2;
    uint64_t x = a[lo], y = a[mid], z = a[hi], piv;
    if (x < y) { uint64_t t = x; x = y; y = t; }
    if (y < z) { uint64_t t = y; y = z; z = t; }
    if (x < y) { uint64_t t = x; x = y; y = t; }
    piv = y; /* median */
    long i = lo, j = hi;
    while (i <= j) { /* descending partition */
      while (a[i] > piv) i++;
      while (a[j] < piv) j--;
      if (i <= j) {
        uint64_t t = a[i];
        a[i] = a[j];
        a[j] = t;
        i++;
        j--;
      }
    }
    if (target <= j) hi = j;
    else if (target >= i) lo = i;
    else return;
  }
}

static int cmp_desc(const void* pa, const void* pb) {
  uint64_t a = *(const uint64_t*)pa, b = *(const uint64_t*)pb;
  return (a < b) - (a > b);
}

/* ------------------------------------------------------------- row sampler */

typedef struct {
  int V;
  int32_t* counts; /* [V] history counts */
  uint64_t* keys;  /* [V] composite keys */
  uint64_t* cdf;   /* [V] prefix masses  */
} scratch_t;

static int scratch_init(scratch_t* s, int V) {
  s->V = V;
  s->counts = (int32_t*)calloc((size_t)V, sizeof(int32_t));
  s->keys = (uint64_t*)malloc((size_t)V * sizeof(uint64_t));
  s->cdf = (uint64_t*)malloc((size_t)V * sizeof(uint64_t));
  return (s->counts && s->keys && s->cdf) ? 0 : -1;
}
static void scratch_free(scratch_t* s) {
  free(s->counts);
  free(s->keys);
  free(s->cdf);
}

static int row_invalid(tgo_row_result* r) {
  memset(r, 0, sizeof(*r));
  r->token = -2;
  r->cut_id = -1;
  return -2;
}

static int sample_row_impl(const float* x, int V, const int32_t* hist, int H, const tgo_params* p,
                           const uint32_t* mask_row, float u, tgo_row_result* r,
                           int32_t* kept_ids, float* kept_probs, int kept_cap,
                           float* post_logits, scratch_t* s) {
  tgo_row_result res;
  memset(&res, 0, sizeof(res));
  res.cut_id = -1;
  if (kept_ids)
    for (int i = 0; i < kept_cap; i++) kept_ids[i] = -1;
  if (kept_probs)
    for (int i = 0; i < kept_cap; i++) kept_probs[i] = 0.0f;

  /* ---- parameter validation (same rules as the kernels) ---- */
  const float T = p->temperature;
  if (isnan(T)) return row_invalid(r);
  const int greedy = (p->flags & TGO_FLAG_GREEDY) || T <= 0.0f;
  float invT = 1.0f;
  if (!greedy) {
    if (!isfinite(T)) return row_invalid(r);
    invT = 1.0f / T;
    if (!isfinite(invT)) return row_invalid(r);
    if (isnan(p->top_p) || p->top_p <= 0.0f) return row_invalid(r);
    if (isnan(u) || u < 0.0f || u >= 1.0f) return row_invalid(r);
  }
  if (!(p->repetition > 0.0f) || !isfinite(p->repetition)) return row_invalid(r);
  if (!isfinite(p->presence) || !isfinite(p->frequency)) return row_invalid(r);
  if (H < 0) return row_invalid(r);
  res.greedy = greedy;

  /* ---- penalties: counts of in-range history ids ---- */
  const int neutral = (p->repetition == 1.0f && p->presence == 0.0f && p->frequency == 0.0f);
  const int use_pen = (H > 0 && !neutral);
  if (use_pen)
    for (int j = 0; j < H; j++)
      if (hist[j] >= 0 && hist[j] < V) s->counts[hist[j]]++;

  /* ---- canonical y for every id ---- */
  long n = 0;
  uint64_t best = 0;
  int have_best = 0;
  for (int v = 0; v < V; v++) {
    float z = x[v];
    if (use_pen && s->counts[v] > 0) {
      const float rp = p->repetition;
      if (rp != 1.0f) z = (z > 0.0f) ? z / rp : z * rp;
      z = z - p->frequency * (float)s->counts[v];
      z = z - p->presence;
    }
    int allowed = 1;
    if (mask_row && !((mask_row[v >> 5] >> (v & 31)) & 1u)) allowed = 0;
    float y = greedy ? z : z / T;
    if (!(y > -INFINITY)) allowed = 0; /* -inf and NaN */
    if (post_logits) post_logits[v] = allowed ? y : -INFINITY;
    if (!allowed) continue;
    uint64_t c = comp_key(y, v);
    if (greedy) {
      if (!have_best || c > best) { best = c; have_best = 1; }
    } else {
      s->keys[n++] = c;
    }
  }
  if (use_pen)
    for (int j = 0; j < H; j++)
      if (hist[j] >= 0 && hist[j] < V) s->counts[hist[j]] = 0;

  if (greedy) {
    if (!have_best) {
      res.token = -1;
    } else {
      res.token = comp_id(best);
      res.n_topk = res.n_topp = 1;
      res.cut_id = res.token;
      if (kept_ids && kept_cap > 0) kept_ids[0] = res.token;
      if (kept_probs && kept_cap > 0) kept_probs[0] = 1.0f;
    }
    *r = res;
    return 0;
  }
  if (n == 0) {
    res.token = -1;
    *r = res;
    return 0;
  }

  /* ---- top-k: the kk largest composite keys, sorted ---- */
  long kk = (p->top_k >= 1 && p->top_k < V) ? (p->top_k < n ? p->top_k : n) : n;
  select_top(s->keys, n, kk);
  qsort(s->keys, (size_t)kk, sizeof(uint64_t), cmp_desc);
  if (kk < n) { /* how many more ids the keep-all-ties rule would keep */
    uint32_t kth = (uint32_t)(s->keys[kk - 1] >> 32);
    for (long i = kk; i < n; i++)
      if ((uint32_t)(s->keys[i] >> 32) == kth) res.ref_tie_extra++;
  }

  /* ---- exact integer masses and prefix ---- */
  const float m = comp_y(s->keys[0]);
  uint64_t acc = 0;
  for (long i = 0; i < kk; i++) {
    acc += tgo_q40(tgo_weight(comp_y(s->keys[i]), m));
    s->cdf[i] = acc;
  }
  const uint64_t S = acc;

  /* ---- top-p ---- */
  long istar = kk - 1;
  if (p->top_p < 1.0f) {
    uint32_t pq = (uint32_t)(p->top_p * 16777216.0f);
    uint64_t P = (uint64_t)(((u128)S * pq) >> 24);
    for (long i = 0; i < kk; i++)
      if (s->cdf[i] >= P) { istar = i; break; }
    double pr = (double)p->top_p * (double)S, tol = 1e-6 * (double)S;
    if (fabs((double)s->cdf[istar] - pr) <= tol ||
        (istar > 0 && fabs((double)s->cdf[istar - 1] - pr) <= tol))
      res.topp_boundary = 1;
  }
  const uint64_t Sp = s->cdf[istar];

  /* ---- draw ---- */
  uint32_t uq = (uint32_t)(u * 16777216.0f);
  uint64_t t = (uint64_t)(((u128)Sp * uq) >> 24);
  long pick = istar;
  for (long i = 0; i <= istar; i++)
    if (s->cdf[i] > t) { pick = i; break; }
  {
    double tr = (double)u * (double)Sp, tol = 1e-6 * (double)Sp;
    if (fabs((double)s->cdf[pick] - tr) <= tol ||
        (pick > 0 && fabs((double)s->cdf[pick - 1] - tr) <= tol))
      res.draw_boundary = 1;
  }

  res.token = comp_id(s->keys[pick]);
  res.n_topk = (int32_t)kk;
  res.n_topp = (int32_t)(istar + 1);
  res.cut_id = comp_id(s->keys[istar]);
  res.mass_k = S;
  res.mass_p = Sp;
  if (kept_ids)
    for (long i = 0; i < kk && i < kept_cap; i++) kept_ids[i] = comp_id(s->keys[i]);
  if (kept_probs) { /* float weights over the top-p mass (not the floored integer masses) */
    float fs = tgo_u64_to_f32(Sp);
    for (long i = 0; i <= istar && i < kept_cap; i++)
      kept_probs[i] = tgo_kept_prob(comp_y(s->keys[i]), m, fs);
  }
  *r = res;
  return 0;
}

int tgo_sample_row(const float* x, int V, const int32_t* hist, int H, const tgo_params* p,
                   const uint32_t* mask_row, float u, tgo_row_result* r, int32_t* kept_ids,
                   float* kept_probs, int kept_cap, float* post_logits) {
  scratch_t s;
  if (V <= 0 || scratch_init(&s, V) != 0) {
    scratch_free(&s);
    return row_invalid(r);
  }
  int rc = sample_row_impl(x, V, hist, H, p, mask_row, u, r, kept_ids, kept_probs, kept_cap,
                           post_logits, &s);
  scratch_free(&s);
  return rc;
}

/* ------------------------------------------------------------- batch */

typedef struct {
  const void* logits;
  int dtype, B, V;
  int64_t row_stride;
  const int32_t* hist;
  const int32_t* hist_len;
  int hist_cap;
  const tgo_params* params;
  const uint32_t* mask_table;
  int n_states;
  const float* u;
  int32_t* out_ids;
  tgo_row_result* results;
  int32_t* kept_ids;
  float* kept_probs;
  int kept_cap;
  float* post_logits;
  int row_begin, row_end;
} batch_job;

static void* batch_worker(void* arg) {
  batch_job* j = (batch_job*)arg;
  scratch_t s;
  if (scratch_init(&s, j->V) != 0) {
    scratch_free(&s);
    return (void*)1;
  }
  float* conv = NULL;
  if (j->dtype == 1) conv = (float*)malloc((size_t)j->V * sizeof(float));
  const int words = (j->V + 31) / 32;
  for (int b = j->row_begin; b < j->row_end; b++) {
    tgo_row_result res;
    const float* row;
    if (j->dtype == 1) {
      const uint16_t* src = (const uint16_t*)j->logits + (int64_t)b * j->row_stride;
      for (int v = 0; v < j->V; v++) conv[v] = bf16_to_f32(src[v]);
      row = conv;
    } else {
      row = (const float*)j->logits + (int64_t)b * j->row_stride;
    }
    const tgo_params* p = &j->params[b];
    int H = j->hist_len ? j->hist_len[b] : j->hist_cap;
    const uint32_t* mrow = NULL;
    int bad = (H < 0 || H > j->hist_cap);
    if (p->mask_state >= 0) {
      if (p->mask_state >= j->n_states || !j->mask_table) bad = 1;
      else mrow = j->mask_table + (int64_t)p->mask_state * words;
    }
    int32_t* kid = j->kept_ids ? j->kept_ids + (int64_t)b * j->kept_cap : NULL;
    float* kpr = j->kept_probs ? j->kept_probs + (int64_t)b * j->kept_cap : NULL;
    float* post = j->post_logits ? j->post_logits + (int64_t)b * j->V : NULL;
    if (bad) {
      row_invalid(&res);
      if (kid)
        for (int i = 0; i < j->kept_cap; i++) kid[i] = -1;
      if (kpr)
        for (int i = 0; i < j->kept_cap; i++) kpr[i] = 0.0f;
    } else {
      sample_row_impl(row, j->V, j->hist ? j->hist + (int64_t)b * j->hist_cap : NULL, H, p, mrow,
                      j->u[b], &res, kid, kpr, j->kept_cap, post, &s);
    }
    if (j->out_ids) j->out_ids[b] = res.token;
    if (j->results) j->results[b] = res;
  }
  free(conv);
  scratch_free(&s);
  return NULL;
}

int tgo_sample_batch(const void* logits, int dtype, int B, int V, int64_t row_stride,
                     const int32_t* hist, const int32_t* hist_len, int hist_cap,
                     const tgo_params* params, const uint32_t* mask_table, int n_states,
                     const float* u, int32_t* out_ids, tgo_row_result* results,
                     int32_t* kept_ids, float* kept_probs, int kept_cap, float* post_logits,
                     int nthreads) {
  if (B < 0 || V <= 0 || (dtype != 0 && dtype != 1) || row_stride < V || hist_cap < 0) return -1;
  if (B == 0) return 0;
  if (nthreads < 1) nthreads = 1;
  if (nthreads > B) nthreads = B;
  batch_job* jobs = (batch_job*)calloc((size_t)nthreads, sizeof(batch_job));
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  int rc = 0;
  for (int t = 0; t < nthreads; t++) {
    batch_job* j = &jobs[t];
    j->logits = logits;
    j->dtype = dtype;
    j->B = B;
    j->V = V;
    j->row_stride = row_stride;
    j->hist = hist;
    j->hist_len = hist_len;
    j->hist_cap = hist_cap;
    j->params = params;
    j->mask_table = mask_table;
    j->n_states = n_states;
    j->u = u;
    j->out_ids = out_ids;
    j->results = results;
    j->kept_ids = kept_ids;
    j->kept_probs = kept_probs;
    j->kept_cap = kept_cap;
    j->post_logits = post_logits;
    j->row_begin = (int)((int64_t)B * t / nthreads);
    j->row_end = (int)((int64_t)B * (t + 1) / nthreads);
  }
  if (nthreads == 1) {
    if (batch_worker(&jobs[0]) != NULL) rc = -1;
  } else {
    for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, batch_worker, &jobs[t]);
    for (int t = 0; t < nthreads; t++) {
      void* ret;
      pthread_join(th[t], &ret);
      if (ret != NULL) rc = -1;
    }
  }
  free(jobs);
  free(th);
  return rc;
}

/* --------------------------------------------------- speculative verify */

/* Canonical softmax denominator of one row of y values:
 *   m = max y;  per aligned block of TGO_SPEC_BLOCK ids with block max m_b:
 *   Q_b = sum q40(weight(y_v, m_b)) (exact), term_b = (f32(Q_b) * 2^-40) * weight(m_b, m);
 *   S = pairwise tree over term_0..term_{nb-1}, padded with zeros to a power of two.
 * Returns S (0 if no element is allowed) and writes m. */
float tgo_spec_row_stats(const float* y, int V, float* m_out) {
  float m = -INFINITY;
  for (int v = 0; v < V; v++)
    if (y[v] > m) m = y[v];
  *m_out = m;
  if (!(m > -INFINITY)) return 0.0f;
  int nb = (V + TGO_SPEC_BLOCK - 1) / TGO_SPEC_BLOCK;
  int np = 1;
  while (np < nb) np <<= 1;
  float* terms = (float*)calloc((size_t)np, sizeof(float));
  for (int b = 0; b < nb; b++) {
    int lo = b * TGO_SPEC_BLOCK, hi = lo + TGO_SPEC_BLOCK < V ? lo + TGO_SPEC_BLOCK : V;
    float mb = -INFINITY;
    for (int v = lo; v < hi; v++)
      if (y[v] > mb) mb = y[v];
    if (!(mb > -INFINITY)) continue;
    uint64_t Q = 0;
    for (int v = lo; v < hi; v++)
      if (y[v] > -INFINITY) Q += tgo_q40(tgo_weight(y[v], mb));
    terms[b] = (tgo_u64_to_f32(Q) * 0x1p-40f) * tgo_weight(mb, m);
  }
  for (int w = np; w > 1; w >>= 1)
    for (int i = 0; i < w / 2; i++) terms[i] = terms[2 * i] + terms[2 * i + 1];
  float S = terms[0];
  free(terms);
  return S;
}

/* y = z / T (IEEE division), -inf for NaN / -inf inputs (greedy rows: T == 1).
 * SpeculativeDecode.swift:141,158 scales by the clamped temperature. */
static void spec_scale_row(const void* base, int dtype, int64_t off, int V, float T, float* y) {
  for (int v = 0; v < V; v++) {
    float z = dtype == 1 ? bf16_to_f32(((const uint16_t*)base)[off + v]) : ((const float*)base)[off + v];
    float t = z / T;
    y[v] = (t > -INFINITY) ? t : -INFINITY;
  }
}

static int spec_argmax(const float* y, int V) {
  uint64_t best = 0;
  int have = 0;
  for (int v = 0; v < V; v++) {
    if (!(y[v] > -INFINITY)) continue;
    uint64_t c = comp_key(y[v], v);
    if (!have || c > best) { best = c; have = 1; }
  }
  return have ? comp_id(best) : -1;
}

/* id-order CDF draw over exact masses w[0..V): first v with prefix > t. */
static int draw_id_order(const uint64_t* w, int V, uint64_t total, uint32_t uq, int* boundary,
                         float u) {
  uint64_t t = (uint64_t)(((u128)total * uq) >> 24);
  uint64_t acc = 0, prev = 0;
  int pick = -1;
  for (int v = 0; v < V; v++) {
    prev = acc;
    acc += w[v];
    if (acc > t) { pick = v; break; }
  }
  if (boundary) {
    double tr = (double)u * (double)total, tol = 1e-6 * (double)total;
    *boundary = (pick >= 0 && (fabs((double)acc - tr) <= tol || fabs((double)prev - tr) <= tol));
  }
  return pick;
}

int tgo_spec_verify_row(const void* target, const void* draft, int dtype, int64_t row_stride,
                        const int32_t* dtok, int k, int V, float T, const float* u_acc,
                        float u_res, int32_t* out, tgo_spec_info* info) {
  tgo_spec_info inf;
  memset(&inf, 0, sizeof(inf));
  for (int j = 0; j <= k; j++) out[j] = -1;
  if (k < 0 || V <= 0 || isnan(T)) {
    out[0] = -2;
    inf.n_acc = -1;
    if (info) *info = inf;
    return -2;
  }
  for (int j = 0; j < k; j++)
    if (dtok[j] < 0 || dtok[j] >= V) {
      out[0] = -2;
      inf.n_acc = -1;
      if (info) *info = inf;
      return -2;
    }
  float* yt = (float*)malloc((size_t)V * sizeof(float));
  float* yd = (float*)malloc((size_t)V * sizeof(float));
  uint64_t* w = (uint64_t*)malloc((size_t)V * sizeof(uint64_t));
  int rc = 0;

  if (T <= 0.0f) { /* greedy verify: SpeculativeDecode.swift:41-98 */
    int j;
    for (j = 0; j < k; j++) {
      spec_scale_row(target, dtype, (int64_t)j * row_stride, V, 1.0f, yt);
      int a = spec_argmax(yt, V);
      out[j] = a;
      if (a != dtok[j]) break;
    }
    if (j == k) {
      spec_scale_row(target, dtype, (int64_t)k * row_stride, V, 1.0f, yt);
      out[k] = spec_argmax(yt, V);
      inf.resampled = 3;
    }
    inf.n_acc = j;
    inf.n_out = j + 1;
    goto done;
  }

  {
    /* stochastic verify: SpeculativeDecode.swift:121-210 with T = max(T, 1e-5) */
    const float Tc = T > 1e-5f ? T : 1e-5f;
    const float invT = 1.0f / Tc;
    if (!(invT > 0.0f) || !isfinite(invT)) {
      out[0] = -2;
      inf.n_acc = -1;
      rc = -2;
      goto done;
    }
    for (int j = 0; j < k; j++)
      if (isnan(u_acc[j]) || u_acc[j] < 0.0f || u_acc[j] >= 1.0f) {
        out[0] = -2;
        inf.n_acc = -1;
        rc = -2;
        goto done;
      }
    if (isnan(u_res) || u_res < 0.0f || u_res >= 1.0f) {
      out[0] = -2;
      inf.n_acc = -1;
      rc = -2;
      goto done;
    }
    const uint32_t uq = (uint32_t)(u_res * 16777216.0f);
    int j;
    for (j = 0; j < k; j++) {
      float mt, md;
      spec_scale_row(target, dtype, (int64_t)j * row_stride, V, Tc, yt);
      spec_scale_row(draft, dtype, (int64_t)j * row_stride, V, Tc, yd);
      float St = tgo_spec_row_stats(yt, V, &mt);
      float Sd = tgo_spec_row_stats(yd, V, &md);
      if (j < 16) {
        inf.s_target[j] = St;
        inf.s_draft[j] = Sd;
      }
      if (!(St > 0.0f) || !(Sd > 0.0f)) {
        out[0] = -1;
        inf.n_acc = -1;
        rc = -1;
        goto done;
      }
      const int d = dtok[j];
      float pt = tgo_weight(yt[d], mt) / St;
      float pd = tgo_weight(yd[d], md) / Sd;
      float ratio = pt / fmaxf(pd, 1e-10f);
      inf.ratio_last = ratio;
      if (fabsf(u_acc[j] - ratio) <= 1e-6f) inf.accept_boundary = 1;
      if (u_acc[j] < ratio) {
        out[j] = d;
        continue;
      }
      /* rejected: residual max(pT - pD, 0), drawn in id order */
      uint64_t R = 0;
      for (int v = 0; v < V; v++) {
        float a = tgo_weight(yt[v], mt) / St;
        float b = tgo_weight(yd[v], md) / Sd;
        float rv = fmaxf(a - b, 0.0f);
        w[v] = tgo_q40(rv);
        R += w[v];
      }
      inf.resid_mass = R;
      if (R >= 110) { /* R * 2^-40 > 1e-10 */
        out[j] = draw_id_order(w, V, R, uq, &inf.draw_boundary, u_res);
        inf.resampled = 1;
      } else { /* p_target <= p_draft everywhere: draw from p_target */
        uint64_t Sq = 0;
        for (int v = 0; v < V; v++) {
          w[v] = tgo_q40(tgo_weight(yt[v], mt));
          Sq += w[v];
        }
        out[j] = draw_id_order(w, V, Sq, uq, &inf.draw_boundary, u_res);
        inf.resampled = 2;
      }
      break;
    }
    if (j == k) { /* all accepted: bonus token from target row k */
      float mt;
      spec_scale_row(target, dtype, (int64_t)k * row_stride, V, Tc, yt);
      tgo_spec_row_stats(yt, V, &mt);
      if (!(mt > -INFINITY)) {
        out[0] = -1;
        inf.n_acc = -1;
        rc = -1;
        goto done;
      }
      uint64_t Sq = 0;
      for (int v = 0; v < V; v++) {
        w[v] = tgo_q40(tgo_weight(yt[v], mt));
        Sq += w[v];
      }
      out[k] = draw_id_order(w, V, Sq, uq, &inf.draw_boundary, u_res);
      inf.resampled = 3;
    }
    inf.n_acc = j;
    inf.n_out = j + 1;
  }
done:
  free(yt);
  free(yd);
  free(w);
  if (info) *info = inf;
  return rc;
}

typedef struct {
  const void* target;
  const void* draft;
  int dtype;
  const int32_t* dtok;
  int k, V;
  const float* T;
  const float* u_acc;
  const float* u_res;
  int32_t* n_acc;
  int32_t* out;
  tgo_spec_info* infos;
  int b0, b1;
} spec_job;

static void* spec_worker(void* arg) {
  spec_job* j = (spec_job*)arg;
  const int64_t V = j->V;
  const size_t esz = j->dtype == 1 ? 2 : 4;
  for (int b = j->b0; b < j->b1; b++) {
    tgo_spec_info inf;
    const char* tb = (const char*)j->target + (size_t)b * (j->k + 1) * V * esz;
    const char* db = (const char*)j->draft + (size_t)b * j->k * V * esz;
    tgo_spec_verify_row(tb, db, j->dtype, V, j->dtok + (int64_t)b * j->k, j->k, j->V, j->T[b],
                        j->u_acc + (int64_t)b * j->k, j->u_res[b], j->out + (int64_t)b * (j->k + 1),
                        &inf);
    if (j->n_acc) j->n_acc[b] = inf.n_acc;
    if (j->infos) j->infos[b] = inf;
  }
  return NULL;
}

int tgo_spec_verify_batch(const void* target, const void* draft, int dtype, const int32_t* dtok,
                          int B, int k, int V, const float* T, const float* u_acc,
                          const float* u_res, int32_t* n_acc, int32_t* out,
                          tgo_spec_info* infos, int nthreads) {
  if (B < 0 || k < 0 || V <= 0 || (dtype != 0 && dtype != 1)) return -1;
  if (B == 0) return 0;
  if (nthreads < 1) nthreads = 1;
  if (nthreads > B) nthreads = B;
  spec_job* jobs = (spec_job*)calloc((size_t)nthreads, sizeof(spec_job));
  pthread_t* th = (pthread_t*)calloc((size_t)nthreads, sizeof(pthread_t));
  for (int t = 0; t < nthreads; t++) {
    spec_job* j = &jobs[t];
    j->target = target;
    j->draft = draft;
    j->dtype = dtype;
    j->dtok = dtok;
    j->k = k;
    j->V = V;
    j->T = T;
    j->u_acc = u_acc;
    j->u_res = u_res;
    j->n_acc = n_acc;
    j->out = out;
    j->infos = infos;
    j->b0 = (int)((int64_t)B * t / nthreads);
    j->b1 = (int)((int64_t)B * (t + 1) / nthreads);
  }
  if (nthreads == 1) {
    spec_worker(&jobs[0]);
  } else {
    for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, spec_worker, &jobs[t]);
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
  }
  free(jobs);
  free(th);
  return 0;
}
