/* tgo_sample_batch and tgo_spec_verify_batch on 16 threads under
 * ThreadSanitizer (test infrastructure only).  Each batch runs on one
 * thread and on 16, and every output (ids, per-row results, kept lists,
 * post-penalty logits; speculative ids and counts) must be equal byte for
 * byte.  Rows mix top-k, top-p, penalties over a shared history, grammar
 * mask rows and greedy rows, in fp32 and bf16.  Exit 0 on success. */
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tgs_oracle.h"

static uint64_t g_state = 0x9E3779B97F4A7C15ull;
static uint32_t rnd(void) {
  g_state ^= g_state << 13;
  g_state ^= g_state >> 7;
  g_state ^= g_state << 17;
  return (uint32_t)(g_state >> 11);
}
static float unif(void) { return (float)(rnd() >> 8) * (1.0f / 16777216.0f); }
static float normal(void) {  /* sum of four uniforms, centred */
  return (unif() + unif() + unif() + unif() - 2.0f) * 1.7f;
}

static int sample_case(int B, int V, int dtype, int H, int n_states) {
  const int words = (V + 31) / 32, kept_cap = 64;
  float* x = malloc(sizeof(float) * (size_t)B * V);
  uint16_t* xb = malloc(sizeof(uint16_t) * (size_t)B * V);
  int32_t* hist = malloc(sizeof(int32_t) * (size_t)B * (H > 0 ? H : 1));
  int32_t* hl = malloc(sizeof(int32_t) * B);
  tgo_params* p = calloc(B, sizeof(tgo_params));
  uint32_t* mask = malloc(sizeof(uint32_t) * (size_t)(n_states > 0 ? n_states : 1) * words);
  float* u = malloc(sizeof(float) * B);
  for (size_t i = 0; i < (size_t)B * V; i++) {
    x[i] = normal() * 2.0f;
    uint32_t bits;
    memcpy(&bits, &x[i], 4);
    xb[i] = (uint16_t)(bits >> 16);
  }
  for (int b = 0; b < B; b++) {
    for (int j = 0; j < H; j++) hist[(size_t)b * H + j] = (int32_t)(rnd() % (uint32_t)(V + 8)) - 4;
    hl[b] = H > 0 ? (int32_t)(rnd() % (uint32_t)(H + 1)) : 0;
    u[b] = unif();
    const int kind = b % 5;
    p[b].temperature = kind == 4 ? 0.0f : 0.5f + unif();
    p[b].top_k = kind == 0 ? 1 + (int)(rnd() % 64) : kind == 1 ? 0 : 1 + (int)(rnd() % 1000);
    p[b].top_p = kind == 2 ? 1.0f : 0.5f + 0.49f * unif();
    p[b].repetition = 1.0f + 0.3f * unif();
    p[b].presence = 0.5f * unif();
    p[b].frequency = 0.3f * unif();
    p[b].mask_state = n_states > 0 && (b % 3 == 0) ? (int32_t)(rnd() % (uint32_t)n_states) : -1;
  }
  for (size_t i = 0; i < (size_t)n_states * words; i++) mask[i] = rnd() | rnd();
  const void* lg = dtype == 1 ? (const void*)xb : (const void*)x;
  int32_t* ids[2];
  tgo_row_result* res[2];
  int32_t* kid[2];
  float* kpr[2];
  float* post[2];
  for (int r = 0; r < 2; r++) {
    ids[r] = calloc(B, sizeof(int32_t));
    res[r] = calloc(B, sizeof(tgo_row_result));
    kid[r] = calloc((size_t)B * kept_cap, sizeof(int32_t));
    kpr[r] = calloc((size_t)B * kept_cap, sizeof(float));
    post[r] = calloc((size_t)B * V, sizeof(float));
    const int rc = tgo_sample_batch(lg, dtype, B, V, V, H > 0 ? hist : NULL, H > 0 ? hl : NULL, H, p,
                                    n_states > 0 ? mask : NULL, n_states, u, ids[r], res[r], kid[r], kpr[r],
                                    kept_cap, post[r], r == 0 ? 1 : 16);
    if (rc != 0) {
      fprintf(stderr, "tgo_sample_batch returned %d\n", rc);
      return 1;
    }
  }
  int bad = memcmp(ids[0], ids[1], sizeof(int32_t) * B) != 0 ||
            memcmp(res[0], res[1], sizeof(tgo_row_result) * B) != 0 ||
            memcmp(kid[0], kid[1], sizeof(int32_t) * (size_t)B * kept_cap) != 0 ||
            memcmp(kpr[0], kpr[1], sizeof(float) * (size_t)B * kept_cap) != 0 ||
            memcmp(post[0], post[1], sizeof(float) * (size_t)B * V) != 0;
  printf("sample B=%d V=%d dtype=%d H=%d states=%d: %s\n", B, V, dtype, H, n_states,
         bad ? "16 threads differ from 1" : "ok");
  for (int r = 0; r < 2; r++) {
    free(ids[r]);
    free(res[r]);
    free(kid[r]);
    free(kpr[r]);
    free(post[r]);
  }
  free(x);
  free(xb);
  free(hist);
  free(hl);
  free(p);
  free(mask);
  free(u);
  return bad;
}

static int spec_case(int B, int k, int V) {
  const size_t nt = (size_t)B * (k + 1) * V, nd = (size_t)B * k * V;
  float* tg = malloc(sizeof(float) * nt);
  float* dr = malloc(sizeof(float) * nd);
  int32_t* dtok = malloc(sizeof(int32_t) * (size_t)B * k);
  float* T = malloc(sizeof(float) * B);
  float* ua = malloc(sizeof(float) * (size_t)B * k);
  float* ur = malloc(sizeof(float) * B);
  for (size_t i = 0; i < nt; i++) tg[i] = normal() * 2.0f;
  for (size_t i = 0; i < nd; i++) dr[i] = normal() * 2.0f;
  for (int i = 0; i < B * k; i++) {
    dtok[i] = (int32_t)(rnd() % (uint32_t)V);
    ua[i] = unif();
  }
  for (int b = 0; b < B; b++) {
    T[b] = b % 4 == 0 ? 0.0f : 0.5f + unif();
    ur[b] = unif();
  }
  int32_t* nacc[2];
  int32_t* out[2];
  for (int r = 0; r < 2; r++) {
    nacc[r] = calloc(B, sizeof(int32_t));
    out[r] = calloc((size_t)B * (k + 1), sizeof(int32_t));
    const int rc = tgo_spec_verify_batch(tg, dr, 0, dtok, B, k, V, T, ua, ur, nacc[r], out[r], NULL,
                                         r == 0 ? 1 : 16);
    if (rc != 0) {
      fprintf(stderr, "tgo_spec_verify_batch returned %d\n", rc);
      return 1;
    }
  }
  const int bad = memcmp(nacc[0], nacc[1], sizeof(int32_t) * B) != 0 ||
                  memcmp(out[0], out[1], sizeof(int32_t) * (size_t)B * (k + 1)) != 0;
  printf("spec B=%d k=%d V=%d: %s\n", B, k, V, bad ? "16 threads differ from 1" : "ok");
  for (int r = 0; r < 2; r++) {
    free(nacc[r]);
    free(out[r]);
  }
  free(tg);
  free(dr);
  free(dtok);
  free(T);
  free(ua);
  free(ur);
  return bad;
}

int main(void) {
  int bad = 0;
  bad |= sample_case(64, 5000, 0, 32, 0);
  bad |= sample_case(48, 3000, 1, 16, 4);
  bad |= sample_case(16, 20000, 0, 0, 2);
  bad |= sample_case(5, 700, 0, 8, 0);  /* fewer rows than threads */
  bad |= spec_case(20, 4, 3000);
  return bad;
}
