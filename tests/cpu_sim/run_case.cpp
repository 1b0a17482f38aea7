// run_case.cpp -- drives tgs_sample / tgs_spec_verify through the C ABI on the
// CPU simulation of the kernels (TEST INFRASTRUCTURE ONLY).
//   run_case sample <dir>   reads <dir>/meta.txt and the raw input arrays,
//                           writes the outputs next to them.
#include <cstdint>
#include <cstdio>
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include <unistd.h>

#include "../../include/tgs_sampler.h"

static std::vector<char> slurp(const std::string& path) {
  std::vector<char> v;
  FILE* f = std::fopen(path.c_str(), "rb");
  if (!f) return v;
  std::fseek(f, 0, SEEK_END);
  long n = std::ftell(f);
  std::fseek(f, 0, SEEK_SET);
  v.resize(n);
  if (n && std::fread(v.data(), 1, n, f) != (size_t)n) v.clear();
  std::fclose(f);
  return v;
}
static void dump(const std::string& path, const void* p, size_t n) {
  FILE* f = std::fopen(path.c_str(), "wb");
  std::fwrite(p, 1, n, f);
  std::fclose(f);
}

int main(int argc, char** argv) {
  if (argc < 3) return 2;
  // a simulated run that has not ended after this long is stopped by
  // SIGALRM (a deadlock in a simulated kernel ends the test, not the suite)
  const char* al = std::getenv("TGS_SIM_ALARM");
  alarm(al ? (unsigned)std::atoi(al) : 900u);
  const std::string mode = argv[1], dir = argv[2];
  FILE* m = std::fopen((dir + "/meta.txt").c_str(), "r");
  if (!m) return 3;
  if (mode == "sample") {
    int B, V, dtype, hist_cap, has_len, n_states, hint, kept_cap, post, hint_min;
    long long stride;
    if (std::fscanf(m, "%d %d %lld %d %d %d %d %d %d %d %d", &B, &V, &stride, &dtype, &hist_cap, &has_len,
                    &n_states, &hint, &kept_cap, &post, &hint_min) != 11)
      return 4;
    std::fclose(m);
    auto logits = slurp(dir + "/logits.bin");
    auto params = slurp(dir + "/params.bin");
    auto u = slurp(dir + "/u.bin");
    auto hist = slurp(dir + "/hist.bin");
    auto hlen = slurp(dir + "/hist_len.bin");
    auto mask = slurp(dir + "/mask.bin");
    tgs_handle h;
    int rc = tgs_create(&h, 0, B > 0 ? B : 1, V, hist_cap);
    if (rc) { std::printf("create %d\n", rc); return 5; }
    if (n_states > 0) {
      rc = tgs_mask_table_set(h, (const uint32_t*)mask.data(), n_states, V);
      if (rc) { std::printf("mask %d\n", rc); return 6; }
    }
    std::vector<int32_t> out(B), kid((size_t)B * kept_cap), counts(2 * (size_t)B), cut(B);
    std::vector<float> kpr((size_t)B * kept_cap), postv(post ? (size_t)B * V : 1);
    std::vector<uint64_t> mass(2 * (size_t)B);
    tgs_debug dbg = {kid.data(), kpr.data(), kept_cap, counts.data(), mass.data(), cut.data(),
                     post ? postv.data() : nullptr};
    tgs_batch_hint hb = {hint, hint_min};
    // TGS_SIM_REPEAT=n: n calls on the same inputs, each of whose ids must
    // equal the first call's (the split kernel's state carries over calls)
    const char* rep_env = std::getenv("TGS_SIM_REPEAT");
    int reps = rep_env ? std::max(1, std::atoi(rep_env)) : 1;
    // TGS_SIM_FIRST_MERGE_SPINS=n: three more calls first, on the rows
    // reversed (other candidates) and with the merge's poll limit n, so that
    // merges give up and late lists stay behind in the workspace; their ids
    // are not kept, and the calls after them must not take any of their
    // entries
    const char* fms = std::getenv("TGS_SIM_FIRST_MERGE_SPINS");
    const int lead = fms ? 3 : 0;
    int gave_up = 0;
    std::vector<char> logits_rev;
    if (fms) {
      reps += lead;
      const size_t es = dtype == 1 ? 2 : 4;
      logits_rev = logits;
      for (int b = 0; b < B; b++)
        for (int v = 0; v < V; v++)
          std::memcpy(logits_rev.data() + ((size_t)b * stride + v) * es,
                      logits.data() + ((size_t)b * stride + (V - 1 - v)) * es, es);
      setenv("TGS_MERGE_SPINS", fms, 1);
    }
    std::vector<int32_t> first;
    for (int it0 = 0; it0 < reps; it0++) {
    const int it = it0 - lead;  // below 0: the leading calls
    const char* lg = it < 0 ? logits_rev.data() : logits.data();
    if (std::getenv("TGS_SIM_NOALLOC")) {  // the allocation-free entry point (static workspace)
      rc = tgs_sample_noalloc(0, lg, (tgs_dtype)dtype, B, V, stride,
                              hist_cap ? (const int32_t*)hist.data() : nullptr,
                              has_len ? (const int32_t*)hlen.data() : nullptr, hist_cap,
                              (const tgs_row_params*)params.data(), (const float*)u.data(), out.data(),
                              n_states > 0 ? (const uint32_t*)mask.data() : nullptr, n_states, V,
                              hint >= 0 ? &hb : nullptr, &dbg, nullptr);
      if (rc) { std::printf("sample_noalloc %d %s\n", rc, tgs_last_error(nullptr)); return 7; }
    } else {
      rc = tgs_sample(h, lg, (tgs_dtype)dtype, B, V, stride,
                      hist_cap ? (const int32_t*)hist.data() : nullptr,
                      has_len ? (const int32_t*)hlen.data() : nullptr, hist_cap, (const tgs_row_params*)params.data(),
                      (const float*)u.data(), out.data(), hint >= 0 ? &hb : nullptr, &dbg, nullptr);
      if (rc) { std::printf("sample %d %s\n", rc, tgs_last_error(h)); return 7; }
    }
    if (it < 0) {
      for (int b = 0; b < B; b++) gave_up += out[b] == -4;
      if (it == -1) {
        std::printf("leading calls: %d rows gave up\n", gave_up);
        unsetenv("TGS_MERGE_SPINS");
      }
    } else if (it == 0) {
      first = out;
    } else if (out != first) {
      std::printf("call %d: ids differ from the first call's\n", it);
      return 9;
    }
    }
    dump(dir + "/out_ids.bin", first.data(), first.size() * 4);
    dump(dir + "/out_kept_ids.bin", kid.data(), kid.size() * 4);
    dump(dir + "/out_kept_probs.bin", kpr.data(), kpr.size() * 4);
    dump(dir + "/out_counts.bin", counts.data(), counts.size() * 4);
    dump(dir + "/out_mass.bin", mass.data(), mass.size() * 8);
    dump(dir + "/out_cut.bin", cut.data(), cut.size() * 4);
    if (post) dump(dir + "/out_post.bin", postv.data(), postv.size() * 4);
    tgs_destroy(h);
    return 0;
  }
  if (mode == "spec") {
    int B, k, V, dtype;
    if (std::fscanf(m, "%d %d %d %d", &B, &k, &V, &dtype) != 4) return 4;
    std::fclose(m);
    auto tgt = slurp(dir + "/target.bin");
    auto dft = slurp(dir + "/draft.bin");
    auto dtok = slurp(dir + "/dtok.bin");
    auto T = slurp(dir + "/T.bin");
    auto ua = slurp(dir + "/u_acc.bin");
    auto ur = slurp(dir + "/u_res.bin");
    tgs_handle h;
    int rc = tgs_create(&h, 0, B, V, 0);
    if (rc) return 5;
    std::vector<int32_t> nacc(B), out((size_t)B * (k + 1));
    rc = tgs_spec_verify(h, tgt.data(), dft.data(), (tgs_dtype)dtype, (const int32_t*)dtok.data(), B, k, V,
                         (const float*)T.data(), (const float*)ua.data(), (const float*)ur.data(), nacc.data(),
                         out.data(), nullptr);
    if (rc) { std::printf("spec %d %s\n", rc, tgs_last_error(h)); return 7; }
    dump(dir + "/out_nacc.bin", nacc.data(), nacc.size() * 4);
    dump(dir + "/out_spec.bin", out.data(), out.size() * 4);
    tgs_destroy(h);
    return 0;
  }
  if (mode == "maskbuild") {
    int n_dfa, n_cls, V, n, eos, n_rows;
    if (std::fscanf(m, "%d %d %d %d %d %d", &n_dfa, &n_cls, &V, &n, &eos, &n_rows) != 6) return 4;
    std::fclose(m);
    auto bcls = slurp(dir + "/byte_class.bin");
    auto trans = slurp(dir + "/trans.bin");
    auto comp = slurp(dir + "/complete.bin");
    auto off = slurp(dir + "/tok_off.bin");
    auto bytes = slurp(dir + "/tok_bytes.bin");
    auto st = slurp(dir + "/states.bin");
    auto rows = slurp(dir + "/rows.bin");
    tgs_handle h;
    int rc = tgs_create(&h, 0, n_rows, V, 0);
    if (rc) return 5;
    const int words = (V + 31) / 32;
    std::vector<uint32_t> ones((size_t)n_rows * words, 0xFFFFFFFFu);
    rc = tgs_mask_table_set(h, ones.data(), n_rows, V);
    if (rc) return 6;
    rc = tgs_mask_rows_from_dfa(h, (const uint8_t*)bcls.data(), (const int32_t*)trans.data(), n_cls,
                                (const uint8_t*)comp.data(), n_dfa,
                                (const int32_t*)off.data(), (const uint8_t*)bytes.data(), (int64_t)bytes.size(), V, eos,
                                (const int32_t*)st.data(), (const int32_t*)rows.data(), n, nullptr);
    if (rc) { std::printf("maskbuild %d %s\n", rc, tgs_last_error(h)); return 7; }
    // read the rows back through greedy rows over zero logits
    std::vector<float> zeros((size_t)n_rows * V, 0.0f), u(n_rows, 0.0f), post((size_t)n_rows * V);
    std::vector<tgs_row_params> p(n_rows);
    for (int i = 0; i < n_rows; i++) {
      p[i] = tgs_row_params{0.0f, 0, 1.0f, 1.0f, 0.0f, 0.0f, i, 0};
    }
    std::vector<int32_t> out(n_rows);
    tgs_debug dbg = {nullptr, nullptr, 0, nullptr, nullptr, nullptr, post.data()};
    rc = tgs_sample(h, zeros.data(), TGS_F32, n_rows, V, V, nullptr, nullptr, 0, p.data(), u.data(), out.data(),
                    nullptr, &dbg, nullptr);
    if (rc) { std::printf("sample %d %s\n", rc, tgs_last_error(h)); return 8; }
    dump(dir + "/out_post.bin", post.data(), post.size() * 4);
    tgs_destroy(h);
    return 0;
  }
  if (mode == "logprob") {
    int B, V, dtype;
    long long stride;
    if (std::fscanf(m, "%d %d %lld %d", &B, &V, &stride, &dtype) != 4) return 4;
    std::fclose(m);
    auto logits = slurp(dir + "/logits.bin");
    auto tok = slurp(dir + "/tokens.bin");
    tgs_handle h;
    int rc = tgs_create(&h, 0, 1, 1, 0);
    if (rc) return 5;
    std::vector<float> lp(B), lse(B);
    rc = tgs_token_logprobs(h, logits.data(), (tgs_dtype)dtype, B, V, stride, (const int32_t*)tok.data(), lp.data(),
                            lse.data(), nullptr);
    if (rc) { std::printf("logprob %d %s\n", rc, tgs_last_error(h)); return 7; }
    dump(dir + "/out_lp.bin", lp.data(), lp.size() * 4);
    dump(dir + "/out_lse.bin", lse.data(), lse.size() * 4);
    tgs_destroy(h);
    return 0;
  }
  return 2;
}
