// tg_ref_harness.cpp -- TEST INFRASTRUCTURE ONLY.
//
// Builds the reference's own C++ sampler (the tg_generate loop of the
// reference checkout's wasm/src/model.cpp:473-519) into oracle/_ref/ so the
// CPU oracle can be checked against it.  The reference sources are compiled
// where they lie (oracle/Makefile, target `ref`); nothing of them is copied
// into this repository.  model.cpp is included into this translation unit
// only to reach its forward pass (an internal function), so that a test can
// read the exact logits row tg_generate samples from at each step.
//
// Exports (besides the reference's own tg_* C ABI, model.h:17-56):
//   tgref_last_logits  logits of the last position for a token window, by
//                      the same window rule tg_generate uses
//                      (model.cpp:479-487: the last min(n, ctx) ids; an
//                      empty prompt is replaced by '\n').
#include "model.cpp"  // resolved through -I<reference>/wasm/src

extern "C" int tgref_last_logits(TgModel handle, const int* ids, int n, float* out) {
  Model* m = static_cast<Model*>(handle);
  const int nl = '\n';
  if (n <= 0) {
    ids = &nl;
    n = 1;
  }
  const int t = std::min(n, m->ctx);
  forward(*m, ids + (n - t), 1, t);
  const float* row = m->acts.logits.data() + static_cast<long>(t - 1) * m->V;
  std::copy(row, row + m->V, out);
  return m->V;
}

extern "C" int tgref_vocab(TgModel handle) { return static_cast<Model*>(handle)->V; }
