#!/usr/bin/env python3
"""Writes tests/golden/tg_ref_c1.npz from the reference's own C++ sampler.

Loads oracle/_ref/libtg_ref.so, which `make -C oracle ref` compiles from the
reference checkout's wasm/src sources (model.cpp + kernels, compiled where
they lie).  The sampler under test is the decode loop of tg_generate
(wasm/src/model.cpp:473-519): greedy strict-'>' argmax, or
p_v = exp((l_v - max)/T), top-k by an nth_element value threshold, and an
id-order walk of a mt19937 draw r ~ U(0, sum p).

The byte-level model has the configuration of the reference's model test
(tests/test_wasm_model.cpp:28: V=256, ctx 32, 2 layers, 2 heads, d_model 64,
d_mlp 128, seed 42) and is trained for a few AdamW steps on that test's
repeated sentence (tests/test_wasm_model.cpp:38-42), so its next-byte
distributions are neither uniform nor one-hot.

Contents:
  greedy_prompt  int32[n]      prompt bytes
  greedy_out     int32[32]     tg_generate(prompt, T=0, 32 new bytes)
  greedy_logits  float32[32,256] the logits row each greedy byte was chosen from
  samp_prompt_*  int32[n]      prompt of sampling case i
  samp_logits    float32[C,256] last-position logits of each sampling case
  samp_T         float32[C]    temperature
  samp_k         int32[C]      top_k (0: disabled)
  samp_counts    int64[C,256]  histogram of tg_generate(prompt, T, top_k, seed=s, 1 byte), s < N
  samp_n         int64         N

Run from the repository root:  python3 tests/golden/make_tg_ref.py
"""
from __future__ import annotations

import ctypes as C
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
LIB = os.path.join(ROOT, "oracle", "_ref", "libtg_ref.so")
OUT = os.path.join(ROOT, "tests", "golden", "tg_ref_c1.npz")

MODEL = dict(vocab=256, ctx=32, n_layers=2, n_heads=2, d_model=64, d_mlp=128, seed=42)
TRAIN_STEPS = 60
CORPUS_UNIT = b"the quick brown fox jumps over the lazy dog. "
GREEDY_PROMPT = b"the quick"
GREEDY_NEW = 32
N_DRAWS = 20000
# (prompt, temperature, top_k); case 0 uses the byte-level config's T and k.
CASES = [
    (b"the quick brown ", 0.8, 40),
    (b"the lazy ", 1.5, 0),
    (b"jumps ov", 1.2, 5),
    (b"\n", 2.0, 2),
]


def load():
    L = C.CDLL(LIB)
    P = C.c_void_p
    L.tg_model_create.restype = P
    L.tg_model_create.argtypes = [C.c_int] * 6 + [C.c_uint]
    L.tg_model_free.argtypes = [P]
    L.tg_set_data.argtypes = [P, C.c_char_p, C.c_int, C.c_float]
    L.tg_train_step.restype = C.c_float
    L.tg_train_step.argtypes = [P, C.c_int, C.c_float, C.c_float]
    L.tg_generate.restype = C.c_int
    L.tg_generate.argtypes = [P, C.c_char_p, C.c_int, C.c_char_p, C.c_int, C.c_float, C.c_int, C.c_uint]
    L.tgref_last_logits.restype = C.c_int
    L.tgref_last_logits.argtypes = [P, P, C.c_int, P]
    return L


def trained_model(L):
    m = L.tg_model_create(MODEL["vocab"], MODEL["ctx"], MODEL["n_layers"], MODEL["n_heads"],
                          MODEL["d_model"], MODEL["d_mlp"], MODEL["seed"])
    corpus = CORPUS_UNIT * (3000 // len(CORPUS_UNIT) + 1)
    L.tg_set_data(m, corpus, len(corpus), 0.9)
    for _ in range(TRAIN_STEPS):
        L.tg_train_step(m, 8, 1e-3, 1.0)
    return m


def last_logits(L, m, ids):
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    out = np.empty(MODEL["vocab"], dtype=np.float32)
    L.tgref_last_logits(m, ids.ctypes.data_as(C.c_void_p), len(ids), out.ctypes.data_as(C.c_void_p))
    return out


def generate(L, m, prompt, n, T, k, seed):
    buf = C.create_string_buffer(n)
    got = L.tg_generate(m, prompt, len(prompt), buf, n, T, k, seed)
    return np.frombuffer(buf.raw[:got], dtype=np.uint8).astype(np.int32)


def main():
    if not os.path.exists(LIB):
        sys.exit(f"{LIB} is missing: run `make -C oracle ref` with the reference checkout present")
    L = load()
    m = trained_model(L)
    data = {}
    g = generate(L, m, GREEDY_PROMPT, GREEDY_NEW, 0.0, 0, 0)
    ids = list(GREEDY_PROMPT)
    rows = []
    for t in g:
        rows.append(last_logits(L, m, ids))
        ids.append(int(t))
    data["greedy_prompt"] = np.frombuffer(GREEDY_PROMPT, dtype=np.uint8).astype(np.int32)
    data["greedy_out"] = g
    data["greedy_logits"] = np.stack(rows)
    logits, Ts, ks, counts = [], [], [], []
    for i, (prompt, T, k) in enumerate(CASES):
        data[f"samp_prompt_{i}"] = np.frombuffer(prompt, dtype=np.uint8).astype(np.int32)
        logits.append(last_logits(L, m, list(prompt)))
        Ts.append(T)
        ks.append(k)
        h = np.zeros(MODEL["vocab"], dtype=np.int64)
        for s in range(N_DRAWS):
            h[generate(L, m, prompt, 1, T, k, s)[0]] += 1
        counts.append(h)
    data["samp_logits"] = np.stack(logits).astype(np.float32)
    data["samp_T"] = np.array(Ts, dtype=np.float32)
    data["samp_k"] = np.array(ks, dtype=np.int32)
    data["samp_counts"] = np.stack(counts)
    data["samp_n"] = np.int64(N_DRAWS)
    L.tg_model_free(m)
    np.savez_compressed(OUT, **data)
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
