"""Seeded synthetic inputs for the five benchmark configurations.

Each generator returns numpy arrays (host); the same arrays feed the GPU
sampler and the CPU baseline.  Seeds are S_c = 0x74696E7967707400 + c.
Uniforms are k * 2^-24 for integer k (exactly representable in fp32).

  C1  B=1,    V=256,    fp32 N(0,2^2); T .8, top-k 40, top-p .95, rep 1.1,
      64-id history; 1000 decode steps (history appends the sampled id).
  C2  B=64,   V=128256, fp32 N(0,3^2) with 8 spike ids per row set to 12.0;
      T .7, top-k 50, top-p .9, presence .5, frequency .3, 512-id Zipf(1.1)
      history.
  C3  B=128,  V=32000,  fp32 N(0,2.5^2); 4096 mask states, density
      log-uniform in [0.1%, 30%]; rows 0..63 greedy, 64..127 T 1, top-p .95.
  C4  B=1024, V=151936, bf16 of N(0,3^2) + per-row N(0,3^2) offset; per-row
      top-k U{1..1024}, top-p U[.5,1], T U[.3,1.5], rep U[1.05,1.3],
      256-id uniform history.
  C5  B=32, k=8, V=128256: target N(0,3^2) [B,9,V]; draft = target[:, :8] +
      N(0,1^2); draft tokens drawn from softmax(draft) (T = 1).
"""
from __future__ import annotations

import numpy as np

from .sampler import make_params

SEED_BASE = 0x74696E7967707400


def rng(c: int) -> np.random.Generator:
    return np.random.default_rng(SEED_BASE + c)


def uniforms(g: np.random.Generator, shape) -> np.ndarray:
    return (g.integers(0, 1 << 24, size=shape, dtype=np.int64) * (1.0 / (1 << 24))).astype(np.float32)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16, returned as uint16 bits."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    bias = ((b >> 16) & 1) + 0x7FFF
    out = ((b + bias) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    if nan.any():
        out[nan] = 0x7FC0
    return out


def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (h.astype(np.uint32) << 16).view(np.float32)


def zipf_ids(g: np.random.Generator, n: int, V: int, s: float = 1.1, shape=None) -> np.ndarray:
    w = np.arange(1, V + 1, dtype=np.float64) ** (-s)
    cdf = np.cumsum(w)
    cdf /= cdf[-1]
    u = g.random(size=shape if shape is not None else n)
    return np.minimum(np.searchsorted(cdf, u, side="right"), V - 1).astype(np.int32)


def normal_f32(g: np.random.Generator, shape, sigma: float) -> np.ndarray:
    return (g.standard_normal(size=shape, dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def config2(B: int = 64, V: int = 128256, H: int = 512, seed_offset: int = 0):
    g = rng(2 + seed_offset)
    logits = normal_f32(g, (B, V), 3.0)
    for b in range(B):
        spikes = g.choice(V, size=8, replace=False)
        logits[b, spikes] = 12.0
    params = make_params(B, temperature=0.7, top_k=50, top_p=0.9, presence=0.5, frequency=0.3)
    hist = zipf_ids(g, 0, V, shape=(B, H))
    u = uniforms(g, B)
    return dict(name="c2_llama3_bpe", logits=logits, params=params, hist=hist,
                hist_len=np.full(B, H, np.int32), u=u, mask_table=None, V=V)


def mask_table_loguniform(g: np.random.Generator, n_states: int, V: int, lo: float = 0.001, hi: float = 0.30):
    """Per-state vocab bitmasks (V/32 words) whose allowed-token density is
    log-uniform in [lo, hi], at least one token per state."""
    words = (V + 31) // 32
    table = np.zeros((n_states, words), dtype=np.uint32)
    dens = np.exp(g.uniform(np.log(lo), np.log(hi), size=n_states))
    for s in range(n_states):
        n = max(1, int(round(dens[s] * V)))
        ids = g.choice(V, size=n, replace=False)
        np.bitwise_or.at(table[s], ids >> 5, (np.uint32(1) << (ids & 31).astype(np.uint32)))
    return table


def config2_masked(B: int = 64, V: int = 128256, H: int = 512, n_states: int = 1024, seed_offset: int = 0):
    """C2 with the grammar mask stage: the north star's full chain (penalties,
    mask, temperature, top-k 50, top-p 0.9, draw).  The mask table follows
    C3's automaton statistics (density log-uniform in [0.1%, 30%], at least
    one token per state) at V = 128256; each row draws a uniform state."""
    c = config2(B=B, V=V, H=H, seed_offset=seed_offset)
    g = rng(20 + seed_offset)
    c["mask_table"] = mask_table_loguniform(g, n_states, V)
    c["params"]["mask_state"] = g.integers(0, n_states, size=B).astype(np.int32)
    c["name"] = "c2m_full_chain_masked"
    return c


def config3(B: int = 128, V: int = 32000, n_states: int = 4096, seed_offset: int = 0):
    g = rng(3 + seed_offset)
    logits = normal_f32(g, (B, V), 2.5)
    table = mask_table_loguniform(g, n_states, V)
    states = g.integers(0, n_states, size=B).astype(np.int32)
    half = B // 2
    params = make_params(B, temperature=1.0, top_k=0, top_p=0.95, mask_state=states)
    params["temperature"][:half] = 0.0
    u = uniforms(g, B)
    return dict(name="c3_grammar", logits=logits, params=params, hist=None, hist_len=None, u=u,
                mask_table=table, V=V)


def config4(B: int = 1024, V: int = 151936, H: int = 256, seed_offset: int = 0):
    g = rng(4 + seed_offset)
    x = normal_f32(g, (B, V), 3.0)
    x += normal_f32(g, (B, 1), 3.0)
    logits = f32_to_bf16_bits(x)
    del x
    params = make_params(
        B,
        temperature=g.uniform(0.3, 1.5, size=B).astype(np.float32),
        top_k=g.integers(1, 1025, size=B).astype(np.int32),
        top_p=g.uniform(0.5, 1.0, size=B).astype(np.float32),
        repetition=g.uniform(1.05, 1.3, size=B).astype(np.float32),
    )
    hist = g.integers(0, V, size=(B, H)).astype(np.int32)
    u = uniforms(g, B)
    return dict(name="c4_large_batch_bf16", logits=logits, params=params, hist=hist,
                hist_len=np.full(B, H, np.int32), u=u, mask_table=None, V=V)


def _softmax_rows(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float64)
    x = x - x.max(axis=-1, keepdims=True)
    e = np.exp(x)
    return e / e.sum(axis=-1, keepdims=True)


def config5(B: int = 32, k: int = 8, V: int = 128256, seed_offset: int = 0, T: float = 1.0):
    g = rng(5 + seed_offset)
    target = normal_f32(g, (B, k + 1, V), 3.0)
    draft = (target[:, :k, :] + normal_f32(g, (B, k, V), 1.0)).astype(np.float32)
    dtok = np.empty((B, k), dtype=np.int32)
    for b in range(B):
        p = _softmax_rows(draft[b] / T)
        c = np.cumsum(p, axis=-1)
        uu = g.random(size=(k, 1))
        dtok[b] = np.minimum((c < uu).sum(axis=-1), V - 1)
    u_acc = uniforms(g, (B, k))
    u_res = uniforms(g, B)
    return dict(name="c5_spec_verify", target=target, draft=draft, dtok=dtok,
                T=np.full(B, T, np.float32), u_acc=u_acc, u_res=u_res, V=V, k=k)


def config1_step_inputs(steps: int = 1000, V: int = 256, H: int = 64):
    """C1: per-step logits and uniforms plus the initial history ring."""
    g = rng(1)
    logits = normal_f32(g, (steps, V), 2.0)
    u = uniforms(g, steps)
    hist0 = g.integers(0, V, size=H).astype(np.int32)
    params = make_params(1, temperature=0.8, top_k=40, top_p=0.95, repetition=1.1)
    return dict(name="c1_byte_level", logits=logits, u=u, hist0=hist0, params=params, V=V, H=H)


# Algorithmic bytes per unit (one sampled row / one verified sequence).
def algorithmic_bytes_per_row(name: str, V: int, H: int = 0, k: int = 8, dtype_bytes: int = 4) -> int:
    if name.startswith("c3"):
        return 4 * V + V // 8
    if name.startswith("c5"):
        return (2 * k + 1) * V * dtype_bytes
    if name.startswith("c2m"):  # logits, history ids, the row's mask bits
        return dtype_bytes * V + 4 * H + V // 8
    return dtype_bytes * V + 4 * H
