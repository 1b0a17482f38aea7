"""ctypes binding of the CPU oracle (oracle/build/libtgs_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# TGS_ORACLE_LIB: another build of the same source (the sanitizer build of
# tests/oracle_san), used as it is, without building
LIB_PATH = os.environ.get("TGS_ORACLE_LIB") or os.path.join(HERE, "build", "libtgs_oracle.so")

FLAG_GREEDY = 1

PARAMS_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_k", "<i4"),
        ("top_p", "<f4"),
        ("repetition", "<f4"),
        ("presence", "<f4"),
        ("frequency", "<f4"),
        ("mask_state", "<i4"),
        ("flags", "<i4"),
    ]
)
assert PARAMS_DTYPE.itemsize == 32

ROW_RESULT_DTYPE = np.dtype(
    [
        ("token", "<i4"),
        ("n_topk", "<i4"),
        ("n_topp", "<i4"),
        ("cut_id", "<i4"),
        ("mass_k", "<u8"),
        ("mass_p", "<u8"),
        ("draw_boundary", "<i4"),
        ("topp_boundary", "<i4"),
        ("ref_tie_extra", "<i4"),
        ("greedy", "<i4"),
    ]
)

SPEC_INFO_DTYPE = np.dtype(
    [
        ("n_acc", "<i4"),
        ("n_out", "<i4"),
        ("resampled", "<i4"),
        ("accept_boundary", "<i4"),
        ("draw_boundary", "<i4"),
        ("ratio_last", "<f4"),
        ("resid_mass", "<u8"),
        ("s_target", "<f4", (16,)),
        ("s_draft", "<f4", (16,)),
    ]
)

_lib = None


def build() -> str:
    """Compile the oracle with its Makefile (gcc; no GPU needed)."""
    if os.environ.get("TGS_ORACLE_LIB"):
        return LIB_PATH
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def build_ref(ref_root: str = "/root/reference") -> str | None:
    """Compile the reference's own C++ sampler into oracle/_ref/ (the
    checker's checker) when the reference checkout is present; else None."""
    if not os.path.isdir(os.path.join(ref_root, "wasm", "src")):
        return None
    subprocess.run(["make", "-s", "-C", HERE, "ref", f"REF={ref_root}"], check=True)
    return os.path.join(HERE, "_ref", "libtg_ref.so")


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.c_void_p
        L.tgo_expf.restype = C.c_float
        L.tgo_expf.argtypes = [C.c_float]
        L.tgo_weight.restype = C.c_float
        L.tgo_weight.argtypes = [C.c_float, C.c_float]
        L.tgo_weight_wide.restype = C.c_float
        L.tgo_weight_wide.argtypes = [C.c_float, C.c_float]
        L.tgo_q40.restype = C.c_uint64
        L.tgo_q40.argtypes = [C.c_float]
        L.tgo_u64_to_f32.restype = C.c_float
        L.tgo_u64_to_f32.argtypes = [C.c_uint64]
        L.tgo_key.restype = C.c_uint32
        L.tgo_key.argtypes = [C.c_float]
        L.tgo_unkey.restype = C.c_float
        L.tgo_unkey.argtypes = [C.c_uint32]
        L.tgo_spec_row_stats.restype = C.c_float
        L.tgo_spec_row_stats.argtypes = [P, C.c_int, P]
        L.tgo_sample_row.restype = C.c_int
        L.tgo_sample_row.argtypes = [P, C.c_int, P, C.c_int, P, P, C.c_float, P, P, P, C.c_int, P]
        L.tgo_sample_batch.restype = C.c_int
        L.tgo_sample_batch.argtypes = [
            P, C.c_int, C.c_int, C.c_int, C.c_int64, P, P, C.c_int, P, P, C.c_int, P, P, P,
            P, P, C.c_int, P, C.c_int,
        ]
        L.tgo_spec_verify_row.restype = C.c_int
        L.tgo_spec_verify_row.argtypes = [
            P, P, C.c_int, C.c_int64, P, C.c_int, C.c_int, C.c_float, P, C.c_float, P, P,
        ]
        L.tgo_spec_verify_batch.restype = C.c_int
        L.tgo_spec_verify_batch.argtypes = [
            P, P, C.c_int, P, C.c_int, C.c_int, C.c_int, P, P, P, P, P, P, C.c_int,
        ]
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def make_params(n, temperature=1.0, top_k=0, top_p=1.0, repetition=1.0, presence=0.0,
                frequency=0.0, mask_state=-1, flags=0) -> np.ndarray:
    p = np.zeros(n, dtype=PARAMS_DTYPE)
    p["temperature"] = temperature
    p["top_k"] = top_k
    p["top_p"] = top_p
    p["repetition"] = repetition
    p["presence"] = presence
    p["frequency"] = frequency
    p["mask_state"] = mask_state
    p["flags"] = flags
    return p


def sample_batch(logits, params, u, hist=None, hist_len=None, mask_table=None, kept_cap=0,
                 want_post=False, nthreads=1):
    """Run the oracle over a [B, V] batch.  logits: float32 or bfloat16 stored
    as uint16 ([B, V] or [B, row_stride]).  Returns a dict of numpy arrays."""
    logits = np.ascontiguousarray(logits)
    if logits.dtype == np.float32:
        dtype = 0
    elif logits.dtype == np.uint16:
        dtype = 1
    else:
        raise TypeError("logits must be float32 or uint16 (bf16 bits)")
    B, stride = logits.shape
    V = int(params.get("V", stride)) if isinstance(params, dict) else stride
    params = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
    u = np.ascontiguousarray(u, dtype=np.float32)
    if hist is None:
        hist = np.zeros((B, 0), dtype=np.int32)
    hist = np.ascontiguousarray(hist, dtype=np.int32)
    hist_cap = hist.shape[1]
    if hist_len is not None:
        hist_len = np.ascontiguousarray(hist_len, dtype=np.int32)
    n_states = 0
    if mask_table is not None:
        mask_table = np.ascontiguousarray(mask_table, dtype=np.uint32)
        n_states = mask_table.shape[0]
    out = np.empty(B, dtype=np.int32)
    res = np.zeros(B, dtype=ROW_RESULT_DTYPE)
    kept_ids = np.empty((B, kept_cap), dtype=np.int32) if kept_cap else None
    kept_probs = np.empty((B, kept_cap), dtype=np.float32) if kept_cap else None
    post = np.empty((B, V), dtype=np.float32) if want_post else None
    rc = lib().tgo_sample_batch(
        _p(logits), dtype, B, V, stride, _p(hist) if hist_cap else None, _p(hist_len), hist_cap,
        _p(params), _p(mask_table), n_states, _p(u), _p(out), _p(res), _p(kept_ids),
        _p(kept_probs), kept_cap, _p(post), nthreads,
    )
    if rc != 0:
        raise RuntimeError(f"tgo_sample_batch failed ({rc})")
    return {"ids": out, "res": res, "kept_ids": kept_ids, "kept_probs": kept_probs, "post": post}


def spec_verify_batch(target, draft, dtok, T, u_acc, u_res, nthreads=1):
    """target [B, k+1, V], draft [B, k, V] (float32 or uint16 bf16 bits)."""
    target = np.ascontiguousarray(target)
    draft = np.ascontiguousarray(draft)
    dtype = 1 if target.dtype == np.uint16 else 0
    B, k1, V = target.shape
    k = k1 - 1
    dtok = np.ascontiguousarray(dtok, dtype=np.int32).reshape(B, k)
    T = np.ascontiguousarray(T, dtype=np.float32).reshape(B)
    u_acc = np.ascontiguousarray(u_acc, dtype=np.float32).reshape(B, k)
    u_res = np.ascontiguousarray(u_res, dtype=np.float32).reshape(B)
    n_acc = np.empty(B, dtype=np.int32)
    out = np.empty((B, k + 1), dtype=np.int32)
    infos = np.zeros(B, dtype=SPEC_INFO_DTYPE)
    rc = lib().tgo_spec_verify_batch(
        _p(target), _p(draft), dtype, _p(dtok), B, k, V, _p(T), _p(u_acc), _p(u_res), _p(n_acc),
        _p(out), _p(infos), nthreads,
    )
    if rc != 0:
        raise RuntimeError(f"tgo_spec_verify_batch failed ({rc})")
    return {"n_acc": n_acc, "out": out, "info": infos}


def expf(x):
    f = lib().tgo_expf
    return np.array([f(float(v)) for v in np.asarray(x, dtype=np.float32).ravel()], dtype=np.float32)


def weight_wide(x):
    """tgo_weight_wide(x, 0) over an array of x <= 0."""
    f = lib().tgo_weight_wide
    return np.array([f(float(v), 0.0) for v in np.asarray(x, dtype=np.float32).ravel()], dtype=np.float32)


def spec_row_stats(y):
    y = np.ascontiguousarray(y, dtype=np.float32)
    m = np.zeros(1, dtype=np.float32)
    s = lib().tgo_spec_row_stats(_p(y), y.size, _p(m))
    return float(m[0]), float(s)


def token_logprobs(logits, tokens, V=None):
    """log(softmax(x))[b, tokens[b]] and logsumexp(x[b]) of each row, in
    float64: the restatement of scoreLogprobs' `MLX.log(MLX.softmax(logits,
    axis: -1))` gathered at the next token
    (native-mac/Sources/TinyGPTServe/Serve.swift:983-993).

    logits: float32 or bf16 bits (uint16), [B, row_stride], the first V
    columns used.  A row holding NaN or +inf, or only -inf, gives NaN; a token
    outside [0, V) gives NaN.  Returns (logprob [B], lse [B]) float64."""
    x = np.asarray(logits)
    if x.dtype == np.uint16:
        x = (x.astype(np.uint32) << np.uint32(16)).view(np.float32)
    V = x.shape[1] if V is None else V
    x = x[:, :V].astype(np.float64)
    tokens = np.asarray(tokens, dtype=np.int64)
    bad = np.isnan(x).any(axis=1) | np.isposinf(x).any(axis=1)
    m = np.max(np.where(np.isnan(x), -np.inf, x), axis=1)
    bad |= m == -np.inf
    mm = np.where(bad, 0.0, m)
    with np.errstate(invalid="ignore", over="ignore"):
        lse = mm + np.log(np.exp(x - mm[:, None]).sum(axis=1))
    lse[bad] = np.nan
    ok = (tokens >= 0) & (tokens < V)
    xt = np.where(ok, x[np.arange(x.shape[0]), np.clip(tokens, 0, V - 1)], np.nan)
    return xt - lse, lse


def dfa_mask_rows(trans, complete, tokens, states, eos=-1):
    """Mask words (uint32 [n, ceil(V / 32)]) of DFA states: bit v set when
    token v is non-empty and every byte of it has a transition walking from
    the state (the per-token byte replay of ServeTokenMasker.mask(for:),
    native-mac/Sources/TinyGPTServe/Serve.swift:2005-2025, and
    LogitsMasker.mask(forFSM:), ConstrainedGen.swift:805-822); a complete
    state allows only token eos (none when eos < 0).  Vectorised over the
    tokens, one byte position at a time."""
    trans = np.asarray(trans, dtype=np.int64)
    complete = np.asarray(complete, dtype=bool)
    V = len(tokens)
    L = max((len(t) for t in tokens), default=0)
    mat = np.zeros((V, max(L, 1)), dtype=np.int64)
    lens = np.array([len(t) for t in tokens], dtype=np.int64)
    for v, t in enumerate(tokens):
        mat[v, :len(t)] = np.frombuffer(t, dtype=np.uint8)
    words = (V + 31) // 32
    out = np.zeros((len(states), words), dtype=np.uint32)
    for i, s in enumerate(states):
        if complete[s]:
            ok = np.zeros(V, dtype=bool)
            if 0 <= eos < V:
                ok[eos] = True
        else:
            cur = np.full(V, s, dtype=np.int64)
            for p in range(L):
                step = (p < lens) & (cur >= 0)
                cur = np.where(step, trans[np.where(cur >= 0, cur, 0), mat[:, p]], cur)
            ok = (lens > 0) & (cur >= 0)
        pad = np.zeros(words * 32, dtype=bool)
        pad[:V] = ok
        out[i] = np.packbits(pad.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").ravel().astype(np.uint32)
    return out
