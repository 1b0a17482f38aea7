"""Device-side sampler handle over the C ABI (torch tensors in, torch out).

`Sampler` owns one `tgs_handle`.  Inputs are torch tensors already on the
handle's device; the call is asynchronous on torch's current stream (or the
stream given).  torch provides device memory and streams only; all sampling
arithmetic runs in the HIP kernels of libtgs_sampler.so.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib
from ._lib import ROW_PARAMS_DTYPE, TGS_BF16, TGS_F32, TgsDebug, TgsError, TgsHint


def _torch():
    import torch

    return torch


def _ptr(t):
    return None if t is None else C.c_void_p(t.data_ptr())


def make_params(n, temperature=1.0, top_k=0, top_p=1.0, repetition=1.0, presence=0.0,
                frequency=0.0, mask_state=-1, flags=0) -> np.ndarray:
    """Structured numpy array of tgs_row_params (broadcasts scalars/arrays)."""
    p = np.zeros(n, dtype=ROW_PARAMS_DTYPE)
    p["temperature"] = temperature
    p["top_k"] = top_k
    p["top_p"] = top_p
    p["repetition"] = repetition
    p["presence"] = presence
    p["frequency"] = frequency
    p["mask_state"] = mask_state
    p["flags"] = flags
    return p


class BatchHint(int):
    """A batch's max_top_k (an int) carrying its min_top_k too."""

    def __new__(cls, max_top_k: int, min_top_k: int = 0):
        obj = super().__new__(cls, max_top_k)
        obj.min_top_k = int(min_top_k)
        return obj


def batch_hint(params: np.ndarray, vocab: int) -> BatchHint:
    """tgs_batch_hint computed from host params (see the C helper): an int,
    max_top_k, with the batch's min_top_k as an attribute."""
    p = np.ascontiguousarray(params, dtype=ROW_PARAMS_DTYPE)
    h = TgsHint()
    rc = _lib.load().tgs_hint_from_params(p.ctypes.data_as(C.c_void_p), p.size, vocab, C.byref(h))
    if rc != 0:
        raise TgsError(rc, "tgs_hint_from_params")
    return BatchHint(h.max_top_k, h.min_top_k)


def params_to_device(params: np.ndarray, device):
    torch = _torch()
    raw = np.ascontiguousarray(params, dtype=ROW_PARAMS_DTYPE).view(np.uint8)
    return torch.from_numpy(raw.copy()).to(device)


def _debug_struct(debug):
    if not debug:
        return None
    dbg = TgsDebug()
    for name in ("kept_ids", "kept_probs", "counts", "mass", "cut_ids", "post_logits"):
        t = debug.get(name)
        setattr(dbg, name, None if t is None else t.data_ptr())
    kc = debug.get("kept_ids", debug.get("kept_probs"))
    dbg.kept_cap = 0 if kc is None else kc.shape[1]
    return dbg


def _hint_struct(hint):
    if hint is None:
        return None
    hs = TgsHint()
    hs.max_top_k = int(hint)
    hs.min_top_k = int(getattr(hint, "min_top_k", 0))  # 0: unknown
    return hs


def _dtype_code(logits):
    torch = _torch()
    if logits.dtype == torch.float32:
        return TGS_F32
    if logits.dtype == torch.bfloat16:
        return TGS_BF16
    raise TypeError("logits must be float32 or bfloat16")


def _check_sample_inputs(fn, logits, params_dev, u, hist, hist_len, out, V, mask_table=None, mask_vocab=0):
    """The tensors of one sampling call, checked before anything is
    launched: the C ABI takes bare pointers, so a wrong dtype, a short
    buffer or a tensor on another device would be read as garbage there.
    Returns B."""
    torch = _torch()

    def bad(msg):
        raise ValueError(f"{fn}: {msg}")

    if logits.dim() != 2 or logits.stride(1) != 1:
        bad("logits must be [B, V] with unit stride along V")
    _dtype_code(logits)
    B = logits.shape[0]
    if not 1 <= V <= logits.shape[1]:
        bad(f"vocab {V} outside [1, {logits.shape[1]}]")
    nb = ROW_PARAMS_DTYPE.itemsize * B
    need = [("params", params_dev, (torch.uint8,), nb), ("u", u, (torch.float32,), B)]
    if out is not None:
        need.append(("out", out, (torch.int32,), B))
    if hist_len is not None:
        need.append(("hist_len", hist_len, (torch.int32,), B))
    for name, t, dts, n in need:
        if t is None:
            bad(f"{name} is required")
        if t.dtype not in dts or not t.is_contiguous() or t.numel() < n:
            bad(f"{name} must be a contiguous {dts[0]} tensor of at least {n} elements")
    if hist is not None:
        if hist.dtype != torch.int32 or hist.dim() != 2 or not hist.is_contiguous() or hist.shape[0] < B:
            bad("hist must be a contiguous int32 [B, hist_cap] tensor")
    elif hist_len is not None:
        bad("hist_len without hist")
    if mask_table is not None:
        if mask_table.dtype not in (torch.int32, torch.uint32) or mask_table.dim() != 2 \
                or not mask_table.is_contiguous():
            bad("mask_table must be a contiguous int32/uint32 [n_states, words] tensor")
        if mask_vocab < V:
            bad(f"mask_vocab {mask_vocab} is below the vocabulary {V}")
        if mask_table.shape[1] != (mask_vocab + 31) // 32:
            bad(f"mask_table rows hold {mask_table.shape[1]} words; mask_vocab {mask_vocab} needs "
                f"{(mask_vocab + 31) // 32}")
    for name, t in (("params", params_dev), ("u", u), ("out", out), ("hist", hist), ("hist_len", hist_len),
                    ("mask_table", mask_table)):
        if t is not None and t.device != logits.device:
            bad(f"{name} is on {t.device}, logits on {logits.device}")
    if logits.device.type != "cuda":
        bad("tensors must be on a GPU")
    return B


def sample_noalloc(logits, params_dev, u, hist=None, hist_len=None, out=None, vocab=None, mask_table=None,
                   mask_vocab=None, debug=None, stream=None, hint=None):
    """tgs_sample_noalloc: Sampler.sample without a handle (the library's
    static device workspace; no allocation inside the call).  mask_table:
    uint32 device tensor [n_states, ceil(mask_vocab / 32)] or None.  `out`
    must be given by callers that cannot allocate (it is allocated here
    otherwise).  Every tensor is checked (dtype, layout, length, device)
    before the call."""
    torch = _torch()
    if logits.dim() != 2:
        raise ValueError("tgs_sample_noalloc: logits must be [B, V]")
    V = logits.shape[1] if vocab is None else vocab
    mv = (V if mask_vocab is None else mask_vocab) if mask_table is not None else 0
    B = _check_sample_inputs("tgs_sample_noalloc", logits, params_dev, u, hist, hist_len, out, V, mask_table, mv)
    dt = _dtype_code(logits)
    if out is None:
        out = torch.empty(B, dtype=torch.int32, device=logits.device)
    hist_cap = 0 if hist is None else hist.shape[1]
    n_states = 0 if mask_table is None else mask_table.shape[0]
    dbg = _debug_struct(debug)
    hs = _hint_struct(hint)
    st = stream if stream is not None else torch.cuda.current_stream(logits.device).cuda_stream
    L = _lib.load()
    rc = L.tgs_sample_noalloc(
        logits.device.index or 0, _ptr(logits), dt, B, V, logits.stride(0), _ptr(hist), _ptr(hist_len), hist_cap,
        _ptr(params_dev), _ptr(u), _ptr(out), _ptr(mask_table), n_states, mv,
        C.byref(hs) if hs is not None else None, C.byref(dbg) if dbg is not None else None, C.c_void_p(st),
    )
    if rc != 0:
        raise TgsError(rc, f"tgs_sample_noalloc: {L.tgs_last_error(None).decode()}")
    return out


class Sampler:
    """One sampler handle on one GPU.

    max_batch / max_vocab / max_hist bound every call; the workspace is
    allocated once here.
    """

    def __init__(self, device: int = 0, max_batch: int = 1024, max_vocab: int = 152064,
                 max_hist: int = 1024):
        self._L = _lib.load()
        self.device = device
        h = C.c_void_p()
        rc = self._L.tgs_create(C.byref(h), device, max_batch, max_vocab, max_hist)
        if rc != 0:
            raise TgsError(rc, f"tgs_create failed: {_lib.status_string(rc)}")
        self._h = h
        self.max_batch, self.max_vocab, self.max_hist = max_batch, max_vocab, max_hist

    def close(self):
        if getattr(self, "_h", None):
            self._L.tgs_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, rc, what):
        if rc != 0:
            msg = self._L.tgs_last_error(self._h).decode()
            raise TgsError(rc, f"{what}: {msg}")

    # ---------------------------------------------------------------- mask
    def set_mask_table(self, words: np.ndarray, vocab: int):
        words = np.ascontiguousarray(words, dtype=np.uint32)
        n_states = words.shape[0] if words.size else 0
        rc = self._L.tgs_mask_table_set(self._h, words.ctypes.data_as(C.c_void_p), n_states, vocab)
        self._check(rc, "tgs_mask_table_set")
        self._mask_words = (int(vocab) + 31) // 32 if n_states else 0

    def update_mask_rows(self, states: np.ndarray, words: np.ndarray):
        states = np.ascontiguousarray(states, dtype=np.int32)
        words = np.ascontiguousarray(words, dtype=np.uint32)
        rc = self._L.tgs_mask_table_update(self._h, states.ctypes.data_as(C.c_void_p),
                                           words.ctypes.data_as(C.c_void_p), states.size)
        self._check(rc, "tgs_mask_table_update")

    def mask_rows(self, first: int, n: int) -> np.ndarray:
        """Rows [first, first + n) of the mask table as stored on the device
        (uint32 [n, words]); waits for the device's queued work."""
        words = int(getattr(self, "_mask_words", 0))
        out = np.zeros((max(n, 0), words), dtype=np.uint32)
        rc = self._L.tgs_mask_table_get(self._h, int(first), int(n), out.ctypes.data_as(C.c_void_p))
        self._check(rc, "tgs_mask_table_get")
        return out

    # -------------------------------------------------------------- sample
    def sample(self, logits, params_dev, u, hist=None, hist_len=None, out=None, vocab=None,
               debug=None, stream=None, hint=None):
        """logits: [B, >=V] float32 or bfloat16 (row stride = logits.stride(0));
        params_dev: uint8 tensor of B*32 bytes (see params_to_device);
        u: float32 [B]; hist: int32 [B, hist_cap]; hist_len: int32 [B].
        hint: the batch's batch_hint (or a plain int max_top_k) or None (general kernel).
        debug: dict of preallocated tensors (kept_ids, kept_probs, counts,
        mass, cut_ids, post_logits).  Returns the int32 [B] ids tensor."""
        torch = _torch()
        if logits.dim() != 2:
            raise ValueError("tgs_sample: logits must be [B, V]")
        V = logits.shape[1] if vocab is None else vocab
        B = _check_sample_inputs("tgs_sample", logits, params_dev, u, hist, hist_len, out, V)
        dt = _dtype_code(logits)
        if out is None:
            out = torch.empty(B, dtype=torch.int32, device=logits.device)
        hist_cap = 0 if hist is None else hist.shape[1]
        dbg = _debug_struct(debug)
        st = stream if stream is not None else torch.cuda.current_stream(logits.device).cuda_stream
        hs = _hint_struct(hint)
        rc = self._L.tgs_sample(
            self._h, _ptr(logits), dt, B, V, logits.stride(0), _ptr(hist), _ptr(hist_len), hist_cap,
            _ptr(params_dev), _ptr(u), _ptr(out), C.byref(hs) if hs is not None else None,
            C.byref(dbg) if dbg is not None else None, C.c_void_p(st),
        )
        self._check(rc, "tgs_sample")
        return out

    # -------------------------------------------------------------- spec
    def reserve_spec(self, max_batch: int, max_k: int):
        self._check(self._L.tgs_reserve_spec(self._h, max_batch, max_k), "tgs_reserve_spec")

    def spec_verify(self, target, draft, draft_tok, T, u_acc, u_res, n_acc=None, out=None,
                    stream=None):
        """target [B, k+1, V], draft [B, k, V] (float32 or bfloat16, contiguous);
        draft_tok int32 [B, k]; T float32 [B]; u_acc float32 [B, k]; u_res [B].
        Returns (n_acc int32 [B], out int32 [B, k+1])."""
        torch = _torch()
        B, k1, V = target.shape
        k = k1 - 1
        dt = TGS_BF16 if target.dtype == torch.bfloat16 else TGS_F32
        if not target.is_contiguous() or not draft.is_contiguous():
            raise ValueError("target and draft must be contiguous")
        if n_acc is None:
            n_acc = torch.empty(B, dtype=torch.int32, device=target.device)
        if out is None:
            out = torch.empty(B, k + 1, dtype=torch.int32, device=target.device)
        st = stream if stream is not None else torch.cuda.current_stream(target.device).cuda_stream
        rc = self._L.tgs_spec_verify(
            self._h, _ptr(target), _ptr(draft), dt, _ptr(draft_tok), B, k, V, _ptr(T), _ptr(u_acc),
            _ptr(u_res), _ptr(n_acc), _ptr(out), C.c_void_p(st),
        )
        self._check(rc, "tgs_spec_verify")
        return n_acc, out

    def mask_rows_from_dfa(self, byte_class, trans, complete, tok_off, tok_bytes, states, rows, eos=-1,
                           stream=None):
        """Fills rows of the mask table on the device from a byte-level DFA
        (see tinygpt_amd.grammar, Dfa.byte_classes): byte_class uint8 [256],
        trans int32 [n_dfa, n_cls], complete uint8 [n_dfa], tok_off int32
        [V + 1], tok_bytes uint8, states / rows int32 [n] (device tensors).
        The table must exist (set_mask_table)."""
        torch = _torch()
        dev = torch.device("cuda", self.device) if isinstance(self.device, int) else torch.device(self.device)
        want = (("byte_class", byte_class, torch.uint8), ("trans", trans, torch.int32), ("complete", complete, torch.uint8),
                ("tok_off", tok_off, torch.int32), ("tok_bytes", tok_bytes, torch.uint8),
                ("states", states, torch.int32), ("rows", rows, torch.int32))
        for name, t, dt in want:
            if t.dtype != dt or not t.is_contiguous() or t.device != dev:
                raise ValueError(f"mask_rows_from_dfa: {name} must be a contiguous {dt} tensor on {dev}")
        if trans.dim() != 2 or byte_class.numel() != 256 or complete.numel() != trans.shape[0]:
            raise ValueError("mask_rows_from_dfa: byte_class [256], trans [n_dfa, n_cls], complete [n_dfa]")
        if states.numel() != rows.numel() or tok_off.numel() < 1:
            raise ValueError("mask_rows_from_dfa: states and rows of one length, tok_off [V + 1]")
        n_dfa, n_cls = trans.shape
        V = tok_off.numel() - 1
        n = states.numel()
        st = stream if stream is not None else torch.cuda.current_stream(trans.device).cuda_stream
        rc = self._L.tgs_mask_rows_from_dfa(
            self._h, _ptr(byte_class), _ptr(trans), n_cls, _ptr(complete), n_dfa, _ptr(tok_off), _ptr(tok_bytes),
            tok_bytes.numel(), V, int(eos), _ptr(states), _ptr(rows), n, C.c_void_p(st),
        )
        self._check(rc, "tgs_mask_rows_from_dfa")

    def token_logprobs(self, logits, tokens, out=None, lse=None, stream=None):
        """log(softmax(logits))[b, tokens[b]] for each row b of logits [B, V]
        (float32 or bfloat16, rows may be strided); tokens int32 [B].
        Returns out float32 [B] (and fills lse [B] with each row's
        logsumexp when given)."""
        torch = _torch()
        B, V = logits.shape
        dt = TGS_BF16 if logits.dtype == torch.bfloat16 else TGS_F32
        if logits.stride(1) != 1:
            raise ValueError("logits rows must be contiguous")
        if out is None:
            out = torch.empty(B, dtype=torch.float32, device=logits.device)
        st = stream if stream is not None else torch.cuda.current_stream(logits.device).cuda_stream
        rc = self._L.tgs_token_logprobs(
            self._h, _ptr(logits), dt, B, V, logits.stride(0), _ptr(tokens), _ptr(out), _ptr(lse), C.c_void_p(st),
        )
        self._check(rc, "tgs_token_logprobs")
        return out
