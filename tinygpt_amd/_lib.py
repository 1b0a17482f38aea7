"""ctypes binding of the C ABI in include/tgs_sampler.h (libtgs_sampler.so).

The shared library is built in-tree by tinygpt_amd.build.  torch is
imported before the library is loaded so that both resolve the same HIP
runtime (libamdhip64.so.7, matched by SONAME).  There is no fallback: if the
library is missing, loading raises.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtgs_sampler.so")

TGS_OK = 0
TGS_EINVAL = -1
TGS_ENOMEM = -2
TGS_EHIP = -3
TGS_EALLMASKED = -4
TGS_ETOOBIG = -5

TGS_F32 = 0
TGS_BF16 = 1
TGS_FLAG_GREEDY = 1

# Exported entry points of include/tgs_sampler.h.
EXPORTS = (
    "tgs_abi_version",
    "tgs_status_string",
    "tgs_hint_from_params",
    "tgs_create",
    "tgs_destroy",
    "tgs_last_error",
    "tgs_mask_table_set",
    "tgs_mask_table_update",
    "tgs_mask_table_get",
    "tgs_sample",
    "tgs_sample_noalloc",
    "tgs_reserve_spec",
    "tgs_spec_verify",
    "tgs_token_logprobs",
    "tgs_mask_rows_from_dfa",
)

ROW_PARAMS_DTYPE = np.dtype(
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
assert ROW_PARAMS_DTYPE.itemsize == 32


class TgsDebug(C.Structure):
    _fields_ = [
        ("kept_ids", C.c_void_p),
        ("kept_probs", C.c_void_p),
        ("kept_cap", C.c_int32),
        ("counts", C.c_void_p),
        ("mass", C.c_void_p),
        ("cut_ids", C.c_void_p),
        ("post_logits", C.c_void_p),
    ]


class TgsHint(C.Structure):
    _fields_ = [("max_top_k", C.c_int32), ("min_top_k", C.c_int32)]


class TgsError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{msg} (status {status})")
        self.status = status


_lib = None


def load() -> C.CDLL:
    """Load libtgs_sampler.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    try:  # share torch's HIP runtime when torch is present
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    L = C.CDLL(LIB_PATH)
    P, I = C.c_void_p, C.c_int
    L.tgs_abi_version.restype = I
    L.tgs_abi_version.argtypes = []
    L.tgs_status_string.restype = C.c_char_p
    L.tgs_status_string.argtypes = [I]
    L.tgs_create.restype = I
    L.tgs_create.argtypes = [C.POINTER(P), I, I, I, I]
    L.tgs_destroy.restype = None
    L.tgs_destroy.argtypes = [P]
    L.tgs_last_error.restype = C.c_char_p
    L.tgs_last_error.argtypes = [P]
    L.tgs_mask_table_set.restype = I
    L.tgs_mask_table_set.argtypes = [P, P, I, I]
    L.tgs_mask_table_update.restype = I
    L.tgs_mask_table_update.argtypes = [P, P, P, I]
    L.tgs_mask_table_get.restype = I
    L.tgs_mask_table_get.argtypes = [P, I, I, P]
    L.tgs_sample.restype = I
    L.tgs_hint_from_params.restype = I
    L.tgs_hint_from_params.argtypes = [P, I, I, C.POINTER(TgsHint)]
    L.tgs_sample.argtypes = [P, P, I, I, I, C.c_int64, P, P, I, P, P, P, C.POINTER(TgsHint),
                             C.POINTER(TgsDebug), P]
    L.tgs_sample_noalloc.restype = I
    L.tgs_sample_noalloc.argtypes = [I, P, I, I, I, C.c_int64, P, P, I, P, P, P, P, I, I, C.POINTER(TgsHint),
                                     C.POINTER(TgsDebug), P]
    L.tgs_reserve_spec.restype = I
    L.tgs_reserve_spec.argtypes = [P, I, I]
    L.tgs_spec_verify.restype = I
    L.tgs_spec_verify.argtypes = [P, P, P, I, P, I, I, I, P, P, P, P, P, P]
    L.tgs_token_logprobs.restype = I
    L.tgs_token_logprobs.argtypes = [P, P, I, I, I, C.c_int64, P, P, P, P]
    L.tgs_mask_rows_from_dfa.restype = I
    L.tgs_mask_rows_from_dfa.argtypes = [P, P, P, I, P, I, P, P, C.c_int64, I, I, P, P, I, P]
    _lib = L
    return L


def status_string(status: int) -> str:
    return load().tgs_status_string(status).decode()
