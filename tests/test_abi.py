"""The C ABI library: builds, loads, exports every declared entry point, and
rejects bad arguments on the host (no GPU work).  CPU only."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tgs_sampler.h")


def declared_functions():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(tgs_[a-z_0-9]+)\s*\(", src)))


@pytest.fixture(scope="module")
def lib():
    import tinygpt_amd._lib as L

    if not os.path.exists(L.LIB_PATH):
        from tinygpt_amd import build

        build.build()
    return L.load()


def test_every_declared_symbol_is_exported(lib):
    import tinygpt_amd._lib as L

    names = declared_functions()
    assert names == sorted(L.EXPORTS)
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version_and_status_strings(lib):
    assert lib.tgs_abi_version() == 4
    assert lib.tgs_status_string(0) == b"ok"
    assert b"invalid" in lib.tgs_status_string(-1)
    assert lib.tgs_status_string(12345) == b"unknown status"


def test_create_rejects_bad_arguments(lib):
    h = C.c_void_p()
    assert lib.tgs_create(None, 0, 1, 1, 0) == -1
    assert lib.tgs_create(C.byref(h), 0, 0, 100, 0) == -1
    assert lib.tgs_create(C.byref(h), 0, 4, 300000, 0) == -1  # vocab beyond 262144
    assert lib.tgs_create(C.byref(h), 0, 4, 100, 5000) == -1  # history beyond 4096
    assert h.value is None


def test_null_handle_calls_fail_cleanly(lib):
    assert lib.tgs_sample(None, None, 0, 1, 1, 1, None, None, 0, None, None, None, None, None, None) == -1
    assert lib.tgs_spec_verify(None, None, None, 0, None, 1, 1, 1, None, None, None, None, None, None) == -1
    assert lib.tgs_mask_table_set(None, None, 0, 1) == -1
    assert lib.tgs_mask_table_get(None, 0, 1, None) == -1
    assert lib.tgs_token_logprobs(None, None, 0, 1, 1, 1, None, None, None, None) == -1
    assert lib.tgs_mask_rows_from_dfa(None, None, None, 1, None, 1, None, None, 0, 1, -1, None, None, 1, None) == -1
    assert lib.tgs_last_error(None) == b"null handle"
    lib.tgs_destroy(None)


def test_hint_from_params(lib):
    import numpy as np

    import tinygpt_amd as tg

    V = 1000
    p = tg.make_params(4, temperature=[0.0, 0.7, 1.0, 0.5], top_k=[0, 50, 7, 3])
    h = tg.batch_hint(p, V)
    assert h == 50 and h.min_top_k == 3
    p["top_k"][3] = 0  # top-k disabled on a sampling row: the full row
    h = tg.batch_hint(p, V)
    assert h == V and h.min_top_k == 7
    p["top_k"][3] = V + 3
    assert tg.batch_hint(p, V) == V
    p["top_k"][1:] = [0, V, -1]  # no sampling row with a usable top-k
    h = tg.batch_hint(p, V)
    assert h == V and h.min_top_k == V
    p = tg.make_params(3, temperature=0.0, top_k=0)
    h = tg.batch_hint(p, V)
    assert h == 0 and h.min_top_k == V  # all greedy
    p = tg.make_params(2, temperature=[np.nan, 0.9], top_k=[5, 9], flags=[0, 1])
    assert tg.batch_hint(p, V) == 0  # NaN rows are invalid, flagged rows greedy


def test_library_has_no_cpu_sampling_path():
    """The product sources carry no host implementation of the sampler:
    every sampling computation is a __global__ kernel."""
    api = open(os.path.join(ROOT, "tinygpt_amd", "csrc", "tgs_api.hip")).read()
    for needle in ("tg_expf", "tg_q40", "qsort", "nth_element", "oracle"):
        assert needle not in api


def test_noalloc_rejects_sizes_beyond_its_workspace(lib):
    """tgs_sample_noalloc checks its fixed limits before any device work."""
    import ctypes as C

    p = C.c_void_p(16)  # never dereferenced: the call returns before any launch
    args = lambda B, V, hc: (0, p, 0, B, V, V, p, None, hc, p, p, p, None, 0, 0, None, None, None)
    assert lib.tgs_sample_noalloc(*args(257, 1000, 0)) == -5
    assert b"at most 256 rows" in lib.tgs_last_error(None)
    assert lib.tgs_sample_noalloc(*args(4, 262145, 0)) == -5
    assert lib.tgs_sample_noalloc(*args(4, 1000, 1025)) == -5
    assert lib.tgs_sample_noalloc(0, p, 0, 4, 1000, 1000, None, None, 0, p, p, p, None, 3, 1000, None, None,
                                  None) == -1  # a table needs its pointer
    assert lib.tgs_sample_noalloc(0, p, 5, 4, 1000, 1000, None, None, 0, p, p, p, None, 0, 0, None, None,
                                  None) == -1  # dtype
    # an empty batch only prepares the device (the set-up a captured call
    # cannot do): TGS_OK on a GPU, TGS_EHIP where there is none
    assert lib.tgs_sample_noalloc(*args(0, 1000, 0)) in (0, -3)
