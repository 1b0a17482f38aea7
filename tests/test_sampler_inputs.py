"""The Python entry points check every tensor before a launch (CPU only: no
GPU and no library call is needed to reach these errors)."""
import numpy as np
import pytest
import torch

import tinygpt_amd as tg


def _inputs(B=4, V=1000, H=8):
    logits = torch.zeros(B, V, dtype=torch.float32)
    pd = torch.from_numpy(np.ascontiguousarray(tg.make_params(B, top_k=5)).view(np.uint8).copy())
    u = torch.zeros(B, dtype=torch.float32)
    hist = torch.zeros(B, H, dtype=torch.int32)
    hl = torch.zeros(B, dtype=torch.int32)
    out = torch.empty(B, dtype=torch.int32)
    return logits, pd, u, hist, hl, out


def _raises(match, **kw):
    logits, pd, u, hist, hl, out = _inputs()
    args = dict(logits=logits, params_dev=pd, u=u, hist=hist, hist_len=hl, out=out)
    args.update(kw)
    with pytest.raises(ValueError, match=match):
        tg.sample_noalloc(**args)


def test_mask_table_width_is_checked_before_launch():
    V = 1000
    words = (V + 31) // 32
    _raises("needs 32", mask_table=torch.zeros(3, words - 1, dtype=torch.int32))
    _raises("needs 32", mask_table=torch.zeros(3, words + 1, dtype=torch.int32))
    _raises("needs 63", mask_table=torch.zeros(3, words, dtype=torch.int32), mask_vocab=2000)
    _raises("below the vocabulary", mask_table=torch.zeros(3, words, dtype=torch.int32), mask_vocab=999)
    _raises("int32/uint32", mask_table=torch.zeros(3, words, dtype=torch.int64))
    _raises("int32/uint32", mask_table=torch.zeros(words, 3, dtype=torch.int32).t())
    # a table of the right width gets as far as the device check
    _raises("on a GPU", mask_table=torch.zeros(3, words, dtype=torch.int32))
    _raises("on a GPU", mask_table=torch.zeros(3, words, dtype=torch.uint32))


def test_dtypes_lengths_and_devices_are_checked():
    logits, pd, u, hist, hl, out = _inputs()
    _raises("u must be", u=u.double())
    _raises("u must be", u=u[:3])
    _raises("params must be", params_dev=pd[:-1])
    _raises("params must be", params_dev=pd.view(torch.int32))
    _raises("hist_len must be", hist_len=hl.long())
    _raises("out must be", out=out[:2])
    _raises("hist must be", hist=hist.t())
    _raises("hist must be", hist=hist[:2])
    _raises("hist_len without hist", hist=None)
    _raises("vocab", vocab=1001)
    _raises("logits must be", logits=logits.t())
    _raises("u is on meta", u=torch.empty(4, dtype=torch.float32, device="meta"))
    _raises("mask_table is on meta", mask_table=torch.empty(3, 32, dtype=torch.int32, device="meta"))
    with pytest.raises(TypeError):
        tg.sample_noalloc(logits.half(), pd, u)
    _raises("on a GPU")
