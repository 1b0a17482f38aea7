"""Runs the device sampler and the CPU oracle on the same inputs and compares
every output (GPU tests only)."""
from __future__ import annotations

import sys

import numpy as np


def log(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def to_dev(a, dev="cuda:0"):
    import torch

    if a is None:
        return None
    if a.dtype == np.uint16:
        return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def table_bits(sampler, rows, V):
    """Allowed ids of mask-table rows read straight from the device table
    (tgs_mask_table_get): bool [len(rows), V].  Bits past V must be clear."""
    rows = np.asarray(rows, dtype=np.int64)
    lo, hi = int(rows.min()), int(rows.max()) + 1
    tab = sampler.mask_rows(lo, hi - lo)[rows - lo]
    bits = np.unpackbits(np.ascontiguousarray(tab).view(np.uint8), axis=1, bitorder="little")
    assert not bits[:, V:].any(), "bits past the vocabulary are set"
    return bits[:, :V].astype(bool)


def run_gpu(sampler, logits, params, u, hist=None, hist_len=None, mask_table=None, V=None,
            kept_cap=64, post=True, hint=None):
    """hint: None (general kernel), "auto" (computed from params) or an int."""
    import torch

    import tinygpt_amd as tg

    dev = "cuda:0"
    B = logits.shape[0]
    V = logits.shape[1] if V is None else V
    if mask_table is not None:
        sampler.set_mask_table(mask_table, V)
    else:
        sampler.set_mask_table(np.zeros((0, 1), np.uint32), 1)
    if isinstance(hint, str):
        hint = tg.batch_hint(params, V)
    lg = to_dev(logits)
    dbg = dict(
        kept_ids=torch.full((B, kept_cap), -7, dtype=torch.int32, device=dev),
        kept_probs=torch.full((B, kept_cap), -7.0, dtype=torch.float32, device=dev),
        counts=torch.full((B, 2), -7, dtype=torch.int32, device=dev),
        mass=torch.zeros((B, 2), dtype=torch.int64, device=dev),
        cut_ids=torch.full((B,), -7, dtype=torch.int32, device=dev),
        post_logits=torch.full((B, V), float("nan"), dtype=torch.float32, device=dev) if post else None,
    )
    out = sampler.sample(lg, tg.params_to_device(params, dev), to_dev(np.asarray(u, np.float32)),
                         hist=to_dev(hist), hist_len=to_dev(hist_len), vocab=V, debug=dbg, hint=hint)
    torch.cuda.synchronize()
    r = {k: (v.cpu().numpy() if v is not None else None) for k, v in dbg.items()}
    r["ids"] = out.cpu().numpy()
    r["mass"] = r["mass"].view(np.uint64)
    return r


def run_oracle(oracle, logits, params, u, hist=None, hist_len=None, mask_table=None, V=None,
               kept_cap=64, post=True, nthreads=8):
    if V is not None and V != logits.shape[1]:
        raise ValueError("oracle harness expects V == row length")
    return oracle.sample_batch(logits, params, u, hist=hist, hist_len=hist_len,
                               mask_table=mask_table, kept_cap=kept_cap, want_post=post,
                               nthreads=nthreads)


def row_modes(params, V):
    """0 greedy, 1 candidate path (kept list written), 2 full path, -1 invalid-ish."""
    T = params["temperature"]
    greedy = ((params["flags"] & 1) != 0) | (T <= 0)
    k = params["top_k"]
    cand = (~greedy) & (k >= 1) & (k <= 1024) & (k < V)
    return np.where(greedy, 0, np.where(cand, 1, 2))


def compare(gpu, orc, params, V, check_post=True, what=""):
    """Asserts bit-exact agreement; returns a small report dict."""
    ids_o = orc["ids"]
    ids_g = gpu["ids"]
    bad = np.nonzero(ids_o != ids_g)[0]
    assert bad.size == 0, f"{what}: id mismatch rows {bad[:10]} gpu {ids_g[bad[:10]]} oracle {ids_o[bad[:10]]}"
    res = orc["res"]
    valid = ids_o != -2
    np.testing.assert_array_equal(gpu["counts"][valid, 0], res["n_topk"][valid], err_msg=f"{what}: n_topk")
    np.testing.assert_array_equal(gpu["counts"][valid, 1], res["n_topp"][valid], err_msg=f"{what}: n_topp")
    np.testing.assert_array_equal(gpu["mass"][valid, 0], res["mass_k"][valid], err_msg=f"{what}: mass S")
    np.testing.assert_array_equal(gpu["mass"][valid, 1], res["mass_p"][valid], err_msg=f"{what}: mass S'")
    np.testing.assert_array_equal(gpu["cut_ids"][valid], res["cut_id"][valid], err_msg=f"{what}: cut id")
    modes = row_modes(params, V)
    kc = gpu["kept_ids"].shape[1]
    for b in np.nonzero(valid & (modes != 2))[0]:
        n = min(kc, int(res["n_topk"][b]))
        np.testing.assert_array_equal(gpu["kept_ids"][b, :n], orc["kept_ids"][b, :n], err_msg=f"{what}: kept ids row {b}")
        m = min(kc, int(res["n_topp"][b]))
        np.testing.assert_array_equal(gpu["kept_probs"][b, :m], orc["kept_probs"][b, :m], err_msg=f"{what}: probs row {b}")
    if check_post and gpu.get("post_logits") is not None and orc.get("post") is not None:
        rows = np.nonzero(valid)[0]
        np.testing.assert_array_equal(gpu["post_logits"][rows], orc["post"][rows], err_msg=f"{what}: post logits")
    return dict(rows=int(len(ids_o)), draw_boundary=int(res["draw_boundary"].sum()),
                topp_boundary=int(res["topp_boundary"].sum()), ref_tie_extra=int((res["ref_tie_extra"] > 0).sum()))
