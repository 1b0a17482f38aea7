"""GPU: tgs_sample_noalloc (static device workspace, no allocation in the
call) against tgs_sample (the handle's workspace) on the same inputs, through
the C ABI.  Every output is compared bit for bit: ids, kept lists and
probabilities, counts, exact masses, cut ids and post-penalty logits.  Calls
come in pairs, the second on a smaller batch, so the second reads workspace
the first left behind."""
import numpy as np
import pytest

import gpu_harness as H

pytestmark = pytest.mark.gpu

FIELDS = ("ids", "kept_ids", "kept_probs", "counts", "mass", "cut_ids", "post_logits")


def _run_noalloc(logits, params, u, hist=None, hist_len=None, mask_table=None, kept_cap=64, post=True,
                 hint=None):
    import torch

    import tinygpt_amd as tg

    dev = "cuda:0"
    B, V = logits.shape
    if isinstance(hint, str):
        hint = tg.batch_hint(params, V)
    dbg = dict(
        kept_ids=torch.full((B, kept_cap), -7, dtype=torch.int32, device=dev),
        kept_probs=torch.full((B, kept_cap), -7.0, dtype=torch.float32, device=dev),
        counts=torch.full((B, 2), -7, dtype=torch.int32, device=dev),
        mass=torch.zeros((B, 2), dtype=torch.int64, device=dev),
        cut_ids=torch.full((B,), -7, dtype=torch.int32, device=dev),
        post_logits=torch.full((B, V), float("nan"), dtype=torch.float32, device=dev) if post else None,
    )
    out = torch.full((B,), -9, dtype=torch.int32, device=dev)
    mt = None if mask_table is None else H.to_dev(np.ascontiguousarray(mask_table, np.uint32))
    tg.sample_noalloc(H.to_dev(logits), tg.params_to_device(params, dev), H.to_dev(np.asarray(u, np.float32)),
                      hist=H.to_dev(hist), hist_len=H.to_dev(hist_len), out=out, mask_table=mt, debug=dbg,
                      hint=hint)
    torch.cuda.synchronize()
    r = {k: (v.cpu().numpy() if v is not None else None) for k, v in dbg.items()}
    r["ids"] = out.cpu().numpy()
    r["mass"] = r["mass"].view(np.uint64)
    return r


def _same(sampler, oracle, name, logits, params, u, hist=None, hist_len=None, mask_table=None, kept_cap=64,
          post=True, hint=None):
    H.log(f"case noalloc {name}: B={logits.shape[0]} V={logits.shape[1]} hint={hint}")
    n = _run_noalloc(logits, params, u, hist, hist_len, mask_table, kept_cap=kept_cap, post=post, hint=hint)
    g = H.run_gpu(sampler, logits, params, u, hist, hist_len, mask_table, kept_cap=kept_cap, post=post, hint=hint)
    for f in FIELDS:
        if g.get(f) is None:
            continue
        np.testing.assert_array_equal(n[f], g[f], err_msg=f"{name}: {f} differs from tgs_sample")
    ref = oracle.sample_batch(logits, params, u, hist=hist, hist_len=hist_len, mask_table=mask_table)["ids"]
    np.testing.assert_array_equal(n["ids"], ref, err_msg=f"{name}: ids differ from the oracle")
    H.log(f"case noalloc {name}: ok")


def test_noalloc_k64_path_then_smaller(sampler, oracle):
    from tinygpt_amd import workloads as W

    c = W.config2()
    _same(sampler, oracle, "c2", c["logits"], c["params"], c["u"], c["hist"], c["hist_len"], hint="auto")
    c = W.config2(B=16, V=50000, H=100, seed_offset=3)
    _same(sampler, oracle, "c2-small", c["logits"], c["params"], c["u"], c["hist"], c["hist_len"], hint="auto")


def test_noalloc_general_path_then_smaller(sampler, oracle):
    from test_gpu_sampler import _random_batch

    x, params, u, hist, hist_len = _random_batch(np.random.default_rng(4242), 48, 5000, oracle)
    _same(sampler, oracle, "general", x, params, u, hist, hist_len, kept_cap=1025)
    x, params, u, hist, hist_len = _random_batch(np.random.default_rng(4243), 8, 300, oracle)
    params["top_k"] = np.where(params["top_k"] > 0, np.minimum(params["top_k"], 64), 5)
    _same(sampler, oracle, "general-small", x, params, u, hist, hist_len, kept_cap=1025)


def test_noalloc_mask_table_and_topk_path(sampler, oracle):
    from test_gpu_sampler import _random_batch
    from tinygpt_amd import workloads as W

    g = np.random.default_rng(4244)
    V = 40000
    x, params, u, hist, hist_len = _random_batch(g, 32, V, oracle)
    table = g.integers(0, 1 << 32, size=(4, (V + 31) // 32), dtype=np.uint64).astype(np.uint32)
    table[2] = 0
    params["mask_state"] = g.integers(-1, 4, size=32)
    _same(sampler, oracle, "masked", x, params, u, hist, hist_len, mask_table=table, kept_cap=1025)
    c = W.config4(B=24)
    _same(sampler, oracle, "c4-24", c["logits"], c["params"], c["u"], c["hist"], c["hist_len"], kept_cap=1024,
          post=False, hint="auto")


def test_noalloc_under_graph_capture(sampler, oracle):
    """tgs_sample_noalloc captured in a HIP graph: one call with B = 0 sets
    the device up outside any capture, then a graph holds one call on fixed
    tensors.  Four replays, each after new inputs are copied into those
    tensors, with eager tgs_sample calls and synchronisations between them;
    every replay's ids match tgs_sample's on the same inputs bit for bit and
    the oracle's."""
    import torch

    import tinygpt_amd as tg
    from tinygpt_amd import workloads as W

    dev = "cuda:0"
    sets = [W.config2(B=32, V=50000, H=64, seed_offset=20 + i) for i in range(4)]
    c0 = sets[0]
    B, V = c0["logits"].shape
    x, u = H.to_dev(c0["logits"]), H.to_dev(c0["u"])
    hist, hl = H.to_dev(c0["hist"]), H.to_dev(c0["hist_len"])
    pd = tg.params_to_device(c0["params"], dev)
    out = torch.full((B,), -9, dtype=torch.int32, device=dev)
    hint = tg.batch_hint(c0["params"], V)
    for c in sets[1:]:
        assert tg.batch_hint(c["params"], V) == hint
    stream = torch.cuda.Stream(device=dev)
    H.log("case noalloc capture: set-up call with B = 0")
    tg.sample_noalloc(x[:0], pd, u, out=out, stream=stream.cuda_stream)
    torch.cuda.synchronize()
    H.log(f"case noalloc capture: capturing B={B} V={V}")
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream, capture_error_mode="thread_local"):
        tg.sample_noalloc(x, pd, u, hist=hist, hist_len=hl, out=out, hint=hint)
    torch.cuda.synchronize()
    for i, c in enumerate(sets):
        H.log(f"case noalloc capture: replay {i}")
        x.copy_(H.to_dev(c["logits"]))
        u.copy_(H.to_dev(c["u"]))
        hist.copy_(H.to_dev(c["hist"]))
        hl.copy_(H.to_dev(c["hist_len"]))
        pd.copy_(tg.params_to_device(c["params"], dev))
        out.fill_(-9)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        eager = H.run_gpu(sampler, c["logits"], c["params"], c["u"], c["hist"], c["hist_len"], hint="auto")
        np.testing.assert_array_equal(got, eager["ids"], err_msg=f"replay {i}: ids differ from tgs_sample")
        ref = oracle.sample_batch(c["logits"], c["params"], c["u"], hist=c["hist"], hist_len=c["hist_len"])["ids"]
        np.testing.assert_array_equal(got, ref, err_msg=f"replay {i}: ids differ from the oracle")
    H.log("case noalloc capture: ok")
