"""The sampler and the log-probability kernel read an LM head's output where
it lies: the last position of a [B, T, V] tensor (rows T*V elements apart),
in bf16 (upcast inside the kernels), with no slice copy and no upcast pass.
Bit-exact ids against the oracle on the same rows copied out."""
import numpy as np
import pytest

import gpu_harness as H

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_sample_last_position_of_lm_head_output(sampler, oracle, dtype):
    import torch

    import tinygpt_amd as tg
    from tinygpt_amd import workloads as W

    B, T, V = 16, 5, 32000
    g = np.random.default_rng(81)
    x = g.normal(0.0, 3.0, (B, T, V)).astype(np.float32)
    xh = W.f32_to_bf16_bits(x) if dtype == "bf16" else x
    full = H.to_dev(xh)  # the producer's [B, T, V] output
    last = full[:, -1, :]  # a view: row stride T*V, no copy
    assert last.stride(0) == T * V and last.data_ptr() == full.data_ptr() + (T - 1) * V * full.element_size()
    params = oracle.make_params(B, temperature=0.8, top_k=[1, 40, 0, 64] * 4, top_p=0.9)
    params["temperature"][::5] = 0.0
    u = g.random(B).astype(np.float32)
    H.log(f"case producer {dtype}: B={B} T={T} V={V}")
    for hint in (None, tg.batch_hint(params, V)):
        ids = sampler.sample(last, tg.params_to_device(params, "cuda:0"), H.to_dev(u), vocab=V, hint=hint)
        torch.cuda.synchronize()
        o = oracle.sample_batch(np.ascontiguousarray(xh[:, -1, :]), params, u)
        np.testing.assert_array_equal(ids.cpu().numpy(), o["ids"])
    tok = torch.from_numpy(g.integers(0, V, B).astype(np.int32)).to("cuda:0")
    lp = sampler.token_logprobs(last, tok)
    torch.cuda.synchronize()
    ref, _ = oracle.token_logprobs(np.ascontiguousarray(xh[:, -1, :]), tok.cpu().numpy())
    assert np.all(np.abs(lp.cpu().numpy() - ref) <= 1e-4 + 1e-6 * np.abs(ref))
    H.log(f"case producer {dtype}: ok")
