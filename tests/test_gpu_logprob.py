"""GPU parity of teacher-forced token log-probabilities
(tgs_token_logprobs, Serve.swift:983-993) against the float64 oracle.

Tolerance: |gpu - oracle| <= 1e-4 + 1e-6 |oracle| for the log-probability
and for the row's logsumexp (fp32 exp2 and fp32 partial sums over up to
128256 ids); NaN exactly where the oracle gives NaN."""
import numpy as np
import pytest

import gpu_harness as H

pytestmark = pytest.mark.gpu

ATOL, RTOL = 1e-4, 1e-6


def _close(name, got, ref):
    nan = np.isnan(ref)
    np.testing.assert_array_equal(np.isnan(got), nan, err_msg=f"{name}: NaN positions")
    err = np.abs(got[~nan].astype(np.float64) - ref[~nan])
    lim = ATOL + RTOL * np.abs(ref[~nan])
    assert np.all(err <= lim), f"{name}: max error {err.max():.3g}"


def _run(sampler, oracle, name, x, tok, V=None):
    import torch

    H.log(f"case {name}: B={x.shape[0]} V={V or x.shape[1]} stride={x.shape[1]} dtype={x.dtype}")
    if x.dtype == np.uint16:
        xd = torch.from_numpy(x.view(np.int16)).to("cuda:0").view(torch.bfloat16)
    else:
        xd = torch.from_numpy(x).to("cuda:0")
    if V is not None:
        xd = xd[:, :V]
    td = torch.from_numpy(np.asarray(tok, np.int32)).to("cuda:0")
    lse = torch.empty(x.shape[0], dtype=torch.float32, device="cuda:0")
    lp = sampler.token_logprobs(xd, td, lse=lse)
    torch.cuda.synchronize()
    r_lp, r_lse = oracle.token_logprobs(x, tok, V=V)
    _close(name + " logprob", lp.cpu().numpy(), r_lp)
    _close(name + " lse", lse.cpu().numpy(), r_lse)
    H.log(f"case {name}: ok")


@pytest.mark.parametrize("bf16", [False, True])
def test_scoring_shape_one_workgroup_per_row(sampler, oracle, bf16):
    g = np.random.default_rng(11)
    B, V = 1100, 4096
    x = g.normal(0.0, 3.0, (B, V)).astype(np.float32)
    if bf16:
        from tinygpt_amd import workloads as W

        x = W.f32_to_bf16_bits(x)
    _run(sampler, oracle, f"B{B}", x, g.integers(0, V, B))


@pytest.mark.parametrize("bf16", [False, True])
def test_few_long_rows_split_into_chunks(sampler, oracle, bf16):
    g = np.random.default_rng(12)
    B, V = 4, 128256
    x = g.normal(0.0, 3.0, (B, V)).astype(np.float32)
    x[1] += 30.0
    x[2, ::7] = -np.inf
    if bf16:
        from tinygpt_amd import workloads as W

        x = W.f32_to_bf16_bits(x)
    _run(sampler, oracle, "split", x, [0, V - 1, 5, 777])


def test_strided_unaligned_rows_and_special_values(sampler, oracle):
    g = np.random.default_rng(13)
    B, V, stride = 9, 5003, 5011  # odd stride: rows not 16-byte aligned
    x = g.normal(0.0, 2.0, (B, stride)).astype(np.float32)
    x[1, :V] = -np.inf       # only -inf: NaN
    x[2, 17] = np.nan        # NaN logit: NaN
    x[3, 40] = np.inf        # +inf logit: NaN
    x[4, :] = 0.0            # uniform: -log V
    x[5, 3:V:2] = -np.inf
    tok = [1, 2, 3, 4, 5, V, -1, 0, V - 1]  # rows 5 and 6: tokens outside [0, V)
    _run(sampler, oracle, "specials", x, tok, V=V)
