"""GPU parity of speculative verification against the CPU oracle (bit-exact
accept counts and emitted tokens)."""
import numpy as np
import pytest

import gpu_harness as H

pytestmark = pytest.mark.gpu


def _run(sampler, c):
    import torch

    d = "cuda:0"
    tgt = H.to_dev(c["target"])
    dft = H.to_dev(c["draft"])
    n_acc, out = sampler.spec_verify(tgt, dft, H.to_dev(c["dtok"]), H.to_dev(c["T"]),
                                     H.to_dev(c["u_acc"]), H.to_dev(c["u_res"]))
    torch.cuda.synchronize()
    return n_acc.cpu().numpy(), out.cpu().numpy()


def _check(sampler, oracle, name, c):
    H.log(f"case {name}: B={c['target'].shape[0]} k={c['target'].shape[1] - 1} V={c['target'].shape[2]}")
    n_g, out_g = _run(sampler, c)
    o = oracle.spec_verify_batch(c["target"], c["draft"], c["dtok"], c["T"], c["u_acc"], c["u_res"], nthreads=16)
    np.testing.assert_array_equal(n_g, o["n_acc"], err_msg=f"{name}: n_acc")
    np.testing.assert_array_equal(out_g, o["out"], err_msg=f"{name}: out")
    H.log(f"case {name}: ok accepted={n_g.tolist()[:8]}")
    return o


def test_c5_spec_verify(sampler, oracle):
    from tinygpt_amd import workloads as W

    _check(sampler, oracle, "c5", W.config5())


@pytest.mark.parametrize("T", [0.0, 0.5, 1.0, 2.0])
def test_spec_small(sampler, oracle, T):
    from tinygpt_amd import workloads as W

    c = W.config5(B=24, k=4, V=3000, seed_offset=10 + int(T * 10), T=1.0)
    c["T"][:] = T
    # force some early rejections: make a few draft tokens unlikely
    c["dtok"][::3, 0] = np.argmin(c["target"][::3, 0], axis=-1)
    c["T"][5] = 0.0  # mixed greedy row
    _check(sampler, oracle, f"spec T={T}", c)


def test_spec_bf16(sampler, oracle):
    from tinygpt_amd import workloads as W

    c = W.config5(B=8, k=3, V=5000, seed_offset=3)
    c["target"] = W.f32_to_bf16_bits(c["target"])
    c["draft"] = W.f32_to_bf16_bits(c["draft"])
    _check(sampler, oracle, "spec bf16", c)


def test_spec_invalid(sampler, oracle):
    from tinygpt_amd import workloads as W

    c = W.config5(B=4, k=2, V=64, seed_offset=4)
    c["dtok"][0, 1] = 64
    c["T"][1] = np.nan
    c["u_acc"][2, 0] = 1.0
    _check(sampler, oracle, "spec invalid", c)


def test_spec_zero_residual_falls_back_to_target(sampler, oracle):
    # draft == target and the first draft token has probability 0 in both:
    # rejected (ratio 0), residual 0 everywhere -> draw from the target row
    from tinygpt_amd import workloads as W

    c = W.config5(B=5, k=3, V=4100, seed_offset=13)
    c["draft"] = c["target"][:, :3].copy()
    c["target"][np.arange(5), 0, c["dtok"][:, 0]] = -np.inf
    c["draft"][np.arange(5), 0, c["dtok"][:, 0]] = -np.inf
    o = _check(sampler, oracle, "spec zero residual", c)
    assert (o["n_acc"] == 0).all() and (o["info"]["resampled"] == 2).all()


def test_spec_k64_all_accepted(sampler, oracle):
    # the longest draft (k = 64) with every token accepted (u_acc = 0): the
    # bonus draw from target row k, and all 65 outputs written
    from tinygpt_amd import workloads as W

    c = W.config5(B=2, k=64, V=2048, seed_offset=14)
    c["u_acc"][:] = 0.0
    o = _check(sampler, oracle, "spec k64", c)
    assert (o["n_acc"] == 64).all()


def special_blocks_case(T):
    """Blocks whose maximum is -inf (every id -inf or NaN) or +inf between
    finite ones, so that a block's exact mass that waits to be reduced with
    the wave's next finite block crosses blocks that store theirs at once; a
    greedy and a NaN-temperature sequence among stochastic ones.  T 1.0 and
    0.5 take the power-of-two form, 0.7 the exact divide."""
    from tinygpt_amd import workloads as W

    c = W.config5(B=6, k=3, V=4096, seed_offset=14, T=1.0)  # four blocks of 1024 ids per row
    c["T"][:] = T
    c["T"][2] = 0.0
    c["T"][4] = np.nan
    tg, dr = c["target"], c["draft"]
    tg[0, 1, 1024:2048] = -np.inf
    dr[0, 0, 2048:3072] = np.nan
    tg[1, 2, 3000] = np.inf
    dr[3, 1, 5] = np.inf
    tg[5, 0, :] = -np.inf  # a whole target row without mass
    tg[5, 0, 7] = 1.0
    c["dtok"][0, 1] = 1500  # inside target row 1's -inf block: p_target 0, rejected there if reached
    return c


@pytest.mark.parametrize("T", [1.0, 0.5, 0.7])
def test_spec_special_blocks(sampler, oracle, T):
    _check(sampler, oracle, f"special_blocks T={T}", special_blocks_case(T))
