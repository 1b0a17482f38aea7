"""Pins the oracle's numerics against mathematics (CPU only).

tgo_expf is checked against fp64 exp in ulps; the mass quantiser, the
u64 -> f32 rounding and the order keys against exact integer / rational
arithmetic computed in Python.
"""
import math
import struct
from fractions import Fraction

import numpy as np
import pytest


def f32(x):
    return struct.unpack("<f", struct.pack("<f", x))[0]


def test_expf_accuracy(oracle):
    g = np.random.default_rng(1)
    x = np.concatenate([
        np.linspace(-32, 0, 100001, dtype=np.float32),
        (-g.random(100000) * 32).astype(np.float32),
        -g.random(20000).astype(np.float32) * 1e-3,
        np.float32([0.0, -0.0, -1e-30, -31.999998, -0.34657359, -0.34657362, 1.0, 5.5]),
    ])
    e = oracle.expf(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    err = np.abs(e - ref) / ulp
    assert err.max() <= 1.0, err.max()


def test_weight_wide_accuracy(oracle):
    """The reported-probability weight: within one ulp of fp64 exp down to
    -86 (normal results only), equal to the mass weight where both are
    defined, 0 below -86."""
    g = np.random.default_rng(3)
    x = np.concatenate([np.linspace(-86, 0, 100001, dtype=np.float32),
                        (-g.random(50000) * 86).astype(np.float32),
                        np.float32([-85.99999, -86.0, -32.0, -32.000004, -0.0])])
    e = oracle.weight_wide(x).astype(np.float64)
    ref = np.exp(x.astype(np.float64))
    ulp = np.spacing(ref.astype(np.float32)).astype(np.float64)
    assert (np.abs(e - ref) / ulp).max() <= 1.0
    assert np.all(e >= np.finfo(np.float32).tiny)  # normal results
    xs = x[x >= -32]
    np.testing.assert_array_equal(oracle.weight_wide(xs), oracle.expf(xs))
    L = oracle.lib()
    assert L.tgo_weight_wide(-86.5, 0.0) == 0.0
    assert L.tgo_weight_wide(float("-inf"), 0.0) == 0.0
    assert L.tgo_weight_wide(2.0, 2.0) == 1.0


def test_expf_special_values(oracle):
    L = oracle.lib()
    assert L.tgo_expf(0.0) == 1.0
    assert L.tgo_expf(-0.0) == 1.0
    assert L.tgo_expf(-32.5) == 0.0
    assert L.tgo_expf(float("-inf")) == 0.0
    assert L.tgo_expf(float("nan")) == 0.0
    # weight: equal values weigh exactly one (also at +inf)
    assert L.tgo_weight(3.0, 3.0) == 1.0
    assert L.tgo_weight(float("inf"), float("inf")) == 1.0
    assert L.tgo_weight(1.0, float("inf")) == 0.0
    # monotone over a dense grid of the working range
    x = np.linspace(-32, 0, 20001, dtype=np.float32)
    e = oracle.expf(x)
    assert np.all(np.diff(e) >= 0)


def test_q40_is_floor_of_scaled_value(oracle):
    L = oracle.lib()
    g = np.random.default_rng(2)
    vals = np.concatenate([g.random(2000).astype(np.float32), np.float32([0, 1, 2.0**-17, 2.0**-40, 2.0**-41, 0.5])])
    for v in vals:
        exact = math.floor(Fraction(float(v)) * (1 << 40))
        assert L.tgo_q40(float(v)) == exact


def _rne_u64_to_f32(x):
    if x == 0:
        return 0.0
    fr = Fraction(x)
    e = x.bit_length() - 24
    if e <= 0:
        return float(x)
    m, r = divmod(x, 1 << e)
    half = 1 << (e - 1)
    if r > half or (r == half and (m & 1)):
        m += 1
    return float(m * (1 << e))


def test_u64_to_f32_round_to_nearest_even(oracle):
    L = oracle.lib()
    g = np.random.default_rng(3)
    cases = [0, 1, (1 << 24) - 1, 1 << 24, (1 << 24) + 1, (1 << 25) + 1, (1 << 25) + 3, (1 << 64) - 1,
             (1 << 40) + (1 << 16), (1 << 40) + (1 << 16) + 1, (1 << 41) + (3 << 17)]
    cases += [int(v) for v in g.integers(0, 1 << 62, size=3000, dtype=np.int64)]
    cases += [int(v) >> int(s) for v, s in zip(g.integers(0, 1 << 62, size=2000, dtype=np.int64), g.integers(0, 40, size=2000))]
    for x in cases:
        assert L.tgo_u64_to_f32(x) == f32(_rne_u64_to_f32(x)), x


def test_keys_preserve_order(oracle):
    L = oracle.lib()
    g = np.random.default_rng(4)
    vals = np.concatenate([
        (g.standard_normal(3000) * 10).astype(np.float32),
        np.float32([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-45, 3.4e38, -3.4e38, 1.0, -1.0]),
    ])
    keys = np.array([L.tgo_key(float(v)) for v in vals], dtype=np.uint64)
    order_k = np.argsort(keys, kind="stable")
    sv = vals[order_k].astype(np.float64)
    assert np.all(np.diff(sv) >= 0)
    # equal values (including -0 / +0) share one key; keys invert exactly
    assert L.tgo_key(0.0) == L.tgo_key(-0.0)
    for v in vals:
        back = L.tgo_unkey(L.tgo_key(float(v)))
        assert back == float(v)
    assert L.tgo_key(float("-inf")) > 0
