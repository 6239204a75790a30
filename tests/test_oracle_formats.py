"""Pins the oracle's number-format primitives against independent implementations
(numpy's IEEE binary16, torch's bfloat16) and libm's exp."""
import numpy as np
import pytest
import torch

import ito


def _special_f32():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e6, -1e6, 6.1035156e-05,
            5.9604645e-08, 2.9802322e-08, 2.9802326e-08, 1e-9, np.inf, -np.inf, 3.4e38,
            1.0009765625, 1.00048828125, 1.000244140625, 1.0014648437]
    return np.array(vals, dtype=np.float32)


def test_float_to_half_matches_numpy_rne():
    rng = np.random.default_rng(0)
    xs = np.concatenate([
        _special_f32(),
        rng.standard_normal(20000).astype(np.float32) * np.float32(0.05),
        (rng.standard_normal(20000) * 1e-5).astype(np.float32),   # subnormal halves
        (rng.standard_normal(5000) * 3e4).astype(np.float32),      # near overflow
        rng.integers(0, 2**32, 20000, dtype=np.uint64).astype(np.uint32).view(np.float32),
    ])
    xs = xs[~np.isnan(xs)]
    ours = np.array([ito.lib.ito_float_to_half(float(x)) for x in xs], dtype=np.uint16)
    ref = xs.astype(np.float16).view(np.uint16)
    assert (ours == ref).all()


def test_half_to_float_exact_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    ours = np.array([ito.lib.ito_half_to_float(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(ref)
    assert (np.isnan(ours) == nan).all()
    assert (ours[~nan].view(np.uint32) == ref[~nan].view(np.uint32)).all()


def test_float_to_bf16_matches_torch_rne():
    rng = np.random.default_rng(1)
    xs = np.concatenate([_special_f32(), rng.standard_normal(50000).astype(np.float32),
                         rng.integers(0, 2**32, 50000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    xs = xs[~np.isnan(xs)]
    ref = torch.from_numpy(xs).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    ours = np.array([ito.lib.ito_float_to_bf16(float(x)) for x in xs], dtype=np.uint16)
    assert (ours == ref).all()


def _ulp_diff(a, b):
    ia = a.view(np.int32).astype(np.int64)
    ib = b.view(np.int32).astype(np.int64)
    return np.abs(ia - ib)


def test_expf_within_two_ulp_of_libm():
    xs = np.concatenate([np.linspace(-87.3, 88.7, 200001, dtype=np.float32),
                         np.linspace(-20, 0, 100001, dtype=np.float32)])
    ours = np.array([ito.lib.ito_expf(float(x)) for x in xs], dtype=np.float32)
    ref = np.exp(xs.astype(np.float64)).astype(np.float32)
    assert _ulp_diff(ours, ref).max() <= 2


def test_expf_special_values():
    f = ito.lib.ito_expf
    assert f(0.0) == 1.0
    assert f(-0.0) == 1.0
    assert f(float("inf")) == float("inf")
    assert f(-float("inf")) == 0.0
    assert f(100.0) == float("inf")
    assert f(-100.0) == 0.0
    assert np.isnan(f(float("nan")))
    # results below FLT_MIN flush to zero
    assert f(-87.5) == 0.0
