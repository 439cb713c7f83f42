"""Pins of the oracle's scalar building blocks: exp2, SiLU, RMSNorm and the
fp32 -> bf16 / fp16 conversions."""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle import oracle as O
from oracle.reference import rmsnorm_reference
from tests import _kat

F = np.float32


def _ulp_err(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    ulp = np.spacing(np.abs(want).astype(F)).astype(np.float64)
    return np.abs(got.astype(np.float64) - want) / ulp


def test_exp2_is_within_two_ulp_over_its_range():
    y = np.concatenate([np.linspace(-125.0, 127.99, 400001, dtype=F),
                        np.linspace(-1, 1, 100001, dtype=F)])
    got = O.exp2(y)
    want = np.exp2(y.astype(np.float64))
    assert _ulp_err(got, want).max() <= 2.0


def test_exp2_special_values():
    y = np.array([0.0, 1.0, -1.0, 10.0, -100.0, -125.0, -125.5, -200.0, 128.0, 1000.0, np.inf, -np.inf, np.nan],
                 dtype=F)
    got = O.exp2(y)
    assert got[0] == 1.0 and got[1] == 2.0 and got[2] == 0.5 and got[3] == 1024.0
    assert got[4] == F(2.0 ** -100) and got[5] == F(2.0 ** -125)
    assert got[6] == 0.0 and got[7] == 0.0 and got[11] == 0.0       # flush below 2^-125
    assert np.isinf(got[8]) and np.isinf(got[9]) and np.isinf(got[10])
    assert np.isnan(got[12])
    ints = np.arange(-125, 128, dtype=F)
    assert np.array_equal(O.exp2(ints), np.exp2(ints.astype(np.float64)).astype(F))


def test_silu_against_fp64():
    g = np.linspace(-40, 40, 200001, dtype=F)
    got = O.silu(g).astype(np.float64)
    want = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))
    # the exponent g * -log2e is formed in fp32, so its rounding (relative
    # 2^-24 of |g| log2e) dominates for large |g|: bound 1e-7 * (4 + |g|)
    bound = 1e-7 * (4.0 + np.abs(g.astype(np.float64)))
    assert np.all(np.abs(got - want) <= bound * np.abs(want) + 1e-30)


def test_rmsnorm_reference_kat():
    # reference tests/test_contracts.py:732-742
    out = rmsnorm_reference([[3.0, 4.0], [0.0, 1.0]], [1.0, 0.5], epsilon=1e-5)
    assert abs(out[0][0] - 0.848528) < 1e-5
    assert abs(out[0][1] - 0.565685) < 1e-5
    assert abs(out[1][1] - 0.7071) < 1e-4


def test_rmsnorm_reference_on_the_smoke_fixture():
    x, w, eps, tol = _kat.rmsnorm_smoke_case()
    got = np.array(rmsnorm_reference(x.tolist(), w.tolist(), epsilon=eps))
    xs = x.astype(np.float64)
    want = xs / np.sqrt((xs * xs).mean(axis=1, keepdims=True) + eps) * w
    assert np.abs(got - want).max() <= tol


def test_bf16_conversion_matches_torch_round_to_nearest_even():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(100000).astype(F),
        np.array([0.0, -0.0, 1.0, np.inf, -np.inf, 3.4e38, 1e-40, -1e-40, 1.00390625, 1.01171875], dtype=F),
        (rng.integers(0, 2 ** 32, size=100000, dtype=np.uint64).astype(np.uint32)).view(F),
    ])
    finite = ~np.isnan(x)
    got = O.f32_to_bf16(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got[finite], want[finite])
    nan_bits = got[~finite]
    assert np.all((nan_bits & 0x7F80) == 0x7F80) and np.all((nan_bits & 0x0040) != 0)


def test_f16_conversion_matches_numpy():
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(F) * F(100),
                        np.array([65504.0, 65520.0, 1e-8, 6.1e-5, -0.0], dtype=F)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(O.f32_to_f16(x), want)
