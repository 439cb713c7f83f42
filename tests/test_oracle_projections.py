"""Pins of the oracle's NF4 projections: GEMV, fused RMSNorm+QKV(+bias),
SwiGLU and the K = 11008 down projection.

Held to (1) the reference smoke tests' fixtures and tolerances
(tests/nf4_tiled_gemv_smoke.cu, tests/nf4_fused_qkv_smoke.cu,
tests/nf4_swiglu_smoke.cu, tests/nf4_swiglu_bf16_smoke.cu), (2) fp64
restatements with the bf16 output tolerance, and (3) exact invariants
(one-hot inputs select a weight column; all-zero code rows).  Planted
mistakes (nibble order, a dropped bias) must fail the same checks.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from oracle.reference import nf4_dequant_f64, rmsnorm_f64, silu_f64
from tests import _kat

F = np.float32


def _qkv_f64(x, gamma, eps, triples, dtype):
    xn = rmsnorm_f64(O.act_to_f32(x, dtype), O.act_to_f32(gamma, dtype), eps)
    outs = []
    for (packed, absmax, bias), rows in zip(triples, (2048, 256, 256)):
        w = nf4_dequant_f64(packed, absmax, rows * 2048).reshape(rows, 2048)
        outs.append(w @ xn + O.act_to_f32(bias, dtype).astype(np.float64))
    return outs


def _swap_nibbles(packed: np.ndarray) -> np.ndarray:
    return (((packed & 0xF) << 4) | (packed >> 4)).astype(np.uint8)


@pytest.mark.parametrize("case", [_kat.tiled_gemv_case, _kat.fused_qkv_case])
def test_qkv_meets_reference_smoke_tolerance(case):
    x, gamma, eps, q, k, v, tol = case("f16")
    got = O.qkv(x, gamma, eps, q, k, v, dtype="f16")
    want = _qkv_f64(x, gamma, eps, (q, k, v), "f16")
    for g, w in zip(got, want):
        err = np.abs(O.f16_to_f32(g) - w)
        assert err.max() <= tol
        # much tighter than the smoke test: one fp16 ulp of the output plus fp32 accumulation
        assert np.all(err <= np.abs(w) * 2.0 ** -10 + 2e-4)


def test_qkv_planted_nibble_swap_fails_the_smoke_check():
    x, gamma, eps, q, k, v, tol = _kat.tiled_gemv_case("f16")
    bad = (_swap_nibbles(q[0]), q[1], q[2])
    got = O.qkv(x, gamma, eps, bad, k, v, dtype="f16")[0]
    want = _qkv_f64(x, gamma, eps, (q, k, v), "f16")[0]
    assert np.abs(O.f16_to_f32(got) - want).max() > tol


def test_qkv_planted_dropped_bias_fails_the_tight_check():
    x, gamma, eps, q, k, v, _ = _kat.fused_qkv_case("f16")
    zero = np.zeros_like(q[2])
    got = O.qkv(x, gamma, eps, (q[0], q[1], zero), k, v, dtype="f16")[0]
    want = _qkv_f64(x, gamma, eps, (q, k, v), "f16")[0]
    assert not np.all(np.abs(O.f16_to_f32(got) - want) <= np.abs(want) * 2.0 ** -10 + 2e-4)


def test_qkv_bf16_on_random_weights_and_normalised_copy():
    rng = np.random.default_rng(20260824)
    x = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    gamma = O.f32_to_bf16((F(1) + rng.standard_normal(2048).astype(F) * F(0.1)))
    triples = []
    for rows in (2048, 256, 256):
        p, a = O.nf4_quantize(rng.standard_normal(rows * 2048).astype(F) * F(0.02))
        triples.append((p, a, O.f32_to_bf16(rng.standard_normal(rows).astype(F) * F(0.01))))
    qo, ko, vo, norm = O.qkv(x, gamma, 1e-6, *triples, dtype="bf16", want_norm=True)
    want_norm = rmsnorm_f64(O.bf16_to_f32(x), O.bf16_to_f32(gamma), 1e-6)
    assert np.allclose(norm, want_norm, rtol=2e-6, atol=1e-7)
    for g, w in zip((qo, ko, vo), _qkv_f64(x, gamma, 1e-6, triples, "bf16")):
        assert np.all(np.abs(O.bf16_to_f32(g) - w) <= 1e-2 * np.abs(w) + 1e-3)


def test_gemv_one_hot_input_selects_a_column_exactly():
    rng = np.random.default_rng(1)
    rows = 2048
    packed, absmax = O.nf4_quantize(rng.standard_normal(rows * 2048).astype(F))
    w = O.nf4_dequantize(packed, absmax, rows * 2048).reshape(rows, 2048)
    for j in (0, 1, 31, 32, 1000, 2047):
        x = np.zeros(2048, dtype=np.uint16)
        x[j] = O.f32_to_bf16(np.array([1.0], dtype=F))[0]
        y = O.nf4_gemv2048(x, packed, absmax, rows)
        assert y.tobytes() == O.f32_to_bf16(w[:, j]).tobytes()


def test_gemv_all_zero_codes_give_minus_absmax_times_sum():
    rows = 64
    packed = np.zeros(rows * 1024, dtype=np.uint8)            # code 0 = -1.0
    absmax = np.full(rows * 32, 0.5, dtype=F)
    x = O.f32_to_bf16(np.full(2048, 0.25, dtype=F))
    y = O.bf16_to_f32(O.nf4_gemv2048(x, packed, absmax, rows))
    assert np.all(y == F(-0.5 * 0.25 * 2048))


@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("with_residual", [False, True])
def test_gemv_epilogue_against_fp64(with_bias, with_residual):
    rng = np.random.default_rng(9)
    rows = 512
    packed, absmax = O.nf4_quantize(rng.standard_normal(rows * 2048).astype(F) * F(0.02))
    x = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    bias = O.f32_to_bf16(rng.standard_normal(rows).astype(F) * F(0.05)) if with_bias else None
    res = O.f32_to_bf16(rng.standard_normal(rows).astype(F)) if with_residual else None
    y = O.bf16_to_f32(O.nf4_gemv2048(x, packed, absmax, rows, bias=bias, residual=res))
    dot = nf4_dequant_f64(packed, absmax, rows * 2048).reshape(rows, 2048) @ O.bf16_to_f32(x).astype(np.float64)
    if bias is not None:
        dot = dot + O.bf16_to_f32(bias)
    if res is not None:
        dot = O.bf16_to_f32(res) + O.bf16_to_f32(O.f32_to_bf16(dot.astype(F)))
    assert np.all(np.abs(y - dot) <= 1e-2 * np.abs(dot) + 1e-3)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_swiglu_meets_reference_smoke_tolerance(dtype):
    x, gamma, eps, gate, up, tol = _kat.swiglu_case(dtype)
    got = O.act_to_f32(O.swiglu(x, gamma, eps, gate, up, dtype=dtype), dtype)
    xn = rmsnorm_f64(O.act_to_f32(x, dtype), O.act_to_f32(gamma, dtype), eps)
    g = nf4_dequant_f64(gate[0], gate[1], 11008 * 2048).reshape(11008, 2048) @ xn
    u = nf4_dequant_f64(up[0], up[1], 11008 * 2048).reshape(11008, 2048) @ xn
    want = silu_f64(g) * u
    err = np.abs(got - want)
    assert err.max() <= tol
    ulp = 2.0 ** -10 if dtype == "f16" else 2.0 ** -7
    assert np.all(err <= np.abs(want) * ulp + 1e-3)


def test_down_projection_with_residual_against_fp64():
    rng = np.random.default_rng(13)
    packed, absmax = O.nf4_quantize(rng.standard_normal(2048 * 11008).astype(F) * F(0.02))
    h = O.f32_to_bf16(rng.standard_normal(11008).astype(F))
    res = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    y = O.bf16_to_f32(O.down11008(h, packed, absmax, residual=res))
    dot = nf4_dequant_f64(packed, absmax, 2048 * 11008).reshape(2048, 11008) @ O.bf16_to_f32(h).astype(np.float64)
    want = O.bf16_to_f32(res) + O.bf16_to_f32(O.f32_to_bf16(dot.astype(F)))
    assert np.all(np.abs(y - want) <= 1e-2 * np.abs(want) + 1e-3)
