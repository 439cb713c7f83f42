"""Pins of the oracle's NF4 format code (dequantise, quantise, nibble order).

The oracle restates reference kernels/common/nf4_device.cuh:10-40; these tests
hold it to the published bitsandbytes NF4 table, to the closed form of the
dequantisation, and to brute-force nearest-code search.
"""

from __future__ import annotations

import re
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O
from oracle.reference import nf4_dequant_f64

ROOT = Path(__file__).resolve().parents[1]

# The NF4 data type's 16 values as published with QLoRA / bitsandbytes
# (normal-distribution quantiles, exact zero, +-1), in decimal.
PUBLISHED_NF4 = [
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
]


def _codes(packed: np.ndarray) -> np.ndarray:
    out = np.empty(packed.size * 2, dtype=np.int64)
    out[0::2] = packed >> 4
    out[1::2] = packed & 0xF
    return out


def test_oracle_codebook_is_the_published_table():
    packed = np.array([(2 * c << 4) | (2 * c + 1) for c in range(8)], dtype=np.uint8)
    got = O.nf4_dequantize(packed, np.ones(1, dtype=np.float32), 16, 64)
    assert got.tobytes() == np.array(PUBLISHED_NF4, dtype=np.float32).tobytes()


def test_device_codebook_literals_are_the_published_table():
    """The kernels' hex literals (kc_device.h) equal fp32 of the published values."""

    src = (ROOT / "kudacuda_amd" / "csrc" / "kc_device.h").read_text()
    tables = re.findall(r"\{([^{}]*0x1\.000000p\+0f[^{}]*)\}", src)
    assert tables, "codebook tables not found"
    want = np.array(PUBLISHED_NF4, dtype=np.float32)
    for body in tables:
        vals = [float.fromhex(t.rstrip("f")) for t in re.findall(r"-?0x[0-9a-fA-F.]+p[+-]\d+f", body)]
        assert np.array(vals, dtype=np.float32).tobytes() == want.tobytes()


def test_nibble_order_even_element_high():
    # byte 0xAB: element 0 = code 10, element 1 = code 11 (nf4_device.cuh:36-39)
    got = O.nf4_dequantize(np.array([0xAB], dtype=np.uint8), np.array([2.0], dtype=np.float32), 2, 64)
    assert got[0] == np.float32(PUBLISHED_NF4[10]) * np.float32(2.0)
    assert got[1] == np.float32(PUBLISHED_NF4[11]) * np.float32(2.0)


@pytest.mark.parametrize("blocksize", [64, 128])
def test_dequantize_is_the_closed_form_bit_exact(blocksize):
    rng = np.random.default_rng(7)
    n = 64 * 1024
    packed = rng.integers(0, 256, size=n // 2, dtype=np.uint8)
    absmax = rng.uniform(0.001, 3.0, size=n // blocksize).astype(np.float32)
    got = O.nf4_dequantize(packed, absmax, n, blocksize)
    want = np.array(PUBLISHED_NF4, dtype=np.float32)[_codes(packed)] * np.repeat(absmax, blocksize)
    assert got.tobytes() == want.astype(np.float32).tobytes()
    # and the fp64 restatement agrees to fp32 rounding
    assert np.array_equal(got, nf4_dequant_f64(packed, absmax, n, blocksize).astype(np.float32))


def _brute_force_codes(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    blocks = w.reshape(-1, 64).astype(np.float32)
    absmax = np.abs(blocks).max(axis=1)
    inv = np.where(absmax > 0, np.float32(1.0) / np.where(absmax > 0, absmax, 1), 0).astype(np.float32)
    s = (blocks * inv[:, None]).astype(np.float64)
    cb = np.array(PUBLISHED_NF4, dtype=np.float64)
    dist = np.abs(s[..., None] - cb)
    return dist, absmax


def test_quantize_picks_a_nearest_code_and_exact_absmax():
    rng = np.random.default_rng(11)
    w = rng.standard_normal(64 * 4096).astype(np.float32) * np.float32(0.02)
    w[:64] = 0.0                       # all-zero block -> code 7 (exact zero)
    w[64:128] = np.linspace(-1, 1, 64, dtype=np.float32)
    packed, absmax = O.nf4_quantize(w)
    dist, want_absmax = _brute_force_codes(w)
    assert absmax.tobytes() == want_absmax.astype(np.float32).tobytes()
    codes = _codes(packed).reshape(-1, 64)
    assert np.all(codes[0] == 7)
    chosen = np.take_along_axis(dist, codes[..., None], axis=2)[..., 0]
    best = dist.min(axis=2)
    # nearest up to the fp32 rounding of the decision midpoints
    assert np.all(chosen <= best + 1e-7)
    # the block's extreme element maps to +-1 exactly
    ext = np.abs(w.reshape(-1, 64)).argmax(axis=1)
    ext_codes = codes[np.arange(codes.shape[0]), ext]
    nonzero = want_absmax > 0
    assert np.all(np.isin(ext_codes[nonzero], (0, 15)))


def test_quantize_round_trip_error_is_bounded_by_half_the_widest_gap():
    rng = np.random.default_rng(3)
    w = rng.standard_normal(64 * 2048).astype(np.float32)
    packed, absmax = O.nf4_quantize(w)
    back = O.nf4_dequantize(packed, absmax, w.size, 64)
    half_gap = np.max(np.diff(PUBLISHED_NF4)) / 2
    err = np.abs(back - w).reshape(-1, 64)
    assert np.all(err <= absmax[:, None] * (half_gap + 1e-6))


def test_bf16_and_fp32_quantizers_agree_on_bf16_exact_inputs():
    rng = np.random.default_rng(5)
    w32 = rng.standard_normal(64 * 512).astype(np.float32)
    bits = O.f32_to_bf16(w32)
    p_a, a_a = O.nf4_quantize(bits)
    p_b, a_b = O.nf4_quantize(O.bf16_to_f32(bits))
    assert p_a.tobytes() == p_b.tobytes() and a_a.tobytes() == a_b.tobytes()
