"""Known-answer inputs restated from the reference's own smoke tests.

Each generator reproduces the formula-defined fixture of one reference test so
the oracle (and, in the GPU tests, the kernels) can be held to that test's
tolerance.  Formulas only; no reference code is imported or run.
"""

from __future__ import annotations

import numpy as np

from oracle import oracle as O

F = np.float32


def packed_codes(rows: int, cols: int, mult: int, salt: int) -> np.ndarray:
    """Codes (i*mult + salt) & 0xF, even element in the high nibble
    (tests/nf4_tiled_gemv_smoke.cu:28-35, tests/nf4_fused_qkv_smoke.cu:41-46)."""

    i = np.arange(rows * cols, dtype=np.int64)
    codes = ((i * mult + salt) & 0xF).astype(np.uint8)
    return ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)


def ramp(n: int, base: float, mod: int, step: float) -> np.ndarray:
    """base + (i % mod) * step in fp32, as the smoke tests fill scales."""

    i = np.arange(n, dtype=np.int64)
    return (F(base) + (i % mod).astype(F) * F(step)).astype(F)


def tiled_gemv_case(dtype: str = "f16"):
    """tests/nf4_tiled_gemv_smoke.cu:49-75: hidden 2048, q 2048, kv 256,
    salts 1/3/7, eps 1e-5, abs tolerance 0.035."""

    i = np.arange(2048)
    x = O.f32_to_act(np.sin(i.astype(F) * F(0.013)), dtype)
    gamma = O.f32_to_act(F(0.75) + (i % 23).astype(F) * F(0.004), dtype)
    q = (packed_codes(2048, 2048, 5, 1), ramp(2048 * 32, 0.2, 19, 0.009),
         O.f32_to_act(((np.arange(2048) % 11) - 5).astype(F) * F(0.002), dtype))
    k = (packed_codes(256, 2048, 5, 3), ramp(256 * 32, 0.25, 17, 0.011),
         O.f32_to_act(((np.arange(256) % 7) - 3).astype(F) * F(0.003), dtype))
    v = (packed_codes(256, 2048, 5, 7), ramp(256 * 32, 0.18, 13, 0.013),
         O.f32_to_act(((np.arange(256) % 5) - 2).astype(F) * F(0.004), dtype))
    return x, gamma, 1.0e-5, q, k, v, 0.035


def fused_qkv_case(dtype: str = "f16"):
    """tests/nf4_fused_qkv_smoke.cu:59-105: codes (i*7+salt), salts 3/5/9."""

    i = np.arange(2048)
    x = O.f32_to_act(np.sin(i.astype(F) * F(0.017)), dtype)
    gamma = O.f32_to_act(F(0.8) + (i % 31).astype(F) * F(0.003), dtype)
    q = (packed_codes(2048, 2048, 7, 3), ramp(2048 * 32, 0.25, 17, 0.01),
         O.f32_to_act(((np.arange(2048) % 17) - 8).astype(F) * F(0.003), dtype))
    k = (packed_codes(256, 2048, 7, 5), ramp(256 * 32, 0.3, 13, 0.012),
         O.f32_to_act(((np.arange(256) % 13) - 6).astype(F) * F(0.004), dtype))
    v = (packed_codes(256, 2048, 7, 9), ramp(256 * 32, 0.2, 11, 0.014),
         O.f32_to_act(((np.arange(256) % 11) - 5).astype(F) * F(0.005), dtype))
    return x, gamma, 1.0e-5, q, k, v, 0.035


def swiglu_case(dtype: str = "f16"):
    """tests/nf4_swiglu_smoke.cu:48-62 (fp16, tol 0.045) and
    tests/nf4_swiglu_bf16_smoke.cu:48-62 (bf16, tol 0.08)."""

    i = np.arange(2048)
    x = O.f32_to_act(np.sin(i.astype(F) * F(0.013)), dtype)
    gamma = O.f32_to_act(F(0.75) + (i % 23).astype(F) * F(0.004), dtype)
    gate = (packed_codes(11008, 2048, 5, 1), ramp(11008 * 32, 0.12, 19, 0.003))
    up = (packed_codes(11008, 2048, 5, 7), ramp(11008 * 32, 0.15, 17, 0.004))
    tol = 0.045 if dtype in ("f16", "fp16") else 0.08
    return x, gamma, 1.0e-5, gate, up, tol


def gqa_smoke_case(kv_len: int = 37):
    """tests/qwen2_gqa_smoke.cu:34-63: fp16 q sin(i*0.017)*0.75, K cos(i*0.011)*0.55,
    V sin(i*0.023)*0.65, tolerance 3.5e-3."""

    iq = np.arange(16 * 128)
    ic = np.arange(2 * kv_len * 128)
    q = O.f32_to_f16(np.sin(iq.astype(F) * F(0.017)) * F(0.75))
    k = O.f32_to_f16(np.cos(ic.astype(F) * F(0.011)) * F(0.55)).reshape(2, kv_len, 128)
    v = O.f32_to_f16(np.sin(ic.astype(F) * F(0.023)) * F(0.65)).reshape(2, kv_len, 128)
    return q, k, v, 3.5e-3


def rmsnorm_smoke_case():
    """tests/rmsnorm_smoke.cu:27-58: 7 x 513 fp32, tolerance 5e-5."""

    x = (np.sin(np.arange(7 * 513).astype(F) * F(0.013)) * F(0.75)).reshape(7, 513)
    w = (F(0.5) + (np.arange(513) % 17).astype(F) * F(0.03125)).astype(F)
    return x, w, 1.0e-5, 5.0e-5


def gqa_workspace_case(capacity: int = 512):
    """tests/qwen2_gqa_workspace_smoke.cu:29-49: fp16 cache of 512 slots,
    q sin(i*0.013), K cos(i*0.009), V sin(i*0.007); kv_len 1, 7, 64, 128, 512;
    tolerance 6e-3 (:128)."""

    iq = np.arange(16 * 128)
    ic = np.arange(2 * capacity * 128)
    q = O.f32_to_f16(np.sin(iq.astype(F) * F(0.013)))
    k = O.f32_to_f16(np.cos(ic.astype(F) * F(0.009))).reshape(2, capacity, 128)
    v = O.f32_to_f16(np.sin(ic.astype(F) * F(0.007))).reshape(2, capacity, 128)
    return q, k, v, (1, 7, 64, 128, 512), 6.0e-3
