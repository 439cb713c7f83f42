"""Textbook fp64 references and comparison helpers — TEST INFRASTRUCTURE ONLY.

These are written straight from the mathematics (no fixed reduction order, no
kernel structure) and pin the bit-mirroring oracle in ``oracle.py`` with
tolerances; ``compare_values`` and ``rmsnorm_reference`` restate the
reference harness (harness/compare.py:20-95, harness/reference.py:9-31).
"""

from __future__ import annotations

import math
from collections.abc import Sequence
from typing import Any

import numpy as np

NF4_CODEBOOK_F64 = np.array(
    [
        -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
        -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
        0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
        0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
    ],
    dtype=np.float64,
)


def rmsnorm_reference(rows: Sequence[Sequence[float]], weight: Sequence[float], epsilon: float = 1.0e-5):
    """Row-wise RMSNorm with fp64 accumulation (harness/reference.py:9-31)."""

    if epsilon <= 0.0:
        raise ValueError("epsilon must be positive")
    hidden = len(weight)
    if hidden == 0:
        raise ValueError("weight must not be empty")
    out = []
    for row in rows:
        if len(row) != hidden:
            raise ValueError("each input row must match the weight length")
        inv = 1.0 / math.sqrt(sum(float(v) * float(v) for v in row) / hidden + epsilon)
        out.append([float(v) * inv * float(w) for v, w in zip(row, weight)])
    return out


def _flatten(values: Any):
    if isinstance(values, np.ndarray):
        yield from values.reshape(-1).tolist()
        return
    if isinstance(values, Sequence) and not isinstance(values, (str, bytes, bytearray)):
        for value in values:
            yield from _flatten(value)
        return
    yield values


def compare_values(actual: Any, expected: Any, *, atol: float = 1.0e-5, rtol: float = 1.0e-5,
                   exact: bool = False) -> dict[str, Any]:
    """|a - e| <= atol + rtol*|e| per element with NaN/Inf accounting
    (harness/compare.py:20-95)."""

    a_vals = list(_flatten(actual))
    e_vals = list(_flatten(expected))
    shape_match = len(a_vals) == len(e_vals)
    count = min(len(a_vals), len(e_vals))
    max_abs = max_rel = sq = 0.0
    mismatches = nan_a = nan_e = inf_mm = 0
    for av, ev in zip(a_vals, e_vals):
        af, ef = float(av), float(ev)
        an, en = math.isnan(af), math.isnan(ef)
        nan_a += an
        nan_e += en
        if an or en:
            mismatches += int(not (an and en))
            continue
        ai, ei = math.isinf(af), math.isinf(ef)
        if ai or ei:
            if not (ai and ei and af == ef):
                inf_mm += 1
                mismatches += 1
            continue
        if exact:
            ok = av == ev
            err = 0.0 if ok else abs(af - ef)
        else:
            err = abs(af - ef)
            ok = err <= atol + rtol * abs(ef)
        mismatches += int(not ok)
        max_abs = max(max_abs, err)
        max_rel = max(max_rel, err / max(abs(ef), 1.0e-12))
        sq += err * err
    if not shape_match:
        mismatches += abs(len(a_vals) - len(e_vals))
    return {
        "passed": shape_match and mismatches == 0 and nan_a == 0 and nan_e == 0 and inf_mm == 0,
        "exact": exact, "atol": atol, "rtol": rtol, "count": count, "actual_count": len(a_vals),
        "expected_count": len(e_vals), "shape_match": shape_match, "mismatches": mismatches,
        "max_abs_error": max_abs, "max_rel_error": max_rel, "rms_error": math.sqrt(sq / max(count, 1)),
        "nan_actual": nan_a, "nan_expected": nan_e, "inf_mismatch": inf_mm,
    }


def nf4_dequant_f64(packed: np.ndarray, absmax: np.ndarray, n: int, blocksize: int = 64) -> np.ndarray:
    """Unpack nibbles (even element = high nibble) and scale, in fp64."""

    codes = np.empty(n, dtype=np.int64)
    codes[0::2] = packed[: (n + 1) // 2] >> 4
    codes[1::2] = packed[: n // 2] & 0x0F
    return NF4_CODEBOOK_F64[codes] * absmax.astype(np.float64)[np.arange(n) // blocksize]


def rmsnorm_f64(x: np.ndarray, gamma: np.ndarray | None, eps: float) -> np.ndarray:
    """Row-wise over the last axis (a 1-D vector is one row)."""

    x = x.astype(np.float64)
    if gamma is None:
        return x
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * gamma.astype(np.float64)


def silu_f64(g: np.ndarray) -> np.ndarray:
    g = np.asarray(g, dtype=np.float64)
    return g / (1.0 + np.exp(-g))


def gqa_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, kv_len: int, scale: float) -> np.ndarray:
    """Textbook decode attention: q [16,128], k/v [2, >=L, 128], group 8."""

    q = q.reshape(16, 128).astype(np.float64)
    out = np.empty((16, 128))
    for h in range(16):
        g = h // 8
        kk = k[g, :kv_len].astype(np.float64)
        vv = v[g, :kv_len].astype(np.float64)
        s = kk @ q[h] * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vv
    return out.reshape(-1)


def rope_f64(x: np.ndarray, pos: int, theta: float = 1.0e6, head_dim: int = 128) -> np.ndarray:
    """rotate-half RoPE of a [heads*head_dim] vector at one position."""

    half = head_dim // 2
    inv = 1.0 / theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim)
    ang = pos * inv[:half]
    c, s = np.cos(ang), np.sin(ang)
    xs = x.reshape(-1, head_dim).astype(np.float64)
    x1, x2 = xs[:, :half], xs[:, half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=1).reshape(-1)
