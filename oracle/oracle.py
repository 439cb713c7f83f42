"""CPU oracle for the KudaCuda gfx950 decode path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this module, and only as the checker (or the timed CPU
baseline).  The product package ``kudacuda_amd`` never imports it.

Thin numpy wrappers over ``liboracle.so`` (built from ``kc_oracle.c`` by
``build_oracle.sh``), whose functions restate the reference's decode math in
the fixed fp32 operation order the kernels are specified to use, so results
compare bit for bit.  Each wrapper names the reference code it follows; the
restatement is pinned independently in ``tests/test_oracle_*.py``.  The
prefill's MFMA GEMM and the matrix-core attention of long direct calls are
not restated here; their GPU tests hold them to fp64 references instead.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIBRARY = ORACLE_DIR / "liboracle.so"

_u8 = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16 = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_f32 = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_f = ctypes.c_float

_LIB = None

LOG2E_F32 = np.float32(1.0 / math.log(2.0))
NF4_CODEBOOK = np.array(
    [
        -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
        -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
        0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
        0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
    ],
    dtype=np.float32,
)  # bitsandbytes NF4 table, reference kernels/common/nf4_device.cuh:10-27


def build_oracle() -> Path:
    """Compile liboracle.so with the committed recipe (CPU only)."""

    subprocess.run(["sh", str(ORACLE_DIR / "build_oracle.sh")], check=True)
    return LIBRARY


def lib() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIBRARY.exists():
        build_oracle()
    L = ctypes.CDLL(str(LIBRARY))
    L.kco_nf4_quantize_f32.argtypes = [_f32, _i64, _u8, _f32]
    L.kco_nf4_quantize_bf16.argtypes = [_u16, _i64, _u8, _f32]
    L.kco_nf4_dequantize_f32.argtypes = [_u8, _f32, _i64, _i64, _f32]
    L.kco_convert.argtypes = [ctypes.c_int, ctypes.c_int, _vp, _vp, _i64]
    L.kco_exp2_array.argtypes = [_f32, _f32, _i64]
    L.kco_silu_array.argtypes = [_f32, _f32, _i64]
    L.kco_nf4_gemv2048.argtypes = [ctypes.c_int, _u16, _u8, _f32, _vp, _vp, _i64, _u16]
    L.kco_qkv.argtypes = [ctypes.c_int, _u16, _u16, _f, _u8, _f32, _u16, _u8, _f32, _u16, _u8, _f32, _u16,
                          _i64, _i64, _u16, _u16, _u16, _vp]
    L.kco_qkv_rope_cache.argtypes = [_u16, _u16, _f, _u8, _f32, _u16, _u8, _f32, _u16, _u8, _f32, _u16,
                                     _f32, _f32, _i64, _i64, _u16, _u16, _u16]
    L.kco_swiglu.argtypes = [ctypes.c_int, _u16, _vp, _f, _u8, _f32, _u8, _f32, _i64, _u16]
    L.kco_down11008.argtypes = [ctypes.c_int, _u16, _u8, _f32, _vp, _i64, _u16]
    L.kco_gqa_split_tokens.argtypes = [_i64, _i64]
    L.kco_gqa_split_tokens.restype = _i64
    L.kco_gqa_plan.argtypes = [_i64, _i64, ctypes.c_void_p]
    L.kco_gqa_plan.restype = None
    L.kco_gqa.argtypes = [ctypes.c_int, _u16, _u16, _u16, _i64, _i64, _i64, _f, _u16]
    L.kco_lm_head_argmax.argtypes = [_u16, _vp, _f, _u16, _i64, _vp]
    L.kco_lm_head_argmax.restype = ctypes.c_int32
    L.kco_qwen2_step.argtypes = [_i64, _i64, _i64, _f, _vp, _vp]
    _LIB = L
    return L


def _ptr(array: np.ndarray | None) -> int | None:
    return None if array is None else array.ctypes.data


def _act(dtype: str) -> int:
    return {"bf16": 0, "bfloat16": 0, "f16": 1, "fp16": 1, "float16": 1}[dtype]


# ------------------------------------------------------------ conversions
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bits (uint16)."""

    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().kco_convert(0, 1, x.ctypes.data, out.ctypes.data, x.size)
    return out


def bf16_to_f32(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.uint16)
    return (x.astype(np.uint32) << 16).view(np.float32)


def f32_to_f16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().kco_convert(0, 2, x.ctypes.data, out.ctypes.data, x.size)
    return out


def f16_to_f32(x: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.uint16).view(np.float16).astype(np.float32)


def act_to_f32(x: np.ndarray, dtype: str) -> np.ndarray:
    return bf16_to_f32(x) if _act(dtype) == 0 else f16_to_f32(x)


def f32_to_act(x: np.ndarray, dtype: str) -> np.ndarray:
    return f32_to_bf16(x) if _act(dtype) == 0 else f32_to_f16(x)


def exp2(y: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(y, dtype=np.float32)
    out = np.empty_like(y)
    lib().kco_exp2_array(y, out, y.size)
    return out


def silu(g: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    out = np.empty_like(g)
    lib().kco_silu_array(g, out, g.size)
    return out


# ------------------------------------------------------------------- NF4
def nf4_quantize(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Blockwise (64) NF4 quantisation of fp32 or bf16-bits input.

    Returns (packed u8 [n/2], absmax f32 [n/64]).  The bitsandbytes packing
    (even element in the high nibble) follows
    kernels/common/nf4_device.cuh:36-39; the quantiser itself restates
    blockwise absmax + nearest codebook value (bitsandbytes parity unpinned).
    """

    flat = np.ascontiguousarray(w).reshape(-1)
    n = flat.size
    packed = np.empty(n // 2, dtype=np.uint8)
    absmax = np.empty(n // 64, dtype=np.float32)
    if flat.dtype == np.float32:
        lib().kco_nf4_quantize_f32(flat, n, packed, absmax)
    elif flat.dtype == np.uint16:
        lib().kco_nf4_quantize_bf16(flat, n, packed, absmax)
    else:
        raise TypeError("nf4_quantize expects float32 or bf16 bits (uint16)")
    return packed, absmax


def nf4_dequantize(packed: np.ndarray, absmax: np.ndarray, n: int, blocksize: int = 64) -> np.ndarray:
    """codebook[code] * absmax[i / blocksize] (kernels/common/nf4_device.cuh:29-40)."""

    out = np.empty(n, dtype=np.float32)
    lib().kco_nf4_dequantize_f32(np.ascontiguousarray(packed), np.ascontiguousarray(absmax), n, blocksize, out)
    return out


def nf4_gemv2048(x: np.ndarray, packed: np.ndarray, absmax: np.ndarray, rows: int, *, bias=None, residual=None,
                 dtype: str = "bf16") -> np.ndarray:
    out = np.empty(rows, dtype=np.uint16)
    lib().kco_nf4_gemv2048(_act(dtype), np.ascontiguousarray(x), packed, absmax, _ptr(bias), _ptr(residual), rows, out)
    return out


def qkv(x, gamma, eps, q, k, v, *, dtype: str = "bf16", want_norm: bool = False):
    """Fused RMSNorm + Q/K/V + bias; q/k/v are (packed, absmax, bias) triples."""

    qo = np.empty(2048, dtype=np.uint16)
    ko = np.empty(256, dtype=np.uint16)
    vo = np.empty(256, dtype=np.uint16)
    norm = np.empty(2048, dtype=np.float32) if want_norm else None
    lib().kco_qkv(_act(dtype), x, gamma, eps, q[0], q[1], q[2], k[0], k[1], k[2], v[0], v[1], v[2], 2048, 256,
                  qo, ko, vo, _ptr(norm))
    return (qo, ko, vo, norm) if want_norm else (qo, ko, vo)


def qkv_rope_cache(x, gamma, eps, q, k, v, rope_cos, rope_sin, pos, kcache, vcache):
    qo = np.empty(2048, dtype=np.uint16)
    capacity = kcache.shape[1]
    lib().kco_qkv_rope_cache(x, gamma, eps, q[0], q[1], q[2], k[0], k[1], k[2], v[0], v[1], v[2], rope_cos, rope_sin,
                             pos, capacity, qo, kcache, vcache)
    return qo


def swiglu(x, gamma, eps, gate, up, *, rows: int = 11008, dtype: str = "bf16") -> np.ndarray:
    out = np.empty(rows, dtype=np.uint16)
    lib().kco_swiglu(_act(dtype), x, _ptr(gamma), eps, gate[0], gate[1], up[0], up[1], rows, out)
    return out


def down11008(h, packed, absmax, *, residual=None, rows: int = 2048, dtype: str = "bf16") -> np.ndarray:
    out = np.empty(rows, dtype=np.uint16)
    lib().kco_down11008(_act(dtype), np.ascontiguousarray(h), packed, absmax, _ptr(residual), rows, out)
    return out


GQA_STEP_SPLITS = 32  # split cap of the decode step's plan


def gqa_split_tokens(kv_len: int, split_cap: int) -> int:
    """Tokens per split at kv_len with at most split_cap splits (whole 32-token rounds)."""

    return int(lib().kco_gqa_split_tokens(int(kv_len), int(split_cap)))


def gqa_plan(capacity: int, split_limit: int = 0) -> tuple[int, int]:
    """(split_cap, max_splits) of the kernels for a cache of `capacity` rows."""

    plan = np.zeros(2, dtype=np.int64)
    lib().kco_gqa_plan(int(capacity), int(split_limit), plan.ctypes.data)
    return int(plan[0]), int(plan[1])


def gqa(q, kcache, vcache, kv_len: int, *, split_cap: int | None = None, split_limit: int = 0,
        scale: float | None = None, dtype: str = "bf16") -> np.ndarray:
    """Split-KV GQA decode (16 q heads, 2 kv heads, d 128), caches [2, cap, 128].

    split_cap defaults to the kernels' plan for the cache's capacity
    (split_limit as for a caller-sized workspace, GQA_STEP_SPLITS for the
    decode step); split_cap=1 is one split of every token."""

    capacity = kcache.shape[1]
    split_cap = gqa_plan(capacity, split_limit)[0] if split_cap is None else split_cap
    scale = np.float32(1.0 / math.sqrt(128.0)) if scale is None else np.float32(scale)
    qk = np.float32(scale * LOG2E_F32)
    out = np.zeros(2048, dtype=np.uint16)
    lib().kco_gqa(_act(dtype), np.ascontiguousarray(q), np.ascontiguousarray(kcache), np.ascontiguousarray(vcache),
                  capacity, kv_len, split_cap, float(qk), out)
    return out


def lm_head_argmax(x, gamma, eps, weight, *, want_logits: bool = True):
    vocab = weight.shape[0]
    logits = np.empty(vocab, dtype=np.uint16) if want_logits else None
    tok = lib().kco_lm_head_argmax(x, _ptr(gamma), eps, np.ascontiguousarray(weight), vocab, _ptr(logits))
    return int(tok), logits


def qwen2_step(num_layers: int, vocab: int, capacity: int, eps: float, layer_table: np.ndarray,
               model_table: np.ndarray) -> None:
    """One decode step over host buffers addressed by the same pointer tables
    as kudacuda_qwen2_model_create."""

    lib().kco_qwen2_step(num_layers, vocab, capacity, eps, layer_table.ctypes.data, model_table.ctypes.data)


def set_threads(n: int) -> None:
    os.environ["OMP_NUM_THREADS"] = str(n)
