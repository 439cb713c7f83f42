"""ctypes binding of libkudacuda.so (include/kudacuda.h) for the native path.

Loading fails loudly when the library is missing: the decode path has no
CPU or PyTorch fallback of its own (framework fallback lives only in the
Transformers guards of ``kudacuda_sidecar``).
"""

from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Any

PACKAGE_DIR = Path(__file__).resolve().parent
DEFAULT_LIBRARY = PACKAGE_DIR / "libkudacuda.so"

_vp = ctypes.c_void_p
_u64 = ctypes.c_uint64
_i64 = ctypes.c_int64
_f = ctypes.c_float
_i = ctypes.c_int

QWEN2_LAYER_FIELDS = (
    "input_norm", "q_packed", "q_absmax", "q_bias", "k_packed", "k_absmax", "k_bias", "v_packed", "v_absmax",
    "v_bias", "o_packed", "o_absmax", "post_norm", "gate_packed", "gate_absmax", "up_packed", "up_absmax",
    "down_packed", "down_absmax", "key_cache", "value_cache",
)
QWEN2_MODEL_FIELDS = (
    "embed", "final_norm", "rope_cos", "rope_sin", "hidden", "query", "attn", "mlp", "logits", "tokens",
    "control", "attn_partials", "attn_counters", "lm_best", "lm_counter",
)

# name -> (argtypes, restype)
SIGNATURES: dict[str, tuple[list[Any], Any]] = {
    "kudacuda_create": ([_i], _vp),
    "kudacuda_freeze": ([_vp], _i),
    "kudacuda_can_dispatch": ([_vp, ctypes.c_char_p, _i64, _i64], _i),
    "kudacuda_vector_add": ([_vp, _u64, _u64, _u64, _i64, _u64], _i),
    "kudacuda_rmsnorm": ([_vp, _u64, _u64, _u64, _i64, _i64, _f, _u64], _i),
    "kudacuda_fused_rmsnorm_qkv": ([_vp] + [_u64] * 5 + [_i64, _i64, _f, _u64], _i),
    "kudacuda_qwen2_fused_rmsnorm_qkv_nf4": ([_vp] + [_u64] * 14 + [_i64] * 5 + [_f, _u64], _i),
    "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v2": ([_vp] + [_u64] * 15 + [_i64] * 5 + [_f, _u64], _i),
    "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v3": ([_vp] + [_u64] * 15 + [_i64] * 5 + [_f, _u64], _i),
    "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_bf16": ([_vp] + [_u64] * 14 + [_i64] * 5 + [_f, _u64], _i),
    "kudacuda_qwen2_qkv_rope_cache_nf4_bf16": ([_vp] + [_u64] * 17 + [_i64] * 5 + [_f, _u64], _i),
    "kudacuda_qwen2_swiglu_nf4": ([_vp] + [_u64] * 7 + [_i64] * 4 + [_f, _u64], _i),
    "kudacuda_qwen2_swiglu_nf4_bf16": ([_vp] + [_u64] * 7 + [_i64] * 4 + [_f, _u64], _i),
    "kudacuda_qwen2_mlp_nf4_bf16": ([_vp] + [_u64] * 11 + [_i64] * 4 + [_f, _u64], _i),
    "kudacuda_nf4_gemv_bf16": ([_vp] + [_u64] * 6 + [_i64] * 4 + [_u64], _i),
    "kudacuda_nf4_gemm_bf16": ([_vp] + [_u64] * 6 + [_i64] * 4 + [_u64], _i),
    "kudacuda_nf4_gemm_swiglu_bf16": ([_vp] + [_u64] * 6 + [_i64] * 4 + [_u64], _i),
    "kudacuda_nf4_quantize": ([_vp, _u64, _i64, _i64, _i64, _u64, _u64, _u64], _i),
    "kudacuda_nf4_dequantize": ([_vp, _u64, _u64, _i64, _i64, _i64, _u64, _u64], _i),
    "kudacuda_qwen2_gqa_decode_workspace_v3": ([_vp] + [_u64] * 6 + [_i64] * 6 + [_f, _u64], _i),
    "kudacuda_qwen2_gqa_decode": ([_vp] + [_u64] * 4 + [_i64] * 6 + [_f, _u64], _i),
    "kudacuda_qwen2_gqa_decode_graph": ([_vp] + [_u64] * 4 + [_i64] * 6 + [_f, _u64, _u64], _i),
    "kudacuda_qwen2_gqa_decode_group_tiled": ([_vp] + [_u64] * 4 + [_i64] * 6 + [_f, _u64], _i),
    "kudacuda_qwen2_gqa_decode_vectorized": ([_vp] + [_u64] * 4 + [_i64] * 6 + [_f, _u64], _i),
    "kudacuda_qwen2_gqa_decode_bf16": ([_vp] + [_u64] * 4 + [_i64] * 6 + [_f, _u64], _i),
    "kudacuda_qwen2_gqa_decode_graph_bf16": ([_vp] + [_u64] * 4 + [_i64] * 6 + [_f, _u64, _u64], _i),
    "kudacuda_qwen2_gqa_decode_graph_bf16_noalloc": ([_vp] + [_u64] * 4 + [_i64] * 6 + [_f, _u64, _u64], _i),
    "kudacuda_gqa_split_chunk": ([_i64], _i64),
    "kudacuda_gqa_workspace_floats": ([_i64], _i64),
    "kudacuda_lm_head_argmax_bf16": ([_vp] + [_u64] * 5 + [_i64, _i64, _f, _u64], _i),
    "kudacuda_lm_head_workspace_floats": ([], _i64),
    "kudacuda_begin_capture": ([_vp, _u64], _i),
    "kudacuda_end_capture": ([_vp, _u64], _i),
    "kudacuda_replay_graph": ([_vp, _u64], _i),
    "kudacuda_reset_graph": ([_vp], _i),
    "kudacuda_last_error": ([_vp], ctypes.c_char_p),
    "kudacuda_destroy": ([_vp], None),
    "kudacuda_qwen2_model_create": ([_vp, _i64, _i64, _i64, _f, _vp, _vp], _vp),
    "kudacuda_qwen2_model_step": ([_vp, _u64], _i),
    "kudacuda_qwen2_model_capture": ([_vp, _u64], _i),
    "kudacuda_qwen2_model_replay": ([_vp, _i64, _u64], _i),
    "kudacuda_qwen2_model_set_position": ([_vp, _i64], _i),
    "kudacuda_qwen2_model_time_op": ([_vp, _i64, _i64, _u64, ctypes.POINTER(_f)], _i),
    "kudacuda_qwen2_prefill_workspace_bytes": ([_i64], _i64),
    "kudacuda_qwen2_model_prefill": ([_vp, _u64, _i64, _i64, _i64, _u64], _i),
    "kudacuda_qwen2_model_destroy": ([_vp], None),
}


class NativeError(RuntimeError):
    """A libkudacuda entry point returned a non-zero status."""


def load_library(path: str | Path | None = None) -> ctypes.CDLL:
    """Load libkudacuda.so and configure every exported signature."""

    library = Path(path) if path is not None else DEFAULT_LIBRARY
    if not library.exists():
        raise FileNotFoundError(
            f"libkudacuda.so not found at {library}; build it with `python -m kudacuda_amd.build`"
        )
    lib = ctypes.CDLL(str(library))
    for name, (argtypes, restype) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = restype
    return lib


class Native:
    """One frozen handle on one device plus checked calls."""

    def __init__(self, device_id: int = 0, lib: ctypes.CDLL | None = None) -> None:
        self.lib = lib or load_library()
        self.handle = self.lib.kudacuda_create(int(device_id))
        if not self.handle:
            raise NativeError("kudacuda_create returned a null handle")
        self.check(self.lib.kudacuda_freeze(self.handle), "kudacuda_freeze")

    def error(self) -> str:
        raw = self.lib.kudacuda_last_error(self.handle)
        return raw.decode("utf-8", errors="replace") if raw else ""

    def check(self, status: int, operation: str) -> None:
        if int(status) != 0:
            raise NativeError(f"{operation} failed: {self.error()}")

    def call(self, name: str, *args: Any) -> None:
        self.check(getattr(self.lib, name)(self.handle, *args), name)

    def close(self) -> None:
        if self.handle:
            self.lib.kudacuda_destroy(self.handle)
            self.handle = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
