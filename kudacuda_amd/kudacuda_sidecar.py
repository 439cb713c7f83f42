"""Python bridge to libkudacuda.so (gfx950) with the reference sidecar's API.

Mirrors reference python/kudacuda_sidecar.py: the same public names
(``KudaCudaBridge``, ``TensorContract``, ``Qwen2GqaContract``,
``patch_qwen2_attention``, ``patch_qwen2_fused_qkv``, ``patch_qwen2_swiglu``,
``prepare_qwen2_*``, ...), the same argument meaning, the same fail-closed
validation (``ValueError`` for a tensor that breaks the contract,
``NativeCudaError("<op> failed: <message>")`` for a native rejection) and the
same Transformers fallback rules.  Differences are MI355X ones: the library
is found next to this package, tactics are named for ``gfx950`` in
``manifests/mi355x-gfx950.json``, and a tactic whose contract dtype is
``bfloat16`` launches the bf16 entry points (the reference GQA and fused QKV
kernels are fp16-only).

Only the standard library is imported at module import; PyTorch and
Transformers are imported by the integration paths that need them.  The
ctypes signatures come from ``kudacuda_amd._native`` (one table for the whole
package).
"""

from __future__ import annotations

import ctypes
import json
import math
import sys
from dataclasses import dataclass, fields
from functools import wraps
from pathlib import Path
from types import MethodType
from typing import Any, Callable, Mapping, Optional

from ._native import SIGNATURES

PACKAGE_DIR = Path(__file__).resolve().parent
DEFAULT_MANIFEST = PACKAGE_DIR / "manifests" / "mi355x-gfx950.json"

DEFAULT_GQA_TACTIC = "qwen2_gqa_decode_gfx950_bf16"
DEFAULT_GQA_GRAPH_TACTIC = "qwen2_gqa_decode_gfx950_bf16_graph_v1"
DEFAULT_GQA_WORKSPACE_TACTIC = "qwen2_gqa_decode_gfx950_fp16_workspace_v3"
DEFAULT_QKV_TACTIC = "qwen2_fused_rmsnorm_qkv_gfx950_bf16_nf4_v1"
DEFAULT_QKV_V2_TACTIC = "qwen2_fused_rmsnorm_qkv_gfx950_nf4_v2"
DEFAULT_QKV_V3_TACTIC = "qwen2_fused_rmsnorm_qkv_gfx950_nf4_v3"
DEFAULT_SWIGLU_TACTIC = "qwen2_swiglu_gfx950_nf4_v1"
DEFAULT_SWIGLU_BF16_TACTIC = "qwen2_swiglu_gfx950_bf16_nf4_v1"

_HIDDEN = 2048
_Q_OUT = 2048
_KV_OUT = 256
_INTERMEDIATE = 11008
_BLOCKSIZE = 64


class NativeCudaError(RuntimeError):
    """The native library rejected a request or a launch failed."""


class CacheCommittedError(NativeCudaError):
    """Attention failed after this token was already written to the KV cache.

    The Transformers guards re-raise it instead of running the framework's
    forward: that forward would update the cache a second time and every
    later step would attend to a duplicated key/value row."""


def _normalize_cuda_handle(value: int) -> int:
    """PyTorch reports stream handles as signed integers; the ABI takes uint64."""

    return int(value) % (1 << 64)


def select_library_name(platform_name: Optional[str] = None) -> str:
    name = platform_name or sys.platform
    if name.startswith("win"):
        return "kudacuda.dll"
    return "libkudacuda.dylib" if name == "darwin" else "libkudacuda.so"


# Required top-level manifest keys and the JSON type each must have (None:
# any); the error texts name the type as the manifest schema does.
_MANIFEST_SCHEMA: tuple[tuple[str, Optional[type]], ...] = (
    ("target_arch", None),
    ("implemented_tactics", list),
    ("contracts", dict),
)
_JSON_KIND = {list: "a list", dict: "an object"}


def load_manifest(path: str | Path) -> dict[str, Any]:
    """Read a tactic manifest and check its required keys and their types."""

    manifest_path = Path(path)
    manifest = json.loads(manifest_path.read_text(encoding="utf-8"))
    if not isinstance(manifest, dict):
        raise ValueError(f"Manifest must contain a JSON object: {manifest_path}")
    absent = [key for key, _ in _MANIFEST_SCHEMA if key not in manifest]
    if absent:
        raise ValueError(f"Manifest missing required key '{absent[0]}': {manifest_path}")
    wrong = [(key, kind) for key, kind in _MANIFEST_SCHEMA if kind is not None and not isinstance(manifest[key], kind)]
    if wrong:
        key, kind = wrong[0]
        raise ValueError(f"Manifest '{key}' must be {_JSON_KIND[kind]}")
    return manifest


def _normalize_dtype(dtype: Any) -> str:
    """'torch.bfloat16' -> 'bfloat16'."""

    return str(dtype).split(".")[-1].lower()


def _shape(tensor: Any) -> tuple[int, ...]:
    return tuple(int(v) for v in getattr(tensor, "shape", ()))


def _on_device(tensor: Any) -> bool:
    # PyTorch-ROCm reports HIP tensors as is_cuda
    return bool(getattr(tensor, "is_cuda", False))


def _call_or(tensor: Any, method: str, default: Any) -> Any:
    """tensor.method() when the tensor has that method, else default."""

    bound = getattr(tensor, method, None)
    return bound() if callable(bound) else default


def _is_contiguous(tensor: Any) -> bool:
    return bool(_call_or(tensor, "is_contiguous", False))


def _rank(tensor: Any) -> int:
    return int(_call_or(tensor, "dim", -1))


def _tensor_rules(tensor: Any, *, layout: Optional[str], dtype: Optional[str], rank: Optional[int] = None,
                  count_min: Optional[int] = None, shape: Optional[tuple[int, ...]] = None):
    """The checks a contract makes of one tensor, cheapest first, as a lazy
    sequence of booleans (the caller stops at the first False).  A None
    parameter is not checked."""

    yield _on_device(tensor)
    yield layout != "contiguous" or _is_contiguous(tensor)
    yield dtype is None or _normalize_dtype(getattr(tensor, "dtype", "")) == dtype
    yield rank is None or _rank(tensor) == rank
    yield count_min is None or int(_call_or(tensor, "numel", -1)) >= count_min
    yield shape is None or _shape(tensor) == shape


def _contract_kwargs(cls: type, mapping: Mapping[str, Any], *, required: bool) -> dict[str, Any]:
    """Constructor arguments of a contract dataclass from a manifest entry: the
    text fields normalised (dtype names, lower-case layout), the rest ints;
    with required=False an absent or empty text field and an absent number
    become None."""

    text = {"dtype": _normalize_dtype, "layout": lambda v: str(v).lower()}
    out: dict[str, Any] = {}
    for field in fields(cls):
        value = mapping[field.name] if required else mapping.get(field.name)
        if field.name in text:
            out[field.name] = text[field.name](value) if (required or value) else None
        else:
            out[field.name] = None if value is None else int(value)
    return out


@dataclass(frozen=True)
class TensorContract:
    """dtype / layout / rank / exact-shape / minimum-size contract of one tactic."""

    dtype: Optional[str] = None
    layout: Optional[str] = None
    rank: Optional[int] = None
    batch_size: Optional[int] = None
    seq_len: Optional[int] = None
    count_min: Optional[int] = None

    @classmethod
    def from_mapping(cls, mapping: Mapping[str, Any]) -> "TensorContract":
        return cls(**_contract_kwargs(cls, mapping, required=False))

    def matches_shape(self, batch_size: int, seq_len: int) -> bool:
        pairs = ((self.batch_size, batch_size), (self.seq_len, seq_len))
        return all(actual > 0 and declared in (None, actual) for declared, actual in pairs)

    def matches_tensor(self, tensor: Any) -> bool:
        return tensor is None or all(
            _tensor_rules(tensor, layout=self.layout, dtype=self.dtype, rank=self.rank, count_min=self.count_min))


# the one grouped-query geometry the kernels serve: (query heads, KV heads, head_dim)
_GQA_GEOMETRY = (16, 2, 128)


@dataclass(frozen=True)
class Qwen2GqaContract:
    """Decode-only Qwen2 grouped-query attention: batch 1, one query token,
    16 query heads, 2 KV heads, head_dim 128, bounded kv_len."""

    dtype: str
    layout: str
    batch_size: int
    query_len: int
    kv_len_min: int
    kv_len_max: int
    query_heads: int
    kv_heads: int
    head_dim: int

    @classmethod
    def from_mapping(cls, mapping: Mapping[str, Any]) -> "Qwen2GqaContract":
        return cls(**_contract_kwargs(cls, mapping, required=True))

    def matches(self, batch_size: int, query_len: int, kv_len: int) -> bool:
        served = (self.query_heads, self.kv_heads, self.head_dim) == _GQA_GEOMETRY
        call = (int(batch_size), int(query_len))
        return served and call == (self.batch_size, self.query_len) and self.kv_len_min <= int(kv_len) <= self.kv_len_max

    def matches_tensor(self, tensor: Any, expected_shape: tuple[int, ...]) -> bool:
        return all(_tensor_rules(tensor, layout=self.layout, dtype=self.dtype, shape=tuple(expected_shape)))


def _qwen2_attention_dimensions(module: Any) -> tuple[int, int, int]:
    """(query heads, kv heads, head_dim): the module's own attribute where
    Transformers sets one, else its config's; head_dim falls back to
    hidden_size / heads."""

    config = getattr(module, "config", None)

    def attribute(own: str, from_config: str) -> Any:
        value = getattr(module, own, None)
        return getattr(config, from_config, 0) if value is None else value

    heads = int(attribute("num_heads", "num_attention_heads"))
    kv_heads = int(attribute("num_key_value_heads", "num_key_value_heads"))
    head_dim = getattr(module, "head_dim", None)
    if head_dim is None:
        head_dim = int(getattr(config, "hidden_size", 0)) // heads if heads else 0
    return heads, kv_heads, int(head_dim)


# positional parameters of Qwen2Attention.forward after hidden_states
_ATTENTION_POSITIONAL = ("position_embeddings", "attention_mask", "past_key_values", "cache_position")


@dataclass
class _AttentionCall:
    """One Qwen2 attention call as the dispatcher sees it: its arguments bound
    by name, the head layout, and whether the KV cache has taken the token."""

    module: Any
    hidden_states: Any
    position_embeddings: Any
    mask: Any
    cache: Any
    cache_position: Any
    output_attentions: bool
    heads: int
    kv_heads: int
    head_dim: int
    committed: bool = False

    @classmethod
    def bind(cls, module: Any, hidden_states: Any, args: tuple[Any, ...], kwargs: Mapping[str, Any]) -> "_AttentionCall":
        named = dict(zip(_ATTENTION_POSITIONAL, args))
        for name in _ATTENTION_POSITIONAL:
            if kwargs.get(name) is not None:
                named[name] = kwargs[name]
        if named.get("past_key_values") is None and kwargs.get("past_key_value") is not None:
            named["past_key_values"] = kwargs["past_key_value"]  # older Transformers spelling
        heads, kv_heads, head_dim = _qwen2_attention_dimensions(module)
        return cls(module, hidden_states, named.get("position_embeddings"), named.get("attention_mask"),
                   named.get("past_key_values"), named.get("cache_position"),
                   bool(kwargs.get("output_attentions", False)), heads, kv_heads, head_dim)

    @property
    def lead(self) -> tuple[int, ...]:
        return tuple(self.hidden_states.shape[:-1])

    def admission_refusal(self, graph_mode: bool) -> Optional[str]:
        """Why the native path cannot take this call, decided before anything
        is computed or written; ``None`` admits it."""

        shape = _shape(self.hidden_states)
        if len(shape) != 3 or shape[:2] != (1, 1):
            return f"shape:{shape}"
        if self.output_attentions:
            return "output_attentions"
        for label, value, want in (("query_heads", self.heads, 16), ("kv_heads", self.kv_heads, 2),
                                   ("head_dim", self.head_dim, 128)):
            if value != want:
                return f"{label}:{value}"
        if self.position_embeddings is None:
            return "missing_position_embeddings"
        if graph_mode and getattr(self.module, "sliding_window", None) is not None:
            return "graph_sliding_window_unsupported"
        if not graph_mode and self.mask is not None and _rank(self.mask) != 4:
            return f"attention_mask_shape:{_shape(self.mask)}"
        return None


# GQA tactic variant (name suffix) -> (fp16 symbol, bf16 symbol)
_GQA_VARIANTS = (
    ("graph_v1", "kudacuda_qwen2_gqa_decode_graph", "kudacuda_qwen2_gqa_decode_graph_bf16"),
    ("workspace_v3", "kudacuda_qwen2_gqa_decode_workspace_v3", None),
    ("group_tiled_v2", "kudacuda_qwen2_gqa_decode_group_tiled", None),
    ("vectorized_v2", "kudacuda_qwen2_gqa_decode_vectorized", None),
    ("", "kudacuda_qwen2_gqa_decode", "kudacuda_qwen2_gqa_decode_bf16"),
)


class KudaCudaBridge:
    """One native handle plus guarded pointer launches for the decode path."""

    def __init__(self, *, manifest: Mapping[str, Any] | str | Path = DEFAULT_MANIFEST,
                 lib_path: str | Path | None = None, device_id: int = 0, native_lib: Any = None) -> None:
        self.manifest = load_manifest(manifest) if isinstance(manifest, (str, Path)) else dict(manifest)
        self.implemented_tactics = frozenset(self.manifest.get("implemented_tactics", ()))
        self.experimental_tactics = frozenset(self.manifest.get("experimental_tactics", ()))
        self.planned_tactics = frozenset(self.manifest.get("planned_tactics", ()))
        raw_contracts = self.manifest.get("contracts", {})
        self.contracts = {name: TensorContract.from_mapping(c) for name, c in raw_contracts.items()}
        self.qwen_contracts = {name: Qwen2GqaContract.from_mapping(c) for name, c in raw_contracts.items()
                               if "query_heads" in c}
        self._contract_dtypes = {name: _normalize_dtype(c["dtype"]) for name, c in raw_contracts.items()
                                 if c.get("dtype")}
        self.library_path = Path(lib_path) if lib_path else None
        self.lib = native_lib if native_lib is not None else self._load_library(lib_path)
        self._symbols = self._configure_abi()
        self.native_attention_dispatcher = any(
            self._symbols.get(name) is not None for _, fp16, bf16 in _GQA_VARIANTS for name in (fp16, bf16) if name)
        self.native_attention_dispatches = 0
        self.native_fused_qkv_dispatches = 0
        self.native_fused_qkv_v2_dispatches = 0
        self.native_fused_qkv_v3_dispatches = 0
        self.native_swiglu_dispatches = 0
        self.native_swiglu_bf16_dispatches = 0
        self.native_swiglu_hook_calls = 0
        self.native_mlp_dispatches = 0
        self.native_gemv_dispatches = 0
        self.last_qwen2_dispatch_reason: Optional[str] = None
        self._graph_kv_len_device: Any = None
        self._graph_kv_capacity: Optional[int] = None
        self._graph_workspace: Any = None
        self._closed = True
        self.engine_handle = self.lib.kudacuda_create(int(device_id))
        if not self.engine_handle:
            raise NativeCudaError("kudacuda_create returned a null handle")
        self._closed = False
        self.freeze()

    # ------------------------------------------------------------ library
    def _load_library(self, lib_path: str | Path | None) -> Any:
        if lib_path is not None:
            candidates = [Path(lib_path)]
        else:
            name = select_library_name()
            candidates = [PACKAGE_DIR / name, PACKAGE_DIR.parent / name, PACKAGE_DIR.parent / "build" / name]
        for path in candidates:
            if path.exists():
                self.library_path = path
                return ctypes.CDLL(str(path))
        searched = ", ".join(str(p) for p in candidates)
        raise FileNotFoundError(f"KudaCuda native library not found; searched: {searched}")

    def _configure_abi(self) -> dict[str, Any]:
        """Attach argtypes/restype to every symbol the library exports.

        The base lifecycle symbols are required; the rest are feature-detected
        (a missing one makes its tactics 'unavailable')."""

        symbols: dict[str, Any] = {}
        for name, (argtypes, restype) in SIGNATURES.items():
            fn = getattr(self.lib, name, None)
            if fn is None:
                continue
            fn.argtypes = argtypes
            fn.restype = restype
            symbols[name] = fn
        required = ("kudacuda_create", "kudacuda_freeze", "kudacuda_can_dispatch", "kudacuda_begin_capture",
                    "kudacuda_end_capture", "kudacuda_replay_graph", "kudacuda_reset_graph", "kudacuda_last_error",
                    "kudacuda_destroy")
        missing = [name for name in required if name not in symbols]
        if missing:
            raise NativeCudaError(f"native library lacks required symbols: {', '.join(missing)}")
        return symbols

    def _symbol(self, name: Optional[str]) -> Any:
        return self._symbols.get(name) if name else None

    def _native_error(self) -> str:
        raw = self.lib.kudacuda_last_error(self.engine_handle)
        if raw is None:
            return "unknown native error"
        return raw.decode("utf-8", errors="replace") if isinstance(raw, bytes) else str(raw)

    def _raise_if_failed(self, status: int, operation: str) -> None:
        if int(status) != 0:
            raise NativeCudaError(f"{operation} failed: {self._native_error()}")

    def _ensure_open(self) -> None:
        if self._closed:
            raise NativeCudaError("KudaCuda bridge is closed")

    def freeze(self) -> None:
        self._raise_if_failed(self.lib.kudacuda_freeze(self.engine_handle), "kudacuda_freeze")

    def call(self, symbol: str, *args: Any) -> None:
        """Checked call of any handle-taking entry point by name (raw pointers)."""

        self._ensure_open()
        fn = self._symbol(symbol)
        if fn is None:
            raise NativeCudaError(f"native library does not export {symbol}")
        self._raise_if_failed(fn(self.engine_handle, *args), symbol)

    # ------------------------------------------------------------ tactics
    def _tactic_dtype(self, tactic_name: str) -> str:
        dtype = self._contract_dtypes.get(tactic_name)
        if dtype:
            return dtype
        return "bfloat16" if "_bf16" in tactic_name else "float16"

    def _tactic_enabled(self, tactic_name: str) -> bool:
        return tactic_name in self.implemented_tactics or tactic_name in self.experimental_tactics

    def _qwen_symbol(self, tactic_name: str) -> Any:
        bf16 = self._tactic_dtype(tactic_name) == "bfloat16"
        for suffix, fp16_name, bf16_name in _GQA_VARIANTS:
            if suffix in tactic_name:
                return self._symbol(bf16_name if bf16 else fp16_name)
        return None

    def _qkv_symbol(self, tactic_name: str) -> Any:
        if self._tactic_dtype(tactic_name) == "bfloat16":
            # the bf16 fused QKV has the v1 argument list (no normalized workspace)
            return None if tactic_name.endswith(("_v2", "_v3")) else self._symbol(
                "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_bf16")
        if tactic_name.endswith("_v3"):
            return self._symbol("kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v3")
        if tactic_name.endswith("_v2"):
            return self._symbol("kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v2")
        return self._symbol("kudacuda_qwen2_fused_rmsnorm_qkv_nf4")

    def _swiglu_symbol(self, tactic_name: str) -> Any:
        bf16 = "_bf16_" in tactic_name or self._tactic_dtype(tactic_name) == "bfloat16"
        return self._symbol("kudacuda_qwen2_swiglu_nf4_bf16" if bf16 else "kudacuda_qwen2_swiglu_nf4")

    def tactic_status(self, tactic_name: str) -> str:
        """'unavailable' when the library lacks the tactic's symbol, else the
        manifest's classification: implemented / experimental / planned / unknown."""

        if tactic_name.startswith("qwen2_gqa_decode_") and self._qwen_symbol(tactic_name) is None:
            return "unavailable"
        if tactic_name.startswith("qwen2_fused_rmsnorm_qkv_") and self._qkv_symbol(tactic_name) is None:
            return "unavailable"
        if tactic_name.startswith("qwen2_swiglu_") and self._swiglu_symbol(tactic_name) is None:
            return "unavailable"
        for status, names in (("implemented", self.implemented_tactics),
                              ("experimental", self.experimental_tactics),
                              ("planned", self.planned_tactics)):
            if tactic_name in names:
                return status
        return "unknown"

    def matches_contract(self, tactic_name: str, batch_size: int, seq_len: int, *, tensor: Any = None) -> bool:
        if self._closed or tactic_name not in self.implemented_tactics:
            return False
        contract = self.contracts.get(tactic_name)
        if contract is None or not contract.matches_shape(int(batch_size), int(seq_len)):
            return False
        if not contract.matches_tensor(tensor):
            return False
        return bool(self.lib.kudacuda_can_dispatch(self.engine_handle, tactic_name.encode("utf-8"),
                                                   int(batch_size), int(seq_len)))

    # ------------------------------------------------------------ tensors
    @staticmethod
    def _tensor_pointer(tensor: Any, label: str) -> int:
        data_ptr = getattr(tensor, "data_ptr", None)
        if not callable(data_ptr):
            raise ValueError(f"{label} does not expose data_ptr()")
        value = int(data_ptr())
        if value <= 0:
            raise ValueError(f"{label} has an invalid device pointer")
        return value

    @staticmethod
    def _tensor_contract_matches(tensor: Any, *, dtype: Optional[str], rank: int) -> bool:
        return (_on_device(tensor) and _is_contiguous(tensor) and _rank(tensor) == rank
                and (dtype is None or _normalize_dtype(getattr(tensor, "dtype", "")) == dtype))

    def _expect(self, tensor: Any, label: str, *, dtype: str, shape: tuple[int, ...], what: str) -> None:
        if not self._tensor_contract_matches(tensor, dtype=dtype, rank=len(shape)):
            raise ValueError(f"{label} must be contiguous device {dtype} rank-{len(shape)} ({what})")
        if _shape(tensor) != shape:
            raise ValueError(f"{label} must have shape {shape} ({what})")

    @staticmethod
    def _validate_nf4_weight(weight: Any, absmax: Any, *, expected_shape: tuple[int, int], label: str) -> int:
        """bitsandbytes Params4bit layout: packed uint8 (N*K/2, 1) plus a
        non-nested quant_state (nf4, blocksize 64) with fp32 absmax [N*K/64]
        (reference python/kudacuda_sidecar.py:1018-1049)."""

        state = getattr(weight, "quant_state", None)
        if state is None:
            raise ValueError(f"{label} is missing quant_state")
        if str(getattr(state, "quant_type", "")) != "nf4":
            raise ValueError(f"{label} quant_type must be nf4")
        blocksize = int(getattr(state, "blocksize", 0))
        if blocksize != _BLOCKSIZE:
            raise ValueError(f"{label} blocksize must be {_BLOCKSIZE}")
        if bool(getattr(state, "nested", False)):
            raise ValueError(f"{label} nested quantization is unsupported")
        if tuple(int(v) for v in getattr(state, "shape", ())) != tuple(expected_shape):
            raise ValueError(f"{label} logical shape must be {tuple(expected_shape)}")
        count = expected_shape[0] * expected_shape[1]
        if not KudaCudaBridge._tensor_contract_matches(weight, dtype="uint8", rank=2):
            raise ValueError(f"{label} packed storage must be contiguous device uint8")
        if _shape(weight) != ((count + 1) // 2, 1):
            raise ValueError(f"{label} packed shape must be {((count + 1) // 2, 1)}")
        if not KudaCudaBridge._tensor_contract_matches(absmax, dtype="float32", rank=1):
            raise ValueError(f"{label} absmax must be contiguous device float32")
        blocks = (count + blocksize - 1) // blocksize
        if int(absmax.numel()) != blocks:
            raise ValueError(f"{label} absmax must contain {blocks} blocks")
        return blocksize

    # ------------------------------------------------------------ basic ops
    def vector_add(self, a: Any, b: Any, output: Any, *, stream_ptr: int) -> None:
        self._ensure_open()
        contract = self.contracts.get("vector_add")
        if "vector_add" not in self.implemented_tactics or contract is None:
            raise NativeCudaError("vector_add is not implemented by this manifest")
        for label, tensor in (("a", a), ("b", b), ("output", output)):
            if not contract.matches_tensor(tensor):
                raise ValueError(f"{label} does not satisfy the vector_add device contract")
        sizes = [int(t.numel()) for t in (a, b, output)]
        if len(set(sizes)) != 1:
            raise ValueError(f"vector_add tensors must have equal sizes, got {sizes}")
        status = self.lib.kudacuda_vector_add(self.engine_handle, self._tensor_pointer(a, "a"),
                                              self._tensor_pointer(b, "b"), self._tensor_pointer(output, "output"),
                                              sizes[0], _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, "kudacuda_vector_add")

    def rmsnorm(self, input_tensor: Any, weight: Any, output: Any, *, epsilon: float = 1.0e-5,
                stream_ptr: int) -> None:
        self._ensure_open()
        contract = self.contracts.get("rmsnorm")
        if "rmsnorm" not in self.implemented_tactics or contract is None:
            raise NativeCudaError("rmsnorm is not implemented by this manifest")
        if not contract.matches_tensor(input_tensor) or not contract.matches_tensor(output):
            raise ValueError("input and output do not satisfy the RMSNorm device contract")
        if not self._tensor_contract_matches(weight, dtype=contract.dtype, rank=1):
            raise ValueError("weight does not satisfy the RMSNorm device contract")
        shape = _shape(input_tensor)
        if len(shape) != 2 or _shape(output) != shape:
            raise ValueError("RMSNorm input and output must have the same 2D shape")
        if _shape(weight) != (shape[1],):
            raise ValueError("RMSNorm weight must match the input hidden dimension")
        if epsilon <= 0.0:
            raise ValueError("epsilon must be positive")
        status = self.lib.kudacuda_rmsnorm(self.engine_handle, self._tensor_pointer(input_tensor, "input"),
                                           self._tensor_pointer(weight, "weight"),
                                           self._tensor_pointer(output, "output"), shape[0], shape[1],
                                           float(epsilon), _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, "kudacuda_rmsnorm")

    def fused_rmsnorm_qkv(self, input_tensor: Any, norm_weight: Any, qkv_weight: Any, bias: Any, output: Any, *,
                          epsilon: float = 1.0e-5, stream_ptr: int) -> None:
        """Dense fp16 RMSNorm + QKV (reference include/kudacuda.h:50)."""

        self._ensure_open()
        fn = self._symbol("kudacuda_fused_rmsnorm_qkv")
        if fn is None:
            raise NativeCudaError("native library does not export kudacuda_fused_rmsnorm_qkv")
        for label, tensor, rank in (("input", input_tensor, 2), ("norm_weight", norm_weight, 1),
                                    ("qkv_weight", qkv_weight, 2), ("bias", bias, 1), ("output", output, 2)):
            if not self._tensor_contract_matches(tensor, dtype="float16", rank=rank):
                raise ValueError(f"{label} does not satisfy the fused RMSNorm-QKV device contract")
        rows, hidden = _shape(input_tensor)
        if _shape(norm_weight) != (hidden,):
            raise ValueError("norm_weight must match the input hidden dimension")
        if _shape(qkv_weight) != (3 * hidden, hidden):
            raise ValueError("qkv_weight must have shape (3 * hidden, hidden)")
        if _shape(bias) != (3 * hidden,):
            raise ValueError("bias must have shape (3 * hidden,)")
        if _shape(output) != (rows, 3 * hidden):
            raise ValueError("output must have shape (rows, 3 * hidden)")
        if epsilon <= 0.0:
            raise ValueError("epsilon must be positive")
        status = fn(self.engine_handle, self._tensor_pointer(input_tensor, "input"),
                    self._tensor_pointer(norm_weight, "norm_weight"), self._tensor_pointer(qkv_weight, "qkv_weight"),
                    self._tensor_pointer(bias, "bias"), self._tensor_pointer(output, "output"), rows, hidden,
                    float(epsilon), _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, "kudacuda_fused_rmsnorm_qkv")

    # ------------------------------------------------------------ attention
    def _gqa_checks(self, tactic_name: str, tensors: tuple[Any, Any, Any, Any], cache_len: int,
                    what: str) -> Qwen2GqaContract:
        contract = self.qwen_contracts.get(tactic_name)
        if contract is None:
            raise NativeCudaError(f"{tactic_name} has no Qwen2 GQA contract in this manifest")
        shapes = ((1, contract.query_heads, 1, contract.head_dim),
                  (1, contract.kv_heads, int(cache_len), contract.head_dim),
                  (1, contract.kv_heads, int(cache_len), contract.head_dim),
                  (1, contract.query_heads, 1, contract.head_dim))
        for label, tensor, shape in zip(("query", "key_cache", "value_cache", "output"), tensors, shapes):
            if not contract.matches_tensor(tensor, shape):
                raise ValueError(f"{label} does not satisfy the Qwen2 {what} device contract")
        return contract

    def _check_kv_len_device(self, kv_len_device: Any, what: str) -> None:
        if not self._tensor_contract_matches(kv_len_device, dtype="int32", rank=1):
            raise ValueError(f"kv_len_device does not satisfy the Qwen2 {what} device contract")
        if _shape(kv_len_device) != (1,):
            raise ValueError("kv_len_device must have shape (1,)")

    def dispatch_qwen2_gqa_decode(self, query: Any, key_cache: Any, value_cache: Any, output: Any, *, kv_len: int,
                                  stream_ptr: int, tactic_name: str = DEFAULT_GQA_TACTIC) -> None:
        """Decode attention over a cache of exactly kv_len rows
        (reference include/kudacuda.h:192)."""

        self._ensure_open()
        if "graph_v1" in tactic_name:
            raise NativeCudaError("graph tactic requires an active static decode graph context")
        if not self._tactic_enabled(tactic_name) or tactic_name not in self.qwen_contracts:
            raise NativeCudaError(f"{tactic_name} is not implemented by this manifest")
        fn = self._qwen_symbol(tactic_name)
        if fn is None:
            raise NativeCudaError(f"native library does not export the {tactic_name} dispatcher")
        contract = self.qwen_contracts[tactic_name]
        if not contract.matches(1, 1, kv_len):
            raise ValueError(f"Qwen2 GQA decode contract does not accept kv_len={kv_len}")
        self._gqa_checks(tactic_name, (query, key_cache, value_cache, output), kv_len, "GQA")
        status = fn(self.engine_handle, self._tensor_pointer(query, "query"),
                    self._tensor_pointer(key_cache, "key_cache"), self._tensor_pointer(value_cache, "value_cache"),
                    self._tensor_pointer(output, "output"), 1, 1, int(kv_len), contract.query_heads,
                    contract.kv_heads, contract.head_dim, 1.0 / math.sqrt(contract.head_dim),
                    _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, tactic_name)
        self.native_attention_dispatches += 1

    def _graph_capacity_limit(self) -> int:
        limits = [c.kv_len_max for name, c in self.qwen_contracts.items() if "graph_v1" in name]
        return max(limits) if limits else 512

    def configure_qwen2_graph_dispatch(self, *, kv_len_device: Any, kv_capacity: int, workspace: Any = None) -> None:
        """Arm graph-mode attention: kv_len is read from device memory at replay."""

        if self._symbol("kudacuda_qwen2_gqa_decode_graph") is None and \
                self._symbol("kudacuda_qwen2_gqa_decode_graph_bf16") is None:
            raise NativeCudaError("native library does not export kudacuda_qwen2_gqa_decode_graph")
        limit = self._graph_capacity_limit()
        if not 1 <= int(kv_capacity) <= limit:
            raise ValueError(f"kv_capacity must be in the range 1..{limit}")
        self._graph_kv_len_device = kv_len_device
        self._graph_kv_capacity = int(kv_capacity)
        self._graph_workspace = workspace

    def clear_qwen2_graph_dispatch(self) -> None:
        self._graph_kv_len_device = None
        self._graph_kv_capacity = None
        self._graph_workspace = None

    def dispatch_qwen2_gqa_decode_workspace(self, query: Any, key_cache: Any, value_cache: Any, output: Any, *,
                                            kv_capacity: int, kv_len_device: Any, workspace: Any, stream_ptr: int,
                                            tactic_name: str = DEFAULT_GQA_WORKSPACE_TACTIC) -> None:
        """fp16 two-stage split-KV with a caller workspace of >= 16*8*130 floats
        (reference include/kudacuda.h:174)."""

        self._ensure_open()
        fn = self._qwen_symbol(tactic_name) if "workspace_v3" in tactic_name else None
        if tactic_name not in self.qwen_contracts or fn is None:
            raise NativeCudaError(f"{tactic_name} workspace contract or dispatcher is unavailable")
        if not self._tactic_enabled(tactic_name):
            raise NativeCudaError(f"{tactic_name} is not enabled by this manifest")
        if int(kv_capacity) != 512:
            raise ValueError("workspace GQA requires kv_capacity=512")
        contract = self._gqa_checks(tactic_name, (query, key_cache, value_cache, output), kv_capacity, "workspace")
        self._check_kv_len_device(kv_len_device, "workspace")
        need = contract.query_heads * 8 * (2 + contract.head_dim)
        if not self._tensor_contract_matches(workspace, dtype="float32", rank=1):
            raise ValueError("workspace does not satisfy the Qwen2 workspace device contract")
        if int(workspace.numel()) < need:
            raise ValueError(f"workspace must contain at least {need} float32 values")
        status = fn(self.engine_handle, self._tensor_pointer(query, "query"),
                    self._tensor_pointer(key_cache, "key_cache"), self._tensor_pointer(value_cache, "value_cache"),
                    self._tensor_pointer(output, "output"), self._tensor_pointer(workspace, "workspace"),
                    self._tensor_pointer(kv_len_device, "kv_len_device"), 1, 1, int(kv_capacity),
                    contract.query_heads, contract.kv_heads, contract.head_dim, 1.0 / math.sqrt(contract.head_dim),
                    _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, tactic_name)
        self.native_attention_dispatches += 1

    def dispatch_qwen2_gqa_decode_graph(self, query: Any, key_cache: Any, value_cache: Any, output: Any, *,
                                        kv_capacity: int, kv_len_device: Any, stream_ptr: int,
                                        tactic_name: str = DEFAULT_GQA_GRAPH_TACTIC) -> None:
        """Capture-safe attention over a cache of kv_capacity rows whose valid
        length is read from kv_len_device at run time (reference include/kudacuda.h:208)."""

        self._ensure_open()
        fn = self._qwen_symbol(tactic_name) if "graph_v1" in tactic_name else None
        if tactic_name not in self.qwen_contracts or fn is None:
            raise NativeCudaError(f"{tactic_name} graph contract or dispatcher is unavailable")
        contract = self._gqa_checks(tactic_name, (query, key_cache, value_cache, output), kv_capacity, "graph")
        self._check_kv_len_device(kv_len_device, "graph")
        args = (self.engine_handle, self._tensor_pointer(query, "query"),
                self._tensor_pointer(key_cache, "key_cache"), self._tensor_pointer(value_cache, "value_cache"),
                self._tensor_pointer(output, "output"), 1, 1, int(kv_capacity), contract.query_heads,
                contract.kv_heads, contract.head_dim, 1.0 / math.sqrt(contract.head_dim),
                self._tensor_pointer(kv_len_device, "kv_len_device"), _normalize_cuda_handle(stream_ptr))
        try:
            status = fn(*args)
        except (OverflowError, ctypes.ArgumentError) as error:
            raise NativeCudaError(f"graph dispatcher argument conversion failed: {args}") from error
        self._raise_if_failed(status, tactic_name)
        self.native_attention_dispatches += 1

    def dispatch_qwen2_attention(self, module: Any, hidden_states: Any, *args: Any,
                                 tactic_name: str = DEFAULT_GQA_TACTIC, **kwargs: Any) -> Any:
        """Qwen2 decode attention through the native kernel, or ``None`` so the
        caller runs the framework's own forward.

        The division of work is the reference's (python/kudacuda_sidecar.py:
        767-958): Transformers keeps the projections (unless the fused QKV
        hook pre-computed them), rotary embedding, the cache update and
        o_proj, and the native kernel runs attention over the materialised
        contiguous cache.  The call runs in two phases:

        * admission, free of side effects: token shape, head layout, rotary
          inputs, mask rank and the graph-mode limits.  A refusal returns
          ``None`` and the framework forward runs as if no hook existed;
        * execution: projections, rotary, then the cache update.  From that
          update on the cache holds this token, so the call always returns
          the layer's attention output -- from the native kernel when the
          cache and mask allow it, otherwise from the framework's eager
          softmax on the same tensors (reason prefixed
          ``framework_fallback:``).  When even that fails it raises
          ``CacheCommittedError``, which the guards pass on instead of
          re-running the forward (that would append the token twice).

        The reason of the last decision is left in ``last_qwen2_dispatch_reason``.
        """

        import torch

        self.last_qwen2_dispatch_reason = "started"
        call = _AttentionCall.bind(module, hidden_states, args, kwargs)
        graph_mode = (("graph_v1" in tactic_name or "workspace_v3" in tactic_name)
                      and self._graph_kv_len_device is not None and self._graph_kv_capacity is not None)
        refusal = call.admission_refusal(graph_mode)
        if refusal is not None:
            self.last_qwen2_dispatch_reason = refusal
            return None

        try:
            from transformers.models.qwen2.modeling_qwen2 import apply_rotary_pos_emb

            query, key, value = self._qwen2_projections(module, hidden_states, call.lead)
            cos, sin = call.position_embeddings
            query, key = apply_rotary_pos_emb(query, key, cos, sin)
        except Exception as error:  # nothing is written yet: the framework can redo it all
            self.last_qwen2_dispatch_reason = f"exception:{type(error).__name__}:{error}"
            return None
        if call.cache is not None:
            call.committed = True  # a failing update may already have appended
            try:
                key, value = self._qwen2_cache_update(module, call.cache, key, value, cos, sin, call.cache_position)
            except Exception as error:
                raise CacheCommittedError(f"KV cache update failed: {type(error).__name__}: {error}") from error

        route = self._attention_route(torch, call, query, key, value, graph_mode)
        if route.startswith("decline:"):
            self.last_qwen2_dispatch_reason = route[len("decline:"):]
            return None
        if route == "native":
            try:
                if graph_mode:
                    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
                context = self._attention_native(torch, hidden_states, query, key, value, tactic_name, graph_mode)
                self.last_qwen2_dispatch_reason = "native"
                return module.o_proj(context.transpose(1, 2).reshape(*call.lead, -1).contiguous()), None
            except Exception as error:
                if graph_mode:  # a capture must not silently record framework attention
                    if call.committed:
                        raise CacheCommittedError(f"native graph attention failed: {error}") from error
                    raise
                route = f"framework_fallback:native_exception:{type(error).__name__}:{error}"
        self.last_qwen2_dispatch_reason = route
        try:
            return self._qwen2_eager_attention(torch, module, query, key, value, call.mask, call.lead,
                                               call.heads // call.kv_heads, call.head_dim)
        except Exception as error:
            if not call.committed:
                self.last_qwen2_dispatch_reason = f"exception:{type(error).__name__}:{error}"
                return None
            raise CacheCommittedError(f"attention after the cache update failed ({route}): {error}") from error

    def _attention_route(self, torch: Any, call: "_AttentionCall", query: Any, key: Any, value: Any,
                         graph_mode: bool) -> str:
        """``"native"`` when the native kernel can take the materialised
        tensors, else the reason the framework's eager softmax runs instead."""

        if key.dim() != 4 or tuple(value.shape) != tuple(key.shape):
            return f"framework_fallback:cache_shape:{tuple(key.shape)}:{tuple(value.shape)}"
        kv_len = int(key.shape[-2])
        if graph_mode:
            if kv_len != self._graph_kv_capacity:
                return f"framework_fallback:graph_cache_capacity:{kv_len}:{self._graph_kv_capacity}"
            return "native"
        mask = call.mask
        if mask is not None:
            if int(mask.shape[-1]) != kv_len:
                reason = f"attention mask covers {int(mask.shape[-1])} keys but the cache holds {kv_len}"
                if call.committed:
                    raise CacheCommittedError(reason)
                return f"decline:mask_length:{reason}"  # nothing written: the framework forward can run
            if not bool(torch.all(mask == 0)):
                return "framework_fallback:attention_mask_values"
        if not (query.is_contiguous() and key.is_contiguous()):
            return f"framework_fallback:non_contiguous:q={query.stride()}:k={key.stride()}"
        return "native"

    def _attention_native(self, torch: Any, hidden_states: Any, query: Any, key: Any, value: Any, tactic_name: str,
                          graph_mode: bool) -> Any:
        """Launch the tactic's GQA entry point; returns [1, 16, 1, 128] like ``query``."""

        output = torch.empty_like(query)
        stream_ptr = int(torch.cuda.current_stream(hidden_states.device).cuda_stream)
        capacity = int(self._graph_kv_capacity or 0)
        if "workspace_v3" in tactic_name:
            if self._graph_workspace is None:
                raise NativeCudaError("workspace GQA tactic requires a configured workspace")
            self.dispatch_qwen2_gqa_decode_workspace(query, key, value, output, kv_capacity=capacity,
                                                     kv_len_device=self._graph_kv_len_device,
                                                     workspace=self._graph_workspace, stream_ptr=stream_ptr,
                                                     tactic_name=tactic_name)
        elif graph_mode:
            self.dispatch_qwen2_gqa_decode_graph(query, key, value, output, kv_capacity=capacity,
                                                 kv_len_device=self._graph_kv_len_device, stream_ptr=stream_ptr,
                                                 tactic_name=tactic_name)
        else:
            self.dispatch_qwen2_gqa_decode(query, key, value, output, kv_len=int(key.shape[-2]),
                                           stream_ptr=stream_ptr, tactic_name=tactic_name)
        return output

    @staticmethod
    def _qwen2_projections(module: Any, hidden_states: Any, lead: tuple[int, ...]) -> tuple[Any, Any, Any]:
        view = (*lead, -1, module.head_dim)
        prefused = getattr(module, "_kudacuda_prefused_qkv", None)
        if prefused is not None:
            flat = prefused
        else:
            flat = (module.q_proj(hidden_states), module.k_proj(hidden_states), module.v_proj(hidden_states))
        return tuple(t.view(view).transpose(1, 2) for t in flat)  # type: ignore[return-value]

    @staticmethod
    def _qwen2_cache_update(module: Any, cache: Any, key: Any, value: Any, cos: Any, sin: Any,
                            cache_position: Any) -> tuple[Any, Any]:
        extra = {"sin": sin, "cos": cos}
        if cache_position is not None:
            extra["cache_position"] = cache_position
        try:
            return cache.update(key, value, module.layer_idx, extra)
        except TypeError:
            return cache.update(key, value, module.layer_idx)

    @staticmethod
    def _qwen2_eager_attention(torch: Any, module: Any, query: Any, key: Any, value: Any, mask: Any,
                               lead: tuple[int, ...], group: int, head_dim: int) -> Any:
        """Framework softmax attention (reference python/kudacuda_sidecar.py:871-885):
        fp32 scores and softmax, result in the query dtype.  Products run in
        fp32 on contiguous operands."""

        k = key.repeat_interleave(group, dim=1).float()
        v = value.repeat_interleave(group, dim=1).float()
        scale = float(getattr(module, "scaling", 1.0 / math.sqrt(head_dim)))
        scores = torch.matmul(query.float(), k.transpose(-1, -2).contiguous()) * scale
        if mask is not None:
            scores = scores + mask.float()
        probs = torch.softmax(scores, dim=-1, dtype=torch.float32).to(query.dtype).float()
        context = torch.matmul(probs, v).to(query.dtype)
        context = context.transpose(1, 2).reshape(*lead, -1).contiguous()
        return module.o_proj(context), None

    # ------------------------------------------------------------ NF4 QKV
    def dispatch_qwen2_fused_rmsnorm_qkv_nf4(self, input_tensor: Any, norm_weight: Any, q_weight: Any, q_absmax: Any,
                                             q_bias: Any, k_weight: Any, k_absmax: Any, k_bias: Any, v_weight: Any,
                                             v_absmax: Any, v_bias: Any, q_output: Any, k_output: Any,
                                             v_output: Any, *, normalized_workspace: Any = None,
                                             epsilon: float = 1.0e-5, stream_ptr: int,
                                             tactic_name: str = DEFAULT_QKV_TACTIC) -> None:
        """RMSNorm + NF4 Q/K/V + bias for Qwen2.5-3B (reference include/kudacuda.h:63,88,114).

        v2/v3 tactics also write the fp32 normalised input to
        ``normalized_workspace``; a bfloat16 tactic launches the bf16 entry point."""

        self._ensure_open()
        fn = self._qkv_symbol(tactic_name)
        if fn is None:
            raise NativeCudaError("native library does not export the requested NF4 fused QKV ABI")
        if not self._tactic_enabled(tactic_name):
            raise NativeCudaError(f"{tactic_name} is not enabled by this manifest")
        dtype = self._tactic_dtype(tactic_name)
        tiled = tactic_name.endswith(("_v2", "_v3"))
        what = "NF4 fused QKV"
        if not self._tensor_contract_matches(input_tensor, dtype=dtype, rank=2):
            raise ValueError(f"input must be contiguous device {dtype} rank-2")
        if not self._tensor_contract_matches(norm_weight, dtype=dtype, rank=1):
            raise ValueError(f"norm_weight must be contiguous device {dtype} rank-1")
        if _shape(input_tensor) != (1, _HIDDEN) or _shape(norm_weight) != (_HIDDEN,):
            raise ValueError("NF4 fused QKV requires input (1, 2048) and norm_weight (2048,)")
        self._validate_nf4_weight(q_weight, q_absmax, expected_shape=(_Q_OUT, _HIDDEN), label="q_weight")
        for label, bias, n in (("q_bias", q_bias, _Q_OUT), ("k_bias", k_bias, _KV_OUT), ("v_bias", v_bias, _KV_OUT)):
            self._expect(bias, label, dtype=dtype, shape=(n,), what=what)
        self._validate_nf4_weight(k_weight, k_absmax, expected_shape=(_KV_OUT, _HIDDEN), label="k_weight")
        self._validate_nf4_weight(v_weight, v_absmax, expected_shape=(_KV_OUT, _HIDDEN), label="v_weight")
        for label, tensor, n in (("q_output", q_output, _Q_OUT), ("k_output", k_output, _KV_OUT),
                                 ("v_output", v_output, _KV_OUT)):
            self._expect(tensor, label, dtype=dtype, shape=(1, n), what=what)
        if tiled:
            self._expect(normalized_workspace, "normalized_workspace", dtype="float32", shape=(1, _HIDDEN),
                         what=what)
        if epsilon <= 0.0:
            raise ValueError("epsilon must be positive")
        ptr = self._tensor_pointer
        args = [self.engine_handle, ptr(input_tensor, "input"), ptr(norm_weight, "norm_weight"),
                ptr(q_weight, "q_weight"), ptr(q_absmax, "q_absmax"), ptr(q_bias, "q_bias"),
                ptr(k_weight, "k_weight"), ptr(k_absmax, "k_absmax"), ptr(k_bias, "k_bias"),
                ptr(v_weight, "v_weight"), ptr(v_absmax, "v_absmax"), ptr(v_bias, "v_bias")]
        if tiled:
            args.append(ptr(normalized_workspace, "normalized_workspace"))
        args += [ptr(q_output, "q_output"), ptr(k_output, "k_output"), ptr(v_output, "v_output"),
                 1, _HIDDEN, _Q_OUT, _KV_OUT, _BLOCKSIZE, float(epsilon), _normalize_cuda_handle(stream_ptr)]
        self._raise_if_failed(fn(*args), tactic_name)
        self.native_fused_qkv_dispatches += 1
        if tactic_name.endswith("_v2"):
            self.native_fused_qkv_v2_dispatches += 1
        elif tactic_name.endswith("_v3"):
            self.native_fused_qkv_v3_dispatches += 1

    def dispatch_qwen2_fused_rmsnorm_qkv_nf4_v2(self, *tensors: Any, normalized_workspace: Any,
                                                epsilon: float = 1.0e-5, stream_ptr: int,
                                                tactic_name: str = DEFAULT_QKV_V2_TACTIC) -> None:
        self.dispatch_qwen2_fused_rmsnorm_qkv_nf4(*tensors, normalized_workspace=normalized_workspace,
                                                  epsilon=epsilon, stream_ptr=stream_ptr, tactic_name=tactic_name)

    def dispatch_qwen2_fused_rmsnorm_qkv_nf4_v3(self, *tensors: Any, normalized_workspace: Any,
                                                epsilon: float = 1.0e-5, stream_ptr: int,
                                                tactic_name: str = DEFAULT_QKV_V3_TACTIC) -> None:
        self.dispatch_qwen2_fused_rmsnorm_qkv_nf4(*tensors, normalized_workspace=normalized_workspace,
                                                  epsilon=epsilon, stream_ptr=stream_ptr, tactic_name=tactic_name)

    def dispatch_qwen2_qkv_rope_cache_nf4_bf16(self, input_tensor: Any, norm_weight: Any, q_weight: Any,
                                               q_absmax: Any, q_bias: Any, k_weight: Any, k_absmax: Any,
                                               k_bias: Any, v_weight: Any, v_absmax: Any, v_bias: Any,
                                               rope_cos: Any, rope_sin: Any, position_device: Any, q_output: Any,
                                               key_cache: Any, value_cache: Any, *, epsilon: float = 1.0e-6,
                                               stream_ptr: int) -> None:
        """RMSNorm + QKV + bias + RoPE with k/v written into [2, capacity, 128]
        caches at the device-resident position (no reference counterpart: the
        reference leaves RoPE and the cache write to Transformers)."""

        self._ensure_open()
        fn = self._symbol("kudacuda_qwen2_qkv_rope_cache_nf4_bf16")
        if fn is None:
            raise NativeCudaError("native library does not export kudacuda_qwen2_qkv_rope_cache_nf4_bf16")
        what = "QKV+RoPE+cache"
        self._expect(input_tensor, "input", dtype="bfloat16", shape=(1, _HIDDEN), what=what)
        self._expect(norm_weight, "norm_weight", dtype="bfloat16", shape=(_HIDDEN,), what=what)
        self._validate_nf4_weight(q_weight, q_absmax, expected_shape=(_Q_OUT, _HIDDEN), label="q_weight")
        self._validate_nf4_weight(k_weight, k_absmax, expected_shape=(_KV_OUT, _HIDDEN), label="k_weight")
        self._validate_nf4_weight(v_weight, v_absmax, expected_shape=(_KV_OUT, _HIDDEN), label="v_weight")
        for label, bias, n in (("q_bias", q_bias, _Q_OUT), ("k_bias", k_bias, _KV_OUT), ("v_bias", v_bias, _KV_OUT)):
            self._expect(bias, label, dtype="bfloat16", shape=(n,), what=what)
        cache_shape = _shape(key_cache)
        if len(cache_shape) != 4 or cache_shape[:2] != (1, 2) or cache_shape[3] != 128:
            raise ValueError("key_cache must have shape (1, 2, capacity, 128)")
        capacity = cache_shape[2]
        self._expect(key_cache, "key_cache", dtype="bfloat16", shape=cache_shape, what=what)
        self._expect(value_cache, "value_cache", dtype="bfloat16", shape=cache_shape, what=what)
        self._expect(rope_cos, "rope_cos", dtype="float32", shape=(capacity, 64), what=what)
        self._expect(rope_sin, "rope_sin", dtype="float32", shape=(capacity, 64), what=what)
        self._check_kv_len_device(position_device, what)
        self._expect(q_output, "q_output", dtype="bfloat16", shape=(1, _Q_OUT), what=what)
        if epsilon <= 0.0:
            raise ValueError("epsilon must be positive")
        ptr = self._tensor_pointer
        status = fn(self.engine_handle, ptr(input_tensor, "input"), ptr(norm_weight, "norm_weight"),
                    ptr(q_weight, "q_weight"), ptr(q_absmax, "q_absmax"), ptr(q_bias, "q_bias"),
                    ptr(k_weight, "k_weight"), ptr(k_absmax, "k_absmax"), ptr(k_bias, "k_bias"),
                    ptr(v_weight, "v_weight"), ptr(v_absmax, "v_absmax"), ptr(v_bias, "v_bias"),
                    ptr(rope_cos, "rope_cos"), ptr(rope_sin, "rope_sin"), ptr(position_device, "position_device"),
                    ptr(q_output, "q_output"), ptr(key_cache, "key_cache"), ptr(value_cache, "value_cache"),
                    capacity, _HIDDEN, _Q_OUT, _KV_OUT, _BLOCKSIZE, float(epsilon),
                    _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, "kudacuda_qwen2_qkv_rope_cache_nf4_bf16")
        self.native_fused_qkv_dispatches += 1

    # ------------------------------------------------------------ NF4 MLP
    def _swiglu(self, fn: Any, dtype: str, input_tensor: Any, norm_weight: Any, gate_weight: Any, gate_absmax: Any,
                up_weight: Any, up_absmax: Any, output: Any, epsilon: float, stream_ptr: int,
                tactic_name: str) -> None:
        what = "NF4 SwiGLU"
        if not self._tensor_contract_matches(input_tensor, dtype=dtype, rank=2):
            raise ValueError(f"input must be contiguous device {dtype} rank-2")
        if not self._tensor_contract_matches(norm_weight, dtype=dtype, rank=1):
            raise ValueError(f"norm_weight must be contiguous device {dtype} rank-1")
        if _shape(input_tensor) != (1, _HIDDEN) or _shape(norm_weight) != (_HIDDEN,):
            raise ValueError(f"{what} requires input (1, 2048) and norm_weight (2048,)")
        for label, w, a in (("gate_weight", gate_weight, gate_absmax), ("up_weight", up_weight, up_absmax)):
            self._validate_nf4_weight(w, a, expected_shape=(_INTERMEDIATE, _HIDDEN), label=label)
        self._expect(output, "output", dtype=dtype, shape=(1, _INTERMEDIATE), what=what)
        if epsilon <= 0.0:
            raise ValueError("epsilon must be positive")
        ptr = self._tensor_pointer
        status = fn(self.engine_handle, ptr(input_tensor, "input"), ptr(norm_weight, "norm_weight"),
                    ptr(gate_weight, "gate_weight"), ptr(gate_absmax, "gate_absmax"), ptr(up_weight, "up_weight"),
                    ptr(up_absmax, "up_absmax"), ptr(output, "output"), 1, _HIDDEN, _INTERMEDIATE, _BLOCKSIZE,
                    float(epsilon), _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, tactic_name)
        self.native_swiglu_dispatches += 1

    def dispatch_qwen2_swiglu_nf4(self, input_tensor: Any, norm_weight: Any, gate_weight: Any, gate_absmax: Any,
                                  up_weight: Any, up_absmax: Any, output: Any, *, epsilon: float = 1.0e-5,
                                  stream_ptr: int, tactic_name: str = DEFAULT_SWIGLU_TACTIC) -> None:
        """fp16 silu(gate(norm x)) * up(norm x) (reference include/kudacuda.h:140)."""

        self._ensure_open()
        fn = self._symbol("kudacuda_qwen2_swiglu_nf4")
        if fn is None:
            raise NativeCudaError("native library does not export the NF4 SwiGLU ABI")
        if not self._tactic_enabled(tactic_name):
            raise NativeCudaError(f"{tactic_name} is not enabled by this manifest")
        self._swiglu(fn, "float16", input_tensor, norm_weight, gate_weight, gate_absmax, up_weight, up_absmax,
                     output, epsilon, stream_ptr, tactic_name)

    def dispatch_qwen2_swiglu_nf4_bf16(self, input_tensor: Any, norm_weight: Any, gate_weight: Any,
                                       gate_absmax: Any, up_weight: Any, up_absmax: Any, output: Any, *,
                                       epsilon: float = 1.0e-6, stream_ptr: int,
                                       tactic_name: str = DEFAULT_SWIGLU_BF16_TACTIC) -> None:
        """bf16 twin of the SwiGLU (reference include/kudacuda.h:157)."""

        self._ensure_open()
        fn = self._symbol("kudacuda_qwen2_swiglu_nf4_bf16")
        if fn is None:
            raise NativeCudaError("native library does not export the BF16 NF4 SwiGLU ABI")
        if not self._tactic_enabled(tactic_name):
            raise NativeCudaError(f"{tactic_name} is not enabled by this manifest")
        self._swiglu(fn, "bfloat16", input_tensor, norm_weight, gate_weight, gate_absmax, up_weight, up_absmax,
                     output, epsilon, stream_ptr, tactic_name)
        self.native_swiglu_bf16_dispatches += 1

    def dispatch_qwen2_mlp_nf4_bf16(self, input_tensor: Any, norm_weight: Any, gate_weight: Any, gate_absmax: Any,
                                    up_weight: Any, up_absmax: Any, down_weight: Any, down_absmax: Any,
                                    intermediate_workspace: Any, output: Any, *, residual: Any = None,
                                    epsilon: float = 1.0e-6, stream_ptr: int) -> None:
        """Whole MLP: output = [residual +] down(silu(gate(n)) * up(n)), n the
        RMSNorm of input (no reference counterpart: the reference runs the down
        projection through bitsandbytes, python/kudacuda_sidecar.py:1746)."""

        self._ensure_open()
        fn = self._symbol("kudacuda_qwen2_mlp_nf4_bf16")
        if fn is None:
            raise NativeCudaError("native library does not export kudacuda_qwen2_mlp_nf4_bf16")
        what = "NF4 MLP"
        self._expect(input_tensor, "input", dtype="bfloat16", shape=(1, _HIDDEN), what=what)
        self._expect(norm_weight, "norm_weight", dtype="bfloat16", shape=(_HIDDEN,), what=what)
        for label, w, a in (("gate_weight", gate_weight, gate_absmax), ("up_weight", up_weight, up_absmax)):
            self._validate_nf4_weight(w, a, expected_shape=(_INTERMEDIATE, _HIDDEN), label=label)
        self._validate_nf4_weight(down_weight, down_absmax, expected_shape=(_HIDDEN, _INTERMEDIATE),
                                  label="down_weight")
        self._expect(intermediate_workspace, "intermediate_workspace", dtype="bfloat16", shape=(1, _INTERMEDIATE),
                     what=what)
        self._expect(output, "output", dtype="bfloat16", shape=(1, _HIDDEN), what=what)
        if residual is not None:
            self._expect(residual, "residual", dtype="bfloat16", shape=(1, _HIDDEN), what=what)
        if epsilon <= 0.0:
            raise ValueError("epsilon must be positive")
        ptr = self._tensor_pointer
        status = fn(self.engine_handle, ptr(input_tensor, "input"), ptr(norm_weight, "norm_weight"),
                    ptr(gate_weight, "gate_weight"), ptr(gate_absmax, "gate_absmax"), ptr(up_weight, "up_weight"),
                    ptr(up_absmax, "up_absmax"), ptr(down_weight, "down_weight"), ptr(down_absmax, "down_absmax"),
                    ptr(intermediate_workspace, "intermediate_workspace"),
                    0 if residual is None else ptr(residual, "residual"), ptr(output, "output"), 1, _HIDDEN,
                    _INTERMEDIATE, _BLOCKSIZE, float(epsilon), _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, "kudacuda_qwen2_mlp_nf4_bf16")
        self.native_mlp_dispatches += 1

    def dispatch_nf4_gemv_bf16(self, input_tensor: Any, weight: Any, absmax: Any, output: Any, *, bias: Any = None,
                               residual: Any = None, stream_ptr: int) -> None:
        """y = [residual +] bf16(W x [+ bias]) for a [N, 2048] NF4 weight."""

        self._ensure_open()
        fn = self._symbol("kudacuda_nf4_gemv_bf16")
        if fn is None:
            raise NativeCudaError("native library does not export kudacuda_nf4_gemv_bf16")
        state = getattr(weight, "quant_state", None)
        logical = tuple(int(v) for v in getattr(state, "shape", ())) if state is not None else ()
        if len(logical) != 2 or logical[1] != _HIDDEN:
            raise ValueError("NF4 GEMV weight must have logical shape (N, 2048)")
        rows = logical[0]
        self._validate_nf4_weight(weight, absmax, expected_shape=(rows, _HIDDEN), label="weight")
        what = "NF4 GEMV"
        self._expect(input_tensor, "input", dtype="bfloat16", shape=(1, _HIDDEN), what=what)
        self._expect(output, "output", dtype="bfloat16", shape=(1, rows), what=what)
        if bias is not None:
            self._expect(bias, "bias", dtype="bfloat16", shape=(rows,), what=what)
        if residual is not None:
            self._expect(residual, "residual", dtype="bfloat16", shape=(1, rows), what=what)
        ptr = self._tensor_pointer
        status = fn(self.engine_handle, ptr(input_tensor, "input"), ptr(weight, "weight"), ptr(absmax, "absmax"),
                    0 if bias is None else ptr(bias, "bias"), 0 if residual is None else ptr(residual, "residual"),
                    ptr(output, "output"), 1, _HIDDEN, rows, _BLOCKSIZE, _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, "kudacuda_nf4_gemv_bf16")
        self.native_gemv_dispatches += 1

    def lm_head_argmax_bf16(self, input_tensor: Any, norm_weight: Any, weight: Any, argmax_out: Any, *,
                            logits: Any = None, epsilon: float = 1.0e-6, stream_ptr: int) -> None:
        """Greedy token of RMSNorm(x) against a bf16 [vocab, 2048] table, on
        device (the handle owns the cross-block scratch)."""

        self._ensure_open()
        fn = self._symbol("kudacuda_lm_head_argmax_bf16")
        if fn is None:
            raise NativeCudaError("native library does not export kudacuda_lm_head_argmax_bf16")
        what = "lm_head argmax"
        self._expect(input_tensor, "input", dtype="bfloat16", shape=(1, _HIDDEN), what=what)
        if norm_weight is not None:
            self._expect(norm_weight, "norm_weight", dtype="bfloat16", shape=(_HIDDEN,), what=what)
        wshape = _shape(weight)
        if len(wshape) != 2 or wshape[1] != _HIDDEN:
            raise ValueError("weight must have shape (vocab, 2048)")
        self._expect(weight, "weight", dtype="bfloat16", shape=wshape, what=what)
        self._expect(argmax_out, "argmax_out", dtype="int32", shape=(1,), what=what)
        if logits is not None:
            self._expect(logits, "logits", dtype="bfloat16", shape=(1, wshape[0]), what=what)
        ptr = self._tensor_pointer
        status = fn(self.engine_handle, ptr(input_tensor, "input"),
                    0 if norm_weight is None else ptr(norm_weight, "norm_weight"), ptr(weight, "weight"),
                    0 if logits is None else ptr(logits, "logits"), ptr(argmax_out, "argmax_out"), wshape[0],
                    _HIDDEN, float(epsilon), _normalize_cuda_handle(stream_ptr))
        self._raise_if_failed(status, "kudacuda_lm_head_argmax_bf16")

    # ------------------------------------------------------------ graphs
    def begin_capture(self, *, stream_ptr: int) -> None:
        self._raise_if_failed(self.lib.kudacuda_begin_capture(self.engine_handle, _normalize_cuda_handle(stream_ptr)),
                              "kudacuda_begin_capture")

    def end_capture(self, *, stream_ptr: int) -> None:
        self._raise_if_failed(self.lib.kudacuda_end_capture(self.engine_handle, _normalize_cuda_handle(stream_ptr)),
                              "kudacuda_end_capture")

    def replay_graph(self, *, stream_ptr: int) -> None:
        self._raise_if_failed(self.lib.kudacuda_replay_graph(self.engine_handle, _normalize_cuda_handle(stream_ptr)),
                              "kudacuda_replay_graph")

    def reset_graph(self) -> None:
        self._raise_if_failed(self.lib.kudacuda_reset_graph(self.engine_handle), "kudacuda_reset_graph")

    # ------------------------------------------------------------ lifetime
    def shutdown(self) -> None:
        if not self._closed:
            self.lib.kudacuda_destroy(self.engine_handle)
            self._closed = True
            self.engine_handle = None

    def __enter__(self) -> "KudaCudaBridge":
        return self

    def __exit__(self, exc_type: Any, exc_value: Any, traceback: Any) -> None:
        self.shutdown()

    def __del__(self) -> None:
        try:
            self.shutdown()
        except Exception:
            pass


# ---------------------------------------------------------------- Transformers
def _swap_forward(cls: Any, replacement: Callable[..., Any]) -> Callable[[], None]:
    """Install ``replacement`` as ``cls.forward``; return an idempotent undo."""

    original = cls.forward
    cls.forward = replacement
    done = [False]

    def unpatch() -> None:
        if not done[0]:
            cls.forward = original
            done[0] = True

    return unpatch


def patch_llama_attention(bridge: Any, *, attention_cls: Any = None,
                          tactic_name: str = "gqa8_attn") -> Callable[[], None]:
    """Guarded Llama attention hook (reference python/kudacuda_sidecar.py:1471-1521):
    only a bridge exposing ``dispatch_attention`` and an implemented contract
    takes the call; everything else runs the original forward."""

    if attention_cls is None:
        from transformers.models.llama.modeling_llama import LlamaAttention

        attention_cls = LlamaAttention
    original = attention_cls.forward

    @wraps(original)
    def guarded_forward(self: Any, hidden_states: Any, *args: Any, **kwargs: Any) -> Any:
        try:
            shape = _shape(hidden_states)
            dispatcher = getattr(bridge, "dispatch_attention", None)
            if (len(shape) >= 2 and callable(dispatcher)
                    and bridge.matches_contract(tactic_name, shape[0], shape[1], tensor=hidden_states)):
                return dispatcher(self, hidden_states, *args, **kwargs)
        except Exception:
            pass
        return original(self, hidden_states, *args, **kwargs)

    return _swap_forward(attention_cls, guarded_forward)


def patch_qwen2_attention(bridge: Any, *, attention_cls: Any = None,
                          tactic_name: str = DEFAULT_GQA_TACTIC) -> Callable[[], None]:
    """Route Qwen2 attention through ``bridge.dispatch_qwen2_attention`` with
    framework fallback (reference python/kudacuda_sidecar.py:1524-1561)."""

    if attention_cls is None:
        from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention

        attention_cls = Qwen2Attention
    original = attention_cls.forward

    @wraps(original)
    def guarded_forward(self: Any, hidden_states: Any, *args: Any, **kwargs: Any) -> Any:
        try:
            dispatcher = getattr(bridge, "dispatch_qwen2_attention", None)
            if len(_shape(hidden_states)) >= 2 and callable(dispatcher):
                result = dispatcher(self, hidden_states, *args, tactic_name=tactic_name, **kwargs)
                if result is not None:
                    return result
        except CacheCommittedError:
            raise  # the cache already holds this token: running the forward again would duplicate it
        except Exception:
            pass
        return original(self, hidden_states, *args, **kwargs)

    return _swap_forward(attention_cls, guarded_forward)


def _decoder_layers(model: Any) -> list[Any]:
    layers = getattr(getattr(model, "model", None), "layers", None)
    if layers is None:
        raise ValueError("Qwen2 model does not expose model.layers")
    return list(layers)


def prepare_qwen2_fused_qkv(model: Any, *, torch_module: Any = None) -> None:
    """Give every decoder layer's attention fixed Q/K/V (and fp32 normalised)
    buffers, allocated before graph capture so replays see stable addresses."""

    if torch_module is None:
        import torch as torch_module
    for layer in _decoder_layers(model):
        attention = getattr(layer, "self_attn", None)
        norm_weight = getattr(getattr(layer, "input_layernorm", None), "weight", None)
        if attention is None or norm_weight is None:
            raise ValueError("Qwen2 decoder layer is missing self_attn or input_layernorm")
        device = getattr(norm_weight, "device", None)
        dtype = getattr(norm_weight, "dtype", None)
        if device is None or dtype is None:
            raise ValueError("Qwen2 input layernorm weight has no device/dtype")
        attention._kudacuda_fused_qkv_state = {
            "normalized": torch_module.empty((1, _HIDDEN), device=device, dtype=torch_module.float32),
            "query": torch_module.empty((1, _Q_OUT), device=device, dtype=dtype),
            "key": torch_module.empty((1, _KV_OUT), device=device, dtype=dtype),
            "value": torch_module.empty((1, _KV_OUT), device=device, dtype=dtype),
        }


def prepare_qwen2_swiglu(model: Any, *, torch_module: Any = None) -> None:
    """Give every decoder layer a fixed [1, 11008] SwiGLU output buffer."""

    if torch_module is None:
        import torch as torch_module
    for layer in _decoder_layers(model):
        norm_weight = getattr(getattr(layer, "post_attention_layernorm", None), "weight", None)
        if getattr(layer, "mlp", None) is None or norm_weight is None:
            raise ValueError("Qwen2 decoder layer is missing mlp or post-attention layernorm")
        layer._kudacuda_swiglu_state = {
            "output": torch_module.empty((1, _INTERMEDIATE), device=norm_weight.device, dtype=norm_weight.dtype),
        }


def _current_stream(torch_module: Any, device: Any) -> int:
    if torch_module is None:
        import torch as torch_module
    return int(torch_module.cuda.current_stream(device).cuda_stream)


_MISSING = object()


def _restore_attr(obj: Any, name: str, previous: Any) -> None:
    if previous is _MISSING:
        if hasattr(obj, name):
            try:
                delattr(obj, name)
            except AttributeError:
                pass
    else:
        setattr(obj, name, previous)


def patch_qwen2_swiglu(model: Any, bridge: Any, *, tactic_name: str = DEFAULT_SWIGLU_TACTIC, prepare: bool = True,
                       torch_module: Any = None) -> Callable[[], None]:
    """Decoder-layer hook: the post-attention RMSNorm + gate/up + SiLU*up run
    natively, the down projection and residuals stay in the framework
    (reference python/kudacuda_sidecar.py:1624-1782)."""

    layers = _decoder_layers(model)
    if not layers:
        raise ValueError("Qwen2 model does not expose decoder layers")
    dispatch = (bridge.dispatch_qwen2_swiglu_nf4_bf16 if "_bf16_" in tactic_name
                else bridge.dispatch_qwen2_swiglu_nf4)
    saved = [(layer, layer.forward, getattr(layer, "_kudacuda_swiglu_state", _MISSING)) for layer in layers]
    if prepare:
        prepare_qwen2_swiglu(model, torch_module=torch_module)

    def make_forward(layer: Any, original: Any) -> Callable[..., Any]:
        def swiglu_forward(self: Any, hidden_states: Any, attention_mask: Any = None, position_ids: Any = None,
                           past_key_values: Any = None, use_cache: Any = False, position_embeddings: Any = None,
                           **kwargs: Any) -> Any:
            call = dict(attention_mask=attention_mask, position_ids=position_ids, past_key_values=past_key_values,
                        use_cache=use_cache, position_embeddings=position_embeddings, **kwargs)
            bridge.native_swiglu_hook_calls = int(getattr(bridge, "native_swiglu_hook_calls", 0)) + 1
            shape = _shape(hidden_states)
            if shape != (1, 1, _HIDDEN):
                bridge.last_swiglu_dispatch_reason = f"shape:{shape}"
                return original(hidden_states, **call)
            state = getattr(layer, "_kudacuda_swiglu_state", None)
            if not isinstance(state, dict) or "output" not in state:
                bridge.last_swiglu_dispatch_reason = "missing_workspace"
                return original(hidden_states, **call)
            residual = None
            try:
                attn_out, _ = layer.self_attn(hidden_states=layer.input_layernorm(hidden_states), **call)
                residual = hidden_states + attn_out

                def framework_mlp() -> Any:
                    return residual + layer.mlp(layer.post_attention_layernorm(residual))

                flat = residual.reshape(1, _HIDDEN)
                if not bool(flat.is_contiguous()):
                    bridge.last_swiglu_dispatch_reason = "non_contiguous_input"
                    return framework_mlp()
                gate, up = layer.mlp.gate_proj, layer.mlp.up_proj
                g_state = getattr(gate.weight, "quant_state", None)
                u_state = getattr(up.weight, "quant_state", None)
                if g_state is None or u_state is None:
                    bridge.last_swiglu_dispatch_reason = "missing_quant_state"
                    return framework_mlp()
                if getattr(gate, "bias", None) is not None or getattr(up, "bias", None) is not None:
                    bridge.last_swiglu_dispatch_reason = "unexpected_projection_bias"
                    return framework_mlp()
                norm = layer.post_attention_layernorm
                dispatch(flat, norm.weight, gate.weight, g_state.absmax, up.weight, u_state.absmax, state["output"],
                         epsilon=float(getattr(norm, "variance_epsilon", 1.0e-6)),
                         stream_ptr=_current_stream(torch_module, flat.device), tactic_name=tactic_name)
                bridge.last_swiglu_dispatch_reason = "native"
                return residual + layer.mlp.down_proj(state["output"].reshape(1, 1, _INTERMEDIATE))
            except CacheCommittedError:
                raise
            except Exception as error:
                bridge.last_swiglu_dispatch_reason = f"fallback:{type(error).__name__}:{error}"
                if residual is not None:
                    return residual + layer.mlp(layer.post_attention_layernorm(residual))
                return original(hidden_states, **call)

        return swiglu_forward

    for layer, original, _ in saved:
        layer.forward = MethodType(make_forward(layer, original), layer)
    done = [False]

    def unpatch() -> None:
        if done[0]:
            return
        for layer, original, previous in saved:
            layer.forward = original
            _restore_attr(layer, "_kudacuda_swiglu_state", previous)
        done[0] = True

    return unpatch


def patch_qwen2_fused_qkv(model: Any, bridge: Any, *, tactic_name: str = DEFAULT_QKV_TACTIC,
                          attention_tactic_name: str = DEFAULT_GQA_TACTIC, prepare: bool = True,
                          torch_module: Any = None, attention_cls: Any = None) -> Callable[[], None]:
    """Decoder-layer hook: input RMSNorm + NF4 Q/K/V + bias run natively into
    fixed buffers that the attention hook then consumes
    (reference python/kudacuda_sidecar.py:1785-1952).  Anything off-contract
    runs the original decoder layer unchanged."""

    layers = _decoder_layers(model)
    if not layers:
        raise ValueError("Qwen2 model does not expose decoder layers")
    if attention_cls is None:
        attention_cls = type(layers[0].self_attn)
    # snapshot before prepare so unpatch also removes the buffers it created
    saved = [(layer, layer.forward, getattr(layer.self_attn, "_kudacuda_fused_qkv_state", _MISSING),
              getattr(layer.self_attn, "_kudacuda_prefused_qkv", _MISSING)) for layer in layers]
    if prepare:
        prepare_qwen2_fused_qkv(model, torch_module=torch_module)
    attention_unpatch = patch_qwen2_attention(bridge, attention_cls=attention_cls, tactic_name=attention_tactic_name)

    def make_forward(layer: Any, original: Any) -> Callable[..., Any]:
        attention = layer.self_attn

        def fused_forward(self: Any, hidden_states: Any, *args: Any, **kwargs: Any) -> Any:
            bridge.native_fused_qkv_hook_calls = int(getattr(bridge, "native_fused_qkv_hook_calls", 0)) + 1
            shape = _shape(hidden_states)
            if shape != (1, 1, _HIDDEN):
                if int(getattr(bridge, "native_fused_qkv_dispatches", 0)) == 0:
                    bridge.last_qwen2_fused_qkv_dispatch_reason = f"shape:{shape}"
                return original(hidden_states, *args, **kwargs)
            state = getattr(attention, "_kudacuda_fused_qkv_state", None)
            if not isinstance(state, dict) or not all(k in state for k in ("query", "key", "value")):
                bridge.last_qwen2_fused_qkv_dispatch_reason = "missing_workspace"
                return original(hidden_states, *args, **kwargs)
            previous = getattr(attention, "_kudacuda_prefused_qkv", _MISSING)
            try:
                flat = hidden_states.reshape(1, _HIDDEN)
                if not bool(flat.is_contiguous()):
                    bridge.last_qwen2_fused_qkv_dispatch_reason = "non_contiguous_input"
                    return original(hidden_states, *args, **kwargs)
                projections = (attention.q_proj, attention.k_proj, attention.v_proj)
                quant = [getattr(p.weight, "quant_state", None) for p in projections]
                if any(q is None for q in quant):
                    bridge.last_qwen2_fused_qkv_dispatch_reason = "missing_quant_state"
                    return original(hidden_states, *args, **kwargs)
                biases = [getattr(p, "bias", None) for p in projections]
                if any(b is None for b in biases):
                    bridge.last_qwen2_fused_qkv_dispatch_reason = "missing_projection_bias"
                    return original(hidden_states, *args, **kwargs)
                norm = layer.input_layernorm
                bridge.dispatch_qwen2_fused_rmsnorm_qkv_nf4(
                    flat, norm.weight,
                    projections[0].weight, quant[0].absmax, biases[0],
                    projections[1].weight, quant[1].absmax, biases[1],
                    projections[2].weight, quant[2].absmax, biases[2],
                    state["query"], state["key"], state["value"],
                    normalized_workspace=state.get("normalized"),
                    epsilon=float(getattr(norm, "variance_epsilon", 1.0e-6)),
                    stream_ptr=_current_stream(torch_module, hidden_states.device), tactic_name=tactic_name)
                bridge.last_qwen2_fused_qkv_dispatch_reason = "native"
                attention._kudacuda_prefused_qkv = (state["query"], state["key"], state["value"])
                out = attention(hidden_states, *args, **kwargs)
            except CacheCommittedError:
                raise
            except Exception as error:
                bridge.last_qwen2_fused_qkv_dispatch_reason = f"fallback:{type(error).__name__}:{error}"
                return original(hidden_states, *args, **kwargs)
            finally:
                _restore_attr(attention, "_kudacuda_prefused_qkv", previous)
            # the attention (and its cache update) has run: finish the layer in
            # the framework, never by re-running the whole forward
            residual = hidden_states + (out[0] if isinstance(out, tuple) else out)
            return residual + layer.mlp(layer.post_attention_layernorm(residual))

        return fused_forward

    for layer, original, _, _ in saved:
        layer.forward = MethodType(make_forward(layer, original), layer)
    done = [False]

    def unpatch() -> None:
        if done[0]:
            return
        for layer, original, prev_state, prev_prefused in saved:
            layer.forward = original
            _restore_attr(layer.self_attn, "_kudacuda_fused_qkv_state", prev_state)
            _restore_attr(layer.self_attn, "_kudacuda_prefused_qkv", prev_prefused)
        attention_unpatch()
        done[0] = True

    return unpatch
