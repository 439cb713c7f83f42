"""Fixed-shape whole-forward graph capture for Qwen2 decode.

Mirrors reference python/kudacuda_static_decode.py:85-447.  A
``GraphStaticCache`` holds one fixed-capacity K/V tensor pair per layer and a
device-resident write position, so one captured decode forward stays valid
for every later token; ``StaticDecodeGraphRunner`` captures that forward
(torch's HIP graph when a capture stream is given, else the bridge's native
capture), then replays it after copying the next token, position and kv_len
into the captured buffers.  Replays are refused unless every pointer, shape,
the stream and the model fingerprint match the capture.
"""

from __future__ import annotations

from contextlib import nullcontext
from dataclasses import dataclass
from typing import Any, Mapping, Optional

from .kudacuda_graph_plan import DecodeGraphKey, GraphContractError


def _shape(value: Any) -> tuple[int, ...]:
    return tuple(int(v) for v in getattr(value, "shape", ()))


def _pointer(value: Any, label: str) -> int:
    data_ptr = getattr(value, "data_ptr", None)
    if not callable(data_ptr):
        raise GraphContractError(f"{label} does not expose data_ptr()")
    address = int(data_ptr())
    if address <= 0:
        raise GraphContractError(f"{label} has an invalid device pointer")
    return address


def _clone_value(torch_module: Any, value: Any) -> Any:
    """Deep copy of nested tensors (mappings, lists, tuples kept as such)."""

    if isinstance(value, Mapping):
        return {k: _clone_value(torch_module, v) for k, v in value.items()}
    if isinstance(value, (list, tuple)):
        items = [_clone_value(torch_module, v) for v in value]
        return tuple(items) if isinstance(value, tuple) else items
    clone = getattr(value, "clone", None)
    return clone() if callable(clone) else value


def _tensor_records(value: Any, out: list[tuple[int, tuple[int, ...]]]) -> None:
    """(pointer, shape) of every tensor in a nested value, mapping keys sorted."""

    if isinstance(value, Mapping):
        for key in sorted(value, key=str):
            _tensor_records(value[key], out)
    elif isinstance(value, (list, tuple)):
        for item in value:
            _tensor_records(item, out)
    elif callable(getattr(value, "data_ptr", None)) and getattr(value, "shape", None) is not None:
        out.append((_pointer(value, "graph tensor"), _shape(value)))


def _cache_layers(cache: Any) -> list[Any]:
    layers = getattr(cache, "layers", None)
    if layers is not None:
        return list(layers)
    keys, values = getattr(cache, "key_cache", None), getattr(cache, "value_cache", None)
    return list(zip(keys, values)) if keys is not None and values is not None else []


def _layer_tensors(cache: Any, index: int) -> tuple[Any, Any]:
    layer = _cache_layers(cache)[index]
    if isinstance(layer, tuple) and len(layer) == 2:
        return layer
    key = getattr(layer, "keys", None)
    if key is None:
        key = getattr(layer, "key_cache", None)
    value = getattr(layer, "values", None)
    if value is None:
        value = getattr(layer, "value_cache", None)
    if key is None or value is None:
        raise GraphContractError(f"cache layer {index} has no key/value tensors")
    return key, value


class GraphStaticCache:
    """Per-layer [batch, kv_heads, max_cache_len, head_dim] K/V with the write
    position held in a device tensor (``cache_position``)."""

    def __init__(self, *, key_cache: list[Any], value_cache: list[Any], cache_position: Any, sequence_length: int,
                 max_cache_len: int) -> None:
        self.key_cache = key_cache
        self.value_cache = value_cache
        self.cache_position = cache_position
        self._sequence_length = int(sequence_length)
        self.max_cache_len = int(max_cache_len)
        self.layers = list(zip(self.key_cache, self.value_cache))

    @classmethod
    def from_dynamic_cache(cls, torch_module: Any, dynamic_cache: Any, *, max_cache_len: int) -> "GraphStaticCache":
        """Copy a prefilled framework cache into zero-padded fixed-capacity tensors."""

        count = len(_cache_layers(dynamic_cache))
        if count == 0:
            raise GraphContractError("dynamic cache does not expose cache layers")
        keys: list[Any] = []
        values: list[Any] = []
        for index in range(count):
            key, value = _layer_tensors(dynamic_cache, index)
            if key.dim() != 4 or value.shape != key.shape:
                raise GraphContractError(f"cache layer {index} is not a rank-4 KV pair")
            length = int(key.shape[-2])
            if length > int(max_cache_len):
                raise GraphContractError("max_cache_len is smaller than the prefetched cache")
            shape = (int(key.shape[0]), int(key.shape[1]), int(max_cache_len), int(key.shape[3]))
            for source, sink in ((key, keys), (value, values)):
                target = torch_module.zeros(shape, dtype=source.dtype, device=source.device)
                target[..., :length, :].copy_(source)
                sink.append(target)
        length = int(dynamic_cache.get_seq_length())
        position = torch_module.tensor([length], dtype=torch_module.long, device=keys[0].device)
        return cls(key_cache=keys, value_cache=values, cache_position=position, sequence_length=length,
                   max_cache_len=max_cache_len)

    def update(self, key_states: Any, value_states: Any, layer_idx: int, *args: Any,
               **kwargs: Any) -> tuple[Any, Any]:
        del args, kwargs
        if int(key_states.shape[-2]) != int(self.cache_position.numel()):
            raise GraphContractError("graph cache position count does not match key update length")
        self.key_cache[layer_idx].index_copy_(2, self.cache_position, key_states)
        self.value_cache[layer_idx].index_copy_(2, self.cache_position, value_states)
        return self.key_cache[layer_idx], self.value_cache[layer_idx]

    def get_seq_length(self, layer_idx: int = 0) -> int:
        del layer_idx
        return self._sequence_length

    def get_max_length(self, layer_idx: int = 0) -> int:
        del layer_idx
        return self.max_cache_len

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return self.get_max_length(layer_idx)

    def __len__(self) -> int:
        return len(self.key_cache)


@dataclass(frozen=True)
class StaticDecodeContract:
    key: DecodeGraphKey
    stream_ptr: int
    logical_kv_len: int


class StaticDecodeGraphRunner:
    """Capture one whole decode forward of a model and replay it by pointer identity."""

    def __init__(self, bridge: Any, model: Any, torch_module: Any) -> None:
        self.bridge = bridge
        self.model = model
        self.torch = torch_module
        self.contract: Optional[StaticDecodeContract] = None
        self.static_inputs: dict[str, Any] = {}
        self.cache: Any = None
        self.kv_len_device: Any = None
        self.logits: Any = None
        self.status = "not-requested"
        self.reason: Optional[str] = None
        self.capture_ms: Optional[float] = None
        self.replay_count = 0
        self.backend = "native"
        self.cuda_graph: Any = None
        self.workspace: Any = None

    @property
    def captured(self) -> bool:
        return self.contract is not None and self.status == "captured"

    def _update_static_attention_mask(self, valid_kv_len: int) -> None:
        """Mask cache slots >= valid_kv_len for the framework attention path
        (the native kernels read kv_len_device instead)."""

        masks = self.static_inputs.get("attention_mask")
        finfo = getattr(self.torch, "finfo", None)
        if not isinstance(masks, Mapping) or not callable(finfo):
            return
        for mask in masks.values():
            shape = _shape(mask)
            if not shape or not callable(getattr(mask, "fill_", None)):
                continue
            try:
                lowest = finfo(getattr(mask, "dtype", None)).min
            except (TypeError, ValueError, RuntimeError):
                continue
            valid = max(0, min(int(valid_kv_len), shape[-1]))
            mask.fill_(0.0)
            if valid < shape[-1]:
                mask[..., valid:].fill_(lowest)

    @staticmethod
    def model_fingerprint(model: Any) -> str:
        config = getattr(model, "config", None)
        parts = [type(model).__name__] + [str(getattr(config, name, "")) for name in
                                          ("model_type", "num_hidden_layers", "hidden_size", "vocab_size",
                                           "torch_dtype")]
        return "|".join(parts)

    def _layer_count(self) -> int:
        count = getattr(getattr(self.model, "config", None), "num_hidden_layers", None)
        if count is not None:
            return int(count)
        layers = getattr(getattr(self.model, "model", None), "layers", None)
        return len(layers) if layers is not None else 0

    def _key(self, *, tactic_name: str, device_id: int, kv_bucket: int) -> DecodeGraphKey:
        records: list[tuple[int, tuple[int, ...]]] = []
        _tensor_records(self.static_inputs, records)
        _tensor_records(self.cache.key_cache, records)
        _tensor_records(self.cache.value_cache, records)
        records.append((_pointer(self.kv_len_device, "kv_len_device"), _shape(self.kv_len_device)))
        input_ids = self.static_inputs["input_ids"]
        return DecodeGraphKey(
            device_id=int(device_id), tactic_name=tactic_name, layer_count=self._layer_count(),
            query_shape=_shape(input_ids), key_shape=_shape(self.cache.key_cache[0]),
            value_shape=_shape(self.cache.value_cache[0]),
            output_shape=_shape(self.logits) if self.logits is not None else (), kv_bucket=int(kv_bucket),
            pointers=tuple(p for p, _ in records), model_fingerprint=self.model_fingerprint(self.model),
            dtype=str(getattr(input_ids, "dtype", "")),
            quantization=str(getattr(getattr(self.model, "config", None), "quantization_config", "")))

    def _device_scalar(self, value: int, dtype: Any, device: Any) -> Any:
        return self.torch.tensor([int(value)], dtype=dtype, device=device)

    def capture(self, *, input_ids: Any, position_ids: Any, attention_mask: Any, cache_position: Any,
                past_key_values: GraphStaticCache, logical_kv_len: int, kv_bucket: int, tactic_name: str,
                stream_ptr: int, stream: Any = None, device_id: int = 0,
                model_kwargs: Mapping[str, Any] | None = None, workspace: Any = None) -> Any:
        """Record one decode forward at position ``logical_kv_len`` (the cache
        then holds logical_kv_len + 1 tokens) and run it once."""

        if self.captured:
            raise GraphContractError("graph runner already has a captured forward")
        self.static_inputs = {
            "input_ids": _clone_value(self.torch, input_ids),
            "position_ids": _clone_value(self.torch, position_ids),
            "attention_mask": _clone_value(self.torch, attention_mask),
            "cache_position": cache_position,
        }
        valid = int(logical_kv_len) + 1
        self._update_static_attention_mask(valid)
        self.cache = past_key_values
        self.kv_len_device = self._device_scalar(valid, self.torch.int32, input_ids.device)
        if hasattr(self.bridge, "configure_qwen2_graph_dispatch"):
            self.bridge.configure_qwen2_graph_dispatch(kv_len_device=self.kv_len_device, kv_capacity=int(kv_bucket),
                                                       workspace=workspace)
        self.workspace = workspace
        self.cache.cache_position.copy_(self._device_scalar(logical_kv_len, self.torch.long,
                                                            self.cache.cache_position.device))
        cuda = getattr(self.torch, "cuda", None)
        use_torch_graph = (stream is not None and hasattr(cuda, "CUDAGraph") and callable(getattr(cuda, "graph", None)))
        self.backend = "torch_cuda_graph" if use_torch_graph else "native"
        self.bridge.reset_graph()
        try:
            kwargs = dict(model_kwargs or {})
            kwargs.update(input_ids=self.static_inputs["input_ids"], position_ids=self.static_inputs["position_ids"],
                          attention_mask=self.static_inputs["attention_mask"], past_key_values=self.cache,
                          cache_position=self.static_inputs["cache_position"], use_cache=True, return_dict=True)
            inference_mode = getattr(self.torch, "inference_mode", None)
            context = inference_mode() if callable(inference_mode) else nullcontext()
            if use_torch_graph:
                self.cuda_graph = cuda.CUDAGraph()
                with cuda.graph(self.cuda_graph, stream=stream):
                    with context:
                        outputs = self.model(**kwargs)
                # capture records the work without running it
                self.cuda_graph.replay()
            else:
                self.bridge.begin_capture(stream_ptr=int(stream_ptr))
                with context:
                    outputs = self.model(**kwargs)
            self.logits = getattr(outputs, "logits", None)
            if self.logits is None:
                raise GraphContractError("model decode output does not expose logits")
            if not use_torch_graph:
                self.bridge.end_capture(stream_ptr=int(stream_ptr))
                self.bridge.replay_graph(stream_ptr=int(stream_ptr))
            self.replay_count = 1
        except Exception as error:
            try:
                self.bridge.reset_graph()
            finally:
                if hasattr(self.bridge, "clear_qwen2_graph_dispatch"):
                    self.bridge.clear_qwen2_graph_dispatch()
            self.status = "fallback"
            self.reason = f"capture_failed:{type(error).__name__}:{error}"
            raise GraphContractError(self.reason) from error
        finally:
            if hasattr(self.bridge, "clear_qwen2_graph_dispatch"):
                self.bridge.clear_qwen2_graph_dispatch()
        self.contract = StaticDecodeContract(key=self._key(tactic_name=tactic_name, device_id=device_id,
                                                           kv_bucket=kv_bucket),
                                             stream_ptr=int(stream_ptr), logical_kv_len=valid)
        self.status = "captured"
        self.reason = None
        return self.logits

    def replay(self, *, next_token: Any, position_ids: Any, cache_position: int, logical_kv_len: int,
               stream_ptr: int) -> Any:
        """Run the captured forward for the token at ``cache_position``."""

        if not self.captured or self.contract is None:
            raise GraphContractError("graph runner has no captured forward")
        if int(stream_ptr) != self.contract.stream_ptr:
            raise GraphContractError("graph replay stream changed")
        valid = int(logical_kv_len) + 1
        if valid > self.contract.key.kv_bucket:
            raise GraphContractError("graph replay KV length exceeds the captured bucket")
        if _shape(next_token) != _shape(self.static_inputs["input_ids"]):
            raise GraphContractError("graph replay token shape changed")
        if _shape(position_ids) != _shape(self.static_inputs["position_ids"]):
            raise GraphContractError("graph replay position shape changed")
        key = self.contract.key
        if self._key(tactic_name=key.tactic_name, device_id=key.device_id, kv_bucket=key.kv_bucket) != key:
            raise GraphContractError("graph replay pointer, shape, or model contract changed")
        self.static_inputs["input_ids"].copy_(next_token)
        self.static_inputs["position_ids"].copy_(position_ids)
        self.cache.cache_position.copy_(self._device_scalar(cache_position, self.torch.long,
                                                            self.cache.cache_position.device))
        self.kv_len_device.copy_(self._device_scalar(valid, self.torch.int32, self.kv_len_device.device))
        self._update_static_attention_mask(valid)
        if self.backend == "torch_cuda_graph" and self.cuda_graph is not None:
            self.cuda_graph.replay()
        else:
            self.bridge.replay_graph(stream_ptr=int(stream_ptr))
        self.replay_count += 1
        return self.logits

    def invalidate(self, reason: str) -> None:
        try:
            self.bridge.reset_graph()
        finally:
            if hasattr(self.bridge, "clear_qwen2_graph_dispatch"):
                self.bridge.clear_qwen2_graph_dispatch()
        self.contract = None
        self.status = "fallback"
        self.reason = str(reason)
