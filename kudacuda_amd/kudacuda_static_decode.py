"""Whole-forward graph capture for batch-1 Qwen2 decode.

Public API of the reference's python/kudacuda_static_decode.py:85-447
(``GraphStaticCache``, ``StaticDecodeContract``, ``StaticDecodeGraphRunner``
with ``capture`` / ``replay`` / ``invalidate``, the same arguments and the
same ``GraphContractError`` messages).

A decode forward can be recorded once and replayed for every later token
only if every address it baked in stays put and every per-token scalar is
read from device memory.  The pieces:

* ``GraphStaticCache`` -- per layer a fixed-capacity ``[batch, kv_heads,
  capacity, head_dim]`` K/V pair and the write position as a device tensor,
  so the cache update inside the forward is an ``index_copy_`` at a device
  index (the native attention reads the valid length from ``kv_len_device``);
* the runner's device-resident inputs (token, position ids, additive masks,
  cache position, kv_len), written in place before each replay;
* ``_KeyBuilder`` -- the one place that turns the runner's state into the
  ``DecodeGraphKey`` (device, tactic, layer count, shapes, bucket, model
  fingerprint and the address of every tensor the graph uses); a replay is
  refused unless it rebuilds the captured key exactly;
* two recorders with ``record(forward)`` / ``replay()``: PyTorch's HIP graph
  (``torch.cuda.CUDAGraph``, when a capture stream is given) and the
  bridge's own hipGraph on the caller's stream.
"""

from __future__ import annotations

import time
from contextlib import nullcontext
from dataclasses import dataclass
from typing import Any, Callable, Iterator, Mapping, Optional

from .kudacuda_graph_plan import DecodeGraphKey, GraphContractError


# ------------------------------------------------------------ tensor trees
def _is_tensor(value: Any) -> bool:
    return callable(getattr(value, "data_ptr", None)) and getattr(value, "shape", None) is not None


def _walk(value: Any) -> Iterator[Any]:
    """Tensors of a nested value in one canonical order (mapping keys sorted)."""

    if isinstance(value, Mapping):
        for key in sorted(value, key=str):
            yield from _walk(value[key])
    elif isinstance(value, (list, tuple)):
        for item in value:
            yield from _walk(item)
    elif _is_tensor(value):
        yield value


def _rebuild(value: Any, leaf: Callable[[Any], Any]) -> Any:
    """The same nesting (mappings, lists, tuples) with ``leaf`` applied to the rest."""

    if isinstance(value, Mapping):
        return {key: _rebuild(item, leaf) for key, item in value.items()}
    if isinstance(value, (list, tuple)):
        items = [_rebuild(item, leaf) for item in value]
        return tuple(items) if isinstance(value, tuple) else items
    return leaf(value)


def _own_copy(value: Any) -> Any:
    clone = getattr(value, "clone", None)
    return clone() if callable(clone) else value


def _dims(value: Any) -> tuple[int, ...]:
    return tuple(int(v) for v in getattr(value, "shape", ()))


def _address(tensor: Any, label: str) -> int:
    data_ptr = getattr(tensor, "data_ptr", None)
    if not callable(data_ptr):
        raise GraphContractError(f"{label} does not expose data_ptr()")
    address = int(data_ptr())
    if address <= 0:
        raise GraphContractError(f"{label} has an invalid device pointer")
    return address


def _kv_pairs(cache: Any) -> list[tuple[Any, Any]]:
    """(key, value) tensors per layer of a framework cache: Transformers'
    ``layers`` of ``keys`` / ``values`` objects, or the older parallel
    ``key_cache`` / ``value_cache`` lists."""

    layers = getattr(cache, "layers", None)
    if layers is None:
        keys, values = getattr(cache, "key_cache", None), getattr(cache, "value_cache", None)
        return [] if keys is None or values is None else list(zip(keys, values))
    pairs = []
    for index, layer in enumerate(layers):
        if isinstance(layer, tuple) and len(layer) == 2:
            pairs.append(layer)
            continue
        key = next((getattr(layer, n) for n in ("keys", "key_cache") if getattr(layer, n, None) is not None), None)
        value = next((getattr(layer, n) for n in ("values", "value_cache") if getattr(layer, n, None) is not None),
                     None)
        if key is None or value is None:
            raise GraphContractError(f"cache layer {index} has no key/value tensors")
        pairs.append((key, value))
    return pairs


def _padded(torch_module: Any, tensor: Any, capacity: int) -> Any:
    """Zero tensor with dimension 2 widened to ``capacity``, prefix copied in."""

    dims = _dims(tensor)
    out = torch_module.zeros(dims[:2] + (capacity,) + dims[3:], dtype=tensor.dtype, device=tensor.device)
    out[..., : dims[2], :].copy_(tensor)
    return out


def _open_prefix(torch_module: Any, masks: Any, valid: int) -> None:
    """Set every additive mask to admit cache slots [0, valid) and hide the
    rest (the framework attention path reads it; the native kernels read
    kv_len_device instead)."""

    finfo = getattr(torch_module, "finfo", None)
    if not callable(finfo):
        return
    for mask in _walk(masks):
        dims = _dims(mask)
        if not dims or not callable(getattr(mask, "fill_", None)):
            continue
        try:
            hidden = finfo(getattr(mask, "dtype", None)).min
        except (TypeError, ValueError, RuntimeError):
            continue
        cut = max(0, min(int(valid), dims[-1]))
        mask.fill_(0.0)
        if cut < dims[-1]:
            mask[..., cut:].fill_(hidden)


# ------------------------------------------------------------ static cache
class GraphStaticCache:
    """Per-layer [batch, kv_heads, max_cache_len, head_dim] K/V with the write
    position held in a device tensor (``cache_position``)."""

    def __init__(self, *, key_cache: list[Any], value_cache: list[Any], cache_position: Any, sequence_length: int,
                 max_cache_len: int) -> None:
        if len(key_cache) != len(value_cache):
            raise GraphContractError("graph cache needs one value tensor per key tensor")
        self.key_cache = list(key_cache)
        self.value_cache = list(value_cache)
        self.cache_position = cache_position
        self._sequence_length = int(sequence_length)
        self.max_cache_len = int(max_cache_len)
        self.layers = list(zip(self.key_cache, self.value_cache))

    @classmethod
    def from_dynamic_cache(cls, torch_module: Any, dynamic_cache: Any, *, max_cache_len: int) -> "GraphStaticCache":
        """Copy a prefilled framework cache into zero-padded fixed-capacity tensors."""

        pairs = _kv_pairs(dynamic_cache)
        if not pairs:
            raise GraphContractError("dynamic cache does not expose cache layers")
        capacity = int(max_cache_len)
        for index, (key, value) in enumerate(pairs):
            if key.dim() != 4 or _dims(value) != _dims(key):
                raise GraphContractError(f"cache layer {index} is not a rank-4 KV pair")
            if _dims(key)[2] > capacity:
                raise GraphContractError("max_cache_len is smaller than the prefetched cache")
        keys = [_padded(torch_module, key, capacity) for key, _ in pairs]
        values = [_padded(torch_module, value, capacity) for _, value in pairs]
        length = int(dynamic_cache.get_seq_length())
        position = torch_module.tensor([length], dtype=torch_module.long, device=keys[0].device)
        return cls(key_cache=keys, value_cache=values, cache_position=position, sequence_length=length,
                   max_cache_len=capacity)

    def update(self, key_states: Any, value_states: Any, layer_idx: int, *args: Any,
               **kwargs: Any) -> tuple[Any, Any]:
        """Write this step's rows at the device-resident position(s)."""

        del args, kwargs
        if _dims(key_states)[-2] != int(self.cache_position.numel()):
            raise GraphContractError("graph cache position count does not match key update length")
        key, value = self.key_cache[layer_idx], self.value_cache[layer_idx]
        key.index_copy_(2, self.cache_position, key_states)
        value.index_copy_(2, self.cache_position, value_states)
        return key, value

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


# ------------------------------------------------------------ recorders
class _TorchGraphRecorder:
    """PyTorch's HIP graph on a capture stream."""

    name = "torch_cuda_graph"

    def __init__(self, torch_module: Any, stream: Any) -> None:
        self.graph = torch_module.cuda.CUDAGraph()
        self._cuda = torch_module.cuda
        self._stream = stream

    def record(self, forward: Callable[[], Any]) -> Any:
        with self._cuda.graph(self.graph, stream=self._stream):
            outputs = forward()
        self.graph.replay()  # recording does not execute: run the first step
        return outputs

    def replay(self) -> None:
        self.graph.replay()


class _HandleGraphRecorder:
    """The bridge's native hipGraph (kudacuda_begin/end_capture, replay)."""

    name = "native"
    graph = None

    def __init__(self, bridge: Any, stream_ptr: int) -> None:
        self._bridge = bridge
        self._stream_ptr = int(stream_ptr)

    def record(self, forward: Callable[[], Any]) -> Any:
        self._bridge.begin_capture(stream_ptr=self._stream_ptr)
        try:
            outputs = forward()
        except Exception:
            try:  # end the stream capture before the caller resets the graph
                self._bridge.end_capture(stream_ptr=self._stream_ptr)
            except Exception:
                pass
            raise
        self._bridge.end_capture(stream_ptr=self._stream_ptr)
        self._bridge.replay_graph(stream_ptr=self._stream_ptr)
        return outputs

    def replay(self) -> None:
        self._bridge.replay_graph(stream_ptr=self._stream_ptr)


# ------------------------------------------------------------ graph key
@dataclass(frozen=True)
class _KeyBuilder:
    """Builds the DecodeGraphKey of a runner's current state."""

    tactic_name: str
    device_id: int
    kv_bucket: int

    def build(self, runner: "StaticDecodeGraphRunner") -> DecodeGraphKey:
        inputs, cache = runner.static_inputs, runner.cache
        baked = [*_walk(inputs), *cache.key_cache, *cache.value_cache, runner.kv_len_device]
        config = getattr(runner.model, "config", None)
        token = inputs["input_ids"]
        return DecodeGraphKey(
            device_id=self.device_id, tactic_name=self.tactic_name, layer_count=runner.layer_count(),
            query_shape=_dims(token), key_shape=_dims(cache.key_cache[0]), value_shape=_dims(cache.value_cache[0]),
            output_shape=_dims(runner.logits) if runner.logits is not None else (), kv_bucket=self.kv_bucket,
            pointers=tuple(_address(t, "graph tensor") for t in baked),
            model_fingerprint=runner.model_fingerprint(runner.model), dtype=str(getattr(token, "dtype", "")),
            quantization=str(getattr(config, "quantization_config", "")))


@dataclass(frozen=True)
class StaticDecodeContract:
    key: DecodeGraphKey
    stream_ptr: int
    logical_kv_len: int


# ------------------------------------------------------------ runner
class StaticDecodeGraphRunner:
    """Capture one whole decode forward of a model and replay it by pointer identity."""

    _FINGERPRINT_FIELDS = ("model_type", "num_hidden_layers", "hidden_size", "vocab_size", "torch_dtype")

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
        self._recorder: Any = None
        self._keys: Optional[_KeyBuilder] = None

    @property
    def captured(self) -> bool:
        return self.contract is not None and self.status == "captured"

    @classmethod
    def model_fingerprint(cls, model: Any) -> str:
        config = getattr(model, "config", None)
        return "|".join([type(model).__name__, *(str(getattr(config, f, "")) for f in cls._FINGERPRINT_FIELDS)])

    def layer_count(self) -> int:
        count = getattr(getattr(self.model, "config", None), "num_hidden_layers", None)
        if count is not None:
            return int(count)
        layers = getattr(getattr(self.model, "model", None), "layers", None)
        return 0 if layers is None else len(layers)

    # -------------------------------------------------------- device state
    def _scalar(self, value: int, dtype: Any, device: Any) -> Any:
        return self.torch.tensor([int(value)], dtype=dtype, device=device)

    def _load_step(self, *, cache_position: int, valid: int) -> None:
        """Write the per-step device scalars and masks for a cache that will
        hold ``valid`` tokens after this step writes position ``cache_position``."""

        position = self.cache.cache_position
        position.copy_(self._scalar(cache_position, self.torch.long, position.device))
        self.kv_len_device.copy_(self._scalar(valid, self.torch.int32, self.kv_len_device.device))
        _open_prefix(self.torch, self.static_inputs.get("attention_mask"), valid)

    def _bridge_graph_dispatch(self, kv_bucket: int, workspace: Any) -> None:
        configure = getattr(self.bridge, "configure_qwen2_graph_dispatch", None)
        if callable(configure):
            configure(kv_len_device=self.kv_len_device, kv_capacity=int(kv_bucket), workspace=workspace)

    def _end_bridge_graph_dispatch(self) -> None:
        clear = getattr(self.bridge, "clear_qwen2_graph_dispatch", None)
        if callable(clear):
            clear()

    def _forward(self, model_kwargs: Mapping[str, Any] | None) -> Any:
        inputs = self.static_inputs
        kwargs = dict(model_kwargs or {})
        kwargs.update(input_ids=inputs["input_ids"], position_ids=inputs["position_ids"],
                      attention_mask=inputs["attention_mask"], past_key_values=self.cache,
                      cache_position=inputs["cache_position"], use_cache=True, return_dict=True)
        inference_mode = getattr(self.torch, "inference_mode", None)
        with inference_mode() if callable(inference_mode) else nullcontext():
            return self.model(**kwargs)

    def _recorder_for(self, stream: Any, stream_ptr: int) -> Any:
        cuda = getattr(self.torch, "cuda", None)
        if stream is not None and hasattr(cuda, "CUDAGraph") and callable(getattr(cuda, "graph", None)):
            return _TorchGraphRecorder(self.torch, stream)
        return _HandleGraphRecorder(self.bridge, stream_ptr)

    # -------------------------------------------------------- capture
    def capture(self, *, input_ids: Any, position_ids: Any, attention_mask: Any, cache_position: Any,
                past_key_values: GraphStaticCache, logical_kv_len: int, kv_bucket: int, tactic_name: str,
                stream_ptr: int, stream: Any = None, device_id: int = 0,
                model_kwargs: Mapping[str, Any] | None = None, workspace: Any = None) -> Any:
        """Record one decode forward at position ``logical_kv_len`` (the cache
        then holds logical_kv_len + 1 tokens) and run it once."""

        if self.captured:
            raise GraphContractError("graph runner already has a captured forward")
        valid = int(logical_kv_len) + 1
        self.static_inputs = {"input_ids": _rebuild(input_ids, _own_copy),
                              "position_ids": _rebuild(position_ids, _own_copy),
                              "attention_mask": _rebuild(attention_mask, _own_copy),
                              "cache_position": cache_position}
        self.cache = past_key_values
        self.kv_len_device = self._scalar(valid, self.torch.int32, input_ids.device)
        self.workspace = workspace
        self._load_step(cache_position=int(logical_kv_len), valid=valid)
        recorder = self._recorder_for(stream, stream_ptr)
        self.backend = recorder.name
        self._bridge_graph_dispatch(kv_bucket, workspace)
        self.bridge.reset_graph()
        started = time.perf_counter()
        try:
            outputs = recorder.record(lambda: self._forward(model_kwargs))
            logits = getattr(outputs, "logits", None)
            if logits is None:
                raise GraphContractError("model decode output does not expose logits")
        except Exception as error:
            try:
                self.bridge.reset_graph()
            finally:
                self.status = "fallback"
                self.reason = f"capture_failed:{type(error).__name__}:{error}"
            raise GraphContractError(self.reason) from error
        finally:
            self._end_bridge_graph_dispatch()
        self.capture_ms = (time.perf_counter() - started) * 1e3
        self.logits = logits
        self._recorder = recorder
        self.cuda_graph = recorder.graph
        self.replay_count = 1
        self._keys = _KeyBuilder(tactic_name=tactic_name, device_id=int(device_id), kv_bucket=int(kv_bucket))
        self.contract = StaticDecodeContract(key=self._keys.build(self), stream_ptr=int(stream_ptr),
                                             logical_kv_len=valid)
        self.status = "captured"
        self.reason = None
        return self.logits

    # -------------------------------------------------------- replay
    def _replay_refusal(self, next_token: Any, position_ids: Any, valid: int, stream_ptr: int) -> Optional[str]:
        contract = self.contract
        if not self.captured or contract is None or self._keys is None:
            return "graph runner has no captured forward"
        if int(stream_ptr) != contract.stream_ptr:
            return "graph replay stream changed"
        if valid > contract.key.kv_bucket:
            return "graph replay KV length exceeds the captured bucket"
        if _dims(next_token) != _dims(self.static_inputs["input_ids"]):
            return "graph replay token shape changed"
        if _dims(position_ids) != _dims(self.static_inputs["position_ids"]):
            return "graph replay position shape changed"
        if self._keys.build(self) != contract.key:
            return "graph replay pointer, shape, or model contract changed"
        return None

    def replay(self, *, next_token: Any, position_ids: Any, cache_position: int, logical_kv_len: int,
               stream_ptr: int) -> Any:
        """Run the captured forward for the token at ``cache_position``."""

        valid = int(logical_kv_len) + 1
        refusal = self._replay_refusal(next_token, position_ids, valid, stream_ptr)
        if refusal is not None:
            raise GraphContractError(refusal)
        self.static_inputs["input_ids"].copy_(next_token)
        self.static_inputs["position_ids"].copy_(position_ids)
        self._load_step(cache_position=int(cache_position), valid=valid)
        self._recorder.replay()
        self.replay_count += 1
        return self.logits

    def invalidate(self, reason: str) -> None:
        try:
            self.bridge.reset_graph()
        finally:
            self._end_bridge_graph_dispatch()
            self.contract = None
            self._recorder = None
            self._keys = None
            self.status = "fallback"
            self.reason = str(reason)
