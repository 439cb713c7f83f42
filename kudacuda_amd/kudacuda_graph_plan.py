"""Static-key guard around the bridge's graph capture/replay primitives.

Mirrors reference python/kudacuda_graph_plan.py:13-92: a captured decode
graph may only be replayed with the identical key (device, tactic, layer
count, tensor shapes, KV bucket and every device pointer the graph baked in)
on the identical stream; anything else is a ``GraphContractError`` before the
bridge is touched.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Optional


class GraphContractError(RuntimeError):
    """A capture or replay broke the static contract of the graph."""


@dataclass(frozen=True)
class DecodeGraphKey:
    """State that must not change between capture and replay."""

    device_id: int
    tactic_name: str
    layer_count: int
    query_shape: tuple[int, ...]
    key_shape: tuple[int, ...]
    value_shape: tuple[int, ...]
    output_shape: tuple[int, ...]
    kv_bucket: int
    pointers: tuple[int, ...]
    model_fingerprint: str = ""
    dtype: str = ""
    quantization: str = ""


class KudaCudaGraphPlan:
    """Capture once, replay only under the captured key and stream."""

    def __init__(self, bridge: Any) -> None:
        self.bridge = bridge
        self._capturing: Optional[tuple[DecodeGraphKey, int]] = None
        self._captured: Optional[tuple[DecodeGraphKey, int]] = None

    @property
    def captured(self) -> bool:
        return self._captured is not None

    @property
    def capturing(self) -> bool:
        return self._capturing is not None

    def begin_capture(self, key: DecodeGraphKey, *, stream_ptr: int) -> None:
        if self.capturing:
            raise GraphContractError("graph plan is already capturing")
        if self.captured:
            raise GraphContractError("graph plan already has a captured key; invalidate it first")
        self.bridge.begin_capture(stream_ptr=int(stream_ptr))
        self._capturing = (key, int(stream_ptr))

    def end_capture(self, key: DecodeGraphKey, *, stream_ptr: int) -> None:
        if self._capturing is None:
            raise GraphContractError("graph plan is not capturing")
        if self._capturing != (key, int(stream_ptr)):
            raise GraphContractError("graph capture key or stream changed")
        pending, self._capturing = self._capturing, None
        self.bridge.end_capture(stream_ptr=int(stream_ptr))
        self._captured = pending

    def can_replay(self, key: DecodeGraphKey, *, stream_ptr: int) -> bool:
        return self._captured is not None and self._captured == (key, int(stream_ptr))

    def replay(self, key: DecodeGraphKey, *, stream_ptr: int) -> None:
        if self._captured is None:
            raise GraphContractError("graph plan has no captured graph")
        if not self.can_replay(key, stream_ptr=stream_ptr):
            raise GraphContractError("graph replay key or stream changed")
        self.bridge.replay_graph(stream_ptr=int(stream_ptr))

    def invalidate(self) -> None:
        self._capturing = None
        self._captured = None
