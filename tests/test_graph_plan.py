"""The graph plan's key guard: a captured decode graph is replayed only under
the exact key (tactic, shapes, bucket, pointers) and stream it was captured
with, and every misuse is a GraphContractError, never a silent replay."""

from __future__ import annotations

from dataclasses import replace

import pytest

from kudacuda_amd.kudacuda_graph_plan import DecodeGraphKey, GraphContractError, KudaCudaGraphPlan

STREAM = 77
BASE = DecodeGraphKey(device_id=0, tactic_name="qwen2_gqa_decode_gfx950_bf16_graph_v1", layer_count=36,
                      query_shape=(1, 16, 1, 128), key_shape=(1, 2, 2048, 128), value_shape=(1, 2, 2048, 128),
                      output_shape=(1, 16, 1, 128), kv_bucket=2048, pointers=(100, 101, 102, 103))


class Recorder:
    """Stands in for the bridge: every method call is logged as (name, stream);
    the methods named in `raising` raise instead."""

    def __init__(self, *raising: str) -> None:
        self.log: list[tuple[str, int]] = []
        self.raising = set(raising)

    def __getattr__(self, name: str):
        if name not in ("begin_capture", "end_capture", "replay_graph"):
            raise AttributeError(name)

        def call(*, stream_ptr: int) -> None:
            if name in self.raising:
                raise RuntimeError(f"{name} failed")
            self.log.append((name, stream_ptr))

        return call


def captured_plan(bridge=None) -> KudaCudaGraphPlan:
    plan = KudaCudaGraphPlan(bridge if bridge is not None else Recorder())
    plan.begin_capture(BASE, stream_ptr=STREAM)
    plan.end_capture(BASE, stream_ptr=STREAM)
    return plan


def test_one_capture_then_replays_under_the_same_key():
    bridge = Recorder()
    plan = KudaCudaGraphPlan(bridge)
    plan.begin_capture(BASE, stream_ptr=STREAM)
    assert (plan.capturing, plan.captured) == (True, False)
    plan.end_capture(replace(BASE), stream_ptr=STREAM)  # an equal key, another object
    for _ in range(3):
        plan.replay(BASE, stream_ptr=STREAM)
    assert [name for name, _ in bridge.log] == ["begin_capture", "end_capture"] + ["replay_graph"] * 3
    assert {stream for _, stream in bridge.log} == {STREAM}


@pytest.mark.parametrize("field,value", [("pointers", (200, 101, 102, 103)), ("kv_bucket", 4096),
                                         ("key_shape", (1, 2, 4096, 128)), ("layer_count", 35),
                                         ("tactic_name", "qwen2_gqa_decode_gfx950_fp16_graph_v1")])
def test_any_changed_key_field_is_refused(field, value):
    plan = captured_plan()
    changed = replace(BASE, **{field: value})
    assert not plan.can_replay(changed, stream_ptr=STREAM)
    with pytest.raises(GraphContractError, match="key or stream changed"):
        plan.replay(changed, stream_ptr=STREAM)
    assert plan.can_replay(BASE, stream_ptr=STREAM)  # the refusal left the graph intact


def test_another_stream_is_refused():
    plan = captured_plan()
    with pytest.raises(GraphContractError, match="key or stream changed"):
        plan.replay(BASE, stream_ptr=STREAM + 1)


def test_capture_state_machine_misuse():
    plan = KudaCudaGraphPlan(Recorder())
    with pytest.raises(GraphContractError, match="not capturing"):
        plan.end_capture(BASE, stream_ptr=STREAM)
    with pytest.raises(GraphContractError, match="no captured graph"):
        plan.replay(BASE, stream_ptr=STREAM)
    plan.begin_capture(BASE, stream_ptr=STREAM)
    with pytest.raises(GraphContractError, match="already capturing"):
        plan.begin_capture(BASE, stream_ptr=STREAM)
    with pytest.raises(GraphContractError, match="capture key or stream changed"):
        plan.end_capture(replace(BASE, pointers=(5, 6, 7, 8)), stream_ptr=STREAM)


def test_a_second_capture_needs_invalidate():
    plan = captured_plan()
    with pytest.raises(GraphContractError, match="invalidate it first"):
        plan.begin_capture(BASE, stream_ptr=STREAM)
    plan.invalidate()
    assert not plan.captured
    with pytest.raises(GraphContractError, match="no captured graph"):
        plan.replay(BASE, stream_ptr=STREAM)
    plan.begin_capture(BASE, stream_ptr=STREAM)  # allowed again


def test_a_failed_end_capture_leaves_no_graph():
    plan = KudaCudaGraphPlan(Recorder("end_capture"))
    plan.begin_capture(BASE, stream_ptr=STREAM)
    with pytest.raises(RuntimeError, match="end_capture failed"):
        plan.end_capture(BASE, stream_ptr=STREAM)
    assert (plan.capturing, plan.captured) == (False, False)
