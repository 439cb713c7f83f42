"""Graph plan key guard (intent of the reference's tests/test_graph_plan.py)."""

from __future__ import annotations

import pytest

from kudacuda_amd.kudacuda_graph_plan import DecodeGraphKey, GraphContractError, KudaCudaGraphPlan


class Bridge:
    def __init__(self, fail_end=False):
        self.calls = []
        self.fail_end = fail_end

    def begin_capture(self, *, stream_ptr):
        self.calls.append(("begin", stream_ptr))

    def end_capture(self, *, stream_ptr):
        if self.fail_end:
            raise RuntimeError("end failed")
        self.calls.append(("end", stream_ptr))

    def replay_graph(self, *, stream_ptr):
        self.calls.append(("replay", stream_ptr))


def key(seed=100, bucket=2048):
    return DecodeGraphKey(device_id=0, tactic_name="qwen2_gqa_decode_gfx950_bf16_graph_v1", layer_count=36,
                          query_shape=(1, 16, 1, 128), key_shape=(1, 2, bucket, 128),
                          value_shape=(1, 2, bucket, 128), output_shape=(1, 16, 1, 128), kv_bucket=bucket,
                          pointers=(seed, seed + 1, seed + 2, seed + 3))


def test_capture_then_replay_with_the_same_key():
    bridge = Bridge()
    plan = KudaCudaGraphPlan(bridge)
    plan.begin_capture(key(), stream_ptr=77)
    assert plan.capturing and not plan.captured
    plan.end_capture(key(), stream_ptr=77)
    plan.replay(key(), stream_ptr=77)
    assert bridge.calls == [("begin", 77), ("end", 77), ("replay", 77)]


@pytest.mark.parametrize("changed", [key(seed=200), key(bucket=4096)])
def test_changed_key_or_stream_is_refused(changed):
    plan = KudaCudaGraphPlan(Bridge())
    plan.begin_capture(key(), stream_ptr=77)
    plan.end_capture(key(), stream_ptr=77)
    with pytest.raises(GraphContractError, match="key"):
        plan.replay(changed, stream_ptr=77)
    with pytest.raises(GraphContractError, match="stream"):
        plan.replay(key(), stream_ptr=78)
    assert not plan.can_replay(changed, stream_ptr=77)


def test_nested_capture_end_mismatch_and_invalidate():
    plan = KudaCudaGraphPlan(Bridge())
    with pytest.raises(GraphContractError, match="not capturing"):
        plan.end_capture(key(), stream_ptr=77)
    plan.begin_capture(key(), stream_ptr=77)
    with pytest.raises(GraphContractError, match="capturing"):
        plan.begin_capture(key(), stream_ptr=77)
    with pytest.raises(GraphContractError, match="changed"):
        plan.end_capture(key(seed=5), stream_ptr=77)
    plan.invalidate()
    with pytest.raises(GraphContractError, match="captured"):
        plan.replay(key(), stream_ptr=77)


def test_failed_end_capture_leaves_no_graph():
    plan = KudaCudaGraphPlan(Bridge(fail_end=True))
    plan.begin_capture(key(), stream_ptr=77)
    with pytest.raises(RuntimeError, match="end failed"):
        plan.end_capture(key(), stream_ptr=77)
    assert not plan.capturing and not plan.captured
