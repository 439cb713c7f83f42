"""GraphStaticCache and StaticDecodeGraphRunner on real CPU tensors.

The intent of the reference's tests/test_static_decode.py -- capture once,
replay by pointer identity, refuse any contract change, fall back cleanly
when capture fails -- checked on PyTorch CPU tensors (and a real
Transformers DynamicCache), so the masks, device scalars and cache rows the
runner writes are inspected by value.  Only the bridge (a call log standing
in for libkudacuda's hipGraph API) and the model (a tiny decode forward that
writes this token's K/V through the cache and logits into a fixed buffer)
are stand-ins.
"""

from __future__ import annotations

from types import SimpleNamespace

import pytest

torch = pytest.importorskip("torch")

from kudacuda_amd.kudacuda_graph_plan import GraphContractError  # noqa: E402
from kudacuda_amd.kudacuda_static_decode import GraphStaticCache, StaticDecodeGraphRunner  # noqa: E402

LAYERS, HEADS, DIM, BUCKET, VOCAB = 2, 2, 8, 16, 32
TACTIC = "qwen2_gqa_decode_gfx950_bf16_graph_v1"
STREAM = 4242


class CallLog:
    """Bridge stand-in: records the graph API calls in order."""

    def __init__(self) -> None:
        self.calls: list[tuple] = []
        self.dispatch: dict = {}

    def configure_qwen2_graph_dispatch(self, *, kv_len_device, kv_capacity, workspace=None):
        self.dispatch = dict(kv_len_device=kv_len_device, kv_capacity=kv_capacity)
        self.calls.append(("configure", kv_capacity))

    def clear_qwen2_graph_dispatch(self):
        self.dispatch = {}
        self.calls.append(("clear",))

    def __getattr__(self, name):
        if name in ("reset_graph", "begin_capture", "end_capture", "replay_graph"):
            return lambda **kw: self.calls.append((name, kw.get("stream_ptr")))
        raise AttributeError(name)

    def names(self) -> list[str]:
        return [c[0] for c in self.calls]


class TinyDecoder:
    """A decode forward: K/V of the token through ``past_key_values.update``,
    logits into one persistent buffer (as a captured graph's output is)."""

    def __init__(self, fail: bool = False) -> None:
        self.fail = fail
        self.runs = 0
        self.out = torch.zeros(1, 1, VOCAB)
        self.config = SimpleNamespace(model_type="qwen2", num_hidden_layers=LAYERS, hidden_size=HEADS * DIM,
                                      vocab_size=VOCAB, torch_dtype="float32", quantization_config="nf4")

    def __call__(self, *, input_ids, past_key_values, cache_position, **kwargs):
        self.runs += 1
        if self.fail:
            raise RuntimeError("decode forward failed")
        row = input_ids.float().reshape(1, 1, 1, 1).expand(1, HEADS, 1, DIM)
        for layer in range(LAYERS):
            past_key_values.update(row + layer, -row - layer, layer)
        self.out.copy_(input_ids.float().reshape(1, 1, 1).expand(1, 1, VOCAB))
        return SimpleNamespace(logits=self.out)


def _prefilled_cache(tokens: int):
    from transformers import DynamicCache

    cache = DynamicCache()
    for layer in range(LAYERS):
        k = torch.arange(tokens, dtype=torch.float32).reshape(1, 1, tokens, 1).expand(1, HEADS, tokens, DIM)
        cache.update(k.contiguous() + layer, -k.contiguous() - layer, layer)
    return cache


def _captured(model=None, pos: int = 5):
    bridge, model = CallLog(), model or TinyDecoder()
    static = GraphStaticCache.from_dynamic_cache(torch, _prefilled_cache(pos), max_cache_len=BUCKET)
    runner = StaticDecodeGraphRunner(bridge, model, torch)
    mask = {"full_attention": torch.zeros(1, 1, 1, BUCKET)}
    runner.capture(input_ids=torch.tensor([[7]]), position_ids=torch.tensor([[pos]]), attention_mask=mask,
                   cache_position=static.cache_position, past_key_values=static, logical_kv_len=pos, kv_bucket=BUCKET,
                   tactic_name=TACTIC, stream_ptr=STREAM)
    return runner, bridge, model, static


def _mask_admits(runner) -> int:
    mask = runner.static_inputs["attention_mask"]["full_attention"][0, 0, 0]
    admitted = int((mask == 0).sum())
    assert torch.all(mask[:admitted] == 0) and torch.all(mask[admitted:] == torch.finfo(mask.dtype).min)
    return admitted


def test_static_cache_pads_a_framework_cache_and_writes_at_the_device_position():
    static = GraphStaticCache.from_dynamic_cache(torch, _prefilled_cache(5), max_cache_len=BUCKET)
    assert len(static) == LAYERS and static.get_seq_length() == 5 and static.get_max_cache_shape() == BUCKET
    assert static.cache_position.tolist() == [5]
    for layer in range(LAYERS):
        key = static.key_cache[layer]
        assert tuple(key.shape) == (1, HEADS, BUCKET, DIM)
        assert torch.equal(key[0, 0, :5, 0], torch.arange(5, dtype=torch.float32) + layer)
        assert not key[..., 5:, :].any() and not static.value_cache[layer][..., 5:, :].any()
    k, v = static.update(torch.full((1, HEADS, 1, DIM), 9.0), torch.full((1, HEADS, 1, DIM), -9.0), 1)
    assert k is static.key_cache[1] and torch.all(k[0, :, 5] == 9.0) and torch.all(v[0, :, 5] == -9.0)
    with pytest.raises(GraphContractError, match="position count"):
        static.update(torch.zeros(1, HEADS, 2, DIM), torch.zeros(1, HEADS, 2, DIM), 0)
    with pytest.raises(GraphContractError, match="smaller"):
        GraphStaticCache.from_dynamic_cache(torch, _prefilled_cache(BUCKET + 1), max_cache_len=BUCKET)


def test_capture_records_once_runs_once_and_binds_the_device_state():
    runner, bridge, model, static = _captured()
    assert runner.captured and runner.backend == "native" and runner.replay_count == 1 and model.runs == 1
    assert bridge.names() == ["configure", "reset_graph", "begin_capture", "end_capture", "replay_graph", "clear"]
    assert all(c[1] == STREAM for c in bridge.calls if c[0] in ("begin_capture", "end_capture", "replay_graph"))
    assert bridge.calls[0] == ("configure", BUCKET) and bridge.dispatch == {}
    assert runner.kv_len_device.tolist() == [6] and runner.kv_len_device.dtype == torch.int32
    assert static.cache_position.tolist() == [5] and _mask_admits(runner) == 6
    assert torch.all(static.key_cache[0][0, :, 5] == 7.0)  # the forward wrote this token's row
    assert runner.logits is model.out and runner.capture_ms is not None


def test_replay_rebinds_position_kv_len_and_mask_without_rerunning_the_model():
    runner, bridge, model, static = _captured()
    for pos in (6, 7, 11):
        out = runner.replay(next_token=torch.tensor([[pos]]), position_ids=torch.tensor([[pos]]), cache_position=pos,
                            logical_kv_len=pos, stream_ptr=STREAM)
        assert out is model.out
        assert static.cache_position.tolist() == [pos] and runner.kv_len_device.tolist() == [pos + 1]
        assert runner.static_inputs["input_ids"].tolist() == [[pos]] and _mask_admits(runner) == pos + 1
    assert model.runs == 1 and runner.replay_count == 4 and bridge.names().count("replay_graph") == 4


@pytest.mark.parametrize("change,message", [
    (dict(stream_ptr=STREAM + 1), "stream changed"),
    (dict(logical_kv_len=BUCKET), "exceeds the captured bucket"),
    (dict(next_token=torch.tensor([[1, 2]])), "token shape changed"),
    (dict(position_ids=torch.tensor([[1, 2]])), "position shape changed"),
])
def test_replay_refuses_a_changed_contract(change, message):
    runner, bridge, _, _ = _captured()
    before = list(bridge.calls)
    args = dict(next_token=torch.tensor([[6]]), position_ids=torch.tensor([[6]]), cache_position=6, logical_kv_len=6,
                stream_ptr=STREAM)
    args.update(change)
    with pytest.raises(GraphContractError, match=message):
        runner.replay(**args)
    assert bridge.calls == before  # refused before anything ran


def test_replay_refuses_a_reallocated_cache_and_a_second_capture():
    runner, _, _, static = _captured()
    static.key_cache[1] = static.key_cache[1].clone()  # same shape, new address
    with pytest.raises(GraphContractError, match="pointer, shape, or model contract changed"):
        runner.replay(next_token=torch.tensor([[6]]), position_ids=torch.tensor([[6]]), cache_position=6,
                      logical_kv_len=6, stream_ptr=STREAM)
    with pytest.raises(GraphContractError, match="already has a captured forward"):
        runner.capture(input_ids=torch.tensor([[7]]), position_ids=torch.tensor([[5]]), attention_mask=None,
                       cache_position=static.cache_position, past_key_values=static, logical_kv_len=5,
                       kv_bucket=BUCKET, tactic_name=TACTIC, stream_ptr=STREAM)


def test_failed_capture_ends_the_stream_capture_resets_and_falls_back():
    with pytest.raises(GraphContractError, match="capture_failed:RuntimeError:decode forward failed"):
        _captured(TinyDecoder(fail=True))
    runner = StaticDecodeGraphRunner(CallLog(), TinyDecoder(fail=True), torch)
    static = GraphStaticCache.from_dynamic_cache(torch, _prefilled_cache(3), max_cache_len=BUCKET)
    with pytest.raises(GraphContractError):
        runner.capture(input_ids=torch.tensor([[1]]), position_ids=torch.tensor([[3]]), attention_mask=None,
                       cache_position=static.cache_position, past_key_values=static, logical_kv_len=3,
                       kv_bucket=BUCKET, tactic_name=TACTIC, stream_ptr=STREAM)
    names = runner.bridge.names()
    assert names[names.index("begin_capture") + 1] == "end_capture"  # the capture is closed first
    assert names[-2:] == ["reset_graph", "clear"] and runner.status == "fallback" and not runner.captured
    with pytest.raises(GraphContractError, match="no captured forward"):
        runner.replay(next_token=torch.tensor([[1]]), position_ids=torch.tensor([[4]]), cache_position=4,
                      logical_kv_len=4, stream_ptr=STREAM)
    runner.invalidate("given up")
    assert runner.reason == "given up" and runner.status == "fallback"


def test_a_capture_stream_selects_the_torch_graph_recorder():
    events = []

    class Graph:
        def replay(self):
            events.append("graph.replay")

    class GraphContext:
        def __init__(self, graph, stream):
            events.append(("graph.begin", stream))

        def __enter__(self):
            return self

        def __exit__(self, *exc):
            events.append("graph.end")
            return False

    fake_cuda = SimpleNamespace(CUDAGraph=Graph, graph=GraphContext)
    torch_like = SimpleNamespace(cuda=fake_cuda, tensor=torch.tensor, zeros=torch.zeros, long=torch.long,
                                 int32=torch.int32, finfo=torch.finfo, inference_mode=torch.inference_mode)
    bridge, model = CallLog(), TinyDecoder()
    static = GraphStaticCache.from_dynamic_cache(torch, _prefilled_cache(2), max_cache_len=BUCKET)
    runner = StaticDecodeGraphRunner(bridge, model, torch_like)
    runner.capture(input_ids=torch.tensor([[3]]), position_ids=torch.tensor([[2]]), attention_mask=None,
                   cache_position=static.cache_position, past_key_values=static, logical_kv_len=2, kv_bucket=BUCKET,
                   tactic_name=TACTIC, stream_ptr=STREAM, stream="capture-stream")
    assert runner.backend == "torch_cuda_graph" and isinstance(runner.cuda_graph, Graph)
    assert events == [("graph.begin", "capture-stream"), "graph.end", "graph.replay"]
    assert "begin_capture" not in bridge.names()
    runner.replay(next_token=torch.tensor([[4]]), position_ids=torch.tensor([[3]]), cache_position=3,
                  logical_kv_len=3, stream_ptr=STREAM)
    assert events[-1] == "graph.replay" and events.count("graph.replay") == 2
