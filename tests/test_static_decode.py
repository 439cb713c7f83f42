"""StaticDecodeGraphRunner and GraphStaticCache with fakes (intent of the
reference's tests/test_static_decode.py)."""

from __future__ import annotations

from types import SimpleNamespace

import pytest

from kudacuda_amd.kudacuda_graph_plan import GraphContractError
from kudacuda_amd.kudacuda_static_decode import GraphStaticCache, StaticDecodeGraphRunner

_NEXT = [1000]


class Tensor:
    def __init__(self, shape, *, pointer=None, dtype="bfloat16", device="cuda"):
        self.shape, self.dtype, self.device = tuple(shape), dtype, device
        if pointer is None:
            pointer = _NEXT[0]
            _NEXT[0] += 1
        self.pointer = pointer
        self.copies = 0
        self.fills = []

    def data_ptr(self):
        return self.pointer

    def clone(self):
        return Tensor(self.shape, dtype=self.dtype, device=self.device)

    def copy_(self, other):
        self.copies += 1
        return self

    def __getitem__(self, item):
        return self

    def fill_(self, value):
        self.fills.append(value)
        return self

    def numel(self):
        n = 1
        for s in self.shape:
            n *= s
        return n


class Torch:
    int32, long, float32, bfloat16 = "int32", "int64", "float32", "bfloat16"

    class _Ctx:
        def __enter__(self):
            return self

        def __exit__(self, *a):
            return False

    @classmethod
    def inference_mode(cls):
        return cls._Ctx()

    @staticmethod
    def tensor(values, *, dtype, device):
        return Tensor((len(values),), dtype=dtype, device=device)

    @staticmethod
    def finfo(dtype):
        return SimpleNamespace(min=-3.0e38 if dtype == "bfloat16" else -1.0)


class Bridge:
    def __init__(self):
        self.calls = []

    def configure_qwen2_graph_dispatch(self, *, kv_len_device, kv_capacity, workspace=None):
        self.calls.append(("configure", kv_len_device.data_ptr(), kv_capacity))

    def clear_qwen2_graph_dispatch(self):
        self.calls.append(("clear",))

    def reset_graph(self):
        self.calls.append(("reset",))

    def begin_capture(self, *, stream_ptr):
        self.calls.append(("begin", stream_ptr))

    def end_capture(self, *, stream_ptr):
        self.calls.append(("end", stream_ptr))

    def replay_graph(self, *, stream_ptr):
        self.calls.append(("replay", stream_ptr))


class Cache:
    def __init__(self):
        self.key_cache = [Tensor((1, 2, 2048, 128), pointer=200)]
        self.value_cache = [Tensor((1, 2, 2048, 128), pointer=300)]
        self.cache_position = Tensor((1,), pointer=400, dtype="int64")


class Model:
    def __init__(self, fail=False):
        self.calls = 0
        self.fail = fail
        self.config = SimpleNamespace(model_type="qwen2", num_hidden_layers=1, hidden_size=2048, vocab_size=4096,
                                      torch_dtype="bfloat16", quantization_config="nf4")

    def __call__(self, **kwargs):
        self.calls += 1
        if self.fail:
            raise RuntimeError("capture boom")
        return SimpleNamespace(logits=Tensor((1, 1, 4096), pointer=500))


def setup(model=None):
    bridge = Bridge()
    model = model or Model()
    runner = StaticDecodeGraphRunner(bridge, model, Torch)
    args = dict(input_ids=Tensor((1, 1), dtype="int64", pointer=10),
                position_ids=Tensor((1, 1), dtype="int64", pointer=11),
                attention_mask={"full_attention": Tensor((1, 1, 1, 2048), pointer=12)},
                cache_position=Tensor((1,), dtype="int64", pointer=13), past_key_values=Cache(), logical_kv_len=63,
                kv_bucket=2048, tactic_name="qwen2_gqa_decode_gfx950_bf16_graph_v1", stream_ptr=77)
    return runner, bridge, model, args


def replay(runner, **over):
    kw = dict(next_token=Tensor((1, 1), dtype="int64"), position_ids=Tensor((1, 1), dtype="int64"),
              cache_position=64, logical_kv_len=64, stream_ptr=77)
    kw.update(over)
    return runner.replay(**kw)


def test_capture_runs_the_model_once_and_replays_natively():
    runner, bridge, model, args = setup()
    logits = runner.capture(**args)
    assert replay(runner) is logits
    assert model.calls == 1 and runner.status == "captured" and runner.backend == "native"
    names = [c[0] for c in bridge.calls]
    assert names[:4] == ["configure", "reset", "begin", "end"]
    assert ("configure", runner.kv_len_device.data_ptr(), 2048) in bridge.calls
    assert names.count("replay") == 2 and runner.replay_count == 2
    assert ("clear",) in bridge.calls


def test_attention_mask_tracks_the_valid_length():
    runner, _, _, args = setup()
    runner.capture(**args)
    mask = runner.static_inputs["attention_mask"]["full_attention"]
    assert -3.0e38 in mask.fills
    replay(runner)
    assert mask.fills.count(-3.0e38) >= 2


def test_replay_guards():
    runner, _, _, args = setup()
    with pytest.raises(GraphContractError, match="no captured"):
        replay(runner)
    runner.capture(**args)
    with pytest.raises(GraphContractError, match="stream changed"):
        replay(runner, stream_ptr=88)
    with pytest.raises(GraphContractError, match="bucket"):
        replay(runner, logical_kv_len=2048)
    with pytest.raises(GraphContractError, match="token shape"):
        replay(runner, next_token=Tensor((1, 2), dtype="int64"))
    runner.cache.key_cache[0].pointer = 999   # a reallocated cache breaks the key
    with pytest.raises(GraphContractError, match="pointer"):
        replay(runner)
    with pytest.raises(GraphContractError, match="already"):
        runner.capture(**args)


def test_capture_failure_resets_and_records_fallback():
    runner, bridge, _, args = setup(Model(fail=True))
    with pytest.raises(GraphContractError, match="capture_failed"):
        runner.capture(**args)
    assert runner.status == "fallback" and ("reset",) in bridge.calls[2:]
    runner.invalidate("done")
    assert runner.reason == "done" and not runner.captured


def test_static_cache_update_and_shape_checks():
    class Dyn:
        def __init__(self, length):
            self.key_cache = [Tensor((1, 2, length, 128))]
            self.value_cache = [Tensor((1, 2, length, 128))]
            for t in self.key_cache + self.value_cache:
                t.dim = lambda: 4

        def get_seq_length(self):
            return int(self.key_cache[0].shape[2])

    class Zeros(Torch):
        @staticmethod
        def zeros(shape, *, dtype, device):
            return Tensor(shape, dtype=dtype, device=device)

    cache = GraphStaticCache.from_dynamic_cache(Zeros, Dyn(10), max_cache_len=64)
    assert cache.key_cache[0].shape == (1, 2, 64, 128) and cache.get_seq_length() == 10
    assert cache.get_max_cache_shape() == 64 and len(cache) == 1
    with pytest.raises(GraphContractError, match="smaller"):
        GraphStaticCache.from_dynamic_cache(Zeros, Dyn(100), max_cache_len=64)
