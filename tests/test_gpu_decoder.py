"""GPU parity of the native Qwen2 decode step against the oracle.

The GPU model is built by the product path (seeded fp32 streams, GPU NF4
quantiser, bf16 conversion by the product), the host model by the oracle's
own code from the same streams.  Every intermediate buffer must agree bit for
bit after every step, and hipGraph replay must reproduce eager execution.
"""

from __future__ import annotations

import numpy as np
import pytest

from kudacuda_amd import synthetic
from kudacuda_amd.qwen2_decoder import Qwen2Nf4Decoder
from tests._gpu_util import host
from tests._host_model import HostModel

pytestmark = pytest.mark.gpu

SEED = 20260824


@pytest.fixture(scope="module")
def small_pair(torch_gpu, native):
    kw = dict(num_layers=2, vocab=4096, kv_capacity=128, token_capacity=128)
    gpu = Qwen2Nf4Decoder.synthetic(native, torch_gpu, seed=SEED, **kw)
    cpu = HostModel(SEED, **kw)
    yield gpu, cpu
    gpu.close()


def test_quantised_weights_match_oracle(small_pair):
    gpu, cpu = small_pair
    for li in range(2):
        for name in ("q", "k", "v", "o", "gate", "up", "down"):
            assert np.array_equal(host(gpu.layers[li][f"{name}_packed"]), cpu.layers[li][f"{name}_packed"]), name
            assert np.array_equal(host(gpu.layers[li][f"{name}_absmax"]), cpu.layers[li][f"{name}_absmax"]), name
        for name in ("q_bias", "k_bias", "v_bias", "input_norm", "post_norm"):
            assert np.array_equal(host(gpu.layers[li][name]), cpu.layers[li][name]), name
    assert np.array_equal(host(gpu.embed), cpu.embed)
    assert np.array_equal(host(gpu.rope_cos), cpu.rope_cos)


def test_eager_steps_match_oracle_bit_for_bit(small_pair):
    gpu, cpu = small_pair
    prompt = synthetic.prompt_ids(SEED, 5, 4096)
    gpu.reset(prompt)
    cpu.reset(prompt)
    for step in range(14):
        gpu.step()
        gpu.stream.synchronize()
        cpu.step()
        ctx = f"step {step}"
        assert np.array_equal(host(gpu.control), cpu.control), ctx
        assert np.array_equal(host(gpu.query), cpu.query), ctx
        assert np.array_equal(host(gpu.attn), cpu.attn), ctx
        assert np.array_equal(host(gpu.mlp), cpu.mlp), ctx
        assert np.array_equal(host(gpu.hidden), cpu.hidden), ctx
        for li in range(2):
            kc = host(gpu.layers[li]["key_cache"])
            vc = host(gpu.layers[li]["value_cache"])
            assert np.array_equal(kc[:, : step + 1], cpu.layers[li]["key_cache"][:, : step + 1]), ctx
            assert np.array_equal(vc[:, : step + 1], cpu.layers[li]["value_cache"][:, : step + 1]), ctx
        if step + 1 >= prompt.size:
            assert np.array_equal(host(gpu.logits), cpu.logits), ctx
        assert np.array_equal(host(gpu.tokens)[: step + 2], cpu.tokens[: step + 2]), ctx


def test_graph_replay_matches_eager(small_pair):
    gpu, _ = small_pair
    prompt = synthetic.prompt_ids(SEED + 1, 7, 4096)
    eager = gpu.generate(prompt, 20, graph=False)
    graph = gpu.generate(prompt, 20, graph=True)
    again = gpu.generate(prompt, 20, graph=True)
    assert np.array_equal(eager, graph)
    assert np.array_equal(graph, again)


def test_generate_matches_oracle_tokens(small_pair):
    gpu, cpu = small_pair
    prompt = synthetic.prompt_ids(SEED + 2, 9, 4096)
    assert np.array_equal(gpu.generate(prompt, 24), cpu.generate(prompt, 24))


@pytest.mark.parametrize("graph", [False, True])
def test_stop_token_is_decided_on_the_device(small_pair, graph):
    gpu, cpu = small_pair
    prompt = synthetic.prompt_ids(SEED + 6, 6, 4096)
    free = cpu.generate(prompt, 20)
    k = next(i for i in range(2, 20) if free[i] not in free[:i])
    stop = int(free[k])
    got = gpu.generate(prompt, 20, graph=graph, stop_token=stop)  # all 25 steps launched, no host sync between
    assert got.tolist() == free[: k + 1].tolist()
    assert gpu.stopped_at() == prompt.size + k
    assert np.array_equal(cpu.generate(prompt, 20, stop_token=stop), got)
    assert np.array_equal(host(gpu.control), cpu.control)
    # what this decode wrote (the host model's earlier unstopped run left
    # more tokens and cache rows behind the stop position)
    end = prompt.size + k
    assert np.array_equal(host(gpu.tokens)[: end + 1], cpu.tokens[: end + 1])
    for li in range(2):
        assert np.array_equal(host(gpu.layers[li]["key_cache"])[:, :end], cpu.layers[li]["key_cache"][:, :end])
    # more steps after the stop change nothing the decode owns
    before = (host(gpu.tokens), host(gpu.control), host(gpu.layers[0]["value_cache"]), host(gpu.logits))
    gpu.run_steps(5, graph=graph)
    gpu.stream.synchronize()
    after = (host(gpu.tokens), host(gpu.control), host(gpu.layers[0]["value_cache"]), host(gpu.logits))
    assert all(np.array_equal(a, b) for a, b in zip(before, after))


def test_prefill_emitting_the_stop_token_stops_the_decode(small_pair):
    gpu, _ = small_pair
    prompt = synthetic.prompt_ids(SEED + 7, 9, 4096)
    gpu.prefill(prompt)
    gpu.stream.synchronize()
    first = int(host(gpu.tokens)[prompt.size])
    gpu.reset(prompt, stop_token=first)
    gpu.prefill(prompt)  # resets with no stop token, then emits `first` ...
    gpu.stream.synchronize()
    assert gpu.stopped_at() is None
    gpu.reset(prompt, stop_token=first)
    lib = gpu.native.lib
    nbytes = int(lib.kudacuda_qwen2_prefill_workspace_bytes(prompt.size))
    gpu.native.check(lib.kudacuda_qwen2_model_prefill(gpu.model, gpu._prefill_ws.data_ptr(), nbytes, 0, prompt.size,
                                                      gpu.stream.cuda_stream), "prefill")
    gpu.stream.synchronize()
    assert gpu.stopped_at() == prompt.size  # ... and with the stop token set, the prefill's token stops it
    tokens = host(gpu.tokens)
    gpu.run_steps(3)
    gpu.stream.synchronize()
    assert int(host(gpu.control)[0]) == prompt.size and np.array_equal(host(gpu.tokens), tokens)


@pytest.mark.parametrize("prompt_len,new,capacity", [(600, 24, 1024), (1030, 8, 2048)])
def test_long_context_decode_matches_oracle(torch_gpu, native, prompt_len, new, capacity):
    # Decode-step attention past the short-context regime: at 600-624 cached
    # tokens the step's plan (at most 32 splits per KV head) makes 19-20
    # one-round (32-token) splits, more than o_proj merges, so the attention
    # kernel's ticket merge runs; at 1030-1038 tokens the splits grow to two
    # rounds (64 tokens, 17 splits).
    kw = dict(num_layers=2, vocab=4096, kv_capacity=capacity, token_capacity=capacity)
    gpu = Qwen2Nf4Decoder.synthetic(native, torch_gpu, seed=SEED, **kw)
    cpu = HostModel(SEED, **kw)
    try:
        prompt = synthetic.prompt_ids(SEED + 3, prompt_len, 4096)
        assert np.array_equal(gpu.generate(prompt, new), cpu.generate(prompt, new))
        assert np.array_equal(host(gpu.logits), cpu.logits)
        assert np.array_equal(host(gpu.attn), cpu.attn)
    finally:
        gpu.close()


@pytest.mark.parametrize("start,capacity,mode", [
    (2100, 4096, "eager"), (4200, 8192, "eager"),
    (700, 1024, "graph"), (700, 1024, "graph, position unknown"), (189, 1024, "graph"), (509, 1024, "graph"),
    (61, 1024, "graph"), (100, 1024, "graph, position stale low"), (100, 1024, "graph, position stale high"),
    (700, 1024, "graph, position stale low"), (300, 1024, "graph, position unknown"),
])
def test_decode_from_a_seeded_long_cache_matches_oracle(torch_gpu, native, start, capacity, mode):
    # Longer splits inside the decode step: both models get the same random
    # cache rows 0..start-1 and decode from position start.  At 2100+ tokens
    # the step's plan makes 22 splits of three 32-token rounds, at 4200 of an
    # 8192-row cache 27 splits of five rounds, at 700 22 one-round splits.
    # The step runs in the form for the split count at the position the
    # library believes is next: up to 16 splits a form whose o_proj merges
    # exactly that many (from 61 the steps cross 2 -> 3 splits, from 189
    # 6 -> 7), past 16 splits (512 cached tokens) the long-cache form
    # (gqa_merge_kernel merges the splits, o_proj is a plain GEMV; from 509
    # the steps cross into it), and the 6-split form when the position is
    # unknown (past 6 splits the attention kernel's ticket merges: 300 and
    # 700 tokens).  A stale position picks a form made for another length:
    # too few o_proj slots (the attention kernel then merges by its ticket)
    # or the long form at a short cache.  Every case must equal the oracle.
    torch = torch_gpu
    new = 6
    kw = dict(num_layers=2, vocab=4096, kv_capacity=capacity, token_capacity=capacity)
    gpu = Qwen2Nf4Decoder.synthetic(native, torch, seed=SEED, **kw)
    cpu = HostModel(SEED, **kw)
    try:
        for li in range(2):
            _, k, v = synthetic.gqa_inputs(SEED + 10 + li, start, capacity)
            k = k.reshape(2, capacity, 128).copy()
            v = v.reshape(2, capacity, 128).copy()
            k[:, start:] = 0
            v[:, start:] = 0
            cpu.layers[li]["key_cache"][...] = k
            cpu.layers[li]["value_cache"][...] = v
            gpu.layers[li]["key_cache"].copy_(torch.from_numpy(k.view(np.int16)).view(torch.bfloat16))
            gpu.layers[li]["value_cache"].copy_(torch.from_numpy(v.view(np.int16)).view(torch.bfloat16))
        torch.cuda.synchronize()  # the copies ran on torch's current stream, the steps run on the model's
        prompt = synthetic.prompt_ids(SEED + 4, start + 1, 4096)
        gpu.reset(prompt, start_step=start)
        cpu.reset(prompt, start_step=start)
        if mode != "eager":
            gpu.capture()
        if mode == "graph, position unknown":
            gpu._set_position(-1)
        elif mode == "graph, position stale low":
            gpu._set_position(0)  # the one-split form
        elif mode == "graph, position stale high":
            gpu._set_position(capacity - 8)  # the long-cache form
        print(f"seeded cache: start {start}, capacity {capacity}, {mode}", flush=True)
        for step in range(new):
            if mode == "eager":
                gpu.step()
            else:
                gpu.replay(1)
            gpu.stream.synchronize()
            cpu.step()
            ctx = f"position {start + step}"
            assert np.array_equal(host(gpu.attn), cpu.attn), ctx
            assert np.array_equal(host(gpu.hidden), cpu.hidden), ctx
            assert np.array_equal(host(gpu.logits), cpu.logits), ctx
        assert np.array_equal(host(gpu.tokens)[: start + new + 1], cpu.tokens[: start + new + 1])
    finally:
        gpu.close()
