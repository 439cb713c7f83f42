"""The allocation-free GQA entry point against the allocating one.

kudacuda_qwen2_gqa_decode_graph_bf16_noalloc keeps its split partials and
ticket counters in the library's static device array; its output must equal
kudacuda_qwen2_gqa_decode_graph_bf16's bit for bit (and the oracle's) on two
calls in a row, the second with a smaller cache and kv_len, so state left by
the first call cannot leak into the second.  It is also replayed from a
captured graph with a new device kv_len before each replay (the ticket
counters in the shared array must be back at zero after every call), and a
call must leave the device's free memory unchanged.
"""

from __future__ import annotations

import numpy as np
import pytest

from kudacuda_amd import synthetic
from oracle import oracle as O
from tests._gpu_util import dev, empty, host, p

pytestmark = pytest.mark.gpu

SEED = 20260824
ARGS_TAIL = (16, 2, 128)
TICKET_MAX = 16  # standalone calls: up to this many splits the last block merges in-kernel


def _call(native, symbol, d_q, d_k, d_v, out, capacity, d_len, stream):
    native.call(symbol, p(d_q), p(d_k), p(d_v), p(out), 1, 1, capacity, *ARGS_TAIL, synthetic.default_scale(),
                p(d_len), stream.cuda_stream)


def _route(kv_len: int, capacity: int) -> str:
    """How the kernels finish this call: the split count of the graph-mode
    plan for the cache's capacity, then in place / ticket / merge kernel."""

    split_cap, _ = O.gqa_plan(capacity)
    per = O.gqa_split_tokens(kv_len, split_cap)
    splits = -(-kv_len // per)
    if splits == 1:
        return "in place"
    return "ticket" if splits <= TICKET_MAX else f"merge kernel ({splits} splits)"


# (kv_len, capacity) pairs, each run twice in a row: large first, then smaller.
# Routes (split cap 256 per KV head, one-round splits up to 8192 tokens):
# 8000 of 32768 -> 250 splits, merge kernel; 1500 of 2048 -> 47, merge kernel;
# 600 of 2048 -> 19, merge kernel (17-32 splits: the merge kernel's first
# group of 16 plus a second); 512 of 512 -> 16, ticket at its limit; 100 of
# 512 -> 4, ticket; 1 of 64 -> one split, finished in place.
SEQUENCES = [((8000, 32768), (1500, 2048)), ((1500, 2048), (600, 2048)), ((600, 2048), (512, 512)),
             ((512, 512), (100, 512)), ((100, 512), (1, 64))]
ROUTES = {(8000, 32768): "merge kernel (250 splits)", (1500, 2048): "merge kernel (47 splits)",
          (600, 2048): "merge kernel (19 splits)", (512, 512): "ticket", (100, 512): "ticket", (1, 64): "in place"}


def test_routes_are_the_ones_the_cases_claim():
    for case, route in ROUTES.items():
        assert _route(*case) == route, case


@pytest.mark.parametrize("first,second", SEQUENCES)
def test_noalloc_matches_allocating_entry_point(torch_gpu, native, stream, first, second):
    torch = torch_gpu
    for kv_len, capacity in (first, second):
        print(f"[no_alloc] kv_len {kv_len} capacity {capacity}: {_route(kv_len, capacity)}", flush=True)
        q, k, v = synthetic.gqa_inputs(SEED + kv_len, kv_len, capacity)
        d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
        d_len = dev(torch, np.array([kv_len], dtype=np.int32))
        want = empty(torch, 2048, "u16")
        got = empty(torch, 2048, "u16")
        _call(native, "kudacuda_qwen2_gqa_decode_graph_bf16", d_q, d_k, d_v, want, capacity, d_len, stream)
        _call(native, "kudacuda_qwen2_gqa_decode_graph_bf16_noalloc", d_q, d_k, d_v, got, capacity, d_len, stream)
        stream.synchronize()
        assert np.array_equal(host(got), host(want)), (kv_len, capacity)
        assert np.array_equal(host(got), O.gqa(q, k, v, kv_len)), (kv_len, capacity)


def test_noalloc_call_leaves_free_device_memory_unchanged(torch_gpu, native, stream):
    torch = torch_gpu
    kv_len, capacity = 1500, 2048
    q, k, v = synthetic.gqa_inputs(SEED, kv_len, capacity)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    d_len = dev(torch, np.array([kv_len], dtype=np.int32))
    out = empty(torch, 2048, "u16")
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        _call(native, "kudacuda_qwen2_gqa_decode_graph_bf16_noalloc", d_q, d_k, d_v, out, capacity, d_len, stream)
    stream.synchronize()
    free_after, _ = torch.cuda.mem_get_info()
    assert free_after == free_before
    assert np.array_equal(host(out), O.gqa(q, k, v, kv_len))


def test_noalloc_replays_from_a_captured_graph_with_new_lengths(torch_gpu, native, stream):
    """One call captured through the handle's graph API, replayed for device
    kv_lens that take every route in turn (merge kernel, ticket, in place,
    ticket again): each replay equals the oracle, so the shared counters are
    back at zero after each."""

    torch = torch_gpu
    capacity = 2048
    q, k, v = synthetic.gqa_inputs(SEED + 7, capacity, capacity)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    d_len = dev(torch, np.array([capacity], dtype=np.int32))
    out = empty(torch, 2048, "u16")
    lib, h, s = native.lib, native.handle, stream.cuda_stream
    torch.cuda.synchronize()
    assert lib.kudacuda_begin_capture(h, s) == 0, native.error()
    status = lib.kudacuda_qwen2_gqa_decode_graph_bf16_noalloc(h, p(d_q), p(d_k), p(d_v), p(out), 1, 1, capacity,
                                                              *ARGS_TAIL, synthetic.default_scale(), p(d_len), s)
    assert lib.kudacuda_end_capture(h, s) == 0, native.error()
    assert status == 0
    try:
        for kv_len in (2048, 300, 1, 40, 1999, 2048):
            print(f"[no_alloc graph] replay at kv_len {kv_len}: {_route(kv_len, capacity)}", flush=True)
            with torch.cuda.stream(stream):
                d_len.fill_(kv_len)
            assert lib.kudacuda_replay_graph(h, s) == 0, native.error()
            stream.synchronize()
            assert np.array_equal(host(out), O.gqa(q, k, v, kv_len)), kv_len
    finally:
        assert lib.kudacuda_reset_graph(h) == 0


def test_noalloc_rejects_capacity_beyond_its_scratch(torch_gpu, native, stream):
    torch = torch_gpu
    d_q = empty(torch, 2048, "u16")
    d_len = dev(torch, np.array([1], dtype=np.int32))
    lib = native.lib
    status = lib.kudacuda_qwen2_gqa_decode_graph_bf16_noalloc(
        native.handle, p(d_q), p(d_q), p(d_q), p(d_q), 1, 1, 65537, *ARGS_TAIL, synthetic.default_scale(), p(d_len),
        stream.cuda_stream)
    assert status == 1
    assert "kv_capacity=1..65536" in native.error()
