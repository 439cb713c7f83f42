"""The allocation-free GQA entry point against the allocating one.

kudacuda_qwen2_gqa_decode_graph_bf16_noalloc keeps its split partials and
ticket counters in the library's static device array; its output must equal
kudacuda_qwen2_gqa_decode_graph_bf16's bit for bit (and the oracle's) on two
calls in a row, the second with a smaller cache and kv_len, so state left by
the first call cannot leak into the second.
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


def _call(native, symbol, d_q, d_k, d_v, out, capacity, d_len, stream):
    native.call(symbol, p(d_q), p(d_k), p(d_v), p(out), 1, 1, capacity, *ARGS_TAIL, synthetic.default_scale(),
                p(d_len), stream.cuda_stream)


# (kv_len, capacity) pairs, each run twice in a row: large first, then smaller.
# 8000 of 32768 takes the round path and the separate merge kernel, 1500 of
# 2048 the two-token flat path with the ticket merge, 100 of 512 the flat
# path, 1 of 64 a single split.
SEQUENCES = [((8000, 32768), (1500, 2048)), ((1500, 2048), (100, 512)), ((100, 512), (1, 64))]


@pytest.mark.parametrize("first,second", SEQUENCES)
def test_noalloc_matches_allocating_entry_point(torch_gpu, native, stream, first, second):
    torch = torch_gpu
    for kv_len, capacity in (first, second):
        print(f"[no_alloc] kv_len {kv_len} capacity {capacity}", flush=True)
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


def test_noalloc_rejects_capacity_beyond_its_scratch(torch_gpu, native, stream):
    torch = torch_gpu
    d_q = empty(torch, 2048, "u16")
    d_len = dev(torch, np.array([1], dtype=np.int32))
    lib = native.lib
    status = lib.kudacuda_qwen2_gqa_decode_graph_bf16_noalloc(
        native.handle, p(d_q), p(d_q), p(d_q), p(d_q), 1, 1, 32769, *ARGS_TAIL, synthetic.default_scale(), p(d_len),
        stream.cuda_stream)
    assert status == 1
    assert "kv_capacity=1..32768" in native.error()
