"""The PyTorch-CPU baseline (oracle/torch_cpu.py) computes the same model.

It is the timing baseline beside the GPU numbers, so it must compute the
decode step, not an approximation of its cost: its dequantisation equals
the oracle's bit for bit, its ops match the fp64 textbook references, and a
2-layer decode tracks the independent fp64 decoder's logits and tokens.
"""

from __future__ import annotations

import numpy as np
import pytest

torch = pytest.importorskip("torch")

from kudacuda_amd import synthetic  # noqa: E402
from oracle import oracle as O  # noqa: E402
from oracle import reference as R  # noqa: E402
from oracle import torch_cpu as T  # noqa: E402
from tests._f64_decoder import F64Decoder  # noqa: E402
from tests._host_model import HostModel  # noqa: E402

SEED = 20260824


def test_dequantize_equals_the_oracle():
    _, w = synthetic.gemv_inputs(SEED, 256, 2048)
    packed, absmax = O.nf4_quantize(w)
    got = T.dequantize(torch.from_numpy(packed), torch.from_numpy(absmax), 256, 2048).numpy()
    assert np.array_equal(got.reshape(-1).view(np.uint32), O.nf4_dequantize(packed, absmax, w.size).view(np.uint32))


def test_ops_match_fp64():
    x, gamma, w, b = synthetic.qkv_inputs(SEED)
    q = {n: O.nf4_quantize(w[n]) for n in ("q", "k", "v")}
    deq = {n: T.dequantize(torch.from_numpy(q[n][0]), torch.from_numpy(q[n][1]), *w[n].shape) for n in q}
    xs, gs = T.bf16_bits_to_f32(x), T.bf16_bits_to_f32(gamma)
    bias = {n: T.bf16_bits_to_f32(b[n]) for n in b}
    got = T.qkv(xs, gs, 1e-6, deq["q"], bias["q"], deq["k"], bias["k"], deq["v"], bias["v"])
    xn = R.rmsnorm_f64(O.bf16_to_f32(x), O.bf16_to_f32(gamma), 1e-6)
    for out, n in zip(got, ("q", "k", "v")):
        W = R.nf4_dequant_f64(q[n][0], q[n][1], w[n].size).reshape(w[n].shape)
        want = W @ xn + O.bf16_to_f32(b[n])
        assert np.abs(out.numpy() - want).max() <= 1e-4 * np.abs(want).max()
    for kv_len in (1, 37, 600):
        qq, k, v = synthetic.gqa_inputs(SEED, kv_len)
        att = T.gqa(T.bf16_bits_to_f32(qq).reshape(16, 128), T.bf16_bits_to_f32(k).reshape(2, kv_len, 128),
                    T.bf16_bits_to_f32(v).reshape(2, kv_len, 128), synthetic.default_scale())
        want = R.gqa_f64(O.bf16_to_f32(qq), O.bf16_to_f32(k).reshape(2, kv_len, 128),
                         O.bf16_to_f32(v).reshape(2, kv_len, 128), kv_len, synthetic.default_scale())
        assert np.abs(att.numpy().reshape(-1) - want.reshape(-1)).max() <= 1e-5


def test_decode_tracks_the_fp64_decoder():
    hm = HostModel(SEED, num_layers=2, vocab=4096, kv_capacity=32, token_capacity=32)
    ref = F64Decoder(hm)
    dec = T.TorchCpuDecoder(hm.layers, hm.embed, hm.final_norm, eps=hm.cfg.eps, capacity=32)
    token = int(synthetic.prompt_ids(SEED, 1, 4096)[0])
    agree = 0
    for pos in range(12):
        want = ref.step(token, pos)
        got = dec.step(token, pos)
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 2 ** -5 * np.abs(want).max():  # beyond bf16 storage noise
            assert got == int(np.argmax(want)), pos
            agree += 1
        token = int(np.argmax(want))
    assert agree >= 6
