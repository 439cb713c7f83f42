"""GPU: the Python bridge drives the real library with PyTorch-ROCm tensors.

Every dispatch goes through ``KudaCudaBridge`` (contract checks, ctypes
marshalling, the caller's stream) and must reproduce the oracle bit for bit,
as the C-ABI tests do.  Weights are bitsandbytes-layout NF4 parameters made by
``kudacuda_amd.nf4_params``.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from kudacuda_amd import kudacuda_sidecar as S
from kudacuda_amd import nf4_params as P
from oracle import oracle as O
from tests._gpu_util import host

pytestmark = pytest.mark.gpu
SEED = 20260824


@pytest.fixture(scope="module")
def bridge(torch_gpu):
    b = S.KudaCudaBridge()
    yield b
    b.shutdown()


def _bf16(torch, array: np.ndarray, shape=None):
    t = torch.from_numpy(np.ascontiguousarray(array).view(np.int16)).view(torch.bfloat16).to("cuda:0")
    return t.reshape(shape) if shape is not None else t


def _nf4(torch, bridge, rng, rows, cols, std=0.02):
    w = torch.from_numpy(rng.standard_normal((rows, cols)).astype(np.float32) * np.float32(std)).to("cuda:0")
    packed = P.quantize_weight(bridge, torch, w)
    torch.cuda.synchronize()
    return packed, (host(packed).reshape(-1), host(packed.quant_state.absmax))


def test_every_manifest_tactic_resolves_on_the_real_library(bridge):
    for name in bridge.implemented_tactics | bridge.experimental_tactics:
        assert bridge.tactic_status(name) in ("implemented", "experimental"), name
    assert bridge.matches_contract("qwen2_gqa_decode_gfx950_bf16", 1, 1)


@pytest.mark.parametrize("kv_len", [1, 77, 1024])
def test_gqa_direct_and_graph_match_the_oracle(torch_gpu, bridge, kv_len):
    torch = torch_gpu
    rng = np.random.default_rng([SEED, kv_len])
    q = O.f32_to_bf16(rng.standard_normal(2048).astype(np.float32))
    k = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(np.float32))
    v = O.f32_to_bf16(rng.standard_normal((2, kv_len, 128)).astype(np.float32))
    want = O.gqa(q, k, v, kv_len)
    qt, kt, vt = _bf16(torch, q, (1, 16, 1, 128)), _bf16(torch, k, (1, 2, kv_len, 128)), _bf16(torch, v, (1, 2, kv_len, 128))
    out = torch.empty_like(qt)
    stream = torch.cuda.current_stream().cuda_stream
    bridge.dispatch_qwen2_gqa_decode(qt, kt, vt, out, kv_len=kv_len, stream_ptr=stream)
    torch.cuda.synchronize()
    assert host(out).reshape(-1).tobytes() == want.tobytes()
    # graph tactic: same cache in a larger bucket, valid length from device memory
    cap = 2048
    kb = torch.zeros((1, 2, cap, 128), dtype=torch.bfloat16, device="cuda:0")
    vb = torch.zeros_like(kb)
    kb[:, :, :kv_len] = kt
    vb[:, :, :kv_len] = vt
    kv_dev = torch.tensor([kv_len], dtype=torch.int32, device="cuda:0")
    out2 = torch.empty_like(qt)
    bridge.dispatch_qwen2_gqa_decode_graph(qt, kb, vb, out2, kv_capacity=cap, kv_len_device=kv_dev,
                                           stream_ptr=stream)
    torch.cuda.synchronize()
    want_cap = O.gqa(q, host(kb).reshape(2, cap, 128), host(vb).reshape(2, cap, 128), kv_len)
    assert host(out2).reshape(-1).tobytes() == want_cap.tobytes()


def test_fused_qkv_bf16_through_the_bridge(torch_gpu, bridge):
    torch = torch_gpu
    rng = np.random.default_rng(SEED)
    x = O.f32_to_bf16(rng.standard_normal(2048).astype(np.float32))
    gamma = O.f32_to_bf16(np.float32(1) + rng.standard_normal(2048).astype(np.float32) * np.float32(0.02))
    ws, hs, bs = [], [], []
    for rows in (2048, 256, 256):
        w, h = _nf4(torch, bridge, rng, rows, 2048)
        b = O.f32_to_bf16(rng.standard_normal(rows).astype(np.float32) * np.float32(0.02))
        ws.append(w), hs.append(h), bs.append(b)
    outs = [torch.empty((1, n), dtype=torch.bfloat16, device="cuda:0") for n in (2048, 256, 256)]
    args = [_bf16(torch, x, (1, 2048)), _bf16(torch, gamma)]
    for w, b in zip(ws, bs):
        args += [w, w.quant_state.absmax, _bf16(torch, b)]
    bridge.dispatch_qwen2_fused_rmsnorm_qkv_nf4(*args, *outs, epsilon=1e-6,
                                                stream_ptr=torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    want = O.qkv(x, gamma, 1e-6, (*hs[0], bs[0]), (*hs[1], bs[1]), (*hs[2], bs[2]), dtype="bf16")
    for got, exp in zip(outs, want):
        assert host(got).reshape(-1).tobytes() == exp.tobytes()


def test_swiglu_mlp_gemv_and_lm_head_through_the_bridge(torch_gpu, bridge):
    torch = torch_gpu
    rng = np.random.default_rng(SEED + 1)
    x = O.f32_to_bf16(rng.standard_normal(2048).astype(np.float32))
    gamma = O.f32_to_bf16(np.float32(1) + rng.standard_normal(2048).astype(np.float32) * np.float32(0.02))
    gw, gh = _nf4(torch, bridge, rng, 11008, 2048)
    uw, uh = _nf4(torch, bridge, rng, 11008, 2048)
    dw, dh = _nf4(torch, bridge, rng, 2048, 11008)
    stream = torch.cuda.current_stream().cuda_stream
    xt, gt = _bf16(torch, x, (1, 2048)), _bf16(torch, gamma)
    h = torch.empty((1, 11008), dtype=torch.bfloat16, device="cuda:0")
    bridge.dispatch_qwen2_swiglu_nf4_bf16(xt, gt, gw, gw.quant_state.absmax, uw, uw.quant_state.absmax, h,
                                          epsilon=1e-6, stream_ptr=stream)
    torch.cuda.synchronize()
    want_h = O.swiglu(x, gamma, 1e-6, gh, uh)
    assert host(h).reshape(-1).tobytes() == want_h.tobytes()

    out = torch.empty((1, 2048), dtype=torch.bfloat16, device="cuda:0")
    inter = torch.empty((1, 11008), dtype=torch.bfloat16, device="cuda:0")
    bridge.dispatch_qwen2_mlp_nf4_bf16(xt, gt, gw, gw.quant_state.absmax, uw, uw.quant_state.absmax, dw,
                                       dw.quant_state.absmax, inter, out, residual=xt, epsilon=1e-6,
                                       stream_ptr=stream)
    torch.cuda.synchronize()
    want = O.down11008(want_h, *dh, residual=x)
    assert host(out).reshape(-1).tobytes() == want.tobytes()

    ow, oh = _nf4(torch, bridge, rng, 2048, 2048)
    y = torch.empty((1, 2048), dtype=torch.bfloat16, device="cuda:0")
    bridge.dispatch_nf4_gemv_bf16(xt, ow, ow.quant_state.absmax, y, residual=xt, stream_ptr=stream)
    torch.cuda.synchronize()
    assert host(y).reshape(-1).tobytes() == O.nf4_gemv2048(x, *oh, 2048, residual=x).tobytes()

    table = O.f32_to_bf16(rng.standard_normal((4096, 2048)).astype(np.float32) * np.float32(0.02))
    tok = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    logits = torch.empty((1, 4096), dtype=torch.bfloat16, device="cuda:0")
    bridge.lm_head_argmax_bf16(xt, gt, _bf16(torch, table, (4096, 2048)), tok, logits=logits, epsilon=1e-6,
                               stream_ptr=stream)
    torch.cuda.synchronize()
    want_tok, want_logits = O.lm_head_argmax(x, gamma, 1e-6, table)
    assert int(tok.item()) == want_tok
    assert host(logits).reshape(-1).tobytes() == want_logits.tobytes()


def test_dequantize_and_nf4_linear_framework_path(torch_gpu, bridge):
    torch = torch_gpu
    rng = np.random.default_rng(SEED + 2)
    lin = torch.nn.Linear(2048, 512, bias=True).to(device="cuda:0", dtype=torch.bfloat16)
    mod = P.make_nf4_linear(bridge, torch, lin)
    packed, absmax = host(mod.weight).reshape(-1), host(mod.weight.quant_state.absmax)
    dense = P.dequantize(bridge, torch, mod.weight, dtype=torch.float32)
    torch.cuda.synchronize()
    assert host(dense).reshape(-1).tobytes() == O.nf4_dequantize(packed, absmax, 512 * 2048).tobytes()
    x = torch.from_numpy(rng.standard_normal((1, 2048)).astype(np.float32)).to("cuda:0", torch.bfloat16)
    y = mod(x).float()
    ref = x.float() @ dense.t().contiguous() + lin.bias.float()
    assert torch.allclose(y, ref, rtol=2e-2, atol=2e-2)


def test_bridge_error_surfaces_native_message(torch_gpu, bridge):
    torch = torch_gpu
    with pytest.raises(S.NativeCudaError, match="kudacuda_nf4_quantize failed"):
        bridge.call("kudacuda_nf4_quantize", 0, 0, 64, 64, 0, 0, 0)
