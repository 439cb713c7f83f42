"""GPU: double-quantised (nested) Params4bit weights through the native path.

bitsandbytes stores the absmax of a 4-bit weight loaded with
``compress_statistics=True`` (the reference's chat tool loads its checkpoint
that way, tools/chat_qwen2_kudacuda.py:244-249) as 8-bit codes: the fp32
absmax minus its mean (``offset``) is quantised blockwise (256 values per
block, per-block absmax ``state2.absmax``) against the signed dynamic 8-bit
map ``state2.code``.  This test writes such a state from that published
algorithm (T. Dettmers et al., "8-bit Optimizers via Block-wise
Quantization", 2022: the dynamic map and nearest-code blockwise
quantisation, as bitsandbytes' quantize_4bit / quantize_blockwise implement
it) -- not from ``nf4_params.denest`` -- hands the nested parameter to
``nf4_params.adopt_params4bit``, and runs the native fused RMSNorm+QKV (through
the bridge, which validates the Params4bit layout, reference
python/kudacuda_sidecar.py:1018-1049) and SwiGLU (through the C ABI) with it.
The flattened absmax must equal code[q] * absmax2 + offset computed here in
fp32; the outputs must equal the oracle on that absmax bit for bit and lie
within rel 1e-2 / abs 1e-3 of an fp64 dequantised product.  Parity with
bitsandbytes' own kernels is unpinned (bitsandbytes is not installed).
"""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from kudacuda_amd import kudacuda_sidecar as S
from kudacuda_amd import nf4_params as P
from kudacuda_amd import synthetic
from oracle import oracle as O
from oracle import reference as R
from tests._gpu_util import dev, empty, host, p

pytestmark = pytest.mark.gpu

SEED = 20260824
ATOL, RTOL = 1.0e-3, 1.0e-2
QKV_TACTIC = "qwen2_fused_rmsnorm_qkv_gfx950_bf16_nf4_v1"


def dynamic_map_signed() -> np.ndarray:
    """The signed dynamic 8-bit quantisation map (7 exponent bits): for
    exponent i = 0..6, 2^i linearly spaced fractions in (0.1, 1] (bin
    midpoints) scaled by 10^(i-6), both signs, plus 0 and 1; sorted."""

    values = [0.0, 1.0]
    for i in range(7):
        bounds = np.linspace(0.1, 1.0, 2 ** i + 1, dtype=np.float32)
        means = (bounds[:-1] + bounds[1:]) / np.float32(2.0)
        scaled = (10.0 ** (i - 6)) * means.astype(np.float64)
        values += scaled.tolist() + (-scaled).tolist()
    code = np.sort(np.asarray(values, dtype=np.float32))
    assert code.size == 256
    return code


def double_quantize(absmax: np.ndarray, code: np.ndarray, block: int = 256):
    """(uint8 codes, per-block fp32 absmax2, fp32 offset) of a fp32 absmax."""

    offset = np.float32(absmax.astype(np.float64).mean())
    centred = (absmax - offset).astype(np.float32)
    n = centred.size
    blocks = (n + block - 1) // block
    padded = np.zeros(blocks * block, dtype=np.float32)
    padded[:n] = centred
    absmax2 = np.abs(padded.reshape(blocks, block)).max(axis=1).astype(np.float32)
    scaled = (padded.reshape(blocks, block) / absmax2[:, None]).astype(np.float32).reshape(-1)[:n]
    # nearest code value (the map is sorted: compare the two neighbours)
    hi = np.clip(np.searchsorted(code, scaled), 1, 255)
    lo = hi - 1
    q = np.where(np.abs(code[hi] - scaled) < np.abs(scaled - code[lo]), hi, lo).astype(np.uint8)
    return q, absmax2, offset


def flattened_absmax(q: np.ndarray, absmax2: np.ndarray, code: np.ndarray, offset: np.float32,
                     block: int = 256) -> np.ndarray:
    """bitsandbytes' dequantize_blockwise(q, state2) + offset, in fp32."""

    return (code[q] * absmax2[np.arange(q.size) // block]).astype(np.float32) + offset


def nested_param(torch, w32: np.ndarray, code: np.ndarray):
    """A Params4bit-shaped parameter with a nested quant_state, and the fp32
    absmax it stands for: codes NF4-quantised by the oracle, absmax double
    quantised here."""

    rows, cols = w32.shape
    packed, absmax = O.nf4_quantize(w32)
    q, absmax2, offset = double_quantize(absmax, code)
    state = SimpleNamespace(
        absmax=dev(torch, q), shape=(rows, cols), blocksize=64, quant_type="nf4", nested=True,
        offset=torch.tensor(float(offset), dtype=torch.float32, device="cuda:0"), dtype=torch.bfloat16,
        state2=SimpleNamespace(absmax=dev(torch, absmax2), code=dev(torch, code), blocksize=256))
    param = dev(torch, packed).reshape(-1, 1)  # the packed storage carries its state, as a Params4bit does
    param.quant_state = state
    return param, packed, flattened_absmax(q, absmax2, code, offset)


def _close(actual_bits: np.ndarray, expected_f64: np.ndarray) -> None:
    actual = O.bf16_to_f32(actual_bits).astype(np.float64)
    expected = O.bf16_to_f32(O.f32_to_bf16(expected_f64.astype(np.float32))).astype(np.float64)
    bad = np.abs(actual - expected) > ATOL + RTOL * np.abs(expected)
    assert not bad.any(), f"{bad.sum()} elements outside tolerance"


def test_dynamic_map_is_the_signed_8bit_map():
    code = dynamic_map_signed()
    assert code[0] == -code[-2] and code[-1] == 1.0 and (code == 0).sum() == 1
    assert np.all(np.diff(code) > 0) and np.all(np.abs(code) <= 1.0)


def test_nested_qkv_through_the_bridge(torch_gpu, native):
    torch = torch_gpu
    code = dynamic_map_signed()
    x, gamma, w, b = synthetic.qkv_inputs(SEED)
    bridge = S.KudaCudaBridge()
    try:
        adopted, packed, absmax = {}, {}, {}
        for n in ("q", "k", "v"):
            param, packed[n], absmax[n] = nested_param(torch, w[n], code)
            # the bridge takes only the flat Params4bit layout ...
            with pytest.raises(ValueError, match="nested"):
                bridge._validate_nf4_weight(param, param.quant_state.absmax,
                                            expected_shape=param.quant_state.shape, label=n)
            # ... which adopt_params4bit produces from the nested state
            adopted[n] = P.adopt_params4bit(torch, param)
            assert not adopted[n].quant_state.nested
            got_absmax = host(adopted[n].quant_state.absmax)
            assert np.array_equal(got_absmax.view(np.uint32), absmax[n].view(np.uint32)), n
        as_bf16 = lambda bits, shape: dev(torch, bits).view(torch.bfloat16).reshape(shape)  # noqa: E731
        d_x, d_g = as_bf16(x, (1, 2048)), as_bf16(gamma, (2048,))
        outs = {n: torch.empty((1, r), dtype=torch.bfloat16, device="cuda:0")
                for n, r in (("q", 2048), ("k", 256), ("v", 256))}
        stream = torch.cuda.current_stream()
        bridge.dispatch_qwen2_fused_rmsnorm_qkv_nf4(
            d_x, d_g,
            adopted["q"], adopted["q"].quant_state.absmax, as_bf16(b["q"], (2048,)),
            adopted["k"], adopted["k"].quant_state.absmax, as_bf16(b["k"], (256,)),
            adopted["v"], adopted["v"].quant_state.absmax, as_bf16(b["v"], (256,)),
            outs["q"], outs["k"], outs["v"], epsilon=1.0e-6, stream_ptr=stream.cuda_stream, tactic_name=QKV_TACTIC)
        torch.cuda.synchronize()
        want = O.qkv(x, gamma, 1.0e-6, *((packed[n], absmax[n], b[n]) for n in ("q", "k", "v")))
        xn = R.rmsnorm_f64(O.bf16_to_f32(x), O.bf16_to_f32(gamma), 1.0e-6)
        for (n, rows), ref in zip((("q", 2048), ("k", 256), ("v", 256)), want):
            got = host(outs[n]).reshape(-1)
            assert np.array_equal(got, ref), n
            W = R.nf4_dequant_f64(packed[n], absmax[n], rows * 2048).reshape(rows, 2048)
            _close(got, W @ xn + O.bf16_to_f32(b[n]))
    finally:
        bridge.shutdown()


def test_nested_swiglu_through_the_c_abi(torch_gpu, native, stream):
    torch = torch_gpu
    code = dynamic_map_signed()
    x, gate, up, _ = synthetic.mlp_inputs(SEED)
    gamma = synthetic.f32_to_bf16_bits(np.ones(2048, dtype=np.float32))
    g_param, g_packed, g_absmax = nested_param(torch, gate, code)
    u_param, u_packed, u_absmax = nested_param(torch, up, code)
    g, u = P.adopt_params4bit(torch, g_param), P.adopt_params4bit(torch, u_param)
    d_x, d_g = dev(torch, x), dev(torch, gamma)
    out = empty(torch, 11008, "u16")
    torch.cuda.synchronize()
    native.call("kudacuda_qwen2_swiglu_nf4_bf16", p(d_x), p(d_g), p(g), p(g.quant_state.absmax), p(u),
                p(u.quant_state.absmax), p(out), 1, 2048, 11008, 64, 1.0e-6, stream.cuda_stream)
    stream.synchronize()
    got = host(out)
    assert np.array_equal(got, O.swiglu(x, gamma, 1.0e-6, (g_packed, g_absmax), (u_packed, u_absmax)))
    xn = R.rmsnorm_f64(O.bf16_to_f32(x), O.bf16_to_f32(gamma), 1.0e-6)
    gv = R.nf4_dequant_f64(g_packed, g_absmax, 11008 * 2048).reshape(11008, 2048) @ xn
    uv = R.nf4_dequant_f64(u_packed, u_absmax, 11008 * 2048).reshape(11008, 2048) @ xn
    _close(got, gv / (1.0 + np.exp(-gv)) * uv)
