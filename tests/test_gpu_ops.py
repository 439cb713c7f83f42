"""GPU parity of every decode-path op, called through the C ABI.

Each kernel's output must equal the oracle bit for bit (integer/byte results
and the fixed-order fp32 ops alike) and lie within the benchmark's stated
tolerance of an fp64 textbook reference: rel 1e-2 / abs 1e-3 after bf16
rounding.  Inputs are the BASELINE configs, seeded.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from kudacuda_amd import synthetic
from oracle import oracle as O
from oracle import reference as R
from tests._gpu_util import dev, empty, host, p

pytestmark = pytest.mark.gpu

SEED = 20260824
ATOL, RTOL = 1.0e-3, 1.0e-2


def _close(actual_bits: np.ndarray, expected_f64: np.ndarray, dtype: str = "bf16", atol=ATOL, rtol=RTOL) -> None:
    actual = O.act_to_f32(actual_bits, dtype).astype(np.float64)
    # the fp64 reference is itself rounded to the output dtype before comparing
    expected = O.act_to_f32(O.f32_to_act(expected_f64.astype(np.float32), dtype), dtype).astype(np.float64)
    bad = np.abs(actual - expected) > atol + rtol * np.abs(expected)
    assert not bad.any(), f"{bad.sum()} elements outside tolerance; max abs err {np.abs(actual - expected).max()}"


def _bf16_round(v: np.ndarray) -> np.ndarray:
    return O.bf16_to_f32(O.f32_to_bf16(np.asarray(v, dtype=np.float32))).astype(np.float64)


def _quantize_gpu(torch, native, stream, w32: np.ndarray):
    n = w32.size
    src = dev(torch, w32.reshape(-1))
    packed = empty(torch, n // 2, "u8")
    absmax = empty(torch, n // 64, "f32")
    native.call("kudacuda_nf4_quantize", p(src), 0, n, 64, p(packed), p(absmax), stream.cuda_stream)
    stream.synchronize()
    return packed, absmax


def test_nf4_quantize_and_dequantize_are_bit_exact(torch_gpu, native, stream):
    torch = torch_gpu
    _, w = synthetic.gemv_inputs(SEED)
    packed, absmax = _quantize_gpu(torch, native, stream, w)
    ref_packed, ref_absmax = O.nf4_quantize(w)
    assert np.array_equal(host(packed), ref_packed)
    assert np.array_equal(host(absmax).view(np.uint32), ref_absmax.view(np.uint32))

    n = w.size
    out32 = empty(torch, n, "f32")
    native.call("kudacuda_nf4_dequantize", p(packed), p(absmax), n, 64, 0, p(out32), stream.cuda_stream)
    out16 = empty(torch, n, "u16")
    native.call("kudacuda_nf4_dequantize", p(packed), p(absmax), n, 64, 1, p(out16), stream.cuda_stream)
    stream.synchronize()
    deq = O.nf4_dequantize(ref_packed, ref_absmax, n)
    assert np.array_equal(host(out32).view(np.uint32), deq.view(np.uint32))
    assert np.array_equal(host(out16), O.f32_to_bf16(deq))
    # and the dequantised value is the closed form codebook[code] * absmax: the
    # fp64 product of two fp32 values is exact, so its fp32 rounding is the
    # correctly rounded fp32 product
    assert np.array_equal(deq, R.nf4_dequant_f64(ref_packed, ref_absmax, n).astype(np.float32))

    # bf16 input path
    wb = synthetic.f32_to_bf16_bits(w[:256])
    src = dev(torch, wb.reshape(-1))
    pk = empty(torch, wb.size // 2, "u8")
    am = empty(torch, wb.size // 64, "f32")
    native.call("kudacuda_nf4_quantize", p(src), 1, wb.size, 64, p(pk), p(am), stream.cuda_stream)
    stream.synchronize()
    rp, ra = O.nf4_quantize(wb)
    assert np.array_equal(host(pk), rp) and np.array_equal(host(am), ra)


@pytest.mark.parametrize("with_bias,with_residual", [(False, False), (True, False), (False, True)])
def test_nf4_gemv_config1(torch_gpu, native, stream, with_bias, with_residual):
    torch = torch_gpu
    x, w = synthetic.gemv_inputs(SEED)
    packed, absmax = O.nf4_quantize(w)
    bias = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (7,), (2048,), 0.01)) if with_bias else None
    res = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (8,), (2048,), 1.0)) if with_residual else None
    d_x, d_w, d_a = dev(torch, x), dev(torch, packed), dev(torch, absmax)
    d_b = dev(torch, bias) if bias is not None else None
    d_r = dev(torch, res) if res is not None else None
    out = empty(torch, 2048, "u16")
    native.call("kudacuda_nf4_gemv_bf16", p(d_x), p(d_w), p(d_a), p(d_b), p(d_r), p(out), 1, 2048, 2048, 64,
                stream.cuda_stream)
    stream.synchronize()
    got = host(out)
    assert np.array_equal(got, O.nf4_gemv2048(x, packed, absmax, 2048, bias=bias, residual=res))
    ref = R.nf4_dequant_f64(packed, absmax, w.size).reshape(2048, 2048) @ O.bf16_to_f32(x).astype(np.float64)
    if with_bias:
        ref = ref + O.bf16_to_f32(bias)
    if with_residual:
        # residual semantics: the projection is rounded to bf16 before the add
        ref = O.bf16_to_f32(res) + _bf16_round(ref)
    _close(got, ref)


@pytest.mark.parametrize("symbol,dtype,with_norm", [
    ("kudacuda_qwen2_fused_rmsnorm_qkv_nf4_bf16", "bf16", False),
    ("kudacuda_qwen2_fused_rmsnorm_qkv_nf4", "f16", False),
    ("kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v2", "f16", True),
    ("kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v3", "f16", True),
])
def test_fused_rmsnorm_qkv_config2(torch_gpu, native, stream, symbol, dtype, with_norm):
    torch = torch_gpu
    x, gamma, w, b = synthetic.qkv_inputs(SEED)
    if dtype == "f16":
        x = O.f32_to_f16(O.bf16_to_f32(x))
        gamma = O.f32_to_f16(O.bf16_to_f32(gamma))
        b = {k: O.f32_to_f16(O.bf16_to_f32(v)) for k, v in b.items()}
    q = {n: O.nf4_quantize(w[n]) for n in ("q", "k", "v")}
    d = {n: (dev(torch, q[n][0]), dev(torch, q[n][1]), dev(torch, b[n])) for n in q}
    d_x, d_g = dev(torch, x), dev(torch, gamma)
    qo, ko, vo = empty(torch, 2048, "u16"), empty(torch, 256, "u16"), empty(torch, 256, "u16")
    norm = empty(torch, 2048, "f32")
    args = [p(d_x), p(d_g)]
    for n in ("q", "k", "v"):
        args += [p(d[n][0]), p(d[n][1]), p(d[n][2])]
    if with_norm:
        args.append(p(norm))
    args += [p(qo), p(ko), p(vo), 1, 2048, 2048, 256, 64, 1.0e-6, stream.cuda_stream]
    native.call(symbol, *args)
    stream.synchronize()
    eq, ek, ev, enorm = O.qkv(x, gamma, 1.0e-6, (q["q"][0], q["q"][1], b["q"]), (q["k"][0], q["k"][1], b["k"]),
                              (q["v"][0], q["v"][1], b["v"]), dtype=dtype, want_norm=True)
    assert np.array_equal(host(qo), eq)
    assert np.array_equal(host(ko), ek)
    assert np.array_equal(host(vo), ev)
    if with_norm:
        assert np.array_equal(host(norm).view(np.uint32), enorm.view(np.uint32))
    xn = R.rmsnorm_f64(O.act_to_f32(x, dtype), O.act_to_f32(gamma, dtype), 1.0e-6)
    for n, got, rows in (("q", qo, 2048), ("k", ko, 256), ("v", vo, 256)):
        W = R.nf4_dequant_f64(q[n][0], q[n][1], rows * 2048).reshape(rows, 2048)
        _close(host(got), W @ xn + O.act_to_f32(b[n], dtype), dtype)


@pytest.mark.parametrize("symbol,dtype", [("kudacuda_qwen2_swiglu_nf4_bf16", "bf16"),
                                          ("kudacuda_qwen2_swiglu_nf4", "f16")])
def test_swiglu(torch_gpu, native, stream, symbol, dtype):
    torch = torch_gpu
    x, gate, up, _ = synthetic.mlp_inputs(SEED)
    gamma = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (9,), (2048,), 0.1) + np.float32(1.0))
    if dtype == "f16":
        x = O.f32_to_f16(O.bf16_to_f32(x))
        gamma = O.f32_to_f16(O.bf16_to_f32(gamma))
    gq, uq = O.nf4_quantize(gate), O.nf4_quantize(up)
    d_x, d_g = dev(torch, x), dev(torch, gamma)
    d_gw, d_ga, d_uw, d_ua = (dev(torch, a) for a in (*gq, *uq))
    out = empty(torch, 11008, "u16")
    native.call(symbol, p(d_x), p(d_g), p(d_gw), p(d_ga), p(d_uw), p(d_ua), p(out), 1, 2048, 11008, 64, 1.0e-6,
                stream.cuda_stream)
    stream.synchronize()
    got = host(out)
    assert np.array_equal(got, O.swiglu(x, gamma, 1.0e-6, gq, uq, dtype=dtype))
    xn = R.rmsnorm_f64(O.act_to_f32(x, dtype), O.act_to_f32(gamma, dtype), 1.0e-6)
    G = R.nf4_dequant_f64(*gq, gate.size).reshape(11008, 2048) @ xn
    U = R.nf4_dequant_f64(*uq, up.size).reshape(11008, 2048) @ xn
    _close(got, R.silu_f64(G) * U, dtype)


@pytest.mark.parametrize("with_norm,with_residual", [(False, False), (True, True)])
def test_mlp_config3(torch_gpu, native, stream, with_norm, with_residual):
    torch = torch_gpu
    x, gate, up, down = synthetic.mlp_inputs(SEED)
    gamma = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (9,), (2048,), 0.1) + np.float32(1.0))
    res = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (10,), (2048,), 1.0))
    gq, uq, dq = O.nf4_quantize(gate), O.nf4_quantize(up), O.nf4_quantize(down)
    d_x, d_g, d_r = dev(torch, x), dev(torch, gamma), dev(torch, res)
    dd = [dev(torch, a) for a in (*gq, *uq, *dq)]
    h = empty(torch, 11008, "u16")
    out = empty(torch, 2048, "u16")
    native.call("kudacuda_qwen2_mlp_nf4_bf16", p(d_x), p(d_g) if with_norm else 0, *(p(t) for t in dd), p(h),
                p(d_r) if with_residual else 0, p(out), 1, 2048, 11008, 64, 1.0e-6, stream.cuda_stream)
    stream.synchronize()
    eh = O.swiglu(x, gamma if with_norm else None, 1.0e-6, gq, uq)
    assert np.array_equal(host(h), eh)
    eo = O.down11008(eh, *dq, residual=res if with_residual else None)
    assert np.array_equal(host(out), eo)
    xn = R.rmsnorm_f64(O.bf16_to_f32(x), O.bf16_to_f32(gamma) if with_norm else None, 1.0e-6)
    G = R.nf4_dequant_f64(*gq, gate.size).reshape(11008, 2048) @ xn
    U = R.nf4_dequant_f64(*uq, up.size).reshape(11008, 2048) @ xn
    hh = O.bf16_to_f32(O.f32_to_bf16((R.silu_f64(G) * U).astype(np.float32))).astype(np.float64)
    y = R.nf4_dequant_f64(*dq, down.size).reshape(2048, 11008) @ hh
    if with_residual:
        y = O.bf16_to_f32(res) + _bf16_round(y)
    _close(host(out), y)


# Round path (bit-exact to the oracle): one-round (32-token) splits, finished
# in place up to 32 tokens, ticket merge up to 4 splits (128), merge kernel
# beyond, with one merge group up to 512 and more past it.  From
# MFMA_MIN_KV on, direct calls take the matrix-core tactic (splits of 128
# tokens, 2 chunks per wave past 16384, the generic chunk loop past 32768).
KV_LENS = [1, 7, 32, 33, 37, 128, 129, 511, 512, 513, 585, 1024, 2048, 2049, 8191, 8192, 8193, 16385, 32768,
           65536]
MFMA_MIN_KV = 8192  # kGqaMfmaMinKv of kc_runtime.hip


def _matrix_core_parity(got: np.ndarray, q, k, v, kv_len: int, scale: float, dtype: str) -> None:
    """The matrix-core tactic sums in another order than the round path, with
    the weights entering as a 16-bit hi + lo pair.  Every output must lie
    within one step of the output dtype (at the reference's magnitude) plus
    2^-20 -- the fp32 accumulation error of a softmax average, which decides
    near zero -- of the fp64 result, and within twice that of the round-path
    oracle.  A dropped token, split or rescale is far outside either bound."""

    to32 = O.bf16_to_f32 if dtype == "bf16" else O.f16_to_f32
    ref = R.gqa_f64(to32(q), to32(k).reshape(2, kv_len, 128), to32(v).reshape(2, kv_len, 128), kv_len, scale)
    _close(got, ref, dtype)
    rounded = O.f32_to_act(ref.astype(np.float32), dtype)
    step = np.abs(to32((rounded + 1).astype(np.uint16)).astype(np.float64) - to32(rounded).astype(np.float64))
    value = to32(got).astype(np.float64)
    err = np.abs(value - ref)
    assert (err <= step + 2.0**-20).all(), f"max error {err.max():.3e}, {(err > step + 2.0**-20).sum()} outside"
    oracle = to32(O.gqa(q, k, v, kv_len, scale=scale, dtype=dtype)).astype(np.float64)
    assert (np.abs(value - oracle) <= step + 2.0**-19).all()


@pytest.mark.parametrize("kv_len", KV_LENS)
def test_gqa_decode_bf16_config4(torch_gpu, native, stream, kv_len):
    torch = torch_gpu
    q, k, v = synthetic.gqa_inputs(SEED, kv_len)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    out = empty(torch, 2048, "u16")
    scale = synthetic.default_scale()
    native.call("kudacuda_qwen2_gqa_decode_bf16", p(d_q), p(d_k), p(d_v), p(out), 1, 1, kv_len, 16, 2, 128, scale,
                stream.cuda_stream)
    stream.synchronize()
    got = host(out)
    if kv_len >= MFMA_MIN_KV:
        _matrix_core_parity(got, q, k, v, kv_len, scale, "bf16")
        return
    assert np.array_equal(got, O.gqa(q, k, v, kv_len))
    ref = R.gqa_f64(O.bf16_to_f32(q), O.bf16_to_f32(k).reshape(2, kv_len, 128),
                    O.bf16_to_f32(v).reshape(2, kv_len, 128), kv_len, scale)
    _close(got, ref)
    if kv_len == 1:  # a single key: the output is exactly that V row
        assert np.array_equal(got.reshape(16, 128), np.repeat(v.reshape(2, 128), 8, axis=0))


@pytest.mark.parametrize("kv_len,capacity", [(1, 512), (100, 512), (512, 512), (33, 2048), (513, 2048), (585, 2048),
                                             (2048, 2048), (200, 32768), (8000, 32768), (8193, 32768),
                                             (30001, 32768), (32768, 32768)])
def test_gqa_graph_reads_device_kv_len(torch_gpu, native, stream, kv_len, capacity):
    torch = torch_gpu
    q, k, v = synthetic.gqa_inputs(SEED, kv_len, capacity)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    d_len = dev(torch, np.array([kv_len], dtype=np.int32))
    out = empty(torch, 2048, "u16")
    scale = synthetic.default_scale()
    native.call("kudacuda_qwen2_gqa_decode_graph_bf16", p(d_q), p(d_k), p(d_v), p(out), 1, 1, capacity, 16, 2, 128,
                scale, p(d_len), stream.cuda_stream)
    stream.synchronize()
    assert np.array_equal(host(out), O.gqa(q, k, v, kv_len))


@pytest.mark.parametrize("symbol,capacity,excess", [("kudacuda_qwen2_gqa_decode_graph_bf16", 2048, 1),
                                                    ("kudacuda_qwen2_gqa_decode_graph_bf16", 2048, 100000),
                                                    ("kudacuda_qwen2_gqa_decode_workspace_v3", 512, 37)])
def test_gqa_device_kv_len_beyond_capacity_is_clamped(torch_gpu, native, stream, symbol, capacity, excess):
    # a device kv_len past the cache's capacity reads the whole cache and no
    # further, as the reference workspace kernel clamps it
    # (qwen2_gqa_workspace.cuh:35-36)
    torch = torch_gpu
    q, k, v = synthetic.gqa_inputs(SEED + 5, capacity, capacity)
    scale = synthetic.default_scale()
    d_len = dev(torch, np.array([capacity + excess], dtype=np.int32))
    out = empty(torch, 2048, "u16")
    if symbol.endswith("workspace_v3"):
        q = O.f32_to_f16(O.bf16_to_f32(q))
        k, v = (O.f32_to_f16(O.bf16_to_f32(t)).reshape(2, capacity, 128) for t in (k, v))
        d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
        ws = empty(torch, 16 * 8 * 130, "f32")
        native.call(symbol, p(d_q), p(d_k), p(d_v), p(out), p(ws), p(d_len), 1, 1, capacity, 16, 2, 128, scale,
                    stream.cuda_stream)
        stream.synchronize()
        assert np.array_equal(host(out), O.gqa(q, k, v, capacity, scale=scale, dtype="f16", split_limit=8))
    else:
        d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
        native.call(symbol, p(d_q), p(d_k), p(d_v), p(out), 1, 1, capacity, 16, 2, 128, scale, p(d_len),
                    stream.cuda_stream)
        stream.synchronize()
        assert np.array_equal(host(out), O.gqa(q, k, v, capacity))


@pytest.mark.parametrize("symbol", ["kudacuda_qwen2_gqa_decode", "kudacuda_qwen2_gqa_decode_group_tiled",
                                    "kudacuda_qwen2_gqa_decode_vectorized"])
def test_gqa_fp16_reference_entry_points(torch_gpu, native, stream, symbol):
    torch = torch_gpu
    kv_len = 37
    # reference smoke-test fixture (tests/qwen2_gqa_smoke.cu:34-63)
    i_q = np.arange(16 * 128, dtype=np.float32)
    i_c = np.arange(2 * kv_len * 128, dtype=np.float32)
    q = O.f32_to_f16(np.sin(i_q * np.float32(0.017)) * np.float32(0.75))
    k = O.f32_to_f16(np.cos(i_c * np.float32(0.011)) * np.float32(0.55)).reshape(2, kv_len, 128)
    v = O.f32_to_f16(np.sin(i_c * np.float32(0.023)) * np.float32(0.65)).reshape(2, kv_len, 128)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    out = empty(torch, 2048, "u16")
    scale = 1.0 / 11.313708498984761
    native.call(symbol, p(d_q), p(d_k), p(d_v), p(out), 1, 1, kv_len, 16, 2, 128, scale, stream.cuda_stream)
    stream.synchronize()
    got = host(out)
    assert np.array_equal(got, O.gqa(q, k, v, kv_len, scale=scale, dtype="f16"))
    ref = R.gqa_f64(O.f16_to_f32(q), O.f16_to_f32(k), O.f16_to_f32(v), kv_len, scale)
    assert np.abs(O.f16_to_f32(got) - ref).max() <= 3.5e-3  # the smoke test's tolerance


@pytest.mark.parametrize("kv_len,needle", [(8192, 0), (8192, 4100), (9001, 9000), (32768, 20001)])
def test_gqa_matrix_cores_needle_returns_its_value_row(torch_gpu, native, stream, kv_len, needle):
    """One key whose score exceeds every other by >= 72 (log2 units) takes all
    the weight: every other weight is below 2^-72, far under one fp32 step
    of the output, so each head's output is that token's V row exactly --
    whichever split and chunk hold it, and whatever the other splits hold."""
    torch = torch_gpu
    rng = np.random.default_rng(SEED + needle)
    scale = synthetic.default_scale()
    u = rng.standard_normal((2, 128)).astype(np.float32)
    u /= np.linalg.norm(u, axis=1, keepdims=True)
    q32 = np.repeat(u, 8, axis=0) * np.float32(8.0)             # the 8 heads of a group share q
    k32 = rng.standard_normal((2, kv_len, 128)).astype(np.float32) * np.float32(0.01)
    # score (log2 units) = 8 |u|^2 alpha scale log2(e) = 80 for the needle
    k32[:, needle] = u * np.float32(10.0 / (scale * math.log2(math.e)))
    v32 = rng.standard_normal((2, kv_len, 128)).astype(np.float32)
    q, k, v = O.f32_to_bf16(q32), O.f32_to_bf16(k32), O.f32_to_bf16(v32)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    out = empty(torch, 2048, "u16")
    native.call("kudacuda_qwen2_gqa_decode_bf16", p(d_q), p(d_k), p(d_v), p(out), 1, 1, kv_len, 16, 2, 128, scale,
                stream.cuda_stream)
    stream.synchronize()
    got = host(out).reshape(16, 128)
    # the needle's log2-domain score really is >= 72 above every other key's
    qk = np.einsum("gd,gtd->gt", O.bf16_to_f32(q).reshape(16, 128)[::8].astype(np.float64),
                   O.bf16_to_f32(k).astype(np.float64)) * scale * math.log2(math.e)
    others = np.delete(qk, needle, axis=1)
    assert (qk[:, needle] - others.max(axis=1)).min() >= 72.0
    assert np.array_equal(got, np.repeat(v[:, needle], 8, axis=0))


@pytest.mark.parametrize("kv_len", [8192, 9000])
def test_gqa_fp16_long_cache_matrix_cores(torch_gpu, native, stream, kv_len):
    torch = torch_gpu
    q32, k32, v32 = (O.bf16_to_f32(x) for x in synthetic.gqa_inputs(SEED + 1, kv_len))
    q, k, v = O.f32_to_f16(q32), O.f32_to_f16(k32), O.f32_to_f16(v32)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    out = empty(torch, 2048, "u16")
    scale = synthetic.default_scale()
    native.call("kudacuda_qwen2_gqa_decode", p(d_q), p(d_k), p(d_v), p(out), 1, 1, kv_len, 16, 2, 128, scale,
                stream.cuda_stream)
    stream.synchronize()
    _matrix_core_parity(host(out), q, k, v, kv_len, scale, "f16")


def test_gqa_workspace_v3(torch_gpu, native, stream):
    torch = torch_gpu
    capacity = 512
    scale = synthetic.default_scale()
    ws = empty(torch, 16 * 8 * 130, "f32")
    # reference tests/qwen2_gqa_workspace_smoke.cu:29-49, plus the edges of
    # this 8-split workspace's rule (up to 256 tokens one-round splits, then
    # two-round splits)
    for kv_len in (1, 7, 64, 128, 256, 257, 300, 511, 512):
        q, k, v = synthetic.gqa_inputs(SEED + kv_len, kv_len, capacity)
        q16 = O.f32_to_f16(O.bf16_to_f32(q))
        k16 = O.f32_to_f16(O.bf16_to_f32(k)).reshape(2, capacity, 128)
        v16 = O.f32_to_f16(O.bf16_to_f32(v)).reshape(2, capacity, 128)
        d_q, d_k, d_v = dev(torch, q16), dev(torch, k16), dev(torch, v16)
        d_len = dev(torch, np.array([kv_len], dtype=np.int32))
        out = empty(torch, 2048, "u16")
        native.call("kudacuda_qwen2_gqa_decode_workspace_v3", p(d_q), p(d_k), p(d_v), p(out), p(ws), p(d_len), 1, 1,
                    capacity, 16, 2, 128, scale, stream.cuda_stream)
        stream.synchronize()
        assert np.array_equal(host(out), O.gqa(q16, k16, v16, kv_len, split_limit=8, dtype="f16"))


@pytest.mark.parametrize("symbol", ["kudacuda_qwen2_gqa_decode_workspace_v3", "kudacuda_qwen2_gqa_decode_graph",
                                    "kudacuda_qwen2_gqa_decode_graph_bf16"])
@pytest.mark.parametrize("device_len", [0, -3])
def test_gqa_empty_cache_writes_zeros(torch_gpu, native, stream, symbol, device_len):
    # a device kv_len below 1 means an empty cache: the output is zero, as the
    # reference workspace kernel writes (qwen2_gqa_workspace.cuh:118)
    torch = torch_gpu
    capacity = 512
    q, k, v = synthetic.gqa_inputs(SEED, 1, capacity)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    d_len = dev(torch, np.array([device_len], dtype=np.int32))
    out = dev(torch, np.full(2048, 0x3C00, dtype=np.uint16))  # 1.0 in fp16, 1.875 in bf16
    scale = synthetic.default_scale()
    if symbol.endswith("workspace_v3"):
        ws = empty(torch, 16 * 8 * 130, "f32")
        native.call(symbol, p(d_q), p(d_k), p(d_v), p(out), p(ws), p(d_len), 1, 1, capacity, 16, 2, 128, scale,
                    stream.cuda_stream)
    else:
        native.call(symbol, p(d_q), p(d_k), p(d_v), p(out), 1, 1, capacity, 16, 2, 128, scale, p(d_len),
                    stream.cuda_stream)
    stream.synchronize()
    assert not host(out).any()
    assert not O.gqa(q, k, v, 0).any()


@pytest.mark.parametrize("vocab,with_norm", [(151936, True), (1000, False), (1, True)])
def test_lm_head_argmax(torch_gpu, native, stream, vocab, with_norm):
    torch = torch_gpu
    x = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (11,), (2048,), 1.0))
    gamma = synthetic.final_norm_bits(SEED)
    emb = synthetic.embedding_bits(SEED, vocab=vocab)
    d_x, d_g, d_e = dev(torch, x), dev(torch, gamma), dev(torch, emb)
    logits = empty(torch, vocab, "u16")
    arg = empty(torch, 1, "i32")
    native.call("kudacuda_lm_head_argmax_bf16", p(d_x), p(d_g) if with_norm else 0, p(d_e), p(logits), p(arg), vocab,
                2048, 1.0e-6, stream.cuda_stream)
    stream.synchronize()
    tok, elog = O.lm_head_argmax(x, gamma if with_norm else None, 1.0e-6, emb)
    assert np.array_equal(host(logits), elog)
    assert int(host(arg)[0]) == tok
    lf = O.bf16_to_f32(elog)
    assert tok == int(np.argmax(lf))  # first maximum, as torch.argmax


def test_lm_head_argmax_ties_across_waves_and_blocks(torch_gpu, native, stream):
    """One maximal row planted at several indices: in one wave's ring (rows
    3072 apart at 768 blocks of 4 waves), in other blocks and at the last
    row.  Their logits are bit-equal, so the lowest index must win through
    the wave, the block and the one-block winner reduction alike."""
    torch = torch_gpu
    vocab = 151936
    x = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (14,), (2048,), 1.0))
    emb = synthetic.embedding_bits(SEED, vocab=vocab)
    # a row along x, well above every random row's logit
    xf = O.bf16_to_f32(x).astype(np.float64)
    hot = synthetic.f32_to_bf16_bits((0.05 * xf / np.sqrt(np.mean(xf * xf))).astype(np.float32))
    planted = [7, 7 + 3072, 40001, 98765, vocab - 1]
    emb[planted] = hot
    d_x, d_e = dev(torch, x), dev(torch, emb)
    logits = empty(torch, vocab, "u16")
    arg = empty(torch, 1, "i32")
    native.call("kudacuda_lm_head_argmax_bf16", p(d_x), 0, p(d_e), p(logits), p(arg), vocab, 2048, 1.0e-6,
                stream.cuda_stream)
    stream.synchronize()
    tok, elog = O.lm_head_argmax(x, None, 1.0e-6, emb)
    lf = O.bf16_to_f32(elog)
    assert tok == 7 and np.all(lf[planted] == lf.max()) and np.count_nonzero(lf == lf.max()) == len(planted)
    assert np.array_equal(host(logits), elog)
    assert int(host(arg)[0]) == 7


def test_handle_scratch_is_refused_to_a_second_busy_stream(torch_gpu, native, stream):
    """The handle's scratch (here lm_head's block winners) serves
    one stream at a time: a call on another stream is refused while the last
    user's stream still has work queued, and accepted once it is idle."""
    torch = torch_gpu
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("this torch has no device sleep to keep a stream busy")
    vocab = 4096
    x = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (12,), (2048,), 1.0))
    emb = synthetic.embedding_bits(SEED, vocab=vocab)
    d_x, d_e = dev(torch, x), dev(torch, emb)
    outs = [(empty(torch, vocab, "u16"), empty(torch, 1, "i32")) for _ in range(2)]
    other = torch.cuda.Stream()
    lib = native.lib

    def lm_head(k, s):
        return lib.kudacuda_lm_head_argmax_bf16(native.handle, p(d_x), 0, p(d_e), p(outs[k][0]), p(outs[k][1]), vocab,
                                                 2048, 1.0e-6, s.cuda_stream)

    stream.synchronize()
    with torch.cuda.stream(stream):
        torch.cuda._sleep(1_000_000_000)  # keeps the first stream busy (bounded spin, ~0.4-0.5 s)
    assert lm_head(0, stream) == 0
    assert lm_head(1, other) == 1 and "scratch" in native.error()
    stream.synchronize()
    assert lm_head(1, other) == 0
    other.synchronize()
    assert np.array_equal(host(outs[1][0]), host(outs[0][0]))
    assert int(host(outs[1][1])[0]) == int(host(outs[0][1])[0])
    assert lm_head(0, stream) == 0  # back on the first stream: the second is idle
    stream.synchronize()


def test_handle_graph_replay_takes_part_in_the_scratch_claim(torch_gpu, native, stream):
    """A graph captured through kudacuda_begin_capture that holds a
    scratch-using call is claimed at each kudacuda_replay_graph like an eager
    call: refused while another stream's scratch work is queued, and its own
    replay keeps an eager call on another stream out until it completes."""
    torch = torch_gpu
    if not hasattr(torch.cuda, "_sleep"):
        pytest.skip("this torch has no device sleep to keep a stream busy")
    vocab = 4096
    x = synthetic.f32_to_bf16_bits(synthetic.normal(SEED, (13,), (2048,), 1.0))
    emb = synthetic.embedding_bits(SEED, vocab=vocab)
    d_x, d_e = dev(torch, x), dev(torch, emb)
    outs = [(empty(torch, vocab, "u16"), empty(torch, 1, "i32")) for _ in range(2)]
    other = torch.cuda.Stream()
    lib, h = native.lib, native.handle

    def lm_head(k, s):
        return lib.kudacuda_lm_head_argmax_bf16(h, p(d_x), 0, p(d_e), p(outs[k][0]), p(outs[k][1]), vocab, 2048,
                                                 1.0e-6, s.cuda_stream)

    stream.synchronize()
    assert lib.kudacuda_begin_capture(h, stream.cuda_stream) == 0, native.error()
    assert lm_head(0, stream) == 0, native.error()
    assert lib.kudacuda_end_capture(h, stream.cuda_stream) == 0, native.error()
    try:
        with torch.cuda.stream(other):
            torch.cuda._sleep(1_000_000_000)  # keeps the other stream busy (bounded spin)
        assert lm_head(1, other) == 0, native.error()
        assert lib.kudacuda_replay_graph(h, stream.cuda_stream) == 1 and "scratch" in native.error()
        other.synchronize()
        assert lib.kudacuda_replay_graph(h, stream.cuda_stream) == 0, native.error()
        stream.synchronize()
        assert np.array_equal(host(outs[0][0]), host(outs[1][0]))
        assert int(host(outs[0][1])[0]) == int(host(outs[1][1])[0])
        with torch.cuda.stream(stream):
            torch.cuda._sleep(1_000_000_000)
        assert lib.kudacuda_replay_graph(h, stream.cuda_stream) == 0, native.error()
        assert lm_head(1, other) == 1 and "scratch" in native.error()
        stream.synchronize()
        assert lm_head(1, other) == 0, native.error()
        other.synchronize()
    finally:
        stream.synchronize()
        other.synchronize()
        assert lib.kudacuda_reset_graph(h) == 0, native.error()


def test_vector_add_and_rmsnorm_plumbing(torch_gpu, native, stream):
    torch = torch_gpu
    a = np.arange(1000, dtype=np.float32)
    b = np.full(1000, 0.5, dtype=np.float32)
    d_a, d_b = dev(torch, a), dev(torch, b)
    out = empty(torch, 1000, "f32")
    native.call("kudacuda_vector_add", p(d_a), p(d_b), p(out), 1000, stream.cuda_stream)
    x = np.array([[3.0, 4.0], [0.0, 1.0]], dtype=np.float32)
    w = np.array([1.0, 0.5], dtype=np.float32)
    d_x, d_w = dev(torch, x), dev(torch, w)
    y = empty(torch, 4, "f32")
    native.call("kudacuda_rmsnorm", p(d_x), p(d_w), p(y), 2, 2, 1.0e-5, stream.cuda_stream)
    stream.synchronize()
    assert np.array_equal(host(out), a + b)
    # reference KAT tests/test_contracts.py:732-742
    got = host(y).reshape(2, 2)
    assert abs(got[0, 0] - 0.848528) < 1e-5 and abs(got[0, 1] - 0.565685) < 1e-5 and abs(got[1, 1] - 0.7071) < 1e-4


def test_guards_reject_off_contract_shapes(torch_gpu, native, stream):
    lib = native.lib
    status = lib.kudacuda_qwen2_gqa_decode_bf16(native.handle, 1, 1, 1, 1, 1, 1, 0, 16, 2, 128, 0.1,
                                                stream.cuda_stream)
    assert status == 1 and "kv_len" in native.error()
    status = lib.kudacuda_qwen2_fused_rmsnorm_qkv_nf4_bf16(native.handle, *([1] * 14), 1, 4096, 2048, 256, 64, 1e-6,
                                                           stream.cuda_stream)
    assert status == 1 and "hidden=2048" in native.error()
    status = lib.kudacuda_nf4_gemv_bf16(native.handle, 0, 1, 1, 0, 0, 1, 1, 2048, 2048, 64, stream.cuda_stream)
    assert status == 1 and "non-null" in native.error()
