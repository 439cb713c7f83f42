"""GPU parity of the reference ABI's plumbing entry points, on the reference's
own C++ smoke fixtures, all called through the C ABI:

* the handle-level graph API (``kudacuda_begin_capture`` / ``end_capture`` /
  ``replay_graph`` / ``reset_graph``) restating tests/cuda_graph_smoke.cu:25-101
  (vector_add then rmsnorm of 513 fp32 values captured on the caller's
  stream, replayed, tolerance 5e-5), extended to several replays with the
  inputs changed in place between them, a reset and a second capture, and
  the refusals of runtime/kudacuda_runtime.cu:1106-1214;
* ``kudacuda_rmsnorm`` on tests/rmsnorm_smoke.cu:27-58 (7 x 513, 5e-5);
* the dense fp16 ``kudacuda_fused_rmsnorm_qkv`` on
  tests/rmsnorm_qkv_smoke.cu:30-125 (2 rows, hidden 16, tolerance 5e-3);
* the fp16 direct GQA entry point at the lengths of
  tools/correctness/run_qwen2_gqa_check.py:41-47 ({1, 7, 128, 512, 585, 1024,
  2048}, seed 20260824, atol = rtol = 3.5e-3 by compare_values,
  :94-99) -- bit-exact to the oracle as well.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from oracle import reference as R
from tests._gpu_util import dev, empty, host, p
from tests._kat import rmsnorm_smoke_case

pytestmark = pytest.mark.gpu

F = np.float32


def _graph_smoke_inputs(variant: int):
    """tests/cuda_graph_smoke.cu:38-42 for variant 0; later variants change
    the values (same sizes) so that a replay which ignored them would fail."""

    i = np.arange(513).astype(F)
    a = np.sin(i * F(0.017)).astype(F)
    b = (np.cos(i * F(0.011)) * F(0.25)).astype(F)
    w = (F(0.75) + (np.arange(513) % 13).astype(F) * F(0.03125)).astype(F)
    if variant:
        a = (a * F(0.5 + 0.25 * variant) + F(0.1 * variant)).astype(F)
        b = (b - F(0.05 * variant)).astype(F)
        w = (w * F(1.0 + 0.1 * variant)).astype(F)
    return a, b, w


def _graph_smoke_expected(a, b, w, eps=1.0e-5):
    """The fixture's own expectation (tests/cuda_graph_smoke.cu:43-51): fp32
    sums, fp64 sum of squares, fp32 inverse RMS."""

    v = (a + b).astype(F)
    ss = float(np.sum(v.astype(np.float64) ** 2))
    inv = F(1.0 / np.sqrt(ss / v.size + eps))
    return (v * inv * w).astype(F), v


def test_graph_abi_capture_replay_reset_recapture(torch_gpu, native, stream):
    torch = torch_gpu
    lib, h, s = native.lib, native.handle, stream.cuda_stream
    a, b, w = _graph_smoke_inputs(0)
    d_a, d_b, d_w = dev(torch, a), dev(torch, b), dev(torch, w)
    mid, out = empty(torch, 513, "f32"), empty(torch, 513, "f32")
    torch.cuda.synchronize()

    # refusals before any graph exists (runtime/kudacuda_runtime.cu:1125-1130, 1166-1172)
    assert lib.kudacuda_replay_graph(h, s) == 1
    assert "before graph instantiation" in native.error()
    assert lib.kudacuda_end_capture(h, s) == 1
    assert "without active capture" in native.error()

    print("graph ABI: capture vector_add + rmsnorm on the caller's stream", flush=True)
    assert lib.kudacuda_begin_capture(h, s) == 0
    # inside the capture: a second begin and a reset are refused, nothing is launched
    assert lib.kudacuda_begin_capture(h, s) == 1 and "already active" in native.error()
    assert lib.kudacuda_reset_graph(h) == 1 and "during active capture" in native.error()
    assert lib.kudacuda_vector_add(h, p(d_a), p(d_b), p(mid), 513, s) == 0
    assert lib.kudacuda_rmsnorm(h, p(mid), p(d_w), p(out), 1, 513, 1.0e-5, s) == 0
    assert lib.kudacuda_end_capture(h, s) == 0, native.error()
    stream.synchronize()
    # capturing records the launches, it does not run them
    assert not host(out).any() and not host(mid).any()

    for variant in range(3):
        if variant:  # new inputs written in place, same pointers, on the graph's stream
            na, nb, nw = _graph_smoke_inputs(variant)
            with torch.cuda.stream(stream):
                d_a.copy_(torch.from_numpy(na).to("cuda:0", non_blocking=False))
                d_b.copy_(torch.from_numpy(nb).to("cuda:0", non_blocking=False))
                d_w.copy_(torch.from_numpy(nw).to("cuda:0", non_blocking=False))
            a, b, w = na, nb, nw
        stream.synchronize()
        assert lib.kudacuda_replay_graph(h, s) == 0, native.error()
        stream.synchronize()
        want, v = _graph_smoke_expected(a, b, w)
        assert np.array_equal(host(mid), v)  # fp32 add is exact to the host's
        err = np.abs(host(out) - want).max()
        print(f"graph replay {variant}: max |out - fixture| {err:.3g}", flush=True)
        assert err <= 5.0e-5  # tests/cuda_graph_smoke.cu:28

    assert lib.kudacuda_reset_graph(h) == 0
    assert lib.kudacuda_replay_graph(h, s) == 1 and "before graph instantiation" in native.error()
    assert lib.kudacuda_reset_graph(h) == 0  # resetting nothing is not an error

    # a second capture on the same handle: rmsnorm only, of the add's output
    out2 = empty(torch, 513, "f32")
    torch.cuda.synchronize()
    assert lib.kudacuda_begin_capture(h, s) == 0
    assert lib.kudacuda_rmsnorm(h, p(mid), p(d_w), p(out2), 1, 513, 1.0e-5, s) == 0
    assert lib.kudacuda_end_capture(h, s) == 0, native.error()
    for _ in range(2):
        assert lib.kudacuda_replay_graph(h, s) == 0, native.error()
    stream.synchronize()
    want, _ = _graph_smoke_expected(a, b, w)
    assert np.abs(host(out2) - want).max() <= 5.0e-5
    assert lib.kudacuda_reset_graph(h) == 0


def test_rmsnorm_reference_fixture_7x513(torch_gpu, native, stream):
    torch = torch_gpu
    x, w, eps, tol = rmsnorm_smoke_case()
    d_x, d_w = dev(torch, x), dev(torch, w)
    y = empty(torch, x.size, "f32")
    native.call("kudacuda_rmsnorm", p(d_x), p(d_w), p(y), 7, 513, eps, stream.cuda_stream)
    stream.synchronize()
    got = host(y).reshape(7, 513)
    # the fixture's expectation (tests/rmsnorm_smoke.cu:45-58): fp64 sum of
    # squares, fp32 inverse RMS, fp32 products
    ss = np.sum(x.astype(np.float64) ** 2, axis=1, keepdims=True)
    inv = (1.0 / np.sqrt(ss / 513 + eps)).astype(F)
    want = (x * inv * w).astype(F)
    assert np.abs(got - want).max() <= tol
    assert np.abs(got - R.rmsnorm_f64(x.astype(np.float64), w.astype(np.float64), eps)).max() <= tol


def _dense_qkv_fixture():
    """tests/rmsnorm_qkv_smoke.cu:39-70: fp16 input sin(i*0.13), gamma
    0.75 + i*0.01, weight [48, 16] cos(i*0.017)*0.2, bias sin(i*0.07)*0.05."""

    rows, hidden = 2, 16
    x = O.f32_to_f16(np.sin(np.arange(rows * hidden).astype(F) * F(0.13)))
    gamma = O.f32_to_f16(F(0.75) + np.arange(hidden).astype(F) * F(0.01))
    weight = O.f32_to_f16(np.cos(np.arange(3 * hidden * hidden).astype(F) * F(0.017)) * F(0.2))
    bias = O.f32_to_f16(np.sin(np.arange(3 * hidden).astype(F) * F(0.07)) * F(0.05))
    return rows, hidden, x, gamma, weight, bias


def _dense_qkv_fixture_expected(rows, hidden, x, gamma, weight, bias, eps):
    """The fixture's own CPU loop (tests/rmsnorm_qkv_smoke.cu:72-91): fp32
    sequential sums, output rounded to fp16."""

    xf, gf = O.f16_to_f32(x).reshape(rows, hidden), O.f16_to_f32(gamma)
    wf, bf = O.f16_to_f32(weight).reshape(3 * hidden, hidden), O.f16_to_f32(bias)
    out = np.zeros((rows, 3 * hidden), dtype=np.uint16)
    for r in range(rows):
        ss = F(0.0)
        for d in range(hidden):
            ss = F(ss + xf[r, d] * xf[r, d])
        inv = F(F(1.0) / np.sqrt(F(ss / F(hidden) + F(eps))))
        norm = (xf[r] * inv * gf).astype(F)
        for o in range(3 * hidden):
            acc = bf[o]
            for d in range(hidden):
                acc = F(acc + norm[d] * wf[o, d])
            out[r, o] = O.f32_to_f16(np.array([acc], dtype=F))[0]
    return out


def _dense_qkv_f64(rows, hidden, x, gamma, weight, bias, eps):
    xf = O.f16_to_f32(x).reshape(rows, hidden).astype(np.float64)
    n = R.rmsnorm_f64(xf, O.f16_to_f32(gamma).astype(np.float64), eps)
    wf = O.f16_to_f32(weight).reshape(3 * hidden, hidden).astype(np.float64)
    return n @ wf.T + O.f16_to_f32(bias).astype(np.float64)


def test_dense_fused_rmsnorm_qkv_reference_fixture(torch_gpu, native, stream):
    torch = torch_gpu
    eps = 1.0e-5
    rows, hidden, x, gamma, weight, bias = _dense_qkv_fixture()
    d = [dev(torch, t) for t in (x, gamma, weight, bias)]
    out = empty(torch, rows * 3 * hidden, "u16")
    native.call("kudacuda_fused_rmsnorm_qkv", *map(p, d), p(out), rows, hidden, eps, stream.cuda_stream)
    stream.synchronize()
    got = O.f16_to_f32(host(out)).reshape(rows, 3 * hidden)
    want = O.f16_to_f32(_dense_qkv_fixture_expected(rows, hidden, x, gamma, weight, bias, eps).reshape(-1))
    assert np.abs(got - want.reshape(rows, 3 * hidden)).max() <= 5.0e-3  # tests/rmsnorm_qkv_smoke.cu:35
    ref = _dense_qkv_f64(rows, hidden, x, gamma, weight, bias, eps)
    # one fp16 rounding step of the output plus the fp32 sums' error
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 1.0e-4)


def test_dense_fused_rmsnorm_qkv_model_width(torch_gpu, native, stream):
    """Same op at the Qwen2.5-3B width (3 rows of 2048, weight [6144, 2048]):
    every output within one fp16 step of the fp64 result."""

    torch = torch_gpu
    rng = np.random.default_rng(20260824)
    rows, hidden, eps = 3, 2048, 1.0e-6
    x = O.f32_to_f16(rng.standard_normal(rows * hidden, dtype=F))
    gamma = O.f32_to_f16(F(1.0) + rng.standard_normal(hidden, dtype=F) * F(0.1))
    weight = O.f32_to_f16(rng.standard_normal(3 * hidden * hidden, dtype=F) * F(0.02))
    bias = O.f32_to_f16(rng.standard_normal(3 * hidden, dtype=F) * F(0.01))
    d = [dev(torch, t) for t in (x, gamma, weight, bias)]
    out = empty(torch, rows * 3 * hidden, "u16")
    native.call("kudacuda_fused_rmsnorm_qkv", *map(p, d), p(out), rows, hidden, eps, stream.cuda_stream)
    stream.synchronize()
    got = O.f16_to_f32(host(out)).reshape(rows, 3 * hidden).astype(np.float64)
    ref = _dense_qkv_f64(rows, hidden, x, gamma, weight, bias, eps)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2.0 ** -10 + 2.0e-4)
    assert R.compare_values(got.reshape(-1).tolist(), ref.reshape(-1).tolist(), atol=1.0e-3, rtol=1.0e-2)["passed"]


@pytest.mark.parametrize("kv_len", [1, 7, 128, 512, 585, 1024, 2048])
def test_gqa_fp16_direct_reference_check_lengths(torch_gpu, native, stream, kv_len):
    """tools/correctness/run_qwen2_gqa_check.py: fp16 q [1,16,1,128], K/V
    [1,2,L,128] standard normal, seed 20260824, scale 1/sqrt(128), checked by
    compare_values at atol = rtol = 3.5e-3 against fp32-or-better attention."""

    torch = torch_gpu
    print(f"gqa fp16 direct, kv_len {kv_len}", flush=True)
    rng = np.random.default_rng([20260824, kv_len])
    q = O.f32_to_f16(rng.standard_normal(16 * 128, dtype=F))
    k = O.f32_to_f16(rng.standard_normal(2 * kv_len * 128, dtype=F)).reshape(2, kv_len, 128)
    v = O.f32_to_f16(rng.standard_normal(2 * kv_len * 128, dtype=F)).reshape(2, kv_len, 128)
    d_q, d_k, d_v = dev(torch, q), dev(torch, k), dev(torch, v)
    out = empty(torch, 2048, "u16")
    scale = 1.0 / np.sqrt(128.0)
    native.call("kudacuda_qwen2_gqa_decode", p(d_q), p(d_k), p(d_v), p(out), 1, 1, kv_len, 16, 2, 128, scale,
                stream.cuda_stream)
    stream.synchronize()
    got = host(out)
    assert np.array_equal(got, O.gqa(q, k, v, kv_len, scale=scale, dtype="f16"))
    ref = R.gqa_f64(O.f16_to_f32(q), O.f16_to_f32(k), O.f16_to_f32(v), kv_len, scale)
    metrics = R.compare_values(O.f16_to_f32(got).tolist(), ref.reshape(-1).tolist(), atol=3.5e-3, rtol=3.5e-3)
    assert metrics["passed"], metrics
