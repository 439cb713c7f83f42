"""GPU: the multi-token prefill path (NF4 GEMM on MFMA).

The GEMM multiplies bf16 activations by NF4 weights dequantised to bf16
(bf16(codebook[code] * absmax), what bitsandbytes feeds its bf16 GEMM,
python/kudacuda_sidecar.py:1719-1738) with fp32 accumulation in the matrix
cores.  The matrix cores' summation order is not restated on the host, so
parity is to a tolerance: the reference sums the same bf16 weights in fp64
and applies the kernel's epilogue in fp32; outputs must agree to one bf16
ulp (|diff| <= 2^-7 |ref| + 2^-16: a different fp32 summation order can move
a value across a bf16 rounding boundary), well inside the north-star bound
(rel 1e-2 / abs 1e-3).
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle import oracle as O
from tests._gpu_util import dev, empty, host, p

pytestmark = pytest.mark.gpu
SEED = 20260824


def _weights(rng, n, k, std=0.02):
    w = (rng.standard_normal((n, k)) * std).astype(np.float32)
    packed, absmax = O.nf4_quantize(w)
    wbf = O.bf16_to_f32(O.f32_to_bf16(O.nf4_dequantize(packed, absmax, n * k))).reshape(n, k)
    return packed, absmax, wbf.astype(np.float64)


def _acts(rng, m, k, std=1.0):
    bits = O.f32_to_bf16((rng.standard_normal((m, k)) * std).astype(np.float32))
    return bits, O.bf16_to_f32(bits).astype(np.float64)


def _close(got_bits, want_f32, inner=None):
    """inner: a value rounded to bf16 inside the epilogue (the residual case),
    whose own one-ulp move carries into the output."""

    got = O.bf16_to_f32(got_bits).astype(np.float64)
    want = O.bf16_to_f32(O.f32_to_bf16(want_f32.astype(np.float32))).astype(np.float64)
    bound = 2.0 ** -7 * (np.abs(want) + (0.0 if inner is None else np.abs(inner))) + 2.0 ** -16
    bad = np.abs(got - want) > bound
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} beyond one bf16 ulp; max {np.abs(got - want).max()}"
    # the summation order moves only a few values across a rounding boundary
    assert np.count_nonzero(got != want) <= max(8, got.size // 100)


@pytest.mark.parametrize("m,n,k", [(1, 64, 128), (7, 2560, 2048), (64, 2048, 2048), (100, 128, 2048),
                                   (33, 2048, 11008)])
@pytest.mark.parametrize("epi", ["plain", "bias", "residual"])
def test_nf4_gemm_matches_fp64(torch_gpu, native, stream, m, n, k, epi):
    torch = torch_gpu
    rng = np.random.default_rng([SEED, m, n, k])
    print(f"nf4_gemm m={m} n={n} k={k} epi={epi}", flush=True)
    packed, absmax, wbf = _weights(rng, n, k)
    xb, x = _acts(rng, m, k)
    acc = (x @ wbf.T).astype(np.float32)
    bias = res = None
    if epi == "bias":
        bias = O.f32_to_bf16((rng.standard_normal(n) * 0.02).astype(np.float32))
        want = acc + O.bf16_to_f32(bias)
    elif epi == "residual":
        res = O.f32_to_bf16(rng.standard_normal((m, n)).astype(np.float32))
        want = O.bf16_to_f32(res) + O.bf16_to_f32(O.f32_to_bf16(acc))
    else:
        want = acc
    d_x, d_w, d_a = dev(torch, xb), dev(torch, packed), dev(torch, absmax)
    d_b = dev(torch, bias) if bias is not None else None
    out = dev(torch, res) if res is not None else empty(torch, m * n, "u16")  # residual in place
    native.call("kudacuda_nf4_gemm_bf16", p(d_x), p(d_w), p(d_a), p(d_b), p(out) if res is not None else 0,
                p(out), m, k, n, 64, stream.cuda_stream)
    stream.synchronize()
    _close(host(out).reshape(m, n), want, inner=acc if epi == "residual" else None)


@pytest.mark.parametrize("m", [1, 13, 64])
def test_nf4_gemm_swiglu_matches_fp64(torch_gpu, native, stream, m):
    torch = torch_gpu
    n, k = 11008, 2048
    rng = np.random.default_rng([SEED, 7, m])
    print(f"nf4_gemm_swiglu m={m}", flush=True)
    gp, ga, gw = _weights(rng, n, k)
    up, ua, uw = _weights(rng, n, k)
    xb, x = _acts(rng, m, k)
    g = (x @ gw.T).astype(np.float32)
    u = (x @ uw.T).astype(np.float32)
    want = O.silu(g) * u
    out = empty(torch, m * n, "u16")
    # keep every upload alive until the launch has run (a temporary's memory
    # could be handed to the next upload)
    bufs = [dev(torch, a) for a in (xb, gp, ga, up, ua)]
    native.call("kudacuda_nf4_gemm_swiglu_bf16", *[p(b) for b in bufs], p(out), m, k, n, 64, stream.cuda_stream)
    stream.synchronize()
    _close(host(out).reshape(m, n), want)


def test_nf4_gemm_guards(torch_gpu, native):
    lib = native.lib
    assert lib.kudacuda_nf4_gemm_bf16(native.handle, 1, 2, 3, 0, 0, 4, 1, 2048, 100, 64, 0) == 1
    assert b"multiple of 64" in lib.kudacuda_last_error(native.handle)
    assert lib.kudacuda_nf4_gemm_bf16(native.handle, 1, 2, 3, 5, 6, 4, 1, 2048, 128, 64, 0) == 1
    assert b"not both" in lib.kudacuda_last_error(native.handle)
    assert lib.kudacuda_nf4_gemm_swiglu_bf16(native.handle, 1, 2, 3, 4, 5, 6, 0, 2048, 128, 64, 0) == 1
