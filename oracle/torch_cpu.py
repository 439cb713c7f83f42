"""PyTorch-CPU restatement of the decode path: the CPU baseline.

TEST AND MEASUREMENT INFRASTRUCTURE, never the product: only bench.py's
cpu_baseline leg and tests/ use it.  It is the "PyTorch eager" CPU path the
benchmark is measured beside -- the reference's eager control runs the same
model through Transformers with bitsandbytes NF4 linears
(tools/benchmark/benchmark_gemma.py:235-389, python/kudacuda_sidecar.py:
1719-1738: dequantise, then matmul) -- written as plain torch ops on the host
cores: weights dequantised ONCE from the NF4 codes (codebook[code] * absmax,
reference kernels/common/nf4_device.cuh:29-40) into fp32 and excluded from
timing, then fp32 math per token: RMSNorm (harness/reference.py:9-31),
QKV + bias, rotate-half RoPE (theta 1e6), GQA softmax attention in fp32
(tools/correctness/run_qwen2_gqa_check.py:19-28), o_proj + residual, SwiGLU
(kernels/common/nf4_swiglu.cuh:61-63), down + residual, tied lm_head,
greedy argmax.  Activations stay fp32 (no bf16 rounding), so its tokens may
part from the bit-exact oracle's after the first near-tie; it is a timing
baseline, not a parity reference.
"""

from __future__ import annotations

import math
import time
from typing import Any, Callable

import numpy as np
import torch

from .oracle import NF4_CODEBOOK

_CODEBOOK = torch.from_numpy(np.asarray(NF4_CODEBOOK, dtype=np.float32))
# values of both nibbles of every byte: entry e = (codebook[e >> 4], codebook[e & 15])
_PAIRS = torch.stack((_CODEBOOK.repeat_interleave(16), _CODEBOOK.repeat(16)), dim=1)


def dequantize(packed: Any, absmax: Any, rows: int, cols: int) -> torch.Tensor:
    """fp32 [rows, cols] from bitsandbytes NF4 storage (element 2i in the high
    nibble of byte i, one absmax per 64 elements)."""

    codes = torch.as_tensor(packed).reshape(-1).to(torch.int64)
    scale = torch.as_tensor(absmax).reshape(-1, 1).to(torch.float32)
    return (_PAIRS[codes].reshape(-1, 64) * scale).reshape(rows, cols)


def bf16_bits_to_f32(bits: Any) -> torch.Tensor:
    b = torch.as_tensor(np.ascontiguousarray(np.asarray(bits, dtype=np.uint16)).view(np.int16))
    return b.view(torch.bfloat16).to(torch.float32)


def rmsnorm(x: torch.Tensor, gamma: torch.Tensor | None, eps: float) -> torch.Tensor:
    y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return y if gamma is None else y * gamma


def gemv(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    y = torch.mv(w, x)
    return y if bias is None else y + bias


def qkv(x, gamma, eps, wq, bq, wk, bk, wv, bv):
    n = rmsnorm(x, gamma, eps)
    return gemv(n, wq, bq), gemv(n, wk, bk), gemv(n, wv, bv)


def swiglu_mlp(x, gamma, eps, w_gate, w_up, w_down):
    n = rmsnorm(x, gamma, eps)
    return torch.mv(w_down, torch.nn.functional.silu(torch.mv(w_gate, n)) * torch.mv(w_up, n))


def gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float) -> torch.Tensor:
    """q [16, 128], k / v [2, L, 128]: fp32 softmax attention, group 8."""

    qg = q.reshape(2, 8, 128)
    probs = torch.softmax(torch.bmm(qg, k.transpose(1, 2)) * scale, dim=-1)  # [2, 8, L]
    return torch.bmm(probs, v).reshape(16, 128)


def rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of [heads, 128] rows with cos / sin [64] of one position."""

    a, b = x[:, :64], x[:, 64:]
    return torch.cat((a * cos - b * sin, b * cos + a * sin), dim=1)


class TorchCpuDecoder:
    """The batch-1 Qwen2 NF4 decode step in torch CPU fp32 ops.

    ``layers``: per layer the NF4 storage (``{name}_packed`` / ``{name}_absmax``
    for q, k, v, o, gate, up, down) and bf16 bits of the biases and norms;
    ``embed`` / ``final_norm`` bf16 bits.  Weights are dequantised here, once."""

    SHAPES = {"q": (2048, 2048), "k": (256, 2048), "v": (256, 2048), "o": (2048, 2048), "gate": (11008, 2048),
              "up": (11008, 2048), "down": (2048, 11008)}

    def __init__(self, layers: list[dict[str, Any]], embed_bits: Any, final_norm_bits: Any, *, eps: float,
                 capacity: int, theta: float = 1.0e6) -> None:
        self.eps = float(eps)
        self.layers = []
        for src in layers:
            d = {n: dequantize(src[f"{n}_packed"], src[f"{n}_absmax"], *shape) for n, shape in self.SHAPES.items()}
            for n in ("q_bias", "k_bias", "v_bias", "input_norm", "post_norm"):
                d[n] = bf16_bits_to_f32(src[n])
            d["K"] = torch.zeros(2, capacity, 128)
            d["V"] = torch.zeros(2, capacity, 128)
            self.layers.append(d)
        self.embed = bf16_bits_to_f32(embed_bits)
        self.final_norm = bf16_bits_to_f32(final_norm_bits)
        inv_freq = 1.0 / theta ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128.0)
        angles = torch.arange(capacity, dtype=torch.float64)[:, None] * inv_freq[None, :]
        self.cos, self.sin = angles.cos().float(), angles.sin().float()
        self.scale = 1.0 / math.sqrt(128.0)

    @torch.inference_mode()
    def step(self, token: int, pos: int) -> int:
        h = self.embed[int(token)].clone()
        cos, sin = self.cos[pos], self.sin[pos]
        for d in self.layers:
            q, k, v = qkv(h, d["input_norm"], self.eps, d["q"], d["q_bias"], d["k"], d["k_bias"], d["v"], d["v_bias"])
            d["K"][:, pos] = rope(k.reshape(2, 128), cos, sin)
            d["V"][:, pos] = v.reshape(2, 128)
            att = gqa(rope(q.reshape(16, 128), cos, sin), d["K"][:, : pos + 1], d["V"][:, : pos + 1], self.scale)
            h = h + torch.mv(d["o"], att.reshape(-1))
            h = h + swiglu_mlp(h, d["post_norm"], self.eps, d["gate"], d["up"], d["down"])
        logits = torch.mv(self.embed, rmsnorm(h, self.final_norm, self.eps))
        return int(torch.argmax(logits))


def median_us(fn: Callable[[], Any], iters: int = 20, warmup: int = 3) -> float:
    """Median wall time of ``fn`` in microseconds over ``iters`` calls."""

    for _ in range(warmup):
        fn()
    times = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)) * 1e6
