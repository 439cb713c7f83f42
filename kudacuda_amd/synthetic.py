"""Seeded synthetic inputs for the decode path (no checkpoint, no network).

Shapes follow the Qwen2.5-3B decode configuration named by the benchmark
(hidden 2048, intermediate 11008, 16/2 heads, head_dim 128, RoPE theta 1e6,
QKV bias, tied bf16 embedding / lm_head, vocab 151936).  Every tensor is drawn
from its own numpy PCG64 stream keyed by (seed, layer, tensor id), so any
subset can be regenerated independently and in parallel, identically on any
machine with the same numpy.

Initialisation: linear weights, biases and the embedding ~ N(0, 0.02)
(Transformers' Qwen2 initializer_range); RMSNorm weights 1 + N(0, 0.02) so the
gamma path is exercised.
"""

from __future__ import annotations

import math
from concurrent.futures import ThreadPoolExecutor
from dataclasses import dataclass

import numpy as np

EMBED_ID = 1_000_000
FINAL_ID = 1_000_001
PROMPT_ID = 1_000_002

TENSOR_IDS = {
    "q": 0, "k": 1, "v": 2, "o": 3, "gate": 4, "up": 5, "down": 6,
    "q_bias": 7, "k_bias": 8, "v_bias": 9, "input_norm": 10, "post_norm": 11,
}


@dataclass(frozen=True)
class Qwen2Config:
    hidden: int = 2048
    intermediate: int = 11008
    heads: int = 16
    kv_heads: int = 2
    head_dim: int = 128
    layers: int = 36
    vocab: int = 151936
    rope_theta: float = 1.0e6
    eps: float = 1.0e-6
    std: float = 0.02

    def shapes(self) -> dict[str, tuple[int, ...]]:
        h, i, kv = self.hidden, self.intermediate, self.kv_heads * self.head_dim
        return {
            "q": (h, h), "k": (kv, h), "v": (kv, h), "o": (h, h),
            "gate": (i, h), "up": (i, h), "down": (h, i),
            "q_bias": (h,), "k_bias": (kv,), "v_bias": (kv,),
            "input_norm": (h,), "post_norm": (h,),
        }


QWEN25_3B = Qwen2Config()


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (finite inputs)."""

    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) >> np.uint32(16)).astype(np.uint16)


def bf16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(bits, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


def normal(seed: int, key: tuple[int, ...], shape: tuple[int, ...], std: float) -> np.ndarray:
    rng = np.random.default_rng([int(seed), *[int(k) for k in key]])
    n = int(np.prod(shape))
    return (rng.standard_normal(n, dtype=np.float32) * np.float32(std)).reshape(shape)


def layer_tensor(seed: int, layer: int, name: str, cfg: Qwen2Config = QWEN25_3B) -> np.ndarray:
    """One layer tensor: fp32 weights [out, in]; bf16 bits for biases/norms."""

    shape = cfg.shapes()[name]
    values = normal(seed, (layer, TENSOR_IDS[name]), shape, cfg.std)
    if name.endswith("_norm"):
        return f32_to_bf16_bits(values + np.float32(1.0))
    if name.endswith("_bias"):
        return f32_to_bf16_bits(values)
    return values


def layer_tensors(seed: int, layer: int, cfg: Qwen2Config = QWEN25_3B, threads: int = 8) -> dict[str, np.ndarray]:
    names = list(TENSOR_IDS)
    with ThreadPoolExecutor(max_workers=max(1, threads)) as pool:
        arrays = list(pool.map(lambda n: layer_tensor(seed, layer, n, cfg), names))
    return dict(zip(names, arrays))


def embedding_bits(seed: int, cfg: Qwen2Config = QWEN25_3B, vocab: int | None = None, threads: int = 8) -> np.ndarray:
    """Tied embedding / lm_head table as bf16 bits [vocab, hidden]."""

    vocab = cfg.vocab if vocab is None else int(vocab)
    rows_per_chunk = 8192
    chunks = (vocab + rows_per_chunk - 1) // rows_per_chunk
    out = np.empty((vocab, cfg.hidden), dtype=np.uint16)

    def fill(c: int) -> None:
        r0 = c * rows_per_chunk
        r1 = min(vocab, r0 + rows_per_chunk)
        out[r0:r1] = f32_to_bf16_bits(normal(seed, (EMBED_ID, c), (r1 - r0, cfg.hidden), cfg.std))

    with ThreadPoolExecutor(max_workers=max(1, threads)) as pool:
        list(pool.map(fill, range(chunks)))
    return out


def final_norm_bits(seed: int, cfg: Qwen2Config = QWEN25_3B) -> np.ndarray:
    return f32_to_bf16_bits(normal(seed, (FINAL_ID,), (cfg.hidden,), cfg.std) + np.float32(1.0))


def prompt_ids(seed: int, n: int, vocab: int) -> np.ndarray:
    rng = np.random.default_rng([int(seed), PROMPT_ID])
    return rng.integers(0, vocab, size=n, dtype=np.int64).astype(np.int32)


def rope_tables(capacity: int, head_dim: int = 128, theta: float = 1.0e6) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin [capacity, head_dim/2] in fp32, computed in fp64.

    inv_freq[i] = theta^(-2i/head_dim); angle = position * inv_freq (the
    rotate-half convention of Transformers' Qwen2 rotary embedding, where
    dims d and d + head_dim/2 share a frequency)."""

    half = head_dim // 2
    inv_freq = 1.0 / (theta ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    angles = np.arange(capacity, dtype=np.float64)[:, None] * inv_freq[None, :half]
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


def gemv_inputs(seed: int, out_features: int = 2048, in_features: int = 2048):
    """Config 1: x ~ N(0,1) bf16 [in], W ~ N(0,0.02) fp32 [out, in]."""

    x = f32_to_bf16_bits(normal(seed, (2001,), (in_features,), 1.0))
    w = normal(seed, (2002,), (out_features, in_features), 0.02)
    return x, w


def qkv_inputs(seed: int):
    """Config 2: hidden ~ N(0,1), gamma ~ 1 + N(0,0.1), Wq/Wk/Wv ~ N(0,0.02),
    biases ~ N(0,0.01) (bf16 bits for activations/biases, fp32 weights)."""

    x = f32_to_bf16_bits(normal(seed, (3001,), (2048,), 1.0))
    gamma = f32_to_bf16_bits(normal(seed, (3002,), (2048,), 0.1) + np.float32(1.0))
    w = {n: normal(seed, (3003 + i,), s, 0.02) for i, (n, s) in enumerate((("q", (2048, 2048)), ("k", (256, 2048)), ("v", (256, 2048))))}
    b = {n: f32_to_bf16_bits(normal(seed, (3010 + i,), (s,), 0.01)) for i, (n, s) in enumerate((("q", 2048), ("k", 256), ("v", 256)))}
    return x, gamma, w, b


def mlp_inputs(seed: int):
    """Config 3: x ~ N(0,1) bf16, gate/up [11008, 2048] and down [2048, 11008] ~ N(0,0.02)."""

    x = f32_to_bf16_bits(normal(seed, (4001,), (2048,), 1.0))
    gate = normal(seed, (4002,), (11008, 2048), 0.02)
    up = normal(seed, (4003,), (11008, 2048), 0.02)
    down = normal(seed, (4004,), (2048, 11008), 0.02)
    return x, gate, up, down


def gqa_inputs(seed: int, kv_len: int, capacity: int | None = None):
    """Config 4: q [16,128], K/V [2, capacity, 128] ~ N(0,1) bf16 bits."""

    capacity = kv_len if capacity is None else capacity
    q = f32_to_bf16_bits(normal(seed, (5001,), (16 * 128,), 1.0))
    k = f32_to_bf16_bits(normal(seed, (5002, capacity), (2, capacity, 128), 1.0))
    v = f32_to_bf16_bits(normal(seed, (5003, capacity), (2, capacity, 128), 1.0))
    return q, k, v


def default_scale(head_dim: int = 128) -> float:
    return 1.0 / math.sqrt(head_dim)
