"""Native batch-1 Qwen2 NF4 decoder on one MI355X (gfx950).

PyTorch-ROCm provides device memory and the HIP stream; every step of the
decode runs in libkudacuda's kernels (``kudacuda_qwen2_model_*``):

    per layer: RMSNorm+QKV+bias+RoPE+KV write | split-KV GQA | O GEMV+res |
               RMSNorm+gate/up+SiLU*up | down GEMV+res
    then:      final RMSNorm + tied bf16 lm_head + argmax + token bookkeeping

One step is captured once into a hipGraph and replayed per token.  The prompt
is consumed by the same step (one token per replay; the lm_head is skipped
until the last prompt token), and the greedy tokens are written to a device
array, so a whole generation needs no host synchronisation.

Reference behaviour replaced: ``StaticDecodeGraphRunner`` + Transformers
forward + host ``torch.argmax`` per token
(python/kudacuda_static_decode.py:271-437,
tools/benchmark/benchmark_gemma.py:235-389).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any

import numpy as np

from . import synthetic
from ._native import QWEN2_LAYER_FIELDS, QWEN2_MODEL_FIELDS, Native, NativeError
from .synthetic import Qwen2Config

OPS = {"qkv_rope": 0, "attention": 1, "o_proj": 2, "gate_up": 3, "down": 4, "lm_head": 5}


def _bits_to_bf16(torch: Any, bits: np.ndarray, device: Any) -> Any:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).view(torch.bfloat16).to(device)


@dataclass
class Nf4Tensor:
    packed: Any  # uint8 [out * in / 2]
    absmax: Any  # fp32 [out * in / 64]
    shape: tuple[int, int]


def quantize_nf4(native: Native, torch: Any, weight_f32: np.ndarray | Any, device: Any, stream: Any) -> Nf4Tensor:
    """Upload an fp32 [out, in] weight and NF4-quantise it on the GPU."""

    src = weight_f32 if hasattr(weight_f32, "data_ptr") else torch.from_numpy(np.ascontiguousarray(weight_f32))
    shape = tuple(int(s) for s in src.shape)
    n = int(src.numel())
    with torch.cuda.stream(stream):
        dev = src.to(device=device, dtype=torch.float32, non_blocking=False).contiguous()
        packed = torch.empty(n // 2, dtype=torch.uint8, device=device)
        absmax = torch.empty(n // 64, dtype=torch.float32, device=device)
        native.call("kudacuda_nf4_quantize", dev.data_ptr(), 0, n, 64, packed.data_ptr(), absmax.data_ptr(),
                    stream.cuda_stream)
        stream.synchronize()
        del dev
    return Nf4Tensor(packed, absmax, (shape[0], shape[1]))


class Qwen2Nf4Decoder:
    """Device-resident NF4 Qwen2 decoder driven through the C ABI."""

    def __init__(self, native: Native, torch: Any, cfg: Qwen2Config, layers: list[dict[str, Any]], embed: Any,
                 final_norm: Any, *, kv_capacity: int, token_capacity: int, device: Any, stream: Any) -> None:
        self.native = native
        self.torch = torch
        self.cfg = cfg
        self.device = device
        self.stream = stream
        self.kv_capacity = int(kv_capacity)
        self.token_capacity = int(token_capacity)
        self.layers = layers
        self.embed = embed
        self.final_norm = final_norm
        self.num_layers = len(layers)
        self.vocab = int(embed.shape[0])
        lib = native.lib
        t = torch
        cos, sin = synthetic.rope_tables(self.kv_capacity, cfg.head_dim, cfg.rope_theta)
        with t.cuda.stream(stream):
            self.rope_cos = t.from_numpy(cos).to(device)
            self.rope_sin = t.from_numpy(sin).to(device)
            self.hidden = t.zeros(cfg.hidden, dtype=t.bfloat16, device=device)
            self.query = t.zeros(cfg.heads * cfg.head_dim, dtype=t.bfloat16, device=device)
            self.attn = t.zeros(cfg.heads * cfg.head_dim, dtype=t.bfloat16, device=device)
            self.mlp = t.zeros(cfg.intermediate, dtype=t.bfloat16, device=device)
            self.logits = t.zeros(self.vocab, dtype=t.bfloat16, device=device)
            self.tokens = t.zeros(self.token_capacity, dtype=t.int32, device=device)
            self.control = t.zeros(8, dtype=t.int32, device=device)
            self.attn_partials = t.zeros(int(lib.kudacuda_gqa_workspace_floats(self.kv_capacity)), dtype=t.float32,
                                         device=device)
            self.attn_counters = t.zeros(2, dtype=t.int32, device=device)
            self.lm_best = t.zeros(int(lib.kudacuda_lm_head_workspace_floats()), dtype=t.float32, device=device)
            for layer in self.layers:
                layer["key_cache"] = t.zeros((cfg.kv_heads, self.kv_capacity, cfg.head_dim), dtype=t.bfloat16,
                                             device=device)
                layer["value_cache"] = t.zeros_like(layer["key_cache"])
        stream.synchronize()
        self.layer_table = np.zeros((self.num_layers, len(QWEN2_LAYER_FIELDS)), dtype=np.uint64)
        for li, layer in enumerate(self.layers):
            for fi, name in enumerate(QWEN2_LAYER_FIELDS):
                self.layer_table[li, fi] = layer[name].data_ptr()
        model_values = {
            "embed": self.embed, "final_norm": self.final_norm, "rope_cos": self.rope_cos,
            "rope_sin": self.rope_sin, "hidden": self.hidden, "query": self.query, "attn": self.attn,
            "mlp": self.mlp, "logits": self.logits, "tokens": self.tokens, "control": self.control,
            "attn_partials": self.attn_partials, "attn_counters": self.attn_counters, "lm_best": self.lm_best,
            "lm_counter": None,  # reserved field, unused by the library
        }
        self.model_table = np.array([0 if model_values[n] is None else model_values[n].data_ptr()
                                     for n in QWEN2_MODEL_FIELDS], dtype=np.uint64)
        self.model = lib.kudacuda_qwen2_model_create(
            native.handle, self.num_layers, self.vocab, self.kv_capacity, float(cfg.eps),
            self.layer_table.ctypes.data, self.model_table.ctypes.data,
        )
        if not self.model:
            raise NativeError(f"kudacuda_qwen2_model_create failed: {native.error()}")
        self.captured = False
        self._prefill_ws: Any = None

    # ------------------------------------------------------------ building
    @classmethod
    def synthetic(cls, native: Native, torch: Any, *, seed: int, cfg: Qwen2Config = synthetic.QWEN25_3B,
                  num_layers: int | None = None, vocab: int | None = None, kv_capacity: int = 2048,
                  token_capacity: int | None = None, device: Any = "cuda:0", threads: int = 8,
                  stream: Any = None) -> "Qwen2Nf4Decoder":
        """Random-init model from ``synthetic`` streams, NF4-quantised on the GPU."""

        num_layers = cfg.layers if num_layers is None else int(num_layers)
        vocab = cfg.vocab if vocab is None else int(vocab)
        token_capacity = kv_capacity if token_capacity is None else int(token_capacity)
        stream = stream or torch.cuda.Stream(device=device)
        layers: list[dict[str, Any]] = []
        for li in range(num_layers):
            arrays = synthetic.layer_tensors(seed, li, cfg, threads=threads)
            layer: dict[str, Any] = {}
            for name in ("q", "k", "v", "o", "gate", "up", "down"):
                q = quantize_nf4(native, torch, arrays[name], device, stream)
                layer[f"{name}_packed"] = q.packed
                layer[f"{name}_absmax"] = q.absmax
            for name in ("q_bias", "k_bias", "v_bias", "input_norm", "post_norm"):
                layer[name] = _bits_to_bf16(torch, arrays[name], device)
            layers.append(layer)
            del arrays
        embed = _bits_to_bf16(torch, synthetic.embedding_bits(seed, cfg, vocab, threads=threads), device)
        final_norm = _bits_to_bf16(torch, synthetic.final_norm_bits(seed, cfg), device)
        return cls(native, torch, cfg, layers, embed, final_norm, kv_capacity=kv_capacity,
                   token_capacity=token_capacity, device=device, stream=stream)

    # ------------------------------------------------------------ running
    def reset(self, prompt: np.ndarray, *, start_step: int = 0, stop_token: int | None = None) -> None:
        """Load prompt ids into the token array and set step/prompt/capacity.

        With ``stop_token`` the device stops the decode at the step that emits
        it (kept in the token array); later steps change nothing."""

        prompt = np.asarray(prompt, dtype=np.int32)
        if prompt.size < 1 or prompt.size > self.token_capacity:
            raise ValueError("prompt must have 1..token_capacity ids")
        stop = -1 if stop_token is None else int(stop_token)
        t = self.torch
        with t.cuda.stream(self.stream):
            self.tokens[: prompt.size].copy_(t.from_numpy(prompt))
            self.control.copy_(t.tensor([start_step, prompt.size, self.token_capacity, stop, 0, 0, 0, 0],
                                        dtype=t.int32))
        self.stream.synchronize()
        self._set_position(start_step)

    def stopped_at(self) -> int | None:
        """Position of the stop token in the token array, or None while running."""

        control = self.control.cpu().numpy()
        return int(control[5]) if int(control[4]) != 0 else None

    def set_step(self, step: int) -> None:
        t = self.torch
        with t.cuda.stream(self.stream):
            self.control[0:1].copy_(t.tensor([int(step)], dtype=t.int32))
        self.stream.synchronize()
        self._set_position(step)

    def _set_position(self, step: int) -> None:
        # tells the library which step runs next, so that replays pick the
        # faster form of the step for the cache length (results do not depend on it)
        self.native.check(self.native.lib.kudacuda_qwen2_model_set_position(self.model, int(step)),
                          "kudacuda_qwen2_model_set_position")

    def step(self) -> None:
        self.native.check(self.native.lib.kudacuda_qwen2_model_step(self.model, self.stream.cuda_stream),
                          "kudacuda_qwen2_model_step")

    def capture(self) -> None:
        self.native.check(self.native.lib.kudacuda_qwen2_model_capture(self.model, self.stream.cuda_stream),
                          "kudacuda_qwen2_model_capture")
        self.captured = True

    def replay(self, steps: int = 1) -> None:
        if not self.captured:
            self.capture()
        self.native.check(self.native.lib.kudacuda_qwen2_model_replay(self.model, int(steps), self.stream.cuda_stream),
                          "kudacuda_qwen2_model_replay")

    def run_steps(self, steps: int, *, graph: bool = True) -> None:
        if steps <= 0:
            return
        if graph:
            self.replay(steps)
        else:
            for _ in range(steps):
                self.step()

    def generate(self, prompt: np.ndarray, new_tokens: int, *, graph: bool = True,
                 stop_token: int | None = None) -> np.ndarray:
        """Greedy-decode up to ``new_tokens`` ids after ``prompt``; returns
        them, ending with ``stop_token`` if the decode emitted it.  The stop is
        decided on the device: all steps are launched without a host sync."""

        prompt = np.asarray(prompt, dtype=np.int32)
        total = prompt.size + int(new_tokens)
        if total > min(self.token_capacity, self.kv_capacity + 1):
            raise ValueError("prompt + new tokens exceed the token/KV capacity")
        self.reset(prompt, stop_token=stop_token)
        self.run_steps(total - 1, graph=graph)
        self.stream.synchronize()
        stop = self.stopped_at()
        end = total if stop is None else stop + 1
        return self.tokens[prompt.size:end].cpu().numpy().copy()

    def prefill(self, prompt: np.ndarray) -> None:
        """Load ``prompt`` and run it through the model in one multi-token pass
        (``kudacuda_qwen2_model_prefill``): KV cache rows 0..P-1 are written,
        tokens[P] receives the greedy token and the step moves to P, so
        ``replay``/``step`` continue the decode from there."""

        prompt = np.asarray(prompt, dtype=np.int32)
        if prompt.size > min(self.token_capacity - 1, self.kv_capacity):
            raise ValueError("prompt exceeds the token/KV capacity")
        self.reset(prompt)
        lib = self.native.lib
        nbytes = int(lib.kudacuda_qwen2_prefill_workspace_bytes(prompt.size))
        if self._prefill_ws is None or self._prefill_ws.numel() < nbytes:
            self._prefill_ws = self.torch.empty(nbytes, dtype=self.torch.uint8, device=self.tokens.device)
        self.native.check(lib.kudacuda_qwen2_model_prefill(self.model, self._prefill_ws.data_ptr(), nbytes, 0,
                                                           prompt.size, self.stream.cuda_stream),
                          "kudacuda_qwen2_model_prefill")

    def generate_prefilled(self, prompt: np.ndarray, new_tokens: int) -> np.ndarray:
        """``generate`` with a multi-token prefill instead of one decode step
        per prompt token."""

        prompt = np.asarray(prompt, dtype=np.int32)
        total = prompt.size + int(new_tokens)
        if total > min(self.token_capacity, self.kv_capacity + 1):
            raise ValueError("prompt + new tokens exceed the token/KV capacity")
        self.prefill(prompt)
        self.run_steps(total - prompt.size - 1, graph=True)
        self.stream.synchronize()
        return self.tokens[prompt.size:total].cpu().numpy().copy()

    def time_op(self, op: str | int, iters: int) -> float:
        """Mean duration (ms) of one kernel of the step, HIP events on the step stream."""

        avg = ctypes.c_float(0.0)
        code = OPS[op] if isinstance(op, str) else int(op)
        self.native.check(
            self.native.lib.kudacuda_qwen2_model_time_op(self.model, code, int(iters), self.stream.cuda_stream,
                                                         ctypes.byref(avg)),
            "kudacuda_qwen2_model_time_op",
        )
        return float(avg.value)

    def close(self) -> None:
        if getattr(self, "model", None):
            self.native.lib.kudacuda_qwen2_model_destroy(self.model)
            self.model = None

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass
