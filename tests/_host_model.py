"""Oracle-side (host) copy of a synthetic Qwen2 NF4 model.

Built from the same seeded fp32 streams as the GPU model, but quantised and
converted by the oracle's own code, and laid out with the same pointer
tables as kudacuda_qwen2_model_create so ``oracle.qwen2_step`` can run it.
"""

from __future__ import annotations

import numpy as np

from kudacuda_amd import synthetic
from kudacuda_amd._native import QWEN2_LAYER_FIELDS, QWEN2_MODEL_FIELDS
from oracle import oracle as O


class HostModel:
    def __init__(self, seed: int, *, num_layers: int, vocab: int, kv_capacity: int, token_capacity: int,
                 cfg: synthetic.Qwen2Config = synthetic.QWEN25_3B, threads: int = 8) -> None:
        self.cfg = cfg
        self.num_layers = num_layers
        self.vocab = vocab
        self.kv_capacity = kv_capacity
        self.token_capacity = token_capacity
        self.layers = []
        for li in range(num_layers):
            arrays = synthetic.layer_tensors(seed, li, cfg, threads=threads)
            layer = {}
            for name in ("q", "k", "v", "o", "gate", "up", "down"):
                # the oracle's own fp32 -> NF4 quantiser (bf16 inputs are not involved)
                layer[f"{name}_packed"], layer[f"{name}_absmax"] = O.nf4_quantize(arrays[name])
            for name in ("q_bias", "k_bias", "v_bias", "input_norm", "post_norm"):
                layer[name] = np.ascontiguousarray(arrays[name])
            layer["key_cache"] = np.zeros((2, kv_capacity, 128), dtype=np.uint16)
            layer["value_cache"] = np.zeros((2, kv_capacity, 128), dtype=np.uint16)
            self.layers.append(layer)
        self.embed = synthetic.embedding_bits(seed, cfg, vocab, threads=threads)
        self.final_norm = synthetic.final_norm_bits(seed, cfg)
        self.rope_cos, self.rope_sin = synthetic.rope_tables(kv_capacity, cfg.head_dim, cfg.rope_theta)
        self.hidden = np.zeros(2048, dtype=np.uint16)
        self.query = np.zeros(2048, dtype=np.uint16)
        self.attn = np.zeros(2048, dtype=np.uint16)
        self.mlp = np.zeros(11008, dtype=np.uint16)
        self.logits = np.zeros(vocab, dtype=np.uint16)
        self.tokens = np.zeros(token_capacity, dtype=np.int32)
        self.control = np.zeros(8, dtype=np.int32)
        self._dummy = np.zeros(16, dtype=np.float32)
        self.layer_table = np.zeros((num_layers, len(QWEN2_LAYER_FIELDS)), dtype=np.uint64)
        for li, layer in enumerate(self.layers):
            for fi, name in enumerate(QWEN2_LAYER_FIELDS):
                self.layer_table[li, fi] = layer[name].ctypes.data
        values = {
            "embed": self.embed, "final_norm": self.final_norm, "rope_cos": self.rope_cos,
            "rope_sin": self.rope_sin, "hidden": self.hidden, "query": self.query, "attn": self.attn,
            "mlp": self.mlp, "logits": self.logits, "tokens": self.tokens, "control": self.control,
            "attn_partials": self._dummy, "attn_counters": self._dummy, "lm_best": self._dummy,
            "lm_counter": self._dummy,
        }
        self.model_table = np.array([values[n].ctypes.data for n in QWEN2_MODEL_FIELDS], dtype=np.uint64)

    def reset(self, prompt: np.ndarray, start_step: int = 0, stop_token: int | None = None) -> None:
        prompt = np.asarray(prompt, dtype=np.int32)
        self.tokens[: prompt.size] = prompt
        self.control[:] = [start_step, prompt.size, self.token_capacity, -1 if stop_token is None else stop_token,
                           0, 0, 0, 0]

    def step(self) -> None:
        O.qwen2_step(self.num_layers, self.vocab, self.kv_capacity, self.cfg.eps, self.layer_table, self.model_table)

    def generate(self, prompt: np.ndarray, new_tokens: int, stop_token: int | None = None) -> np.ndarray:
        prompt = np.asarray(prompt, dtype=np.int32)
        self.reset(prompt, stop_token=stop_token)
        for _ in range(prompt.size + new_tokens - 1):
            self.step()
        end = int(self.control[5]) + 1 if self.control[4] else prompt.size + new_tokens
        return self.tokens[prompt.size: end].copy()
