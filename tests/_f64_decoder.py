"""Independent fp64 restatement of one Qwen2 decode step (test infrastructure).

Written from the model definition (Qwen2: RMSNorm, QKV with bias, rotate-half
RoPE theta 1e6, grouped-query attention 16/2, SwiGLU MLP, tied lm_head), not
from the oracle: every dot product, the norms, the softmax and the rotary
angles are evaluated in fp64.  Activations are rounded to bf16 exactly where
the model stores them in bf16 (projection outputs, attention output, residual
stream, MLP intermediate, logits), so the comparison with the fp32 oracle
measures accumulation-order error only.
"""

from __future__ import annotations

import numpy as np

from oracle.reference import nf4_dequant_f64


def rb(x: np.ndarray) -> np.ndarray:
    """Round fp64 -> fp32 -> bf16 (nearest even) and back to fp64."""

    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32).astype(np.float64)


def bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32).astype(np.float64)


class F64Decoder:
    def __init__(self, host_model, theta: float = 1.0e6) -> None:
        self.m = host_model
        self.layers = []
        for L in host_model.layers:
            d = {}
            for name, rows, cols in (("q", 2048, 2048), ("k", 256, 2048), ("v", 256, 2048), ("o", 2048, 2048),
                                     ("gate", 11008, 2048), ("up", 11008, 2048), ("down", 2048, 11008)):
                d[name] = nf4_dequant_f64(L[f"{name}_packed"], L[f"{name}_absmax"], rows * cols).reshape(rows, cols)
            for name in ("q_bias", "k_bias", "v_bias", "input_norm", "post_norm"):
                d[name] = bits(L[name])
            d["K"] = {}
            d["V"] = {}
            self.layers.append(d)
        self.embed = host_model.embed
        self.final_norm = bits(host_model.final_norm)
        self.inv_freq = 1.0 / theta ** (np.arange(0, 128, 2, dtype=np.float64) / 128.0)
        self.eps = float(host_model.cfg.eps)

    def _norm(self, x, g):
        return x / np.sqrt(np.mean(x * x) + self.eps) * g

    def _rope(self, x, pos):
        ang = pos * self.inv_freq
        c, s = np.cos(ang), np.sin(ang)
        h = x.reshape(-1, 128)
        a, b = h[:, :64], h[:, 64:]
        return np.concatenate([a * c - b * s, b * c + a * s], axis=1).reshape(-1)

    def qkv(self, li: int, hidden: np.ndarray, pos: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """bf16-rounded q (after RoPE), k (after RoPE) and v of layer ``li``."""

        d = self.layers[li]
        xn = self._norm(hidden, d["input_norm"])
        q = rb(self._rope(d["q"] @ xn + d["q_bias"], pos))
        k = rb(self._rope(d["k"] @ xn + d["k_bias"], pos))
        v = rb(d["v"] @ xn + d["v_bias"])
        return q, k, v

    @staticmethod
    def attention(q: np.ndarray, keys: np.ndarray, vals: np.ndarray) -> np.ndarray:
        """bf16-rounded softmax attention of q [2048] over keys/vals [2, L, 128]."""

        att = np.empty((16, 128))
        for h in range(16):
            sc = keys[h // 8] @ q.reshape(16, 128)[h] / np.sqrt(128.0)
            p = np.exp(sc - sc.max())
            att[h] = (p / p.sum()) @ vals[h // 8]
        return rb(att.reshape(-1))

    def swiglu(self, li: int, hidden: np.ndarray) -> np.ndarray:
        d = self.layers[li]
        xn = self._norm(hidden, d["post_norm"])
        g = d["gate"] @ xn
        u = d["up"] @ xn
        return rb(g / (1.0 + np.exp(-g)) * u)

    def o_proj(self, li: int, att: np.ndarray) -> np.ndarray:
        return rb(self.layers[li]["o"] @ att)

    def down(self, li: int, h_mlp: np.ndarray) -> np.ndarray:
        return rb(self.layers[li]["down"] @ h_mlp)

    def layer(self, li: int, hidden: np.ndarray, pos: int, past_keys: np.ndarray | None = None,
              past_values: np.ndarray | None = None) -> dict[str, np.ndarray]:
        """Layer ``li`` at position ``pos`` on the fp64 residual stream
        ``hidden``; returns the bf16-rounded query (after RoPE), attention
        output, MLP intermediate and layer output.  With ``past_keys`` /
        ``past_values`` ([2, pos, 128], e.g. another implementation's cache)
        those rows are attended to instead of this decoder's own history."""

        d = self.layers[li]
        q, k, v = self.qkv(li, hidden, pos)
        d["K"][pos] = k.reshape(2, 128)
        d["V"][pos] = v.reshape(2, 128)
        if past_keys is None:
            keys = np.stack([d["K"][p] for p in range(pos + 1)], axis=1)    # [2, L, 128]
            vals = np.stack([d["V"][p] for p in range(pos + 1)], axis=1)
        else:
            keys = np.concatenate([past_keys, k.reshape(2, 1, 128)], axis=1)
            vals = np.concatenate([past_values, v.reshape(2, 1, 128)], axis=1)
        att = self.attention(q, keys, vals)
        hidden = rb(hidden + self.o_proj(li, att))
        h_mlp = self.swiglu(li, hidden)
        hidden = rb(hidden + self.down(li, h_mlp))
        return {"query": q, "attn": att, "mlp": h_mlp, "hidden": hidden}

    def step(self, token: int, pos: int) -> np.ndarray:
        hidden = bits(self.embed[token])
        for li in range(len(self.layers)):
            hidden = self.layer(li, hidden, pos)["hidden"]
        xn = self._norm(hidden, self.final_norm)
        return rb(bits(self.embed) @ xn)
