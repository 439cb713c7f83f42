"""Host restatement of the multi-token prefill (test infrastructure).

Same math and rounding points as the GPU prefill: RMSNorm rows rounded to
bf16, NF4 weights dequantised to bf16 (bf16(codebook[code] * absmax)),
products summed in fp64 (the matrix cores' fp32 summation order is not
restated: parity is to a tolerance), bias in fp32 before one rounding,
RoPE in fp32 on the bf16 q/k, causal softmax attention in fp64, residuals
T(res + T(dot)), SwiGLU silu(g)*u in fp32; the last row then goes through
the oracle's own lm_head + argmax (bit-exact restatement of the kernel).
"""

from __future__ import annotations

import numpy as np

from oracle import oracle as O

F = np.float32


def _bf(x: np.ndarray) -> np.ndarray:
    """Round to bf16 and back (fp32 values)."""

    return O.bf16_to_f32(O.f32_to_bf16(np.ascontiguousarray(x, dtype=F)))


def _weight(layer: dict, name: str, rows: int, cols: int) -> np.ndarray:
    w = O.nf4_dequantize(layer[f"{name}_packed"], layer[f"{name}_absmax"], rows * cols)
    return _bf(w).reshape(rows, cols).astype(np.float64)


def _norm(x: np.ndarray, gamma_bits: np.ndarray, eps: float) -> np.ndarray:
    g = O.bf16_to_f32(gamma_bits).astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True) + eps)
    return _bf((x * inv) * g)


def prefill_reference(hm, prompt: np.ndarray) -> dict:
    """Run ``prompt`` (positions 0..P-1) through the host model ``hm``
    (tests/_host_model.HostModel); returns the KV cache rows, the residual
    stream and the last row's logits and greedy token."""

    cfg = hm.cfg
    prompt = np.asarray(prompt, dtype=np.int64)
    P = prompt.size
    eps = cfg.eps
    hidden = O.bf16_to_f32(hm.embed.reshape(-1, 2048)[prompt]).astype(F)
    scale = 1.0 / np.sqrt(128.0)
    kcaches, vcaches = [], []
    for layer in hm.layers:
        xn = _norm(hidden, layer["input_norm"], eps).astype(np.float64)
        q = _bf(xn @ _weight(layer, "q", 2048, 2048).T + O.bf16_to_f32(layer["q_bias"]))
        k = _bf(xn @ _weight(layer, "k", 256, 2048).T + O.bf16_to_f32(layer["k_bias"]))
        v = _bf(xn @ _weight(layer, "v", 256, 2048).T + O.bf16_to_f32(layer["v_bias"]))
        c = hm.rope_cos[:P][:, None, :].astype(F)
        s = hm.rope_sin[:P][:, None, :].astype(F)

        def rope(x: np.ndarray, heads: int) -> np.ndarray:
            x = x.reshape(P, heads, 128)
            lo, hi = x[..., :64], x[..., 64:]
            return _bf(np.concatenate([(lo * c) - (hi * s), (hi * c) + (lo * s)], axis=-1)).reshape(P, heads * 128)

        q = rope(q, 16)
        k = rope(k, 2)
        kc = k.reshape(P, 2, 128).transpose(1, 0, 2)
        vc = v.reshape(P, 2, 128).transpose(1, 0, 2)
        kcaches.append(kc)
        vcaches.append(vc)
        attn = np.zeros((P, 2048), dtype=np.float64)
        qh = q.reshape(P, 16, 128).astype(np.float64)
        for h in range(16):
            g = h // 8
            sc = (qh[:, h, :] @ kc[g].astype(np.float64).T) * scale  # [P, P]
            sc[np.triu_indices(P, 1)] = -np.inf
            sc -= sc.max(axis=1, keepdims=True)
            p = np.exp(sc)
            p /= p.sum(axis=1, keepdims=True)
            attn[:, h * 128:(h + 1) * 128] = p @ vc[g].astype(np.float64)
        attn = _bf(attn).astype(np.float64)
        hidden = _bf(hidden + _bf(attn @ _weight(layer, "o", 2048, 2048).T))
        xn = _norm(hidden, layer["post_norm"], eps).astype(np.float64)
        gate = (xn @ _weight(layer, "gate", 11008, 2048).T).astype(F)
        up = (xn @ _weight(layer, "up", 11008, 2048).T).astype(F)
        h = _bf(O.silu(gate) * up).astype(np.float64)
        hidden = _bf(hidden + _bf(h @ _weight(layer, "down", 2048, 11008).T))
    last = O.f32_to_bf16(hidden[P - 1])
    token, logits = O.lm_head_argmax(last, hm.final_norm, eps, hm.embed.reshape(-1, 2048))
    return {"kcache": kcaches, "vcache": vcaches, "hidden": hidden, "logits": logits, "token": token}
