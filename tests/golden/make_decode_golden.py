"""Write the greedy-decode golden fixtures from the CPU oracle.

Fixture = the seeded synthetic Qwen2.5-3B-shaped NF4 model (
36 layers, vocab 151936, 64 random prompt ids, 128 greedy tokens, KV bucket
2048) decoded by the oracle (oracle/kc_oracle.c), plus a 2-layer / 4096-vocab
variant small enough for the CPU test suite.  Stored: prompt, generated ids,
the bf16 top-1 minus top-2 logit margin at each generated token, SHA-256
digests of the bf16 logits and of the final hidden state (the residual stream
after the last layer) after every step that emits a token, SHA-256 digests
of every layer's key and value cache rows of the prompt tokens (rows
0..prompt_len-1 of [2, capacity, 128] bf16, written by the prompt steps and
never changed after), and SHA-256 digests of the oracle-quantised layer-0
weights.

Usage: python tests/golden/make_decode_golden.py [--small-only]
"""

from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from kudacuda_amd import synthetic  # noqa: E402
from oracle import oracle as O  # noqa: E402
from tests._host_model import HostModel  # noqa: E402

SEED = 20260824
OUT = Path(__file__).resolve().parent


def run(name: str, *, num_layers: int, vocab: int, kv_capacity: int, prompt_len: int, new_tokens: int) -> None:
    t0 = time.time()
    model = HostModel(SEED, num_layers=num_layers, vocab=vocab, kv_capacity=kv_capacity, token_capacity=kv_capacity)
    t1 = time.time()
    prompt = synthetic.prompt_ids(SEED, prompt_len, vocab)
    model.reset(prompt)
    margins, logit_digests, hidden_digests = [], [], []
    for _ in range(prompt_len + new_tokens - 1):
        step = int(model.control[0])
        model.step()
        if step + 1 >= prompt_len:
            logits = O.bf16_to_f32(model.logits)
            top2 = np.sort(logits)[-2:]
            margins.append(float(top2[1] - top2[0]))
            logit_digests.append(hashlib.sha256(model.logits.tobytes()).hexdigest())
            hidden_digests.append(hashlib.sha256(model.hidden.tobytes()).hexdigest())
    tokens = model.tokens[prompt_len: prompt_len + new_tokens].astype(int).tolist()
    digests = {
        f"layer0_{n}": hashlib.sha256(model.layers[0][n].tobytes()).hexdigest()
        for n in ("q_packed", "q_absmax", "down_packed", "down_absmax")
    }
    prompt_kv = [
        {"key": hashlib.sha256(np.ascontiguousarray(layer["key_cache"][:, :prompt_len]).tobytes()).hexdigest(),
         "value": hashlib.sha256(np.ascontiguousarray(layer["value_cache"][:, :prompt_len]).tobytes()).hexdigest()}
        for layer in model.layers
    ]
    payload = {
        "seed": SEED, "num_layers": num_layers, "vocab": vocab, "kv_capacity": kv_capacity,
        "prompt": prompt.astype(int).tolist(), "tokens": tokens, "logit_margins": margins,
        "logits_sha256": logit_digests, "hidden_sha256": hidden_digests, "weight_digests": digests,
        "prompt_kv_sha256": prompt_kv, "generator": "tests/golden/make_decode_golden.py (oracle/kc_oracle.c)",
    }
    (OUT / f"{name}.json").write_text(json.dumps(payload, indent=1) + "\n", encoding="utf-8")
    print(f"{name}: build {t1 - t0:.1f}s decode {time.time() - t1:.1f}s tokens {tokens[:16]}... "
          f"min margin {min(margins):.4g}")


if __name__ == "__main__":
    run("decode_small_2l_v4096", num_layers=2, vocab=4096, kv_capacity=256, prompt_len=16, new_tokens=32)
    if "--small-only" not in sys.argv:
        run("decode_qwen25_3b_nf4", num_layers=36, vocab=151936, kv_capacity=2048, prompt_len=64, new_tokens=128)
