"""Pins of the oracle's full decode step, RoPE/cache write and lm_head argmax."""

from __future__ import annotations

import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest

from kudacuda_amd import synthetic
from oracle import oracle as O
from oracle.reference import nf4_dequant_f64, rmsnorm_f64, rope_f64
from tests._f64_decoder import F64Decoder
from tests._host_model import HostModel

F = np.float32
SEED = 20260824
GOLDEN = Path(__file__).resolve().parent / "golden"


def test_rope_tables_are_the_closed_form():
    cos, sin = synthetic.rope_tables(4096)
    inv = 1.0 / 1.0e6 ** (np.arange(0, 128, 2, dtype=np.float64) / 128.0)
    ang = np.arange(4096, dtype=np.float64)[:, None] * inv[None, :]
    assert cos.tobytes() == np.cos(ang).astype(F).tobytes()
    assert sin.tobytes() == np.sin(ang).astype(F).tobytes()


@pytest.mark.parametrize("pos", [0, 1, 37, 2047])
def test_qkv_rope_cache_against_fp64(pos):
    rng = np.random.default_rng([SEED, pos])
    x = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    gamma = O.f32_to_bf16(F(1) + rng.standard_normal(2048).astype(F) * F(0.02))
    triples = []
    for rows in (2048, 256, 256):
        p, a = O.nf4_quantize(rng.standard_normal(rows * 2048).astype(F) * F(0.02))
        triples.append((p, a, O.f32_to_bf16(rng.standard_normal(rows).astype(F) * F(0.02))))
    cos, sin = synthetic.rope_tables(2048)
    kc = np.full((2, 2048, 128), 0x1234, dtype=np.uint16)
    vc = np.full((2, 2048, 128), 0x1234, dtype=np.uint16)
    q = O.bf16_to_f32(O.qkv_rope_cache(x, gamma, 1e-6, *triples, cos, sin, pos, kc, vc))
    xn = rmsnorm_f64(O.bf16_to_f32(x), O.bf16_to_f32(gamma), 1e-6)
    proj = [nf4_dequant_f64(p, a, r * 2048).reshape(r, 2048) @ xn + O.bf16_to_f32(b)
            for (p, a, b), r in zip(triples, (2048, 256, 256))]
    want_q = rope_f64(proj[0], pos)
    want_k = rope_f64(proj[1], pos)
    tol = lambda w: 1e-2 * np.abs(w) + 1e-3  # noqa: E731
    assert np.all(np.abs(q - want_q) <= tol(want_q))
    assert np.all(np.abs(O.bf16_to_f32(kc[:, pos]).reshape(-1) - want_k) <= tol(want_k))
    assert np.all(np.abs(O.bf16_to_f32(vc[:, pos]).reshape(-1) - proj[2]) <= tol(proj[2]))
    others = np.ones(2048, dtype=bool)
    others[pos] = False
    assert np.all(kc[:, others] == 0x1234) and np.all(vc[:, others] == 0x1234)


def test_planted_rope_sign_error_fails():
    x = np.arange(2048, dtype=np.float64) / 2048.0
    right = rope_f64(x, 5)
    half = x.reshape(-1, 128)
    ang = 5 * (1.0 / 1.0e6 ** (np.arange(0, 128, 2) / 128.0))
    wrong = np.concatenate([half[:, :64] * np.cos(ang) + half[:, 64:] * np.sin(ang),
                            half[:, 64:] * np.cos(ang) - half[:, :64] * np.sin(ang)], axis=1).reshape(-1)
    assert not np.all(np.abs(wrong - right) <= 1e-2 * np.abs(right) + 1e-3)


@pytest.mark.parametrize("with_norm", [False, True])
def test_lm_head_logits_and_first_max_argmax(with_norm):
    rng = np.random.default_rng(3)
    vocab = 5000
    w = O.f32_to_bf16(rng.standard_normal((vocab, 2048)).astype(F) * F(0.02))
    w[4321] = w[77]      # duplicate row: tie, lowest index must win if it is the max
    x = O.f32_to_bf16(rng.standard_normal(2048).astype(F))
    gamma = O.f32_to_bf16(F(1) + rng.standard_normal(2048).astype(F) * F(0.02)) if with_norm else None
    tok, logits = O.lm_head_argmax(x, gamma, 1e-6, w)
    lf = O.bf16_to_f32(logits)
    xn = rmsnorm_f64(O.bf16_to_f32(x), None if gamma is None else O.bf16_to_f32(gamma), 1e-6)
    want = O.bf16_to_f32(w).astype(np.float64) @ xn
    assert np.all(np.abs(lf - want) <= 2.0 ** -8 * np.abs(want) + 1e-3)
    assert tok == int(np.argmax(lf))          # numpy argmax returns the first maximum
    assert logits[4321] == logits[77]
    # force the tie to be the maximum
    w2 = w.copy()
    w2[77] = O.f32_to_bf16(O.bf16_to_f32(x) * F(0.05))
    w2[4321] = w2[77]
    tok2, _ = O.lm_head_argmax(x, gamma, 1e-6, w2)
    assert tok2 == 77


def test_two_layer_decode_against_fp64_restatement():
    hm = HostModel(SEED, num_layers=2, vocab=4096, kv_capacity=64, token_capacity=64)
    ref = F64Decoder(hm)
    prompt = synthetic.prompt_ids(SEED, 6, 4096)
    hm.reset(prompt)
    worst = 0.0
    for step in range(6 + 10 - 1):
        want = ref.step(int(hm.tokens[step]), step)
        hm.step()
        if step + 1 < 6:
            continue
        got = O.bf16_to_f32(hm.logits).astype(np.float64)
        scale = np.abs(want).max()
        err = np.abs(got - want).max() / scale
        worst = max(worst, err)
        assert err <= 2.0 ** -6, (step, err)
        top2 = np.sort(want)[-2:]
        if top2[1] - top2[0] > 2 * 2.0 ** -6 * scale:
            assert int(hm.tokens[step + 1]) == int(np.argmax(want)), step
    assert worst > 0.0  # the two restatements are genuinely different computations


def test_oracle_reproduces_the_small_golden_fixture():
    golden = json.loads((GOLDEN / "decode_small_2l_v4096.json").read_text())
    hm = HostModel(golden["seed"], num_layers=golden["num_layers"], vocab=golden["vocab"],
                   kv_capacity=golden["kv_capacity"], token_capacity=golden["kv_capacity"])
    prompt = np.asarray(golden["prompt"], dtype=np.int32)
    assert prompt.tolist() == synthetic.prompt_ids(golden["seed"], prompt.size, golden["vocab"]).tolist()
    out = hm.generate(prompt, len(golden["tokens"]))
    assert out.tolist() == golden["tokens"]
    for layer, want in zip(hm.layers, golden["prompt_kv_sha256"]):
        for name, key in (("key_cache", "key"), ("value_cache", "value")):
            rows = np.ascontiguousarray(layer[name][:, : prompt.size])
            assert hashlib.sha256(rows.tobytes()).hexdigest() == want[key]


def test_stop_token_ends_the_decode_and_freezes_the_state():
    # the reference stops greedy decoding at EOS, keeping the EOS token
    # (tools/benchmark/benchmark_gemma.py:100-112,147); here the step that
    # emits the stop token sets the done flag, later steps change nothing
    golden = json.loads((GOLDEN / "decode_small_2l_v4096.json").read_text())
    want = golden["tokens"]
    k = next(i for i in range(3, len(want)) if want[i] not in want[:i])  # first token seen for the first time
    hm = HostModel(golden["seed"], num_layers=golden["num_layers"], vocab=golden["vocab"],
                   kv_capacity=golden["kv_capacity"], token_capacity=golden["kv_capacity"])
    prompt = np.asarray(golden["prompt"], dtype=np.int32)
    out = hm.generate(prompt, len(want), stop_token=want[k])
    assert out.tolist() == want[: k + 1]
    stop_pos = prompt.size + k
    assert hm.control[4] == 1 and hm.control[5] == stop_pos and hm.control[0] == stop_pos
    snapshot = (hm.tokens.copy(), hm.control.copy(), hm.layers[1]["key_cache"].copy(), hm.logits.copy())
    for _ in range(3):
        hm.step()
    assert np.array_equal(hm.tokens, snapshot[0]) and np.array_equal(hm.control, snapshot[1])
    assert np.array_equal(hm.layers[1]["key_cache"], snapshot[2]) and np.array_equal(hm.logits, snapshot[3])
    # a stop token that never appears changes nothing
    assert hm.generate(prompt, len(want), stop_token=golden["vocab"] + 5).tolist() == want
