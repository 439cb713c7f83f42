"""GPU: BASELINE config 5 at full size against the oracle's golden decode.

The 36-layer Qwen2.5-3B-shaped NF4 model (vocab 151,936, tied bf16
lm_head, KV bucket 2048) is built by the product path from the seeded
streams, the 64-token prompt runs through the captured decode step and 128
greedy tokens follow, one hipGraph replay per token.  After every step that
emits a token, the SHA-256 of the bf16 logits and of the final hidden state
must equal the oracle's (tests/golden/decode_qwen25_3b_nf4.json, written by
tests/golden/make_decode_golden.py from oracle/kc_oracle.c), and so must the
128 token ids: the reference's headline parity claim, exact greedy tokens
over a 128-token decode (README.md:36-39).  Three of the 128 steps have an exact
bf16 tie between the top two logits; there the token is fixed by the
lowest-index rule and the bit-identical logits, which only a bit-exact
oracle can pin.
"""

from __future__ import annotations

import hashlib
import json
from pathlib import Path

import numpy as np
import pytest

from kudacuda_amd.qwen2_decoder import Qwen2Nf4Decoder
from tests._gpu_util import host

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "decode_qwen25_3b_nf4.json"
# Measured on MI355X: the prefill's relative L2 divergence is 0.67-1.00 times
# that of the one-ulp perturbed decode at every layer (relL2 0.0036 at layer 0
# to 0.049 at layer 35, against 0.0046 to 0.049).
PREFILL_VS_PERTURBED = 1.25


def _sha(tensor) -> str:
    return hashlib.sha256(host(tensor).tobytes()).hexdigest()


def test_config5_full_model_matches_golden_for_128_greedy_tokens(torch_gpu, native):
    torch = torch_gpu
    golden = json.loads(GOLDEN.read_text())
    assert golden["num_layers"] == 36 and golden["vocab"] == 151936 and golden["kv_capacity"] == 2048
    prompt = np.asarray(golden["prompt"], dtype=np.int32)
    new = len(golden["tokens"])
    assert prompt.size == 64 and new == 128
    print("[full_model] building the 36-layer model", flush=True)
    model = Qwen2Nf4Decoder.synthetic(native, torch, seed=golden["seed"], kv_capacity=golden["kv_capacity"],
                                      token_capacity=golden["kv_capacity"], threads=16)
    try:
        layer0 = model.layers[0]
        for name, digest in golden["weight_digests"].items():
            assert _sha(layer0[name.removeprefix("layer0_")]) == digest, name
        print("[full_model] decoding 64 + 128 tokens", flush=True)
        model.reset(prompt)
        model.capture()
        model.replay(prompt.size - 1)  # the prompt's own steps: lm_head skipped on device
        for i in range(new):
            if i == 1:  # the prompt's K/V rows are complete (row 63 came with the first emitting step)
                for li, (layer, want) in enumerate(zip(model.layers, golden["prompt_kv_sha256"])):
                    for name, key in (("key_cache", "key"), ("value_cache", "value")):
                        rows = layer[name][:, : prompt.size].contiguous()
                        assert _sha(rows) == want[key], f"layer {li} {name} rows of the prompt"
            model.replay(1)  # emits tokens[64 + i]
            model.stream.synchronize()
            assert _sha(model.logits) == golden["logits_sha256"][i], f"logits of generated token {i}"
            assert _sha(model.hidden) == golden["hidden_sha256"][i], f"final hidden state at generated token {i}"
        tokens = host(model.tokens)[prompt.size: prompt.size + new]
        assert tokens.tolist() == golden["tokens"]
        assert int(host(model.control)[0]) == prompt.size + new - 1
    finally:
        model.close()


def _bf16_f32(t):
    import torch

    return t.contiguous().view(torch.int16).to(torch.int32).bitwise_left_shift(16).view(torch.float32)


def _divergence(got, ref) -> tuple[float, float, float]:
    """(relative L2 error, largest |error| / RMS of its 128-value row, share of
    elements outside rel 1e-2 / abs 1e-3) of bf16 cache rows against others."""

    g, r = _bf16_f32(got).double(), _bf16_f32(ref).double()
    err = (g - r).abs()
    rms = r.pow(2).mean(dim=-1, keepdim=True).sqrt().clamp_min(1e-6)
    rel_l2 = (err.pow(2).sum() / r.pow(2).sum()).sqrt().item()
    return rel_l2, (err / rms).max().item(), float((err > 1.0e-3 + 1.0e-2 * r.abs()).double().mean())


def _prompt_caches(model, p: int):
    return [tuple(layer[n][:, :p].clone(memory_format=model.torch.contiguous_format)
                  for n in ("key_cache", "value_cache")) for layer in model.layers]


def test_config5_prefill_matches_the_sequential_decode_cache(torch_gpu, native):
    """kudacuda_qwen2_model_prefill of the 64-token prompt through all 36
    layers at once must write the K/V cache rows the sequential decode writes
    and emit the golden first token with the decode bookkeeping.  The decode
    path's rows are pinned first: their digests equal the oracle's (golden).

    The prefill GEMMs take bf16 operands -- the weights as bf16(codebook *
    absmax), as the reference's bitsandbytes dequantize-then-matmul prefill
    does, and the normalised activations as stored bf16 rows -- where the
    decode kernels form fp32 products of fp32 normalised values.  Each
    product therefore differs by up to ~2^-8 relative, so layer 0's rows
    already differ by up to ~2 % of their RMS (half of them by a bf16 ulp or
    more), and every later layer inherits and amplifies what the earlier ones
    changed in the residual stream.  rel 1e-2 / abs 1e-3 per element is not
    reachable for such a pair past layer 0.  What the test holds instead:

    * the model's own sensitivity, measured in the same run: the sequential
      decode repeated with the prompt's embedding rows perturbed by one bf16
      ulp in half of their elements (a perturbation of the size of one
      bf16 rounding of the input) diverges layer by layer the same way; the
      prefill's relative L2 divergence at every layer stays within
      PREFILL_VS_PERTURBED times the perturbed decode's at that layer;
    * layer 0 (identical inputs): every row within 3 % of its RMS and
      relative L2 <= 1 %;
    * every layer: relative L2 <= 6 %, no element beyond 35 % of its row's
      RMS; the share outside rel 1e-2 / abs 1e-3 is printed for each layer.
    """

    torch = torch_gpu
    golden = json.loads(GOLDEN.read_text())
    prompt = np.asarray(golden["prompt"], dtype=np.int32)
    p = prompt.size
    print("[prefill full] building the 36-layer model", flush=True)
    model = Qwen2Nf4Decoder.synthetic(native, torch, seed=golden["seed"], kv_capacity=golden["kv_capacity"],
                                      token_capacity=golden["kv_capacity"], threads=16)
    try:
        print("[prefill full] sequential decode of the prompt", flush=True)
        model.reset(prompt)
        model.capture()
        model.replay(p)  # the 64 prompt steps: rows 0..63, then tokens[64]
        model.stream.synchronize()
        assert int(host(model.tokens)[p]) == golden["tokens"][0]
        seq = _prompt_caches(model, p)
        for li, ((k, v), want) in enumerate(zip(seq, golden["prompt_kv_sha256"])):
            assert _sha(k) == want["key"] and _sha(v) == want["value"], f"layer {li} decode cache vs oracle"

        print("[prefill full] sequential decode with the prompt embeddings perturbed by one ulp", flush=True)
        rows = torch.as_tensor(np.unique(prompt).astype(np.int64), device=model.embed.device)
        gen = torch.Generator(device="cpu").manual_seed(golden["seed"])
        flip = (torch.rand((rows.numel(), model.embed.shape[1]), generator=gen) < 0.5).to(torch.int16).to(
            model.embed.device)
        bits = model.embed.view(torch.int16)
        bits[rows] ^= flip  # the lowest mantissa bit: one ulp up or down
        model.reset(prompt)
        model.replay(p)
        model.stream.synchronize()
        perturbed = _prompt_caches(model, p)
        bits[rows] ^= flip  # restored
        model.stream.synchronize()

        print("[prefill full] multi-token prefill of the same prompt", flush=True)
        for layer in model.layers:  # nothing of the decode may survive into the prefill's rows
            layer["key_cache"].zero_()
            layer["value_cache"].zero_()
        model.prefill(prompt)
        model.stream.synchronize()
        assert int(host(model.tokens)[p]) == golden["tokens"][0]  # golden margin 0.109 at this token
        assert int(host(model.control)[0]) == p
        ratios = []
        for li, (layer, (k_seq, v_seq), (k_pt, v_pt)) in enumerate(zip(model.layers, seq, perturbed)):
            for name, ref, pt in (("key_cache", k_seq, k_pt), ("value_cache", v_seq, v_pt)):
                pre = _divergence(layer[name][:, :p], ref)
                sens = _divergence(pt, ref)
                ratios.append(pre[0] / max(sens[0], 1e-12))
                print(f"[prefill full] layer {li:2d} {name[0]}: prefill relL2 {pre[0]:.4f} max/rms {pre[1]:.4f} "
                      f"outside {pre[2]:.3f} | perturbed decode relL2 {sens[0]:.4f} max/rms {sens[1]:.4f} "
                      f"outside {sens[2]:.3f} | ratio {ratios[-1]:.2f}", flush=True)
                if li == 0:
                    assert pre[0] <= 0.01 and pre[1] <= 0.03, (li, name, pre)
                assert pre[0] <= 0.06 and pre[1] <= 0.35, (li, name, pre)
                assert ratios[-1] <= PREFILL_VS_PERTURBED, (li, name, pre, sens)
        print(f"[prefill full] prefill / perturbed-decode divergence ratio: min {min(ratios):.2f} "
              f"max {max(ratios):.2f}", flush=True)
    finally:
        model.close()
