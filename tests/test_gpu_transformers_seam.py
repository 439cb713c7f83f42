"""GPU: the Transformers seam end to end.

A random-init Transformers ``Qwen2ForCausalLM`` with the Qwen2.5-3B layer
shape (hidden 2048, intermediate 11008, 16/2 heads of 128, QKV bias, RoPE
theta 1e6; 2 layers and a 4096-token tied vocabulary to keep it small) is
NF4-quantised on the GPU (``nf4_params.quantize_qwen2_model``) and decoded
greedily one token at a time through the reference's patch API
(python/kudacuda_sidecar.py:1524-1952): the fused RMSNorm+QKV hook with the
native GQA attention, and the SwiGLU hook with the native GQA attention.  The
logits are checked against the same model in fp32 on the CPU (its NF4
weights dequantised), the native dispatch reasons are checked at every step,
and ``StaticDecodeGraphRunner`` on ``torch.cuda.CUDAGraph``
(python/kudacuda_static_decode.py:177-447) replays decode steps that must
equal the eager patched steps.

Every decode step here is a single token, so the patched layers take every
call and no framework bf16 attention runs on the GPU (its batched products
are avoided on this pool); the CPU reference uses Transformers' eager
attention in fp32.
"""

from __future__ import annotations

import copy

import numpy as np
import pytest

from kudacuda_amd import kudacuda_sidecar as S
from kudacuda_amd import nf4_params as P
from kudacuda_amd.kudacuda_graph_plan import GraphContractError
from kudacuda_amd.kudacuda_static_decode import GraphStaticCache, StaticDecodeGraphRunner

pytestmark = pytest.mark.gpu
SEED = 20260824
LAYERS = 2
VOCAB = 4096
PROMPT = 6
NEW = 10
BUCKET = 64
QKV_TACTIC = "qwen2_fused_rmsnorm_qkv_gfx950_bf16_nf4_v1"
GQA_TACTIC = "qwen2_gqa_decode_gfx950_bf16"
GQA_GRAPH_TACTIC = "qwen2_gqa_decode_gfx950_bf16_graph_v1"
SWIGLU_TACTIC = "qwen2_swiglu_gfx950_bf16_nf4_v1"
# bf16 activations on the GPU against fp32 on the CPU, 2 layers: logits
# (|logit| up to ~4) agree to this absolute bound (measured: 0.05)
LOGIT_ATOL = 0.1


@pytest.fixture(scope="module")
def bridge(torch_gpu):
    b = S.KudaCudaBridge()
    yield b
    b.shutdown()


@pytest.fixture(scope="module")
def models(torch_gpu, bridge):
    torch = torch_gpu
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=VOCAB, hidden_size=2048, intermediate_size=11008, num_hidden_layers=LAYERS,
                      num_attention_heads=16, num_key_value_heads=2, max_position_embeddings=4096, rope_theta=1e6,
                      rms_norm_eps=1e-6, tie_word_embeddings=True)
    cfg._attn_implementation = "eager"
    torch.manual_seed(SEED)
    cpu = Qwen2ForCausalLM(cfg).eval()
    with torch.no_grad():  # non-trivial norms and biases so every epilogue term matters
        for layer in cpu.model.layers:
            layer.input_layernorm.weight.normal_(1.0, 0.1)
            layer.post_attention_layernorm.weight.normal_(1.0, 0.1)
            for proj in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj):
                proj.bias.normal_(0.0, 0.02)
        cpu.model.norm.weight.normal_(1.0, 0.1)
    gpu = copy.deepcopy(cpu).to(device="cuda:0", dtype=torch.bfloat16).eval()
    P.quantize_qwen2_model(bridge, torch, gpu)
    # the CPU reference holds exactly what the GPU model holds, in fp32
    with torch.no_grad():
        for lc, lg in zip(cpu.model.layers, gpu.model.layers):
            for pc, pg, names in ((lc.self_attn, lg.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                                  (lc.mlp, lg.mlp, ("gate_proj", "up_proj", "down_proj"))):
                for name in names:
                    src, dst = getattr(pg, name), getattr(pc, name)
                    dst.weight.copy_(P.dequantize(bridge, torch, src.weight, dtype=torch.float32).cpu())
                    if src.bias is not None:
                        dst.bias.copy_(src.bias.float().cpu())
            lc.input_layernorm.weight.copy_(lg.input_layernorm.weight.float().cpu())
            lc.post_attention_layernorm.weight.copy_(lg.post_attention_layernorm.weight.float().cpu())
        cpu.model.norm.weight.copy_(gpu.model.norm.weight.float().cpu())
        cpu.model.embed_tokens.weight.copy_(gpu.model.embed_tokens.weight.float().cpu())
    torch.cuda.synchronize()
    prompt = np.random.default_rng(SEED).integers(0, VOCAB, PROMPT).tolist()
    return cpu, gpu, prompt


def _step(torch, model, token, pos, cache, **extra):
    dev = "cuda:0"
    out = model(torch.tensor([[token]], device=dev), past_key_values=cache, use_cache=True,
                cache_position=torch.tensor([pos], device=dev), position_ids=torch.tensor([[pos]], device=dev),
                **extra)
    return out.logits[0, -1]


def _greedy_eager(torch, model, prompt, new, check=None):
    """Token-by-token greedy decode; returns tokens and the logits of every
    position from the last prompt token on."""

    from transformers import DynamicCache

    cache = DynamicCache(config=model.config)
    tokens, logits = list(prompt), []
    with torch.inference_mode():
        for pos in range(len(prompt) + new - 1):
            lg = _step(torch, model, tokens[pos], pos, cache).float()
            if check is not None:
                check(pos)
            if pos >= len(prompt) - 1:
                logits.append(lg.cpu())
                if pos + 1 == len(tokens):
                    tokens.append(int(torch.argmax(lg)))
    torch.cuda.synchronize()
    return tokens, torch.stack(logits)


def _cpu_logits(torch, cpu, tokens):
    with torch.inference_mode():
        return cpu(torch.tensor([tokens])).logits[0].float()


def _check_against_cpu(torch, cpu, tokens, logits):
    ref = _cpu_logits(torch, cpu, tokens)[PROMPT - 1: PROMPT - 1 + logits.shape[0]]
    err = (logits - ref).abs().max().item()
    print(f"max |gpu - cpu fp32| logit error {err:.4f} (logit range {ref.abs().max().item():.3f})", flush=True)
    assert err <= LOGIT_ATOL
    # every logit is within err of the reference, so the greedy token must
    # agree wherever the reference's top-2 margin exceeds 2 * err
    top2 = torch.topk(ref, 2, dim=-1).values
    decisive = (top2[:, 0] - top2[:, 1]) > 2 * err
    got, want = logits.argmax(-1), ref.argmax(-1)
    print(f"greedy token checked at {int(decisive.sum())} of {logits.shape[0]} positions", flush=True)
    assert bool(torch.all((got == want) | ~decisive))
    assert int(decisive.sum()) >= 3  # the check is not vacuous


def test_fused_qkv_and_attention_patches_decode_like_the_fp32_model(torch_gpu, bridge, models):
    torch = torch_gpu
    cpu, gpu, prompt = models
    print(f"seam: fused QKV + GQA patches, {LAYERS} layers, prompt {prompt}", flush=True)
    unpatch = S.patch_qwen2_fused_qkv(gpu, bridge, tactic_name=QKV_TACTIC, attention_tactic_name=GQA_TACTIC)
    before = int(getattr(bridge, "native_fused_qkv_dispatches", 0))

    def native_every_step(pos):
        assert bridge.last_qwen2_fused_qkv_dispatch_reason == "native", (pos, bridge.last_qwen2_fused_qkv_dispatch_reason)
        assert bridge.last_qwen2_dispatch_reason == "native", (pos, bridge.last_qwen2_dispatch_reason)

    try:
        tokens, logits = _greedy_eager(torch, gpu, prompt, NEW, check=native_every_step)
    finally:
        unpatch()
    steps = PROMPT + NEW - 1
    assert int(getattr(bridge, "native_fused_qkv_dispatches", 0)) - before == steps * LAYERS
    _check_against_cpu(torch, cpu, tokens, logits)
    assert not hasattr(gpu.model.layers[0].self_attn, "_kudacuda_fused_qkv_state")  # unpatched cleanly


def test_swiglu_and_attention_patches_decode_like_the_fp32_model(torch_gpu, bridge, models):
    torch = torch_gpu
    cpu, gpu, prompt = models
    print("seam: SwiGLU + GQA patches", flush=True)
    unpatch_attn = S.patch_qwen2_attention(bridge, tactic_name=GQA_TACTIC)
    unpatch_mlp = S.patch_qwen2_swiglu(gpu, bridge, tactic_name=SWIGLU_TACTIC)

    def native_every_step(pos):
        assert bridge.last_swiglu_dispatch_reason == "native", (pos, bridge.last_swiglu_dispatch_reason)
        assert bridge.last_qwen2_dispatch_reason == "native", (pos, bridge.last_qwen2_dispatch_reason)

    try:
        tokens, logits = _greedy_eager(torch, gpu, prompt, NEW, check=native_every_step)
    finally:
        unpatch_mlp()
        unpatch_attn()
    _check_against_cpu(torch, cpu, tokens, logits)


def test_static_graph_runner_replays_decode_like_the_fp32_model(torch_gpu, bridge, models):
    """Capture one patched decode forward with torch.cuda.CUDAGraph (graph-mode
    attention reads kv_len from device memory) and replay it for the next
    tokens: every replay's logits match the fp32 model as the eager steps do.
    (Replays are not bit-equal to the eager steps: the framework's own GEMMs
    for o_proj and the MLP may run other library kernels under capture.)"""

    from transformers import DynamicCache

    torch = torch_gpu
    cpu, gpu, prompt = models
    print("seam: StaticDecodeGraphRunner on torch.cuda.CUDAGraph", flush=True)
    unpatch = S.patch_qwen2_fused_qkv(gpu, bridge, tactic_name=QKV_TACTIC, attention_tactic_name=GQA_GRAPH_TACTIC)
    try:
        want_tokens, want_logits = _greedy_eager(torch, gpu, prompt, NEW)
        cache = DynamicCache(config=gpu.config)
        with torch.inference_mode():
            for pos in range(PROMPT):  # prefill (direct-mode attention)
                _step(torch, gpu, prompt[pos], pos, cache)
        torch.cuda.synchronize()
        static = GraphStaticCache.from_dynamic_cache(torch, cache, max_cache_len=BUCKET)
        runner = StaticDecodeGraphRunner(bridge, gpu, torch)
        stream = torch.cuda.Stream()
        dev = "cuda:0"
        mask = {"full_attention": torch.zeros((1, 1, 1, BUCKET), dtype=torch.bfloat16, device=dev)}
        got = []
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            pos = PROMPT
            runner.capture(input_ids=torch.tensor([[want_tokens[pos]]], device=dev),
                           position_ids=torch.tensor([[pos]], device=dev), attention_mask=mask,
                           cache_position=static.cache_position, past_key_values=static, logical_kv_len=pos,
                           kv_bucket=BUCKET, tactic_name=GQA_GRAPH_TACTIC, stream_ptr=int(stream.cuda_stream),
                           stream=stream)
            stream.synchronize()
            assert bridge.last_qwen2_dispatch_reason == "native", bridge.last_qwen2_dispatch_reason
            got.append(runner.logits[0, -1].float().cpu())
            for pos in range(PROMPT + 1, PROMPT + NEW - 1):
                runner.replay(next_token=torch.tensor([[want_tokens[pos]]], device=dev),
                              position_ids=torch.tensor([[pos]], device=dev), cache_position=pos,
                              logical_kv_len=pos, stream_ptr=int(stream.cuda_stream))
                stream.synchronize()
                got.append(runner.logits[0, -1].float().cpu())
        torch.cuda.synchronize()
        assert runner.replay_count == NEW - 1  # the capture's own run counts as the first
        got = torch.stack(got)
        ref = want_logits[1: 1 + got.shape[0]]
        err = (got - ref).abs().max().item()
        print(f"graph replay vs eager max |diff| {err:.3g} over {got.shape[0]} steps", flush=True)
        assert err <= LOGIT_ATOL
        # positions PROMPT .. PROMPT+NEW-2, teacher-forced on the eager tokens
        _check_against_cpu(torch, cpu, want_tokens[: PROMPT + NEW - 1],
                           torch.cat([want_logits[:1], got]))
    finally:
        runner_state = locals().get("runner")
        if runner_state is not None and runner_state.captured:
            runner_state.invalidate("test end")
        unpatch()


def test_static_graph_runner_native_recorder_replays_decode_like_the_fp32_model(torch_gpu, bridge, models):
    """The same runner with ``stream=None``: the forward is recorded by the
    bridge's own hipGraph (kudacuda_begin_capture / end_capture on the
    caller's stream, replayed by kudacuda_replay_graph), the path the
    reference takes when PyTorch has no graph API
    (python/kudacuda_static_decode.py:317-348).  PyTorch does not know about
    this capture, so the forward's temporaries are allocated from a private
    memory pool that is warmed by one eager forward first (no device
    allocation inside the capture) and kept until the graph is reset: blocks
    the replays write are never handed to other tensors."""

    torch = torch_gpu
    cpu, gpu, prompt = models
    print("seam: StaticDecodeGraphRunner on the native recorder", flush=True)
    unpatch = S.patch_qwen2_fused_qkv(gpu, bridge, tactic_name=QKV_TACTIC, attention_tactic_name=GQA_GRAPH_TACTIC)
    runner = None
    pool = torch.cuda.MemPool()
    try:
        want_tokens, want_logits = _greedy_eager(torch, gpu, prompt, NEW)
        from transformers import DynamicCache

        cache = DynamicCache(config=gpu.config)
        with torch.inference_mode():
            for pos in range(PROMPT):
                _step(torch, gpu, prompt[pos], pos, cache)
        torch.cuda.synchronize()
        static = GraphStaticCache.from_dynamic_cache(torch, cache, max_cache_len=BUCKET)
        stream = torch.cuda.Stream()
        dev = "cuda:0"
        mask = {"full_attention": torch.zeros((1, 1, 1, BUCKET), dtype=torch.bfloat16, device=dev)}
        got = []
        pos = PROMPT
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream), torch.cuda.use_mem_pool(pool):
            # warm the pool: the capture's forward then finds every block it needs
            kv_len_device = torch.tensor([pos + 1], dtype=torch.int32, device=dev)
            static.cache_position.copy_(torch.tensor([pos], device=dev))
            bridge.configure_qwen2_graph_dispatch(kv_len_device=kv_len_device, kv_capacity=BUCKET)
            try:
                with torch.inference_mode():
                    gpu(input_ids=torch.tensor([[want_tokens[pos]]], device=dev),
                        position_ids=torch.tensor([[pos]], device=dev), attention_mask=mask, past_key_values=static,
                        cache_position=static.cache_position, use_cache=True, return_dict=True)
            finally:
                bridge.clear_qwen2_graph_dispatch()
            stream.synchronize()
            runner = StaticDecodeGraphRunner(bridge, gpu, torch)
            runner.capture(input_ids=torch.tensor([[want_tokens[pos]]], device=dev),
                           position_ids=torch.tensor([[pos]], device=dev), attention_mask=mask,
                           cache_position=static.cache_position, past_key_values=static, logical_kv_len=pos,
                           kv_bucket=BUCKET, tactic_name=GQA_GRAPH_TACTIC, stream_ptr=int(stream.cuda_stream),
                           stream=None)
        assert runner.backend == "native" and runner.cuda_graph is None
        with torch.cuda.stream(stream):
            stream.synchronize()
            assert bridge.last_qwen2_dispatch_reason == "native", bridge.last_qwen2_dispatch_reason
            got.append(runner.logits[0, -1].float().cpu())
            for pos in range(PROMPT + 1, PROMPT + NEW - 1):
                runner.replay(next_token=torch.tensor([[want_tokens[pos]]], device=dev),
                              position_ids=torch.tensor([[pos]], device=dev), cache_position=pos,
                              logical_kv_len=pos, stream_ptr=int(stream.cuda_stream))
                stream.synchronize()
                got.append(runner.logits[0, -1].float().cpu())
        torch.cuda.synchronize()
        assert runner.replay_count == NEW - 1
        got = torch.stack(got)
        ref = want_logits[1: 1 + got.shape[0]]
        err = (got - ref).abs().max().item()
        print(f"native graph replay vs eager max |diff| {err:.3g} over {got.shape[0]} steps", flush=True)
        assert err <= LOGIT_ATOL
        _check_against_cpu(torch, cpu, want_tokens[: PROMPT + NEW - 1], torch.cat([want_logits[:1], got]))
        # a replay whose stream differs from the captured one is refused before anything runs
        with pytest.raises(GraphContractError, match="stream changed"):
            runner.replay(next_token=torch.tensor([[0]], device=dev), position_ids=torch.tensor([[pos]], device=dev),
                          cache_position=pos, logical_kv_len=pos, stream_ptr=int(stream.cuda_stream) + 1)
    finally:
        torch.cuda.synchronize()
        if runner is not None and runner.captured:
            runner.invalidate("test end")
        unpatch()
        del runner
