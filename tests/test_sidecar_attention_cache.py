"""The Qwen2 attention guard writes each decode token to the KV cache once.

A real Transformers ``Qwen2Attention`` (Qwen2.5-3B head layout, fp32, CPU)
and a ``DynamicCache`` run through ``patch_qwen2_attention`` with a bridge
whose native library is the recording fake.  On the CPU the native GQA call
always raises (its tensors are not device tensors), so every decode step
exercises a fallback: a refusal before the cache update (2-D mask), the
framework softmax after it (native exception, non-zero mask), or a loud
``CacheCommittedError`` (a 4-D mask whose key count disagrees with the
cache).  In every case the cache must grow by exactly one row per step,
and the output must equal the unpatched forward on an identical cache.
"""

from __future__ import annotations

import pytest

torch = pytest.importorskip("torch")
transformers = pytest.importorskip("transformers")

from transformers import DynamicCache, Qwen2Config  # noqa: E402
from transformers.models.qwen2.modeling_qwen2 import Qwen2Attention, Qwen2RotaryEmbedding  # noqa: E402

from kudacuda_amd import kudacuda_sidecar as S  # noqa: E402
from tests.test_sidecar_contracts import FakeNative  # noqa: E402

PROMPT = 3


def _config() -> Qwen2Config:
    cfg = Qwen2Config(vocab_size=64, hidden_size=2048, intermediate_size=64, num_hidden_layers=1,
                      num_attention_heads=16, num_key_value_heads=2, max_position_embeddings=64, rope_theta=1e6)
    cfg._attn_implementation = "eager"
    return cfg


@pytest.fixture()
def setup():
    torch.manual_seed(7)
    cfg = _config()
    module = Qwen2Attention(cfg, layer_idx=0).eval()
    rotary = Qwen2RotaryEmbedding(cfg)
    original = Qwen2Attention.forward
    bridge = S.KudaCudaBridge(manifest=S.load_manifest(S.DEFAULT_MANIFEST), native_lib=FakeNative())
    unpatch = S.patch_qwen2_attention(bridge, attention_cls=Qwen2Attention,
                                      tactic_name="qwen2_gqa_decode_gfx950_bf16")
    patched_cache, reference_cache = DynamicCache(config=cfg), DynamicCache(config=cfg)
    hidden = torch.randn(1, PROMPT, 2048)
    pos = torch.arange(PROMPT)[None]
    emb = rotary(hidden, pos)
    with torch.no_grad():  # prompt: the guard refuses multi-token calls, the framework runs
        module(hidden, emb, None, past_key_values=patched_cache, cache_position=pos[0])
        original(module, hidden, emb, None, past_key_values=reference_cache, cache_position=pos[0])
    yield dict(module=module, rotary=rotary, original=original, bridge=bridge, patched=patched_cache,
               reference=reference_cache)
    unpatch()


def _decode_inputs(s, step):
    hidden = torch.randn(1, 1, 2048)
    pos = torch.tensor([[PROMPT + step]])
    return hidden, s["rotary"](hidden, pos), pos[0]


def _mask(kind: str, keys: int):
    if kind == "none":
        return None
    if kind == "2d":
        return torch.zeros(1, keys)
    if kind == "4d_nonzero":
        m = torch.zeros(1, 1, 1, keys)
        m[..., 0] = torch.finfo(torch.float32).min  # hide the first key
        return m
    raise AssertionError(kind)


@pytest.mark.parametrize("kind,reason", [
    ("none", "framework_fallback:native_exception:"),
    ("4d_nonzero", "framework_fallback:attention_mask_values"),
])
def test_fallbacks_after_the_cache_update_write_the_token_once(setup, kind, reason):
    s = setup
    for step in range(4):
        before = s["patched"].get_seq_length(0)
        hidden, emb, cache_pos = _decode_inputs(s, step)
        mask = _mask(kind, before + 1)
        with torch.no_grad():
            got, _ = s["module"](hidden, emb, mask, past_key_values=s["patched"], cache_position=cache_pos)
            want, _ = s["original"](s["module"], hidden, emb, mask, past_key_values=s["reference"],
                                    cache_position=cache_pos)
        assert s["bridge"].last_qwen2_dispatch_reason.startswith(reason), s["bridge"].last_qwen2_dispatch_reason
        assert s["patched"].get_seq_length(0) == before + 1
        assert s["reference"].get_seq_length(0) == before + 1
        assert torch.equal(s["patched"].layers[0].keys, s["reference"].layers[0].keys)
        assert torch.allclose(got, want, rtol=1e-5, atol=1e-6)


def test_two_dimensional_mask_is_refused_before_the_cache_update(setup):
    s = setup
    before = s["patched"].get_seq_length(0)
    hidden, emb, cache_pos = _decode_inputs(s, 0)
    mask = _mask("2d", before + 1)
    # the framework's own forward then runs (and may reject the 2-D mask
    # itself); either way the cache took the token once
    try:
        with torch.no_grad():
            s["module"](hidden, emb, mask, past_key_values=s["patched"], cache_position=cache_pos)
    except Exception:
        pass
    assert s["bridge"].last_qwen2_dispatch_reason == f"attention_mask_shape:(1, {before + 1})"
    assert s["patched"].get_seq_length(0) == before + 1


def test_mask_disagreeing_with_the_cache_raises_instead_of_rerunning(setup):
    s = setup
    before = s["patched"].get_seq_length(0)
    hidden, emb, cache_pos = _decode_inputs(s, 0)
    mask = torch.zeros(1, 1, 1, before + 5)
    with pytest.raises(S.CacheCommittedError, match="attention mask covers"):
        with torch.no_grad():
            s["module"](hidden, emb, mask, past_key_values=s["patched"], cache_position=cache_pos)
    assert s["patched"].get_seq_length(0) == before + 1


def test_mask_disagreeing_without_a_cache_declines_to_the_framework(setup):
    """Without a cache nothing is written before the route is chosen, so a
    mask of another key count is a plain decline: the guard returns None and
    the framework forward runs on the same arguments -- here the framework
    rejects the mask itself, with its own error and not CacheCommittedError."""

    s = setup
    hidden, emb, cache_pos = _decode_inputs(s, 0)
    mask = torch.zeros(1, 1, 1, 5)  # one token attends to itself; the mask is longer
    with torch.no_grad():
        with pytest.raises(RuntimeError) as framework:
            s["original"](s["module"], hidden, emb, mask, past_key_values=None, cache_position=cache_pos)
        with pytest.raises(RuntimeError) as patched:
            s["module"](hidden, emb, mask, past_key_values=None, cache_position=cache_pos)
    assert not isinstance(patched.value, S.CacheCommittedError)
    assert str(patched.value) == str(framework.value)
    assert s["bridge"].last_qwen2_dispatch_reason.startswith("mask_length:"), s["bridge"].last_qwen2_dispatch_reason
