"""Transformers-side hooks with fake modules (intent of the reference's
tests/test_contracts.py:780-1015): fallback, reversibility, workspace
handling and bf16 dispatch selection."""

from __future__ import annotations

from types import SimpleNamespace

from kudacuda_amd import kudacuda_sidecar as S
from tests.test_sidecar_contracts import FakeTensor as _BaseTensor
from tests.test_sidecar_contracts import nf4


class T(_BaseTensor):
    def __add__(self, other):
        return self


class Attention:
    def forward(self, hidden_states, *args, **kwargs):
        return ("fallback", hidden_states, args, kwargs)


class Proj:
    def __init__(self, weight, bias=None):
        self.weight = weight
        self.bias = bias

    def __call__(self, value):
        return value


class Norm:
    def __init__(self, dtype="bfloat16"):
        self.weight = T(dtype=dtype, shape=(2048,), pointer=72)
        self.variance_epsilon = 1.0e-6

    def __call__(self, value):
        return value


class DecoderAttention(Attention):
    def __init__(self):
        self.config = SimpleNamespace(num_attention_heads=16, num_key_value_heads=2)
        self.head_dim = 128
        self.q_proj = Proj(nf4(2048, 2048, 73)[0], T(dtype="bfloat16", shape=(2048,), pointer=76))
        self.k_proj = Proj(nf4(256, 2048, 74)[0], T(dtype="bfloat16", shape=(256,), pointer=77))
        self.v_proj = Proj(nf4(256, 2048, 75)[0], T(dtype="bfloat16", shape=(256,), pointer=78))

    def __call__(self, hidden_states, *args, **kwargs):
        return hidden_states, None


class DecoderLayer:
    def __init__(self):
        self.input_layernorm = Norm()
        self.self_attn = DecoderAttention()
        self.post_attention_layernorm = Norm()
        self.mlp = lambda value: value

    def forward(self, hidden_states, *args, **kwargs):
        return ("layer-fallback", hidden_states, args, kwargs)


class SwiGluMlp:
    def __init__(self):
        self.gate_proj = Proj(nf4(11008, 2048, 131)[0])
        self.up_proj = Proj(nf4(11008, 2048, 141)[0])
        self.down_proj = Proj(T(dtype="uint8", shape=(2048, 1), pointer=151))

    def forward(self, hidden_states, *args, **kwargs):
        return ("mlp-fallback", hidden_states)

    def __call__(self, hidden_states, *args, **kwargs):
        return self.forward(hidden_states, *args, **kwargs)


class SwiGluAttention:
    def __call__(self, *, hidden_states, **kwargs):
        return hidden_states, None


class SwiGluLayer:
    def __init__(self, dtype="float16"):
        self.input_layernorm = lambda value: value
        self.self_attn = SwiGluAttention()
        self.post_attention_layernorm = Norm(dtype)
        self.mlp = SwiGluMlp()

    def forward(self, hidden_states, *args, **kwargs):
        return ("layer-fallback", hidden_states, args, kwargs)


class Model:
    def __init__(self, layer):
        self.model = SimpleNamespace(layers=[layer])
        self.config = SimpleNamespace(model_type="qwen2")


class RecordingBridge:
    def __init__(self, enabled=True):
        self.enabled = enabled
        self.calls = []
        self.native_swiglu_hook_calls = 0

    def matches_contract(self, tactic_name, batch_size, seq_len, *, tensor=None):
        return self.enabled and tactic_name == "gqa8_attn"

    def dispatch_attention(self, module, hidden_states, *args, **kwargs):
        self.calls.append(("attention", hidden_states))
        return ("hot", hidden_states)

    def dispatch_qwen2_swiglu_nf4(self, *args, **kwargs):
        self.calls.append(("swiglu", args, kwargs))

    def dispatch_qwen2_swiglu_nf4_bf16(self, *args, **kwargs):
        self.calls.append(("swiglu_bf16", args, kwargs))

    def dispatch_qwen2_fused_rmsnorm_qkv_nf4(self, *args, **kwargs):
        self.calls.append(("qkv", args, kwargs))
        self.native_fused_qkv_dispatches = getattr(self, "native_fused_qkv_dispatches", 0) + 1


class FakeTorch:
    float32 = "float32"
    cuda = SimpleNamespace(current_stream=lambda device: SimpleNamespace(cuda_stream=77))

    @staticmethod
    def empty(shape, *, device, dtype):
        return T(dtype=dtype, shape=tuple(shape), device=device, pointer=900)


def test_llama_patch_falls_back_dispatches_and_unpatches():
    original = Attention.forward
    off = S.patch_llama_attention(RecordingBridge(enabled=False), attention_cls=Attention)
    assert Attention().forward(T(shape=(1, 2, 8)), flag=True)[0] == "fallback"
    off()
    assert Attention.forward is original
    bridge = RecordingBridge(enabled=True)
    off = S.patch_llama_attention(bridge, attention_cls=Attention)
    assert Attention().forward(T(shape=(1, 2, 8)))[0] == "hot"
    off()
    off()  # idempotent
    assert Attention.forward is original and len(bridge.calls) == 1


def test_qwen2_attention_patch_falls_back_when_dispatcher_declines():
    original = Attention.forward

    class Declining:
        def dispatch_qwen2_attention(self, module, hidden_states, *args, tactic_name, **kwargs):
            return None

    off = S.patch_qwen2_attention(Declining(), attention_cls=Attention)
    assert Attention().forward(T(shape=(1, 1, 2048)))[0] == "fallback"
    off()
    assert Attention.forward is original


def test_qwen2_attention_patch_uses_dispatcher_result_and_survives_errors():
    class Accepting:
        def dispatch_qwen2_attention(self, module, hidden_states, *args, tactic_name, **kwargs):
            return ("native", tactic_name)

    class Raising:
        def dispatch_qwen2_attention(self, *a, **k):
            raise RuntimeError("boom")

    off = S.patch_qwen2_attention(Accepting(), attention_cls=Attention, tactic_name="t")
    assert Attention().forward(T(shape=(1, 1, 2048))) == ("native", "t")
    off()
    off = S.patch_qwen2_attention(Raising(), attention_cls=Attention)
    assert Attention().forward(T(shape=(1, 1, 2048)))[0] == "fallback"
    off()


def test_fused_qkv_patch_dispatches_prefuses_and_is_reversible():
    model = Model(DecoderLayer())
    layer = model.model.layers[0]
    original_layer = layer.forward
    original_attention = DecoderAttention.forward
    bridge = RecordingBridge(enabled=False)
    off = S.patch_qwen2_fused_qkv(model, bridge, torch_module=FakeTorch())
    state = layer.self_attn._kudacuda_fused_qkv_state
    assert state["query"].shape == (1, 2048) and state["normalized"].dtype == "float32"
    out = layer.forward(T(dtype="bfloat16", shape=(1, 1, 2048), pointer=111))
    assert isinstance(out, T)
    kind, args, kwargs = bridge.calls[0]
    assert kind == "qkv" and args[0].shape == (1, 2048) and kwargs["stream_ptr"] == 77
    assert kwargs["tactic_name"] == S.DEFAULT_QKV_TACTIC
    assert bridge.last_qwen2_fused_qkv_dispatch_reason == "native"
    assert not hasattr(layer.self_attn, "_kudacuda_prefused_qkv")   # cleared after the layer
    # off-contract shape goes to the original layer
    assert layer.forward(T(dtype="bfloat16", shape=(1, 4, 2048)))[0] == "layer-fallback"
    off()
    assert layer.forward.__func__ is original_layer.__func__
    assert DecoderAttention.forward is original_attention
    assert not hasattr(layer.self_attn, "_kudacuda_fused_qkv_state")


def test_fused_qkv_patch_falls_back_without_bias():
    model = Model(DecoderLayer())
    layer = model.model.layers[0]
    layer.self_attn.k_proj.bias = None
    bridge = RecordingBridge()
    off = S.patch_qwen2_fused_qkv(model, bridge, torch_module=FakeTorch())
    assert layer.forward(T(dtype="bfloat16", shape=(1, 1, 2048)))[0] == "layer-fallback"
    assert bridge.last_qwen2_fused_qkv_dispatch_reason == "missing_projection_bias"
    off()


def test_swiglu_patch_runs_native_and_is_reversible():
    model = Model(SwiGluLayer())
    layer = model.model.layers[0]
    original_layer = layer.forward
    original_mlp = layer.mlp.forward
    bridge = RecordingBridge()
    off = S.patch_qwen2_swiglu(model, bridge, torch_module=FakeTorch())
    assert layer.mlp.forward.__func__ is original_mlp.__func__
    result = layer.forward(T(dtype="float16", shape=(1, 1, 2048), pointer=111))
    assert isinstance(result, T)
    kind, args, kwargs = bridge.calls[0]
    assert kind == "swiglu" and args[0].shape == (1, 2048) and kwargs["stream_ptr"] == 77
    assert bridge.native_swiglu_hook_calls == 1 and bridge.last_swiglu_dispatch_reason == "native"
    off()
    assert layer.forward.__func__ is original_layer.__func__
    assert not hasattr(layer, "_kudacuda_swiglu_state")


def test_swiglu_patch_selects_bf16_dispatch_and_keeps_framework_fallbacks():
    model = Model(SwiGluLayer("bfloat16"))
    layer = model.model.layers[0]
    bridge = RecordingBridge()
    off = S.patch_qwen2_swiglu(model, bridge, tactic_name=S.DEFAULT_SWIGLU_BF16_TACTIC, torch_module=FakeTorch())
    layer.forward(T(dtype="bfloat16", shape=(1, 1, 2048)))
    assert bridge.calls[0][0] == "swiglu_bf16"
    assert bridge.calls[0][2]["tactic_name"] == S.DEFAULT_SWIGLU_BF16_TACTIC
    # wrong shape -> original layer
    assert layer.forward(T(dtype="bfloat16", shape=(2, 1, 2048)))[0] == "layer-fallback"
    # projection bias -> framework MLP after native attention
    layer.mlp.gate_proj.bias = T(dtype="bfloat16", shape=(11008,))
    out = layer.forward(T(dtype="bfloat16", shape=(1, 1, 2048)))
    assert isinstance(out, T) and bridge.last_swiglu_dispatch_reason == "unexpected_projection_bias"
    off()
