"""Bridge marshalling and guards against a recording fake of libkudacuda.

Restates the intent of the reference's tests/test_contracts.py:
the positional argument tuple each native symbol receives, the
manifest/contract gating, fail-closed validation and error surfacing, with
the gfx950 manifest and the bf16 tactics added.
"""

from __future__ import annotations

import copy
import math
from types import SimpleNamespace

import pytest

from kudacuda_amd import kudacuda_sidecar as S
from kudacuda_amd._native import SIGNATURES

HANDLE = 101


class FakeFn:
    def __init__(self, name, owner):
        self.name = name
        self.owner = owner
        self.argtypes = None
        self.restype = None

    def __call__(self, *args):
        self.owner.calls.append((self.name, *args))
        return self.owner.results.get(self.name, 0)


class FakeNative:
    """Every header symbol records its call; statuses are configurable."""

    def __init__(self, missing=(), **results):
        self.calls = []
        self.results = {"kudacuda_can_dispatch": 1}
        self.results.update({f"kudacuda_{k}": v for k, v in results.items()})
        for name in SIGNATURES:
            if name not in missing:
                setattr(self, name, FakeFn(name, self))
        self.kudacuda_create = lambda device: HANDLE
        self.kudacuda_last_error = lambda handle: b"fake native error"
        self.kudacuda_lm_head_workspace_floats = lambda: 1536


class FakeTensor:
    def __init__(self, *, dtype="float32", shape=(4,), device="cuda", contiguous=True, pointer=100,
                 quant_state=None):
        self.dtype, self.shape, self.device = dtype, tuple(shape), device
        self._contiguous, self._pointer, self.quant_state = contiguous, pointer, quant_state

    @property
    def is_cuda(self):
        return self.device == "cuda"

    def is_contiguous(self):
        return self._contiguous

    def dim(self):
        return len(self.shape)

    def numel(self):
        return math.prod(self.shape)

    def data_ptr(self):
        return self._pointer

    def reshape(self, *shape):
        return FakeTensor(dtype=self.dtype, shape=shape, device=self.device, contiguous=self._contiguous,
                          pointer=self._pointer, quant_state=self.quant_state)


class QuantState:
    def __init__(self, shape, *, blocksize=64, quant_type="nf4", nested=False, pointer=500):
        self.shape, self.blocksize, self.quant_type, self.nested = shape, blocksize, quant_type, nested
        self.absmax = FakeTensor(dtype="float32", shape=((shape[0] * shape[1] + blocksize - 1) // blocksize,),
                                 pointer=pointer)


def nf4(rows, cols, pointer, **kw):
    state = QuantState((rows, cols), pointer=pointer + 1, **kw)
    return FakeTensor(dtype="uint8", shape=(rows * cols // 2, 1), pointer=pointer, quant_state=state), state.absmax


def manifest():
    return S.load_manifest(S.DEFAULT_MANIFEST)


def bridge(native=None, man=None):
    return S.KudaCudaBridge(manifest=man or manifest(), native_lib=native or FakeNative())


def qkv_tensors(dtype="bfloat16", **kw):
    qw, qa = nf4(2048, 2048, 31, **kw)
    kw_, ka = nf4(256, 2048, 41, **kw)
    vw, va = nf4(256, 2048, 51, **kw)
    t = lambda shape, p: FakeTensor(dtype=dtype, shape=shape, pointer=p)  # noqa: E731
    return (t((1, 2048), 11), t((2048,), 22), qw, qa, t((2048,), 33), kw_, ka, t((256,), 43), vw, va,
            t((256,), 53), t((1, 2048), 61), t((1, 256), 62), t((1, 256), 63))


def swiglu_tensors(dtype="float16", **kw):
    gw, ga = nf4(11008, 2048, 131, **kw)
    uw, ua = nf4(11008, 2048, 141, **kw)
    return (FakeTensor(dtype=dtype, shape=(1, 2048), pointer=111), FakeTensor(dtype=dtype, shape=(2048,), pointer=122),
            gw, ga, uw, ua, FakeTensor(dtype=dtype, shape=(1, 11008), pointer=151))


def gqa_tensors(dtype, kv):
    return (FakeTensor(dtype=dtype, shape=(1, 16, 1, 128), pointer=11),
            FakeTensor(dtype=dtype, shape=(1, 2, kv, 128), pointer=22),
            FakeTensor(dtype=dtype, shape=(1, 2, kv, 128), pointer=33),
            FakeTensor(dtype=dtype, shape=(1, 16, 1, 128), pointer=44))


# ------------------------------------------------------------------ manifest
def test_manifest_loader_and_library_names(tmp_path):
    m = manifest()
    assert m["target_arch"] == "gfx950"
    assert {"vector_add", "rmsnorm", "qwen2_gqa_decode_gfx950_bf16"} <= set(m["implemented_tactics"])
    assert S.select_library_name("linux") == "libkudacuda.so"
    assert S.select_library_name("win32") == "kudacuda.dll"
    bad = tmp_path / "m.json"
    bad.write_text('{"target_arch": "gfx950", "contracts": {}}')
    with pytest.raises(ValueError, match="implemented_tactics"):
        S.load_manifest(bad)


def test_every_preferred_tactic_is_enabled_and_resolves_to_a_symbol():
    b = bridge()
    m = manifest()
    for key, name in m.items():
        if key.startswith("preferred_"):
            assert b.tactic_status(name) in ("implemented", "experimental"), name
    assert b.tactic_status("gqa8_attn") == "planned"
    assert b.tactic_status("not_a_tactic") == "unknown"


def test_missing_symbol_makes_the_tactic_unavailable():
    b = bridge(FakeNative(missing=("kudacuda_qwen2_gqa_decode_bf16",)))
    assert b.tactic_status("qwen2_gqa_decode_gfx950_bf16") == "unavailable"
    assert b.tactic_status("qwen2_gqa_decode_gfx950_fp16") == "implemented"


def test_missing_required_symbol_fails_at_construction():
    with pytest.raises(S.NativeCudaError, match="kudacuda_reset_graph"):
        bridge(FakeNative(missing=("kudacuda_reset_graph",)))


def test_null_handle_raises():
    native = FakeNative()
    native.kudacuda_create = lambda device: None
    with pytest.raises(S.NativeCudaError, match="null handle"):
        bridge(native)


# ------------------------------------------------------------------ contracts
def test_tensor_contract_shape_and_metadata():
    c = S.TensorContract.from_mapping({"dtype": "float32", "layout": "contiguous", "rank": 3, "batch_size": 2,
                                       "seq_len": 4})
    assert c.matches_shape(2, 4) and not c.matches_shape(1, 4) and not c.matches_shape(2, 8)
    v = S.TensorContract.from_mapping({"dtype": "torch.float32", "layout": "contiguous", "rank": 1, "count_min": 1})
    assert v.matches_tensor(FakeTensor())
    assert not v.matches_tensor(FakeTensor(device="cpu"))
    assert not v.matches_tensor(FakeTensor(contiguous=False))
    assert not v.matches_tensor(FakeTensor(dtype="float16"))
    assert not v.matches_tensor(FakeTensor(shape=(0,)))


def test_qwen2_contract_profile():
    c = S.Qwen2GqaContract.from_mapping(manifest()["contracts"]["qwen2_gqa_decode_gfx950_bf16"])
    assert c.matches(1, 1, 1) and c.matches(1, 1, 65536)
    assert not c.matches(2, 1, 128) and not c.matches(1, 2, 128) and not c.matches(1, 1, 0)
    assert not c.matches(1, 1, 65537)
    ws = S.Qwen2GqaContract.from_mapping(manifest()["contracts"]["qwen2_gqa_decode_gfx950_fp16_workspace_v3"])
    assert ws.matches(1, 1, 512) and not ws.matches(1, 1, 513)


def test_attention_dimensions_from_config():
    module = SimpleNamespace(config=SimpleNamespace(num_attention_heads=16, num_key_value_heads=2), head_dim=128)
    assert S._qwen2_attention_dimensions(module) == (16, 2, 128)
    module = SimpleNamespace(config=SimpleNamespace(num_attention_heads=16, num_key_value_heads=2, hidden_size=2048))
    assert S._qwen2_attention_dimensions(module) == (16, 2, 128)


def test_matches_contract_consults_manifest_and_native():
    b = bridge()
    assert b.matches_contract("vector_add", 1, 4, tensor=FakeTensor())
    assert not b.matches_contract("gqa8_attn", 1, 16)
    native = FakeNative(can_dispatch=0)
    assert not bridge(native).matches_contract("vector_add", 1, 4)


# ------------------------------------------------------------------ basic ops
def test_vector_add_and_rmsnorm_marshalling_and_errors():
    native = FakeNative()
    b = bridge(native)
    b.vector_add(FakeTensor(pointer=11), FakeTensor(pointer=22), FakeTensor(pointer=33), stream_ptr=77)
    assert native.calls[-1] == ("kudacuda_vector_add", HANDLE, 11, 22, 33, 4, 77)
    b.rmsnorm(FakeTensor(shape=(2, 4), pointer=11), FakeTensor(shape=(4,), pointer=22),
              FakeTensor(shape=(2, 4), pointer=33), epsilon=1e-5, stream_ptr=-1)
    name, *args = native.calls[-1]
    assert name == "kudacuda_rmsnorm" and args[:6] == [HANDLE, 11, 22, 33, 2, 4]
    assert args[7] == (1 << 64) - 1            # signed stream handle masked to uint64
    with pytest.raises(ValueError, match="weight"):
        b.rmsnorm(FakeTensor(shape=(2, 4)), FakeTensor(shape=(3,)), FakeTensor(shape=(2, 4)), stream_ptr=0)
    with pytest.raises(S.NativeCudaError, match="fake native error"):
        bridge(FakeNative(vector_add=7)).vector_add(FakeTensor(), FakeTensor(), FakeTensor(), stream_ptr=0)


def test_fused_rmsnorm_qkv_dense():
    native = FakeNative()
    b = bridge(native)
    b.fused_rmsnorm_qkv(FakeTensor(dtype="float16", shape=(2, 4), pointer=11),
                        FakeTensor(dtype="float16", shape=(4,), pointer=22),
                        FakeTensor(dtype="float16", shape=(12, 4), pointer=33),
                        FakeTensor(dtype="float16", shape=(12,), pointer=44),
                        FakeTensor(dtype="float16", shape=(2, 12), pointer=55), epsilon=1e-5, stream_ptr=77)
    assert native.calls[-1][:9] == ("kudacuda_fused_rmsnorm_qkv", HANDLE, 11, 22, 33, 44, 55, 2, 4)


# ------------------------------------------------------------------ attention
@pytest.mark.parametrize("tactic,dtype,symbol", [
    ("qwen2_gqa_decode_gfx950_bf16", "bfloat16", "kudacuda_qwen2_gqa_decode_bf16"),
    ("qwen2_gqa_decode_gfx950_fp16", "float16", "kudacuda_qwen2_gqa_decode"),
    ("qwen2_gqa_decode_gfx950_fp16_group_tiled_v2", "float16", "kudacuda_qwen2_gqa_decode_group_tiled"),
    ("qwen2_gqa_decode_gfx950_fp16_vectorized_v2", "float16", "kudacuda_qwen2_gqa_decode_vectorized"),
])
def test_gqa_direct_passes_pointers_dims_scale_and_stream(tactic, dtype, symbol):
    native = FakeNative()
    b = bridge(native)
    b.dispatch_qwen2_gqa_decode(*gqa_tensors(dtype, 128), kv_len=128, stream_ptr=77, tactic_name=tactic)
    call = native.calls[-1]
    assert call[0] == symbol
    assert call[1:6] == (HANDLE, 11, 22, 33, 44)
    assert call[6:12] == (1, 1, 128, 16, 2, 128)
    assert call[12] == pytest.approx(1.0 / math.sqrt(128.0))
    assert call[13] == 77


def test_gqa_rejects_wrong_dtype_length_and_graph_tactic():
    b = bridge()
    with pytest.raises(ValueError, match="query"):
        b.dispatch_qwen2_gqa_decode(*gqa_tensors("float16", 128), kv_len=128, stream_ptr=0)
    with pytest.raises(ValueError, match="kv_len"):
        b.dispatch_qwen2_gqa_decode(*gqa_tensors("bfloat16", 70000), kv_len=70000, stream_ptr=0)
    with pytest.raises(S.NativeCudaError, match="graph"):
        b.dispatch_qwen2_gqa_decode(*gqa_tensors("bfloat16", 8), kv_len=8, stream_ptr=0,
                                    tactic_name="qwen2_gqa_decode_gfx950_bf16_graph_v1")
    with pytest.raises(S.NativeCudaError, match="fake native error"):
        bridge(FakeNative(qwen2_gqa_decode_bf16=9)).dispatch_qwen2_gqa_decode(*gqa_tensors("bfloat16", 8), kv_len=8,
                                                                             stream_ptr=0)


@pytest.mark.parametrize("tactic,dtype,symbol", [
    ("qwen2_gqa_decode_gfx950_bf16_graph_v1", "bfloat16", "kudacuda_qwen2_gqa_decode_graph_bf16"),
    ("qwen2_gqa_decode_gfx950_fp16_graph_v1", "float16", "kudacuda_qwen2_gqa_decode_graph"),
])
def test_gqa_graph_passes_capacity_and_length_pointer(tactic, dtype, symbol):
    native = FakeNative()
    b = bridge(native)
    b.dispatch_qwen2_gqa_decode_graph(*gqa_tensors(dtype, 2048), kv_capacity=2048,
                                      kv_len_device=FakeTensor(dtype="int32", shape=(1,), pointer=55),
                                      stream_ptr=77, tactic_name=tactic)
    call = native.calls[-1]
    assert call[0] == symbol and call[6:9] == (1, 1, 2048) and call[-2:] == (55, 77)


def test_gqa_workspace_passes_workspace_and_length_pointer():
    native = FakeNative()
    b = bridge(native)
    ws = FakeTensor(dtype="float32", shape=(16 * 8 * 130,), pointer=66)
    b.dispatch_qwen2_gqa_decode_workspace(*gqa_tensors("float16", 512), kv_capacity=512,
                                          kv_len_device=FakeTensor(dtype="int32", shape=(1,), pointer=55),
                                          workspace=ws, stream_ptr=77)
    call = native.calls[-1]
    assert call[0] == "kudacuda_qwen2_gqa_decode_workspace_v3"
    assert call[6:8] == (66, 55) and call[-1] == 77
    with pytest.raises(ValueError, match="512"):
        b.dispatch_qwen2_gqa_decode_workspace(*gqa_tensors("float16", 256), kv_capacity=256,
                                              kv_len_device=FakeTensor(dtype="int32", shape=(1,)), workspace=ws,
                                              stream_ptr=0)
    with pytest.raises(ValueError, match="at least"):
        b.dispatch_qwen2_gqa_decode_workspace(*gqa_tensors("float16", 512), kv_capacity=512,
                                              kv_len_device=FakeTensor(dtype="int32", shape=(1,)),
                                              workspace=FakeTensor(dtype="float32", shape=(100,)), stream_ptr=0)


def test_graph_dispatch_configuration_bounds():
    b = bridge()
    b.configure_qwen2_graph_dispatch(kv_len_device=FakeTensor(dtype="int32", shape=(1,)), kv_capacity=65536)
    assert b._graph_kv_capacity == 65536
    with pytest.raises(ValueError, match="kv_capacity"):
        b.configure_qwen2_graph_dispatch(kv_len_device=FakeTensor(dtype="int32", shape=(1,)), kv_capacity=0)
    b.clear_qwen2_graph_dispatch()
    assert b._graph_kv_capacity is None


# ------------------------------------------------------------------ NF4 QKV
@pytest.mark.parametrize("tactic,dtype,symbol,workspace", [
    ("qwen2_fused_rmsnorm_qkv_gfx950_bf16_nf4_v1", "bfloat16", "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_bf16", False),
    ("qwen2_fused_rmsnorm_qkv_gfx950_nf4_v1", "float16", "kudacuda_qwen2_fused_rmsnorm_qkv_nf4", False),
    ("qwen2_fused_rmsnorm_qkv_gfx950_nf4_v2", "float16", "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v2", True),
    ("qwen2_fused_rmsnorm_qkv_gfx950_nf4_v3", "float16", "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v3", True),
])
def test_fused_qkv_argument_order(tactic, dtype, symbol, workspace):
    native = FakeNative()
    b = bridge(native)
    kwargs = {}
    if workspace:
        kwargs["normalized_workspace"] = FakeTensor(dtype="float32", shape=(1, 2048), pointer=71)
    b.dispatch_qwen2_fused_rmsnorm_qkv_nf4(*qkv_tensors(dtype), epsilon=1e-5, stream_ptr=77, tactic_name=tactic,
                                           **kwargs)
    call = native.calls[-1]
    assert call[0] == symbol
    pointers = (HANDLE, 11, 22, 31, 32, 33, 41, 42, 43, 51, 52, 53) + ((71,) if workspace else ()) + (61, 62, 63)
    n = len(pointers)
    assert call[1:1 + n] == pointers
    assert call[1 + n:1 + n + 5] == (1, 2048, 2048, 256, 64)
    assert call[1 + n + 5] == pytest.approx(1e-5)
    assert call[-1] == 77


def test_fused_qkv_rejects_nested_blocksize_dtype_and_missing_workspace():
    b = bridge()
    with pytest.raises(ValueError, match="nested"):
        b.dispatch_qwen2_fused_rmsnorm_qkv_nf4(*qkv_tensors(nested=True), stream_ptr=0)
    with pytest.raises(ValueError, match="blocksize"):
        b.dispatch_qwen2_fused_rmsnorm_qkv_nf4(*qkv_tensors(blocksize=128), stream_ptr=0)
    with pytest.raises(ValueError, match="bfloat16"):
        b.dispatch_qwen2_fused_rmsnorm_qkv_nf4(*qkv_tensors("float16"), stream_ptr=0)
    with pytest.raises(ValueError, match="normalized_workspace"):
        b.dispatch_qwen2_fused_rmsnorm_qkv_nf4_v2(*qkv_tensors("float16"), normalized_workspace=None, stream_ptr=0)
    man = copy.deepcopy(manifest())
    man["experimental_tactics"] = []
    man["implemented_tactics"].remove("qwen2_fused_rmsnorm_qkv_gfx950_bf16_nf4_v1")
    with pytest.raises(S.NativeCudaError, match="not enabled"):
        bridge(man=man).dispatch_qwen2_fused_rmsnorm_qkv_nf4(*qkv_tensors(), stream_ptr=0)


# ------------------------------------------------------------------ MLP
def test_swiglu_fp16_and_bf16_marshalling():
    native = FakeNative()
    b = bridge(native)
    b.dispatch_qwen2_swiglu_nf4(*swiglu_tensors("float16"), epsilon=1e-5, stream_ptr=77)
    call = native.calls[-1]
    assert call[0] == "kudacuda_qwen2_swiglu_nf4"
    assert call[1:9] == (HANDLE, 111, 122, 131, 132, 141, 142, 151)
    assert call[9:13] == (1, 2048, 11008, 64) and call[14] == 77
    with pytest.raises(ValueError, match="bfloat16"):
        b.dispatch_qwen2_swiglu_nf4_bf16(*swiglu_tensors("float16"), stream_ptr=77)
    b.dispatch_qwen2_swiglu_nf4_bf16(*swiglu_tensors("bfloat16"), epsilon=1e-6, stream_ptr=77)
    assert native.calls[-1][0] == "kudacuda_qwen2_swiglu_nf4_bf16"
    assert b.native_swiglu_dispatches == 2 and b.native_swiglu_bf16_dispatches == 1


def test_mlp_gemv_and_lm_head_marshalling():
    native = FakeNative()
    b = bridge(native)
    gw, ga = nf4(11008, 2048, 131)
    uw, ua = nf4(11008, 2048, 141)
    dw, da = nf4(2048, 11008, 161)
    bf = lambda shape, p: FakeTensor(dtype="bfloat16", shape=shape, pointer=p)  # noqa: E731
    b.dispatch_qwen2_mlp_nf4_bf16(bf((1, 2048), 111), bf((2048,), 122), gw, ga, uw, ua, dw, da, bf((1, 11008), 171),
                                  bf((1, 2048), 181), residual=bf((1, 2048), 191), stream_ptr=77)
    call = native.calls[-1]
    assert call[0] == "kudacuda_qwen2_mlp_nf4_bf16"
    assert call[1:13] == (HANDLE, 111, 122, 131, 132, 141, 142, 161, 162, 171, 191, 181)
    assert call[13:17] == (1, 2048, 11008, 64) and call[-1] == 77
    ow, oa = nf4(512, 2048, 201)
    b.dispatch_nf4_gemv_bf16(bf((1, 2048), 111), ow, oa, bf((1, 512), 211), stream_ptr=78)
    assert native.calls[-1] == ("kudacuda_nf4_gemv_bf16", HANDLE, 111, 201, 202, 0, 0, 211, 1, 2048, 512, 64, 78)
    b.lm_head_argmax_bf16(bf((1, 2048), 111), bf((2048,), 122), bf((1000, 2048), 221),
                          FakeTensor(dtype="int32", shape=(1,), pointer=231), stream_ptr=79)
    call = native.calls[-1]
    assert call[0] == "kudacuda_lm_head_argmax_bf16"
    assert call[1:9] == (HANDLE, 111, 122, 221, 0, 231, 1000, 2048) and call[-1] == 79


def test_validate_nf4_weight_layout():
    w, a = nf4(256, 2048, 41)
    assert S.KudaCudaBridge._validate_nf4_weight(w, a, expected_shape=(256, 2048), label="w") == 64
    with pytest.raises(ValueError, match="logical shape"):
        S.KudaCudaBridge._validate_nf4_weight(w, a, expected_shape=(2048, 2048), label="w")
    with pytest.raises(ValueError, match="quant_state"):
        S.KudaCudaBridge._validate_nf4_weight(FakeTensor(dtype="uint8", shape=(10, 1)), a,
                                              expected_shape=(256, 2048), label="w")
    w.quant_state.quant_type = "fp4"
    with pytest.raises(ValueError, match="nf4"):
        S.KudaCudaBridge._validate_nf4_weight(w, a, expected_shape=(256, 2048), label="w")


# ------------------------------------------------------------------ graphs and lifetime
def test_graph_lifecycle_and_shutdown():
    native = FakeNative()
    b = bridge(native)
    b.begin_capture(stream_ptr=5)
    b.end_capture(stream_ptr=5)
    b.replay_graph(stream_ptr=5)
    b.reset_graph()
    names = [c[0] for c in native.calls[-4:]]
    assert names == ["kudacuda_begin_capture", "kudacuda_end_capture", "kudacuda_replay_graph",
                     "kudacuda_reset_graph"]
    assert native.calls[-1] == ("kudacuda_reset_graph", HANDLE)
    with pytest.raises(S.NativeCudaError, match="kudacuda_replay_graph failed"):
        bridge(FakeNative(replay_graph=1)).replay_graph(stream_ptr=0)
    b.shutdown()
    assert native.calls[-1] == ("kudacuda_destroy", HANDLE)
    with pytest.raises(S.NativeCudaError, match="closed"):
        b.vector_add(FakeTensor(), FakeTensor(), FakeTensor(), stream_ptr=0)
    assert not b.matches_contract("vector_add", 1, 4)
