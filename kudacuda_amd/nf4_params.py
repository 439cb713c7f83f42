"""NF4 weights in the bitsandbytes ``Params4bit`` layout on PyTorch-ROCm.

The bridge's NF4 entry points take what bitsandbytes keeps for a 4-bit linear
layer (reference python/kudacuda_sidecar.py:1018-1049): packed uint8 storage
of shape (N*K/2, 1) whose ``quant_state`` carries the fp32 absmax [N*K/64],
the logical shape (N, K), blocksize 64 and quant_type "nf4".  bitsandbytes
is not a dependency here, so this module provides that layout itself:

* ``quantize_weight`` -- NF4-quantise a dense [N, K] weight on the GPU
  (``kudacuda_nf4_quantize``) into packed storage with a ``quant_state``;
* ``denest`` -- turn a double-quantised state (uint8 absmax codes of a
  256-entry dynamic map, per-256-block scales and an offset, as bitsandbytes
  stores ``compress_statistics=True``) into the plain fp32 absmax the kernels
  read;
* ``adopt_params4bit`` -- take an existing bitsandbytes-style parameter
  (packed data + quant_state, nested or not) as is;
* ``make_nf4_linear`` / ``quantize_qwen2_model`` -- a drop-in ``nn.Linear``
  replacement holding such a weight (framework path: GPU dequantise then
  ``F.linear``), and a helper that converts a Transformers Qwen2 model's
  projections, leaving norms, embeddings and lm_head in bf16.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Optional

BLOCKSIZE = 64


@dataclass
class Nf4QuantState:
    """The fields of a bitsandbytes QuantState that NF4 consumers read."""

    absmax: Any
    shape: tuple[int, int]
    blocksize: int = BLOCKSIZE
    quant_type: str = "nf4"
    nested: bool = False
    dtype: Any = None
    offset: Any = None
    state2: Any = None
    extra: dict[str, Any] = field(default_factory=dict)


@dataclass
class DynamicMapState:
    """Second-level state of a double-quantised absmax (bitsandbytes ``state2``)."""

    absmax: Any      # fp32 [ceil(n / blocksize)]
    code: Any        # fp32 [256] dynamic quantisation map
    blocksize: int = 256


def _stream_ptr(torch: Any, stream: Any, device: Any) -> int:
    s = stream if stream is not None else torch.cuda.current_stream(device)
    return int(s.cuda_stream)


def quantize_weight(native: Any, torch: Any, weight: Any, *, stream: Any = None) -> Any:
    """Packed uint8 (N*K/2, 1) device tensor with ``quant_state`` for a dense
    [N, K] weight (any float dtype; quantised from its fp32 value)."""

    if weight.dim() != 2:
        raise ValueError("quantize_weight expects a rank-2 [out, in] weight")
    rows, cols = (int(s) for s in weight.shape)
    count = rows * cols
    if count % BLOCKSIZE != 0:
        raise ValueError("NF4 quantisation needs out*in divisible by 64")
    device = weight.device
    src = weight.detach().to(dtype=torch.float32).contiguous()
    packed = torch.empty((count // 2, 1), dtype=torch.uint8, device=device)
    absmax = torch.empty(count // BLOCKSIZE, dtype=torch.float32, device=device)
    native.call("kudacuda_nf4_quantize", src.data_ptr(), 0, count, BLOCKSIZE, packed.data_ptr(), absmax.data_ptr(),
                _stream_ptr(torch, stream, device))
    packed.quant_state = Nf4QuantState(absmax=absmax, shape=(rows, cols), dtype=weight.dtype)
    return packed


def denest(torch: Any, state: Any) -> Nf4QuantState:
    """fp32 absmax of a double-quantised state: code[u8] * scale[i / 256] + offset."""

    if not bool(getattr(state, "nested", False)):
        return state
    state2 = getattr(state, "state2", None)
    if state2 is None:
        raise ValueError("nested quant_state has no state2")
    codes = state.absmax.long()
    block = int(getattr(state2, "blocksize", 256))
    index = torch.arange(codes.numel(), device=codes.device) // block
    absmax = state2.code.float()[codes] * state2.absmax.float()[index]
    offset = getattr(state, "offset", None)
    if offset is not None:
        absmax = absmax + offset
    return Nf4QuantState(absmax=absmax.contiguous(), shape=tuple(int(s) for s in state.shape),
                         blocksize=int(state.blocksize), quant_type=str(state.quant_type), nested=False,
                         dtype=getattr(state, "dtype", None))


def adopt_params4bit(torch: Any, param: Any) -> Any:
    """Accept a bitsandbytes-style 4-bit parameter: packed uint8 data with a
    ``quant_state``.  Nested states are flattened; other fields are checked."""

    state = getattr(param, "quant_state", None)
    if state is None:
        raise ValueError("parameter has no quant_state")
    if str(getattr(state, "quant_type", "")) != "nf4":
        raise ValueError("only nf4 quantisation is supported")
    if int(getattr(state, "blocksize", 0)) != BLOCKSIZE:
        raise ValueError("only blocksize 64 is supported")
    data = getattr(param, "data", param).contiguous()
    rows, cols = (int(s) for s in state.shape)
    data = data.view(torch.uint8).reshape((rows * cols + 1) // 2, 1)
    data.quant_state = denest(torch, state)
    return data


def dequantize(native: Any, torch: Any, packed: Any, *, dtype: Any = None, stream: Any = None) -> Any:
    """Dense [N, K] tensor (bf16, fp16 or fp32) of an NF4 weight, on the GPU."""

    state = packed.quant_state
    rows, cols = state.shape
    dtype = dtype or state.dtype or torch.bfloat16
    kind = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}[dtype]
    out = torch.empty((rows, cols), dtype=dtype, device=packed.device)
    native.call("kudacuda_nf4_dequantize", packed.data_ptr(), state.absmax.data_ptr(), rows * cols, state.blocksize,
                kind, out.data_ptr(), _stream_ptr(torch, stream, packed.device))
    return out


def make_nf4_linear(native: Any, torch: Any, linear: Any) -> Any:
    """An nn.Module replacing ``linear``: weight = packed NF4 (with quant_state),
    bias kept in the linear's dtype; forward dequantises on the GPU."""

    nn = torch.nn

    class Nf4Linear(nn.Module):
        def __init__(self) -> None:
            super().__init__()
            self.in_features = int(linear.in_features)
            self.out_features = int(linear.out_features)
            self.compute_dtype = linear.weight.dtype
            self.weight = quantize_weight(native, torch, linear.weight.data)
            self.bias = None if linear.bias is None else linear.bias.detach().clone()

        def forward(self, x: Any) -> Any:
            w = dequantize(native, torch, self.weight, dtype=x.dtype)
            return torch.nn.functional.linear(x, w, None if self.bias is None else self.bias.to(x.dtype))

    return Nf4Linear()


def quantize_qwen2_model(native: Any, torch: Any, model: Any,
                         names: Optional[tuple[str, ...]] = None) -> Any:
    """Replace the q/k/v/o and gate/up/down projections of every decoder layer
    with NF4 linears (bitsandbytes-style weights); returns the model."""

    attn_names = ("q_proj", "k_proj", "v_proj", "o_proj")
    mlp_names = ("gate_proj", "up_proj", "down_proj")
    wanted = set(names or attn_names + mlp_names)
    for layer in model.model.layers:
        for parent, group in ((layer.self_attn, attn_names), (layer.mlp, mlp_names)):
            for name in group:
                if name in wanted:
                    setattr(parent, name, make_nf4_linear(native, torch, getattr(parent, name)))
    torch.cuda.synchronize()
    return model
