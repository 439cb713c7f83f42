"""NF4 parameter loader on the CPU: double-quantised absmax flattening and
bitsandbytes-layout adoption (kudacuda_amd.nf4_params)."""

from __future__ import annotations

from types import SimpleNamespace

import numpy as np
import pytest

from kudacuda_amd import nf4_params as P

torch = pytest.importorskip("torch")


def test_denest_applies_code_scale_and_offset():
    rng = np.random.default_rng(0)
    n = 1000
    codes = torch.from_numpy(rng.integers(0, 256, size=n).astype(np.uint8))
    code_map = torch.linspace(-1, 1, 256)
    scales = torch.from_numpy(rng.uniform(0.1, 2.0, size=(n + 255) // 256).astype(np.float32))
    state = SimpleNamespace(absmax=codes, shape=(250, 256), blocksize=64, quant_type="nf4", nested=True,
                            offset=torch.tensor(0.25), state2=SimpleNamespace(absmax=scales, code=code_map,
                                                                              blocksize=256))
    flat = P.denest(torch, state)
    want = code_map[codes.long()] * scales[torch.arange(n) // 256] + 0.25
    assert not flat.nested and flat.absmax.dtype == torch.float32
    assert torch.equal(flat.absmax, want)
    plain = P.Nf4QuantState(absmax=torch.ones(4), shape=(4, 64))
    assert P.denest(torch, plain) is plain


def test_adopt_params4bit_checks_format_and_reshapes():
    state = P.Nf4QuantState(absmax=torch.ones(8 * 64 // 64), shape=(8, 64))
    param = SimpleNamespace(data=torch.zeros(8 * 64 // 2, dtype=torch.uint8), quant_state=state)
    out = P.adopt_params4bit(torch, param)
    assert tuple(out.shape) == (256, 1) and out.quant_state.shape == (8, 64)
    with pytest.raises(ValueError, match="nf4"):
        P.adopt_params4bit(torch, SimpleNamespace(data=param.data, quant_state=P.Nf4QuantState(
            absmax=state.absmax, shape=(8, 64), quant_type="fp4")))
    with pytest.raises(ValueError, match="blocksize"):
        P.adopt_params4bit(torch, SimpleNamespace(data=param.data, quant_state=P.Nf4QuantState(
            absmax=state.absmax, shape=(8, 64), blocksize=128)))
    with pytest.raises(ValueError, match="quant_state"):
        P.adopt_params4bit(torch, SimpleNamespace(data=param.data))
