"""Small helpers for GPU tests: numpy <-> device tensors and pointer args."""

from __future__ import annotations

import numpy as np


def dev(torch, array: np.ndarray, stream=None):
    """Upload a numpy array (uint16 arrays are treated as raw 16-bit bits)."""

    a = np.ascontiguousarray(array)
    if a.dtype == np.uint16:
        t = torch.from_numpy(a.view(np.int16))
    else:
        t = torch.from_numpy(a)
    return t.to("cuda:0")


def empty(torch, n: int, dtype: str):
    table = {"u16": torch.int16, "u8": torch.uint8, "f32": torch.float32, "i32": torch.int32}
    return torch.zeros(n, dtype=table[dtype], device="cuda:0")


def host(tensor) -> np.ndarray:
    import torch

    t = tensor.detach()
    if t.dtype in (torch.int16, torch.bfloat16, torch.float16):
        return t.view(torch.int16).cpu().numpy().view(np.uint16)
    return t.cpu().numpy()


def p(tensor) -> int:
    return 0 if tensor is None else int(tensor.data_ptr())
