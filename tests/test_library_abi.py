"""The C ABI: header, exported symbols and ctypes signatures agree, and the
library fails closed on a null handle (no GPU needed)."""

from __future__ import annotations

import ctypes
import re
import subprocess
from pathlib import Path

import pytest

from kudacuda_amd import _native

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "kudacuda.h"

# reference include/kudacuda.h exports (python/kudacuda_sidecar.py:260-419 binds them)
REFERENCE_SYMBOLS = {
    "kudacuda_create", "kudacuda_freeze", "kudacuda_can_dispatch", "kudacuda_vector_add", "kudacuda_rmsnorm",
    "kudacuda_fused_rmsnorm_qkv", "kudacuda_qwen2_fused_rmsnorm_qkv_nf4", "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v2",
    "kudacuda_qwen2_fused_rmsnorm_qkv_nf4_v3", "kudacuda_qwen2_swiglu_nf4", "kudacuda_qwen2_swiglu_nf4_bf16",
    "kudacuda_qwen2_gqa_decode_workspace_v3", "kudacuda_qwen2_gqa_decode", "kudacuda_qwen2_gqa_decode_graph",
    "kudacuda_qwen2_gqa_decode_group_tiled", "kudacuda_qwen2_gqa_decode_vectorized", "kudacuda_begin_capture",
    "kudacuda_end_capture", "kudacuda_replay_graph", "kudacuda_reset_graph", "kudacuda_last_error",
    "kudacuda_destroy",
}


def header_symbols() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"KUDACUDA_API\s+[\w\s\*]*?\b(kudacuda_\w+)\s*\(", text))


def test_header_declares_every_reference_symbol():
    names = header_symbols()
    assert REFERENCE_SYMBOLS <= names
    assert len(REFERENCE_SYMBOLS) == 22


def test_ctypes_table_covers_exactly_the_header():
    assert set(_native.SIGNATURES) == header_symbols()


@pytest.fixture(scope="module")
def lib():
    if not _native.DEFAULT_LIBRARY.exists():
        pytest.skip("libkudacuda.so not built")
    return _native.load_library()


def test_library_exports_every_declared_symbol(lib):
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.DEFAULT_LIBRARY)], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if line.strip()}
    missing = header_symbols() - exported
    assert not missing, missing
    for name in header_symbols():
        assert getattr(lib, name) is not None


def test_null_handle_fails_closed(lib):
    assert lib.kudacuda_last_error(None) == b"invalid KudaCuda handle"
    assert lib.kudacuda_freeze(None) == 1
    assert lib.kudacuda_can_dispatch(None, b"rmsnorm", 1, 1) == 0
    assert lib.kudacuda_vector_add(None, 1, 2, 3, 4, 0) == 1
    assert lib.kudacuda_rmsnorm(None, 1, 2, 3, 1, 4, 1e-5, 0) == 1
    assert lib.kudacuda_qwen2_gqa_decode(None, 1, 2, 3, 4, 1, 1, 8, 16, 2, 128, 0.08, 0) == 1
    assert lib.kudacuda_begin_capture(None, 0) == 1
    assert lib.kudacuda_reset_graph(None) == 1
    lib.kudacuda_destroy(None)


def test_workspace_size_helpers(lib):
    assert lib.kudacuda_gqa_split_chunk(2048) == 32 and lib.kudacuda_gqa_split_chunk(32768) == 128
    floats = lib.kudacuda_gqa_workspace_floats(2048)
    assert floats >= 16 * 8 * 130
    assert lib.kudacuda_lm_head_workspace_floats() >= 2
