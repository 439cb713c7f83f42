"""Split-KV attention plans of kudacuda_amd/csrc/kc_kernels.h, checked
exhaustively by the host program tests/native/split_plan_check (every kv_len
up to 65536; the round path's 32-token units at caps 1..8, 32 and 256, the
matrix-core tactic's 64- and 128-token units at cap 128): whole-unit splits,
at most cap of them, every token in exactly one split, the fewest units per
split, and the grid bound the launchers size for device-side lengths."""

from __future__ import annotations

import subprocess
from pathlib import Path

import pytest

CHECK = Path(__file__).resolve().parent / "native" / "split_plan_check"


def test_split_plans_partition_every_length():
    if not CHECK.exists():
        pytest.skip("native checks not built (python tests/native/build.py)")
    run = subprocess.run([str(CHECK)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "split plan ok" in run.stdout
