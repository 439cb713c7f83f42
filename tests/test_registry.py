"""The module registry of include/kudacuda_registry.h (reference
include/kudacuda_registry.h:10-41, runtime/kudacuda_registry.cu:33-115),
exercised by the native smoke program tests/native/registry_smoke."""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
SMOKE = HERE / "native" / "registry_smoke"
PROBE = HERE / "native" / "registry_probe.hsaco"
PROBE_COMPRESSED = HERE / "native" / "registry_probe_ccob.hsaco"
LIB = HERE.parent / "kudacuda_amd" / "libkudacuda.so"


def _built() -> None:
    if not (SMOKE.exists() and PROBE.exists() and PROBE_COMPRESSED.exists()):
        pytest.skip("native smokes not built (python tests/native/build.py)")


@pytest.mark.skipif(shutil.which("nm") is None, reason="binutils nm not available")
def test_library_exports_the_registry_class():
    out = subprocess.run(["nm", "-DC", "--defined-only", str(LIB)], check=True, capture_output=True,
                         text=True).stdout
    for member in ("KudaCudaModuleRegistry::KudaCudaModuleRegistry(int)",
                   "KudaCudaModuleRegistry::~KudaCudaModuleRegistry()", "KudaCudaModuleRegistry::load(",
                   "KudaCudaModuleRegistry::resolve(", "KudaCudaModuleRegistry::freeze("):
        assert f"kudacuda::{member}" in out, member


@pytest.mark.skipif(os.path.exists("/dev/kfd"), reason="a GPU is present: the device path is tested instead")
def test_registry_without_a_device_refuses_every_call():
    _built()
    run = subprocess.run([str(SMOKE), "--no-device"], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stderr
    assert "registry smoke ok (no device)" in run.stdout


def test_compressed_probe_is_a_compressed_offload_bundle():
    """The second probe starts with the compressed-bundle magic the registry
    passes through to hipModuleLoad (and is smaller than the plain one)."""

    _built()
    assert PROBE_COMPRESSED.read_bytes()[:4] == b"CCOB"
    assert PROBE.read_bytes()[:4] != b"CCOB"


@pytest.mark.gpu
@pytest.mark.parametrize("probe", [PROBE, PROBE_COMPRESSED], ids=["plain", "compressed"])
def test_registry_loads_resolves_launches_and_freezes(probe):
    _built()
    print(f"registry smoke: {SMOKE} {probe}", flush=True)
    run = subprocess.run([str(SMOKE), str(probe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert "registry smoke ok (1000 outputs via probe_affine)" in run.stdout
