"""Build the native smoke tests of the module registry.

    python tests/native/build.py

* registry_probe.hsaco: a gfx950 code object (`hipcc --genco`) that the
  registry loads at run time, and registry_probe_ccob.hsaco, the same as a
  compressed offload bundle (`--offload-compress`);
* registry_smoke: a host program linked against kudacuda_amd/libkudacuda.so
  (rpath relative to this folder) that drives include/kudacuda_registry.h;
* split_plan_check: a host program over the split-KV plan helpers of
  kudacuda_amd/csrc/kc_kernels.h.

All are built here on the CPU and run by tests/test_registry.py and
tests/test_split_plan.py.
"""

from __future__ import annotations

import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))

from kudacuda_amd import build as native_build  # noqa: E402

PROBE = HERE / "registry_probe.hsaco"
PROBE_COMPRESSED = HERE / "registry_probe_ccob.hsaco"
SMOKE = HERE / "registry_smoke"
SPLIT_PLAN = HERE / "split_plan_check"


def build() -> tuple[Path, ...]:
    hipcc = native_build._hipcc()
    subprocess.run([hipcc, *native_build.HIPCC_FLAGS, "--genco", str(HERE / "registry_probe.hip"), "-o", str(PROBE)],
                   check=True, capture_output=True, text=True)
    # the same code object as a compressed offload bundle (CCOB)
    subprocess.run([hipcc, *native_build.HIPCC_FLAGS, "--genco", "--offload-compress",
                    str(HERE / "registry_probe.hip"), "-o", str(PROBE_COMPRESSED)],
                   check=True, capture_output=True, text=True)
    lib_dir = native_build.LIBRARY.parent
    subprocess.run([hipcc, "-O2", "-std=c++17", "-Wall", str(HERE / "registry_smoke.cpp"), "-o", str(SMOKE),
                    f"-L{lib_dir}", "-lkudacuda", f"-Wl,-rpath,$ORIGIN/../../{lib_dir.name}"],
                   check=True, capture_output=True, text=True)
    # host-only program over the split-plan helpers of kc_kernels.h
    subprocess.run([hipcc, "-O2", "-std=c++17", "-Wall", str(HERE / "split_plan_check.cpp"), "-o", str(SPLIT_PLAN)],
                   check=True, capture_output=True, text=True)
    return PROBE, PROBE_COMPRESSED, SMOKE, SPLIT_PLAN


if __name__ == "__main__":
    for path in build():
        print(path)
