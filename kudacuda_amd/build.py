"""Build libkudacuda.so (gfx950) in-tree with hipcc.

Every ``csrc/*.hip`` translation unit is compiled for ``--offload-arch=gfx950``
in parallel and linked into ``kudacuda_amd/libkudacuda.so``.  Floating-point
flags are part of the library's contract: no implicit FMA contraction,
correctly rounded fp32 divide/sqrt and IEEE denormals, so that every kernel
computes exactly the operation sequence its source spells out.

Usage: ``python -m kudacuda_amd.build`` (or ``build()`` from Python).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIBRARY = PACKAGE_DIR / "libkudacuda.so"
OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-result",
]


# Kernel-argument preload: the first scalar/pointer arguments of a kernel are
# loaded into SGPRs as its waves launch, before the first instruction, instead
# of by the wave's own scalar loads from the argument buffer.  The decode
# step's kernels take the pointers their first loads need as leading scalar
# arguments; measured on the down projection alone, the decode step went
# 1.1173 -> 1.1100 ms (36 launches, ~0.2 us each).
PRELOAD = ["-mllvm", "-amdgpu-kernarg-preload-count=6"]

# Per-source additions.  kc_prefill.hip: MFMA accumulators in VGPRs (the
# default AGPR form makes the compiler shuffle accumulators between register
# files inside the GEMM's window loop).
SOURCE_FLAGS = {
    "kc_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    **{name: PRELOAD for name in ("kc_nf4.hip", "kc_gqa.hip", "kc_lmhead.hip")},
}


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise FileNotFoundError("hipcc not found (set HIPCC or install ROCm)")


def _run(command: list[str]) -> None:
    result = subprocess.run(command, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"command failed ({result.returncode}): {' '.join(command)}\n{result.stdout}")
    if result.stdout.strip():
        # hipcc's host pass warns that it does not know the packed-fp32 feature;
        # only surface output that is not that known warning.
        lines = [line for line in result.stdout.splitlines() if "packed-fp32-ops" not in line]
        text = "\n".join(lines).strip()
        if text:
            print(text, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""

    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise FileNotFoundError(f"no HIP sources under {CSRC}")
    objects = [BUILD_DIR / (source.stem + ".o") for source in sources]

    def compile_one(pair: tuple[Path, Path]) -> None:
        source, obj = pair
        command = [hipcc, *HIPCC_FLAGS, *SOURCE_FLAGS.get(source.name, []), "-c", str(source), "-o", str(obj)]
        if verbose:
            print(" ".join(command))
        _run(command)

    workers = jobs or min(len(sources), max(1, min(os.cpu_count() or 1, 16)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(compile_one, zip(sources, objects)))
    tmp = LIBRARY.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-o", str(tmp), *map(str, objects)]
    if verbose:
        print(" ".join(link))
    _run(link)
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
