"""Builds libkiv_hip.so (the C-ABI of include/kiv_hip.h) for gfx950, in-tree.

    python -m kiv_amd.build

Each .hip file is compiled to an object in parallel, then linked into
kiv_amd/_lib/libkiv_hip.so.  Packed fp32 VALU ops are disabled for the device
code (the host pass prints a harmless "not a recognized feature" warning for
that flag, which is filtered from the log).
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "_lib"
LIB = LIBDIR / "libkiv_hip.so"
SOURCES = ("kiv_store.hip", "kiv_retrieve.hip", "kiv_attention.hip", "kiv_prefill.hip", "kiv_probe.hip")
# Per-source flags.  The prefill attention keeps its MFMA accumulators in
# ordinary VGPRs (the softmax rescales them every few tiles; in AGPRs every
# tile would pay a copy in and out).
EXTRA = {"kiv_prefill.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"]}
ARCH = os.environ.get("KIV_OFFLOAD_ARCH", "gfx950")

COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP library cannot be built")


def _run(cmd: list[str]) -> str:
    res = subprocess.run(cmd, capture_output=True, text=True)
    log = "\n".join(
        line for line in (res.stdout + res.stderr).splitlines()
        if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"command failed ({res.returncode}): {' '.join(cmd)}\n{log}")
    return log


def build(verbose: bool = False) -> Path:
    """Compile every .hip source and link the shared library; returns its path."""
    hipcc = _hipcc()
    objdir = LIBDIR / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    jobs = []
    for name in SOURCES:
        obj = objdir / (name + ".o")
        jobs.append((obj, [hipcc, *COMMON, *EXTRA.get(name, []), "-c", str(CSRC / name), "-o", str(obj)]))
    with cf.ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as ex:
        logs = list(ex.map(lambda j: _run(j[1]), jobs))
    tmp = LIB.with_suffix(".so.tmp")
    logs.append(_run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC",
                      *[str(o) for o, _ in jobs], "-o", str(tmp)]))
    os.replace(tmp, LIB)
    if verbose:
        for log in logs:
            if log.strip():
                print(log, file=sys.stderr)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
