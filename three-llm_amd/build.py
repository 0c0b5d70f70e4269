"""Builds libtlm.so (the HIP kernels + C ABI) in-tree for gfx950.

    python three-llm_amd/build.py

hipcc cross-compiles without a GPU.  Packed-FP32 instructions are disabled for
all device code (-packed-fp32-ops); the host pass warns that it does not know
the feature, which is harmless.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
LIB = HERE / "libtlm.so"
SOURCES = ["tlm_api.hip", "tlm_kernels.hip", "tlm_prefill.hip", "tlm_host.cpp"]
ARCH = os.environ.get("TLM_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libtlm.so)")


def build(verbose: bool = False) -> Path:
    out_tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-Wall", "-Wno-unused-result", "-Wno-unused-value", "-Wno-unused-command-line-argument",
           "-o", str(out_tmp)] + [str(CSRC / s) for s in SOURCES] + ["-lpthread"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("hipcc failed building libtlm.so")
    warnings = [l for l in (res.stdout + res.stderr).splitlines()
                if "warning" in l and "packed-fp32-ops" not in l and "target-feature" not in l]
    if verbose and warnings:
        print("\n".join(warnings))
    os.replace(out_tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
