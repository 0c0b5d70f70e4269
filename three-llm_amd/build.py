"""Builds libtlm.so (the HIP kernels + C ABI) in-tree for gfx950.

    python three-llm_amd/build.py

Each source compiles to an object under three-llm_amd/_build/ (in parallel),
then the objects link into libtlm.so.  hipcc cross-compiles without a GPU.  Packed-FP32 instructions are disabled for
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
OBJ = HERE / "_build"
SOURCES = ["tlm_api.hip", "tlm_kernels.hip", "tlm_gqa.hip", "tlm_prefill.hip", "tlm_ps.hip", "tlm_host.cpp"]
ARCH = os.environ.get("TLM_OFFLOAD_ARCH", "gfx950")


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build libtlm.so)")


def _flags():
    return ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wall", "-Wno-unused-result", "-Wno-unused-value", "-Wno-unused-command-line-argument"]


def build(verbose: bool = False) -> Path:
    """Compiles every source to an object in parallel, then links libtlm.so."""
    OBJ.mkdir(exist_ok=True)
    procs = []
    for src in SOURCES:
        obj = OBJ / (src + ".o")
        cmd = [hipcc()] + _flags() + ["-c", "-o", str(obj), str(CSRC / src)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((src, obj, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
    failed = False
    for src, obj, pr in procs:
        out, _ = pr.communicate()
        if pr.returncode != 0:
            sys.stderr.write(out)
            failed = True
        elif verbose:
            warnings = [l for l in out.splitlines()
                        if "warning:" in l and "packed-fp32-ops" not in l and "target-feature" not in l
                        and "reserved registers" not in l]
            if warnings:
                print("\n".join(warnings))
    if failed:
        raise RuntimeError("hipcc failed building libtlm.so")
    out_tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(out_tmp)] + \
          [str(OBJ / (s + ".o")) for s in SOURCES] + ["-lpthread"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError("linking libtlm.so failed")
    os.replace(out_tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
