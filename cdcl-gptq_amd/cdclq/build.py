"""Builds libcdclq_hip.so (gfx950) in-tree from cdcl-gptq_amd/csrc with hipcc.

Each translation unit compiles in its own hipcc process (in parallel), then one link step.
Flags that the engine's bit-exactness depends on:
  -ffp-contract=off   no implicit a*b+c fusion anywhere (fused ops are explicit fma calls)
  -Xclang -target-feature -Xclang -packed-fp32-ops   keep packed-FP32 VALU forms out of the code
hipcc's default correctly-rounded f32 division/sqrt and IEEE denormal handling are kept.
For speed: -mllvm -amdgpu-mfma-vgpr-form keeps MFMA accumulators in ordinary VGPRs (the same
instructions in their VGPR form), so loop-carried accumulators are not copied between AGPRs and
VGPRs around every LDS stage.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
REPO = os.path.dirname(ROOT)
CSRC = os.path.join(ROOT, "csrc")
INCLUDE = os.path.join(REPO, "include")
OBJDIR = os.path.join(ROOT, "_build")
LIB = os.path.join(PKG, "libcdclq_hip.so")
ARCH = os.environ.get("CDCLQ_ARCH", "gfx950")

SOURCES = ["k_gemm.hip", "k_gemm_wide.hip", "k_gram.hip", "k_factor.hip", "k_engine.hip", "k_repair.hip", "k_pack.hip", "k_eval.hip",
           "engine.cpp", "container.cpp", "harness.cpp", "pipeline.cpp"]
COMMON = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function", "-Wno-unknown-pragmas",
    "-I", INCLUDE, "-I", CSRC,
]


def hipcc() -> str:
    for cand in (shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libcdclq_hip.so)")


def _compile(src: str) -> str:
    obj = os.path.join(OBJDIR, os.path.basename(src) + ".o")
    cmd = [hipcc(), *COMMON, "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "packed-fp32-ops"  # hipcc's host pass warns about the device-only feature flag
    msg = "\n".join(line for line in (r.stdout + r.stderr).splitlines() if noise not in line)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{msg}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJDIR, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), 8)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("link failed:\n" + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build()
