"""Builds libmivi_hip.so (HIP kernels + C ABI) for gfx950, in-tree.

    python mivi-v4_amd/build.py            # incremental
    python mivi-v4_amd/build.py --force    # rebuild everything

Objects go to mivi-v4_amd/_build/, the library to mivi-v4_amd/mivi_hip/.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
OUT = os.path.join(HERE, "mivi_hip", "libmivi_hip.so")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HIPCC = os.path.join(ROCM, "bin", "hipcc")
ARCH = "gfx950"

# -ffp-contract=off: FMAs are written explicitly (fmaf) where wanted, so the
# bit-exact dequantization keeps the reference's separate roundings.
# -packed-fp32-ops is disabled for all device code (the host pass warns that
# it does not know the feature; that is harmless).
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-Wall"]

SOURCES = ["errors.cpp", "synth.cpp", "quant.hip", "gemm.hip", "model.hip", "sampler.hip"]

# Per-source device flags. quant.hip: MFMA results straight into VGPRs (the
# GEMV kernels consume each result at once; in AGPRs every one of them costs a
# v_accvgpr_read). The GEMM keeps the default: its accumulator tiles live in AGPRs.
EXTRA_FLAGS = {"quant.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def _deps(src: str) -> list[str]:
    return [os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith(".h")] + [
        os.path.join(HERE, "..", "include", "mivi_hip.h"), src]


def _compile(src: str, force: bool) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(BUILD, src + ".o")
    if not force and os.path.exists(obj):
        t = os.path.getmtime(obj)
        if all(os.path.getmtime(d) <= t for d in _deps(path)):
            return obj
    if src.endswith(".hip"):
        cmd = [HIPCC, *DEVICE_FLAGS, *EXTRA_FLAGS.get(src, []), "-c", path, "-o", obj]
    else:
        cmd = [HIPCC, *HOST_FLAGS, "-c", path, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError(f"compile failed: {src}")
    return obj


def build(force: bool = False) -> str:
    os.makedirs(BUILD, exist_ok=True)
    srcs = [s for s in SOURCES if os.path.exists(os.path.join(CSRC, s))]
    with cf.ThreadPoolExecutor(max_workers=min(8, len(srcs))) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), srcs))
    tmp = OUT + ".tmp"
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs, "-lpthread"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link failed")
    shutil.move(tmp, OUT)
    return OUT


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    a = ap.parse_args()
    print(build(a.force))
