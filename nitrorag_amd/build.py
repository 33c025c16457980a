"""Builds libnitro_paged_attn.so in-tree with hipcc for gfx950.

    python -m nitrorag_amd.build            # or: python nitrorag_amd/build.py

Device sources (*.hip) and the HIP-runtime host glue go through hipcc with
--offload-arch=gfx950; packed FP32 instructions are disabled for all device
code (-Xclang -target-feature -Xclang -packed-fp32-ops).  The host page
bookkeeping is plain C++17 and is compiled with g++.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OBJ = os.path.join(HERE, "_build")
INCLUDE = os.path.join(ROOT, "include")
LIB = os.path.join(HERE, "libnitro_paged_attn.so")

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("NITRO_OFFLOAD_ARCH", "gfx950")
DEVICE_SOURCES = ["paged_attn_decode.hip", "paged_attn_prefill.hip", "kv_append.hip", "q8_matmul.hip",
                  "model_kernels.hip", "scheduler_kernels.hip"]
HIP_HOST_SOURCES = ["capi_device.cpp", "model.cpp", "scheduler_step.cpp"]
HOST_SOURCES = ["paged_memory.cpp", "capi_host.cpp", "scheduler.cpp", "rpc.cpp"]

COMMON = ["-O3", "-std=c++17", "-fPIC", f"-I{INCLUDE}", f"-I{CSRC}", "-Wall"]
# Code object v5: loadable by the HIP runtime torch bundles (ROCm 7.0) as well
# as by /opt/rocm's (7.2), whichever of the two the process has loaded.
HIP_FLAGS = [f"--offload-arch={ARCH}", "-mcode-object-version=5", "-Xclang", "-target-feature",
             "-Xclang", "-packed-fp32-ops"]
# The decode kernel's first arguments (the scalars that locate a workgroup's
# block-table slice) are preloaded into SGPRs, so its first loads do not wait
# for a load of the kernel arguments.
SOURCE_FLAGS = {"paged_attn_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=10"]}


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return r


def _compile(src: str) -> str:
    path = os.path.join(CSRC, src)
    obj = os.path.join(OBJ, src + ".o")
    if src in HOST_SOURCES:
        cmd = ["g++", *COMMON, "-c", path, "-o", obj]
    elif src.endswith(".hip"):
        cmd = [HIPCC, *COMMON, *HIP_FLAGS, *SOURCE_FLAGS.get(src, []), "-x", "hip", "-c", path, "-o", obj]
    else:
        cmd = [HIPCC, *COMMON, *HIP_FLAGS, "-c", path, "-o", obj]
    _run(cmd)
    return obj


def build(verbose: bool = True) -> str:
    """Compiles every source and links the shared library; returns its path."""
    if not os.path.exists(HIPCC):
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    os.makedirs(OBJ, exist_ok=True)
    sources = DEVICE_SOURCES + HIP_HOST_SOURCES + HOST_SOURCES
    with cf.ThreadPoolExecutor(max_workers=min(len(sources), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(_compile, sources))
    tmp = LIB + ".tmp"
    _run([HIPCC, "-shared", f"--offload-arch={ARCH}", "-mcode-object-version=5", "-fPIC", "-o", tmp,
          *objs])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


def clean() -> None:
    shutil.rmtree(OBJ, ignore_errors=True)
    if os.path.exists(LIB):
        os.remove(LIB)


if __name__ == "__main__":
    if "--clean" in sys.argv:
        clean()
    build()
