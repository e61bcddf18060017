"""Builds libtomoul_hip.so (the gfx950 kernels + C ABI) in-tree with hipcc.

    python -m tomoul_amd.build            # or tomoul_amd.build.build()

The library lands next to this file (tomoul_amd/libtomoul_hip.so) so that it
travels with the source tree; nothing is installed.  Translation units are
compiled in parallel and linked into one shared object.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OUT = os.path.join(HERE, "libtomoul_hip.so")
SOURCES = ["runtime.hip", "gemm_mfma.hip", "gemm_dma.hip", "gemm_qbf.hip", "gemv.hip", "gemv_t.hip", "gemv_tm.hip", "quantize.hip", "tl.hip",
           "stream_read.hip", "gemv_x.hip"]
ARCH = os.environ.get("TML_OFFLOAD_ARCH", "gfx950")

# -packed-fp32-ops off: hipcc may otherwise emit v_pk_* fp32 instructions
# on its own from scalar float code.  Shadowed names are errors: a lambda
# parameter named like the enclosing function's row offset once computed
# silently wrong rows (-Wshadow-all is the clang group that covers lambda
# parameters; plain -Wshadow does not).
HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wshadow-all", "-Werror=shadow-all",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP backend cannot be built")


# Per-source flags.  gemm_qbf.hip: keep MFMA accumulators in ordinary VGPRs
# (the compiler otherwise splits them over the accumulation registers and
# copies them back and forth inside the K loop: 72 extra moves a loop trip).
SOURCE_FLAGS = {"gemm_qbf.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"]}


def _compile(src: str, obj_dir: str) -> str:
    obj = os.path.join(obj_dir, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = False) -> str:
    obj_dir = os.path.join(HERE, "_build")
    os.makedirs(obj_dir, exist_ok=True)
    with cf.ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir), SOURCES))
    tmp = OUT + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, OUT)
    if verbose:
        print(f"built {OUT}")
    return OUT


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
