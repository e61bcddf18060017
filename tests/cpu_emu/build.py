"""Bounds-checked CPU build of libtomoul_hip (test infrastructure).

    python tests/cpu_emu/build.py        # -> tests/cpu_emu/_build/emu

Every translation unit of the library (tomoul_amd/build.py SOURCES) is
compiled for the host with clang++ under AddressSanitizer and UBSan, with
tests/cpu_emu/hip/hip_runtime.h standing in for the HIP runtime and the
gfx950 builtins.  The only change made to the sources is mechanical: each
triple-chevron launch `K<<<grid, block, shmem, stream>>>(args)` becomes
`tml_emu_launch(K, grid, block, shmem, stream)(args)`, which runs the kernel
body for every (block, thread) of the grid on the CPU.  emu_main.cpp drives
the library's C ABI with operands allocated at exactly the sizes the
entry points document (see hip_runtime.h for what is and is not emulated).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
CSRC = os.path.join(ROOT, "tomoul_amd", "csrc")
OUT_DIR = os.path.join(HERE, "_build")
EXE = os.path.join(OUT_DIR, "emu")
CLANG = "/opt/rocm/llvm/bin/clang++"
FLAGS = ["-std=c++17", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
         "-fno-sanitize-recover=all", "-Wno-unused-function", "-Wno-unused-variable",
         "-I", HERE, "-I", CSRC, "-I", os.path.join(ROOT, "include"),
         # forced planner overrides at every size (the shipped library refuses
         # them above the sizes its GPU tests run them at)
         "-DTML_FORCED_PLAN_MAX_MNK=0xFFFFFFFFFFFFFFFFull"]

sys.path.insert(0, ROOT)


def sources() -> list[str]:
    from tomoul_amd import build as b
    return list(b.SOURCES)


def _kernel_start(text: str, end: int) -> int:
    """Start of the kernel expression that ends just before text[end]."""
    i = end - 1
    while i >= 0 and text[i].isspace():
        i -= 1
    if text[i] == ">":  # template-id: match the angle brackets backwards,
        depth = 0       # skipping parenthesised template arguments whole
        while i >= 0:
            if text[i] == ")":
                par = 0
                while i >= 0:
                    par += text[i] == ")"
                    par -= text[i] == "("
                    if par == 0:
                        break
                    i -= 1
            elif text[i] == ">":
                depth += 1
            elif text[i] == "<":
                depth -= 1
                if depth == 0:
                    break
            i -= 1
        i -= 1
    while i >= 0 and (text[i].isalnum() or text[i] in "_:"):
        i -= 1
    return i + 1


def transform(text: str) -> str:
    """K<<<g, b, shm, s>>>(args)  ->  tml_emu_launch(K, g, b, shm, s)(args)."""
    out = []
    pos = 0
    for m in re.finditer(r"<<<", text):
        if m.start() < pos:
            continue
        close = text.index(">>>", m.end())
        start = _kernel_start(text, m.start())
        out.append(text[pos:start])
        out.append("tml_emu_launch(" + text[start:m.start()].strip() + ", " + text[m.end():close] + ")")
        pos = close + 3
    out.append(text[pos:])
    return "".join(out)


# The GEMM kernels run over the largest grids, so they are optimised (about
# 100 s to compile each, 16x faster to run); the rest compiles at -O0 (the
# GEMV translation units take 3-7 minutes at -O1).
OPTIMISED = {"gemm_dma", "gemm_mfma", "emu_main"}


def _deps() -> list[str]:
    return [os.path.join(HERE, "hip", "hip_runtime.h"), os.path.join(CSRC, "tml_internal.hpp"),
            os.path.join(CSRC, "host_copier.hpp"), os.path.join(ROOT, "include", "tomoul_hip.h"),
            os.path.abspath(__file__)]


def _stale(out: str, inputs: list[str]) -> bool:
    if not os.path.exists(out):
        return True
    t = os.path.getmtime(out)
    return any(os.path.getmtime(i) > t for i in inputs)


def _compile(src: str, out: str, orig: str) -> str:
    if not _stale(out, [orig, *_deps()]):
        return out
    opt = "-O1" if os.path.splitext(os.path.basename(src))[0] in OPTIMISED else "-O0"
    res = subprocess.run([CLANG, *FLAGS, opt, "-c", src, "-o", out], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"clang++ failed for {src}:\n{res.stderr[-6000:]}")
    return out


def build(verbose: bool = False) -> str:
    os.makedirs(OUT_DIR, exist_ok=True)
    jobs = []
    for s in sources():
        with open(os.path.join(CSRC, s)) as f:
            text = transform(f.read())
        cpp = os.path.join(OUT_DIR, os.path.splitext(s)[0] + ".cpp")
        new = f'#line 1 "{os.path.join(CSRC, s)}"\n' + text
        if not os.path.exists(cpp) or open(cpp).read() != new:
            with open(cpp, "w") as f:
                f.write(new)
        jobs.append((cpp, cpp[:-4] + ".o", os.path.join(CSRC, s)))
    main = os.path.join(HERE, "emu_main.cpp")
    jobs.append((main, os.path.join(OUT_DIR, "emu_main.o"), main))
    with cf.ThreadPoolExecutor(max_workers=min(8, os.cpu_count() or 1)) as ex:
        objs = list(ex.map(lambda j: _compile(*j), jobs))
    if not _stale(EXE, objs):
        return EXE
    res = subprocess.run([CLANG, "-fsanitize=address,undefined", *objs, "-o", EXE], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr[-4000:]}")
    if verbose:
        print(f"built {EXE}")
    return EXE


if __name__ == "__main__":
    build(verbose=True)
