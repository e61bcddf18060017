"""Bounds-checked CPU build of the whole library (tests/cpu_emu/).

Every translation unit of libtomoul_hip -- C ABI, planners, kernels, .tl
reader -- compiled for the host under AddressSanitizer and UBSan, kernels
run thread by thread on the CPU with their real index arithmetic (see
tests/cpu_emu/hip/hip_runtime.h).  Each case calls an entry point with
operands allocated at exactly the sizes it documents; any access outside an
allocation, any buffer resource larger than its allocation, any signed
overflow or other undefined behaviour aborts the case.

* test_planted_mistakes: a B operand 16 bytes short must be reported for
  every kernel family (the harness itself works);
* test_cases: every kernel family, tile config (TML_GEMM_DMA_TILE 1-11,
  TML_GEMM_TILE 1-10, TML_GEMM_QBF_TILE 1-11), K split (1, 2, 3, 4, 8),
  format, epilogue and the fused split-K exchange, on shapes with ragged
  edges in M, N and K;
* test_fault_sweep_replay (TML_EMU_FULL=1): every (format, shape, forced
  plan) of the narrow-format calibration sweep that once ended in a GPU
  memory fault, at its full sizes (946 cases, about 3 minutes on 8 cores).

CPU only; needs /opt/rocm/llvm/bin/clang++ (skipped without it).
"""
import concurrent.futures as cf
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CLANG = "/opt/rocm/llvm/bin/clang++"
F32, Q8_0, Q4_0, Q8_K, F16, Q8_0_PC, Q4_0_PC = 0, 1, 2, 3, 4, 17, 18

pytestmark = pytest.mark.skipif(not os.path.exists(CLANG), reason="no clang++ for the CPU build")


@pytest.fixture(scope="module")
def emu():
    import sys
    sys.path.insert(0, os.path.join(HERE, "cpu_emu"))
    import build as emu_build  # tests/cpu_emu/build.py
    return emu_build.build()


def run_cases(exe, cases, workers=8, timeout=1800):
    """Runs the case lines over `workers` processes; returns (outputs, failures)."""
    chunks = [cases[i::workers] for i in range(workers) if cases[i::workers]]

    def one(chunk):
        p = subprocess.run([exe], input="\n".join(chunk) + "\n", capture_output=True, text=True, timeout=timeout,
                           env={**os.environ, "ASAN_OPTIONS": "detect_leaks=0"})
        return p.returncode, p.stdout, p.stderr

    with cf.ThreadPoolExecutor(max_workers=len(chunks)) as ex:
        results = list(ex.map(one, chunks))
    fails = []
    for rc, out, err in results:
        if rc != 0:
            last = [ln for ln in out.splitlines() if ln.startswith("run ")]
            msg = [ln for ln in err.splitlines() if "ERROR" in ln or "runtime error" in ln][:3]
            fails.append((last[-1] if last else "?", msg))
    return [r[1] for r in results], fails


def _ok_lines(outs):
    return [ln for o in outs for ln in o.splitlines() if ln.startswith("ok ")]


def _err_lines(outs):
    return [ln for o in outs for ln in o.splitlines() if ln.startswith("err ")]


def test_planted_mistakes(emu):
    cases = ["gemm 0 200 320 516 S", "gemm 1 200 320 512 S TML_GEMM_DMA_Q=0", "gemm 2 200 320 512 S TML_GEMM_DMA_Q=1",
             "gemm 1 4 4096 1024 S", "prep 2 8 5120 1280 S", "gemm 3 520 384 1536 S"]
    for c in cases:
        _, fails = run_cases(emu, [c], workers=1)
        assert fails, f"the CPU build did not report a short operand: {c}"


def _default_cases():
    cs = []
    # direct-copy GEMM: every tile x split x format on ragged shapes
    for fmt, (M, N, K) in [(F32, (200, 324, 516)), (F16, (200, 328, 520)), (Q8_0, (200, 336, 516)),
                           (Q4_0, (200, 352, 520)), (Q8_K, (200, 352, 516)), (Q8_0_PC, (150, 336, 260)),
                           (Q4_0_PC, (150, 352, 264))]:
        for tile in range(1, 12):
            for split in (1, 3, 4):
                cs.append(f"gemm {fmt} {M} {N} {K} br TML_GEMM_DMA_Q=1 TML_GEMM_DMA_TILE={tile} TML_GEMM_SPLIT={split}")
        for tile in (1, 2, 3, 7, 8):  # tiles with the fused split-K exchange
            cs.append(f"gemm {fmt} {M} {N} {K} bt TML_GEMM_DMA_Q=1 TML_GEMM_DMA_TILE={tile} TML_GEMM_SPLIT=4 "
                      f"TML_GEMM_FUSED=1")
        cs.append(f"gemm {fmt} {M} {N} {K} bB TML_GEMM_DMA_Q=1 TML_GEMM_XCDPART=0 TML_GEMM_SPLIT=2")
        if fmt == F32:
            # the planner's own plans below 128 rows (32x32 two-group tile, K
            # split 1-4; ragged M and N)
            for (sm, sn, sk) in ((16, 4096, 1024), (64, 1024, 4096), (96, 768, 3072), (16, 3840, 1280),
                                 (100, 1540, 384), (37, 1000, 1032)):
                cs.append(f"gemm {fmt} {sm} {sn} {sk} br")
        # register-staged GEMM: every tile, vector and generic paths
        for tile in range(1, 11):
            cs.append(f"gemm {fmt} {M} {N} {K} bre TML_GEMM_DMA=0 TML_GEMM_TILE={tile}")
        cs.append(f"gemm {fmt} {M} {N - 1 if fmt in (F32, F16, Q8_0, Q8_0_PC) else N} {K - 2} b TML_GEMM_DMA=0")
        if fmt in (Q8_0, Q4_0, Q8_0_PC, Q4_0_PC):
            # the bf16 matrix-core kernel: every tile, K split or not (K a
            # multiple of 8 here), and the planner's own choice
            for tile in range(1, 12):
                for split in (1, 3):
                    cs.append(f"gemm {fmt} {M} {N} {K - K % 8 + 8} br TML_GEMM_QBF=2 TML_GEMM_QBF_TILE={tile} "
                              f"TML_GEMM_QBF_SPLIT={split}")
            cs.append(f"gemm {fmt} 33 {N + 2} 40 te TML_GEMM_QBF=2")
            # the planner's own small-M plans (K split 4, 3, 2 and none)
            cs.append(f"gemm {fmt} 16 1024 1024 br")
            cs.append(f"gemm {fmt} 16 3072 768 b")
            cs.append(f"gemm {fmt} 48 4096 512 bB")
            cs.append(f"gemm {fmt} 100 4096 256 b")
            cs.append(f"gemm {fmt} 300 70 1288 bB")
    # [K,N] GEMV and the prepared GEMV at every row count
    for fmt in (F32, F16, Q8_0, Q4_0, Q8_K, Q8_0_PC, Q4_0_PC):
        for M in range(1, 9):
            cs.append(f"gemm {fmt} {M} 1000 {1030 if fmt != Q8_K else 1024} br")
            cs.append(f"gemm {fmt} {M} 96 4100 bB")
            if fmt != Q8_K:
                cs.append(f"prep {fmt} {M} 1000 {1030 if fmt not in (Q4_0, Q4_0_PC) else 1028} br")
                cs.append(f"prep {fmt} {M} 130 4096 bt")
        if fmt in (Q8_0, Q4_0, Q8_0_PC, Q4_0_PC):
            # the matrix-core decoder GEMV: each workgroup width, chunk batch
            # and staged row count, partial column tiles and partial rounds
            for M in (2, 3, 5, 8):
                cs.append(f"prep {fmt} {M} 4100 256 b")
                cs.append(f"prep {fmt} {M} 2050 1280 br")
                for nw in (1, 3, 5, 10, 16):
                    for it in (1, 2, 4):
                        for t in (1, 2):
                            cs.append(f"prep {fmt} {M} 40 2080 b TML_GEMVTM_NW={nw} TML_GEMVTM_IT={it} "
                                      f"TML_GEMVTM_T={t} TML_GEMVTM_PF={(nw + it + t) % 2}")
            # the staged-activation GEMV (M <= 2; 3-4 below): both thread counts, every
            # layer count, rows ragged against the layers, long rows (224 /
            # 384 chunks, activations near the 64 KiB of LDS the kernel may
            # use at M = 2) and the shortest (one chunk)
            big = 7168 if fmt in (Q4_0, Q4_0_PC) else 6144
            one = 32 if fmt in (Q4_0, Q4_0_PC) else 16
            for M in (1, 2):
                for nt in (256, 512):
                    for pl in (1, 2, 3, 4):
                        cs.append(f"prep {fmt} {M} 997 1280 br TML_GEMVX=3 TML_GEMVX_NT={nt} TML_GEMVX_P={pl}")
                cs.append(f"prep {fmt} {M} 37 {big} bt TML_GEMVX=3")
                cs.append(f"prep {fmt} {M} 7 {one} b TML_GEMVX=3 TML_GEMVX_P=4")
            # three and four rows (three computed as four, the fourth zero)
            for M in (3, 4):
                for pl in (1, 4):
                    cs.append(f"prep {fmt} {M} 997 1280 br TML_GEMVX=3 TML_GEMVX_NT=512 TML_GEMVX_P={pl}")
                cs.append(f"prep {fmt} {M} 37 3072 bt TML_GEMVX=3")
                cs.append(f"prep {fmt} {M} 7 {one} b TML_GEMVX=3")
            # rows split over two workgroups (grid.y), odd row counts included
            for M in (5, 7, 8):
                cs.append(f"prep {fmt} {M} 2050 1280 br TML_GEMVTM_MSPLIT=2")
                cs.append(f"prep {fmt} {M} 40 2080 bt TML_GEMVTM_MSPLIT=2 TML_GEMVTM_T=2")
        if fmt in (F32, F16, Q8_0, Q4_0):
            cs.append(f"rows {fmt} 3 777 260 b")
            cs.append(f"rows {fmt} 13 300 384 b")
            # [K,N] GEMV on rows that are not whole lane chunks (funnel-shifted
            # chunks): B ending inside a dword (K*N odd), every segment width,
            # K split over several workgroups
            for M in (1, 2, 4, 8):
                cs.append(f"gemm {fmt} {M} 1001 1029 br")
                for lpr in (4, 16, 64):
                    cs.append(f"gemm {fmt} {M} 333 517 bB TML_GEMV_LPR={lpr} TML_GEMV_NB=1")
    # vocabulary-sized weights (16 MiB or more: the wide-segment plans)
    cs += ["gemm 0 1 51866 161 br", "gemm 0 4 51866 161 b", "gemm 1 1 51866 700 br", "gemm 2 2 51866 1299 bB"]
    # Q8_0 at M <= 4 with a segment per CU: one lane a row, K in one batch
    cs += ["gemm 1 1 4096 1024 br", "gemm 1 3 4096 1000 bB", "gemm 1 4 8192 1024 bt"]
    # one and two lanes a row forced, every format (the aligned path)
    for fmt in (F32, F16, Q8_0, Q4_0, Q8_K):
        for M in (1, 5, 8):
            for lpr in (1, 2):
                cs.append(f"gemm {fmt} {M} 640 {1024 if fmt == Q8_K else 333} bB TML_GEMV_LPR={lpr} TML_GEMV_NB=1")
    # odd shapes through the generic paths, quantizers, transposing loaders, host API
    cs += ["gemm 0 9 7 5 b", "gemm 2 33 17 9 b", "gemm 3 40 64 32 b", "gemm 4 3 5 7 br", "gemm 0 1 1 1 -",
           "gemm 1 12 48 3000 b TML_GEMV_SPLIT=7", "host 0 70 96 64 b", "host 1 5 4096 1024 b", "host 18 3 256 96 b",
           # pinned staging split over the host copy threads: a 2.8 MB A and an 11 MB weight
           # (three 4 MiB chunks), a 2.4 MB C, a 4.5 MB C (two chunks)
           "host 0 1 4 700000 b", "host 0 600 1024 4 b", "host 0 1100 1024 4 b"]
    for fmt in (Q8_0, Q4_0, Q8_K, F16):
        cs += [f"quant {fmt} 0 1 100003 -", f"quant {fmt} 0 33 17 -"]
    for fmt in (Q8_0_PC, Q4_0_PC):
        cs += [f"quant {fmt} 0 129 77 -"]
    for fmt in (Q8_0, Q4_0, Q8_K):
        cs += [f"treq {fmt} 0 96 64 -", f"treq {fmt} 0 70 33 -"]
    return cs


def test_cases(emu):
    cases = _default_cases()
    outs, fails = run_cases(emu, cases)
    assert not fails, fails
    errs = _err_lines(outs)
    assert len(_ok_lines(outs)) + len(errs) == len(cases)
    # the only refusals are documented ones: Q4_0 has no 96x32 direct-copy
    # tile (the planner skips it), so nothing here may fail
    assert not errs, errs[:5]


def _sweep_cases():
    """The narrow-format calibration sweep: every direct-copy tile forced,
    K split 1 / 2 / 4, TML_GEMM_DMA_Q=1, plus the register-staged kernel at
    every tile, over F16 at the Whisper large-v3-turbo encoder shapes and the
    sentence-transformer shapes, Q4_0 at the encoder shapes and
    128x5120x1280, Q8_K and Q8_0 at the sentence-transformer shapes."""
    enc = [(1500, 3840, 1280), (1500, 5120, 1280), (1500, 1280, 5120)]
    st = [(512, 384, 384), (512, 1536, 384), (512, 384, 1536), (256, 768, 3072), (2048, 768, 3072)]
    plan = {F16: enc + st, Q4_0: enc + [(128, 5120, 1280)], Q8_K: st, Q8_0: st}
    cs = []
    for fmt, shapes in plan.items():
        for (M, N, K) in shapes:
            for tile in range(1, 12):
                for split in (1, 2, 4):
                    cs.append(f"gemm {fmt} {M} {N} {K} - TML_GEMM_DMA_Q=1 TML_GEMM_DMA_TILE={tile} "
                              f"TML_GEMM_SPLIT={split}")
                if tile <= 10:
                    cs.append(f"gemm {fmt} {M} {N} {K} - TML_GEMM_DMA_Q=0 TML_GEMM_TILE={tile}")
    return cs


@pytest.mark.skipif(os.environ.get("TML_EMU_FULL") != "1", reason="full sweep replay: set TML_EMU_FULL=1")
def test_fault_sweep_replay(emu):
    cases = _sweep_cases()
    outs, fails = run_cases(emu, cases, timeout=3600)
    assert not fails, fails
    assert len(_ok_lines(outs)) + len(_err_lines(outs)) == len(cases)
    assert not _err_lines(outs), _err_lines(outs)[:5]


def _tl_variants(tmp_path):
    """The reference's and the exporter's .tl fixtures, then truncated and
    corrupted copies of them: every cut inside the header and table, seeded
    random byte flips, and fields set to extreme values (tensor count,
    name length, rank, dims -- including a shape whose product wraps 2^64 --
    payload offset and size)."""
    import glob
    import random
    import struct
    gold = sorted(glob.glob(os.path.join(HERE, "golden", "tl", "*.tl")))
    out = list(gold)
    rng = random.Random(4242)
    k = 0

    def put(data):
        nonlocal k
        p = tmp_path / f"v{k}.tl"
        k += 1
        p.write_bytes(bytes(data))
        out.append(str(p))

    for g in gold:
        data = open(g, "rb").read()
        for cut in range(0, min(len(data), 160), 3):
            put(data[:cut])
        for _ in range(40):
            d = bytearray(data)
            for _ in range(rng.randint(1, 4)):
                pos = rng.randrange(0, min(len(d), 256))
                d[pos] = rng.randrange(256)
            put(d)
        # extreme fields of the first table entry: count, name length, rank,
        # dims (a product that wraps 2^64 to zero), offset and size
        nlen = struct.unpack_from("<I", data, 16)[0] if len(data) >= 20 else 0
        at_rank = 20 + nlen
        variants = [(8, 0xFFFFFFFF), (16, 0xFFFFFFFF), (at_rank, 0xFFFFFFFF)]
        for off, val in variants:
            if off + 4 <= len(data):
                d = bytearray(data)
                struct.pack_into("<I", d, off, val)
                put(d)
        if at_rank + 4 <= len(data):
            ndim = struct.unpack_from("<I", data, at_rank)[0]
            if ndim and at_rank + 4 + 4 * ndim + 16 <= len(data):
                d = bytearray(data)
                for i in range(ndim):
                    struct.pack_into("<I", d, at_rank + 4 + 4 * i, 1 << 16 if i < 4 else 1)
                put(d)
                if ndim < 4:
                    # rank 4 with dims 2^16 each: the product wraps to 0
                    d = bytearray(data[:at_rank]) + struct.pack("<I", 4) + struct.pack("<4I", *[1 << 16] * 4) + \
                        bytearray(data[at_rank + 4 + 4 * ndim:])
                    put(d)
                ot = at_rank + 4 + 4 * ndim
                for val in ((1 << 64) - 1, 1 << 63, len(data) - 1):
                    d = bytearray(data)
                    struct.pack_into("<Q", d, ot, val)
                    put(d)
                    d = bytearray(data)
                    struct.pack_into("<Q", d, ot + 8, val)
                    put(d)
    return out


def test_tl_parser_on_corrupted_files(emu, tmp_path):
    # The native .tl reader (parse, table, every getter to host and device,
    # getTensorDequantized) on the fixtures and ~900 damaged copies: errors
    # are expected, out-of-bounds accesses and undefined behaviour are not.
    files = _tl_variants(tmp_path)
    assert len(files) > 900
    cases = [f"tlfile 0 0 0 0 {p}" for p in files]
    outs, fails = run_cases(emu, cases)
    assert not fails, fails
    assert len(_ok_lines(outs)) + len(_err_lines(outs)) == len(cases)
    # the untouched fixtures all open
    ok = " ".join(_ok_lines(outs))
    for g in files:
        if os.path.dirname(g) == os.path.join(HERE, "golden", "tl"):
            assert f"tlfile 0 0 0 0 {g}" in ok, g


def test_noalloc_entry_point(emu):
    # tml_hip_gemm_ex_dev_noalloc: its static scratch (partials, counters,
    # zero block) serves the split-K GEMM, the split [K,N] GEMV and plain
    # plans inside bounds; a plan needing more than the array is refused.
    ok_cases = ["noalloc 0 256 512 4096 br TML_GEMM_SPLIT=4", "noalloc 0 96 256 2048 bt TML_GEMM_SPLIT=4",
                "noalloc 1 4 1024 8192 b", "noalloc 1 3 512 4096 br", "noalloc 0 300 260 516 be",
                "noalloc 17 6 1000 3000 b", "noalloc 2 8 640 5120 b", "noalloc 3 5 384 1536 b",
                "noalloc 0 128 256 2048 b TML_GEMM_SPLIT=4 TML_GEMM_DMA_TILE=2 TML_GEMM_FUSED=1",
                "noalloc 1 512 1024 4096 br", "noalloc 2 300 512 1024 b TML_GEMM_QBF_SPLIT=4"]
    outs, fails = run_cases(emu, ok_cases, workers=3)
    assert not fails, fails
    assert len(_ok_lines(outs)) == len(ok_cases), _err_lines(outs)
    outs, fails = run_cases(emu, ["noalloc 0 512 1024 4096 - TML_GEMM_SPLIT=8"], workers=1)
    assert not fails and len(_err_lines(outs)) == 1 and "static scratch" in _err_lines(outs)[0]
