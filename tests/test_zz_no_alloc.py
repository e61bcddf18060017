"""tml_hip_gemm_ex_dev_noalloc, the allocation-free entry point, against
tml_hip_gemm_ex_dev through the C ABI: the same kernels and plans, so the
same bits, on two calls in a row (the second smaller) in every kernel family
that uses split-K scratch -- the direct-copy GEMM with its K split
(partials), the [K,N] GEMV with its split exchange (partials and arrival
counters) -- and in one that uses none; a plan whose scratch exceeds the
static array is refused before any launch; replays of a graph captured on
the no-allocation call match its eager result."""
import os

import numpy as np
import pytest

from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu

SCRATCH = 16 << 20  # TML_NOALLOC_SCRATCH_BYTES


@pytest.fixture
def env():
    keys = ("TML_GEMM_SPLIT", "TML_GEMM_DMA_TILE", "TML_REQUIRE_SPLIT")
    saved = {k: os.environ.get(k) for k in keys}
    yield os.environ
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def _problem(torch, seed, fmt, m, n, k, with_res=False):
    a = torch.from_numpy(synth.normal_matrix(seed, m, k)).cuda()
    w = synth.normal_matrix(seed + 1, k, n, 0.02)
    scale = 1.0
    if fmt == _abi.FMT_F32:
        b = torch.from_numpy(w).cuda()
    else:
        wd = torch.from_numpy(w).cuda()
        nbytes = _abi.weight_bytes(fmt, k, n)
        b = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        sc = torch.empty(1, dtype=torch.float32, device="cuda")
        _abi.quantize_dev(fmt, k * n, wd.data_ptr(), b.data_ptr(), sc.data_ptr())
        torch.cuda.synchronize()
        scale = float(sc.item())
    bias = torch.from_numpy(synth.normal(seed + 2, n, 0.0, 0.02)).cuda()
    res = torch.from_numpy(synth.normal_matrix(seed + 3, m, n)).cuda() if with_res else None
    return a, b, scale, bias, res


def _both(torch, fmt, m, n, k, a, b, scale, bias, res, act):
    out = []
    for fn in (_abi.gemm_ex_dev, _abi.gemm_ex_dev_noalloc):
        c = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda")
        fn(fmt, m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr(), act=act, scale=scale, bias_ptr=bias.data_ptr(),
           residual_ptr=res.data_ptr() if res is not None else None)
        torch.cuda.synchronize()
        out.append(c.cpu().numpy())
    return out


@pytest.mark.parametrize("case", ["gemm_split", "gemv_split", "qbf_split_q8", "qbf_split_q4", "gemm_plain"])
def test_matches_existing_entry_point(env, case):
    import torch
    _abi.init()
    if case == "gemm_split":
        # direct-copy GEMM, K split 4 (partials in the scratch); then a smaller one
        env["TML_GEMM_SPLIT"] = "4"
        shapes, fmt, act = [(256, 512, 4096), (96, 256, 2048)], _abi.FMT_F32, _abi.ACT_GELU_ERF
    elif case == "gemv_split":
        # [K,N] GEMV, M <= 8, long K: split over workgroups (partials + counters)
        shapes, fmt, act = [(4, 1024, 8192), (3, 512, 4096)], _abi.FMT_Q8_0, _abi.ACT_NONE
    elif case == "qbf_split_q8":
        # bf16 matrix-core GEMM with its default K split (few 32 x 64 tiles)
        shapes, fmt, act = [(128, 1024, 4096), (128, 512, 2048)], _abi.FMT_Q8_0, _abi.ACT_GELU_ERF
    elif case == "qbf_split_q4":
        shapes, fmt, act = [(128, 1024, 4096), (128, 512, 2048)], _abi.FMT_Q4_0, _abi.ACT_NONE
    else:
        shapes, fmt, act = [(1500, 1536, 384), (700, 768, 384)], _abi.FMT_F32, _abi.ACT_GELU_TANH
    if case != "gemm_plain":
        # both entry points refuse a plan that does not split K, so the
        # partials (and, for the GEMV, the arrival counters) were used
        env["TML_REQUIRE_SPLIT"] = "1"
    for i, (m, n, k) in enumerate(shapes):
        a, b, scale, bias, res = _problem(torch, 500 + 10 * i, fmt, m, n, k, with_res=(i == 1))
        ref, got = _both(torch, fmt, m, n, k, a, b, scale, bias, res, act)
        assert not np.isnan(ref).any()
        np.testing.assert_array_equal(got, ref)


def test_oversized_plan_is_refused(env):
    import torch
    # K split 8 at 512 x 1024 needs 8 * 512 * 1024 floats = 16 MiB of partial
    # sums, more than the array holds next to its counters
    env["TML_GEMM_SPLIT"] = "8"
    m, n, k = 512, 1024, 4096
    assert 8 * m * n * 4 > SCRATCH - (256 + 4 * 16384)
    a, b, scale, bias, _ = _problem(torch, 700, _abi.FMT_F32, m, n, k)
    c = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    with pytest.raises(_abi.TmlError) as e:
        _abi.gemm_ex_dev_noalloc(_abi.FMT_F32, m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr())
    assert e.value.code == _abi.TML_ERR_INVALID_SHAPE and "static scratch" in str(e.value)
    torch.cuda.synchronize()
    assert float(c.abs().max()) == 0.0  # nothing ran


@pytest.mark.parametrize("fmt", [_abi.FMT_Q8_0, _abi.FMT_Q4_0])
def test_default_plan_too_large_is_refused_not_shrunk(env, fmt):
    """Whisper FFN-down (1500 x 1280 x 5120) in Q8_0 / Q4_0: the bf16 GEMM's
    default plan splits K four ways, 4 * 1500 * 1280 floats = 31 MB of
    partial sums, more than the static scratch.  The allocation-free call
    refuses it rather than running a smaller split with other bits; the
    allocating call runs that plan (TML_REQUIRE_SPLIT=1 shows it splits)."""
    import torch
    m, n, k = 1500, 1280, 5120
    a, b, scale, bias, _ = _problem(torch, 720, fmt, m, n, k)
    env["TML_REQUIRE_SPLIT"] = "1"
    c = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    _abi.gemm_ex_dev(fmt, m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr(), scale=scale)
    torch.cuda.synchronize()
    assert float(c.abs().max()) > 0.0
    c.zero_()
    with pytest.raises(_abi.TmlError) as e:
        _abi.gemm_ex_dev_noalloc(fmt, m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr(), scale=scale)
    assert e.value.code == _abi.TML_ERR_INVALID_SHAPE and "static scratch" in str(e.value)
    torch.cuda.synchronize()
    assert float(c.abs().max()) == 0.0  # nothing ran


def test_graph_of_noalloc_calls(env):
    import torch
    env["TML_GEMM_SPLIT"] = "2"
    m, n, k = 128, 256, 2048
    a, b, scale, bias, _ = _problem(torch, 800, _abi.FMT_F32, m, n, k)
    c = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    side = torch.cuda.Stream()

    def call(st):
        _abi.gemm_ex_dev_noalloc(_abi.FMT_F32, m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr(),
                                 bias_ptr=bias.data_ptr(), stream=st)

    with torch.cuda.stream(side):
        call(side.cuda_stream)
    torch.cuda.synchronize()
    ref = c.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        call(side.cuda_stream)
    torch.cuda.synchronize()
    a2, b2, _, bias2, _ = _problem(torch, 810, _abi.FMT_Q8_0, 5, 2048, 8192)
    c2 = torch.zeros((5, 2048), dtype=torch.float32, device="cuda")
    for _ in range(4):
        c.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(c, ref)
        # another no-allocation call between the replays reuses the scratch
        _abi.gemm_ex_dev_noalloc(_abi.FMT_Q8_0, 5, 2048, 8192, a2.data_ptr(), b2.data_ptr(), c2.data_ptr())
        torch.cuda.synchronize()
    ref64 = (a.double() @ b.double() + bias.double()).cpu().numpy()
    assert float(np.max(np.abs(c.cpu().numpy() - ref64)) / np.max(np.abs(ref64))) <= 1e-4
