"""The split-K workspace under HIP graphs, and the planner's override limit.

* A graph captured on a split-K GEMM keeps its workspace: later calls that
  grow the workspace retire the old buffer instead of freeing it, so every
  replay of the old graph still gives its eager result bit for bit (checked
  over several replays with eager work in between).
* A call that would have to grow the workspace while its stream is being
  captured is refused (TML_ERR_INVALID_ARG) instead of allocating inside
  the capture; the same call made eagerly afterwards works.
* Forced planner overrides (TML_GEMM_*) are refused above the sizes the
  tests run them at; the refusal comes before any launch.
"""
import os

import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu

KEYS = ("TML_GEMM_SPLIT", "TML_GEMM_DMA_TILE", "TML_GEMM_FUSED")


@pytest.fixture
def env():
    saved = {k: os.environ.get(k) for k in KEYS}
    yield os.environ
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def _operands(torch, seed, m, n, k):
    a = torch.from_numpy(synth.normal_matrix(seed, m, k)).cuda()
    b = torch.from_numpy(synth.normal_matrix(seed + 1, k, n, 0.02)).cuda()
    c = torch.zeros((m, n), dtype=torch.float32, device="cuda")
    return a, b, c


def test_growth_refused_during_capture(env):
    # 2048 x 2048 x 512 split 8 needs 8 * 2048 * 2048 partial sums (128 MiB).
    # A fresh library context starts with no workspace, so the call must grow
    # it whatever the tests before this one ran.
    import torch
    torch.cuda.synchronize()
    _abi.shutdown()
    _abi.init()
    env["TML_GEMM_SPLIT"] = "8"
    m, n, k = 2048, 2048, 512
    a, b, c = _operands(torch, 301, m, n, k)
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with pytest.raises(RuntimeError) as e:
        with torch.cuda.graph(g, stream=side):
            _abi.gemm_dev(_abi.FMT_F32, m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr(), stream=side.cuda_stream)
    assert "eagerly" in str(e.value)
    del g
    torch.cuda.synchronize()
    _abi.gemm_dev(_abi.FMT_F32, m, n, k, a.data_ptr(), b.data_ptr(), c.data_ptr())
    torch.cuda.synchronize()
    ref = (a.double() @ b.double()).cpu().numpy()
    assert rel_err(c.cpu().numpy(), ref) <= 1e-4


def test_graph_replays_after_workspace_growth(env):
    import torch
    side = torch.cuda.Stream()
    env["TML_GEMM_SPLIT"] = "2"
    a1, b1, c1 = _operands(torch, 311, 128, 256, 2048)

    def small(st):
        _abi.gemm_dev(_abi.FMT_F32, 128, 256, 2048, a1.data_ptr(), b1.data_ptr(), c1.data_ptr(), stream=st)

    with torch.cuda.stream(side):
        small(side.cuda_stream)
    torch.cuda.synchronize()
    ref = c1.clone()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        small(side.cuda_stream)
    torch.cuda.synchronize()
    # larger problems grow the workspace (eagerly) while the graph lives
    a2, b2, c2 = _operands(torch, 321, 1024, 2048, 1024)
    for split in ("4", "8"):
        env["TML_GEMM_SPLIT"] = split
        _abi.gemm_dev(_abi.FMT_F32, 1024, 2048, 1024, a2.data_ptr(), b2.data_ptr(), c2.data_ptr())
    torch.cuda.synchronize()
    ref2 = c2.clone()
    for _ in range(4):
        c1.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(c1, ref), "replay after workspace growth differs from the eager result"
        c2.zero_()
        _abi.gemm_dev(_abi.FMT_F32, 1024, 2048, 1024, a2.data_ptr(), b2.data_ptr(), c2.data_ptr())
        torch.cuda.synchronize()
        assert torch.equal(c2, ref2)
    ref64 = (a1.double() @ b1.double()).cpu().numpy()
    assert rel_err(c1.cpu().numpy(), ref64) <= 1e-4


def test_forced_plan_refused_above_tested_sizes(env):
    # 1024 x 1024 x 4096 > 512 * 1024 * 4096: a forced split is refused
    # before any launch; the default plan of the same problem runs.
    env["TML_GEMM_SPLIT"] = "2"
    m, n, k = 1024, 1024, 4096
    a = synth.normal_matrix(331, m, k)
    b = synth.normal_matrix(332, k, n, 0.02)
    c = np.zeros((m, n), np.float32)
    with pytest.raises(RuntimeError) as e:
        _abi.sgemm(m, n, k, a, b, c)
    assert "forced GEMM plans" in str(e.value)
    env.pop("TML_GEMM_SPLIT")
    _abi.sgemm(m, n, k, a, b, c)
    ref = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_err(c, ref) <= 1e-4
