"""The host-pointer entry points' transfers (runtime.hip host_gemm) against the
oracle, one test per staging regime: operands and C through pinned buffers
in 4 MiB chunks (C over one chunk, an input read back for beta != 0, Q8_K
block scales and a residual staged beside the weight), and the direct
transfers of calls whose operands exceed the 256 MiB pinned cap.  These are
the calls the Zig shim makes (src/core/ops.zig:266-275); the tolerances are
the north star's (1e-4 fp32, 1e-3 quantized)."""
import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu


def rnd(seed, m, n, std=1.0):
    return synth.normal_matrix(seed, m, n, std)


def test_host_staged_chunks_alpha_beta(orc):
    # C = 700 x 2048 floats = 5.6 MiB: two chunks down, and read up for beta
    m, n, k = 700, 2048, 96
    a, b, c0 = rnd(501, m, k), rnd(502, k, n, 0.02), rnd(503, m, n)
    c = c0.copy()
    _abi.sgemm(m, n, k, a, b, c, 0.5, -1.5)
    assert rel_err(c, orc.sgemm(a, b, c0, 0.5, -1.5)) <= 1e-4
    # the same call twice more: the pinned buffers are reused, not regrown
    for _ in range(2):
        c2 = c0.copy()
        _abi.sgemm(m, n, k, a, b, c2, 0.5, -1.5)
        np.testing.assert_array_equal(c2, c)


def test_host_staged_q8k_residual(orc):
    # a 4 MiB int8 weight, its 128k block scales and a 2 MiB residual staged
    # in one pinned buffer, a bias beside them
    m, n, k = 128, 4096, 1024
    w = rnd(511, k, n, 0.02)
    q, s = orc.quantize_q8k(w)
    a, res = rnd(512, m, k), rnd(513, m, n)
    bias = synth.normal(514, n, 0.0, 0.02)
    c = np.zeros((m, n), np.float32)
    _abi.gemm_residual(_abi.FMT_Q8_K, m, n, k, a, q.reshape(k, n), res, c, scales=s, bias=bias)
    ref = orc.matmul_q8k(a, q.reshape(k, n), s) + bias + res
    assert rel_err(c, ref) <= 1e-3


def test_host_unstaged_weight(orc):
    # a 302 MB fp32 weight: past the pinned cap, so the call's inputs go
    # from the caller's memory directly
    m, n, k = 2, 9216, 8192
    a, b, c0 = rnd(521, m, k), rnd(522, k, n, 0.02), rnd(523, m, n)
    c = c0.copy()
    _abi.sgemm(m, n, k, a, b, c, 1.0, 0.25)
    assert rel_err(c, orc.sgemm(a, b, c0, 1.0, 0.25)) <= 1e-4


def test_host_unstaged_output(orc):
    # C = 8192 x 8200 floats = 269 MB: past the cap, so C comes down
    # directly; the inputs are small and staged
    m, n, k = 8192, 8200, 4
    a, b = rnd(531, m, k), rnd(532, k, n)
    c = np.zeros((m, n), np.float32)
    _abi.sgemm(m, n, k, a, b, c)
    assert rel_err(c, orc.matmul_mt(a, b, 16)) <= 1e-4
