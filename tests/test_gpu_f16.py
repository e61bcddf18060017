"""GPU parity of the F16 weight path (F16Tensor / toF16 / matmulF32F16,
src/core/quantization.zig:1859-1962) against the CPU oracle.

toF16 is compared bitwise (IEEE round to nearest even on both sides).  The
matmuls use the fp32 tolerance, max|G-R|/max|R| <= 1e-4, against the
reference's fallback semantics (f32 accumulation of a * f32(b)); products of
small integers are exact, so there the comparison is bitwise.  Every kernel
family that reads B runs: the [K,N] GEMV (vector and element-wise paths),
the register-staged GEMM, and the prepared K-contiguous GEMV (from [K,N] and
from rows).
"""
import os

import numpy as np
import pytest

from conftest import elementwise_ok, rel_err
from tomoul_amd import _abi, dispatch, quantization as qz, synth
from tomoul_amd.tensor import Tensor

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4


def T(a):
    return Tensor.from_numpy(np.asarray(a, dtype=np.float32))


def rnd(seed, m, n, std=1.0):
    return synth.normal_matrix(seed, m, n, std)


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def test_to_f16_bitwise(orc):
    edge = np.array([0.0, -0.0, 1.0, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 65504.0, 65519.0, 65520.0, 1e6,
                     -65520.0, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -26, 2.0 ** -14,
                     2.0 ** -14 - 2.0 ** -25, np.inf, -np.inf], dtype=np.float32)
    rng = np.random.default_rng(21)
    scaled = (rng.standard_normal(100003) * np.exp2(rng.integers(-30, 18, size=100003))).astype(np.float32)
    for v in (edge, scaled, synth.normal(22, 4097, 0.0, 0.02)):
        got = qz.toF16(T(v)).data
        np.testing.assert_array_equal(got, orc.to_f16(v))
    nan = qz.toF16(T(np.array([np.nan, 1.0], np.float32))).data
    assert np.isnan(nan.view(np.float16)[0]) and nan[1] == 0x3C00


SHAPES = [(1, 4096, 1024), (2, 33, 17), (3, 1000, 96), (5, 45, 77), (8, 1280, 5120), (9, 64, 64),
          (64, 160, 96), (127, 129, 131), (512, 1024, 1024)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_matmul_f16_vs_oracle(orc, m, n, k):
    a = rnd(701, m, k)
    h = orc.to_f16(rnd(702, k, n, 0.02))
    got = qz.matmulF32F16(T(a), qz.F16Tensor(h, (k, n))).numpy()
    ref = orc.matmul_f16(a, h)
    err = rel_err(got, ref)
    assert err <= FP32_TOL and elementwise_ok(got, ref, 1e-4), err


def test_matmul_f16_exact_small_integers(orc):
    rng = np.random.default_rng(23)
    for (m, n, k) in [(1, 640, 300), (4, 96, 64), (70, 130, 50)]:
        a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
        h = orc.to_f16(rng.integers(-8, 9, size=(k, n)).astype(np.float32))
        got = qz.matmulF32F16(T(a), qz.F16Tensor(h, (k, n))).numpy()
        np.testing.assert_array_equal(got, orc.matmul_f16(a, h))


@pytest.mark.parametrize("lpr", [4, 16, 64])
def test_f16_gemv_segments(orc, lpr):
    saved = os.environ.get("TML_GEMV_LPR")
    os.environ["TML_GEMV_LPR"] = str(lpr)
    try:
        k, n = 333, 640
        h = orc.to_f16(rnd(711, k, n, 0.02))
        for m in (1, 2, 3, 5, 8):
            a = rnd(712 + m, m, k)
            got = np.zeros((m, n), np.float32)
            _abi.gemm(_abi.FMT_F16, m, n, k, a, h, got)
            assert rel_err(got, orc.matmul_f16(a, h)) <= FP32_TOL, m
    finally:
        if saved is None:
            os.environ.pop("TML_GEMV_LPR", None)
        else:
            os.environ["TML_GEMV_LPR"] = saved


@pytest.mark.parametrize("m", [1, 2, 3, 5, 8, 9])
def test_f16_prepared(orc, m):
    import torch
    for (k, n) in [(1280, 5120), (77, 45), (1024, 130)]:
        h = orc.to_f16(rnd(721, k, n, 0.02))
        a = rnd(722 + m, m, k)
        bias = synth.normal(723, n, 0.0, 0.5)
        B, A, Bias = _dev(h), _dev(a), _dev(bias)
        C = torch.zeros((m, n), dtype=torch.float32, device="cuda:0")
        w = _abi.prepare_dev(_abi.FMT_F16, k, n, B.data_ptr())
        try:
            _abi.gemm_prepared(w, m, A.data_ptr(), C.data_ptr(), bias_ptr=Bias.data_ptr())
            torch.cuda.synchronize()
        finally:
            _abi.prepared_free(w)
        assert rel_err(C.cpu().numpy(), orc.matmul_f16(a, h) + bias) <= FP32_TOL, (k, n)
        # the same weight given as rows ([N,K], e.g. an f16 embedding)
        R = _dev(np.ascontiguousarray(h.T))
        w = _abi.prepare_rows_dev(_abi.FMT_F16, k, n, R.data_ptr(), 2 * k)
        try:
            _abi.gemm_prepared(w, m, A.data_ptr(), C.data_ptr())
            torch.cuda.synchronize()
        finally:
            _abi.prepared_free(w)
        assert rel_err(C.cpu().numpy(), orc.matmul_f16(a, h)) <= FP32_TOL, (k, n, "rows")


@pytest.mark.parametrize("m", [1, 7, 64])
def test_f16_dispatch_and_epilogues(orc, m):
    # matmulWithWeight / matmulWithWeightBias with an F16Tensor
    # (src/core/attention.zig:114-149), and the fused GELU / residual forms.
    k, n = 96, 162
    a, w = rnd(731, m, k), rnd(732, k, n, 0.05)
    h = orc.to_f16(w)
    f = qz.F16Tensor(h, (k, n))
    bias = synth.normal(733, n, 0.0, 0.5)
    res = rnd(734, m, n)
    tb = Tensor.from_numpy(bias)
    pre = orc.matmul_f16(a, h)
    assert rel_err(dispatch.matmulWithWeight(T(a), f).numpy(), pre) <= FP32_TOL
    assert rel_err(dispatch.matmulWithWeightBias(T(a), f, tb).numpy(), pre + bias) <= FP32_TOL
    got = dispatch.matmulWithWeightBiasGelu(T(a), f, tb).numpy()
    assert rel_err(got, orc.gelu_tanh(pre + bias)) <= FP32_TOL
    got = dispatch.matmulWithWeightBiasResidual(T(a), f, tb, T(res)).numpy()
    assert rel_err(got, pre + bias + res) <= FP32_TOL
