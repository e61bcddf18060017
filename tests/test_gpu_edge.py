"""Degenerate shapes through every weight format and entry point.

The reference validates shapes before it computes (src/core/ops.zig:236-249)
and returns a zero-filled C (:262-264) plus the bias when it has one
(:422-471); an empty inner dimension therefore gives C = bias, and an empty
M or N an empty result.  Here: M = 0 or N = 0 must leave C untouched and
succeed, K = 0 must give exactly beta*C + bias (bitwise), and 1x1x1 products
must equal the oracle's, for f32, Q8_0, Q4_0, Q8_K, F16 and the per-column
formats, through the host-pointer, device-pointer and prepared entry points.
"""
import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu

FMTS = [_abi.FMT_F32, _abi.FMT_Q8_0, _abi.FMT_Q4_0, _abi.FMT_Q8_K, _abi.FMT_F16, _abi.FMT_Q8_0_PC,
        _abi.FMT_Q4_0_PC]


def _weight(orc, fmt, k, n, seed=5):
    """(B bytes, keyword arguments of _abi.gemm, dequantized [k, n] weight)."""
    w = synth.normal_matrix(seed, k, n, 0.5) if k * n else np.zeros((k, n), np.float32)
    if fmt == _abi.FMT_F32:
        return w, {}, w
    if fmt == _abi.FMT_F16:
        h = orc.to_f16(w)
        return h, {}, orc.from_f16(h)
    if fmt == _abi.FMT_Q8_0:
        q, s = orc.quantize_q8(w)
        return q, {"scale": s}, orc.dequantize_q8(q, s).reshape(k, n)
    if fmt == _abi.FMT_Q4_0:
        p, s = orc.quantize_q4(w)
        return p, {"scale": s}, orc.dequantize_q4(p, k * n, s).reshape(k, n)
    if fmt == _abi.FMT_Q8_K:
        q, sc = orc.quantize_q8k(w)
        sc = sc if sc.size else np.ones(1, np.float32)
        return q, {"scales": np.ascontiguousarray(sc, np.float32)}, orc.dequantize_q8k(q, sc).reshape(k, n)
    q, s = orc.quantize_q8_cols(w) if fmt == _abi.FMT_Q8_0_PC else orc.quantize_q4_cols(w)
    s = s if s.size else np.ones(1, np.float32)
    return q, {"scales": np.ascontiguousarray(s, np.float32)}, orc.dequantize_cols(fmt, q, s, k, n)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m,n,k", [(0, 5, 3), (4, 0, 3), (0, 0, 0), (0, 64, 0)])
def test_empty_output_is_a_noop(orc, fmt, m, n, k):
    b, kw, _ = _weight(orc, fmt, k, n)
    a = np.ones((m, k), np.float32)
    c = np.full((max(m, 1), max(n, 1)), 7.0, np.float32)
    bias = np.ones(max(n, 1), np.float32)
    _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(b), c, bias=bias, **kw)
    assert (c == 7.0).all()


@pytest.mark.parametrize("fmt", FMTS)
def test_empty_inner_dimension(orc, fmt):
    # K = 0: the product is an empty sum, so C = beta*C + bias exactly.
    import torch
    m, n = 3, 64
    b, kw, _ = _weight(orc, fmt, 0, n)
    bias = synth.normal(7, n, 0.0, 1.0)
    c = np.full((m, n), 7.0, np.float32)
    _abi.gemm(fmt, m, n, 0, np.zeros((m, 0), np.float32), np.ascontiguousarray(b), c, bias=bias, **kw)
    np.testing.assert_array_equal(c, np.broadcast_to(bias, (m, n)))
    # device pointers with beta = 1: C + bias
    c0 = synth.normal_matrix(8, m, n)
    C = torch.from_numpy(c0).cuda()
    Bias = torch.from_numpy(bias).cuda()
    A = torch.zeros(16, device="cuda")
    Bd = torch.zeros(64, dtype=torch.uint8, device="cuda")
    S = torch.ones(n, device="cuda")
    scales_ptr = S.data_ptr() if "scales" in kw else None
    _abi.gemm_dev(fmt, m, n, 0, A.data_ptr(), Bd.data_ptr(), C.data_ptr(), scale=kw.get("scale", 1.0),
                  scales_ptr=scales_ptr, bias_ptr=Bias.data_ptr(), beta=1.0)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(C.cpu().numpy(), c0 + bias[None, :])


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (1, 2, 1), (2, 1, 3), (9, 1, 1)])
def test_tiny_products(orc, fmt, m, n, k):
    b, kw, deq = _weight(orc, fmt, k, n, seed=11 + m + n + k)
    a = synth.normal_matrix(12, m, k)
    c = np.zeros((m, n), np.float32)
    _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(b), c, **kw)
    ref = orc.matmul(a, np.ascontiguousarray(deq, np.float32))
    assert rel_err(c, ref) <= 1e-6, rel_err(c, ref)


@pytest.mark.parametrize("fmt", [_abi.FMT_F32, _abi.FMT_Q8_0, _abi.FMT_Q4_0, _abi.FMT_F16, _abi.FMT_Q8_0_PC])
def test_prepared_zero_rows(orc, fmt):
    # A prepared weight called with M = 0 does nothing; M = 1 afterwards works.
    import torch
    k, n = 96, 40
    b, kw, deq = _weight(orc, fmt, k, n)
    B = torch.from_numpy(np.ascontiguousarray(b).view(np.uint8).reshape(-1)).cuda()
    S = torch.from_numpy(kw["scales"]).cuda() if "scales" in kw else None
    h = _abi.prepare_ex_dev(fmt, k, n, B.data_ptr(), scale=kw.get("scale", 1.0),
                            scales_ptr=S.data_ptr() if S is not None else None)
    try:
        C = torch.full((1, n), 7.0, device="cuda")
        A = torch.from_numpy(synth.normal_matrix(13, 1, k)).cuda()
        _abi.gemm_prepared(h, 0, A.data_ptr(), C.data_ptr())
        torch.cuda.synchronize()
        assert (C.cpu().numpy() == 7.0).all()
        _abi.gemm_prepared(h, 1, A.data_ptr(), C.data_ptr())
        torch.cuda.synchronize()
        ref = orc.matmul(A.cpu().numpy(), np.ascontiguousarray(deq, np.float32))
        assert rel_err(C.cpu().numpy(), ref) <= 1e-5
    finally:
        _abi.prepared_free(h)
