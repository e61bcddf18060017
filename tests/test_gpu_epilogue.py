"""GPU parity of the fused activation epilogue (GELU erf / GELU tanh).

The reference runs the up-projection, then a separate pass over the whole
output: ops.gelu (tanh form, src/core/transformer.zig:213-221) or
ops.geluExact (erf form, src/models/whisper/encoder.zig:244-247).  The
oracle applies its restatement of that pass (oracle/oracle.c: orc_gelu_tanh,
orc_gelu_exact) to its matmul; the GPU applies it in the kernel epilogue.
Tolerances as for the matmul itself: max|G-R|/max|R| <= 1e-4 (fp32),
<= 1e-3 (quantized).  Shapes are chosen so that M*N % 8 != 0 where the tanh
form's vector/scalar split matters, and so that every kernel family runs:
the [K,N] GEMV (M <= 8), the prepared K-contiguous GEMV, the direct-copy
fp32 GEMM with and without its split-K reduce, and the register-staged GEMM
(quantized weights, or N % 4 != 0).
"""
import os

import numpy as np
import pytest

from conftest import elementwise_ok, rel_err
from tomoul_amd import _abi, dispatch, quantization as qz, synth
from tomoul_amd.tensor import Tensor

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
Q_TOL = 1e-3
ACTS = [_abi.ACT_GELU_ERF, _abi.ACT_GELU_TANH]


def T(a):
    return Tensor.from_numpy(np.asarray(a, dtype=np.float32))


def rnd(seed, m, n, std=1.0):
    return synth.normal_matrix(seed, m, n, std)


SHAPES = [(1, 165, 96), (3, 162, 96), (7, 162, 200), (8, 4097, 64), (64, 160, 96), (300, 262, 136),
          (129, 68, 1028), (1500, 1536, 384)]


@pytest.mark.parametrize("m,n,k", SHAPES)
def test_fused_gelu_all_formats(orc, m, n, k):
    a = rnd(601, m, k)
    w = rnd(602, k, n, 0.05)
    bias = synth.normal(603, n, 0.0, 0.5)
    tb = Tensor.from_numpy(bias)
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    qk, sk = orc.quantize_q8k(w)
    cases = [
        (T(w), orc.matmul_bias(a, w, bias), FP32_TOL),
        (qz.QuantizedTensorQ8(s, q, (k, n)), orc.matmul_q8(a, q, s) + bias, Q_TOL),
        (qz.QuantizedTensorQ4(s4, p, (k, n)), orc.matmul_q4(a, p, k, n, s4) + bias, Q_TOL),
        (qz.QuantizedTensorQ8K(sk, qk, (k, n)), orc.matmul_q8k(a, qk, sk) + bias, Q_TOL),
    ]
    for weight, pre, tol in cases:
        for fn, act in ((dispatch.matmulWithWeightBiasGeluExact, orc.ACT_GELU_ERF),
                        (dispatch.matmulWithWeightBiasGelu, orc.ACT_GELU_TANH)):
            got = fn(T(a), weight, tb).numpy()
            ref = orc.apply_act(pre, act)
            err = rel_err(got, ref)
            assert err <= tol, (type(weight).__name__, act, err)


def test_tanh_split_follows_flat_index(orc):
    # Same pre-activation value in the vector part and in the scalar tail of
    # ops.gelu: M*N = 3*7 = 21, so flat indices 16..20 use tanh itself and
    # 0..15 the rational form.  With A = ones and B chosen so every output
    # is exactly 2.0, the two forms give 1.9762 vs 1.9545 (see the oracle
    # pinning tests); the GPU must reproduce both.
    m, n, k = 3, 7, 4
    a = np.ones((m, k), np.float32)
    w = np.full((k, n), 0.5, np.float32)
    got = np.zeros((m, n), np.float32)
    _abi.gemm_act(_abi.FMT_F32, m, n, k, a, w, got, act=_abi.ACT_GELU_TANH)
    ref = orc.gelu_tanh(np.full((m, n), 2.0, np.float32))
    flat, rflat = got.reshape(-1), ref.reshape(-1)
    assert abs(rflat[0] - rflat[20]) > 0.01
    np.testing.assert_allclose(flat, rflat, rtol=2e-6, atol=0)


@pytest.fixture
def forced_env():
    keys = ("TML_GEMM_SPLIT", "TML_GEMM_DMA_TILE", "TML_GEMM_DMA", "TML_GEMM_TILE", "TML_GEMM_FUSED",
            "TML_GEMM_VEC_EPI", "TML_GEMM_DMA_Q")
    saved = {key: os.environ.get(key) for key in keys}
    yield os.environ
    for key, v in saved.items():
        if v is None:
            os.environ.pop(key, None)
        else:
            os.environ[key] = v


@pytest.mark.parametrize("split", [1, 3])
@pytest.mark.parametrize("act", ACTS)
def test_fused_gelu_split_reduce(orc, forced_env, split, act):
    # With K split, the direct-copy GEMM writes raw partials and the reduce
    # kernel applies bias and activation (its 4-wide path); split 1 takes
    # the GEMM's own epilogue.
    forced_env["TML_GEMM_SPLIT"] = str(split)
    for tile in ("1", "4", "7", "10"):
        forced_env["TML_GEMM_DMA_TILE"] = tile
        for (m, n, k) in [(129, 68, 1028), (300, 260, 516)]:
            a, w = rnd(611, m, k), rnd(612, k, n, 0.03)
            bias = synth.normal(613, n, 0.0, 0.5)
            got = np.zeros((m, n), np.float32)
            _abi.gemm_act(_abi.FMT_F32, m, n, k, a, w, got, act=act, bias=bias)
            ref = orc.apply_act(orc.matmul_bias(a, w, bias), act)
            err = rel_err(got, ref)
            assert err <= FP32_TOL and elementwise_ok(got, ref, 2e-4), (tile, m, n, k, err)


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


@pytest.mark.parametrize("act", ACTS)
@pytest.mark.parametrize("m", [1, 2, 3, 9])
def test_fused_gelu_prepared(orc, act, m):
    # Prepared weights: the K-contiguous kernel for M within its range, the
    # [K,N] fallback beyond it (Q4_0 from M = 3, Q8_0 from M = 5, all at 9).
    import torch
    k, n = 1280, 1283
    w = rnd(621, k, n, 0.03)
    a = rnd(622 + m, m, k)
    bias = synth.normal(623, n, 0.0, 0.5)
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    for fmt, b, scale, pre, tol in [(_abi.FMT_F32, w, 1.0, orc.matmul(a, w), FP32_TOL),
                                    (_abi.FMT_Q8_0, q, s, orc.matmul_q8(a, q, s), Q_TOL),
                                    (_abi.FMT_Q4_0, p, s4, orc.matmul_q4(a, p, k, n, s4), Q_TOL)]:
        B, A, Bias = _dev(b), _dev(a), _dev(bias)
        C = torch.zeros((m, n), dtype=torch.float32, device="cuda:0")
        h = _abi.prepare_dev(fmt, k, n, B.data_ptr(), scale)
        try:
            _abi.gemm_prepared_ex(h, m, A.data_ptr(), C.data_ptr(), act=act, bias_ptr=Bias.data_ptr())
            torch.cuda.synchronize()
        finally:
            _abi.prepared_free(h)
        ref = orc.apply_act(pre + bias, act)
        assert rel_err(C.cpu().numpy(), ref) <= tol, (fmt, m)


@pytest.mark.parametrize("m,n,k", [(3, 200, 300), (64, 256, 128), (70, 90, 33)])
def test_fused_gelu_alpha_beta_dev(orc, m, n, k):
    # The activation applies to alpha * A.B + beta * C + bias as a whole.
    import torch
    a, w, c0 = rnd(631, m, k), rnd(632, k, n, 0.05), rnd(633, m, n)
    bias = synth.normal(634, n, 0.0, 0.5)
    pre = 0.5 * orc.matmul(a, w) - 2.0 * c0 + bias
    for act in ACTS:
        A, B, C, Bias = _dev(a), _dev(w), _dev(c0), _dev(bias)
        _abi.gemm_ex_dev(_abi.FMT_F32, m, n, k, A.data_ptr(), B.data_ptr(), C.data_ptr(), act=act,
                         bias_ptr=Bias.data_ptr(), alpha=0.5, beta=-2.0)
        torch.cuda.synchronize()
        assert rel_err(C.cpu().numpy(), orc.apply_act(pre, act)) <= FP32_TOL, act


def test_act_none_matches_plain_entry_point():
    # act = TML_ACT_NONE is the plain GEMM bit for bit; an unknown
    # activation is rejected before any device work.
    m, n, k = 5, 96, 64
    a, w = rnd(641, m, k), rnd(642, k, n)
    c0, c1 = np.zeros((m, n), np.float32), np.zeros((m, n), np.float32)
    _abi.gemm(_abi.FMT_F32, m, n, k, a, w, c0)
    _abi.gemm_act(_abi.FMT_F32, m, n, k, a, w, c1, act=_abi.ACT_NONE)
    np.testing.assert_array_equal(c0, c1)
    with pytest.raises(_abi.TmlError) as e:
        _abi.gemm_act(_abi.FMT_F32, m, n, k, a, w, c1, act=7)
    assert e.value.code == _abi.TML_ERR_INVALID_ARG


# ------------------------------------------------------------ residual add
@pytest.mark.parametrize("m,n,k", [(1, 1024, 4096), (3, 162, 96), (64, 160, 96), (300, 262, 136),
                                   (512, 1024, 4096)])
def test_fused_residual_all_formats(orc, m, n, k):
    # matmulWithWeightBias then ops.addInPlace (src/core/transformer.zig:
    # 223-228): (A.B + bias) + residual, the same two additions in the same
    # order, for every weight type and kernel family.
    a = rnd(651, m, k)
    w = rnd(652, k, n, 0.02)
    bias = synth.normal(653, n, 0.0, 0.5)
    res = rnd(654, m, n)
    tb, tr = Tensor.from_numpy(bias), T(res)
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    qk, sk = orc.quantize_q8k(w)
    cases = [
        (T(w), orc.matmul_bias(a, w, bias), FP32_TOL),
        (qz.QuantizedTensorQ8(s, q, (k, n)), orc.matmul_q8(a, q, s) + bias, Q_TOL),
        (qz.QuantizedTensorQ4(s4, p, (k, n)), orc.matmul_q4(a, p, k, n, s4) + bias, Q_TOL),
        (qz.QuantizedTensorQ8K(sk, qk, (k, n)), orc.matmul_q8k(a, qk, sk) + bias, Q_TOL),
    ]
    for weight, pre, tol in cases:
        got = dispatch.matmulWithWeightBiasResidual(T(a), weight, tb, tr).numpy()
        ref = pre + res
        assert rel_err(got, ref) <= tol, (type(weight).__name__, rel_err(got, ref))
    with pytest.raises(Exception):
        dispatch.matmulWithWeightBiasResidual(T(a), T(w), tb, T(res[:, :-1]))


@pytest.mark.parametrize("split", [1, 3])
def test_fused_residual_in_place_dev(orc, forced_env, split):
    # residual == C (in-place update of the residual stream) on device
    # pointers, through the GEMM epilogue (split 1) and the split-K reduce.
    import torch
    forced_env["TML_GEMM_SPLIT"] = str(split)
    m, n, k = 200, 256, 1024
    a, w, x = rnd(661, m, k), rnd(662, k, n, 0.02), rnd(663, m, n)
    bias = synth.normal(664, n, 0.0, 0.5)
    A, B, X, Bias = _dev(a), _dev(w), _dev(x), _dev(bias)
    _abi.gemm_ex_dev(_abi.FMT_F32, m, n, k, A.data_ptr(), B.data_ptr(), X.data_ptr(), residual_ptr=X.data_ptr(),
                     bias_ptr=Bias.data_ptr())
    torch.cuda.synchronize()
    ref = orc.matmul_bias(a, w, bias) + x
    assert rel_err(X.cpu().numpy(), ref) <= FP32_TOL


@pytest.mark.parametrize("m", [1, 2, 9])
def test_fused_residual_prepared(orc, m):
    import torch
    k, n = 1280, 1280
    w, a, x = rnd(671, k, n, 0.02), rnd(672, m, k), rnd(673, m, n)
    bias = synth.normal(674, n, 0.0, 0.5)
    q, s = orc.quantize_q8(w)
    for fmt, b, scale, pre, tol in [(_abi.FMT_F32, w, 1.0, orc.matmul(a, w), FP32_TOL),
                                    (_abi.FMT_Q8_0, q, s, orc.matmul_q8(a, q, s), Q_TOL)]:
        B, A, X, Bias = _dev(b), _dev(a), _dev(x), _dev(bias)
        C = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
        h = _abi.prepare_dev(fmt, k, n, B.data_ptr(), scale)
        try:
            _abi.gemm_prepared_ex(h, m, A.data_ptr(), C.data_ptr(), residual_ptr=X.data_ptr(),
                                  bias_ptr=Bias.data_ptr(), act=_abi.ACT_GELU_ERF)
            torch.cuda.synchronize()
        finally:
            _abi.prepared_free(h)
        ref = orc.gelu_exact(pre + bias + x)
        assert rel_err(C.cpu().numpy(), ref) <= tol, (fmt, m)


# ------------------------------------- rows-prepared weights (vocab projection)
def _rows_cases(orc, e):
    # e: [N, K] rows (a token embedding); the product is x . e^T.
    n, k = e.shape
    q, s = orc.quantize_q8(e)
    cases = [(_abi.FMT_F32, e, 4 * k, 1.0, e.T.copy(), FP32_TOL),
             (_abi.FMT_Q8_0, q, k, s, orc.dequantize_q8(q, s).reshape(n, k).T.copy(), Q_TOL)]
    if k % 2 == 0:
        p, s4 = orc.quantize_q4(e)
        cases.append((_abi.FMT_Q4_0, p, k // 2, s4, orc.dequantize_q4(p, n * k, s4).reshape(n, k).T.copy(), Q_TOL))
    return cases


@pytest.mark.parametrize("n,k", [(1000, 1280), (333, 77), (130, 96), (64, 100)])
@pytest.mark.parametrize("m", [1, 2, 3, 9, 20])
def test_prepared_rows_vs_oracle(orc, n, k, m):
    # logits = x . E^T with E [n_vocab, d] as stored (decoder.zig:936-940):
    # in place when a row is a multiple of 16 bytes, a padded copy
    # otherwise; M beyond the prepared kernel runs it over row blocks, with
    # the tanh-GELU split and the residual following the global flat index.
    import torch
    e = rnd(681, n, k, 0.05)
    a = rnd(682 + m, m, k)
    bias = synth.normal(683, n, 0.0, 0.5)
    x = rnd(684, m, n)
    for fmt, rows, ldw, scale, bdeq, tol in _rows_cases(orc, e):
        R, A, Bias, X = _dev(rows), _dev(a), _dev(bias), _dev(x)
        C = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
        h = _abi.prepare_rows_dev(fmt, k, n, R.data_ptr(), ldw, scale)
        try:
            _abi.gemm_prepared(h, m, A.data_ptr(), C.data_ptr())
            torch.cuda.synchronize()
            ref = orc.matmul(a, bdeq)
            assert rel_err(C.cpu().numpy(), ref) <= tol, (fmt, "plain")
            _abi.gemm_prepared_ex(h, m, A.data_ptr(), C.data_ptr(), bias_ptr=Bias.data_ptr(),
                                  residual_ptr=X.data_ptr(), act=_abi.ACT_GELU_TANH)
            torch.cuda.synchronize()
            ref = orc.gelu_tanh(orc.matmul_bias(a, bdeq, bias) + x)
            assert rel_err(C.cpu().numpy(), ref) <= tol, (fmt, "epilogue")
        finally:
            _abi.prepared_free(h)


def test_prepared_rows_in_place_and_errors(orc):
    # An aligned f32 embedding is used where it lies: a later change to it
    # shows in the product.  Odd K for Q4_0 rows and a short stride are
    # rejected.
    import torch
    n, k, m = 256, 64, 1
    e, a = rnd(691, n, k), rnd(692, m, k)
    E, A = _dev(e), _dev(a)
    C = torch.empty((m, n), dtype=torch.float32, device="cuda:0")
    h = _abi.prepare_rows_dev(_abi.FMT_F32, k, n, E.data_ptr(), 4 * k)
    try:
        E.mul_(2.0)
        _abi.gemm_prepared(h, m, A.data_ptr(), C.data_ptr())
        torch.cuda.synchronize()
        assert rel_err(C.cpu().numpy(), orc.matmul(a, 2.0 * e.T.copy())) <= FP32_TOL
    finally:
        _abi.prepared_free(h)
    with pytest.raises(_abi.TmlError) as ex:
        _abi.prepare_rows_dev(_abi.FMT_Q4_0, 65, n, E.data_ptr(), 33)
    assert ex.value.code == _abi.TML_ERR_INVALID_SHAPE
    with pytest.raises(_abi.TmlError) as ex:
        _abi.prepare_rows_dev(_abi.FMT_F32, k, n, E.data_ptr(), 4 * k - 4)
    assert ex.value.code == _abi.TML_ERR_INVALID_ARG


# --------------------------------------------- staged (16-byte) GEMM epilogue
@pytest.mark.parametrize("tile", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
def test_staged_epilogue(orc, forced_env, tile):
    # Every tile writes C through LDS in 16-byte pieces, in passes of BK
    # columns where BN > BK (128x128, 128x64, 64x64, 256x128, 32x64 at BK 32:
    # two or four passes; 128x64, 64x64, 32x64 at BK 64 and 96x32: one; the
    # two-group 32x64 and 32x32 at BK 64: one, by wave group 0 alone).
    # Every epilogue term (alpha, beta * C, bias, residual, GELU, per-column
    # scales) on ragged M and N (N a multiple of 4 but not of the tile):
    # against the oracle, and against the 4-byte epilogue within rounding.
    import torch
    forced_env["TML_GEMM_DMA_TILE"] = str(tile)
    forced_env["TML_GEMM_DMA_Q"] = "1"
    m, n, k = 203, 340, 516
    a, w, c0, r = rnd(681, m, k), rnd(682, k, n, 0.05), rnd(683, m, n), rnd(684, m, n)
    bias = synth.normal(685, n, 0.0, 0.5)
    qc, sc = orc.quantize_q8_cols(w)
    cases = [(_abi.FMT_F32, w, None, orc.matmul(a, w)),
             (_abi.FMT_Q8_0_PC, qc, sc, orc.matmul_cols(a, 17, qc, sc, k, n))]
    for fmt, b, scales, prod in cases:
        ref = orc.gelu_exact(0.75 * prod - 0.5 * c0 + bias + r)
        got = {}
        for staged in ("1", "0"):
            forced_env["TML_GEMM_VEC_EPI"] = staged
            A, B, C, R, Bias = _dev(a), _dev(b), _dev(c0), _dev(r), _dev(bias)
            S = _dev(scales) if scales is not None else None
            _abi.gemm_ex_dev(fmt, m, n, k, A.data_ptr(), B.data_ptr(), C.data_ptr(), act=_abi.ACT_GELU_ERF,
                             residual_ptr=R.data_ptr(), scales_ptr=S.data_ptr() if S is not None else None,
                             bias_ptr=Bias.data_ptr(), alpha=0.75, beta=-0.5)
            torch.cuda.synchronize()
            got[staged] = C.cpu().numpy()
        tol = FP32_TOL if fmt == _abi.FMT_F32 else Q_TOL
        assert rel_err(got["1"], ref) <= tol, (tile, fmt, rel_err(got["1"], ref))
        assert rel_err(got["1"], got["0"]) <= 1e-6, (tile, fmt)
