"""GPU parity of the per-output-column formats (TML_FMT_Q8_0_PC / Q4_0_PC).

An extension, not a reference format: the reference quantizes per tensor
(Q8_0, Q4_0) or per 32 elements (Q8_K); the benchmark configurations ask for
"symmetric int8 with a per-output-row fp32 scale".  Column n of W[K,N] is
quantized by the reference's per-tensor quantizer applied to that column
alone (bitwise against the oracle), and products are checked against the
reference's dequantize-then-f32-accumulate semantics with column n's scale
(oracle.matmul_cols) at the quantized tolerance, 1e-3, through every kernel
family: [K,N] GEMV, prepared GEMV (register and LDS-staged), register-staged
GEMM, direct-copy GEMM with and without its split-K reduce, and the
host-pointer path on a registered weight.
"""
import os

import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu

Q_TOL = 1e-3
FMTS = [_abi.FMT_Q8_0_PC, _abi.FMT_Q4_0_PC]


def rnd(seed, m, n, std=1.0):
    return synth.normal_matrix(seed, m, n, std)


def _weights(seed, k, n):
    # columns of very different magnitude, so a per-tensor scale would lose them
    w = rnd(seed, k, n, 0.02) * np.exp(synth.normal(seed + 1, n, 0.0, 1.0))[None, :].astype(np.float32)
    return np.ascontiguousarray(w.astype(np.float32))


def _quant(orc, fmt, w):
    return orc.quantize_q8_cols(w) if fmt == _abi.FMT_Q8_0_PC else orc.quantize_q4_cols(w)


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


@pytest.fixture
def env():
    keys = ("TML_GEMM_SPLIT", "TML_GEMM_DMA_TILE", "TML_GEMM_DMA_Q", "TML_GEMVT_LDS")
    saved = {key: os.environ.get(key) for key in keys}
    yield os.environ
    for key, v in saved.items():
        if v is None:
            os.environ.pop(key, None)
        else:
            os.environ[key] = v


@pytest.mark.parametrize("fmt", FMTS)
def test_quantize_cols_bitwise(orc, fmt):
    import torch
    for (k, n) in [(1024, 96), (37, 11), (300, 130)]:
        w = _weights(201, k, n)
        w[:, 3] = 0.0
        q_ref, s_ref = _quant(orc, fmt, w)
        nbytes = q_ref.size
        q = np.zeros(nbytes, np.uint8)
        s = np.zeros(n, np.float32)
        _abi.quantize_cols(fmt, w, q, s)
        np.testing.assert_array_equal(q, q_ref.reshape(-1).view(np.uint8))
        np.testing.assert_array_equal(s, s_ref)
        W = _dev(w)
        Q = torch.zeros(nbytes, dtype=torch.uint8, device="cuda:0")
        S = torch.zeros(n, dtype=torch.float32, device="cuda:0")
        _abi.quantize_cols_dev(fmt, k, n, W.data_ptr(), Q.data_ptr(), S.data_ptr())
        torch.cuda.synchronize()
        np.testing.assert_array_equal(Q.cpu().numpy(), q_ref.reshape(-1).view(np.uint8))
        np.testing.assert_array_equal(S.cpu().numpy(), s_ref)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("m", [1, 3, 8, 64, 300])
def test_gemm_cols_vs_oracle(orc, fmt, m):
    k, n = 512, 320
    w = _weights(211, k, n)
    q, s = _quant(orc, fmt, w)
    a = rnd(212 + m, m, k)
    bias = synth.normal(213, n, 0.0, 0.5)
    got = np.zeros((m, n), np.float32)
    _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(q), got, scales=s, bias=bias)
    ref = orc.matmul_cols(a, fmt, q, s, k, n) + bias
    assert rel_err(got, ref) <= Q_TOL, rel_err(got, ref)


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("split", [1, 3])
def test_gemm_cols_direct_copy(orc, env, fmt, split):
    # the direct-copy kernel (forced at M < 1024, and at M = 1100 by the
    # planner), split-K reduce with the column scales on its 4-wide path
    env["TML_GEMM_DMA_Q"] = "1"
    env["TML_GEMM_SPLIT"] = str(split)
    k, n = 1024, 256
    w = _weights(221, k, n)
    q, s = _quant(orc, fmt, w)
    for m in (200, 1100):
        a = rnd(222, m, k)
        got = np.zeros((m, n), np.float32)
        _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(q), got, scales=s)
        ref = orc.matmul_cols(a, fmt, q, s, k, n)
        assert rel_err(got, ref) <= Q_TOL, (m, rel_err(got, ref))


@pytest.mark.parametrize("fmt", FMTS)
@pytest.mark.parametrize("lds", ["0", "1"])
def test_prepared_cols(orc, env, fmt, lds):
    import torch
    env["TML_GEMVT_LDS"] = lds
    k, n = 1280, 640
    w = _weights(231, k, n)
    q, s = _quant(orc, fmt, w)
    Q, S = _dev(q), _dev(s)
    h = _abi.prepare_ex_dev(fmt, k, n, Q.data_ptr(), scales_ptr=S.data_ptr())
    try:
        for m in (1, 2, 4, 8, 9):
            a = rnd(232 + m, m, k)
            A = _dev(a)
            C = torch.zeros((m, n), dtype=torch.float32, device="cuda:0")
            _abi.gemm_prepared(h, m, A.data_ptr(), C.data_ptr())
            torch.cuda.synchronize()
            ref = orc.matmul_cols(a, fmt, q, s, k, n)
            assert rel_err(C.cpu().numpy(), ref) <= Q_TOL, (m, rel_err(C.cpu().numpy(), ref))
    finally:
        _abi.prepared_free(h)
    with pytest.raises(_abi.TmlError):
        _abi.prepare_dev(fmt, k, n, Q.data_ptr())  # per-channel needs its scales


def test_registered_cols_weight(orc):
    # Host-pointer calls on a registered per-channel weight build a prepared
    # copy with the column scales; new scales for the same weight rebuild it.
    # The result equals the prepared kernel's bit for bit (tml_hip_prepare_ex_dev
    # on the same bytes and scales) and differs from the [K,N] kernel's,
    # which sums in another order: the prepared copy is what ran.
    import torch
    fmt = _abi.FMT_Q8_0_PC
    k, n = 640, 384
    w = _weights(241, k, n)
    q, s = _quant(orc, fmt, w)
    q = np.ascontiguousarray(q)
    a = rnd(242, 1, k)
    expect = []
    for scales in (s, s * 2.0):
        sc = np.ascontiguousarray(scales, dtype=np.float32)
        kn = np.zeros((1, n), np.float32)
        _abi.gemm(fmt, 1, n, k, a, q, kn, scales=sc)  # unregistered: the [K,N] kernel
        B, S, A = (torch.from_numpy(v).cuda() for v in (q.reshape(-1).view(np.uint8), sc, a))
        C = torch.zeros((1, n), dtype=torch.float32, device="cuda")
        h = _abi.prepare_ex_dev(fmt, k, n, B.data_ptr(), scales_ptr=S.data_ptr())
        try:
            _abi.gemm_prepared(h, 1, A.data_ptr(), C.data_ptr())
            torch.cuda.synchronize()
        finally:
            _abi.prepared_free(h)
        expect.append((sc, kn, C.cpu().numpy()))
    _abi.weight_register(q)
    try:
        for sc, kn, prep in expect:
            got = np.zeros((1, n), np.float32)
            _abi.gemm(fmt, 1, n, k, a, q, got, scales=sc)
            np.testing.assert_array_equal(got, prep)
            assert not np.array_equal(got, kn)
            assert rel_err(got, orc.matmul_cols(a, fmt, q, sc, k, n)) <= Q_TOL
    finally:
        _abi.weight_release(q)


@pytest.mark.parametrize("cls", ["q8", "q4"])
def test_python_mirror_cols(orc, cls):
    # quantizeCols{Q8,Q4} -> matmulWithWeight / ...Bias / ...BiasGelu, the
    # dispatch a layer would take with a per-column weight.
    from tomoul_amd import dispatch, ops, quantization as qz
    from tomoul_amd.tensor import Tensor
    k, n, m = 384, 256, 5
    w = _weights(251, k, n)
    wt = (qz.quantizeColsQ8 if cls == "q8" else qz.quantizeColsQ4)(Tensor.from_numpy(w))
    fmt = _abi.FMT_Q8_0_PC if cls == "q8" else _abi.FMT_Q4_0_PC
    q_ref, s_ref = _quant(orc, fmt, w)
    np.testing.assert_array_equal(wt.scales, s_ref)
    np.testing.assert_array_equal(wt.data.view(np.uint8), q_ref.reshape(-1).view(np.uint8))
    assert wt.sizeBytes() == 4 * n + q_ref.size
    a = rnd(252, m, k)
    bias = synth.normal(253, n, 0.0, 0.5)
    ref = orc.matmul_cols(a, fmt, q_ref, s_ref, k, n)
    x, b = Tensor.from_numpy(a), Tensor.from_numpy(bias)
    assert rel_err(dispatch.matmulWithWeight(x, wt).numpy(), ref) <= Q_TOL
    assert rel_err(dispatch.matmulWithWeightBias(x, wt, b).numpy(), ref + bias) <= Q_TOL
    got = dispatch.matmulWithWeightBiasGelu(x, wt, b).numpy()
    assert rel_err(got, orc.gelu_tanh(ref + bias)) <= Q_TOL
    with pytest.raises(qz.InvalidShape):
        qz.quantizeColsQ8(Tensor.from_numpy(w.reshape(-1)))


# The shapes and row counts the benchmark times for the per-column reading of
# configs 3 and 4, with its weights (seed 2002, 2003 for 5120 x 1280): each
# plan it times has its own oracle check, on the prepared copy and on the
# [K,N] layout, after the column quantizer is checked bitwise.
TIMED = [(_abi.FMT_Q8_0_PC, 1024, 4096, 2002, (1, 8, 128, 512)),
         (_abi.FMT_Q4_0_PC, 1280, 5120, 2002, (1, 4, 8)),
         (_abi.FMT_Q4_0_PC, 5120, 1280, 2003, (1, 4, 8))]


@pytest.mark.parametrize("fmt,k,n,seed,ms", TIMED, ids=["q8pc_1024x4096", "q4pc_1280x5120", "q4pc_5120x1280"])
def test_cols_at_timed_shapes(orc, fmt, k, n, seed, ms):
    import torch
    w = synth.normal_matrix(seed, k, n, 0.02)
    q_ref, s_ref = _quant(orc, fmt, w)
    W = _dev(w)
    Q = torch.zeros(_abi.weight_bytes(fmt, k, n), dtype=torch.uint8, device="cuda:0")
    S = torch.zeros(_abi.scale_count(fmt, k, n), dtype=torch.float32, device="cuda:0")
    _abi.quantize_cols_dev(fmt, k, n, W.data_ptr(), Q.data_ptr(), S.data_ptr())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(Q.cpu().numpy(), q_ref.reshape(-1).view(np.uint8))
    np.testing.assert_array_equal(S.cpu().numpy(), s_ref)
    h = _abi.prepare_ex_dev(fmt, k, n, Q.data_ptr(), scales_ptr=S.data_ptr())
    try:
        for m in ms:
            a = synth.normal_matrix(1001, m, k)
            ref = orc.matmul_cols(a, fmt, q_ref, s_ref, k, n)
            A = _dev(a)
            for path in ("prepared", "kn"):
                C = torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
                if path == "prepared":
                    _abi.gemm_prepared(h, m, A.data_ptr(), C.data_ptr())
                else:
                    _abi.gemm_dev(fmt, m, n, k, A.data_ptr(), Q.data_ptr(), C.data_ptr(), scales_ptr=S.data_ptr())
                torch.cuda.synchronize()
                err = rel_err(C.cpu().numpy(), ref)
                print(f"{fmt} {k}x{n} M={m} {path}: rel {err:.2e}", flush=True)
                assert err <= Q_TOL, (m, path, err)
    finally:
        _abi.prepared_free(h)
