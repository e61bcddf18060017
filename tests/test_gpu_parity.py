"""GPU parity: the HIP path (through the C ABI) against the CPU oracle.

Tolerances: fp32 paths max relative error
max|G-R|/max|R| <= 1e-4 against the reference's fp32 fallback semantics;
quantized paths <= 1e-3 against the reference's dequantize-then-fp32-
accumulate scalar loops (matmulF32Q8 / Q8K / Q4).  Quantizers and integer
products are compared bitwise.
"""
import os

import numpy as np
import pytest

from conftest import elementwise_ok, rel_err
from tomoul_amd import _abi, ops, quantization as qz, synth
from tomoul_amd.tensor import Tensor

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
Q_TOL = 1e-3
NT = min(16, os.cpu_count() or 1)


def T(a):
    return Tensor.from_numpy(np.asarray(a, dtype=np.float32))


def rnd(seed, m, n, std=1.0):
    return synth.normal_matrix(seed, m, n, std)


# ------------------------------------------------------------- reference KATs
def test_kat_matmul_2x3_3x2():
    # src/core/ops.zig:969-1005
    c = ops.matmul(T([[1, 2, 3], [4, 5, 6]]), T([[7, 8], [9, 10], [11, 12]]))
    assert c.shape == (2, 2)
    assert c.data.tolist() == [58.0, 64.0, 139.0, 154.0]


def test_kat_linear_compat():
    # src/core/ops.zig:937-967: [1,1,1] . W^T with W = [[1,2,3],[4,5,6]]
    w_t = np.array([[1, 2, 3], [4, 5, 6]], dtype=np.float32).T.copy()
    c = ops.matmul(T([[1, 1, 1]]), T(w_t))
    assert c.data.tolist() == [6.0, 15.0]


def test_kat_identity_and_demo():
    # src/core/ops.zig:1023-1046 and src/main.zig:141-148
    assert ops.matmul(T([[1, 2], [3, 4]]), T([[1, 0], [0, 1]])).data.tolist() == [1, 2, 3, 4]
    assert ops.matmul(T([[1, 2, 3]]), T([[1, 2], [3, 4], [5, 6]])).data.tolist() == [22.0, 28.0]


def test_kat_matvec():
    # src/core/ops.zig:1048-1076
    y = ops.matvec(T([[1, 2, 3], [4, 5, 6]]), Tensor.initWithData((3,), [1, 2, 3]))
    assert y.shape == (2,) and y.data.tolist() == [14.0, 32.0]


def test_shape_errors_before_device():
    # src/core/ops.zig:1007-1021
    with pytest.raises(ops.OpsError.ShapeMismatch):
        ops.matmul(Tensor.init((2, 3)), Tensor.init((2, 2)))
    with pytest.raises(ops.OpsError.InvalidShape):
        ops.matmul(Tensor.init((2, 3, 1)), Tensor.init((3, 2)))
    with pytest.raises(ops.OpsError.ShapeMismatch):
        ops.matmulBias(Tensor.init((2, 3)), Tensor.init((3, 2)), Tensor.init((3,)))


def test_abi_error_codes():
    a = np.zeros((2, 2), np.float32)
    with pytest.raises(_abi.TmlError) as e:
        _abi.sgemm(-1, 2, 2, a, a, a)
    assert e.value.code == _abi.TML_ERR_INVALID_SHAPE
    with pytest.raises(_abi.TmlError) as e:
        _abi.check(_abi.lib().tml_hip_gemm_dev(9, 2, 2, 2, 1, 1, 1.0, None, 32, None, 1, 1.0, 0.0, None))
    assert e.value.code == _abi.TML_ERR_INVALID_FORMAT
    _abi.sgemm(0, 5, 3, a, a, a)  # empty output: no-op


def test_exact_small_integers(orc):
    # Products of small integers are exact in f32 whatever the summation
    # order, so the GPU result must equal the oracle bitwise.
    rng = np.random.default_rng(7)
    for (m, n, k) in [(5, 7, 9), (64, 64, 64), (130, 70, 50), (3, 1000, 40)]:
        a = rng.integers(-4, 5, size=(m, k)).astype(np.float32)
        b = rng.integers(-4, 5, size=(k, n)).astype(np.float32)
        got = ops.matmul(T(a), T(b)).numpy()
        np.testing.assert_array_equal(got, orc.matmul(a, b))


# ------------------------------------------------------------------ fp32 GEMM
FP32_SHAPES = [
    (1, 1, 1), (1, 4096, 1024), (2, 33, 17), (4, 100, 64), (8, 1280, 5120), (9, 64, 64),
    (17, 33, 65), (64, 64, 64), (100, 200, 300), (128, 128, 128), (127, 129, 131),
    (1500, 1536, 384),                     # config 1 (Whisper-tiny MLP)
    (512, 3072, 1024), (512, 1024, 1024),  # config 2 (XLM-R large)
    (512, 4096, 1024), (512, 1024, 4096),
]


@pytest.mark.parametrize("m,n,k", FP32_SHAPES)
def test_sgemm_vs_oracle(orc, m, n, k):
    a = rnd(1001, m, k)
    b = rnd(2002, k, n, 0.02)
    ref = orc.matmul_mt(a, b, NT)
    got = ops.matmul(T(a), T(b)).numpy()
    err = rel_err(got, ref)
    print(f"sgemm {m}x{n}x{k}: rel {err:.3e}")
    assert err <= FP32_TOL
    assert elementwise_ok(got, ref, 1e-4)


def test_sgemm_bias_config1(orc):
    a, b = rnd(1001, 1500, 384), rnd(2002, 384, 1536, 0.02)
    bias = synth.normal(3003, 1536, 0.0, 0.02)
    ref = orc.matmul_bias(a, b, bias)
    got = ops.matmulBias(T(a), T(b), Tensor.from_numpy(bias)).numpy()
    assert rel_err(got, ref) <= FP32_TOL


@pytest.mark.parametrize("m", [1, 3, 8, 40])
def test_sgemm_bias_small(orc, m):
    a, b = rnd(11, m, 96), rnd(12, 96, 130, 0.02)
    bias = synth.normal(13, 130, 0.0, 0.02)
    got = ops.matmulBias(T(a), T(b), Tensor.from_numpy(bias)).numpy()
    assert rel_err(got, orc.matmul_bias(a, b, bias)) <= FP32_TOL


@pytest.mark.parametrize("m,n,k", [(4, 64, 32), (70, 96, 48)])
@pytest.mark.parametrize("alpha,beta", [(1.0, 0.0), (0.5, 2.0), (-1.0, 1.0)])
def test_sgemm_alpha_beta(orc, m, n, k, alpha, beta):
    a, b = rnd(21, m, k), rnd(22, k, n)
    c0 = rnd(23, m, n)
    c = c0.copy()
    _abi.sgemm(m, n, k, a, b, c, alpha, beta)
    ref = orc.sgemm(a, b, c0, alpha, beta)
    assert rel_err(c, ref) <= FP32_TOL


def test_sgemm_beta_zero_ignores_nan(orc):
    a, b = rnd(31, 10, 20), rnd(32, 20, 30)
    c = np.full((10, 30), np.nan, np.float32)
    _abi.sgemm(10, 30, 20, a, b, c, 1.0, 0.0)
    assert np.isfinite(c).all()


def test_sgemv_vs_oracle(orc):
    a = rnd(41, 300, 517)
    x = synth.normal(42, 517)
    y = np.zeros(300, np.float32)
    _abi.sgemv(300, 517, a, x, y)
    assert rel_err(y, orc.matvec(a, x)) <= FP32_TOL


def test_unaligned_views(orc):
    # Operands that are not 16-byte aligned take the generic path.
    buf_a = np.zeros(1 + 33 * 20, np.float32)
    buf_b = np.zeros(1 + 20 * 44, np.float32)
    a = buf_a[1:].reshape(33, 20)
    b = buf_b[1:].reshape(20, 44)
    a[:] = rnd(51, 33, 20)
    b[:] = rnd(52, 20, 44)
    assert a.ctypes.data % 16 != 0
    c = np.zeros((33, 44), np.float32)
    _abi.sgemm(33, 44, 20, a, b, c)
    assert rel_err(c, orc.matmul(a, b)) <= FP32_TOL


# ------------------------------------------------------------- quantizers
@pytest.mark.parametrize("n", [1, 31, 32, 33, 1000, 1024 * 4096])
def test_quantize_q8_bitexact(orc, n):
    w = synth.normal(2002, n, 0.0, 0.02)
    q_ref, s_ref = orc.quantize_q8(w)
    q = qz.quantizeQ8(Tensor(w, (n,)))
    assert np.float32(q.scale) == np.float32(s_ref)
    np.testing.assert_array_equal(q.data, q_ref)


@pytest.mark.parametrize("n", [1, 7, 8, 1001, 1280 * 5120])
def test_quantize_q4_bitexact(orc, n):
    w = synth.normal(2003, n, 0.0, 0.02)
    p_ref, s_ref = orc.quantize_q4(w)
    q = qz.quantizeQ4(Tensor(w, (n,)))
    assert np.float32(q.scale) == np.float32(s_ref)
    np.testing.assert_array_equal(q.data, p_ref)


@pytest.mark.parametrize("n", [1, 32, 100, 64 * 32, 1024 * 4096 + 17])
def test_quantize_q8k_bitexact(orc, n):
    w = synth.normal(2004, n, 0.0, 0.02)
    w[: min(n, 32)] = 0.0  # an all-zero first block -> scale 1
    q_ref, s_ref = orc.quantize_q8k(w)
    q = qz.quantizeQ8K(Tensor(w, (n,)))
    np.testing.assert_array_equal(q.scales, s_ref)
    np.testing.assert_array_equal(q.data, q_ref)


def test_quantize_kats():
    # quantization.zig:1022-1038, 1120-1144, 1239-1255, 1337-1360 and the
    # half-away-from-zero tie rule (127 * 0.5/127 = 0.5 -> 1, -0.5 -> -1).
    q = qz.quantizeQ8(Tensor.initWithData((5,), [100, -100, 0, 50, -50]))
    assert q.data[:3].tolist() == [127, -127, 0]
    assert abs(q.scale - 100 / 127) < 1e-4
    z = qz.quantizeQ8(Tensor.init((10,)))
    assert z.scale == 1.0 and not z.data.any()
    q4 = qz.quantizeQ4(Tensor.initWithData((5,), [100, -100, 0, 50, -50]))
    assert [q4.get(i) for i in range(3)] == [7, -7, 0]
    assert abs(q4.scale - 100 / 7) < 1e-4
    z4 = qz.quantizeQ4(Tensor.init((10,)))
    assert z4.scale == 1.0 and not z4.data.any()
    t = qz.quantizeQ8(Tensor.initWithData((3,), [127.0, 0.5, -0.5]))
    assert t.data.tolist() == [127, 1, -1]


# ------------------------------------------------------ weight-only matmuls
Q8_CASES = [(1, 4096, 1024), (8, 4096, 1024), (128, 4096, 1024), (512, 4096, 1024),  # config 3
            (3, 100, 50), (16, 96, 70), (4, 16, 32)]


@pytest.mark.parametrize("m,n,k", Q8_CASES)
def test_q8_vs_oracle(orc, m, n, k):
    a = rnd(1001, m, k)
    w = rnd(2002, k, n, 0.02)
    q, s = orc.quantize_q8(w)
    ref = orc.matmul_q8_mt(a, q, s, NT)
    got = qz.matmulF32Q8Simd(T(a), qz.QuantizedTensorQ8(s, q, (k, n))).numpy()
    err = rel_err(got, ref)
    print(f"q8 {m}x{n}x{k}: rel {err:.3e}")
    assert err <= Q_TOL


Q4_CASES = [(1, 5120, 1280), (4, 5120, 1280), (8, 5120, 1280),   # config 4
            (1, 1280, 5120), (4, 1280, 5120), (8, 1280, 5120),
            (5, 33, 20), (40, 130, 64), (128, 5120, 1280)]


@pytest.mark.parametrize("m,n,k", Q4_CASES)
def test_q4_vs_oracle(orc, m, n, k):
    a = rnd(1001, m, k)
    w = rnd(2002, k, n, 0.02)
    p, s = orc.quantize_q4(w)
    ref = orc.matmul_q4_mt(a, p, k, n, s, NT)
    got = qz.matmulF32Q4Simd(T(a), qz.QuantizedTensorQ4(s, p, (k, n))).numpy()
    err = rel_err(got, ref)
    print(f"q4 {m}x{n}x{k}: rel {err:.3e}")
    assert err <= Q_TOL


Q8K_CASES = [(1, 4096, 1024), (8, 512, 512), (16, 512, 512), (4, 32, 64), (130, 96, 40), (2, 33, 7)]


@pytest.mark.parametrize("m,n,k", Q8K_CASES)
def test_q8k_vs_oracle(orc, m, n, k):
    a = rnd(1001, m, k)
    w = rnd(2002, k, n, 0.02)
    q, sc = orc.quantize_q8k(w)
    ref = orc.matmul_q8k(a, q, sc, 32)
    got = qz.matmulF32Q8KSimd(T(a), qz.QuantizedTensorQ8K(sc, q, (k, n))).numpy()
    err = rel_err(got, ref)
    print(f"q8k {m}x{n}x{k}: rel {err:.3e}")
    assert err <= Q_TOL


def test_q4_exact_integer_products(orc):
    # Integer activations times int4 weights with scale 1: every partial sum
    # is an integer below 2^24, so the GPU result must be exact.
    rng = np.random.default_rng(3)
    for m in (1, 4, 8, 33):
        k, n = 256, 512
        a = rng.integers(-8, 9, size=(m, k)).astype(np.float32)
        qv = rng.integers(-7, 8, size=k * n)
        p = np.zeros((k * n + 1) // 2, np.uint8)
        for i in range(0, k * n, 2):
            p[i // 2] = (qv[i] & 0xF) | ((qv[i + 1] & 0xF) << 4)
        got = np.zeros((m, n), np.float32)
        _abi.sgemm_q4(m, n, k, a, p, 1.0, got)
        np.testing.assert_array_equal(got, orc.matmul_q4(a, p, k, n, 1.0))


def test_gemv_deterministic():
    a = rnd(61, 1, 1024)
    w = rnd(62, 1024, 4096, 0.02)
    q = qz.quantizeQ8(Tensor.from_numpy(w))
    r0 = qz.matmulF32Q8Simd(T(a), q).data.copy()
    for _ in range(5):
        np.testing.assert_array_equal(qz.matmulF32Q8Simd(T(a), q).data, r0)


def test_registered_weight_path(orc):
    # A registered (resident) weight gives the uploaded weight's result: the
    # same kernel bit for bit at M = 9 (the [K,N] GEMM on the resident copy),
    # and to tolerance at M = 8, where the resident weight goes through its
    # prepared copy (another summation order).
    w = rnd(72, 512, 768, 0.02)
    q, s = orc.quantize_q8(w)
    for m in (8, 9):
        a = rnd(71, m, 512)
        c0 = np.zeros((m, 768), np.float32)
        _abi.sgemm_q8(m, 768, 512, a, q, s, c0)
        _abi.weight_register(q)
        try:
            c1 = np.zeros((m, 768), np.float32)
            _abi.sgemm_q8(m, 768, 512, a, q, s, c1)
        finally:
            _abi.weight_release(q)
        if m == 9:
            np.testing.assert_array_equal(c0, c1)
        assert rel_err(c1, c0) <= Q_TOL and rel_err(c1, orc.matmul_q8(a, q, s)) <= Q_TOL


# ------------------------------------------------------- forced kernel plans
@pytest.fixture
def forced_env():
    saved = {k: os.environ.get(k) for k in ("TML_GEMM_SPLIT", "TML_GEMM_DMA_TILE", "TML_GEMM_DMA", "TML_GEMM_TILE", "TML_GEMM_FUSED",
                                   "TML_GEMM_DMA_Q")}
    yield os.environ
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
@pytest.mark.parametrize("split", [1, 2, 3, 8])
def test_sgemm_dma_tiles_and_splits(orc, forced_env, tile, split):
    # Every tile config of the direct-copy kernel with K split 1-8 ways,
    # on ragged shapes (M, N not multiples of the tile; K % 32 != 0).
    forced_env["TML_GEMM_DMA_TILE"] = str(tile)
    forced_env["TML_GEMM_SPLIT"] = str(split)
    for (m, n, k) in [(300, 260, 516), (129, 68, 1028), (512, 1024, 1024)]:
        a, b = rnd(81, m, k), rnd(82, k, n, 0.02)
        bias = synth.normal(83, n, 0.0, 0.02)
        got = ops.matmulBias(T(a), T(b), Tensor.from_numpy(bias)).numpy()
        err = rel_err(got, orc.matmul_bias(a, b, bias))
        assert err <= FP32_TOL, (m, n, k, err)


@pytest.mark.parametrize("tile", [1, 2, 4, 5, 7, 8, 9, 10, 11])
@pytest.mark.parametrize("split", [2, 3, 8])
def test_sgemm_fused_split_equals_two_launch(forced_env, tile, split):
    # Split-K partials combined inside the GEMM (last split to arrive sums
    # them in split order) give the two-launch reduce's result bit for bit,
    # with the fused epilogue (bias, residual, activation) on top.  Tiles 10
    # and 11 (two wave groups along K) have no fused exchange: the request
    # falls back to the two-launch reduce.
    forced_env["TML_GEMM_DMA_TILE"] = str(tile)
    forced_env["TML_GEMM_SPLIT"] = str(split)
    m, n, k = 300, 260, 1028
    a, b = rnd(97, m, k), rnd(98, k, n, 0.02)
    bias = synth.normal(99, n, 0.0, 0.02)
    res = rnd(100, m, n)
    out = {}
    for fused in ("1", "0"):
        forced_env["TML_GEMM_FUSED"] = fused
        c = np.zeros((m, n), np.float32)
        _abi.gemm_residual(_abi.FMT_F32, m, n, k, a, b, res, c, bias=bias)
        g = np.zeros((m, n), np.float32)
        _abi.gemm_act(_abi.FMT_F32, m, n, k, a, b, g, act=_abi.ACT_GELU_TANH, bias=bias)
        out[fused] = (c, g)
    np.testing.assert_array_equal(out["1"][0], out["0"][0])
    np.testing.assert_array_equal(out["1"][1], out["0"][1])


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
@pytest.mark.parametrize("split", [1, 3])
def test_qgemm_dma_tiles(orc, forced_env, tile, split):
    # F16 / Q8_0 / Q4_0 / Q8_K weights through the direct-copy kernel (raw
    # bytes staged in LDS, widened on the fragment read; Q8_K's block scales
    # staged beside them), every tile config, K
    # split or not, on ragged M and K (N a multiple of 32 so int4 rows are
    # 16-byte aligned); the register-staged kernel gives the same result to
    # rounding.  Tiles 9 (96x32) and 11 (32x32) have no int4 variant: the
    # planner ignores the forced tile for Q4_0 B and picks another.
    forced_env["TML_GEMM_DMA_TILE"] = str(tile)
    forced_env["TML_GEMM_SPLIT"] = str(split)
    m, n, k = 200, 320, 516
    a = rnd(171, m, k)
    w = rnd(172, k, n, 0.02)
    bias = synth.normal(173, n, 0.0, 0.02)
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    h = orc.to_f16(w)
    qk, sk = orc.quantize_q8k(w)
    cases = [(_abi.FMT_Q8_0, q, s, orc.matmul_q8(a, q, s), Q_TOL), (_abi.FMT_Q4_0, p, s4, orc.matmul_q4(a, p, k, n, s4), Q_TOL),
             (_abi.FMT_F16, h, 1.0, orc.matmul_f16(a, h), FP32_TOL),
             (_abi.FMT_Q8_K, qk, sk, orc.matmul_q8k(a, qk, sk), Q_TOL)]
    for fmt, b, scale, ref, tol in cases:
        out = {}
        kw = {"scales": np.ascontiguousarray(scale, np.float32), "block": 32} if fmt == _abi.FMT_Q8_K else {"scale": scale}
        for dma in ("1", "0"):
            forced_env["TML_GEMM_DMA_Q"] = dma
            got = np.zeros((m, n), np.float32)
            _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(b), got, bias=bias, **kw)
            out[dma] = got
            assert rel_err(got, ref + bias) <= tol, (fmt, dma, rel_err(got, ref + bias))
        assert rel_err(out["1"], out["0"]) <= 1e-5, fmt


def test_sgemm_split_deterministic(forced_env):
    forced_env["TML_GEMM_SPLIT"] = "8"
    a, b = rnd(91, 512, 4096), rnd(92, 4096, 1024, 0.02)
    r0 = ops.matmul(T(a), T(b)).data.copy()
    for _ in range(3):
        np.testing.assert_array_equal(ops.matmul(T(a), T(b)).data, r0)


def test_sgemm_register_staged_kernel(orc, forced_env):
    # The register-staged kernel (used for quantized B) on fp32 as well.
    forced_env["TML_GEMM_DMA"] = "0"
    for tile in ("1", "2", "3", "4", "5", "6", "7"):
        forced_env["TML_GEMM_TILE"] = tile
        a, b = rnd(95, 200, 136), rnd(96, 136, 264, 0.02)
        assert rel_err(ops.matmul(T(a), T(b)).numpy(), orc.matmul(a, b)) <= FP32_TOL, tile


# --------------------------------------------- weight-type dispatch (callers)
@pytest.mark.parametrize("m", [1, 7, 64])
def test_matmul_with_weight_bias_all_formats(orc, m):
    # matmulWithWeightBias (src/core/attention.zig:132-149): reference =
    # scalar weight-only matmul, then a separate bias add.
    from tomoul_amd import dispatch
    k, n = 96, 160
    a = rnd(101, m, k)
    w = rnd(102, k, n, 0.02)
    bias = synth.normal(103, n, 0.0, 0.02)
    tb = Tensor.from_numpy(bias)
    got = dispatch.matmulWithWeightBias(T(a), T(w), tb).numpy()
    assert rel_err(got, orc.matmul_bias(a, w, bias)) <= FP32_TOL
    q, s = orc.quantize_q8(w)
    got = dispatch.matmulWithWeightBias(T(a), qz.QuantizedTensorQ8(s, q, (k, n)), tb).numpy()
    assert rel_err(got, orc.matmul_q8(a, q, s) + bias) <= Q_TOL
    p, s4 = orc.quantize_q4(w)
    got = dispatch.matmulWithWeightBias(T(a), qz.QuantizedTensorQ4(s4, p, (k, n)), tb).numpy()
    assert rel_err(got, orc.matmul_q4(a, p, k, n, s4) + bias) <= Q_TOL
    qk, sk = orc.quantize_q8k(w)
    got = dispatch.matmulWithWeightBias(T(a), qz.QuantizedTensorQ8K(sk, qk, (k, n)), tb).numpy()
    assert rel_err(got, orc.matmul_q8k(a, qk, sk) + bias) <= Q_TOL
    got = dispatch.matmulWithWeight(T(a), qz.QuantizedTensorQ8(s, q, (k, n))).numpy()
    assert rel_err(got, orc.matmul_q8(a, q, s)) <= Q_TOL


# ---------------------------------------- GEMV plans (M <= 8), every variant
@pytest.fixture
def gemv_env():
    keys = ("TML_GEMV_LPR", "TML_GEMV_NB")
    saved = {k: os.environ.get(k) for k in keys}
    yield os.environ
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


@pytest.mark.parametrize("lpr", [1, 2, 4, 8, 16, 32, 64])
@pytest.mark.parametrize("nb", [1, 3])
def test_gemv_segments_and_splits(orc, gemv_env, lpr, nb):
    # Every segment width (lanes per row) and batches-per-split setting of
    # the GEMV, for every format and row count M = 1..8; K = 333 is ragged
    # for every batch height, so the last split is partial and, for most
    # settings, K is split over several workgroups (exchange path).
    gemv_env["TML_GEMV_LPR"] = str(lpr)
    gemv_env["TML_GEMV_NB"] = str(nb)
    k, n = 333, 640
    w = rnd(111, k, n, 0.02)
    bias = synth.normal(112, n, 0.0, 0.02)
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    qk, sk = orc.quantize_q8k(w)
    for m in (1, 2, 3, 5, 8):
        a = rnd(113 + m, m, k)
        cases = [
            (_abi.FMT_F32, w, 1.0, None, orc.matmul(a, w), FP32_TOL),
            (_abi.FMT_Q8_0, q, s, None, orc.matmul_q8(a, q, s), Q_TOL),
            (_abi.FMT_Q4_0, p, s4, None, orc.matmul_q4(a, p, k, n, s4), Q_TOL),
            (_abi.FMT_Q8_K, qk, 1.0, sk, orc.matmul_q8k(a, qk, sk, 32), Q_TOL),
        ]
        for fmt, b, scale, scales, ref, tol in cases:
            got = np.zeros((m, n), np.float32)
            _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(b), got, scale=scale, scales=scales, bias=bias)
            err = rel_err(got, ref + bias)
            assert err <= tol, (fmt, m, err)


@pytest.mark.parametrize("m", [1, 2, 3, 4])
def test_q8_kn_one_lane_a_row(orc, m):
    # Config 3's Q8_0 1024x4096 in the [K,N] layout at M <= 4: the planner's
    # one-lane-a-row plan (256 segments of 16 columns, all of K in one
    # batch, no K split), with a bias
    k, n = 1024, 4096
    w = rnd(141, k, n, 0.02)
    q, s = orc.quantize_q8(w)
    bias = synth.normal(142, n, 0.0, 0.02)
    a = rnd(143 + m, m, k)
    got = np.zeros((m, n), np.float32)
    _abi.gemm(_abi.FMT_Q8_0, m, n, k, a, q.reshape(k, n), got, scale=s, bias=bias)
    assert rel_err(got, orc.matmul_q8(a, q, s) + bias) <= Q_TOL


@pytest.mark.parametrize("m", [1, 4, 8])
def test_gemv_generic_path(orc, m):
    # Odd N (no vector loads possible) and a Q8_K block that does not divide
    # N take the element-wise path.
    k, n = 77, 45
    a = rnd(121, m, k)
    w = rnd(122, k, n, 0.02)
    got = ops.matmul(T(a), T(w)).numpy()
    assert rel_err(got, orc.matmul(a, w)) <= FP32_TOL
    q, s = orc.quantize_q8(w)
    got = qz.matmulF32Q8Simd(T(a), qz.QuantizedTensorQ8(s, q, (k, n))).numpy()
    assert rel_err(got, orc.matmul_q8(a, q, s)) <= Q_TOL
    p, s4 = orc.quantize_q4(w)
    got = qz.matmulF32Q4Simd(T(a), qz.QuantizedTensorQ4(s4, p, (k, n))).numpy()
    assert rel_err(got, orc.matmul_q4(a, p, k, n, s4)) <= Q_TOL
    qk, sk = orc.quantize_q8k(w)
    got = qz.matmulF32Q8KSimd(T(a), qz.QuantizedTensorQ8K(sk, qk, (k, n))).numpy()
    assert rel_err(got, orc.matmul_q8k(a, qk, sk, 32)) <= Q_TOL


def test_gemv_alpha_beta(orc):
    m, k, n = 3, 200, 256
    a, w = rnd(131, m, k), rnd(132, k, n, 0.02)
    c0 = rnd(133, m, n)
    got = c0.copy()
    _abi.sgemm(m, n, k, a, w, got, 0.5, -2.0)
    assert rel_err(got, 0.5 * orc.matmul(a, w) - 2.0 * c0) <= FP32_TOL


# ------------------------------------- prepared (K-contiguous) decoder weights
def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _prepared_cases(orc, w, k, n, a):
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    h = orc.to_f16(w)
    return [(_abi.FMT_F32, w, 1.0, orc.matmul(a, w), FP32_TOL),
            (_abi.FMT_Q8_0, q, s, orc.matmul_q8(a, q, s), Q_TOL),
            (_abi.FMT_Q4_0, p, s4, orc.matmul_q4(a, p, k, n, s4), Q_TOL),
            (_abi.FMT_F16, h, 1.0, orc.matmul_f16(a, h.reshape(k, n)), FP32_TOL)]


def _run_prepared(fmt, b, scale, k, n, m, a, bias=None, c0=None, alpha=1.0, beta=0.0):
    import torch
    B, A = _dev(b), _dev(a)
    h = _abi.prepare_dev(fmt, k, n, B.data_ptr(), scale)
    try:
        C = _dev(c0) if c0 is not None else torch.zeros((m, n), dtype=torch.float32, device="cuda:0")
        Bias = _dev(bias) if bias is not None else None
        _abi.gemm_prepared(h, m, A.data_ptr(), C.data_ptr(), bias_ptr=Bias.data_ptr() if Bias is not None else None,
                           alpha=alpha, beta=beta)
        torch.cuda.synchronize()
        return C.cpu().numpy()
    finally:
        _abi.prepared_free(h)


@pytest.mark.parametrize("k,n", [(1024, 4096), (1280, 5120), (5120, 1280), (5120, 96), (333, 640), (77, 45),
                                 (1, 3), (2100, 130), (9000, 40)])
@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9])
def test_prepared_vs_oracle(orc, k, n, m):
    # The prepared kernels cover M <= 8 (registers for small M x E, LDS-staged
    # activations beyond); M = 9 runs the [K,N] GEMM on the weight the copy
    # was made from.
    w = rnd(141, k, n, 0.02)
    a = rnd(142 + m, m, k)
    bias = synth.normal(143, n, 0.0, 0.02)
    for fmt, b, scale, ref, tol in _prepared_cases(orc, w, k, n, a):
        got = _run_prepared(fmt, b, scale, k, n, m, a, bias=bias)
        err = rel_err(got, ref + bias)
        assert err <= tol, (fmt, err)


@pytest.mark.parametrize("lk", [16, 64, 256])
@pytest.mark.parametrize("cw", [1, 2, 4])
@pytest.mark.parametrize("jb", [1, 2, 4])
def test_prepared_plan_variants(orc, lk, cw, jb):
    keys = ("TML_GEMVT_LK", "TML_GEMVT_CW", "TML_GEMVT_JB")
    saved = {key: os.environ.get(key) for key in keys}
    os.environ.update({"TML_GEMVT_LK": str(lk), "TML_GEMVT_CW": str(cw), "TML_GEMVT_JB": str(jb)})
    try:
        k, n = 1500, 70
        w = rnd(151, k, n, 0.02)
        for m in (1, 2, 3, 7):
            a = rnd(152 + m, m, k)
            for fmt, b, scale, ref, tol in _prepared_cases(orc, w, k, n, a):
                assert rel_err(_run_prepared(fmt, b, scale, k, n, m, a), ref) <= tol, (fmt, m)
    finally:
        for key, v in saved.items():
            if v is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = v


@pytest.mark.parametrize("lk", [16, 64, 256])
@pytest.mark.parametrize("cw", [1, 2, 4])
@pytest.mark.parametrize("jb", [1, 2])
def test_prepared_buffer_loads(orc, lk, cw, jb):
    # K a whole number of chunks takes the buffer-resource loads (chunks past
    # the row read unchecked and their sums are dropped); they must give the
    # checked loads' result bit for bit, with partial last batches (40, 80,
    # 320 chunks over 16-, 64- and 256-lane groups), several superchunks
    # (K = 3072: 3 of int8) and an inf in the activation row after row 0,
    # which the dropped sums of row 0 must not pick up.
    keys = ("TML_GEMVT_LK", "TML_GEMVT_CW", "TML_GEMVT_JB", "TML_GEMVT_BUF")
    saved = {key: os.environ.get(key) for key in keys}
    os.environ.update({"TML_GEMVT_LK": str(lk), "TML_GEMVT_CW": str(cw), "TML_GEMVT_JB": str(jb)})
    try:
        for (k, n) in [(1280, 200), (3072, 72)]:
            w = rnd(191, k, n, 0.02)
            for m in (1, 2):
                a = rnd(192 + m, m, k)
                if m == 2:
                    a[1, :7] = np.inf
                for fmt, b, scale, ref, tol in _prepared_cases(orc, w, k, n, a):
                    got = {}
                    for buf in ("1", "0"):
                        os.environ["TML_GEMVT_BUF"] = buf
                        got[buf] = _run_prepared(fmt, b, scale, k, n, m, a)
                    np.testing.assert_array_equal(got["1"], got["0"])
                    assert np.all(np.isfinite(got["1"][0])), (fmt, k, m)
                    assert rel_err(got["1"][:1], ref[:1]) <= tol, (fmt, k, m)
    finally:
        for key, v in saved.items():
            if v is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = v


@pytest.mark.parametrize("cw", [1, 2, 4])
def test_prepared_lds_kernel(orc, cw):
    # The LDS-staged prepared kernel (forced for every row count and format)
    # on several superchunks (K = 5000: 2.4 superchunks of int4, 4.9 of
    # int8), an odd K (element-wise activation loads) and ragged N.
    keys = ("TML_GEMVT_LDS", "TML_GEMVT_CW")
    saved = {key: os.environ.get(key) for key in keys}
    os.environ.update({"TML_GEMVT_LDS": "1", "TML_GEMVT_CW": str(cw)})
    try:
        for (k, n) in [(5000, 130), (77, 45), (1280, 600)]:
            w = rnd(181, k, n, 0.02)
            for m in (1, 2, 3, 5, 8):
                a = rnd(182 + m, m, k)
                for fmt, b, scale, ref, tol in _prepared_cases(orc, w, k, n, a):
                    assert rel_err(_run_prepared(fmt, b, scale, k, n, m, a), ref) <= tol, (k, n, m, fmt)
    finally:
        for key, v in saved.items():
            if v is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = v


@pytest.mark.parametrize("nw,it,t", [(1, 1, 1), (3, 2, 2), (10, 1, 1), (10, 2, 2), (16, 4, 1), (5, 4, 2), (16, 1, 2)])
def test_prepared_matrix_core_plans(orc, nw, it, t):
    # The matrix-core decoder GEMV (Q8_0 / Q4_0, M >= 2) under forced plans:
    # 1-16 waves, runs of 4 / 8 / 16 chunks, one or two 16-column tiles, on
    # several superchunks (K = 4160: 4 of int8 plus a partial one, 2 of int4
    # plus 2 chunks) and ragged N, with bias, beta and a residual-free
    # epilogue.  The bound is 2e-5, not the 1e-3 of the quantized paths: the
    # bf16 hi + lo split of an activation leaves 2^-17 of it, while a dropped
    # lo term, a misplaced k or a swapped row costs 1e-3 or more.
    keys = ("TML_GEMVTM", "TML_GEMVTM_NW", "TML_GEMVTM_IT", "TML_GEMVTM_T")
    saved = {key: os.environ.get(key) for key in keys}
    os.environ.update({"TML_GEMVTM": "2", "TML_GEMVTM_NW": str(nw), "TML_GEMVTM_IT": str(it),
                       "TML_GEMVTM_T": str(t)})
    try:
        for (k, n) in [(4160, 70), (1280, 600)]:
            w = rnd(201, k, n, 0.02)
            q, s = orc.quantize_q8(w)
            p, s4 = orc.quantize_q4(w)
            bias = synth.normal(203, n, 0.0, 0.02)
            for m in (1, 2, 3, 5, 8):
                a, c0 = rnd(204 + m, m, k), rnd(214 + m, m, n)
                for fmt, b, scale, ref in [(_abi.FMT_Q8_0, q, s, orc.matmul_q8(a, q, s)),
                                           (_abi.FMT_Q4_0, p, s4, orc.matmul_q4(a, p, k, n, s4))]:
                    got = _run_prepared(fmt, b, scale, k, n, m, a, bias=bias, c0=c0, alpha=0.75, beta=0.5)
                    err = rel_err(got, 0.75 * ref + 0.5 * c0 + bias)
                    assert err <= 2e-5, (k, n, m, fmt, err)
    finally:
        for key, v in saved.items():
            if v is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = v


@pytest.mark.parametrize("t", [1, 2])
def test_prepared_matrix_core_row_parts(orc, t):
    # The matrix-core GEMV with its rows split over two workgroups
    # (TML_GEMVTM_MSPLIT=2, grid.y): M = 5 / 7 / 8 as parts of 3 + 2, 4 + 3,
    # 4 + 4 rows, each part staging its own activations and writing its own
    # rows of C (with beta, bias and alpha), one or two column tiles a
    # workgroup, several superchunks and ragged N.  Bound 2e-5 as for the
    # other matrix-core plans.
    keys = ("TML_GEMVTM", "TML_GEMVTM_MSPLIT", "TML_GEMVTM_T")
    saved = {key: os.environ.get(key) for key in keys}
    os.environ.update({"TML_GEMVTM": "2", "TML_GEMVTM_MSPLIT": "2", "TML_GEMVTM_T": str(t)})
    try:
        for (k, n) in [(4160, 70), (1280, 600), (5120, 1280)]:
            w = rnd(271, k, n, 0.02)
            q, s = orc.quantize_q8(w)
            p, s4 = orc.quantize_q4(w)
            bias = synth.normal(273, n, 0.0, 0.02)
            for m in (5, 7, 8):
                a, c0 = rnd(274 + m, m, k), rnd(284 + m, m, n)
                for fmt, b, scale, ref in [(_abi.FMT_Q8_0, q, s, orc.matmul_q8(a, q, s)),
                                           (_abi.FMT_Q4_0, p, s4, orc.matmul_q4(a, p, k, n, s4))]:
                    got = _run_prepared(fmt, b, scale, k, n, m, a, bias=bias, c0=c0, alpha=0.75, beta=0.5)
                    err = rel_err(got, 0.75 * ref + 0.5 * c0 + bias)
                    assert err <= 2e-5, (k, n, m, fmt, err)
    finally:
        for key, v in saved.items():
            if v is None:
                os.environ.pop(key, None)
            else:
                os.environ[key] = v


@pytest.mark.parametrize("m", [4, 5, 8])
def test_prepared_row_parts_bitwise(orc, m):
    # Splitting the rows over workgroups changes no output's arithmetic
    # (each output row's MFMA sums and its lo-into-hi add are the same), so
    # the row-part plans must equal the unsplit ones bit for bit, fused
    # epilogue included: bias, beta, a residual, GELU (erf) and per-column
    # scales, at 5120 x 1280 (80 column tiles: the planner splits) and with
    # 2, 3 and 4 forced parts.
    import torch
    k, n = 5120, 1280
    w = rnd(291, k, n, 0.02)
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    qc, sc = orc.quantize_q8_cols(w)
    a, c0, res = rnd(292 + m, m, k), rnd(293, m, n), rnd(294, m, n)
    bias = synth.normal(295, n, 0.0, 0.02)
    A, R, Bias = _dev(a), _dev(res), _dev(bias)
    saved = os.environ.get("TML_GEMVTM_MSPLIT")
    try:
        for fmt, b, scale, cols in [(_abi.FMT_Q8_0, q, s, None), (_abi.FMT_Q4_0, p, s4, None),
                                    (_abi.FMT_Q8_0_PC, qc, 1.0, sc)]:
            B = _dev(b)
            S = _dev(cols) if cols is not None else None
            h = _abi.prepare_ex_dev(fmt, k, n, B.data_ptr(), scale=scale,
                                    scales_ptr=S.data_ptr() if S is not None else None)
            try:
                outs = []
                for parts in ("1", None, "2", "3", "4"):
                    if parts is None:
                        os.environ.pop("TML_GEMVTM_MSPLIT", None)
                    else:
                        os.environ["TML_GEMVTM_MSPLIT"] = parts
                    C = _dev(c0)
                    _abi.gemm_prepared_ex(h, m, A.data_ptr(), C.data_ptr(), act=_abi.ACT_GELU_ERF,
                                          residual_ptr=R.data_ptr(), bias_ptr=Bias.data_ptr(), alpha=0.5,
                                          beta=0.25)
                    torch.cuda.synchronize()
                    outs.append(C.cpu().numpy())
                for o in outs[1:]:
                    np.testing.assert_array_equal(o, outs[0])
            finally:
                _abi.prepared_free(h)
    finally:
        if saved is None:
            os.environ.pop("TML_GEMVTM_MSPLIT", None)
        else:
            os.environ["TML_GEMVTM_MSPLIT"] = saved


@pytest.mark.parametrize("gemvx", ["0", "1"])
def test_prepared_matrix_core_vocabulary(orc, gemvx):
    # Q8_0 and Q4_0 at M = 1 on a vocabulary-sized N: with the staged-activation
    # kernel off (TML_GEMVX=0) they take the matrix-core kernel (eight or more
    # workgroups a CU; Q8_0 with two rounds in flight, K = 1280 giving it two
    # rounds), by default the staged-activation kernel; on a layer-sized N
    # Q8_0 stays on the VALU kernel.
    saved = os.environ.get("TML_GEMVX")
    os.environ["TML_GEMVX"] = gemvx
    try:
        for (k, n) in ((256, 33000), (1280, 33000), (256, 5000)):
            w = rnd(231, k, n, 0.02)
            q, s = orc.quantize_q8(w)
            p, s4 = orc.quantize_q4(w)
            a = rnd(232, 1, k)
            for fmt, b, scale, ref in [(_abi.FMT_Q8_0, q, s, orc.matmul_q8(a, q, s)),
                                       (_abi.FMT_Q4_0, p, s4, orc.matmul_q4(a, p, k, n, s4))]:
                got = _run_prepared(fmt, b, scale, k, n, 1, a)
                assert rel_err(got, ref) <= 2e-5, (n, fmt)
    finally:
        if saved is None:
            os.environ.pop("TML_GEMVX", None)
        else:
            os.environ["TML_GEMVX"] = saved


@pytest.mark.parametrize("m", [3, 8])
def test_prepared_matrix_core_inf(orc, m):
    # Infinite and NaN activations through the matrix-core GEMV (the
    # staged-activation kernel, which would take M = 3 here, switched off):
    # each output is inf, -inf or nan exactly where the reference's fp32
    # product is, and the other rows are untouched.  Row 0 carries finite
    # activations above the largest bf16 on weight rows that quantize to 0
    # and +-1: finite outputs within the bound.
    k, n = 1280, 300
    w = rnd(221, k, n, 0.02)
    w[40] = 0.0
    w[41] = np.where(np.arange(n) % 3 == 0, -0.75, 0.75) * np.abs(w).max(axis=0) / 127.0
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    a = rnd(222, m, k)
    a[1, 5] = np.inf
    a[1, 700] = -np.inf
    a[2, 9] = np.nan
    a[0, 40] = np.finfo(np.float32).max
    a[0, 41] = np.float32(-3.4e38)
    saved = os.environ.get("TML_GEMVX")
    os.environ["TML_GEMVX"] = "0"
    try:
        for fmt, b, scale, ref in [(_abi.FMT_Q8_0, q, s, orc.matmul_q8(a, q, s)),
                                   (_abi.FMT_Q4_0, p, s4, orc.matmul_q4(a, p, k, n, s4))]:
            got = _run_prepared(fmt, b, scale, k, n, m, a)
            np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
            np.testing.assert_array_equal(np.isposinf(got), np.isposinf(ref))
            np.testing.assert_array_equal(np.isneginf(got), np.isneginf(ref))
            fin = np.isfinite(ref)
            assert np.all(fin[0]) and rel_err(got[0], ref[0]) <= 2e-5, fmt
            fin[0] = False
            assert rel_err(got[fin], ref[fin]) <= 2e-5, fmt
    finally:
        if saved is None:
            os.environ.pop("TML_GEMVX", None)
        else:
            os.environ["TML_GEMVX"] = saved


def test_prepared_alpha_beta_and_inf(orc):
    k, n, m = 300, 200, 2
    w, a, c0 = rnd(161, k, n, 0.02), rnd(162, m, k), rnd(163, m, n)
    got = _run_prepared(_abi.FMT_F32, w, 1.0, k, n, m, a, c0=c0, alpha=0.5, beta=-2.0)
    assert rel_err(got, 0.5 * orc.matmul(a, w) - 2.0 * c0) <= FP32_TOL
    # An infinite activation must give what the reference gives (inf or
    # nan per output), not a nan from a padded product.
    a2 = a.copy()
    a2[0, 5] = np.inf
    got = _run_prepared(_abi.FMT_F32, w, 1.0, k, n, m, a2)
    ref = orc.matmul(a2, w)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(np.isinf(got), np.isinf(ref))


def test_registered_weight_uses_prepared_copy(orc):
    # Host-pointer decoder calls on a registered weight go through the
    # prepared copy; results agree with the unregistered path to tolerance
    # and with the oracle.
    k, n = 640, 384
    w = rnd(171, k, n, 0.02)
    q, s = orc.quantize_q8(w)
    for m in (1, 2):
        a = rnd(172 + m, m, k)
        c0 = np.zeros((m, n), np.float32)
        _abi.sgemm_q8(m, n, k, a, q, s, c0)
        _abi.weight_register(q)
        try:
            c1 = np.zeros((m, n), np.float32)
            _abi.sgemm_q8(m, n, k, a, q, s, c1)
            c2 = np.zeros((m, n), np.float32)
            _abi.sgemm_q8(m, n, k, a, q, s, c2)
        finally:
            _abi.weight_release(q)
        np.testing.assert_array_equal(c1, c2)
        assert rel_err(c1, c0) <= Q_TOL and rel_err(c1, orc.matmul_q8(a, q, s)) <= Q_TOL
