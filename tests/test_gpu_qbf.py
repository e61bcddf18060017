"""The bf16 matrix-core Q8_0 / Q4_0 GEMM (gemm_qbf.hip, M > 8) against the oracle.

The int8 / int4 weights are exact in bf16 and each fp32 activation is split
into bf16 hi + lo terms (|x - hi - lo| <= 2^-17 |x|), so the product matches
the reference's dequantize-then-fp32-accumulate result (matmulF32Q8 /
matmulF32Q4, src/core/quantization.zig:240-311, :829-957; per-column scales
through oracle.matmul_cols) to ~1e-5.  The bound here is 2e-5, not the 1e-3
bar of the quantized paths: a dropped lo term costs ~4e-3, a misplaced k,
column or nibble far more.  The planner takes this kernel for every M past
the GEMV rows (M > 8); TML_GEMM_QBF=0 turns it off (any other value leaves
it on), a forced tile or split picks its plan.
"""
import os

import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu

TOL = 2e-5
KEYS = ("TML_GEMM_QBF_TILE", "TML_GEMM_QBF", "TML_GEMM_QBF_SPLIT")


def rnd(seed, m, n, std=1.0):
    return synth.normal_matrix(seed, m, n, std)


@pytest.fixture
def env():
    saved = {key: os.environ.get(key) for key in KEYS}
    yield os.environ
    for key, v in saved.items():
        if v is None:
            os.environ.pop(key, None)
        else:
            os.environ[key] = v


def _cases(orc, w, k, n, a):
    """(format, weight bytes, per-tensor scale, per-column scales, oracle product)."""
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    qc, sc = orc.quantize_q8_cols(w)
    pc, sc4 = orc.quantize_q4_cols(w)
    return [(_abi.FMT_Q8_0, q, s, None, orc.matmul_q8(a, q, s)),
            (_abi.FMT_Q4_0, p, s4, None, orc.matmul_q4(a, p, k, n, s4)),
            (_abi.FMT_Q8_0_PC, qc, 1.0, sc, orc.matmul_cols(a, _abi.FMT_Q8_0_PC, qc, sc, k, n)),
            (_abi.FMT_Q4_0_PC, pc, 1.0, sc4, orc.matmul_cols(a, _abi.FMT_Q4_0_PC, pc, sc4, k, n))]


def _gemm(fmt, m, n, k, a, b, scale, scales, bias=None):
    c = np.zeros((m, n), np.float32)
    _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(b), c, scale=scale, scales=scales, bias=bias)
    return c


@pytest.mark.parametrize("tile", [0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
def test_qbf_tiles_vs_oracle(orc, env, tile):
    # Every tile config (0: the planner's choice; 5-8 and 11 on 64-deep
    # slices, 7, 8 and 11 with two wave groups, 11 with four slices of loads
    # in flight, 9 and 10 with eight waves) on
    # shapes ragged in M and N (partial tiles, N not a multiple of 16), K
    # from one slice to many and not a multiple of 64, with a bias.
    env["TML_GEMM_QBF"] = "2"
    if tile:
        env["TML_GEMM_QBF_TILE"] = str(tile)
    for (m, n, k) in [(9, 130, 64), (200, 336, 520), (33, 4098, 40), (300, 70, 1288)]:
        w = rnd(301, k, n, 0.02)
        a = rnd(302 + m, m, k)
        bias = synth.normal(303, n, 0.0, 0.02)
        for fmt, b, scale, scales, ref in _cases(orc, w, k, n, a):
            got = _gemm(fmt, m, n, k, a, b, scale, scales, bias)
            err = rel_err(got, ref + bias)
            assert err <= TOL, (m, n, k, fmt, err)


@pytest.mark.parametrize("m", [9, 16, 48, 96, 127])
def test_qbf_small_m_default_plan(orc, env, m):
    # Below 128 rows the planner takes the 32 x 64 x 64 two-group tile with
    # the largest K split (1-4) that keeps its units within the CUs: every
    # split count appears across these shapes (4096 x 1024 at M = 9 splits
    # 4, at M = 48 2, at M = 96 not at all; 3072 x 768 splits 3 at M = 16).
    for (n, k) in [(4096, 1024), (3072, 768), (1536, 384)]:
        w = rnd(351, k, n, 0.02)
        a = rnd(352 + m, m, k)
        bias = synth.normal(353, n, 0.0, 0.02)
        for fmt, b, scale, scales, ref in _cases(orc, w, k, n, a):
            got = _gemm(fmt, m, n, k, a, b, scale, scales, bias)
            err = rel_err(got, ref + bias)
            assert err <= TOL, (m, n, k, fmt, err)


@pytest.mark.parametrize("split", [2, 3, 5])
@pytest.mark.parametrize("tile", [1, 2, 4, 6, 7, 8, 9, 10, 11])
def test_qbf_split_vs_oracle(orc, env, tile, split):
    # K split over workgroups (each over its own range of 32-deep slices,
    # whole 64-deep ones for tiles 5-8 and 11, the last range short), raw partials
    # summed in split order by the reduce launch, which runs the epilogue:
    # bias and residual here.
    env["TML_GEMM_QBF_TILE"] = str(tile)
    env["TML_GEMM_QBF_SPLIT"] = str(split)
    for (m, n, k) in [(200, 336, 520), (300, 70, 1288)]:
        w = rnd(351, k, n, 0.02)
        a = rnd(352 + m, m, k)
        bias = synth.normal(353, n, 0.0, 0.02)
        res = rnd(354, m, n)
        for fmt, b, scale, scales, ref in _cases(orc, w, k, n, a):
            c = np.zeros((m, n), np.float32)
            _abi.gemm_residual(fmt, m, n, k, a, np.ascontiguousarray(b), res, c, scale=scale, scales=scales,
                               bias=bias)
            err = rel_err(c, ref + bias + res)
            assert err <= TOL, (m, n, k, fmt, err)


@pytest.mark.parametrize("m", [128, 512])
def test_qbf_config3(orc, m):
    # BASELINE config 3 at M = 128 / 512: X[M x 1024] . W[1024 x 4096] in
    # Q8_0 (and Q4_0 on the same weight).
    k, n = 1024, 4096
    w = rnd(2002, k, n, 0.02)
    a = rnd(1001, m, k)
    q, s = orc.quantize_q8(w)
    p, s4 = orc.quantize_q4(w)
    nt = min(16, orc.max_threads())
    for fmt, b, scale, ref in [(_abi.FMT_Q8_0, q, s, orc.matmul_q8_mt(a, q, s, nt)),
                               (_abi.FMT_Q4_0, p, s4, orc.matmul_q4_mt(a, p, k, n, s4, nt))]:
        got = _gemm(fmt, m, n, k, a, b, scale, None)
        assert rel_err(got, ref) <= TOL, (m, fmt, rel_err(got, ref))


def test_qbf_epilogue(orc, env):
    # Residual, GELU (erf and tanh forms) and per-column scales in the
    # kernel's epilogue.
    env["TML_GEMM_QBF"] = "2"
    m, n, k = 150, 200, 264
    w = rnd(311, k, n, 0.02)
    a = rnd(312, m, k)
    bias = synth.normal(313, n, 0.0, 0.02)
    res = rnd(314, m, n)
    for fmt, b, scale, scales, ref in _cases(orc, w, k, n, a):
        c = np.zeros((m, n), np.float32)
        _abi.gemm_residual(fmt, m, n, k, a, np.ascontiguousarray(b), res, c, scale=scale, scales=scales, bias=bias)
        assert rel_err(c, ref + bias + res) <= TOL, fmt
        for act in (_abi.ACT_GELU_ERF, _abi.ACT_GELU_TANH):
            c = np.zeros((m, n), np.float32)
            _abi.gemm_act(fmt, m, n, k, a, np.ascontiguousarray(b), c, act=act, scale=scale, scales=scales, bias=bias)
            assert rel_err(c, orc.apply_act(ref + bias, act)) <= TOL, (fmt, act)


def test_qbf_alpha_beta_device(orc, env):
    # C = alpha * A . W + beta * C on device pointers.
    import torch
    env["TML_GEMM_QBF"] = "2"
    m, n, k = 70, 96, 128
    w = rnd(321, k, n, 0.02)
    a, c0 = rnd(322, m, k), rnd(323, m, n)
    q, s = orc.quantize_q8(w)
    A, Q, C = (torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0") for x in (a, q, c0))
    _abi.gemm_dev(_abi.FMT_Q8_0, m, n, k, A.data_ptr(), Q.data_ptr(), C.data_ptr(), scale=s, alpha=0.5, beta=-2.0)
    torch.cuda.synchronize()
    assert rel_err(C.cpu().numpy(), 0.5 * orc.matmul_q8(a, q, s) - 2.0 * c0) <= TOL


def _near_max_weights(w):
    """Weight rows 40 and 41 set so that every format quantizes them to 0 or
    +-1 (row 40 zero, row 41 at 0.75 of its column's int8 step): a finite
    activation near FLT_MAX on them keeps the reference's product finite."""
    w[40] = 0.0
    sign = np.where(np.arange(w.shape[1]) % 3 == 0, -1.0, 1.0).astype(np.float32)
    w[41] = sign * 0.75 * np.abs(w).max(axis=0) / 127.0
    return w


def test_qbf_inf_nan(orc, env):
    # Infinite and NaN activations: each output is inf, -inf or nan exactly
    # where the reference's fp32 product is (inf . 0 = nan included), the
    # other rows within the bound.  Rows 3 and 4 carry finite activations
    # above the largest bf16 (3.396e38 rounds to an infinite bf16) on weights
    # that quantize to 0 and +-1: finite outputs, within the bound.
    env["TML_GEMM_QBF"] = "2"
    m, n, k = 40, 300, 1280
    w = _near_max_weights(rnd(331, k, n, 0.02))
    a = rnd(332, m, k)
    a[1, 5] = np.inf
    a[1, 700] = -np.inf
    a[2, 9] = np.nan
    a[30, 1279] = np.inf
    big = np.float32(np.finfo(np.float32).max)
    a[3, 40] = big
    a[4, 40] = -big
    a[4, 41] = np.float32(3.4e38)
    for fmt, b, scale, scales, ref in _cases(orc, w, k, n, a):
        got = _gemm(fmt, m, n, k, a, b, scale, scales)
        np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
        np.testing.assert_array_equal(np.isposinf(got), np.isposinf(ref))
        np.testing.assert_array_equal(np.isneginf(got), np.isneginf(ref))
        assert np.all(np.isfinite(ref[3:5])), fmt
        assert rel_err(got[4], ref[4]) <= TOL, fmt
        rest = np.isfinite(ref)
        rest[3:5] = False
        assert rel_err(got[rest], ref[rest]) <= TOL and rel_err(got[3], ref[3]) <= TOL, fmt


def test_qbf_off_switch_agrees(orc, env):
    # TML_GEMM_QBF=0 runs the fp32-MFMA kernels on the same problem: both
    # within the bound of the oracle, and of each other.
    m, n, k = 96, 256, 512
    w = rnd(341, k, n, 0.02)
    a = rnd(342, m, k)
    for fmt, b, scale, scales, ref in _cases(orc, w, k, n, a):
        env["TML_GEMM_QBF"] = "2"
        got = _gemm(fmt, m, n, k, a, b, scale, scales)
        env["TML_GEMM_QBF"] = "0"
        old = _gemm(fmt, m, n, k, a, b, scale, scales)
        env.pop("TML_GEMM_QBF")
        assert rel_err(got, ref) <= TOL and rel_err(old, ref) <= 1e-5 and rel_err(got, old) <= TOL, fmt


@pytest.mark.parametrize("tile", [1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11])
def test_qbf_staged_epilogue(orc, env, tile):
    # With N a multiple of 4 and 16-byte aligned operands the tiles whose C
    # tile fits the staging buffer in one pass (tiles 4-8: 32 x 64, and
    # 64 x 64 on 64-deep slices)
    # write C through LDS in whole 16-byte row pieces, the large ones the
    # per-lane 4-byte path, which TML_GEMM_VEC_EPI=0 takes everywhere.  Every epilogue term
    # (alpha, beta * C, bias, residual, GELU, per-column scales) on ragged M
    # and N, K split or not: against the oracle, and the two paths within
    # rounding of each other.
    import torch
    env["TML_GEMM_QBF_TILE"] = str(tile)
    saved = os.environ.get("TML_GEMM_VEC_EPI")
    m, n, k = 203, 340, 520
    a, w, c0, r = rnd(691, m, k), rnd(692, k, n, 0.05), rnd(693, m, n), rnd(694, m, n)
    bias = synth.normal(695, n, 0.0, 0.5)
    try:
        for split in ("1", "3"):
            env["TML_GEMM_QBF_SPLIT"] = split
            for fmt, b, scale, scales, prod in _cases(orc, w, k, n, a):
                ref = orc.gelu_exact(0.75 * prod - 0.5 * c0 + bias + r)
                got = {}
                for staged in ("1", "0"):
                    os.environ["TML_GEMM_VEC_EPI"] = staged
                    dev = [torch.from_numpy(np.ascontiguousarray(x)).to("cuda:0") for x in (a, b, c0, r, bias)]
                    A, B, C, R, Bias = dev
                    S = torch.from_numpy(scales).to("cuda:0") if scales is not None else None
                    _abi.gemm_ex_dev(fmt, m, n, k, A.data_ptr(), B.data_ptr(), C.data_ptr(), scale=scale,
                                     act=_abi.ACT_GELU_ERF, residual_ptr=R.data_ptr(),
                                     scales_ptr=S.data_ptr() if S is not None else None, bias_ptr=Bias.data_ptr(),
                                     alpha=0.75, beta=-0.5)
                    torch.cuda.synchronize()
                    got[staged] = C.cpu().numpy()
                assert rel_err(got["1"], ref) <= TOL, (tile, split, fmt, rel_err(got["1"], ref))
                assert rel_err(got["1"], got["0"]) <= 1e-6, (tile, split, fmt)
    finally:
        if saved is None:
            os.environ.pop("TML_GEMM_VEC_EPI", None)
        else:
            os.environ["TML_GEMM_VEC_EPI"] = saved
