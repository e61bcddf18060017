"""The staged-activation decoder GEMV (gemv_x.hip): Q8_0 / Q4_0 at M = 1 and
2 on prepared weights (and at 3-4 rows), against the oracle (the reference's
dequantize-then-f32-accumulate loops, quantization.zig:158-203 and
:778-824).  TML_GEMVX=3 makes every such call refuse any other kernel, so
each case proves that this one ran.  Covered: the decoder shapes of configs 3
and 4, the Whisper vocabulary projection (1280 x 51866), rows ragged against the kernel's layers (N not a multiple of its rows
per workgroup), long rows (384 / 224 chunks, activations near the 64 KiB of
LDS the kernel may use at M = 2) and the shortest (one chunk), both
thread counts and every layer count, the fused epilogue (bias, alpha / beta,
per-column scales, residual, both GELUs), and infinite / NaN activations.
The products are fp32 multiply-adds in another order than the oracle's, so
the bar is 1e-5 relative (a dropped chunk or a misplaced activation costs
~1e-2)."""
import os

import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu

TOL = 1e-5
KEYS = ("TML_GEMVX", "TML_GEMVX_NT", "TML_GEMVX_P")


@pytest.fixture
def env():
    saved = {k: os.environ.get(k) for k in KEYS}
    os.environ["TML_GEMVX"] = "3"
    yield os.environ
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def _dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda:0")


def _quant(orc, fmt, w):
    if fmt == _abi.FMT_Q8_0:
        q, s = orc.quantize_q8(w)
        return q, s
    return orc.quantize_q4(w)


def _ref(orc, fmt, a, q, s, k, n):
    return orc.matmul_q8(a, q, s) if fmt == _abi.FMT_Q8_0 else orc.matmul_q4(a, q, k, n, s)


def _prepared(fmt, q, s, k, n):
    B = _dev(q)
    return B, _abi.prepare_dev(fmt, k, n, B.data_ptr(), s)


def _run(h, m, n, a, **kw):
    import torch
    A = _dev(a)
    C = kw.pop("c0", None)
    C = _dev(C) if C is not None else torch.full((m, n), float("nan"), dtype=torch.float32, device="cuda:0")
    dev_kw = {}
    for key in ("bias", "residual"):
        if kw.get(key) is not None:
            dev_kw[key] = _dev(kw[key])
    _abi.gemm_prepared_ex(h, m, A.data_ptr(), C.data_ptr(), act=kw.get("act", _abi.ACT_NONE),
                          residual_ptr=dev_kw["residual"].data_ptr() if "residual" in dev_kw else None,
                          bias_ptr=dev_kw["bias"].data_ptr() if "bias" in dev_kw else None,
                          alpha=kw.get("alpha", 1.0), beta=kw.get("beta", 0.0))
    torch.cuda.synchronize()
    return C.cpu().numpy()


SHAPES = [(_abi.FMT_Q8_0, 1024, 4096), (_abi.FMT_Q4_0, 1280, 5120), (_abi.FMT_Q4_0, 5120, 1280),
          (_abi.FMT_Q8_0, 1280, 5120), (_abi.FMT_Q8_0, 6144, 300), (_abi.FMT_Q4_0, 7168, 37),
          (_abi.FMT_Q8_0, 16, 1001), (_abi.FMT_Q4_0, 32, 7), (_abi.FMT_Q4_0, 224, 1000), (_abi.FMT_Q8_0, 2560, 2049),
          (_abi.FMT_Q8_0, 1280, 51866), (_abi.FMT_Q4_0, 1280, 51866)]


@pytest.mark.parametrize("fmt,k,n", SHAPES, ids=[f"{'q8' if f == 1 else 'q4'}_{k}x{n}" for f, k, n in SHAPES])
@pytest.mark.parametrize("m", [1, 2])
def test_vs_oracle(orc, env, fmt, k, n, m):
    w = synth.normal_matrix(301, k, n, 0.02)
    q, s = _quant(orc, fmt, w)
    a = synth.normal_matrix(302 + m, m, k)
    B, h = _prepared(fmt, q, s, k, n)
    try:
        got = _run(h, m, n, a)
    finally:
        _abi.prepared_free(h)
    err = rel_err(got, _ref(orc, fmt, a, q, s, k, n))
    assert err <= TOL, err


# Shapes the kernel takes at 3-4 rows: activations and partials within its
# 64 KiB of LDS.
MORE = [(_abi.FMT_Q8_0, 1024, 4096, (3, 4)), (_abi.FMT_Q4_0, 1280, 5120, (3, 4)),
        (_abi.FMT_Q8_0, 1280, 5120, (4,)), (_abi.FMT_Q8_0, 16, 1001, (3,)), (_abi.FMT_Q4_0, 32, 7, (4,)),
        (_abi.FMT_Q4_0, 224, 1000, (3, 4)), (_abi.FMT_Q8_0, 1280, 51866, (4,)), (_abi.FMT_Q4_0, 1280, 51866, (4,)),
        (_abi.FMT_Q8_0, 2048, 333, (3, 4)), (_abi.FMT_Q4_0, 3072, 768, (3, 4))]


@pytest.mark.parametrize("fmt,k,n,ms", MORE, ids=[f"{'q8' if f == 1 else 'q4'}_{k}x{n}" for f, k, n, _ in MORE])
def test_more_rows(orc, env, fmt, k, n, ms):
    # 3-4 activation rows: M rounded up to 4 in registers, the rows past M
    # zero and dropped
    w = synth.normal_matrix(305, k, n, 0.02)
    q, s = _quant(orc, fmt, w)
    B, h = _prepared(fmt, q, s, k, n)
    try:
        for m in ms:
            a = synth.normal_matrix(306 + m, m, k)
            err = rel_err(_run(h, m, n, a), _ref(orc, fmt, a, q, s, k, n))
            assert err <= TOL, (m, err)
    finally:
        _abi.prepared_free(h)


@pytest.mark.parametrize("nt", ["256", "512"])
@pytest.mark.parametrize("p", ["1", "2", "3", "4"])
def test_plans(orc, env, nt, p):
    # every thread count and layer count, on rows ragged against the layers
    env["TML_GEMVX_NT"] = nt
    env["TML_GEMVX_P"] = p
    for fmt, k, n in [(_abi.FMT_Q4_0, 1280, 997), (_abi.FMT_Q8_0, 2048, 333), (_abi.FMT_Q4_0, 5120, 130)]:
        w = synth.normal_matrix(311, k, n, 0.02)
        q, s = _quant(orc, fmt, w)
        B, h = _prepared(fmt, q, s, k, n)
        try:
            for m in (1, 2):
                a = synth.normal_matrix(312 + m, m, k)
                err = rel_err(_run(h, m, n, a), _ref(orc, fmt, a, q, s, k, n))
                assert err <= TOL, (fmt, k, n, m, err)
        finally:
            _abi.prepared_free(h)


@pytest.mark.parametrize("fmt", [_abi.FMT_Q8_0, _abi.FMT_Q4_0])
def test_epilogue(orc, env, fmt):
    k, n = 1280, 700
    w = synth.normal_matrix(321, k, n, 0.02)
    q, s = _quant(orc, fmt, w)
    B, h = _prepared(fmt, q, s, k, n)
    try:
        for m in (1, 2, 4):
            a = synth.normal_matrix(322 + m, m, k)
            bias = synth.normal(324, n, 0.0, 0.5)
            res = synth.normal_matrix(325, m, n)
            c0 = synth.normal_matrix(326, m, n)
            base = _ref(orc, fmt, a, q, s, k, n)
            got = _run(h, m, n, a, bias=bias, c0=c0, alpha=0.5, beta=-2.0)
            assert rel_err(got, 0.5 * base - 2.0 * c0 + bias) <= TOL
            for act, fn in ((_abi.ACT_GELU_ERF, orc.gelu_exact), (_abi.ACT_GELU_TANH, orc.gelu_tanh)):
                got = _run(h, m, n, a, bias=bias, residual=res, act=act)
                assert rel_err(got, fn((base + bias) + res)) <= TOL, act
    finally:
        _abi.prepared_free(h)


@pytest.mark.parametrize("fmt", [_abi.FMT_Q8_0_PC, _abi.FMT_Q4_0_PC])
def test_column_scales(orc, env, fmt):
    k, n = 1280, 640
    w = synth.normal_matrix(331, k, n, 0.02) * np.exp(synth.normal(332, n, 0.0, 1.0))[None, :].astype(np.float32)
    w = np.ascontiguousarray(w.astype(np.float32))
    q, sc = orc.quantize_q8_cols(w) if fmt == _abi.FMT_Q8_0_PC else orc.quantize_q4_cols(w)
    Q, S = _dev(q), _dev(sc)
    h = _abi.prepare_ex_dev(fmt, k, n, Q.data_ptr(), scales_ptr=S.data_ptr())
    try:
        for m in (1, 2, 4):
            a = synth.normal_matrix(333 + m, m, k)
            err = rel_err(_run(h, m, n, a), orc.matmul_cols(a, fmt, q, sc, k, n))
            assert err <= TOL, (m, err)
    finally:
        _abi.prepared_free(h)


@pytest.mark.parametrize("fmt", [_abi.FMT_Q8_0, _abi.FMT_Q4_0])
def test_inf_nan(orc, env, fmt):
    # inf, -inf and NaN activations: every output is inf, -inf or NaN exactly
    # where the reference's fp32 product is (inf . 0 = NaN where a weight is
    # zero), finite elsewhere; idle lanes and rows past N (whose weights read
    # as zeros) never reach an output
    k, n = 1280, 301
    w = synth.normal_matrix(341, k, n, 0.02)
    w[:, 7] = 0.0
    q, s = _quant(orc, fmt, w)
    B, h = _prepared(fmt, q, s, k, n)
    try:
        for m, pos in ((1, [(0, 5)]), (2, [(1, 5), (1, 700)]), (4, [(1, 5), (3, 700)])):
            a = synth.normal_matrix(342 + m, m, k)
            for (i, j) in pos:
                a[i, j] = np.inf
            if m >= 2:
                a[1, 700] = -np.inf
                a[0, 9] = np.nan
            got = _run(h, m, n, a)
            ref = _ref(orc, fmt, a, q, s, k, n)
            np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
            np.testing.assert_array_equal(np.isposinf(got), np.isposinf(ref))
            np.testing.assert_array_equal(np.isneginf(got), np.isneginf(ref))
            fin = np.isfinite(ref)
            if fin.any():
                assert rel_err(got[fin], ref[fin]) <= TOL
    finally:
        _abi.prepared_free(h)


def test_refusal_switch(orc, env):
    # TML_GEMVX=3 refuses what the kernel cannot take (K not a whole number
    # of chunks), so a passing case above did run this kernel
    k, n = 1000, 64
    w = synth.normal_matrix(351, k, n, 0.02)
    q, s = _quant(orc, _abi.FMT_Q8_0, w)
    B, h = _prepared(_abi.FMT_Q8_0, q, s, k, n)
    try:
        with pytest.raises(_abi.TmlError):
            _run(h, 1, n, synth.normal_matrix(352, 1, k))
        os_env = os.environ
        os_env["TML_GEMVX"] = "1"
        got = _run(h, 1, n, synth.normal_matrix(352, 1, k))
        assert rel_err(got, orc.matmul_q8(synth.normal_matrix(352, 1, k), q, s)) <= TOL
    finally:
        _abi.prepared_free(h)
