"""GPU parity of the [K,N] GEMV (tomoul_amd/csrc/gemv.hip) on rows that are
not a whole number of lane chunks.  Such a chunk is read as the aligned
dwords that cover it and funnel-shifted into place.  The case that matters is
Whisper's decoder vocabulary projection: ops.matmul of [1, 1280] by the
per-step transpose of the token embedding, [1280, 51866]
(src/models/whisper/decoder.zig:936-940).

* Bitwise equal to the element-wise path (TML_GEMV_RAGGED=0) under the same
  plan (16 lanes a row, forced on both).  The two read the same values and
  add them in the same order.  B ends inside a dword in most cases.
* Against the oracle at the vocabulary shape, f32 / F16 / Q8_0 / Q4_0.
* A non-finite weight at the start of every row.  A chunk that runs past the
  end of its row picks it up, and it must reach only the dropped columns.
* B not 4-byte aligned takes the element-wise path, with the same result.
* Per-output-column scales (the Q8_0_PC / Q4_0_PC extension) on ragged rows,
  through the residual and GELU epilogues.
Tolerances are the north star's (1e-4 fp32 / F16 weights, 1e-3 quantized).
"""
import os

import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-4
Q_TOL = 1e-3
F32, F16, Q8_0, Q4_0 = _abi.FMT_F32, _abi.FMT_F16, _abi.FMT_Q8_0, _abi.FMT_Q4_0


def rnd(seed, m, n, std=1.0):
    return synth.normal_matrix(seed, m, n, std)


@pytest.fixture
def env():
    keys = ("TML_GEMV_LPR", "TML_GEMV_NB", "TML_GEMV_RAGGED")
    saved = {k: os.environ.get(k) for k in keys}
    yield os.environ
    for k, v in saved.items():
        if v is None:
            os.environ.pop(k, None)
        else:
            os.environ[k] = v


def weight(orc, fmt, w):
    """(B as stored, scale, oracle product a -> a.B, tolerance) for f32 weights w[k, n]."""
    k, n = w.shape
    if fmt == F32:
        return w, 1.0, lambda a: orc.matmul(a, w), FP32_TOL
    if fmt == F16:
        h = orc.to_f16(w)
        return h, 1.0, lambda a: orc.matmul_f16(a, h), FP32_TOL
    if fmt == Q8_0:
        q, s = orc.quantize_q8(w)
        return q.reshape(k, n), s, lambda a: orc.matmul_q8(a, q, s), Q_TOL
    p, s = orc.quantize_q4(w)
    return p, s, lambda a: orc.matmul_q4(a, p, k, n, s), Q_TOL


@pytest.mark.parametrize("fmt", [F32, F16, Q8_0, Q4_0])
@pytest.mark.parametrize("nb", [1, 3])
def test_ragged_bitwise_vs_elementwise(orc, env, fmt, nb):
    # nb = 1 splits K over many workgroups (the partial-sum exchange), nb = 3
    # over fewer; K*N is odd for the first three shapes, so B ends inside a
    # dword whatever the format.
    env["TML_GEMV_LPR"] = "16"
    env["TML_GEMV_NB"] = str(nb)
    for k, n in ((517, 333), (1029, 1001), (41, 7), (4, 4099)):
        b, scale, ref, tol = weight(orc, fmt, rnd(901 + n, k, n, 0.02))
        bias = synth.normal(902, n, 0.0, 0.02)
        for m in (1, 2, 3, 5, 8):
            a = rnd(903 + m, m, k)
            outs = []
            for ragged in ("2", "0"):  # 2: the call fails unless it takes the ragged-row loads
                env["TML_GEMV_RAGGED"] = ragged
                c = np.zeros((m, n), np.float32)
                _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(b), c, scale=scale, bias=bias)
                outs.append(c)
            np.testing.assert_array_equal(outs[0], outs[1], err_msg=f"fmt {fmt} k {k} n {n} m {m}")
            assert rel_err(outs[0], ref(a) + bias) <= tol, (fmt, k, n, m)


@pytest.mark.parametrize("fmt", [F32, F16, Q8_0, Q4_0])
def test_vocabulary_projection_shape(orc, env, fmt):
    # [M, 1280] . [1280, 51866] on the planner's own plan (wide segments:
    # B streams more than 16 MiB), on the ragged-row loads
    env["TML_GEMV_RAGGED"] = "2"
    k, n = 1280, 51866
    b, scale, ref, tol = weight(orc, fmt, rnd(911, k, n, 0.02))
    for m in (1, 2, 4):
        a = rnd(912 + m, m, k)
        c = np.zeros((m, n), np.float32)
        _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(b), c, scale=scale)
        assert rel_err(c, ref(a)) <= tol, (fmt, m)


@pytest.mark.parametrize("fmt", [F32, F16])
@pytest.mark.parametrize("lpr", ["", "64"])
def test_next_row_nonfinite_stays_in_dropped_columns(orc, env, fmt, lpr):
    # Column 0 is +inf in every row: the last chunk of each row (N % lane
    # elements == 1) reads it as a column past N.  Column 0 itself must come
    # out NaN (x has both signs), every other column finite and right.
    env["TML_GEMV_LPR"] = lpr
    env["TML_GEMV_RAGGED"] = "2"
    k, n = 300, 1001
    w = rnd(921, k, n, 0.02)
    w[:, 0] = np.inf
    b, scale, ref, tol = weight(orc, fmt, w)
    for m in (1, 3, 8):
        a = rnd(922 + m, m, k)
        c = np.zeros((m, n), np.float32)
        _abi.gemm(fmt, m, n, k, a, np.ascontiguousarray(b), c, scale=scale)
        want = ref(a)
        assert np.isnan(c[:, 0]).all() and np.isnan(want[:, 0]).all()
        assert np.isfinite(c[:, 1:]).all(), (fmt, m)
        assert rel_err(c[:, 1:], want[:, 1:]) <= tol, (fmt, m)


@pytest.mark.parametrize("fmt,offset", [(Q8_0, 1), (Q8_0, 2), (Q4_0, 3), (F16, 2)])
def test_unaligned_weight_pointer(orc, env, fmt, offset):
    # B starting 1-3 bytes past an aligned address cannot take the dword
    # path (TML_GEMV_RAGGED=2 refuses the call); the element-wise one gives
    # the same answer.
    import torch
    k, n = 517, 333
    b, scale, ref, tol = weight(orc, fmt, rnd(931, k, n, 0.02))
    raw = np.ascontiguousarray(b).view(np.uint8).reshape(-1)
    dev = torch.device("cuda:0")
    buf = torch.zeros(raw.size + 64, dtype=torch.uint8, device=dev)
    buf[offset:offset + raw.size] = torch.from_numpy(raw).to(dev)
    for m in (1, 5):
        a = rnd(932 + m, m, k)
        x = torch.from_numpy(a).to(dev)
        y = torch.zeros((m, n), dtype=torch.float32, device=dev)
        env["TML_GEMV_RAGGED"] = "2"
        with pytest.raises(_abi.TmlError):
            _abi.gemm_dev(fmt, m, n, k, x.data_ptr(), buf.data_ptr() + offset, y.data_ptr(), scale=scale)
        env["TML_GEMV_RAGGED"] = "1"
        _abi.gemm_dev(fmt, m, n, k, x.data_ptr(), buf.data_ptr() + offset, y.data_ptr(), scale=scale)
        torch.cuda.synchronize()
        assert rel_err(y.cpu().numpy(), ref(a)) <= tol, (fmt, offset, m)


@pytest.mark.parametrize("fmt", [_abi.FMT_Q8_0_PC, _abi.FMT_Q4_0_PC])
def test_ragged_per_column_scales(orc, env, fmt):
    # Per-output-column scales (Q8_0 / Q4_0 bytes, one scale a column) on
    # ragged rows, with a bias and a residual, and with the exact GELU after
    # the bias.
    env["TML_GEMV_RAGGED"] = "2"
    k, n = 517, 333
    w = rnd(941, k, n, 0.02)
    q, s = (orc.quantize_q8_cols if fmt == _abi.FMT_Q8_0_PC else orc.quantize_q4_cols)(w)
    bias = synth.normal(942, n, 0.0, 0.02)
    for m in (1, 2, 3, 5, 8):
        a = rnd(943 + m, m, k)
        ref = orc.matmul_cols(a, fmt, q, s, k, n) + bias
        res = rnd(950 + m, m, n)
        c = np.zeros((m, n), np.float32)
        _abi.gemm_residual(fmt, m, n, k, a, np.ascontiguousarray(q), res, c, scales=s, bias=bias)
        assert rel_err(c, ref + res) <= Q_TOL, (fmt, m)
        c = np.zeros((m, n), np.float32)
        _abi.gemm_act(fmt, m, n, k, a, np.ascontiguousarray(q), c, act=_abi.ACT_GELU_ERF, scales=s, bias=bias)
        assert rel_err(c, orc.apply_act(ref, _abi.ACT_GELU_ERF)) <= Q_TOL, (fmt, m)
