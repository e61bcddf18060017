"""Config 5 at its full size: the Whisper large-v3-turbo encoder linears at
1500 frames -- X[1500x1280] . W[1280x3840] (Q, K and V), X . W[1280x5120]
(FFN up), H[1500x5120] . W[5120x1280] (FFN down) -- in fp32 and with Q8_0 /
Q4_0 weights, against the oracle's restatement (fp32: ascending-k f32
accumulation, src/core/ops.zig:235-417; quantized: dequantize then f32
accumulate, src/core/quantization.zig:158-203, :778-824).

The reference projects Q, K and V with three GEMMs of their own
(src/core/attention.zig:485-490), each weight quantized with its own
per-tensor scale.  One fused GEMM over W[1280x3840] reproduces them exactly
when column n carries the scale of the tensor it came from: the
per-output-column formats (TML_FMT_Q8_0_PC / Q4_0_PC, an extension) with
scales [s_q]*1280 + [s_k]*1280 + [s_v]*1280.  Each N-slice of the fused
product is checked against its own reference GEMM.
"""
import os

import numpy as np
import pytest

from conftest import elementwise_ok, rel_err
from tomoul_amd import _abi, synth

pytestmark = pytest.mark.gpu

NT = min(16, os.cpu_count() or 1)
FP32_TOL = 1e-4
Q_TOL = 1e-3
D, FF, T_ = 1280, 5120, 1500


@pytest.fixture(scope="module")
def acts():
    return synth.normal_matrix(1001, T_, D), synth.normal_matrix(1002, T_, FF)


def _w(seed, k, n):
    return synth.normal_matrix(seed, k, n, 0.02)


@pytest.mark.parametrize("name,k,n,seed", [("ffn_up", D, FF, 2003), ("ffn_down", FF, D, 2004)])
@pytest.mark.parametrize("fmt", ["f32", "q8_0", "q4_0"])
def test_config5_ffn(orc, acts, name, k, n, seed, fmt):
    a = acts[0] if k == D else acts[1]
    w = _w(seed, k, n)
    got = np.zeros((T_, n), np.float32)
    if fmt == "f32":
        _abi.gemm(_abi.FMT_F32, T_, n, k, a, w, got)
        ref = orc.matmul_mt(a, w, NT)
        assert rel_err(got, ref) <= FP32_TOL, rel_err(got, ref)
        assert elementwise_ok(got, ref, FP32_TOL)
    elif fmt == "q8_0":
        q, s = orc.quantize_q8(w)
        _abi.gemm(_abi.FMT_Q8_0, T_, n, k, a, q, got, scale=s)
        ref = orc.matmul_q8_mt(a, q.reshape(k, n), s, NT)
        assert rel_err(got, ref) <= Q_TOL, rel_err(got, ref)
    else:
        p, s = orc.quantize_q4(w)
        _abi.gemm(_abi.FMT_Q4_0, T_, n, k, a, p, got, scale=s)
        ref = orc.matmul_q4_mt(a, p, k, n, s, NT)
        assert rel_err(got, ref) <= Q_TOL, rel_err(got, ref)


@pytest.mark.parametrize("fmt", ["f32", "q8_0", "q4_0"])
def test_config5_fused_qkv_equals_three_gemms(orc, acts, fmt):
    x = acts[0]
    ws = [_w(2002, D, D), _w(2012, D, D), _w(2022, D, D)]  # Wq, Wk, Wv
    got = np.zeros((T_, 3 * D), np.float32)
    if fmt == "f32":
        _abi.gemm(_abi.FMT_F32, T_, 3 * D, D, x, np.ascontiguousarray(np.concatenate(ws, axis=1)), got)
        refs = [orc.matmul_mt(x, w, NT) for w in ws]
        tol = FP32_TOL
    elif fmt == "q8_0":
        qs = [orc.quantize_q8(w) for w in ws]
        data = np.ascontiguousarray(np.concatenate([q.reshape(D, D) for q, _ in qs], axis=1))
        cols = np.repeat(np.array([s for _, s in qs], np.float32), D)
        _abi.gemm(_abi.FMT_Q8_0_PC, T_, 3 * D, D, x, data, got, scales=cols)
        refs = [orc.matmul_q8_mt(x, q.reshape(D, D), s, NT) for q, s in qs]
        tol = Q_TOL
    else:
        ps = [orc.quantize_q4(w) for w in ws]
        vals = np.concatenate([orc._unpack_q4(p, D * D).reshape(D, D) for p, _ in ps], axis=1)
        data = orc._pack_q4(vals)
        cols = np.repeat(np.array([s for _, s in ps], np.float32), D)
        _abi.gemm(_abi.FMT_Q4_0_PC, T_, 3 * D, D, x, data, got, scales=cols)
        refs = [orc.matmul_q4_mt(x, p, D, D, s, NT) for p, s in ps]
        tol = Q_TOL
    for i, ref in enumerate(refs):
        part = got[:, i * D:(i + 1) * D]
        assert rel_err(part, ref) <= tol, ("qkv"[i], rel_err(part, ref))
