""".tl payloads on the GPU: device reads, getTensorDequantized and the XLM-R
transposing loaders (loadQuantizedTransposed{Q8,Q4,Q8K},
src/models/xlm_roberta_punctuation/model.zig:1272-1362) against the oracle's
restatement, bitwise (every step is a copy, one f32 multiply per element or
the bit-exact quantizer); then two callers end to end: an XLM-R-style
[out,in] quantized layer through the transposing loader into the matmul, and
a Whisper-style tied vocabulary projection from a dequantized embedding used
in place (src/models/whisper/decoder.zig:108, :936-940).
"""
import os

import numpy as np
import pytest

from conftest import rel_err
from tomoul_amd import _abi, loader as tl, quantization as qz, synth
from tomoul_amd.tensor import Tensor

pytestmark = pytest.mark.gpu

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tl")


def _encode(orc, fmt, w):
    if fmt == orc.TL_F32:
        return {"data": w}
    if fmt == orc.TL_F16:
        return {"data": orc.to_f16(w)}
    if fmt == orc.TL_Q8_0:
        q, s = orc.quantize_q8(w)
        return {"scale": s, "data": q}
    if fmt == orc.TL_Q4_0:
        p, s = orc.quantize_q4(w)
        return {"scale": s, "data": p}
    q, sc = orc.quantize_q8k(w)
    return {"scales": sc, "data": q}


SHAPES = [(33, 17), (64, 96), (300, 1024), (7, 1)]


def _file(orc, tmp_path, fmt, seed=900):
    rng = np.random.default_rng(seed + fmt)
    tensors = []
    for i, shp in enumerate(SHAPES):
        w = (rng.standard_normal(shp[0] * shp[1]) * 0.05).astype(np.float32)
        tensors.append((f"t{i}", shp, _encode(orc, fmt, w)))
    data = orc.tl_write(tensors, fmt)
    p = tmp_path / f"f{fmt}.tl"
    p.write_bytes(data)
    return str(p), data, tensors


@pytest.mark.parametrize("fmt", [0, 1, 2, 3, 4])
def test_read_dev_and_dequantized(orc, tmp_path, fmt):
    import torch
    path, data, tensors = _file(orc, tmp_path, fmt)
    ld = tl.ModelLoader(path)
    for name, shp, parts in tensors:
        n = shp[0] * shp[1]
        nbytes = _abi.weight_bytes(fmt, 1, n)
        buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        sc = torch.empty(max((n + 31) // 32, 1), dtype=torch.float32, device="cuda")
        scale = ld.readDev(name, fmt, buf.data_ptr(), sc.data_ptr() if fmt == 3 else None)
        torch.cuda.synchronize()
        raw = np.frombuffer(parts["data"].tobytes(), dtype=np.uint8)
        np.testing.assert_array_equal(buf.cpu().numpy(), raw)
        if fmt in (1, 2):
            assert np.float32(scale) == np.float32(parts["scale"])
        if fmt == 3:
            np.testing.assert_array_equal(sc.cpu().numpy()[: parts["scales"].size], parts["scales"])
        got = ld.getTensorDequantized(name).numpy().reshape(-1)
        want = orc.tl_dequantize(fmt, orc.tl_payload(data, (name, shp) + _entry(ld, name), fmt), n)
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def _entry(ld, name):
    info = ld.getTensorInfo(name)
    return (info.data_offset, info.data_size)


def test_dequantized_reference_fixture(orc):
    data = open(os.path.join(GOLD, "silero_vad_model_tiny.tl"), "rb").read()
    ld = tl.ModelLoader(os.path.join(GOLD, "silero_vad_model_tiny.tl"))
    for e in orc.tl_parse(data)["tensors"]:
        got = ld.getTensorDequantized(e[0]).numpy().reshape(-1)
        np.testing.assert_array_equal(got, orc.tl_payload(data, e, orc.TL_F32)["data"])


@pytest.mark.parametrize("fmt", [1, 2, 3])
def test_transposing_loaders_bitwise(orc, tmp_path, fmt):
    path, data, tensors = _file(orc, tmp_path, fmt)
    ld = tl.ModelLoader(path)
    fn = {1: tl.loadQuantizedTransposedQ8, 2: tl.loadQuantizedTransposedQ4, 3: tl.loadQuantizedTransposedQ8K}[fmt]
    for name, (rows, cols), parts in tensors:
        n = rows * cols
        deq = orc.tl_dequantize(fmt, parts, n).reshape(rows, cols)
        t = np.ascontiguousarray(deq.T)
        got = fn(ld, name)
        assert got.shape == (cols, rows)
        if fmt == 1:
            q, s = orc.quantize_q8(t)
            assert np.float32(got.scale) == np.float32(s)
            np.testing.assert_array_equal(got.data, q.reshape(-1))
        elif fmt == 2:
            p, s = orc.quantize_q4(t)
            assert np.float32(got.scale) == np.float32(s)
            np.testing.assert_array_equal(got.data, p.reshape(-1))
        else:
            q, sc = orc.quantize_q8k(t)
            np.testing.assert_array_equal(got.scales, sc)
            np.testing.assert_array_equal(got.data, q.reshape(-1))


def test_xlmr_layer_end_to_end(orc, tmp_path):
    # An [out, in] Q8_0 weight as XLM-R's exporter writes it, loaded the
    # reference's way (transpose + re-quantize) and multiplied.
    K, N, M = 1024, 384, 16
    w_out_in = synth.normal_matrix(911, N, K, 0.02)
    q, s = orc.quantize_q8(w_out_in)
    p = tmp_path / "xlmr_q8.tl"
    p.write_bytes(orc.tl_write([("encoder.layer.0.output.dense.weight", (N, K), {"scale": s, "data": q})], 1))
    qt = tl.loadQuantizedTransposedQ8(tl.ModelLoader(str(p)), "encoder.layer.0.output.dense.weight")
    x = synth.normal_matrix(912, M, K)
    got = qz.matmulF32Q8Simd(Tensor.from_numpy(x), qt).numpy()
    t = np.ascontiguousarray(orc.dequantize_q8(q, s).reshape(N, K).T)
    q2, s2 = orc.quantize_q8(t)
    assert rel_err(got, orc.matmul_q8(x, q2.reshape(K, N), s2)) <= 1e-3


def test_tied_vocab_projection_end_to_end(orc, tmp_path):
    # decoder.token_embedding stored Q8_0 [n_vocab, d]; the reference
    # dequantizes it at load (decoder.zig:108) and transposes it every step
    # (:936-940).  Here: dequantize into HBM once, wrap it as a rows-prepared
    # weight in place, project.
    import torch
    V, d = 5003, 384
    e = synth.normal_matrix(921, V, d, 0.05)
    q, s = orc.quantize_q8(e)
    p = tmp_path / "whisper_q8.tl"
    p.write_bytes(orc.tl_write([("decoder.token_embedding", (V, d), {"scale": s, "data": q})], 1))
    ld = tl.ModelLoader(str(p))
    emb = torch.empty((V, d), dtype=torch.float32, device="cuda")
    ld.readDequantizedDev("decoder.token_embedding", emb.data_ptr())
    h = _abi.prepare_rows_dev(_abi.FMT_F32, d, V, emb.data_ptr(), 4 * d)
    try:
        x = synth.normal_matrix(922, 1, d)
        X = torch.from_numpy(x).cuda()
        logits = torch.empty((1, V), dtype=torch.float32, device="cuda")
        _abi.gemm_prepared(h, 1, X.data_ptr(), logits.data_ptr())
        torch.cuda.synchronize()
    finally:
        _abi.prepared_free(h)
    deq = orc.dequantize_q8(q, s).reshape(V, d)
    ref = orc.matmul(x, np.ascontiguousarray(deq.T))
    got = logits.cpu().numpy()
    assert rel_err(got, ref) <= 1e-4
    assert int(np.argmax(got)) == int(np.argmax(ref))


# ------------------------------------- files written by the reference's exporter
EXPORTER = {0: "exporter_f32.tl", 1: "exporter_q8_0.tl", 2: "exporter_q4_0.tl", 3: "exporter_q8_k.tl",
            4: "exporter_f16.tl"}


@pytest.mark.parametrize("fmt", sorted(EXPORTER))
def test_exporter_files_to_hbm_and_matmul(orc, fmt):
    # tests/golden/tl/exporter_*.tl hold bytes tools/tl_format.py wrote
    # (tests/golden/make_tl_fixtures.py).  Every payload goes to HBM byte for
    # byte and dequantizes as the oracle says; the [64, 32] weight "w" then
    # multiplies through the C ABI exactly as the reference's matmul of that
    # in-memory tensor (dequantize-then-f32-accumulate).
    import torch
    path = os.path.join(GOLD, EXPORTER[fmt])
    data = open(path, "rb").read()
    ld = tl.ModelLoader(path)
    for e in orc.tl_parse(data)["tensors"]:
        name, shp = e[0], e[1]
        n = int(np.prod(shp))
        parts = orc.tl_payload(data, e, fmt)
        nbytes = _abi.weight_bytes(fmt, 1, n)
        buf = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        sc = torch.empty(max((n + 31) // 32, 1), dtype=torch.float32, device="cuda")
        scale = ld.readDev(name, fmt, buf.data_ptr(), sc.data_ptr() if fmt == 3 else None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(buf.cpu().numpy(), np.frombuffer(parts["data"].tobytes(), dtype=np.uint8))
        if fmt in (1, 2):
            assert np.float32(scale) == np.float32(parts["scale"])
        if fmt == 3:
            np.testing.assert_array_equal(sc.cpu().numpy()[: parts["scales"].size], parts["scales"])
        got = ld.getTensorDequantized(name).numpy().reshape(-1)
        np.testing.assert_array_equal(got.view(np.uint32), orc.tl_dequantize(fmt, parts, n).view(np.uint32))
    e = [t for t in orc.tl_parse(data)["tensors"] if t[0] == "w"][0]
    parts = orc.tl_payload(data, e, fmt)
    K, N = e[1]
    for M in (1, 5, 100):
        x = synth.normal_matrix(1001 + M, M, K)
        c = np.zeros((M, N), dtype=np.float32)
        if fmt == 0:
            _abi.sgemm(M, N, K, x, parts["data"].reshape(K, N), c)
            ref = orc.matmul(x, parts["data"].reshape(K, N))
        elif fmt == 1:
            _abi.sgemm_q8(M, N, K, x, parts["data"], parts["scale"], c)
            ref = orc.matmul_q8(x, parts["data"].reshape(K, N), parts["scale"])
        elif fmt == 2:
            _abi.sgemm_q4(M, N, K, x, parts["data"], parts["scale"], c)
            ref = orc.matmul_q4(x, parts["data"], K, N, parts["scale"])
        elif fmt == 3:
            _abi.sgemm_q8k(M, N, K, x, parts["data"], parts["scales"], 32, c)
            ref = orc.matmul_q8k(x, parts["data"].reshape(K, N), parts["scales"])
        else:
            _abi.sgemm_f16(M, N, K, x, parts["data"], c)
            ref = orc.matmul_f16(x, parts["data"].reshape(K, N))
        tol = 1e-4 if fmt in (0, 4) else 1e-3
        assert rel_err(c, ref) <= tol, (fmt, M, rel_err(c, ref))
