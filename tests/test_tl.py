""".tl files: the native reader (tml_tl_*) through the ModelLoader mirror,
against the reference's own fixtures and tests and against the oracle's
restatement of the format (oracle/oracle.py tl_parse / tl_payload /
tl_write).  CPU only: parsing and the typed getters need no GPU.

Fixtures under tests/golden/tl/ are the reference's committed test files,
unchanged: tests/fixtures/linear/{model,validation}.tl and
tests/fixtures/silero_vad/{model_tiny,validation}.tl.
"""
import os
import struct

import numpy as np
import pytest

from tomoul_amd import loader as tl, quantization as qz

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "tl")


def gold(name):
    return os.path.join(GOLD, name)


# ------------------------------------------------ the reference's own tests
def test_load_exported_model():
    # src/core/loader.zig:650-693 ("load exported model")
    ld = tl.ModelLoader(gold("linear_model.tl"))
    assert ld.tensorCount() == 2
    w = ld.getTensor("weight")
    assert w.shape == (1, 1) and abs(w.data[0] - 2.0) <= 1e-4
    b = ld.getTensor("bias")
    assert b.shape == (1,) and abs(b.data[0] - 1.0) <= 1e-4


def test_linear_model_parity():
    # tests/integration.zig:19-88: y = 2x + 1 on the validation pairs
    m, v = tl.ModelLoader(gold("linear_model.tl")), tl.ModelLoader(gold("linear_validation.tl"))
    w, b = m.getTensor("weight").data[0], m.getTensor("bias").data[0]
    for x_name, y_name in (("input", "expected_output"), ("input_zero", "expected_output_zero"),
                           ("input_negative", "expected_output_negative")):
        x, y = v.getTensor(x_name).data[0], v.getTensor(y_name).data[0]
        assert abs(x * w + b - y) <= 1e-4
    assert [v.getTensor(n).data[0] for n in ("input", "input_zero", "input_negative")] == [10.0, 0.0, -5.0]


def test_tiny_vad_fixture():
    # tests/integration.zig:96-160 (tiny VAD model and its validation file)
    ld = tl.ModelLoader(gold("silero_vad_model_tiny.tl"))
    assert ld.tensorCount() == 15
    for n in ("_model.stft.forward_basis_buffer", "_model.decoder.rnn.weight_ih", "_model.decoder.decoder.2.weight"):
        assert ld.hasTensor(n)
    stft = ld.getTensor("_model.stft.forward_basis_buffer")
    assert len(stft.shape) == 3 and stft.shape[0] == 32
    ih = ld.getTensor("_model.decoder.rnn.weight_ih")
    assert ih.shape == (32, 8)
    v = tl.ModelLoader(gold("silero_vad_validation.tl"))
    for n in ("input_zeros", "output_zeros", "input_ones", "output_ones"):
        assert v.hasTensor(n)
    assert v.getTensor("input_zeros").shape == (1, 64)
    out = v.getTensor("output_zeros").data[0]
    assert 0.0 <= out <= 1.0


def test_invalid_magic_and_missing_file(tmp_path):
    # src/core/loader.zig:625-648
    p = tmp_path / "bad.tl"
    p.write_bytes(b"BADM\x01\x00\x00\x00\x00\x00\x00\x00\x00\x00\x00\x00")
    with pytest.raises(tl.LoadError.InvalidMagic):
        tl.ModelLoader(str(p))
    with pytest.raises(tl.LoadError.FileNotFound):
        tl.ModelLoader("/nonexistent/path/model.tl")


# ----------------------------------------- agreement with the oracle's parse
@pytest.mark.parametrize("fname", ["linear_model.tl", "linear_validation.tl", "silero_vad_model_tiny.tl",
                                   "silero_vad_validation.tl"])
def test_fixture_tables_and_payloads_match_oracle(orc, fname):
    data = open(gold(fname), "rb").read()
    ref = orc.tl_parse(data)
    ld = tl.ModelLoader(gold(fname))
    assert ld.getQuantFormat() == ref["format"]
    assert ld.listTensors() == [e[0] for e in ref["tensors"]]
    for e in ref["tensors"]:
        info = ld.getTensorInfo(e[0])
        assert (info.shape, info.data_offset, info.data_size) == e[1:]
        got = ld.getTensor(e[0]).numpy().reshape(-1)
        want = orc.tl_payload(data, e, orc.TL_F32)["data"]
        np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


def _tensors(orc, fmt, rng):
    shapes = [(3, 5), (7,), (2, 3, 4), (1, 1), (33, 17), (64, 96)]
    out = []
    for i, shp in enumerate(shapes):
        w = (rng.standard_normal(int(np.prod(shp))) * 0.3).astype(np.float32)
        if fmt == orc.TL_F32:
            parts = {"data": w}
        elif fmt == orc.TL_F16:
            parts = {"data": orc.to_f16(w)}
        elif fmt == orc.TL_Q8_0:
            q, s = orc.quantize_q8(w)
            parts = {"scale": s, "data": q}
        elif fmt == orc.TL_Q4_0:
            p, s = orc.quantize_q4(w)
            parts = {"scale": s, "data": p}
        else:
            q, sc = orc.quantize_q8k(w)
            parts = {"scales": sc, "data": q}
        out.append((f"layer.{i}.weight", shp, parts))
    return out


@pytest.mark.parametrize("fmt", [0, 1, 2, 3, 4])
def test_round_trip_every_format(orc, tmp_path, fmt):
    # Files written by the oracle's restatement of tools/tl_format.py come
    # back byte for byte through the typed getter of their format; the other
    # quantized getters refuse them (UnsupportedQuantFormat) and getTensor
    # sees a size mismatch (CorruptedFile) unless the file is f32.
    rng = np.random.default_rng(100 + fmt)
    tensors = _tensors(orc, fmt, rng)
    data = orc.tl_write(tensors, fmt)
    p = tmp_path / "m.tl"
    p.write_bytes(data)
    for ld in (tl.ModelLoader(str(p)), tl.ModelLoader.initFromBytes(data)):
        assert ld.getQuantFormat() == fmt and ld.isQuantized() == (fmt != 0)
        assert ld.tensorCount() == len(tensors)
        for name, shp, parts in tensors:
            assert ld.getTensorInfo(name).shape == tuple(shp)
            if fmt == orc.TL_F32:
                got = ld.getTensor(name)
                np.testing.assert_array_equal(got.numpy().reshape(-1), parts["data"])
            elif fmt == orc.TL_F16:
                got = ld.getF16Tensor(name)
                np.testing.assert_array_equal(got.data, parts["data"])
            elif fmt == orc.TL_Q8_0:
                got = ld.getQuantizedTensorQ8(name)
                assert got.scale == np.float32(parts["scale"])
                np.testing.assert_array_equal(got.data, parts["data"])
            elif fmt == orc.TL_Q4_0:
                got = ld.getQuantizedTensorQ4(name)
                assert got.scale == np.float32(parts["scale"]) and got.shape == tuple(shp)
                np.testing.assert_array_equal(got.data, parts["data"])
            else:
                got = ld.getQuantizedTensorQ8K(name)
                np.testing.assert_array_equal(got.scales, parts["scales"])
                np.testing.assert_array_equal(got.data, parts["data"])
            getters = {1: ld.getQuantizedTensorQ8, 2: ld.getQuantizedTensorQ4, 3: ld.getQuantizedTensorQ8K,
                       4: ld.getF16Tensor}
            for g, fn in getters.items():
                if g != fmt:
                    with pytest.raises(tl.LoadError.UnsupportedQuantFormat):
                        fn(name)
            if fmt != orc.TL_F32:
                with pytest.raises(tl.LoadError.CorruptedFile):
                    ld.getTensor(name)
        with pytest.raises(tl.LoadError.TensorNotFound):
            ld.getTensor("missing")
        assert not ld.hasTensor("missing") and ld.getTensorInfo("missing") is None


def _expect(data, kind, tmp_path, orc):
    p = tmp_path / "x.tl"
    p.write_bytes(data)
    with pytest.raises(getattr(tl.LoadError, kind)):
        tl.ModelLoader(str(p))
    with pytest.raises(orc.TlParseError) as e:
        orc.tl_parse(data)
    assert e.value.kind == kind


def test_header_errors(orc, tmp_path):
    base = orc.tl_write([("w", (2, 2), {"data": np.ones(4, np.float32)})], 0)
    _expect(base[:15], "CorruptedFile", tmp_path, orc)
    _expect(base[:4] + struct.pack("<I", 2) + base[8:], "UnsupportedVersion", tmp_path, orc)
    _expect(base[:12] + bytes([9]) + base[13:], "UnsupportedQuantFormat", tmp_path, orc)
    # a table that claims two tensors but holds one
    _expect(base[:8] + struct.pack("<I", 2) + base[12:], "CorruptedFile", tmp_path, orc)
    # every cut inside the table is caught
    table_end = 16 + 4 + 1 + 4 + 8 + 16
    for cut in range(16, table_end):
        _expect(base[:cut], "CorruptedFile", tmp_path, orc)


def test_payload_errors(orc, tmp_path):
    w = np.arange(6, dtype=np.float32)
    good = orc.tl_write([("w", (2, 3), {"data": w})], 0)
    p = tmp_path / "t.tl"
    # payload past the end of the file: the table parses, the getter fails
    p.write_bytes(good[:-1])
    ld = tl.ModelLoader(str(p))
    with pytest.raises(tl.LoadError.CorruptedFile):
        ld.getTensor("w")
    # shape / size disagreement
    bad = orc.tl_write([("w", (2, 2), {"data": w})], 0)
    p.write_bytes(bad)
    with pytest.raises(tl.LoadError.CorruptedFile):
        tl.ModelLoader(str(p)).getTensor("w")
    # a Q8_K block count that does not match the shape
    q, sc = orc.quantize_q8k(np.linspace(-1, 1, 64).astype(np.float32))
    p.write_bytes(orc.tl_write([("k", (64,), {"scales": sc, "data": q, "num_blocks": 3})], 3))
    with pytest.raises(tl.LoadError.CorruptedFile):
        tl.ModelLoader(str(p)).getQuantizedTensorQ8K("k")


def test_duplicate_names_follow_the_hash_map(orc):
    # parseTensorEntry puts into a StringHashMap and appends to the name
    # list (loader.zig:218-219): the later entry wins, both names are listed,
    # tensorCount counts distinct names.
    data = orc.tl_write([("w", (1,), {"data": np.array([1.0], np.float32)}),
                         ("w", (1,), {"data": np.array([2.0], np.float32)})], 0)
    ld = tl.ModelLoader.initFromBytes(data)
    assert ld.tensorCount() == 1 and ld.listTensors() == ["w", "w"]
    assert ld.getTensor("w").data[0] == 2.0


def test_oracle_writer_matches_fixture_layout(orc):
    # The oracle's writer reproduces the reference fixture byte for byte
    # from the fixture's own tensors: the header, table and offsets follow
    # tools/tl_format.py exactly.
    data = open(gold("silero_vad_validation.tl"), "rb").read()
    ref = orc.tl_parse(data)
    tensors = [(e[0], e[1], orc.tl_payload(data, e, orc.TL_F32)) for e in ref["tensors"]]
    assert orc.tl_write(tensors, 0) == data


def test_oracle_dequantize_matches_definitions(orc):
    rng = np.random.default_rng(5)
    w = rng.standard_normal(77).astype(np.float32)
    q, s = orc.quantize_q8(w)
    np.testing.assert_array_equal(orc.tl_dequantize(1, {"data": q, "scale": s}, 77), orc.dequantize_q8(q, s))
    p, s4 = orc.quantize_q4(w)
    np.testing.assert_array_equal(orc.tl_dequantize(2, {"data": p, "scale": s4}, 77), orc.dequantize_q4(p, 77, s4))
    qk, sk = orc.quantize_q8k(w)
    np.testing.assert_array_equal(orc.tl_dequantize(3, {"data": qk, "scales": sk}, 77),
                                  orc.dequantize_q8k(qk, sk, 32))
    h = orc.to_f16(w)
    np.testing.assert_array_equal(orc.tl_dequantize(4, {"data": h}, 77), orc.from_f16(h))
    assert qz.BLOCK_SIZE == 32


def test_shape_product_that_wraps_is_corrupted(orc):
    # A crafted rank-4 shape of 2^16 x 2^16 x 2^16 x 2^16 elements: the
    # product wraps 2^64 to 0, which would match an empty payload.  The
    # getters compare the element count against what the payload can hold
    # and report CorruptedFile.
    import struct as st
    for fmt, payload in ((0, b""), (1, st.pack("<f", 1.0)), (2, st.pack("<f", 1.0))):
        head = b"TOUL" + st.pack("<II", 1, 1) + bytes([fmt, 0, 0, 0])
        table = st.pack("<I", 1) + b"w" + st.pack("<I", 4) + st.pack("<4I", *[1 << 16] * 4)
        start = len(head) + len(table) + 16
        data = head + table + st.pack("<QQ", start, len(payload)) + payload
        ld = tl.ModelLoader.initFromBytes(data)
        assert ld.getTensorInfo("w").shape == (1 << 16,) * 4
        getter = {0: ld.getTensor, 1: ld.getQuantizedTensorQ8, 2: ld.getQuantizedTensorQ4}[fmt]
        with pytest.raises(tl.LoadError.CorruptedFile):
            getter("w")
