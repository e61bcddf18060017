"""CPU checks of the boundary: the built library loads, exports every
function include/tomoul_hip.h declares, and the host-side mirrors validate
shapes (raising the reference's errors) before any device work.  No GPU
compute is issued here."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest

from tomoul_amd import _abi, ops, quantization as qz
from tomoul_amd.tensor import Tensor

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "tomoul_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tml_(?:hip|tl)_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for required in ("tml_hip_sgemm", "tml_hip_sgemm_bias", "tml_hip_sgemv", "tml_hip_sgemm_q8",
                     "tml_hip_sgemm_q8k", "tml_hip_sgemm_q4", "tml_hip_gemm_dev", "tml_hip_quantize_dev"):
        assert required in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(_abi.LIB_PATH)
    for name in declared_functions():
        assert hasattr(lib, name), name
    # and the Python binding covers exactly the declared set
    assert sorted(_abi.SIGNATURES) == declared_functions()


def test_exported_symbols_have_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", _abi.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (tml_(?:hip|tl)_\w+)$", out, flags=re.M))
    assert set(declared_functions()) <= exported


def test_no_device_is_an_error_code_not_a_crash():
    # Without a GPU the library reports TML_ERR_NO_DEVICE (callers fall back
    # the way the reference HAL does); with one, init succeeds.
    code = _abi.lib().tml_hip_init()
    has_gpu = os.path.exists("/dev/kfd") and code == 0
    if not has_gpu:
        assert code == _abi.TML_ERR_NO_DEVICE
        assert b"device" in _abi.lib().tml_hip_last_error()
        a = np.ones((2, 2), np.float32)
        with pytest.raises(_abi.TmlError) as e:
            _abi.sgemm(2, 2, 2, a, a, a)
        assert e.value.code == _abi.TML_ERR_NO_DEVICE


def test_mirror_shape_errors():
    # src/core/ops.zig:236-249, 425-434 and quantization.zig:172-180
    with pytest.raises(ops.OpsError.ShapeMismatch):
        ops.matmul(Tensor.init((2, 3)), Tensor.init((2, 2)))
    with pytest.raises(ops.OpsError.InvalidShape):
        ops.matmul(Tensor.init((6,)), Tensor.init((6, 1)))
    with pytest.raises(ops.OpsError.InvalidShape):
        ops.matmulBias(Tensor.init((2, 3)), Tensor.init((3, 2)), Tensor.init((1, 2)))
    with pytest.raises(ops.OpsError.ShapeMismatch):
        ops.matmulBias(Tensor.init((2, 3)), Tensor.init((3, 2)), Tensor.init((3,)))
    with pytest.raises(ops.OpsError.ShapeMismatch):
        ops.matvec(Tensor.init((2, 3)), Tensor.init((2,)))
    q = qz.QuantizedTensorQ8(1.0, np.zeros(6, np.int8), (2, 3))
    with pytest.raises(qz.QuantError.ShapeMismatch):
        qz.matmulF32Q8Simd(Tensor.init((4, 4)), q)
    with pytest.raises(qz.QuantError.InvalidShape):
        qz.matmulF32Q8Simd(Tensor.init((4,)), q)


def test_q4_container_accessors():
    # quantization.zig:1185-1214 on the product container
    t = qz.QuantizedTensorQ4.init((8,))
    vals = [-7, -3, 0, 3, 7, -1, 1, -2]
    for i, v in enumerate(vals):
        t.set(i, v)
    assert [t.get(i) for i in range(8)] == vals
    assert t.data.tolist() == [0xD9, 0x30, 0xF7, 0xE1]
    assert t.compressionRatio() > 3.0


def test_tensor_container():
    t = Tensor.init((2, 3))
    assert t.data.dtype == np.float32 and not t.data.any() and t.shape == (2, 3)
    with pytest.raises(ValueError):
        Tensor(np.zeros(5, np.float32), (2, 3))


def test_c_program_links_and_runs(tmp_path):
    # The header compiles as C99 (-Wall -Werror), the library links into a C
    # program, and the no-GPU entry points behave (tests/c/abi_smoke.c).
    import shutil
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "abi_smoke"
    libdir = os.path.dirname(_abi.LIB_PATH)
    cmd = [gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", os.path.join(ROOT, "include"),
           os.path.join(ROOT, "tests", "c", "abi_smoke.c"), "-o", str(exe), "-L", libdir, "-ltomoul_hip",
           f"-Wl,-rpath,{libdir}", "-Wl,-rpath,/opt/rocm/lib", "-Wl,--allow-shlib-undefined"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    fixture = os.path.join(ROOT, "tests", "golden", "tl", "linear_model.tl")
    out = subprocess.run([str(exe), fixture], capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "y(10) = 21" in out.stdout


# Payload framing of each .tl format, written by the reference's exporter
# (tools/tl_format.py:309-360): bytes before the element data, and per scale.
_TL_FRAMING = {_abi.FMT_F32: (0, 0), _abi.FMT_F16: (0, 0), _abi.FMT_Q8_0: (4, 0), _abi.FMT_Q4_0: (4, 0),
               _abi.FMT_Q8_K: (4, 4)}


def test_weight_bytes_match_exporter_payloads(orc):
    """weight_bytes / scale_count against the payload sizes the reference's
    exporter wrote (tests/golden/tl/exporter_*.tl; odd lengths, rank 3 and an
    all-zero tensor among them): payload = framing + 4 * scales + data."""
    gold = os.path.join(ROOT, "tests", "golden", "tl")
    files = {_abi.FMT_F32: "exporter_f32.tl", _abi.FMT_Q8_0: "exporter_q8_0.tl", _abi.FMT_Q4_0: "exporter_q4_0.tl",
             _abi.FMT_Q8_K: "exporter_q8_k.tl", _abi.FMT_F16: "exporter_f16.tl"}
    for fmt, name in files.items():
        with open(os.path.join(gold, name), "rb") as f:
            parsed = orc.tl_parse(f.read())
        head, _ = _TL_FRAMING[fmt]
        for tname, shape, _off, size in parsed["tensors"]:
            n = int(np.prod(shape))
            ns = _abi.scale_count(fmt, 1, n)
            scale_bytes = 4 * ns if fmt == _abi.FMT_Q8_K else 0
            assert head + scale_bytes + _abi.weight_bytes(fmt, 1, n) == size, (fmt, tname, shape)
            # the [K,N] form of the same element count gives the same sizes
            k = shape[0]
            assert _abi.weight_bytes(fmt, k, n // k) == _abi.weight_bytes(fmt, 1, n)


@pytest.mark.parametrize("shape", [(5, 7), (64, 32), (37, 11), (1, 1)])
def test_weight_bytes_match_oracle_quantizers(orc, shape):
    """Every one of the seven formats against the size of what the oracle's
    quantizers (restating src/core/quantization.zig:98-129, :406-446,
    :721-754, :1859-1900 and their per-column forms) produce."""
    k, n = shape
    w = np.linspace(-1.0, 1.0, k * n, dtype=np.float32).reshape(k, n)
    q8, _ = orc.quantize_q8(w)
    q4, _ = orc.quantize_q4(w)
    q8k, s8k = orc.quantize_q8k(w)
    q8c, s8c = orc.quantize_q8_cols(w)
    q4c, s4c = orc.quantize_q4_cols(w)
    expect = {
        _abi.FMT_F32: (w.nbytes, 0), _abi.FMT_F16: (orc.to_f16(w).nbytes, 0), _abi.FMT_Q8_0: (q8.nbytes, 1),
        _abi.FMT_Q4_0: (q4.nbytes, 1), _abi.FMT_Q8_K: (q8k.nbytes, s8k.size), _abi.FMT_Q8_0_PC: (q8c.nbytes, s8c.size),
        _abi.FMT_Q4_0_PC: (q4c.nbytes, s4c.size),
    }
    assert sorted(expect) == sorted(_abi.FORMATS)
    for fmt, (nbytes, nscales) in expect.items():
        assert _abi.weight_bytes(fmt, k, n) == nbytes, fmt
        assert _abi.scale_count(fmt, k, n) == nscales, fmt


def test_weight_bytes_refuse_unknown_format():
    for bad in (5, 16, 19, -1):
        with pytest.raises(ValueError):
            _abi.weight_bytes(bad, 4, 4)
        with pytest.raises(ValueError):
            _abi.scale_count(bad, 4, 4)
