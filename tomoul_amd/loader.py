"""The .tl weight-file loader of src/core/loader.zig, backed by the native
reader in libtomoul_hip (tml_tl_*), plus the device-side layout producers
that turn its tensors into what the matmuls read.

ModelLoader(path)                 ModelLoader.init            loader.zig:55-91
ModelLoader.initFromBytes(data)   initFromBytes               :94-111
getTensor / getQuantizedTensorQ8 / getQuantizedTensorQ4 /
getQuantizedTensorQ8K / getF16Tensor                          :225-437
getTensorDequantized              (computed on the GPU)        :442-569
hasTensor / isQuantized / getQuantFormat / tensorCount /
listTensors / getTensorInfo                                   :572-600
loadQuantizedTransposedQ8 / Q4 / Q8K
    (src/models/xlm_roberta_punctuation/model.zig:1272-1362): dequantize,
    transpose [out,in] -> [in,out], re-quantize -- on the GPU, bit for bit.

Errors are LoadError subclasses with the reference's names.  Parsing and the
typed getters need no GPU; getTensorDequantized and the transposing loaders
do.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np

from . import _abi, quantization as qz
from .tensor import Tensor


class LoadError(Exception):
    """Mirrors `LoadError` (src/core/loader.zig:11-20)."""


class InvalidMagic(LoadError):
    pass


class UnsupportedVersion(LoadError):
    pass


class CorruptedFile(LoadError):
    pass


class TensorNotFound(LoadError):
    pass


class FileNotFound(LoadError):
    pass


class UnsupportedQuantFormat(LoadError):
    pass


for _cls in (InvalidMagic, UnsupportedVersion, CorruptedFile, TensorNotFound, FileNotFound, UnsupportedQuantFormat):
    setattr(LoadError, _cls.__name__, _cls)

_CODES = {
    _abi.TML_ERR_INVALID_MAGIC: InvalidMagic,
    _abi.TML_ERR_UNSUPPORTED_VERSION: UnsupportedVersion,
    _abi.TML_ERR_CORRUPTED_FILE: CorruptedFile,
    _abi.TML_ERR_TENSOR_NOT_FOUND: TensorNotFound,
    _abi.TML_ERR_FILE_NOT_FOUND: FileNotFound,
    _abi.TML_ERR_UNSUPPORTED_QUANT_FORMAT: UnsupportedQuantFormat,
}


class QuantFormat:
    """src/core/loader.zig:23-29 (the header's quant-format byte)."""
    f32 = _abi.FMT_F32
    q8_0 = _abi.FMT_Q8_0
    q4_0 = _abi.FMT_Q4_0
    q8_k = _abi.FMT_Q8_K
    f16 = _abi.FMT_F16


@dataclass
class TensorInfo:
    name: str
    shape: tuple
    data_offset: int
    data_size: int


def _check(code: int) -> None:
    if code != _abi.TML_OK:
        msg = _abi.lib().tml_hip_last_error().decode(errors="replace")
        cls = _CODES.get(code)
        if cls is not None:
            raise cls(msg)
        raise _abi.TmlError(code, msg)


def _numel(shape) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


class ModelLoader:
    def __init__(self, path: str | None = None, *, _handle=None, _keep=None):
        self._keep = _keep  # bytes borrowed by initFromBytes
        if _handle is not None:
            self._h = _handle
            return
        h = ctypes.c_void_p()
        _check(_abi.lib().tml_tl_open(str(path).encode(), ctypes.byref(h)))
        self._h = h

    @classmethod
    def init(cls, path: str) -> "ModelLoader":
        return cls(path)

    @classmethod
    def initFromBytes(cls, data: bytes) -> "ModelLoader":  # noqa: N802
        buf = np.frombuffer(bytes(data), dtype=np.uint8).copy()
        h = ctypes.c_void_p()
        _check(_abi.lib().tml_tl_open_bytes(buf.ctypes.data if buf.size else None, buf.size, ctypes.byref(h)))
        return cls(_handle=h, _keep=buf)

    def deinit(self) -> None:
        if self._h is not None:
            _abi.lib().tml_tl_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.deinit()
        except Exception:  # pragma: no cover - interpreter shutdown
            pass

    # ---------------------------------------------------------- metadata
    def getQuantFormat(self) -> int:  # noqa: N802
        return int(_abi.lib().tml_tl_format(self._h))

    def isQuantized(self) -> bool:  # noqa: N802
        return self.getQuantFormat() != QuantFormat.f32

    def tensorCount(self) -> int:  # noqa: N802
        return int(_abi.lib().tml_tl_count(self._h))

    def listTensors(self) -> list[str]:  # noqa: N802
        out, i = [], 0
        while True:
            name = _abi.lib().tml_tl_name(self._h, i)
            if name is None:
                return out
            out.append(name.decode())
            i += 1

    def getTensorInfo(self, name: str) -> TensorInfo | None:  # noqa: N802
        dims = (ctypes.c_int64 * 16)()
        nd, off, size = ctypes.c_int(), ctypes.c_uint64(), ctypes.c_uint64()
        code = _abi.lib().tml_tl_info(self._h, name.encode(), dims, 16, ctypes.byref(nd), ctypes.byref(off),
                                      ctypes.byref(size))
        if code == _abi.TML_ERR_TENSOR_NOT_FOUND:
            return None
        _check(code)
        if nd.value > 16:
            raise LoadError(f"tensor {name} has rank {nd.value} > 16")
        return TensorInfo(name, tuple(int(dims[i]) for i in range(nd.value)), off.value, size.value)

    def hasTensor(self, name: str) -> bool:  # noqa: N802
        return self.getTensorInfo(name) is not None

    def _shape(self, name: str) -> tuple:
        info = self.getTensorInfo(name)
        if info is None:
            raise TensorNotFound(f"no tensor named {name}")
        # No format stores more than two elements per payload byte: a shape
        # claiming more (e.g. one whose product wraps 2^64 in a native
        # reader) is CorruptedFile before any buffer is sized from it, the
        # rule the native getters apply.
        if _numel(info.shape) > 2 * info.data_size:
            raise CorruptedFile("tensor shape holds more elements than its payload")
        return info.shape

    def _read(self, name: str, getter: int, data: np.ndarray, scales: np.ndarray | None) -> float:
        scale = ctypes.c_float(0.0)
        _check(_abi.lib().tml_tl_read(self._h, name.encode(), getter, data.ctypes.data if data.size else None,
                                      scales.ctypes.data if scales is not None and scales.size else None,
                                      ctypes.byref(scale)))
        return float(scale.value)

    # ----------------------------------------------------------- getters
    def getTensor(self, name: str) -> Tensor:  # noqa: N802
        self._shape(name)
        info = self.getTensorInfo(name)
        data = np.empty(_numel(info.shape), dtype=np.float32)
        self._read(name, QuantFormat.f32, data, None)
        return Tensor.from_numpy(data.reshape(info.shape) if info.shape else data)

    def getQuantizedTensorQ8(self, name: str) -> qz.QuantizedTensorQ8:  # noqa: N802
        if self.getQuantFormat() != QuantFormat.q8_0:
            raise UnsupportedQuantFormat("file is not Q8_0")
        shape = self._shape(name)
        data = np.empty(_numel(shape), dtype=np.int8)
        scale = self._read(name, QuantFormat.q8_0, data, None)
        return qz.QuantizedTensorQ8(scale, data, shape)

    def getQuantizedTensorQ4(self, name: str) -> qz.QuantizedTensorQ4:  # noqa: N802
        if self.getQuantFormat() != QuantFormat.q4_0:
            raise UnsupportedQuantFormat("file is not Q4_0")
        shape = self._shape(name)
        data = np.empty((_numel(shape) + 1) // 2, dtype=np.uint8)
        scale = self._read(name, QuantFormat.q4_0, data, None)
        return qz.QuantizedTensorQ4(scale, data, shape)

    def getQuantizedTensorQ8K(self, name: str) -> qz.QuantizedTensorQ8K:  # noqa: N802
        if self.getQuantFormat() != QuantFormat.q8_k:
            raise UnsupportedQuantFormat("file is not Q8_K")
        shape = self._shape(name)
        n = _numel(shape)
        data = np.empty(n, dtype=np.int8)
        scales = np.empty((n + qz.BLOCK_SIZE - 1) // qz.BLOCK_SIZE, dtype=np.float32)
        self._read(name, QuantFormat.q8_k, data, scales)
        return qz.QuantizedTensorQ8K(scales, data, shape)

    def getF16Tensor(self, name: str) -> qz.F16Tensor:  # noqa: N802
        if self.getQuantFormat() != QuantFormat.f16:
            raise UnsupportedQuantFormat("file is not F16")
        shape = self._shape(name)
        data = np.empty(_numel(shape), dtype=np.uint16)
        self._read(name, QuantFormat.f16, data, None)
        return qz.F16Tensor(data, shape)

    # ------------------------------------------------------ device paths
    def readDev(self, name: str, getter: int, data_ptr: int, scales_ptr: int | None = None,  # noqa: N802
                stream: int | None = None) -> float:
        """The getter's payload straight into device memory; returns the
        per-tensor scale (Q8_0 / Q4_0).  No reference counterpart."""
        scale = ctypes.c_float(0.0)
        _check(_abi.lib().tml_tl_read_dev(self._h, name.encode(), getter, data_ptr, scales_ptr, ctypes.byref(scale),
                                          stream))
        return float(scale.value)

    def readDequantizedDev(self, name: str, out_ptr: int, stream: int | None = None) -> None:  # noqa: N802
        _check(_abi.lib().tml_tl_read_dequantized_dev(self._h, name.encode(), out_ptr, stream))

    def getTensorDequantized(self, name: str) -> Tensor:  # noqa: N802
        import torch
        shape = self._shape(name)
        out = torch.empty(_numel(shape), dtype=torch.float32, device="cuda")
        self.readDequantizedDev(name, out.data_ptr())
        torch.cuda.synchronize()
        data = out.cpu().numpy()
        return Tensor.from_numpy(data.reshape(shape) if shape else data)


# ------------------------------------------- XLM-R transposing loaders
def _transposed(loader: ModelLoader, name: str, fmt: int):
    import torch
    shape = loader._shape(name)
    if len(shape) != 2:
        raise LoadError(f"{name}: transposing loaders need a 2-D tensor, got {shape}")
    rows, cols = shape
    n = rows * cols
    qbytes = (n + 1) // 2 if fmt == QuantFormat.q4_0 else n
    nsc = (n + qz.BLOCK_SIZE - 1) // qz.BLOCK_SIZE if fmt == QuantFormat.q8_k else 1
    q_in = torch.empty(max(qbytes, 1), dtype=torch.uint8, device="cuda")
    s_in = torch.empty(max(nsc, 1), dtype=torch.float32, device="cuda")
    q_out = torch.empty(max(qbytes, 1), dtype=torch.uint8, device="cuda")
    s_out = torch.empty(max(nsc, 1), dtype=torch.float32, device="cuda")
    scale = loader.readDev(name, fmt, q_in.data_ptr(), s_in.data_ptr() if fmt == QuantFormat.q8_k else None)
    _abi.transpose_requant_dev(fmt, rows, cols, q_in.data_ptr(), q_out.data_ptr(), s_out.data_ptr(), scale=scale,
                               scales_ptr=s_in.data_ptr() if fmt == QuantFormat.q8_k else None)
    torch.cuda.synchronize()
    return q_out.cpu().numpy()[:qbytes], s_out.cpu().numpy()[:nsc], (cols, rows)


def loadQuantizedTransposedQ8(loader: ModelLoader, name: str) -> qz.QuantizedTensorQ8:  # noqa: N802
    if loader.getQuantFormat() != QuantFormat.q8_0:
        raise UnsupportedQuantFormat("file is not Q8_0")
    q, s, shape = _transposed(loader, name, QuantFormat.q8_0)
    return qz.QuantizedTensorQ8(float(s[0]), q.view(np.int8), shape)


def loadQuantizedTransposedQ4(loader: ModelLoader, name: str) -> qz.QuantizedTensorQ4:  # noqa: N802
    if loader.getQuantFormat() != QuantFormat.q4_0:
        raise UnsupportedQuantFormat("file is not Q4_0")
    q, s, shape = _transposed(loader, name, QuantFormat.q4_0)
    return qz.QuantizedTensorQ4(float(s[0]), q, shape)


def loadQuantizedTransposedQ8K(loader: ModelLoader, name: str) -> qz.QuantizedTensorQ8K:  # noqa: N802
    if loader.getQuantFormat() != QuantFormat.q8_k:
        raise UnsupportedQuantFormat("file is not Q8_K")
    q, s, shape = _transposed(loader, name, QuantFormat.q8_k)
    return qz.QuantizedTensorQ8K(s, q.view(np.int8), shape)
