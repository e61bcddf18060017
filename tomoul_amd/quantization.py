"""Weight-only quantized matmuls of src/core/quantization.zig on the GPU.

Containers keep the reference's in-memory layouts ([K,N] row-major):
  QuantizedTensorQ8   scale + int8 data          (quantization.zig:39-90)
  QuantizedTensorQ8K  f32 scale per 32 flattened elements + int8 data
                                                  (quantization.zig:327-403)
  QuantizedTensorQ4   scale + packed nibbles, low nibble = even index
                                                  (quantization.zig:627-711)
quantizeQ8 / quantizeQ8K / quantizeQ4 run the bit-exact on-device quantizers;
matmulF32Q8Simd / matmulF32Q8KSimd / matmulF32Q4Simd run the GPU GEMV (M <= 8)
or MFMA GEMM (M > 8).  Errors mirror QuantError (quantization.zig:25-30).
"""
from __future__ import annotations

import numpy as np

from . import _abi
from .tensor import Tensor

BLOCK_SIZE = 32  # quantization.zig:322


class QuantError(Exception):
    pass


class InvalidShape(QuantError):
    pass


class ShapeMismatch(QuantError):
    pass


QuantError.InvalidShape = InvalidShape
QuantError.ShapeMismatch = ShapeMismatch


def _numel(shape) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n


class QuantizedTensorQ8:
    def __init__(self, scale: float, data: np.ndarray, shape):
        self.scale = float(scale)
        self.data = np.ascontiguousarray(data, dtype=np.int8).reshape(-1)
        self.shape = tuple(int(s) for s in shape)

    def numel(self) -> int:
        return _numel(self.shape)

    def sizeBytes(self) -> int:  # noqa: N802
        return 4 + self.data.size

    def compressionRatio(self) -> float:  # noqa: N802
        return self.numel() * 4 / self.sizeBytes()


class QuantizedTensorQ8K:
    def __init__(self, scales: np.ndarray, data: np.ndarray, shape, block_size: int = BLOCK_SIZE):
        self.scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
        self.data = np.ascontiguousarray(data, dtype=np.int8).reshape(-1)
        self.shape = tuple(int(s) for s in shape)
        self.block_size = int(block_size)
        self.num_blocks = self.scales.size
        self.element_count = _numel(self.shape)

    def numel(self) -> int:
        return self.element_count

    def sizeBytes(self) -> int:  # noqa: N802
        return self.scales.size * 4 + self.data.size

    def compressionRatio(self) -> float:  # noqa: N802
        return self.numel() * 4 / self.sizeBytes()


class QuantizedTensorQ4:
    def __init__(self, scale: float, data: np.ndarray, shape):
        self.scale = float(scale)
        self.data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        self.shape = tuple(int(s) for s in shape)
        self.element_count = _numel(self.shape)

    @classmethod
    def init(cls, shape) -> "QuantizedTensorQ4":
        n = _numel(shape)
        return cls(0.0, np.zeros((n + 1) // 2, dtype=np.uint8), shape)

    def numel(self) -> int:
        return self.element_count

    def sizeBytes(self) -> int:  # noqa: N802
        return 4 + self.data.size

    def compressionRatio(self) -> float:  # noqa: N802
        return self.numel() * 4 / self.sizeBytes()

    def get(self, idx: int) -> int:
        """Nibble accessor (quantization.zig:682-695): two's-complement i4."""
        b = int(self.data[idx // 2])
        nib = (b & 0x0F) if idx % 2 == 0 else (b >> 4)
        return nib - 16 if nib & 0x08 else nib

    def set(self, idx: int, value: int) -> None:
        """Nibble store, clamped to [-7, 7] (quantization.zig:698-710)."""
        v = max(-7, min(7, int(value))) & 0x0F
        i = idx // 2
        b = int(self.data[i])
        self.data[i] = (b & 0xF0) | v if idx % 2 == 0 else (b & 0x0F) | (v << 4)


class F16Tensor:
    """F16Tensor (quantization.zig:1859-1905): binary16 weights, held as
    their uint16 bit patterns."""

    def __init__(self, data: np.ndarray, shape):
        self.data = np.ascontiguousarray(data, dtype=np.uint16).reshape(-1)
        self.shape = tuple(int(s) for s in shape)

    @classmethod
    def init(cls, shape) -> "F16Tensor":
        return cls(np.zeros(_numel(shape), dtype=np.uint16), shape)

    def numel(self) -> int:
        return _numel(self.shape)

    def sizeBytes(self) -> int:  # noqa: N802
        return self.numel() * 2

    def compressionRatio(self) -> float:  # noqa: N802
        return self.numel() * 4 / self.sizeBytes()


class QuantizedTensorColsQ8:
    """Not a reference type: a [K,N] weight quantized like QuantizedTensorQ8
    but with one scale per output column n (column n alone goes through the
    reference's Q8_0 quantizer, quantization.zig:39-90)."""

    def __init__(self, scales: np.ndarray, data: np.ndarray, shape):
        self.scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
        self.data = np.ascontiguousarray(data, dtype=np.int8).reshape(-1)
        self.shape = tuple(int(s) for s in shape)

    def numel(self) -> int:
        return _numel(self.shape)

    def sizeBytes(self) -> int:  # noqa: N802
        return 4 * self.scales.size + self.data.size

    def compressionRatio(self) -> float:  # noqa: N802
        return self.numel() * 4 / self.sizeBytes()


class QuantizedTensorColsQ4:
    """Not a reference type: Q4_0 nibbles (packed over the flattened [K,N],
    low nibble = even index, as QuantizedTensorQ4) with one scale per output
    column."""

    def __init__(self, scales: np.ndarray, data: np.ndarray, shape):
        self.scales = np.ascontiguousarray(scales, dtype=np.float32).reshape(-1)
        self.data = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
        self.shape = tuple(int(s) for s in shape)

    def numel(self) -> int:
        return _numel(self.shape)

    def sizeBytes(self) -> int:  # noqa: N802
        return 4 * self.scales.size + self.data.size

    def compressionRatio(self) -> float:  # noqa: N802
        return self.numel() * 4 / self.sizeBytes()


# ---------------------------------------------------------------- quantizers
def toF16(t: Tensor) -> F16Tensor:  # noqa: N802
    """toF16 (quantization.zig:1907-1917), on the GPU: round to nearest even."""
    h = np.empty(t.numel(), dtype=np.uint16)
    _abi.quantize(_abi.FMT_F16, t.data, h, None)
    return F16Tensor(h, t.shape)


def quantizeQ8(t: Tensor) -> QuantizedTensorQ8:  # noqa: N802
    q = np.empty(t.numel(), dtype=np.int8)
    s = np.empty(1, dtype=np.float32)
    _abi.quantize(_abi.FMT_Q8_0, t.data, q, s)
    return QuantizedTensorQ8(float(s[0]), q, t.shape)


def quantizeQ8K(t: Tensor) -> QuantizedTensorQ8K:  # noqa: N802
    n = t.numel()
    q = np.empty(n, dtype=np.int8)
    s = np.empty(max((n + BLOCK_SIZE - 1) // BLOCK_SIZE, 1), dtype=np.float32)
    _abi.quantize(_abi.FMT_Q8_K, t.data, q, s)
    return QuantizedTensorQ8K(s[: (n + BLOCK_SIZE - 1) // BLOCK_SIZE], q, t.shape)


def quantizeQ4(t: Tensor) -> QuantizedTensorQ4:  # noqa: N802
    n = t.numel()
    q = np.empty(max((n + 1) // 2, 1), dtype=np.uint8)
    s = np.empty(1, dtype=np.float32)
    _abi.quantize(_abi.FMT_Q4_0, t.data, q, s)
    return QuantizedTensorQ4(float(s[0]), q[: (n + 1) // 2], t.shape)


def _cols_shape(t: Tensor):
    if len(t.shape) != 2:
        raise InvalidShape(f"per-column quantization needs a 2-D [K,N] tensor, got {t.shape}")
    return int(t.shape[0]), int(t.shape[1])


def quantizeColsQ8(t: Tensor) -> QuantizedTensorColsQ8:  # noqa: N802
    """Per-output-column int8 (an extension; bit-exact on the GPU)."""
    k, n = _cols_shape(t)
    q = np.empty(max(k * n, 1), dtype=np.int8)
    s = np.empty(max(n, 1), dtype=np.float32)
    _abi.quantize_cols(_abi.FMT_Q8_0_PC, t.data.reshape(k, n), q, s)
    return QuantizedTensorColsQ8(s[:n], q[: k * n], t.shape)


def quantizeColsQ4(t: Tensor) -> QuantizedTensorColsQ4:  # noqa: N802
    """Per-output-column int4 (an extension; bit-exact on the GPU)."""
    k, n = _cols_shape(t)
    q = np.empty(max((k * n + 1) // 2, 1), dtype=np.uint8)
    s = np.empty(max(n, 1), dtype=np.float32)
    _abi.quantize_cols(_abi.FMT_Q4_0_PC, t.data.reshape(k, n), q, s)
    return QuantizedTensorColsQ4(s[:n], q[: (k * n + 1) // 2], t.shape)


# ---------------------------------------------------------------- matmuls
def _shape(a: Tensor, b):
    if len(a.shape) != 2 or len(b.shape) != 2:
        raise InvalidShape(f"matmul needs 2-D tensors, got {a.shape} and {b.shape}")
    m, k = a.shape
    kb, n = b.shape
    if k != kb:
        raise ShapeMismatch(f"inner dimensions differ: {a.shape} x {b.shape}")
    return m, n, k


def matmulF32Q8Simd(a: Tensor, b: QuantizedTensorQ8) -> Tensor:  # noqa: N802
    m, n, k = _shape(a, b)
    out = Tensor.init((m, n))
    _abi.sgemm_q8(m, n, k, a.data, b.data, b.scale, out.data)
    return out


def matmulF32Q8KSimd(a: Tensor, b: QuantizedTensorQ8K) -> Tensor:  # noqa: N802
    m, n, k = _shape(a, b)
    out = Tensor.init((m, n))
    _abi.sgemm_q8k(m, n, k, a.data, b.data, b.scales, b.block_size, out.data)
    return out


def matmulF32F16(a: Tensor, b: F16Tensor) -> Tensor:  # noqa: N802
    """matmulF32F16 (quantization.zig:1921-1962): f32 activations x f16
    weights, f32 accumulation."""
    m, n, k = _shape(a, b)
    out = Tensor.init((m, n))
    _abi.sgemm_f16(m, n, k, a.data, b.data, out.data)
    return out


def matmulF32Q4Simd(a: Tensor, b: QuantizedTensorQ4) -> Tensor:  # noqa: N802
    m, n, k = _shape(a, b)
    out = Tensor.init((m, n))
    _abi.sgemm_q4(m, n, k, a.data, b.data, b.scale, out.data)
    return out


def matmulF32Cols(a: Tensor, b) -> Tensor:  # noqa: N802
    """f32 activations x a per-column quantized weight: column n of the
    product is scaled by b.scales[n] (an extension)."""
    m, n, k = _shape(a, b)
    fmt = _abi.FMT_Q8_0_PC if isinstance(b, QuantizedTensorColsQ8) else _abi.FMT_Q4_0_PC
    out = Tensor.init((m, n))
    _abi.gemm(fmt, m, n, k, a.data, b.data, out.data, scales=b.scales)
    return out
