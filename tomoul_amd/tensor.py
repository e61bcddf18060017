"""fp32 tensor container mirroring src/core/tensor.zig:12-52.

`data` is a flat float32 numpy array in row-major order and `shape` a tuple;
`Tensor.init` zero-fills like the reference.  The container lives on the host
(it is what the reference's callers hold); every matmul on it runs on the GPU.
"""
from __future__ import annotations

import numpy as np


class Tensor:
    __slots__ = ("data", "shape")

    def __init__(self, data: np.ndarray, shape):
        self.shape = tuple(int(s) for s in shape)
        n = 1
        for s in self.shape:
            n *= s
        data = np.ascontiguousarray(data, dtype=np.float32).reshape(-1)
        if data.size != n:
            raise ValueError(f"data has {data.size} elements, shape {self.shape} needs {n}")
        self.data = data

    @classmethod
    def init(cls, shape) -> "Tensor":
        """Zero-filled tensor (tensor.zig:40-41)."""
        n = 1
        for s in shape:
            n *= int(s)
        return cls(np.zeros(n, dtype=np.float32), shape)

    @classmethod
    def initWithData(cls, shape, data) -> "Tensor":  # noqa: N802 (reference name)
        return cls(np.asarray(data, dtype=np.float32), shape)

    @classmethod
    def from_numpy(cls, a: np.ndarray) -> "Tensor":
        return cls(np.asarray(a, dtype=np.float32), np.shape(a))

    def numpy(self) -> np.ndarray:
        return self.data.reshape(self.shape)

    def numel(self) -> int:
        return int(self.data.size)

    def fill(self, v: float) -> None:
        self.data[:] = np.float32(v)

    def __repr__(self) -> str:
        return f"Tensor(shape={self.shape})"
