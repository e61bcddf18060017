"""The fp32 matmul family of src/core/ops.zig, backed by the gfx950 kernels.

Same names, argument meaning and errors as the reference:
  matmul(a, b)              ops.zig:235-417   C = A.B
  matmulBias(a, b, bias)    ops.zig:422-471   C = A.B + bias (fused epilogue)
  matmulParallel(ctx, a, b) ops.zig:484-525   same result; ctx is ignored, as
                                              in the reference (ops.zig:485)
  matvec(a, x)              ops.zig:611-642   y = A.x
Shapes are validated before any device work and raise OpsError.InvalidShape
(not 2-D / bias not 1-D) or OpsError.ShapeMismatch (inner dimensions or bias
length).  The result is a fresh Tensor owned by the caller.
"""
from __future__ import annotations

import numpy as np

from . import _abi
from .tensor import Tensor


class OpsError(Exception):
    """Mirrors `OpsError` (src/core/ops.zig:47-52)."""


class InvalidShape(OpsError):
    pass


class ShapeMismatch(OpsError):
    pass


OpsError.InvalidShape = InvalidShape
OpsError.ShapeMismatch = ShapeMismatch


def _check_2d(a: Tensor, b: Tensor):
    if len(a.shape) != 2 or len(b.shape) != 2:
        raise InvalidShape(f"matmul needs 2-D tensors, got {a.shape} and {b.shape}")
    m, k = a.shape
    kb, n = b.shape
    if k != kb:
        raise ShapeMismatch(f"inner dimensions differ: {a.shape} x {b.shape}")
    return m, n, k


def matmul(a: Tensor, b: Tensor) -> Tensor:
    m, n, k = _check_2d(a, b)
    out = Tensor.init((m, n))
    _abi.sgemm(m, n, k, a.data, b.data, out.data, 1.0, 0.0)
    return out


def matmulBias(a: Tensor, b: Tensor, bias: Tensor) -> Tensor:  # noqa: N802
    if len(a.shape) != 2 or len(b.shape) != 2 or len(bias.shape) != 1:
        raise InvalidShape(f"matmulBias needs 2-D, 2-D, 1-D tensors, got {a.shape}, {b.shape}, {bias.shape}")
    m, n, k = _check_2d(a, b)
    if bias.shape[0] != n:
        raise ShapeMismatch(f"bias has {bias.shape[0]} entries, output has {n} columns")
    out = Tensor.init((m, n))
    _abi.sgemm_bias(m, n, k, a.data, b.data, bias.data, out.data)
    return out


def matmulParallel(ctx, a: Tensor, b: Tensor) -> Tensor:  # noqa: N802
    del ctx  # the GPU parallelises internally, as zblas does in the reference
    return matmul(a, b)


def matvec(a: Tensor, x: Tensor) -> Tensor:
    if len(a.shape) != 2 or len(x.shape) != 1:
        raise InvalidShape(f"matvec needs a 2-D matrix and a 1-D vector, got {a.shape}, {x.shape}")
    m, n = a.shape
    if x.shape[0] != n:
        raise ShapeMismatch(f"vector has {x.shape[0]} entries, matrix has {n} columns")
    out = Tensor.init((m,))
    _abi.sgemv(m, n, a.data, x.data, out.data, 1.0, 0.0)
    return out


def sgemm(m: int, n: int, k: int, a: np.ndarray, b: np.ndarray, c: np.ndarray, alpha: float = 1.0,
          beta: float = 0.0) -> None:
    """blas.sgemm (src/core/blas.zig:68-94): C = alpha*A.B + beta*C in place."""
    _abi.sgemm(m, n, k, np.ascontiguousarray(a, np.float32), np.ascontiguousarray(b, np.float32), c, alpha, beta)
