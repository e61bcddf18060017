"""Weight-type dispatch of the reference's attention/transformer layers.

matmulWithWeight(input, weight)         src/core/attention.zig:114-130
                                        (f32, Q8_0, Q4_0, Q8_K and F16 weights)
matmulWithWeightBias(input, weight, b)  src/core/attention.zig:132-149
(duplicated at src/core/transformer.zig:129-166).  The weight's type selects
the kernel family; every branch runs on the GPU.  For quantized weights the
reference runs the matmul and then addBiasInPlace; here the bias is fused
into the kernel epilogue (one launch, no second pass over the output).

The feed-forward up-projections that the reference follows with a GELU pass
over the whole output are fused the same way:
  matmulWithWeightBiasGelu(input, weight, b)
      matmulWithWeightBias + ops.gelu (tanh form)
      src/core/transformer.zig:213-221, ops.zig:1947-1998
  matmulWithWeightBiasGeluExact(input, weight, b)
      ops.matmul + addBiasInPlace + ops.geluExact (erf form)
      src/models/whisper/encoder.zig:244-247, ops.zig:2029-2057
The activation is applied in the kernel epilogue after the bias, per output
element, with the reference's vector/scalar split of ops.gelu preserved (the
flat index decides, see include/tomoul_hip.h).

The down-projection followed by its residual connection is fused too:
  matmulWithWeightBiasResidual(input, weight, b, residual)
      matmulWithWeightBias + ops.addInPlace(out, residual)
      src/core/transformer.zig:223-228; Whisper's matmul + addBiasInPlace +
      ops.add(x1, fc2), src/models/whisper/encoder.zig:249-253

Weights quantized with one scale per output column (QuantizedTensorColsQ8 /
QuantizedTensorColsQ4, not reference types) take every one of these entry
points too; the column scales are applied in the same epilogue.
"""
from __future__ import annotations

from . import _abi, ops, quantization as qz
from .tensor import Tensor


def _check(a: Tensor, w_shape, bias: Tensor | None = None):
    if len(a.shape) != 2 or len(w_shape) != 2 or (bias is not None and len(bias.shape) != 1):
        raise ops.OpsError.InvalidShape(f"matmul needs 2-D operands, got {a.shape} and {w_shape}")
    if a.shape[1] != w_shape[0]:
        raise ops.OpsError.ShapeMismatch(f"inner dimensions differ: {a.shape} x {w_shape}")
    if bias is not None and bias.shape[0] != w_shape[1]:
        raise ops.OpsError.ShapeMismatch(f"bias has {bias.shape[0]} entries, output has {w_shape[1]} columns")
    return a.shape[0], w_shape[1], a.shape[1]


def matmulWithWeight(a: Tensor, weight) -> Tensor:  # noqa: N802 (reference name)
    if isinstance(weight, Tensor):
        return ops.matmul(a, weight)
    if isinstance(weight, qz.QuantizedTensorQ8):
        return qz.matmulF32Q8Simd(a, weight)
    if isinstance(weight, qz.QuantizedTensorQ4):
        return qz.matmulF32Q4Simd(a, weight)
    if isinstance(weight, qz.QuantizedTensorQ8K):
        return qz.matmulF32Q8KSimd(a, weight)
    if isinstance(weight, qz.F16Tensor):
        return qz.matmulF32F16(a, weight)
    if isinstance(weight, (qz.QuantizedTensorColsQ8, qz.QuantizedTensorColsQ4)):
        return qz.matmulF32Cols(a, weight)
    raise TypeError(f"unsupported weight type {type(weight).__name__}")


def matmulWithWeightBias(a: Tensor, weight, bias: Tensor) -> Tensor:  # noqa: N802
    if isinstance(weight, Tensor):
        return ops.matmulBias(a, weight, bias)
    m, n, k = _check(a, weight.shape, bias)
    out = Tensor.init((m, n))
    if isinstance(weight, qz.QuantizedTensorQ8):
        _abi.gemm(_abi.FMT_Q8_0, m, n, k, a.data, weight.data, out.data, scale=weight.scale, bias=bias.data)
    elif isinstance(weight, qz.QuantizedTensorQ4):
        _abi.gemm(_abi.FMT_Q4_0, m, n, k, a.data, weight.data, out.data, scale=weight.scale, bias=bias.data)
    elif isinstance(weight, qz.QuantizedTensorQ8K):
        _abi.gemm(_abi.FMT_Q8_K, m, n, k, a.data, weight.data, out.data, scales=weight.scales,
                  block=weight.block_size, bias=bias.data)
    elif isinstance(weight, qz.F16Tensor):
        _abi.gemm(_abi.FMT_F16, m, n, k, a.data, weight.data, out.data, bias=bias.data)
    elif isinstance(weight, (qz.QuantizedTensorColsQ8, qz.QuantizedTensorColsQ4)):
        fmt, kw = _weight_args(weight)
        _abi.gemm(fmt, m, n, k, a.data, weight.data, out.data, bias=bias.data, **kw)
    else:
        raise TypeError(f"unsupported weight type {type(weight).__name__}")
    return out


def _weight_args(weight) -> tuple[int, dict]:
    """(format, keyword arguments) of the C ABI for a weight of any type."""
    if isinstance(weight, Tensor):
        return _abi.FMT_F32, {}
    if isinstance(weight, qz.QuantizedTensorQ8):
        return _abi.FMT_Q8_0, {"scale": weight.scale}
    if isinstance(weight, qz.QuantizedTensorQ4):
        return _abi.FMT_Q4_0, {"scale": weight.scale}
    if isinstance(weight, qz.QuantizedTensorQ8K):
        return _abi.FMT_Q8_K, {"scales": weight.scales, "block": weight.block_size}
    if isinstance(weight, qz.F16Tensor):
        return _abi.FMT_F16, {}
    if isinstance(weight, qz.QuantizedTensorColsQ8):
        return _abi.FMT_Q8_0_PC, {"scales": weight.scales}
    if isinstance(weight, qz.QuantizedTensorColsQ4):
        return _abi.FMT_Q4_0_PC, {"scales": weight.scales}
    raise TypeError(f"unsupported weight type {type(weight).__name__}")


def _linear_act(a: Tensor, weight, bias: Tensor, act: int) -> Tensor:
    m, n, k = _check(a, weight.shape, bias)
    fmt, kw = _weight_args(weight)
    out = Tensor.init((m, n))
    _abi.gemm_act(fmt, m, n, k, a.data, weight.data, out.data, act=act, bias=bias.data, **kw)
    return out


def matmulWithWeightBiasResidual(a: Tensor, weight, bias: Tensor, residual: Tensor) -> Tensor:  # noqa: N802
    m, n, k = _check(a, weight.shape, bias)
    if tuple(residual.shape) != (m, n):
        raise ops.OpsError.ShapeMismatch(f"residual {residual.shape} does not match the output ({m}, {n})")
    fmt, kw = _weight_args(weight)
    out = Tensor.init((m, n))
    _abi.gemm_residual(fmt, m, n, k, a.data, weight.data, residual.data, out.data, bias=bias.data, **kw)
    return out


def matmulWithWeightBiasGelu(a: Tensor, weight, bias: Tensor) -> Tensor:  # noqa: N802
    return _linear_act(a, weight, bias, _abi.ACT_GELU_TANH)


def matmulWithWeightBiasGeluExact(a: Tensor, weight, bias: Tensor) -> Tensor:  # noqa: N802
    return _linear_act(a, weight, bias, _abi.ACT_GELU_ERF)
