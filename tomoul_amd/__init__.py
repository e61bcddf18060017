"""tomoul_amd -- MI355X (gfx950) backend for Tomoul's matrix-multiply hot path.

  tomoul_amd.ops           ops.matmul / matmulBias / matmulParallel / matvec
  tomoul_amd.quantization  Q8_0 / Q8_K / Q4_0 containers, quantizers and
                           weight-only matmuls
  tomoul_amd.dispatch      matmulWithWeight[Bias] (the weight-type dispatch)
  tomoul_amd._abi          ctypes binding of include/tomoul_hip.h
  tomoul_amd.build         builds libtomoul_hip.so with hipcc

All compute runs in libtomoul_hip.so; importing an op module does not load
it, the first call does (and raises if it has not been built).
"""
from .tensor import Tensor  # noqa: F401

__all__ = ["Tensor"]
