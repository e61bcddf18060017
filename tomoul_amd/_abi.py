"""ctypes binding of include/tomoul_hip.h (libtomoul_hip.so).

This is the Python-side counterpart of the Zig shim a Tomoul build would use
(`extern "c"` declarations, the src/core/blas.zig:24-54 pattern).  Loading
fails loudly when the library has not been built: there is no CPU fallback.
Host-pointer calls take numpy arrays; "_dev" calls take raw device pointers
(ints, e.g. torch's tensor.data_ptr()) and a hipStream_t as an int.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libtomoul_hip.so")

TML_OK = 0
TML_ERR_INVALID_SHAPE = -1
TML_ERR_SHAPE_MISMATCH = -2
TML_ERR_OUT_OF_MEMORY = -3
TML_ERR_INVALID_FORMAT = -4
TML_ERR_INVALID_ARG = -5
TML_ERR_NO_DEVICE = -6
TML_ERR_HIP = -7
TML_ERR_INVALID_MAGIC = -8
TML_ERR_UNSUPPORTED_VERSION = -9
TML_ERR_CORRUPTED_FILE = -10
TML_ERR_TENSOR_NOT_FOUND = -11
TML_ERR_FILE_NOT_FOUND = -12
TML_ERR_UNSUPPORTED_QUANT_FORMAT = -13

FMT_F32, FMT_Q8_0, FMT_Q4_0, FMT_Q8_K, FMT_F16 = 0, 1, 2, 3, 4
FMT_Q8_0_PC, FMT_Q4_0_PC = 17, 18  # per-output-column scales (not reference formats)
ACT_NONE, ACT_GELU_ERF, ACT_GELU_TANH = 0, 1, 2
FORMATS = (FMT_F32, FMT_Q8_0, FMT_Q4_0, FMT_Q8_K, FMT_F16, FMT_Q8_0_PC, FMT_Q4_0_PC)


def weight_bytes(fmt: int, k: int, n: int) -> int:
    """Bytes of a [K,N] weight's element data in format fmt (scales excluded).

    The layouts are the reference's in-memory tensors: f32 `[]f32`
    (src/core/tensor.zig:12-18), Q8_0 `data: []i8` (src/core/quantization.zig:39-90),
    Q8_K `data: []i8` (:327-403), Q4_0 `(n+1)/2` packed bytes (:627-711),
    F16 `[]f16` (:1859-1900); the per-column formats store Q8_0 / Q4_0's bytes.
    Raises ValueError for a format it does not know, so that a new format
    cannot silently take another format's size.
    """
    e = int(k) * int(n)
    if fmt == FMT_F32:
        return 4 * e
    if fmt == FMT_F16:
        return 2 * e
    if fmt in (FMT_Q8_0, FMT_Q8_K, FMT_Q8_0_PC):
        return e
    if fmt in (FMT_Q4_0, FMT_Q4_0_PC):
        return (e + 1) // 2
    raise ValueError(f"unknown weight format {fmt}")


def scale_count(fmt: int, k: int, n: int, block: int = 32) -> int:
    """f32 scales a [K,N] weight in format fmt carries: 0 (f32 / f16), 1 (Q8_0 /
    Q4_0, per tensor), ceil(K*N/block) (Q8_K, src/core/quantization.zig:327-403),
    N (per-column formats).  Raises ValueError for an unknown format."""
    if fmt in (FMT_F32, FMT_F16):
        return 0
    if fmt in (FMT_Q8_0, FMT_Q4_0):
        return 1
    if fmt == FMT_Q8_K:
        return -(-int(k) * int(n) // int(block))
    if fmt in (FMT_Q8_0_PC, FMT_Q4_0_PC):
        return int(n)
    raise ValueError(f"unknown weight format {fmt}")


# Every symbol the header declares, with its ctypes signature.
_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_f = ctypes.c_float
SIGNATURES = {
    "tml_hip_init": (ctypes.c_int, []),
    "tml_hip_shutdown": (None, []),
    "tml_hip_last_error": (ctypes.c_char_p, []),
    "tml_hip_device_name": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_size_t]),
    "tml_hip_sgemm": (ctypes.c_int, [_i64, _i64, _i64, _vp, _vp, _vp, _f, _f]),
    "tml_hip_sgemm_bias": (ctypes.c_int, [_i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "tml_hip_sgemv": (ctypes.c_int, [_i64, _i64, _vp, _vp, _vp, _f, _f]),
    "tml_hip_sgemm_q8": (ctypes.c_int, [_i64, _i64, _i64, _vp, _vp, _f, _vp]),
    "tml_hip_sgemm_q8k": (ctypes.c_int, [_i64, _i64, _i64, _vp, _vp, _vp, _i64, _vp]),
    "tml_hip_sgemm_q4": (ctypes.c_int, [_i64, _i64, _i64, _vp, _vp, _f, _vp]),
    "tml_hip_gemm": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _i64, _vp, _vp, _f, _vp, _i64, _vp, _vp]),
    "tml_hip_quantize": (ctypes.c_int, [ctypes.c_int, _i64, _vp, _vp, _vp]),
    "tml_hip_weight_register": (ctypes.c_int, [_vp, ctypes.c_size_t]),
    "tml_hip_weight_release": (ctypes.c_int, [_vp]),
    "tml_hip_gemm_dev": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _i64, _vp, _vp, _f, _vp, _i64, _vp, _vp, _f, _f,
                                        _vp]),
    "tml_hip_quantize_dev": (ctypes.c_int, [ctypes.c_int, _i64, _vp, _vp, _vp, _vp]),
    "tml_hip_prepare_dev": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _vp, _f, _vp, ctypes.POINTER(_vp)]),
    "tml_hip_gemm_prepared": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, _f, _f, _vp]),
    "tml_hip_prepared_free": (ctypes.c_int, [_vp]),
    "tml_hip_gemm_act": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _i64, _vp, _vp, _f, _vp, _i64, _vp, ctypes.c_int,
                                        _vp]),
    "tml_hip_prepare_rows_dev": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _vp, _i64, _f, _vp,
                                                ctypes.POINTER(ctypes.c_void_p)]),
    "tml_hip_sgemm_f16": (ctypes.c_int, [_i64, _i64, _i64, _vp, _vp, _vp]),
    "tml_hip_gemm_residual": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _i64, _vp, _vp, _f, _vp, _i64, _vp, _vp,
                                             _vp]),
    "tml_hip_gemm_ex_dev": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _i64, _vp, _vp, _f, _vp, _i64, _vp, _vp,
                                           ctypes.c_int, _vp, _f, _f, _vp]),
    "tml_hip_gemm_prepared_ex": (ctypes.c_int, [_vp, _i64, _vp, _vp, _vp, ctypes.c_int, _vp, _f, _f, _vp]),
    "tml_hip_gemm_ex_dev_noalloc": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _i64, _vp, _vp, _f, _vp, _i64, _vp, _vp,
                                                   ctypes.c_int, _vp, _f, _f, _vp]),
    "tml_hip_quantize_cols_dev": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _vp, _vp, _vp, _vp]),
    "tml_hip_quantize_cols": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _vp, _vp, _vp]),
    "tml_hip_prepare_ex_dev": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _vp, _f, _vp, _vp, ctypes.POINTER(_vp)]),
    "tml_hip_transpose_requant_dev": (ctypes.c_int, [ctypes.c_int, _i64, _i64, _vp, _vp, _f, _vp, _vp, _vp]),
    "tml_hip_stream_read_dev": (ctypes.c_int, [_vp, _i64, ctypes.c_int, _vp, _vp]),
    "tml_tl_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "tml_tl_open_bytes": (ctypes.c_int, [_vp, ctypes.c_uint64, ctypes.POINTER(_vp)]),
    "tml_tl_close": (ctypes.c_int, [_vp]),
    "tml_tl_format": (ctypes.c_int, [_vp]),
    "tml_tl_count": (_i64, [_vp]),
    "tml_tl_name": (ctypes.c_char_p, [_vp, _i64]),
    "tml_tl_info": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.POINTER(_i64), ctypes.c_int,
                                   ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_uint64),
                                   ctypes.POINTER(ctypes.c_uint64)]),
    "tml_tl_read": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int, _vp, _vp, ctypes.POINTER(_f)]),
    "tml_tl_read_dev": (ctypes.c_int, [_vp, ctypes.c_char_p, ctypes.c_int, _vp, _vp, ctypes.POINTER(_f), _vp]),
    "tml_tl_read_dequantized_dev": (ctypes.c_int, [_vp, ctypes.c_char_p, _vp, _vp]),
}


class TmlError(RuntimeError):
    """A negative status from the C ABI; .code is the TML_ERR_* value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"tomoul_hip error {code}: {msg}")
        self.code = code


class LibraryNotBuilt(RuntimeError):
    pass


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises LibraryNotBuilt if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise LibraryNotBuilt(f"{LIB_PATH} is missing; build it with `python -m tomoul_amd.build` "
                              "(there is no CPU fallback)")
    L = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def check(code: int) -> None:
    if code != TML_OK:
        msg = lib().tml_hip_last_error().decode(errors="replace")
        raise TmlError(code, msg)


def _ptr(a: np.ndarray | None) -> int | None:
    if a is None:
        return None
    assert a.flags["C_CONTIGUOUS"], "arrays passed to the C ABI must be C-contiguous"
    return a.ctypes.data


def init() -> None:
    check(lib().tml_hip_init())


def shutdown() -> None:
    lib().tml_hip_shutdown()


def device_name() -> str:
    buf = ctypes.create_string_buffer(256)
    check(lib().tml_hip_device_name(buf, 256))
    return buf.value.decode()


# ------------------------------------------------------------- host pointers
def sgemm(m: int, n: int, k: int, a: np.ndarray, b: np.ndarray, c: np.ndarray, alpha: float = 1.0,
          beta: float = 0.0) -> None:
    check(lib().tml_hip_sgemm(m, n, k, _ptr(a), _ptr(b), _ptr(c), alpha, beta))


def sgemm_bias(m: int, n: int, k: int, a: np.ndarray, b: np.ndarray, bias: np.ndarray, c: np.ndarray) -> None:
    check(lib().tml_hip_sgemm_bias(m, n, k, _ptr(a), _ptr(b), _ptr(bias), _ptr(c)))


def sgemv(m: int, n: int, a: np.ndarray, x: np.ndarray, y: np.ndarray, alpha: float = 1.0,
          beta: float = 0.0) -> None:
    check(lib().tml_hip_sgemv(m, n, _ptr(a), _ptr(x), _ptr(y), alpha, beta))


def sgemm_q8(m: int, n: int, k: int, a: np.ndarray, q: np.ndarray, scale: float, c: np.ndarray) -> None:
    check(lib().tml_hip_sgemm_q8(m, n, k, _ptr(a), _ptr(q), scale, _ptr(c)))


def sgemm_q8k(m: int, n: int, k: int, a: np.ndarray, q: np.ndarray, scales: np.ndarray, block: int,
              c: np.ndarray) -> None:
    check(lib().tml_hip_sgemm_q8k(m, n, k, _ptr(a), _ptr(q), _ptr(scales), block, _ptr(c)))


def sgemm_q4(m: int, n: int, k: int, a: np.ndarray, packed: np.ndarray, scale: float, c: np.ndarray) -> None:
    check(lib().tml_hip_sgemm_q4(m, n, k, _ptr(a), _ptr(packed), scale, _ptr(c)))


def sgemm_f16(m: int, n: int, k: int, a: np.ndarray, h: np.ndarray, c: np.ndarray) -> None:
    check(lib().tml_hip_sgemm_f16(m, n, k, _ptr(a), _ptr(h), _ptr(c)))


def gemm(fmt: int, m: int, n: int, k: int, a: np.ndarray, b: np.ndarray, c: np.ndarray, *, scale: float = 1.0,
         scales: np.ndarray | None = None, block: int = 32, bias: np.ndarray | None = None) -> None:
    check(lib().tml_hip_gemm(fmt, m, n, k, _ptr(a), _ptr(b), scale, _ptr(scales), block, _ptr(bias), _ptr(c)))


def gemm_act(fmt: int, m: int, n: int, k: int, a: np.ndarray, b: np.ndarray, c: np.ndarray, *, act: int,
             scale: float = 1.0, scales: np.ndarray | None = None, block: int = 32,
             bias: np.ndarray | None = None) -> None:
    check(lib().tml_hip_gemm_act(fmt, m, n, k, _ptr(a), _ptr(b), scale, _ptr(scales), block, _ptr(bias), act,
                                 _ptr(c)))


def gemm_residual(fmt: int, m: int, n: int, k: int, a: np.ndarray, b: np.ndarray, residual: np.ndarray,
                  c: np.ndarray, *, scale: float = 1.0, scales: np.ndarray | None = None, block: int = 32,
                  bias: np.ndarray | None = None) -> None:
    check(lib().tml_hip_gemm_residual(fmt, m, n, k, _ptr(a), _ptr(b), scale, _ptr(scales), block, _ptr(bias),
                                      _ptr(residual), _ptr(c)))


def quantize(fmt: int, w: np.ndarray, q: np.ndarray, scales: np.ndarray | None) -> None:
    check(lib().tml_hip_quantize(fmt, w.size, _ptr(w), _ptr(q), _ptr(scales)))


def weight_register(a: np.ndarray) -> None:
    check(lib().tml_hip_weight_register(_ptr(a), a.nbytes))


def weight_release(a: np.ndarray) -> None:
    check(lib().tml_hip_weight_release(_ptr(a)))


# ----------------------------------------------------------- device pointers
def gemm_dev(fmt: int, m: int, n: int, k: int, a_ptr: int, b_ptr: int, c_ptr: int, *, scale: float = 1.0,
             scales_ptr: int | None = None, block: int = 32, bias_ptr: int | None = None, alpha: float = 1.0,
             beta: float = 0.0, stream: int | None = None) -> None:
    check(lib().tml_hip_gemm_dev(fmt, m, n, k, a_ptr, b_ptr, scale, scales_ptr, block, bias_ptr, c_ptr, alpha,
                                 beta, stream))


def gemm_ex_dev(fmt: int, m: int, n: int, k: int, a_ptr: int, b_ptr: int, c_ptr: int, *, act: int = ACT_NONE,
                residual_ptr: int | None = None, scale: float = 1.0, scales_ptr: int | None = None, block: int = 32,
                bias_ptr: int | None = None, alpha: float = 1.0, beta: float = 0.0,
                stream: int | None = None) -> None:
    check(lib().tml_hip_gemm_ex_dev(fmt, m, n, k, a_ptr, b_ptr, scale, scales_ptr, block, bias_ptr, residual_ptr,
                                    act, c_ptr, alpha, beta, stream))


def gemm_ex_dev_noalloc(fmt: int, m: int, n: int, k: int, a_ptr: int, b_ptr: int, c_ptr: int, *,
                        act: int = ACT_NONE, residual_ptr: int | None = None, scale: float = 1.0,
                        scales_ptr: int | None = None, block: int = 32, bias_ptr: int | None = None,
                        alpha: float = 1.0, beta: float = 0.0, stream: int | None = None) -> None:
    """tml_hip_gemm_ex_dev_noalloc: gemm_ex_dev with the static split-K scratch (no device allocation)."""
    check(lib().tml_hip_gemm_ex_dev_noalloc(fmt, m, n, k, a_ptr, b_ptr, scale, scales_ptr, block, bias_ptr,
                                            residual_ptr, act, c_ptr, alpha, beta, stream))


def stream_read_dev(src_ptr: int, nbytes: int, chunks_per_lane: int, out_ptr: int,
                    stream: int | None = None) -> None:
    """tml_hip_stream_read_dev: the GEMV read floor (reads nbytes, writes
    ceil(nbytes / (chunks_per_lane * 4096)) partials to out)."""
    check(lib().tml_hip_stream_read_dev(src_ptr, nbytes, chunks_per_lane, out_ptr, stream))


def quantize_dev(fmt: int, n: int, w_ptr: int, q_ptr: int, scales_ptr: int, stream: int | None = None) -> None:
    check(lib().tml_hip_quantize_dev(fmt, n, w_ptr, q_ptr, scales_ptr, stream))


# ---------------------------------------------------------- prepared weights
def prepare_dev(fmt: int, k: int, n: int, b_ptr: int, scale: float = 1.0, stream: int | None = None) -> int:
    """Device-native copy of the [K,N] device weight at b_ptr; returns a handle."""
    h = ctypes.c_void_p()
    check(lib().tml_hip_prepare_dev(fmt, k, n, b_ptr, scale, stream, ctypes.byref(h)))
    return h.value


def prepare_rows_dev(fmt: int, k: int, n: int, w_ptr: int, ldw: int, scale: float = 1.0,
                     stream: int | None = None) -> int:
    """Prepared weight from N rows of K elements at w_ptr (row stride ldw bytes),
    e.g. a token embedding [n_vocab, d] for logits = x . E^T; returns a handle."""
    h = ctypes.c_void_p()
    check(lib().tml_hip_prepare_rows_dev(fmt, k, n, w_ptr, ldw, scale, stream, ctypes.byref(h)))
    return h.value


def gemm_prepared(handle: int, m: int, a_ptr: int, c_ptr: int, *, bias_ptr: int | None = None, alpha: float = 1.0,
                  beta: float = 0.0, stream: int | None = None) -> None:
    check(lib().tml_hip_gemm_prepared(handle, m, a_ptr, bias_ptr, c_ptr, alpha, beta, stream))


def gemm_prepared_ex(handle: int, m: int, a_ptr: int, c_ptr: int, *, act: int = ACT_NONE,
                     residual_ptr: int | None = None, bias_ptr: int | None = None, alpha: float = 1.0,
                     beta: float = 0.0, stream: int | None = None) -> None:
    check(lib().tml_hip_gemm_prepared_ex(handle, m, a_ptr, bias_ptr, residual_ptr, act, c_ptr, alpha, beta, stream))


def prepared_free(handle: int) -> None:
    check(lib().tml_hip_prepared_free(handle))


def transpose_requant_dev(fmt: int, rows: int, cols: int, q_ptr: int, q_out_ptr: int, scales_out_ptr: int, *,
                          scale: float = 1.0, scales_ptr: int | None = None, stream: int | None = None) -> None:
    """loadQuantizedTransposed{Q8,Q4,Q8K} on device pointers: [rows, cols] -> [cols, rows]."""
    check(lib().tml_hip_transpose_requant_dev(fmt, rows, cols, q_ptr, scales_ptr, scale, q_out_ptr, scales_out_ptr,
                                              stream))


def quantize_cols(fmt: int, w: np.ndarray, q: np.ndarray, scales: np.ndarray) -> None:
    """Per-output-column quantizer (FMT_Q8_0_PC / FMT_Q4_0_PC) of w [K,N]."""
    k, n = w.shape
    check(lib().tml_hip_quantize_cols(fmt, k, n, _ptr(w), _ptr(q), _ptr(scales)))


def quantize_cols_dev(fmt: int, k: int, n: int, w_ptr: int, q_ptr: int, scales_ptr: int,
                      stream: int | None = None) -> None:
    check(lib().tml_hip_quantize_cols_dev(fmt, k, n, w_ptr, q_ptr, scales_ptr, stream))


def prepare_ex_dev(fmt: int, k: int, n: int, b_ptr: int, *, scale: float = 1.0, scales_ptr: int | None = None,
                   stream: int | None = None) -> int:
    h = ctypes.c_void_p()
    check(lib().tml_hip_prepare_ex_dev(fmt, k, n, b_ptr, scale, scales_ptr, stream, ctypes.byref(h)))
    return h.value
