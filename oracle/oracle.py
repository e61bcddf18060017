"""ctypes view of the CPU oracle (oracle/oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.  The
product package (tomoul_amd) never imports this module.

Every wrapper takes and returns numpy arrays; shapes follow the reference's
row-major [M,K] x [K,N] convention (src/core/ops.zig:235-264).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i64 = ctypes.c_int64


def build() -> str:
    """Compile oracle.c with its Makefile (a few seconds)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    L = ctypes.CDLL(_LIB_PATH)
    sig = {
        "orc_splitmix64_next": (ctypes.c_uint64, [ctypes.POINTER(ctypes.c_uint64)]),
        "orc_fill_normal": (None, [ctypes.c_uint64, _i64, ctypes.c_double, ctypes.c_double, _f32p]),
        "orc_matmul_f32_naive": (None, [_i64, _i64, _i64, _f32p, _f32p, _f32p]),
        "orc_matmul_f32": (None, [_i64, _i64, _i64, _f32p, _f32p, _f32p]),
        "orc_matmul_f32_mt": (None, [_i64, _i64, _i64, _f32p, _f32p, _f32p, ctypes.c_int]),
        "orc_matmul_bias_f32": (None, [_i64, _i64, _i64, _f32p, _f32p, _f32p, _f32p]),
        "orc_sgemm": (None, [_i64, _i64, _i64, _f32p, _f32p, _f32p, ctypes.c_float, ctypes.c_float]),
        "orc_matmul_f64": (None, [_i64, _i64, _i64, _f32p, _f32p, _f64p]),
        "orc_matvec": (None, [_i64, _i64, _f32p, _f32p, _f32p]),
        "orc_quantize_q8": (None, [_i64, _f32p, _i8p, ctypes.POINTER(ctypes.c_float)]),
        "orc_dequantize_q8": (None, [_i64, _i8p, ctypes.c_float, _f32p]),
        "orc_quantize_q8k": (None, [_i64, _f32p, _i8p, _f32p]),
        "orc_dequantize_q8k": (None, [_i64, _i8p, _f32p, _i64, _f32p]),
        "orc_q4_get": (ctypes.c_int8, [_u8p, _i64]),
        "orc_q4_set": (None, [_u8p, _i64, ctypes.c_int8]),
        "orc_quantize_q4": (None, [_i64, _f32p, _u8p, ctypes.POINTER(ctypes.c_float)]),
        "orc_dequantize_q4": (None, [_i64, _u8p, ctypes.c_float, _f32p]),
        "orc_matmul_q8": (None, [_i64, _i64, _i64, _f32p, _i8p, ctypes.c_float, _f32p]),
        "orc_matmul_q8k": (None, [_i64, _i64, _i64, _f32p, _i8p, _f32p, _i64, _f32p]),
        "orc_matmul_q4": (None, [_i64, _i64, _i64, _f32p, _u8p, ctypes.c_float, _f32p]),
        "orc_matmul_q8_mt": (None, [_i64, _i64, _i64, _f32p, _i8p, ctypes.c_float, _f32p, ctypes.c_int]),
        "orc_matmul_q4_mt": (None, [_i64, _i64, _i64, _f32p, _u8p, ctypes.c_float, _f32p, ctypes.c_int]),
        "orc_max_threads": (ctypes.c_int, []),
        "orc_erf_as": (ctypes.c_float, [ctypes.c_float]),
        "orc_to_f16": (None, [_i64, _f32p, _u16p]),
        "orc_from_f16": (None, [_i64, _u16p, _f32p]),
        "orc_matmul_f16": (None, [_i64, _i64, _i64, _f32p, _u16p, _f32p]),
        "orc_gelu_exact": (None, [_i64, _f32p]),
        "orc_gelu_tanh": (None, [_i64, _f32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _f32(x) -> np.ndarray:
    return np.ascontiguousarray(x, dtype=np.float32)


def _mkn(a: np.ndarray, b: np.ndarray):
    assert a.ndim == 2 and b.ndim == 2 and a.shape[1] == b.shape[0], (a.shape, b.shape)
    return a.shape[0], b.shape[1], a.shape[1]


# ---------------------------------------------------------------- generator
def splitmix64_stream(seed: int, count: int) -> list[int]:
    st = ctypes.c_uint64(seed)
    return [lib().orc_splitmix64_next(ctypes.byref(st)) for _ in range(count)]


def fill_normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(seed, n, mean, std, out)
    return out


# ---------------------------------------------------------------- fp32 GEMM
def matmul(a, b) -> np.ndarray:
    """ops.matmul fallback semantics (src/core/ops.zig:277-414)."""
    a, b = _f32(a), _f32(b)
    m, n, k = _mkn(a, b)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_f32(m, n, k, a, b, c)
    return c


def matmul_naive(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    m, n, k = _mkn(a, b)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_f32_naive(m, n, k, a, b, c)
    return c


def matmul_mt(a, b, nthreads: int) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    m, n, k = _mkn(a, b)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_f32_mt(m, n, k, a, b, c, int(nthreads))
    return c


def matmul_bias(a, b, bias) -> np.ndarray:
    """ops.matmulBias fallback (src/core/ops.zig:446-468)."""
    a, b, bias = _f32(a), _f32(b), _f32(bias)
    m, n, k = _mkn(a, b)
    assert bias.shape == (n,)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_bias_f32(m, n, k, a, b, bias, c)
    return c


def sgemm(a, b, c, alpha: float, beta: float) -> np.ndarray:
    """cblas_sgemm row-major semantics bound at src/core/blas.zig:68-94."""
    a, b = _f32(a), _f32(b)
    m, n, k = _mkn(a, b)
    out = _f32(c).copy() if c is not None else np.zeros((m, n), np.float32)
    lib().orc_sgemm(m, n, k, a, b, out, alpha, beta)
    return out


def matmul_f64(a, b) -> np.ndarray:
    a, b = _f32(a), _f32(b)
    m, n, k = _mkn(a, b)
    c = np.empty((m, n), dtype=np.float64)
    lib().orc_matmul_f64(m, n, k, a, b, c)
    return c


def matvec(a, x) -> np.ndarray:
    a, x = _f32(a), _f32(x)
    assert a.ndim == 2 and x.shape == (a.shape[1],)
    y = np.empty(a.shape[0], dtype=np.float32)
    lib().orc_matvec(a.shape[0], a.shape[1], a, x, y)
    return y


# ---------------------------------------------------------------- quantizers
def quantize_q8(w) -> tuple[np.ndarray, float]:
    w = _f32(w)
    q = np.empty(w.shape, dtype=np.int8)
    s = ctypes.c_float()
    lib().orc_quantize_q8(w.size, w.reshape(-1), q.reshape(-1), ctypes.byref(s))
    return q, s.value


def dequantize_q8(q, scale: float) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    out = np.empty(q.shape, dtype=np.float32)
    lib().orc_dequantize_q8(q.size, q.reshape(-1), scale, out.reshape(-1))
    return out


def quantize_q8k(w) -> tuple[np.ndarray, np.ndarray]:
    w = _f32(w)
    q = np.empty(w.shape, dtype=np.int8)
    scales = np.empty((w.size + 31) // 32, dtype=np.float32)
    lib().orc_quantize_q8k(w.size, w.reshape(-1), q.reshape(-1), scales)
    return q, scales


def dequantize_q8k(q, scales, block: int = 32) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    out = np.empty(q.shape, dtype=np.float32)
    lib().orc_dequantize_q8k(q.size, q.reshape(-1), _f32(scales), block, out.reshape(-1))
    return out


def quantize_q4(w) -> tuple[np.ndarray, float]:
    """Returns (packed bytes of length ceil(n/2), scale)."""
    w = _f32(w)
    packed = np.empty((w.size + 1) // 2, dtype=np.uint8)
    s = ctypes.c_float()
    lib().orc_quantize_q4(w.size, w.reshape(-1), packed, ctypes.byref(s))
    return packed, s.value


def q4_get(packed, idx: int) -> int:
    return int(lib().orc_q4_get(np.ascontiguousarray(packed, dtype=np.uint8), idx))


def q4_set(packed: np.ndarray, idx: int, value: int) -> None:
    assert packed.dtype == np.uint8 and packed.flags["C_CONTIGUOUS"]
    lib().orc_q4_set(packed, idx, value)


def dequantize_q4(packed, n: int, scale: float) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_dequantize_q4(n, np.ascontiguousarray(packed, dtype=np.uint8), scale, out)
    return out


# ---------------------------------------------------------------- quantized matmuls
def matmul_q8(a, q, scale: float) -> np.ndarray:
    """matmulF32Q8 (src/core/quantization.zig:158-203)."""
    a = _f32(a)
    q = np.ascontiguousarray(q, dtype=np.int8)
    m, n, k = _mkn(a, q)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_q8(m, n, k, a, q, scale, c)
    return c


def matmul_q8k(a, q, scales, block: int = 32) -> np.ndarray:
    """matmulF32Q8K (src/core/quantization.zig:477-525)."""
    a = _f32(a)
    q = np.ascontiguousarray(q, dtype=np.int8)
    m, n, k = _mkn(a, q)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_q8k(m, n, k, a, q, _f32(scales), block, c)
    return c


def matmul_q4(a, packed, k: int, n: int, scale: float) -> np.ndarray:
    """matmulF32Q4 (src/core/quantization.zig:778-824); packed holds K*N nibbles."""
    a = _f32(a)
    assert a.ndim == 2 and a.shape[1] == k
    m = a.shape[0]
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_q4(m, n, k, a, np.ascontiguousarray(packed, dtype=np.uint8), scale, c)
    return c


def matmul_q8_mt(a, q, scale: float, nthreads: int) -> np.ndarray:
    a = _f32(a)
    q = np.ascontiguousarray(q, dtype=np.int8)
    m, n, k = _mkn(a, q)
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_q8_mt(m, n, k, a, q, scale, c, int(nthreads))
    return c


def matmul_q4_mt(a, packed, k: int, n: int, scale: float, nthreads: int) -> np.ndarray:
    a = _f32(a)
    m = a.shape[0]
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_q4_mt(m, n, k, a, np.ascontiguousarray(packed, dtype=np.uint8), scale, c, int(nthreads))
    return c


def max_threads() -> int:
    return int(lib().orc_max_threads())


# ---------------------------------------------------------------- F16 weights
def to_f16(w) -> np.ndarray:
    """toF16 (src/core/quantization.zig:1907-1917): binary16 bit patterns."""
    w = _f32(w)
    h = np.empty(w.shape, dtype=np.uint16)
    lib().orc_to_f16(w.size, w.reshape(-1), h.reshape(-1))
    return h


def from_f16(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    v = np.empty(h.shape, dtype=np.float32)
    lib().orc_from_f16(h.size, h.reshape(-1), v.reshape(-1))
    return v


def matmul_f16(a, h) -> np.ndarray:
    """matmulF32F16 fallback (src/core/quantization.zig:1949-1958)."""
    a, h = _f32(a), np.ascontiguousarray(h, dtype=np.uint16)
    m, k = a.shape
    k2, n = h.shape
    assert k == k2
    c = np.empty((m, n), dtype=np.float32)
    lib().orc_matmul_f16(m, n, k, a, h, c)
    return c


# ---------------------------------------------------------------- activations
ACT_NONE, ACT_GELU_ERF, ACT_GELU_TANH = 0, 1, 2


def erf_as(x: float) -> float:
    """A&S 7.1.26 erf of src/core/ops.zig:2000-2022."""
    return float(lib().orc_erf_as(x))


def gelu_exact(v) -> np.ndarray:
    """ops.geluExact (src/core/ops.zig:2029-2057) on a copy of v."""
    out = _f32(v).copy()
    lib().orc_gelu_exact(out.size, out.reshape(-1))
    return out


def gelu_tanh(v) -> np.ndarray:
    """ops.gelu (src/core/ops.zig:1947-1998) on a copy of v: the flat index
    decides between the 8-wide rational tanh and the scalar tail's tanh."""
    out = _f32(v).copy()
    lib().orc_gelu_tanh(out.size, out.reshape(-1))
    return out


def apply_act(v, act: int) -> np.ndarray:
    if act == ACT_GELU_ERF:
        return gelu_exact(v)
    if act == ACT_GELU_TANH:
        return gelu_tanh(v)
    return _f32(v).copy()


# --------------------------------------------------------------- .tl files
# Pure-Python restatement of the file layout: the reader of
# src/core/loader.zig:133-222 (header, tensor table) and :225-569 (payloads),
# and the writer of tools/tl_format.py:250-360 (header, table with offsets
# patched after the data, payload per format).  Small files only.
TL_F32, TL_Q8_0, TL_Q4_0, TL_Q8_K, TL_F16 = 0, 1, 2, 3, 4


class TlParseError(Exception):
    def __init__(self, kind: str):
        super().__init__(kind)
        self.kind = kind  # the LoadError member's name


def tl_parse(data: bytes) -> dict:
    import struct
    if len(data) < 16:
        raise TlParseError("CorruptedFile")
    if data[:4] != b"TOUL":
        raise TlParseError("InvalidMagic")
    version, count = struct.unpack_from("<II", data, 4)
    if version != 1:
        raise TlParseError("UnsupportedVersion")
    fmt = data[12]
    if fmt > 4:
        raise TlParseError("UnsupportedQuantFormat")
    pos, entries = 16, []
    for _ in range(count):
        if pos + 4 > len(data):
            raise TlParseError("CorruptedFile")
        (nlen,) = struct.unpack_from("<I", data, pos)
        pos += 4
        if pos + nlen > len(data):
            raise TlParseError("CorruptedFile")
        name = data[pos:pos + nlen].decode()
        pos += nlen
        if pos + 4 > len(data):
            raise TlParseError("CorruptedFile")
        (nd,) = struct.unpack_from("<I", data, pos)
        pos += 4
        if pos + 4 * nd > len(data):
            raise TlParseError("CorruptedFile")
        shape = struct.unpack_from(f"<{nd}I", data, pos)
        pos += 4 * nd
        if pos + 16 > len(data):
            raise TlParseError("CorruptedFile")
        off, size = struct.unpack_from("<QQ", data, pos)
        pos += 16
        entries.append((name, tuple(shape), off, size))
    return {"version": version, "format": fmt, "tensors": entries}


def tl_payload(data: bytes, entry, fmt: int) -> dict:
    """The parts of one payload in format fmt, with the getters' size checks."""
    import struct
    name, shape, off, size = entry
    n = int(np.prod(shape, dtype=np.int64)) if shape else 1
    if off + size > len(data):
        raise TlParseError("CorruptedFile")
    raw = data[off:off + size]
    want = {TL_F32: 4 * n, TL_F16: 2 * n, TL_Q8_0: 4 + n, TL_Q4_0: 4 + (n + 1) // 2,
            TL_Q8_K: 4 + 4 * ((n + 31) // 32) + n}[fmt]
    if size != want:
        raise TlParseError("CorruptedFile")
    if fmt == TL_F32:
        return {"data": np.frombuffer(raw, dtype="<f4").copy()}
    if fmt == TL_F16:
        return {"data": np.frombuffer(raw, dtype="<u2").copy()}
    if fmt in (TL_Q8_0, TL_Q4_0):
        (scale,) = struct.unpack_from("<f", raw, 0)
        dt = np.int8 if fmt == TL_Q8_0 else np.uint8
        return {"scale": scale, "data": np.frombuffer(raw[4:], dtype=dt).copy()}
    nb = (n + 31) // 32
    (stored,) = struct.unpack_from("<I", raw, 0)
    return {"num_blocks": stored, "scales": np.frombuffer(raw[4:4 + 4 * nb], dtype="<f4").copy(),
            "data": np.frombuffer(raw[4 + 4 * nb:], dtype=np.int8).copy()}


def tl_dequantize(fmt: int, parts: dict, n: int) -> np.ndarray:
    """getTensorDequantized's per-format arithmetic (loader.zig:467-565):
    one f32 multiply f32(q) * scale per element, exact widening of f16."""
    if fmt == TL_F32:
        return parts["data"].astype(np.float32)
    if fmt == TL_F16:
        return from_f16(parts["data"])
    if fmt == TL_Q8_0:
        return parts["data"].astype(np.float32) * np.float32(parts["scale"])
    if fmt == TL_Q4_0:
        b = parts["data"]
        nib = np.empty(2 * b.size, dtype=np.int32)
        nib[0::2], nib[1::2] = b & 0x0F, b >> 4
        nib = np.where(nib & 8, nib - 16, nib)[:n]
        return nib.astype(np.float32) * np.float32(parts["scale"])
    idx = np.arange(n) // 32
    return parts["data"].astype(np.float32) * parts["scales"][idx]


def tl_write(tensors, fmt: int) -> bytes:
    """A .tl file from (name, shape, parts) triples, parts already encoded
    for fmt as tl_payload returns them (tools/tl_format.py:277-360)."""
    import struct
    head = bytearray(b"TOUL" + struct.pack("<II", 1, len(tensors)) + bytes([fmt, 0, 0, 0]))
    patch = []
    for name, shape, _ in tensors:
        nb = name.encode()
        head += struct.pack("<I", len(nb)) + nb + struct.pack("<I", len(shape))
        head += b"".join(struct.pack("<I", d) for d in shape)
        patch.append(len(head))
        head += b"\0" * 16
    body = bytearray()
    for (name, shape, parts), at in zip(tensors, patch):
        start = len(head) + len(body)
        if fmt in (TL_F32, TL_F16):
            blob = parts["data"].astype("<f4" if fmt == TL_F32 else "<u2").tobytes()
        elif fmt in (TL_Q8_0, TL_Q4_0):
            blob = struct.pack("<f", parts["scale"]) + parts["data"].tobytes()
        else:
            sc = parts["scales"].astype("<f4")
            blob = struct.pack("<I", parts.get("num_blocks", sc.size)) + sc.tobytes() + parts["data"].tobytes()
        body += blob
        head[at:at + 16] = struct.pack("<QQ", start, len(blob))
    return bytes(head + body)


# ------------------------------------------------ per-column quantization
# An extension, not a reference format: column n of W[K,N] quantized by the
# reference's per-tensor quantizer applied to that column alone; the product
# is the reference's dequantize-then-f32-accumulate (matmulF32Q8,
# src/core/quantization.zig:158-203) with scale s[n] for column n.
def quantize_q8_cols(w) -> tuple[np.ndarray, np.ndarray]:
    w = _f32(w)
    k, n = w.shape
    q = np.empty((k, n), dtype=np.int8)
    s = np.empty(n, dtype=np.float32)
    for j in range(n):
        qj, s[j] = quantize_q8(np.ascontiguousarray(w[:, j]))
        q[:, j] = qj.reshape(-1)
    return q, s


def _unpack_q4(packed: np.ndarray, count: int) -> np.ndarray:
    b = np.asarray(packed, dtype=np.uint8)
    nib = np.empty(2 * b.size, dtype=np.int8)
    nib[0::2] = (b & 0x0F).astype(np.int8)
    nib[1::2] = (b >> 4).astype(np.int8)
    nib = np.where(nib & 8, nib - 16, nib).astype(np.int8)
    return nib[:count]


def _pack_q4(vals: np.ndarray) -> np.ndarray:
    v = np.asarray(vals, dtype=np.int8).reshape(-1).astype(np.uint8) & 0x0F
    if v.size % 2:
        v = np.concatenate([v, np.zeros(1, np.uint8)])
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


def quantize_q4_cols(w) -> tuple[np.ndarray, np.ndarray]:
    """Packed like Q4_0 over the flattened [K,N] (even element in the low nibble)."""
    w = _f32(w)
    k, n = w.shape
    vals = np.empty((k, n), dtype=np.int8)
    s = np.empty(n, dtype=np.float32)
    for j in range(n):
        pj, s[j] = quantize_q4(np.ascontiguousarray(w[:, j]))
        vals[:, j] = _unpack_q4(pj, k)
    return _pack_q4(vals), s


def dequantize_cols(fmt: int, data, scales, k: int, n: int) -> np.ndarray:
    vals = np.asarray(data, dtype=np.int8).reshape(k, n) if fmt == 17 else _unpack_q4(data, k * n).reshape(k, n)
    return vals.astype(np.float32) * np.asarray(scales, dtype=np.float32)[None, :]


def matmul_cols(a, fmt: int, data, scales, k: int, n: int) -> np.ndarray:
    return matmul(a, dequantize_cols(fmt, data, scales, k, n))
