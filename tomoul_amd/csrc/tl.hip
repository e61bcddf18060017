// .tl weight files: host-side parsing (src/core/loader.zig:55-222), the
// validated payload of each getter (:225-569), and the device kernels that
// turn payloads into the in-memory layouts the matmuls read:
//   * dequant_kernel       getTensorDequantized (:442-569) on the device;
//   * dequant_t_kernel     the dequantize + transpose half of the XLM-R
//                          loaders loadQuantizedTransposed{Q8,Q4,Q8K}
//                          (src/models/xlm_roberta_punctuation/model.zig:
//                          1272-1362); the re-quantization is the bit-exact
//                          quantizer of quantize.hip.
// Payloads are copied byte for byte; no value is rounded on the way, so a
// tensor in HBM equals the one the reference builds in host memory.
#include <hip/hip_runtime.h>

#include <cerrno>
#include <cstdio>
#include <cstring>
#include <limits>

#include "tml_internal.hpp"

namespace tml {

namespace {

uint32_t rd_u32(const uint8_t *p) {
    uint32_t v;
    std::memcpy(&v, p, 4);
    return v;
}
uint64_t rd_u64(const uint8_t *p) {
    uint64_t v;
    std::memcpy(&v, p, 8);
    return v;
}

// parseHeader + parseTensorEntry (loader.zig:133-222).  Every read is
// bounds-checked against the file size; any shortfall is CorruptedFile.
Status parse(TlFile *f) {
    const uint8_t *d = f->data;
    const uint64_t n = f->size;
    if (n < 16) return Status::Err(TML_ERR_CORRUPTED_FILE, "file shorter than the 16-byte header");
    if (std::memcmp(d, "TOUL", 4) != 0) return Status::Err(TML_ERR_INVALID_MAGIC, "magic is not TOUL");
    f->version = rd_u32(d + 4);
    if (f->version != 1) return Status::Err(TML_ERR_UNSUPPORTED_VERSION, "only version 1 is supported");
    const uint32_t count = rd_u32(d + 8);
    const uint8_t fmt = d[12];
    if (fmt > TML_FMT_F16) return Status::Err(TML_ERR_UNSUPPORTED_QUANT_FORMAT, "unknown quant-format byte");
    f->format = fmt;
    uint64_t pos = 16;
    for (uint32_t t = 0; t < count; ++t) {
        if (pos + 4 > n) return Status::Err(TML_ERR_CORRUPTED_FILE, "truncated tensor entry (name length)");
        const uint32_t name_len = rd_u32(d + pos);
        pos += 4;
        if (pos + name_len > n) return Status::Err(TML_ERR_CORRUPTED_FILE, "truncated tensor entry (name)");
        TlTensor info;
        info.name.assign((const char *)d + pos, name_len);
        pos += name_len;
        if (pos + 4 > n) return Status::Err(TML_ERR_CORRUPTED_FILE, "truncated tensor entry (rank)");
        const uint32_t ndim = rd_u32(d + pos);
        pos += 4;
        if (pos + (uint64_t)ndim * 4 > n) return Status::Err(TML_ERR_CORRUPTED_FILE, "truncated tensor entry (shape)");
        info.shape.resize(ndim);
        for (uint32_t i = 0; i < ndim; ++i, pos += 4) info.shape[i] = rd_u32(d + pos);
        if (pos + 16 > n) return Status::Err(TML_ERR_CORRUPTED_FILE, "truncated tensor entry (offset, size)");
        info.offset = rd_u64(d + pos);
        info.size = rd_u64(d + pos + 8);
        pos += 16;
        // StringHashMap.put: a repeated name replaces the earlier entry; the
        // name list keeps both (loader.zig:218-219).
        f->index[info.name] = f->tensors.size();
        f->tensors.push_back(std::move(info));
    }
    return Status::Ok();
}

// Product of the dims, or -1 when it exceeds `cap` (the most elements a
// payload of the file's size could hold) -- a crafted shape whose product
// wraps around 2^64 must not pass the payload-size check.
int64_t numel_of(const TlTensor &t, uint64_t cap) {
    uint64_t e = 1;
    for (int64_t d : t.shape) {
        if (d != 0 && e > cap / (uint64_t)d) return -1;
        e *= (uint64_t)d;
    }
    return (int64_t)e;
}

}  // namespace

Status tl_open_file(const char *path, TlFile **out) {
    *out = nullptr;
    if (path == nullptr) return Status::Err(TML_ERR_INVALID_ARG, "null path");
    FILE *fp = std::fopen(path, "rb");
    if (fp == nullptr)
        return errno == ENOENT ? Status::Err(TML_ERR_FILE_NOT_FOUND, std::string("no such file: ") + path)
                               : Status::Err(TML_ERR_CORRUPTED_FILE, std::string("cannot open: ") + path);
    TlFile *f = new TlFile();
    bool ok = std::fseek(fp, 0, SEEK_END) == 0;
    const long len = ok ? std::ftell(fp) : -1;
    ok = ok && len >= 0 && std::fseek(fp, 0, SEEK_SET) == 0;
    if (ok) {
        f->owned.resize((size_t)len);
        ok = len == 0 || std::fread(f->owned.data(), 1, (size_t)len, fp) == (size_t)len;
    }
    std::fclose(fp);
    if (!ok) {
        delete f;
        return Status::Err(TML_ERR_CORRUPTED_FILE, std::string("cannot read: ") + path);
    }
    f->data = f->owned.data();
    f->size = f->owned.size();
    Status s = parse(f);
    if (!s.ok()) {
        delete f;
        return s;
    }
    *out = f;
    return Status::Ok();
}

Status tl_open_bytes(const void *data, uint64_t size, TlFile **out) {
    *out = nullptr;
    if (data == nullptr && size > 0) return Status::Err(TML_ERR_INVALID_ARG, "null bytes");
    TlFile *f = new TlFile();
    f->data = (const uint8_t *)data;
    f->size = size;
    Status s = parse(f);
    if (!s.ok()) {
        delete f;
        return s;
    }
    *out = f;
    return Status::Ok();
}

const TlTensor *tl_find(const TlFile *f, const char *name) {
    if (name == nullptr) return nullptr;
    auto it = f->index.find(name);
    return it == f->index.end() ? nullptr : &f->tensors[it->second];
}

// The getters' checks, in the reference's order: format (quantized getters
// only), name, bounds, payload size (and Q8_K's stored block count).
Status tl_parts(const TlFile *f, const char *name, int getter, bool by_file_format, TlParts *p) {
    const int fmt = by_file_format ? f->format : getter;
    if (!by_file_format && getter != TML_FMT_F32 && f->format != getter)
        return Status::Err(TML_ERR_UNSUPPORTED_QUANT_FORMAT, "the file's quant format is not the requested one");
    const TlTensor *t = tl_find(f, name);
    if (t == nullptr) return Status::Err(TML_ERR_TENSOR_NOT_FOUND, std::string("no tensor named ") + (name ? name : ""));
    if (t->offset > f->size || t->size > f->size - t->offset)
        return Status::Err(TML_ERR_CORRUPTED_FILE, "tensor data runs past the end of the file");
    // No format stores more than two elements per payload byte.
    const int64_t n = numel_of(*t, 2 * t->size);
    if (n < 0) return Status::Err(TML_ERR_CORRUPTED_FILE, "tensor shape holds more elements than its payload");
    const uint8_t *src = f->data + t->offset;
    *p = TlParts{};
    p->fmt = fmt;
    p->numel = n;
    uint64_t want = 0;
    switch (fmt) {
        case TML_FMT_F32: want = (uint64_t)n * 4; break;
        case TML_FMT_F16: want = (uint64_t)n * 2; break;
        case TML_FMT_Q8_0: want = 4 + (uint64_t)n; break;
        case TML_FMT_Q4_0: want = 4 + ((uint64_t)n + 1) / 2; break;
        default: want = 4 + (((uint64_t)n + 31) / 32) * 4 + (uint64_t)n; break;  // Q8_K
    }
    if (t->size != want) return Status::Err(TML_ERR_CORRUPTED_FILE, "tensor data size does not match its shape");
    switch (fmt) {
        case TML_FMT_F32:
        case TML_FMT_F16:
            p->data = src;
            p->data_bytes = t->size;
            break;
        case TML_FMT_Q8_0:
        case TML_FMT_Q4_0:
            std::memcpy(&p->scale, src, 4);
            p->data = src + 4;
            p->data_bytes = t->size - 4;
            break;
        default: {
            const uint64_t nb = ((uint64_t)n + 31) / 32;
            if (!by_file_format && rd_u32(src) != nb)
                return Status::Err(TML_ERR_CORRUPTED_FILE, "stored Q8_K block count does not match the shape");
            p->scales = src + 4;
            p->nscales = nb;
            p->data = src + 4 + nb * 4;
            p->data_bytes = (uint64_t)n;
            break;
        }
    }
    return Status::Ok();
}

// ------------------------------------------------------------- kernels
namespace {

constexpr int kThreads = 256;

template <int FMT>
__device__ __forceinline__ float deq(const uint8_t *raw, const float *scales, float scale, long long e) {
    if constexpr (FMT == TML_FMT_Q8_0) {
        return (float)(int8_t)raw[e] * scale;
    } else if constexpr (FMT == TML_FMT_Q4_0) {
        const uint32_t byte = raw[e / 2];
        const uint32_t nib = (e & 1) ? (byte >> 4) : (byte & 0xF);
        return (float)((int32_t)(nib << 28) >> 28) * scale;
    } else if constexpr (FMT == TML_FMT_Q8_K) {
        return (float)(int8_t)raw[e] * scales[e / 32];
    } else if constexpr (FMT == TML_FMT_F16) {
        return tml_half_bits(((const uint16_t *)raw)[e]);
    } else {
        return ((const float *)raw)[e];
    }
}

template <int FMT>
__global__ __launch_bounds__(kThreads) void dequant_kernel(const uint8_t *__restrict__ raw,
                                                           const float *__restrict__ scales, float scale,
                                                           long long n, float *__restrict__ out) {
    for (long long i = (long long)blockIdx.x * kThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kThreads)
        out[i] = deq<FMT>(raw, scales, scale, i);
}

// out[c, r] = dequant(in[r, c]) for in [rows, cols]: 32 x 32 tiles through
// LDS so that both the read (along c) and the write (along r) are
// contiguous; the +1 column keeps the transposed LDS reads conflict-free.
template <int FMT>
__global__ __launch_bounds__(kThreads) void dequant_t_kernel(const uint8_t *__restrict__ raw,
                                                             const float *__restrict__ scales, float scale,
                                                             int rows, int cols, float *__restrict__ out) {
    __shared__ float tile[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
#pragma unroll
    for (int i = 0; i < 32; i += 8) {
        const int r = r0 + ty + i, c = c0 + tx;
        if (r < rows && c < cols) tile[ty + i][tx] = deq<FMT>(raw, scales, scale, (long long)r * cols + c);
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 32; i += 8) {
        const int c = c0 + ty + i, r = r0 + tx;
        if (r < rows && c < cols) out[(long long)c * rows + r] = tile[tx][ty + i];
    }
}

unsigned grid_1d(long long n) {
    long long b = (n + kThreads - 1) / kThreads;
    if (b > 8192) b = 8192;
    return (unsigned)(b > 0 ? b : 1);
}

}  // namespace

Status launch_dequant(int fmt, int64_t n, const void *raw, const float *scales, float scale, float *out,
                      hipStream_t s) {
    if (n <= 0) return Status::Ok();
    const uint8_t *r = (const uint8_t *)raw;
    switch (fmt) {
        case TML_FMT_F32: dequant_kernel<TML_FMT_F32><<<grid_1d(n), kThreads, 0, s>>>(r, scales, scale, n, out); break;
        case TML_FMT_Q8_0: dequant_kernel<TML_FMT_Q8_0><<<grid_1d(n), kThreads, 0, s>>>(r, scales, scale, n, out); break;
        case TML_FMT_Q4_0: dequant_kernel<TML_FMT_Q4_0><<<grid_1d(n), kThreads, 0, s>>>(r, scales, scale, n, out); break;
        case TML_FMT_Q8_K: dequant_kernel<TML_FMT_Q8_K><<<grid_1d(n), kThreads, 0, s>>>(r, scales, scale, n, out); break;
        case TML_FMT_F16: dequant_kernel<TML_FMT_F16><<<grid_1d(n), kThreads, 0, s>>>(r, scales, scale, n, out); break;
        default: return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    }
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

Status launch_dequant_transpose(int fmt, int64_t rows, int64_t cols, const void *raw, const float *scales,
                                float scale, float *out, hipStream_t s) {
    if (rows <= 0 || cols <= 0) return Status::Ok();
    if (rows >= ((int64_t)1 << 30) || cols >= ((int64_t)1 << 30))
        return Status::Err(TML_ERR_INVALID_SHAPE, "transpose: dimension exceeds 2^30");
    const int64_t gx = (cols + 31) / 32, gy = (rows + 31) / 32;
    if (gy > 65535) return Status::Err(TML_ERR_INVALID_SHAPE, "transpose: too many rows for one launch");
    const dim3 grid((unsigned)gx, (unsigned)gy);
    const uint8_t *r = (const uint8_t *)raw;
    const int R = (int)rows, C = (int)cols;
    switch (fmt) {
        case TML_FMT_F32: dequant_t_kernel<TML_FMT_F32><<<grid, kThreads, 0, s>>>(r, scales, scale, R, C, out); break;
        case TML_FMT_Q8_0: dequant_t_kernel<TML_FMT_Q8_0><<<grid, kThreads, 0, s>>>(r, scales, scale, R, C, out); break;
        case TML_FMT_Q4_0: dequant_t_kernel<TML_FMT_Q4_0><<<grid, kThreads, 0, s>>>(r, scales, scale, R, C, out); break;
        case TML_FMT_Q8_K: dequant_t_kernel<TML_FMT_Q8_K><<<grid, kThreads, 0, s>>>(r, scales, scale, R, C, out); break;
        case TML_FMT_F16: dequant_t_kernel<TML_FMT_F16><<<grid, kThreads, 0, s>>>(r, scales, scale, R, C, out); break;
        default: return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    }
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

}  // namespace tml
