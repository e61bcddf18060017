// quantize.hip -- on-device weight quantizers producing the reference's
// in-memory layouts, bit-identical to the Zig quantizers:
//   Q8_0 quantizeQ8  (src/core/quantization.zig:98-129)
//   Q8_K quantizeQ8K (src/core/quantization.zig:406-446)
//   Q4_0 quantizeQ4  (src/core/quantization.zig:721-754)
// Arithmetic follows the reference exactly: max|v| over the tensor (or over
// each 32-element block), scale = max / 127 (or / 7) and inv = 127 / max (or
// 7 / max) as correctly rounded f32 divisions, q = clamp(round(v * inv)) with
// round-half-away-from-zero; an all-zero tensor/block gets scale 1 and q = 0.
// The max-abs is found in two passes without atomics: pass 1 writes one
// maximum per workgroup, pass 2 folds those (order does not matter for max)
// and quantizes, so no buffer needs clearing between calls.
#include "tml_internal.hpp"

namespace tml {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxPartials = 1024;  // workgroups of pass 1

// max(|v|) the way the reference loop does it: a NaN never wins a ">".
__device__ __forceinline__ float fold_max(float m, float v) {
    const float a = fabsf(v);
    return a > m ? a : m;
}

__device__ float block_max(float m) {
    __shared__ float red[kThreads / 64];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int i = 1; i < kThreads / 64; ++i) r = fmaxf(r, red[i]);
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(kThreads) void absmax_partials(const float *__restrict__ w, long long n,
                                                             float *__restrict__ partials) {
    float m = 0.0f;
    for (long long i = (long long)blockIdx.x * kThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kThreads)
        m = fold_max(m, w[i]);
    m = block_max(m);
    if (threadIdx.x == 0) partials[blockIdx.x] = m;
}

__device__ __forceinline__ float global_max(const float *partials, int np) {
    float m = 0.0f;
    for (int i = threadIdx.x; i < np; i += kThreads) m = fmaxf(m, partials[i]);
    return block_max(m);
}

__device__ __forceinline__ float quant(float v, float inv, float lim) {
    const float r = roundf(v * inv);
    return r < -lim ? -lim : (r > lim ? lim : r);
}

__global__ __launch_bounds__(kThreads) void quantize_q8_kernel(const float *__restrict__ w, long long n,
                                                                const float *__restrict__ partials, int np,
                                                                int8_t *__restrict__ q, float *__restrict__ scale) {
    const float mx = global_max(partials, np);
    const bool zero = mx == 0.0f;
    const float inv = zero ? 0.0f : 127.0f / mx;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = zero ? 1.0f : mx / 127.0f;
    for (long long i = (long long)blockIdx.x * kThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kThreads)
        q[i] = zero ? (int8_t)0 : (int8_t)quant(w[i], inv, 127.0f);
}

// One output byte (elements 2j, 2j+1) per thread: low nibble = even index.
__global__ __launch_bounds__(kThreads) void quantize_q4_kernel(const float *__restrict__ w, long long n,
                                                                const float *__restrict__ partials, int np,
                                                                uint8_t *__restrict__ packed,
                                                                float *__restrict__ scale) {
    const float mx = global_max(partials, np);
    const bool zero = mx == 0.0f;
    const float inv = zero ? 0.0f : 7.0f / mx;
    if (blockIdx.x == 0 && threadIdx.x == 0) *scale = zero ? 1.0f : mx / 7.0f;
    const long long nb = (n + 1) / 2;
    for (long long j = (long long)blockIdx.x * kThreads + threadIdx.x; j < nb; j += (long long)gridDim.x * kThreads) {
        uint32_t lo = 0, hi = 0;
        if (!zero) {
            lo = (uint32_t)(int)quant(w[2 * j], inv, 7.0f) & 0xF;
            if (2 * j + 1 < n) hi = (uint32_t)(int)quant(w[2 * j + 1], inv, 7.0f) & 0xF;
        }
        packed[j] = (uint8_t)(lo | (hi << 4));
    }
}

// Q8_K: 32 lanes per 32-element block (half a wave), max via shuffles.
__global__ __launch_bounds__(kThreads) void quantize_q8k_kernel(const float *__restrict__ w, long long n,
                                                                 int8_t *__restrict__ q,
                                                                 float *__restrict__ scales) {
    const long long nblocks = (n + 31) / 32;
    const int sub = threadIdx.x & 31;
    const long long first = ((long long)blockIdx.x * kThreads + threadIdx.x) / 32;
    const long long stride = (long long)gridDim.x * kThreads / 32;
    for (long long b = first; b < nblocks; b += stride) {
        const long long i = b * 32 + sub;
        const float v = i < n ? w[i] : 0.0f;
        float m = fold_max(0.0f, v);
#pragma unroll
        for (int off = 16; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off, 32));
        const bool zero = m == 0.0f;
        if (sub == 0) scales[b] = zero ? 1.0f : m / 127.0f;
        if (i < n) q[i] = zero ? (int8_t)0 : (int8_t)quant(v, 127.0f / m, 127.0f);
    }
}

// Per-output-column quantizers (an extension: the reference quantizes per
// tensor or per 32-element block): column n of W[K,N] gets exactly the
// per-tensor quantizer above applied to that column alone.
__global__ __launch_bounds__(kThreads) void colmax_kernel(const float *__restrict__ w, int K, int N,
                                                          float *__restrict__ mx) {
    for (long long n = (long long)blockIdx.x * kThreads + threadIdx.x; n < N; n += (long long)gridDim.x * kThreads) {
        float m = 0.0f;
        for (int k = 0; k < K; ++k) m = fold_max(m, w[(long long)k * N + n]);
        mx[n] = m;
    }
}

__global__ __launch_bounds__(kThreads) void quantize_cols_kernel(const float *__restrict__ w, long long ne, int N,
                                                                 const float *__restrict__ mx, bool int4,
                                                                 void *__restrict__ q, float *__restrict__ scales) {
    const long long stride = (long long)gridDim.x * kThreads;
    const long long t0 = (long long)blockIdx.x * kThreads + threadIdx.x;
    const float lim = int4 ? 7.0f : 127.0f;
    for (long long n = t0; n < N; n += stride) scales[n] = mx[n] == 0.0f ? 1.0f : mx[n] / lim;
    if (!int4) {
        for (long long i = t0; i < ne; i += stride) {
            const float m = mx[i % N];
            ((int8_t *)q)[i] = m == 0.0f ? (int8_t)0 : (int8_t)quant(w[i], 127.0f / m, 127.0f);
        }
    } else {
        // one output byte (elements 2j, 2j+1) per step: low nibble = even index
        for (long long j = t0; j < (ne + 1) / 2; j += stride) {
            uint32_t nib[2] = {0, 0};
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const long long e = 2 * j + h;
                if (e < ne) {
                    const float m = mx[e % N];
                    if (m != 0.0f) nib[h] = (uint32_t)(int)quant(w[e], 7.0f / m, 7.0f) & 0xF;
                }
            }
            ((uint8_t *)q)[j] = (uint8_t)(nib[0] | (nib[1] << 4));
        }
    }
}

int partial_blocks(long long n) {
    long long b = (n + kThreads - 1) / kThreads;
    return (int)(b < 1 ? 1 : (b > kMaxPartials ? kMaxPartials : b));
}

int grid_for(long long items) {
    long long b = (items + kThreads - 1) / kThreads;
    return (int)(b < 1 ? 1 : (b > 65535 ? 65535 : b));
}

}  // namespace

// toF16 (quantization.zig:1907-1917): @floatCast, i.e. IEEE round to
// nearest even, overflow to infinity, NaN kept NaN.
__global__ __launch_bounds__(kThreads) void to_f16_kernel(const float *__restrict__ w, long long n,
                                                          uint16_t *__restrict__ h) {
    for (long long i = (long long)blockIdx.x * kThreads + threadIdx.x; i < n; i += (long long)gridDim.x * kThreads)
        h[i] = __builtin_bit_cast(unsigned short, (_Float16)w[i]);
}

Status launch_quantize_cols(int fmt, int64_t K, int64_t N, const float *w, void *q, float *scales, float *tmp,
                           hipStream_t s) {
    if (fmt != TML_FMT_Q8_0 && fmt != TML_FMT_Q4_0)
        return Status::Err(TML_ERR_INVALID_FORMAT, "column quantizer: data format must be Q8_0 or Q4_0");
    if (K < 0 || N < 0) return Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension");
    if (K >= ((int64_t)1 << 31) || N >= ((int64_t)1 << 31))
        return Status::Err(TML_ERR_INVALID_SHAPE, "column quantizer: dimension exceeds 2^31");
    if (N == 0) return Status::Ok();
    colmax_kernel<<<grid_for(N), kThreads, 0, s>>>(w, (int)K, (int)N, tmp);
    TML_HIP_TRY(hipGetLastError());
    const long long ne = (long long)K * N;
    quantize_cols_kernel<<<grid_for(ne > N ? ne : N), kThreads, 0, s>>>(w, ne, (int)N, tmp, fmt == TML_FMT_Q4_0, q,
                                                                        scales);
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

size_t quantize_tmp_floats(int fmt, int64_t n) {
    return fmt == TML_FMT_Q8_K ? 0 : (size_t)partial_blocks(n);
}

Status launch_quantize(int fmt, int64_t n, const float *w, void *q, float *scales, float *tmp, hipStream_t s) {
    if (n <= 0) return Status::Ok();
    switch (fmt) {
        case TML_FMT_Q8_0:
        case TML_FMT_Q4_0: {
            const int np = partial_blocks(n);
            absmax_partials<<<np, kThreads, 0, s>>>(w, n, tmp);
            TML_HIP_TRY(hipGetLastError());
            if (fmt == TML_FMT_Q8_0)
                quantize_q8_kernel<<<grid_for(n), kThreads, 0, s>>>(w, n, tmp, np, (int8_t *)q, scales);
            else
                quantize_q4_kernel<<<grid_for((n + 1) / 2), kThreads, 0, s>>>(w, n, tmp, np, (uint8_t *)q, scales);
            TML_HIP_TRY(hipGetLastError());
            return Status::Ok();
        }
        case TML_FMT_Q8_K:
            quantize_q8k_kernel<<<grid_for(((n + 31) / 32) * 32), kThreads, 0, s>>>(w, n, (int8_t *)q, scales);
            TML_HIP_TRY(hipGetLastError());
            return Status::Ok();
        case TML_FMT_F16:
            to_f16_kernel<<<grid_for(n), kThreads, 0, s>>>(w, n, (uint16_t *)q);
            TML_HIP_TRY(hipGetLastError());
            return Status::Ok();
        default:
            return Status::Err(TML_ERR_INVALID_FORMAT, "quantize: format must be Q8_0, Q4_0, Q8_K or F16");
    }
}

}  // namespace tml
