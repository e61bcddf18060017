// stream_read.hip -- the read floor of a decoder GEMV: one launch that reads
// a buffer once with 16-byte loads and does nothing else.
//
// A decoder GEMV (M <= 8) streams a few MB of weights per launch.  At that
// size its time is set by the launch and by memory latency, not by HBM
// bandwidth, so "per cent of 8 TB/s" alone says little about the kernel.
// This kernel is the yardstick: the same bytes, read the fastest way this
// hardware allows -- every lane issues all of its U loads back to back,
// each wave-wide load instruction covers 1 KiB of contiguous bytes, loads
// go through a buffer resource (offsets past the end read zeros, no
// branches) with the non-temporal cache policy (kStreamLoadPolicy, which
// read 4 MB in 2.65 against 2.90 us with the default policy) -- then one integer fold of what was read, a reduction over the
// workgroup and one 4-byte store per workgroup, so that nothing of the read
// can be dropped by the compiler.  A GEMV that streams the same bytes
// cannot take less time than this, and its ratio to it is the figure the
// benchmark reports as frac_of_floor.
#include "tml_internal.hpp"

namespace tml {
namespace {

constexpr int kThreads = 256;
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));

template <int U>
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const void *src, unsigned nbytes, float *out) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(src), (short)0, (int)nbytes, 0x00020000);
    // workgroup b reads bytes [b * U * 4 KiB, (b + 1) * U * 4 KiB); load j of a
    // lane is 16 bytes at j * 4 KiB + 16 * threadIdx.x of that range
    const unsigned base = (unsigned)blockIdx.x * (unsigned)(U * kThreads * 16) + threadIdx.x * 16u;
    uintx4 v[U];
#pragma unroll
    for (int j = 0; j < U; ++j)
        v[j] = __builtin_amdgcn_raw_buffer_load_b128(r, base + (unsigned)j * (kThreads * 16u), 0, kStreamLoadPolicy);
    unsigned acc = 0;
#pragma unroll
    for (int j = 0; j < U; ++j) acc += (v[j].x ^ v[j].y) + (v[j].z ^ v[j].w);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    __shared__ unsigned part[kThreads / 64];
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = (float)(part[0] + part[1] + part[2] + part[3]);
}

}  // namespace

int64_t stream_read_outputs(int64_t bytes, int chunks_per_lane) {
    const int64_t per = (int64_t)chunks_per_lane * kThreads * 16;
    return (bytes + per - 1) / per;
}

Status launch_stream_read(const void *src, int64_t bytes, int chunks_per_lane, float *out, hipStream_t s) {
    if (bytes < 0 || bytes >= ((int64_t)1 << 31))
        return Status::Err(TML_ERR_INVALID_SHAPE, "stream read: bytes must be in [0, 2^31)");
    if (bytes == 0) return Status::Ok();
    if (src == nullptr || out == nullptr) return Status::Err(TML_ERR_INVALID_ARG, "null pointer");
    const dim3 grid((unsigned)stream_read_outputs(bytes, chunks_per_lane)), block(kThreads);
    switch (chunks_per_lane) {
        case 1: stream_read_kernel<1><<<grid, block, 0, s>>>(src, (unsigned)bytes, out); break;
        case 2: stream_read_kernel<2><<<grid, block, 0, s>>>(src, (unsigned)bytes, out); break;
        case 4: stream_read_kernel<4><<<grid, block, 0, s>>>(src, (unsigned)bytes, out); break;
        case 8: stream_read_kernel<8><<<grid, block, 0, s>>>(src, (unsigned)bytes, out); break;
        default: return Status::Err(TML_ERR_INVALID_ARG, "stream read: chunks per lane must be 1, 2, 4 or 8");
    }
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

}  // namespace tml
