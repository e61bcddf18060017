// gemv_x.hip -- decoder GEMV at M <= 4 on prepared Q8_0 / Q4_0 weights,
// activations staged once per workgroup.
//
//   C[M,N] = act((alpha * A[M,K] . Bdeq[K,N] + beta * C + bias[N]) + residual)
//
// B is the prepared copy of gemv_t.hip: row n of Bt holds column n of B,
// K contiguous in 16-byte chunks (16 int8 or 32 int4 values) with the
// superchunk interleave of tk_group, rows ldt bytes apart.
//
// The weight is read the way the read floor (stream_read.hip) reads a
// buffer.  Lane t of the workgroup owns slot t of a "layer" of L
// consecutive prepared rows (L = NT / nchunk; slot t is chunk
// c = t mod nchunk of row t / nchunk, lanes past L * nchunk idle), and a
// workgroup covers P layers.  A layer is one contiguous run of L * ldt
// bytes, so each wave-wide 16-byte load covers 1 KiB of consecutive bytes,
// and lane t's chunk index c is the same in every layer: the lane needs the
// activations of that one chunk only (E values per row, read from LDS once
// and held in registers) for all P rows it multiplies.
//
// Why: the per-lane kernel of gemv_t.hip loads, for every 16-byte weight
// chunk, the chunk's fp32 activations (128 bytes for a Q4_0 chunk) with
// vector-memory instructions, and with 40-chunk Q4_0 rows in 64-lane groups
// leaves a third of its lanes idle.  Measured on MI355X at Q4_0 1280x5120,
// M = 1 (3.83 us against a 2.80 us read of the same bytes): removing the
// dequantization or the multiply-adds changed nothing, removing the
// activation loads saved 0.25 us, so the issue rate of vector-memory
// instructions set the time.  Here the activations cost one direct-to-LDS
// copy per workgroup (M*K*4 bytes) and E/4 LDS reads per lane.
//
// Order of work: the activation copies (buffer_load ... lds, no registers)
// are issued first, then the lane's P weight loads.  Loads return in order,
// so after vmcnt(P) and a barrier the activations are in LDS while the
// weights are still in flight.  Each weight chunk is widened and multiplied
// as it arrives (Q8_0 / Q4_0's per-tensor scale -- and Q4_0's 1/16, see
// x16_elem -- stay in alpha).  The P * MR partial sums of a lane go through
// LDS, and 16 lanes add the nchunk partials of an output in a fixed order
// (an ascending run per lane, then a DPP tree), so the result does not
// depend on timing.
#include "tml_internal.hpp"

namespace tml {
namespace {

typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));
constexpr int kBufFlags = 0x00020000;

struct GemvXArgs {
    int M, N, K;
    const float *A;
    const uint8_t *Bt;
    unsigned ldt;             // bytes per prepared row
    const float *bias;
    const float *colscale;    // [N] per-column factor on A.B, or nullptr
    float *C;
    float alpha, beta;        // alpha includes the per-tensor scale (and 1/16 for Q4_0)
    int nchunk;               // 16-byte chunks per prepared row
    int act;
    const float *res;
    long long tail0;          // tml_act_tail0(M * N)
    unsigned wbytes;          // N * ldt: byte count of the Bt resource
    unsigned xbytes;          // M * K * 4: byte count of the A resource
    int rows_layer;           // L: rows per layer
    int xiters;               // activation copies per lane: ceil(M * K / 4 / NT)
};

template <int FMT> struct XElems;
template <> struct XElems<TML_FMT_Q8_0> { static constexpr int value = 16; };
template <> struct XElems<TML_FMT_Q4_0> { static constexpr int value = 32; };

// Element i of a prepared chunk as a float: Q8_0 the signed byte i; Q4_0
// sixteen times the signed nibble i (nibble i % 8 of dword i / 8, moved to
// the top of its byte and read as a signed byte -- one masked word per
// parity serves four nibbles -- the 1/16 being carried by alpha: a power of
// two, so every product and sum is exactly 16 times the unscaled one).
template <int FMT>
__device__ __forceinline__ float x16_elem(const uintx4 &w, int i) {
    if constexpr (FMT == TML_FMT_Q8_0) {
        return (float)((int32_t)(w[i / 4] << (24 - 8 * (i % 4))) >> 24);
    } else {
        const uint32_t word = w[i / 8];
        const int nib = i % 8;
        const uint32_t t = (nib & 1) ? (word & 0xF0F0F0F0u) : ((word << 4) & 0xF0F0F0F0u);
        return (float)(int8_t)(t >> (8 * (nib >> 1)));
    }
}

// First k of element group q (four consecutive k) of chunk ch: superchunks
// of 64 chunks, the last one `width` chunks wide (the prepared layout).
__device__ __forceinline__ int x_group_k(int ch, int q, int nchunk, int E) {
    const int sc = ch >> 6, c = ch & 63;
    const int width = min(64, nchunk - (sc << 6));
    return sc * 64 * E + 4 * (q * width + c);
}

template <int CTRL>
__device__ __forceinline__ float x_dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}

// s_waitcnt vmcnt(N), other counters untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void x_wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void x_wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt((0xF) | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));
}
// Workgroup barrier without a memory fence (a fence would wait for the
// weight loads in flight); the empty asm statements keep the compiler from
// moving memory accesses across it.
__device__ __forceinline__ void x_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int FMT, int MR, int NT, int P>
__global__ __launch_bounds__(NT) void gemv_x_kernel(GemvXArgs a) {
    constexpr int E = XElems<FMT>::value;
    TML_DYNAMIC_LDS(float, lds);  // the kernel's only LDS: its base is 16-byte aligned
    float *xs = lds;                             // [xiters * NT] float4: A, row-major
    float *red = lds + 4 * a.xiters * NT;        // [P][MR][NT] partial sums

    const int t = threadIdx.x;
    const int wave = t >> 6;
    const int L = a.rows_layer;
    const int rl = t / a.nchunk;  // row of the lane's slot within a layer (>= L: idle lane)
    const int c = t - rl * a.nchunk;
    const int row0 = blockIdx.x * (L * P);

    // 1. Activations to LDS: float4 i * NT + t of A lands at the same index
    //    of xs (a wave's copy writes 64 consecutive float4s from its base);
    //    offsets past M*K*4 read zeros.
    {
        const __amdgpu_buffer_rsrc_t rx =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(a.A), (short)0, (int)a.xbytes, kBufFlags);
        for (int i = 0; i < a.xiters; ++i) {
            float *base = xs + 4 * (i * NT + 64 * wave);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (__attribute__((address_space(3))) void *)base, 16,
                                                     16u * (unsigned)(i * NT + t), 0, 0, 0);
        }
    }
    asm volatile("" ::: "memory");
    // 2. The lane's weight chunks, one per layer; idle lanes and rows past N
    //    point past the resource (zeros, no traffic).
    uintx4 w[P];
    {
        const __amdgpu_buffer_rsrc_t rw =
            __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(a.Bt), (short)0, (int)a.wbytes, kBufFlags);
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int n = row0 + p * L + rl;
            const bool ok = rl < L && n < a.N;
            const unsigned off = ok ? (unsigned)n * a.ldt + 16u * (unsigned)c : 0x80000000u;
            w[p] = __builtin_amdgcn_raw_buffer_load_b128(rw, off, 0, kStreamLoadPolicy);
        }
    }
    // 3. Every wave's activation copies done (the P weight loads may still
    //    be in flight), then the lane's activations into registers.
    x_wait_vmcnt<P>();
    x_barrier();
    // (rows past M, when M is rounded up to MR, hold zeros: their products
    // are computed and dropped)
    floatx4 xr[MR][E / 4];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int q = 0; q < E / 4; ++q)
            xr[m][q] = (MR <= 2 || m < a.M) ? *(const floatx4 *)(xs + m * a.K + x_group_k(c, q, a.nchunk, E))
                                           : floatx4{0.f, 0.f, 0.f, 0.f};

    // 4. Dot products of the lane's chunk, layer by layer as the weights
    //    arrive: two chains per row, then their sum.
    float acc[P][MR];
#pragma unroll
    for (int p = 0; p < P; ++p) {
        float wv[E];
#pragma unroll
        for (int e = 0; e < E; ++e) wv[e] = x16_elem<FMT>(w[p], e);
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
            for (int e = 0; e < E; e += 2) {
                s0 += xr[m][e / 4][e % 4] * wv[e];
                s1 += xr[m][(e + 1) / 4][(e + 1) % 4] * wv[e + 1];
            }
            acc[p][m] = s0 + s1;
        }
    }
#pragma unroll
    for (int p = 0; p < P; ++p)
#pragma unroll
        for (int m = 0; m < MR; ++m) red[(p * MR + m) * NT + t] = acc[p][m];
    x_wait_lgkmcnt0();
    x_barrier();

    // 5. Output (layer p, row r, activation row m) = group g = (p L + r) MR
    //    + m: its 16 lanes add partials s, s + 16, ... in ascending order,
    //    then a DPP all-reduce over the 16-lane row; lane 0 of the group
    //    runs the epilogue.  Groups are whole DPP rows, so a row's lanes
    //    take the same trip count.
    const int s = t & 15;
    const int ngroups = L * P * MR;
    for (int g = t >> 4; g < ngroups; g += NT / 16) {
        const int m = g % MR, lr = g / MR;  // lr = p * L + r
        const int p = lr / L, r = lr - p * L;
        const float *part = red + (p * MR + m) * NT + r * a.nchunk;
        // four reads in flight per step (indices past the row read its last
        // partial and are dropped)
        const int last = a.nchunk - 1;
        float v = 0.0f;
        for (int cc = s; cc < a.nchunk; cc += 64) {
            const float v0 = part[cc];
            const float v1 = part[min(cc + 16, last)], v2 = part[min(cc + 32, last)], v3 = part[min(cc + 48, last)];
            v += v0;
            v += cc + 16 <= last ? v1 : 0.0f;
            v += cc + 32 <= last ? v2 : 0.0f;
            v += cc + 48 <= last ? v3 : 0.0f;
        }
        v += x_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
        v += x_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
        v += x_dpp<0x141>(v);  // row_half_mirror
        v += x_dpp<0x140>(v);  // row_mirror
        const int n = row0 + lr;
        if (s == 0 && m < a.M && n < a.N) {
            const long long flat = (long long)m * a.N + n;
            float y = (a.colscale ? a.alpha * a.colscale[n] : a.alpha) * v;
            if (a.beta != 0.0f) y += a.beta * a.C[flat];
            if (a.bias) y += a.bias[n];
            if (a.res) y += a.res[flat];
            a.C[flat] = tml_apply_act(y, a.act, flat, a.tail0);
        }
    }
}

struct XPlan {
    int nt, L, p, xiters;
    size_t lds;
};

int x_elems(int fmt) { return fmt == TML_FMT_Q8_0 ? 16 : 32; }

// Rows a launch computes: M rounded up to 1, 2 or 4.
int x_rows(int64_t M) { return M <= 1 ? 1 : M <= 2 ? 2 : 4; }

bool x_plan(int fmt, int64_t M, int64_t N, int64_t K, int cus, XPlan *out) {
    const int E = x_elems(fmt);
    const int64_t nchunk = K / E;
    if (nchunk < 1 || nchunk > 512) return false;
    // threads: 256 or 512, whichever leaves the smaller share of lanes idle
    // (ties: 256)
    auto idle = [&](int nt) { return nt < nchunk ? 1.0 : (double)(nt % nchunk) / nt; };
    XPlan p;
    p.nt = idle(512) < idle(256) ? 512 : 256;
    const int forced_nt = env_int("TML_GEMVX_NT", 0);
    if (forced_nt == 256 || forced_nt == 512) p.nt = forced_nt;
    if (p.nt < nchunk) p.nt = 512;
    if (p.nt < nchunk) return false;
    p.L = (int)(p.nt / nchunk);
    // two layers per workgroup, one where that leaves most CUs without a
    // workgroup.  Measured on MI355X (us, M = 1, layers 1 / 2 / 3 / 4 at 256
    // threads, or 512 where marked): Q4_0 1280x5120 3.79 / 3.60 / 4.16 /
    // 3.84 (512: 3.59 / 3.56); Q4_0 5120x1280 (512) 3.85 / 3.73 / 3.96 /
    // 4.16, at M = 2 4.65 / 4.29 / - / 5.13; Q8_0 1024x4096 3.41 / 3.37 /
    // 3.49 / 3.34.
    p.p = 2;
    if ((N + 2LL * p.L - 1) / (2LL * p.L) < cus / 2) p.p = 1;
    const int forced_p = env_int("TML_GEMVX_P", 0);
    if (forced_p >= 1 && forced_p <= 4) p.p = forced_p;
    // activations and partials within 64 KiB of LDS: fewer layers if need be
    p.xiters = (int)((M * K / 4 + p.nt - 1) / p.nt);
    auto lds_of = [&](int layers) { return (size_t)p.xiters * p.nt * 16 + (size_t)layers * x_rows(M) * p.nt * 4; };
    while (p.p > 1 && lds_of(p.p) > 64 * 1024) --p.p;
    p.lds = lds_of(p.p);
    if (p.lds > 64 * 1024) return false;
    *out = p;
    return true;
}

template <int FMT, int MR, int NT>
void x_launch_p(const GemvXArgs &ka, const XPlan &p, unsigned grid, hipStream_t s) {
    switch (p.p) {
        case 1: gemv_x_kernel<FMT, MR, NT, 1><<<dim3(grid), dim3(NT), p.lds, s>>>(ka); break;
        case 2: gemv_x_kernel<FMT, MR, NT, 2><<<dim3(grid), dim3(NT), p.lds, s>>>(ka); break;
        case 3: gemv_x_kernel<FMT, MR, NT, 3><<<dim3(grid), dim3(NT), p.lds, s>>>(ka); break;
        default: gemv_x_kernel<FMT, MR, NT, 4><<<dim3(grid), dim3(NT), p.lds, s>>>(ka); break;
    }
}
template <int FMT, int MR>
void x_launch_nt(const GemvXArgs &ka, const XPlan &p, unsigned grid, hipStream_t s) {
    if (p.nt == 512) x_launch_p<FMT, MR, 512>(ka, p, grid, s);
    else x_launch_p<FMT, MR, 256>(ka, p, grid, s);
}
template <int FMT>
void x_launch_m(const GemvXArgs &ka, const XPlan &p, unsigned grid, hipStream_t s) {
    if (ka.M == 1) x_launch_nt<FMT, 1>(ka, p, grid, s);
    else if (ka.M == 2) x_launch_nt<FMT, 2>(ka, p, grid, s);
    else x_launch_nt<FMT, 4>(ka, p, grid, s);
}

}  // namespace

// What the kernel runs: Q8_0 / Q4_0 at M = 1 to 4 (3 as 4), K a whole number of
// chunks (so every activation a lane reads belongs to its row), at most 512
// chunks a row, activations and partials within 64 KiB of LDS (M * K up to
// about 15000), and every buffer offset below 2^31.
bool gemv_x_capable(int fmt, int64_t M, int64_t N, int64_t K) {
    if (fmt != TML_FMT_Q8_0 && fmt != TML_FMT_Q4_0) return false;
    // (at 5-8 rows it measured slower than the matrix-core kernel on every
    // shape tried, 0.2-1.1 us at 1024 x 4096, 1024 x 2048, 1280 x 1280)
    if (M < 1 || M > 4 || K <= 0 || N <= 0 || K % x_elems(fmt) != 0) return false;
    XPlan p;
    if (!x_plan(fmt, M, N, K, 256, &p)) return false;
    const int64_t ldt = prepared_row_bytes(fmt, K);
    return N * ldt < ((int64_t)1 << 31) && M * K * 4 < ((int64_t)1 << 31) && N < ((int64_t)1 << 30);
}

// Where it is the faster kernel (measured on MI355X against the kernels of
// gemv_t.hip / gemv_tm.hip, every launch reading its own weight copy out of
// >= 1 GiB, weights streamed with the non-temporal policy, us):
//   * Q4_0 at M = 1 at every N (1280x5120 3.27 against 3.48, 5120x1280 3.42
//     against 3.70, vocabulary 1280x51866 10.27 against 10.82 on the matrix
//     cores, 2048x51866 13.66 against 15.34), at M = 2 below N = 32768
//     (2048x2048 3.29 against 4.17, 1280x1280 2.86 against 3.48, 5120x1280
//     4.29 against 5.33 before the non-temporal policy; 1280x5120, 1024x4096
//     within 0.05; the vocabulary 14.11 against 10.99 stays on the matrix
//     cores), and at M = 3-4 where N <= 2048 and K >= N, the matrix-core
//     kernel's 16-column tiles being few (3072x768 4.28 / 4.36 against
//     5.79 / 5.14, 2048x2048 3.84 / 3.93 against 4.66 / 4.21; 1280x2048 and
//     1024x4096 0.2-0.6 slower);
//   * Q8_0 from N = 12288 at M = 1 (1024x12288 4.49 against 5.05, vocabulary
//     1280x51866 13.22 against 13.94) and from N = 8192 at M = 2 (1024x8192
//     4.17 against 4.70, 1280x51866 16.46 against 19.30); at M <= 2 also
//     where a row's chunks leave 1-16 over a multiple of 64, which idles most
//     of the per-lane kernel's last 64-lane group (K = 1280: 1280x1280 2.82 /
//     2.96 against 2.97 / 3.57, 1280x5120 3.76 / 4.06 against 3.95 / 4.88);
//     elsewhere below those N the per-lane kernel (1024x4096 2.82 / 3.16
//     against 3.06 / 3.30, 768x3072, 512x4096, 3072x768); at M = 3-4 from
//     K = 1024 up to N = 4096 (1024x4096 3.89 / 4.01 against 4.23 / 4.40,
//     3072x768 4.07 / 4.23 against 6.16 / 5.50, 2048x2048 3.88 / 4.09 against
//     5.22 / 4.74; 768x3072, 1280x5120, 1536x6144 0.1-1.5 slower).
// TML_GEMVX=0 turns it off; TML_GEMVX=2 takes it wherever it can run, and
// TML_GEMVX=3 also makes the prepared GEMV refuse a call it cannot take
// (tests).
bool gemv_x_preferred(int fmt, int64_t M, int64_t N, int64_t K) {
    const int mode = env_int("TML_GEMVX", 1);
    if (mode == 0 || !gemv_x_capable(fmt, M, N, K)) return false;
    if (mode >= 2) return true;
    const int64_t tail = (K / x_elems(fmt)) % 64;
    if (fmt == TML_FMT_Q4_0) {
        if (M == 1) return true;
        if (M == 2) return N < 32768;
        return N <= 2048 && K >= N;
    }
    if (M <= 2) return N >= (M == 1 ? 12288 : 8192) || (tail > 0 && tail <= 16);
    return K >= 1024 && N <= 4096;
}

Status launch_gemv_x(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *Bt, int64_t ldt,
                     const float *bias, const float *res, float *C, float alpha_eff, float beta, int act,
                     long long tail0, const float *colscale, hipStream_t s) {
    if (!gemv_x_capable(fmt, M, N, K)) return Status::Err(TML_ERR_INVALID_ARG, "staged-activation GEMV: unsupported");
    if (ldt < prepared_row_bytes(fmt, K) || ldt % 16 != 0 || ((uintptr_t)Bt % 16) != 0 || ((uintptr_t)A % 16) != 0)
        return Status::Err(TML_ERR_INVALID_ARG, "staged-activation GEMV: prepared layout or alignment");
    if (N * ldt >= ((int64_t)1 << 31))
        return Status::Err(TML_ERR_INVALID_SHAPE, "staged-activation GEMV: weight too large");
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
    }
    XPlan p;
    if (!x_plan(fmt, M, N, K, cus, &p)) return Status::Err(TML_ERR_INVALID_ARG, "staged-activation GEMV: no plan");
    GemvXArgs ka;
    ka.M = (int)M; ka.N = (int)N; ka.K = (int)K;
    ka.A = A; ka.Bt = (const uint8_t *)Bt; ka.ldt = (unsigned)ldt;
    ka.bias = bias; ka.colscale = colscale; ka.C = C;
    ka.alpha = fmt == TML_FMT_Q4_0 ? alpha_eff * 0.0625f : alpha_eff;  // int4 read as 16 q
    ka.beta = beta;
    ka.nchunk = (int)(K / x_elems(fmt));
    ka.act = act; ka.res = res; ka.tail0 = tail0;
    ka.wbytes = (unsigned)(N * ldt);
    ka.xbytes = (unsigned)(M * K * 4);
    ka.rows_layer = p.L;
    ka.xiters = p.xiters;
    const int64_t rows_wg = (int64_t)p.L * p.p;
    const int64_t grid = (N + rows_wg - 1) / rows_wg;
    if (fmt == TML_FMT_Q8_0) x_launch_m<TML_FMT_Q8_0>(ka, p, (unsigned)grid, s);
    else x_launch_m<TML_FMT_Q4_0>(ka, p, (unsigned)grid, s);
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

}  // namespace tml
