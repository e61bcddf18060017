// gemv.hip -- skinny GEMM / GEMV for M <= 8 (decoder shapes), all formats.
//
//   C[M,N] = alpha * A[M,K] . Bdeq[K,N] + beta * C + bias[N]
//
// At M <= 8 the product is HBM-bound on B, so the kernel is built around
// streaming B once with full-width loads:
//   * B stays in its stored [K,N] layout (N contiguous; src/core/
//     quantization.zig:193-197).  Each lane owns E consecutive columns and
//     loads VB bytes of one row per instruction (VB = 16, 8 or 4); CL = 128/VB
//     neighbouring lanes cover one 128-byte row segment, the other RL = 64/CL
//     lane groups of the wave take other rows.  A workgroup (4 waves) owns
//     one column segment and a range of rows ("split"); every lane issues all
//     of its row loads before it touches any of them.
//   * Dequantization happens in registers (sign-extending bit-field
//     extracts); Q8_0 / Q4_0 per-tensor scales are applied once in the
//     epilogue, Q8_K block scales per row chunk.
//   * A's rows of the split are staged in LDS as [k][m] so a lane fetches
//     the M activations of its row with ds_read_b128.
//   * Reduction: lane groups of a wave with __shfl_xor, the 4 waves through
//     LDS, and the splits of a column segment through a workspace: every
//     workgroup stores its partial, the last one to arrive (device-scope
//     counter) sums the partials in split order and writes C, so results do
//     not depend on scheduling.  The counter is reset by that workgroup.
#include "tml_internal.hpp"

namespace tml {
namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerBatch = 8;
constexpr int kMaxStagedFloats = 8192;  // LDS budget of the staged A slice (32 KiB)

struct GemvKArgs {
    int M, N, K;
    const float *A;
    const void *B;
    const float *scales;
    long long block;
    const float *bias;
    float *C;
    float alpha, beta;
    int nseg, nsplit, krows;  // krows = rows per split
    float *ws;
    unsigned *counters;
};

template <int FMT, int VB> struct GemvFmt;
template <int VB> struct GemvFmt<TML_FMT_F32, VB> { static constexpr int E = VB / 4; };
template <int VB> struct GemvFmt<TML_FMT_Q8_0, VB> { static constexpr int E = VB; };
template <int VB> struct GemvFmt<TML_FMT_Q8_K, VB> { static constexpr int E = VB; };
template <int VB> struct GemvFmt<TML_FMT_Q4_0, VB> { static constexpr int E = 2 * VB; };

template <int VB> struct Raw { uint32_t w[VB / 4]; float s; };

// Sign-extending field extracts (compile to v_bfe_i32).
__device__ __forceinline__ float sext8(uint32_t word, int byte) {
    return (float)((int32_t)(word << (24 - 8 * byte)) >> 24);
}
__device__ __forceinline__ float sext4(uint32_t word, int nib) {
    return (float)((int32_t)(word << (28 - 4 * nib)) >> 28);
}

// Vector path: one VB-byte load per row (host guarantees N % E == 0 and
// VB-byte alignment, so a chunk is either wholly inside B or past its end).
template <int FMT, int VB>
__device__ __forceinline__ void load_row(const GemvKArgs &a, int k, int n, Raw<VB> &r) {
    const size_t e = (size_t)k * a.N + n;
    const bool in = n < a.N;
    const void *p = FMT == TML_FMT_F32 ? (const void *)((const float *)a.B + e)
                  : FMT == TML_FMT_Q4_0 ? (const void *)((const uint8_t *)a.B + e / 2)
                                        : (const void *)((const int8_t *)a.B + e);
    if constexpr (VB == 16) {
        uint4 v = in ? *(const uint4 *)p : make_uint4(0, 0, 0, 0);
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else if constexpr (VB == 8) {
        uint2 v = in ? *(const uint2 *)p : make_uint2(0, 0);
        r.w[0] = v.x; r.w[1] = v.y;
    } else {
        r.w[0] = in ? *(const uint32_t *)p : 0u;
    }
    if constexpr (FMT == TML_FMT_Q8_K) r.s = in ? a.scales[e / a.block] : 0.0f;
}

// Generic path: element-wise loads with bounds, any N and alignment; the
// values come back dequantized (Q8_K scale applied, Q8_0 / Q4_0 as integers).
template <int FMT, int E>
__device__ __forceinline__ void load_elems(const GemvKArgs &a, int k, int n, float *w) {
    const size_t e = (size_t)k * a.N + n;
#pragma unroll
    for (int i = 0; i < E; ++i) {
        float v = 0.0f;
        if (n + i < a.N) {
            const size_t ei = e + i;
            if constexpr (FMT == TML_FMT_F32) v = ((const float *)a.B)[ei];
            else if constexpr (FMT == TML_FMT_Q8_0) v = (float)((const int8_t *)a.B)[ei];
            else if constexpr (FMT == TML_FMT_Q8_K) v = (float)((const int8_t *)a.B)[ei] * a.scales[ei / a.block];
            else v = sext4(((const uint8_t *)a.B)[ei / 2], (int)(ei & 1));
        }
        w[i] = v;
    }
}

template <int FMT, int VB>
__device__ __forceinline__ void decode_row(const Raw<VB> &r, float *w) {
    constexpr int E = GemvFmt<FMT, VB>::E;
    if constexpr (FMT == TML_FMT_F32) {
#pragma unroll
        for (int i = 0; i < E; ++i) w[i] = __uint_as_float(r.w[i]);
    } else if constexpr (FMT == TML_FMT_Q8_0) {
#pragma unroll
        for (int i = 0; i < E; ++i) w[i] = sext8(r.w[i / 4], i % 4);
    } else if constexpr (FMT == TML_FMT_Q8_K) {
        // Reference dequantization: f32(q) * scale per element
        // (quantization.zig:598-600).
#pragma unroll
        for (int i = 0; i < E; ++i) w[i] = sext8(r.w[i / 4], i % 4) * r.s;
    } else {
#pragma unroll
        for (int i = 0; i < E; ++i) w[i] = sext4(r.w[i / 8], i % 8);
    }
}

template <int FMT, int MR, int VB, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvKArgs a) {
    constexpr int E = GemvFmt<FMT, VB>::E;
    constexpr int CL = 128 / VB;       // column lanes per row segment
    constexpr int RL = 64 / CL;        // row lanes per wave
    constexpr int SC = CL * E;         // columns per segment
    constexpr int ROWSTEP = 4 * RL;    // rows per step of the workgroup
    constexpr int U = kRowsPerBatch;   // rows per lane per batch

    extern __shared__ __attribute__((aligned(16))) float smem[];
    float *xs = smem;                  // [krows][MR]
    float *red = smem;                 // reused after the main loop: [4][MR][SC]
    __shared__ int s_last;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int cl = lane % CL, rl = lane / CL;
    const int R = wave * RL + rl;      // row lane within the workgroup

    const int seg = blockIdx.x % a.nseg;
    const int split = blockIdx.x / a.nseg;
    const int n = seg * SC + cl * E;
    const int k0 = split * a.krows;
    const int k1 = min(a.K, k0 + a.krows);
    const int nk = k1 - k0;
    const int nb = (nk + U * ROWSTEP - 1) / (U * ROWSTEP);  // batches (uniform)

    float acc[MR][E];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[m][e] = 0.0f;

    // Row kk (relative to k0) of batch b, slot u.
    auto row_of = [&](int b, int u) { return R + (b * U + u) * ROWSTEP; };
    auto load_batch = [&](Raw<VB> *raw, int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kk = row_of(b, u);
            if (kk < nk) load_row<FMT, VB>(a, k0 + kk, n, raw[u]);
        }
    };
    auto compute_batch = [&](const Raw<VB> *raw, int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kk = row_of(b, u);
            if (kk < nk) {
                float w[E];
                if constexpr (VEC) decode_row<FMT, VB>(raw[u], w);
                else load_elems<FMT, E>(a, k0 + kk, n, w);
                float x[MR];
                if constexpr (MR % 4 == 0) {
#pragma unroll
                    for (int m = 0; m < MR; m += 4) {
                        const float4 t = *(const float4 *)&xs[kk * MR + m];
                        x[m] = t.x; x[m + 1] = t.y; x[m + 2] = t.z; x[m + 3] = t.w;
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < MR; ++m) x[m] = xs[kk * MR + m];
                }
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int e = 0; e < E; ++e) acc[m][e] += x[m] * w[e];
            }
        }
    };

    // 1. Issue the first batch of B loads, then stage A[:, k0:k1] in LDS
    //    as [k][m] (zero for m >= M) while they are in flight.
    Raw<VB> raw0[VEC ? U : 1], raw1[VEC ? U : 1];
    if constexpr (VEC) load_batch(raw0, 0);
    for (int i = tid; i < nk * MR; i += kThreads) {
        const int kk = i / MR, m = i % MR;
        xs[kk * MR + m] = m < a.M ? a.A[(size_t)m * a.K + k0 + kk] : 0.0f;
    }
    __syncthreads();

    // 2. Stream B: two register batches in flight.
    for (int b = 0; b < nb; b += 2) {
        if constexpr (VEC) {
            if (b + 1 < nb) load_batch(raw1, b + 1);
        }
        compute_batch(raw0, b);
        if constexpr (VEC) {
            if (b + 2 < nb) load_batch(raw0, b + 2);
        }
        if (b + 1 < nb) compute_batch(raw1, b + 1);
    }

    // 3. Reduce over the RL row lanes of the wave.
#pragma unroll
    for (int off = CL; off < 64; off <<= 1)
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int e = 0; e < E; ++e) acc[m][e] += __shfl_xor(acc[m][e], off);

    // 4. Reduce over the 4 waves through LDS.
    __syncthreads();  // xs is dead; reuse the space
    if (rl == 0) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int e = 0; e < E; ++e) red[(wave * MR + m) * SC + cl * E + e] = acc[m][e];
    }
    __syncthreads();

    const int col0 = seg * SC;
    if (a.nsplit == 1) {
        for (int o = tid; o < MR * SC; o += kThreads) {
            const int m = o / SC, c = o % SC, col = col0 + c;
            if (m < a.M && col < a.N) {
                const float p = red[m * SC + c] + red[(MR + m) * SC + c] + red[(2 * MR + m) * SC + c] +
                                red[(3 * MR + m) * SC + c];
                float *cp = a.C + (size_t)m * a.N + col;
                float v = a.alpha * p;
                if (a.beta != 0.0f) v += a.beta * *cp;
                if (a.bias) v += a.bias[col];
                *cp = v;
            }
        }
        return;
    }

    // 5. Split-K: publish this split's partial; the last workgroup of the
    //    segment to arrive sums all partials in split order.
    for (int o = tid; o < MR * SC; o += kThreads) {
        const int m = o / SC, c = o % SC, col = col0 + c;
        if (m < a.M && col < a.N) {
            a.ws[((size_t)split * MR + m) * a.N + col] = red[m * SC + c] + red[(MR + m) * SC + c] +
                                                         red[(2 * MR + m) * SC + c] + red[(3 * MR + m) * SC + c];
        }
    }
    __threadfence();  // release the partial at device scope
    __syncthreads();
    if (tid == 0) {
        const unsigned prev = __hip_atomic_fetch_add(a.counters + seg, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        s_last = (prev == (unsigned)(a.nsplit - 1));
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();  // acquire every other split's partial
    for (int o = tid; o < MR * SC; o += kThreads) {
        const int m = o / SC, c = o % SC, col = col0 + c;
        if (m < a.M && col < a.N) {
            const float *src = a.ws + (size_t)m * a.N + col;
            const size_t stride = (size_t)MR * a.N;
            float p = 0.0f;
#pragma unroll 8
            for (int s = 0; s < a.nsplit; ++s) p += src[s * stride];
            float *cp = a.C + (size_t)m * a.N + col;
            float v = a.alpha * p;
            if (a.beta != 0.0f) v += a.beta * *cp;
            if (a.bias) v += a.bias[col];
            *cp = v;
        }
    }
    if (tid == 0) a.counters[seg] = 0u;  // ready for the next launch
}

// ---------------------------------------------------------------- host side
struct GemvPlan {
    int mr, vb, e, sc, rowstep;
    int nseg, nsplit, krows;
    bool vec;
    size_t smem;
};

int pick_vb(int fmt, int mr) {
    switch (fmt) {
        case TML_FMT_F32: return 16;
        case TML_FMT_Q8_0:
        case TML_FMT_Q8_K: return mr <= 4 ? 16 : 8;
        default: return mr <= 2 ? 16 : (mr == 4 ? 8 : 4);  // Q4_0
    }
}

int elems_per_lane(int fmt, int vb) {
    return fmt == TML_FMT_F32 ? vb / 4 : (fmt == TML_FMT_Q4_0 ? 2 * vb : vb);
}

bool is_aligned(const void *p, size_t n) { return ((uintptr_t)p % n) == 0; }

GemvPlan make_plan(const MatmulArgs &m) {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
            cus = 256;
    }
    GemvPlan p{};
    p.mr = m.M <= 1 ? 1 : m.M <= 2 ? 2 : m.M <= 4 ? 4 : 8;
    p.vb = pick_vb(m.fmt, p.mr);
    p.e = elems_per_lane(m.fmt, p.vb);
    p.vec = (m.N % p.e == 0) && is_aligned(m.B, (size_t)p.vb);
    if (m.fmt == TML_FMT_Q8_K) p.vec = p.vec && (m.block % p.e == 0);
    const int cl = 128 / p.vb, rl = 64 / cl;
    p.sc = cl * p.e;
    p.rowstep = 4 * rl;
    p.nseg = (int)((m.N + p.sc - 1) / p.sc);
    // Splits: enough workgroups to give every CU one (each streams its rows
    // with two 8-row batches in flight per lane), never so few that the
    // staged A slice outgrows its LDS budget, never less than one ROWSTEP of
    // rows per split.  TML_GEMV_SPLIT forces a split count (experiments).
    const int64_t max_split = m.K > p.rowstep ? m.K / p.rowstep : 1;
    const int64_t min_split = (m.K * p.mr + kMaxStagedFloats - 1) / kMaxStagedFloats;
    int64_t want = (cus + p.nseg - 1) / p.nseg;
    const int forced = env_int("TML_GEMV_SPLIT", 0);
    if (forced > 0) want = forced;
    int64_t nsplit = want < max_split ? want : max_split;
    if (nsplit < min_split) nsplit = min_split;
    if (nsplit < 1) nsplit = 1;
    int64_t kr = (m.K + nsplit - 1) / nsplit;
    kr = ((kr + p.rowstep - 1) / p.rowstep) * p.rowstep;
    if (kr * p.mr > kMaxStagedFloats) kr = (kMaxStagedFloats / p.mr / p.rowstep) * p.rowstep;
    if (kr < p.rowstep) kr = p.rowstep;
    p.krows = (int)kr;
    p.nsplit = (int)((m.K + kr - 1) / kr);
    if (m.K == 0) { p.krows = p.rowstep; p.nsplit = 1; }
    const size_t xs = (size_t)p.krows * p.mr * sizeof(float);
    const size_t red = (size_t)4 * p.mr * p.sc * sizeof(float);
    p.smem = xs > red ? xs : red;
    return p;
}

template <int FMT, int MR, int VB, bool VEC>
void launch_one(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    gemv_kernel<FMT, MR, VB, VEC><<<dim3((unsigned)(p.nseg * p.nsplit)), dim3(kThreads), p.smem, s>>>(ka);
}

template <int FMT, int MR>
Status launch_mr(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    constexpr int VB_VEC = FMT == TML_FMT_F32 ? 16
                         : (FMT == TML_FMT_Q4_0 ? (MR <= 2 ? 16 : (MR == 4 ? 8 : 4)) : (MR <= 4 ? 16 : 8));
    if (p.vb != VB_VEC) return Status::Err(TML_ERR_INVALID_ARG, "gemv plan/instantiation mismatch");
    if (p.vec) launch_one<FMT, MR, VB_VEC, true>(ka, p, s);
    else launch_one<FMT, MR, VB_VEC, false>(ka, p, s);
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

template <int FMT>
Status launch_fmt(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    switch (p.mr) {
        case 1: return launch_mr<FMT, 1>(ka, p, s);
        case 2: return launch_mr<FMT, 2>(ka, p, s);
        case 4: return launch_mr<FMT, 4>(ka, p, s);
        case 8: return launch_mr<FMT, 8>(ka, p, s);
        default: return Status::Err(TML_ERR_INVALID_ARG, "gemv rows");
    }
}

}  // namespace

void gemv_workspace_need(const MatmulArgs &m, size_t *partial_floats, size_t *counters) {
    const GemvPlan p = make_plan(m);
    *partial_floats = p.nsplit > 1 ? (size_t)p.nsplit * p.mr * (size_t)m.N : 0;
    *counters = p.nsplit > 1 ? (size_t)p.nseg : 0;
}

Status launch_gemv(const MatmulArgs &m, const Workspace &ws, hipStream_t s) {
    if (m.M < 1 || m.M > kGemvMaxM) return Status::Err(TML_ERR_INVALID_SHAPE, "gemv needs 1 <= M <= 8");
    const int64_t lim = (int64_t)1 << 30;
    if (m.N >= lim || m.K >= lim) return Status::Err(TML_ERR_INVALID_SHAPE, "GEMV dimension exceeds 2^30");
    const GemvPlan p = make_plan(m);
    if (p.nsplit > 1) {
        const size_t need = (size_t)p.nsplit * p.mr * (size_t)m.N;
        if (ws.partials == nullptr || ws.partial_floats < need || ws.counters == nullptr ||
            ws.counter_count < (size_t)p.nseg)
            return Status::Err(TML_ERR_INVALID_ARG, "gemv workspace too small");
    }
    if ((int64_t)p.nseg * p.nsplit >= ((int64_t)1 << 31))
        return Status::Err(TML_ERR_INVALID_SHAPE, "gemv grid too large");
    GemvKArgs ka;
    ka.M = (int)m.M; ka.N = (int)m.N; ka.K = (int)m.K;
    ka.A = m.A; ka.B = m.B; ka.scales = m.scales; ka.block = m.block;
    ka.bias = m.bias; ka.C = m.C; ka.alpha = m.alpha_eff; ka.beta = m.beta;
    ka.nseg = p.nseg; ka.nsplit = p.nsplit; ka.krows = p.krows;
    ka.ws = ws.partials; ka.counters = ws.counters;
    switch (m.fmt) {
        case TML_FMT_F32: return launch_fmt<TML_FMT_F32>(ka, p, s);
        case TML_FMT_Q8_0: return launch_fmt<TML_FMT_Q8_0>(ka, p, s);
        case TML_FMT_Q8_K: return launch_fmt<TML_FMT_Q8_K>(ka, p, s);
        case TML_FMT_Q4_0: return launch_fmt<TML_FMT_Q4_0>(ka, p, s);
        default: return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    }
}

}  // namespace tml
