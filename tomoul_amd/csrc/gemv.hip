// gemv.hip -- skinny GEMM / GEMV for M <= 8 (decoder shapes), all formats.
//
//   C[M,N] = alpha * A[M,K] . Bdeq[K,N] + beta * C + bias[N]
//
// At M <= 8 the product is bound by streaming B once from HBM; at the
// decoder sizes (3-4 MB of weights) a launch is latency-bound, so the design
// minimises dependent memory round trips:
//   * B stays in its stored [K,N] layout (N contiguous; src/core/
//     quantization.zig:193-197).  A workgroup owns a column strip of CL*VB
//     bytes of every row and walks all K rows of it: each lane loads VB
//     bytes (16, 8 or 4) of one row per instruction, CL lanes span the strip
//     and the 64/CL lane groups of each wave take different rows.  Rows are
//     fetched in batches of U per lane, two batches in flight, with
//     branch-free clamped addresses so the compiler keeps the batch's loads
//     outstanding together; the activations of each row are fetched in the
//     same batch.
//   * Dequantization happens in registers (sign-extending bit-field
//     extracts); Q8_0 / Q4_0 per-tensor scales are applied once in the
//     epilogue, Q8_K block scales per row chunk.
//   * Reduction over the rows of a strip: __shfl_xor across the lane groups
//     of a wave, then the 4 waves through LDS.
//   * Only when the output is too narrow to give enough strips is K split
//     across workgroups; then wave 0 of each workgroup stores its partial,
//     and the last workgroup of the strip to arrive (device-scope counter)
//     sums the partials in split order and writes C, so results do not
//     depend on scheduling.  That workgroup resets the counter.
#include "tml_internal.hpp"

namespace tml {
namespace {

constexpr int kThreads = 256;
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx2 __attribute__((ext_vector_type(2)));

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
    const void *zero;
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

// Vector path: one VB-byte load of row k at column n.  Branch-free: a chunk
// past the end of the row (last strip, N % SC != 0) reads the zero block (the
// address is selected, not the value), so every lane issues the same
// straight-line loads and the compiler keeps a whole batch in flight.  Host
// guarantees N % E == 0 and VB-byte alignment.
template <int FMT, int VB>
__device__ __forceinline__ void load_row(const GemvKArgs &a, int k, int n, Raw<VB> &r) {
    const bool in = n < a.N;
    const size_t e = (size_t)k * a.N + (in ? n : 0);
    const void *p = !in ? a.zero
                  : FMT == TML_FMT_F32 ? (const void *)((const float *)a.B + e)
                  : FMT == TML_FMT_Q4_0 ? (const void *)((const uint8_t *)a.B + e / 2)
                                        : (const void *)((const int8_t *)a.B + e);
    if constexpr (VB == 16) {
        const uintx4 v = *(const uintx4 *)p;
        r.w[0] = v[0]; r.w[1] = v[1]; r.w[2] = v[2]; r.w[3] = v[3];
    } else if constexpr (VB == 8) {
        const uintx2 v = *(const uintx2 *)p;
        r.w[0] = v[0]; r.w[1] = v[1];
    } else {
        r.w[0] = *(const uint32_t *)p;
    }
    if constexpr (FMT == TML_FMT_Q8_K) r.s = a.scales[e / a.block];
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

template <int FMT, int MR, int VB, int CL, int U, bool VEC>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvKArgs a) {
    constexpr int E = GemvFmt<FMT, VB>::E;
    constexpr int RL = 64 / CL;        // row lanes per wave
    constexpr int SC = CL * E;         // columns per segment
    constexpr int ROWSTEP = 4 * RL;    // rows per step of the workgroup

    __shared__ __attribute__((aligned(16))) float red[4 * MR * SC];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int cl = lane % CL, rl = lane / CL;
    const int R = wave * RL + rl;      // row lane within the workgroup

    const int seg = blockIdx.x % a.nseg;
    const int split = blockIdx.x / a.nseg;
    const int n = seg * SC + cl * E;
    const int k0 = split * a.krows;
    const int nk = min(a.K, k0 + a.krows) - k0;             // >= 1 (host)
    const int nb = (nk + U * ROWSTEP - 1) / (U * ROWSTEP);  // batches (uniform)

    float acc[MR][E];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int e = 0; e < E; ++e) acc[m][e] = 0.0f;

    // One batch = U rows per lane: B chunks plus the M activations of each
    // row.  Rows past the split re-read row k0 and get zero activations.
    Raw<VB> w0[U], w1[U];
    float x0[U][MR], x1[U][MR];
    auto load_batch = [&](Raw<VB> *w, float (*x)[MR], int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kk = R + (b * U + u) * ROWSTEP;
            const bool valid = kk < nk;
            const int k = k0 + (valid ? kk : 0);
            if constexpr (VEC) load_row<FMT, VB>(a, k, n, w[u]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const bool ok = valid && m < a.M;
                x[u][m] = *(ok ? a.A + (size_t)m * a.K + k : (const float *)a.zero);
            }
        }
    };
    auto compute_batch = [&](const Raw<VB> *w, const float (*x)[MR], int b) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float wv[E];
            if constexpr (VEC) {
                decode_row<FMT, VB>(w[u], wv);
            } else {
                const int kk = R + (b * U + u) * ROWSTEP;
                load_elems<FMT, E>(a, k0 + (kk < nk ? kk : 0), n, wv);
            }
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int e = 0; e < E; ++e) acc[m][e] += x[u][m] * wv[e];
        }
    };

    // Stream B with two batches in flight.
    load_batch(w0, x0, 0);
    for (int b = 0; b < nb; b += 2) {
        if (b + 1 < nb) load_batch(w1, x1, b + 1);
        compute_batch(w0, x0, b);
        if (b + 2 < nb) load_batch(w0, x0, b + 2);
        if (b + 1 < nb) compute_batch(w1, x1, b + 1);
    }

    // Reduce over the RL row lanes of the wave, then over the 4 waves.
#pragma unroll
    for (int off = CL; off < 64; off <<= 1)
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int e = 0; e < E; ++e) acc[m][e] += __shfl_xor(acc[m][e], off);
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

    // Split-K: wave 0 alone publishes this split's partial and, if this
    // workgroup is the last of its segment to arrive, sums all partials in
    // split order.  Its device-scope fence orders its own partial stores
    // before its counter increment (release) and its partial loads after it
    // (acquire), so one fence per workgroup suffices.
    if (wave != 0) return;
    for (int o = lane; o < MR * SC; o += 64) {
        const int m = o / SC, c = o % SC, col = col0 + c;
        if (m < a.M && col < a.N) {
            a.ws[((size_t)split * MR + m) * a.N + col] = red[m * SC + c] + red[(MR + m) * SC + c] +
                                                         red[(2 * MR + m) * SC + c] + red[(3 * MR + m) * SC + c];
        }
    }
    __threadfence();
    unsigned prev = 0;
    if (lane == 0) prev = __hip_atomic_fetch_add(a.counters + seg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    prev = __shfl(prev, 0);
    if (prev != (unsigned)(a.nsplit - 1)) return;
    __threadfence();
    for (int o = lane; o < MR * SC; o += 64) {
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
    if (lane == 0) a.counters[seg] = 0u;  // ready for the next launch
}

// ---------------------------------------------------------------- host side
struct GemvPlan {
    int mr, vb, e, cl, sc, rowstep;
    int nseg, nsplit, krows;
    bool vec;
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

// Bytes of B one workgroup should stream: enough to keep its CU's memory
// pipeline full for one latency, small enough that the grid reaches many CUs.
constexpr int64_t kBlockBytes = 64 << 10;
constexpr int64_t kMinBlocks = 32;

GemvPlan make_plan(const MatmulArgs &m) {
    GemvPlan p{};
    p.mr = m.M <= 1 ? 1 : m.M <= 2 ? 2 : m.M <= 4 ? 4 : 8;
    p.vb = pick_vb(m.fmt, p.mr);
    p.e = elems_per_lane(m.fmt, p.vb);
    p.vec = (m.N % p.e == 0) && is_aligned(m.B, (size_t)p.vb);
    if (m.fmt == TML_FMT_Q8_K) p.vec = p.vec && (m.block % p.e == 0);
    const int64_t block_bytes = env_int("TML_GEMV_BLOCK_KB", 0) > 0 ? (int64_t)env_int("TML_GEMV_BLOCK_KB", 0) << 10
                                                                     : kBlockBytes;
    // Column strip per workgroup: the widest strip (CL lanes of VB bytes)
    // whose K rows fit the byte budget with enough strips to spread over
    // the CUs; each workgroup then covers all of K and needs no reduction
    // with other workgroups.
    int cl = 1;
    bool fits = false;
    for (int c = 8; c >= 1; c >>= 1) {
        const int64_t nseg = (m.N + (int64_t)c * p.e - 1) / ((int64_t)c * p.e);
        if ((int64_t)c * p.vb * m.K <= block_bytes && nseg >= kMinBlocks) {
            cl = c;
            fits = true;
            break;
        }
    }
    const int forced_cl = env_int("TML_GEMV_CL", 0);
    if (forced_cl == 1 || forced_cl == 2 || forced_cl == 4 || forced_cl == 8) cl = forced_cl;
    p.cl = cl;
    p.sc = cl * p.e;
    p.rowstep = 4 * (64 / cl);
    p.nseg = (int)((m.N + p.sc - 1) / p.sc);
    // Narrow outputs (few strips): split K across workgroups as well.
    int64_t nsplit = 1;
    if (!fits) {
        const int64_t per_strip = (int64_t)p.cl * p.vb * m.K;
        nsplit = (per_strip + block_bytes - 1) / block_bytes;
        const int64_t need = (kMinBlocks + p.nseg - 1) / p.nseg;
        if (nsplit < need) nsplit = need;
    }
    const int forced = env_int("TML_GEMV_SPLIT", 0);
    if (forced > 0) nsplit = forced;
    const int64_t max_split = m.K > p.rowstep ? m.K / p.rowstep : 1;
    if (nsplit > max_split) nsplit = max_split;
    if (nsplit < 1) nsplit = 1;
    int64_t kr = (m.K + nsplit - 1) / nsplit;
    kr = ((kr + p.rowstep - 1) / p.rowstep) * p.rowstep;
    if (kr < p.rowstep) kr = p.rowstep;
    p.krows = (int)kr;
    p.nsplit = m.K == 0 ? 1 : (int)((m.K + kr - 1) / kr);
    return p;
}

template <int FMT, int MR, int VB, int CL, bool VEC>
void launch_one(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    constexpr int U = MR <= 2 ? 8 : 4;  // rows per lane per batch (register budget)
    gemv_kernel<FMT, MR, VB, CL, U, VEC><<<dim3((unsigned)(p.nseg * p.nsplit)), dim3(kThreads), 0, s>>>(ka);
}

template <int FMT, int MR, int VB, bool VEC>
void launch_cl(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    switch (p.cl) {
        case 1: launch_one<FMT, MR, VB, 1, VEC>(ka, p, s); break;
        case 2: launch_one<FMT, MR, VB, 2, VEC>(ka, p, s); break;
        case 4: launch_one<FMT, MR, VB, 4, VEC>(ka, p, s); break;
        default: launch_one<FMT, MR, VB, 8, VEC>(ka, p, s); break;
    }
}

template <int FMT, int MR>
Status launch_mr(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    constexpr int VB_VEC = FMT == TML_FMT_F32 ? 16
                         : (FMT == TML_FMT_Q4_0 ? (MR <= 2 ? 16 : (MR == 4 ? 8 : 4)) : (MR <= 4 ? 16 : 8));
    if (p.vb != VB_VEC) return Status::Err(TML_ERR_INVALID_ARG, "gemv plan/instantiation mismatch");
    if (p.vec) launch_cl<FMT, MR, VB_VEC, true>(ka, p, s);
    else launch_cl<FMT, MR, VB_VEC, false>(ka, p, s);
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
    ka.zero = m.zero;
    switch (m.fmt) {
        case TML_FMT_F32: return launch_fmt<TML_FMT_F32>(ka, p, s);
        case TML_FMT_Q8_0: return launch_fmt<TML_FMT_Q8_0>(ka, p, s);
        case TML_FMT_Q8_K: return launch_fmt<TML_FMT_Q8_K>(ka, p, s);
        case TML_FMT_Q4_0: return launch_fmt<TML_FMT_Q4_0>(ka, p, s);
        default: return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    }
}

}  // namespace tml
