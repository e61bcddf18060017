// gemm_mfma.hip -- tiled GEMM on gfx950 fp32 matrix cores.
//
//   C[M,N] = alpha * A[M,K] . Bdeq[K,N] + beta * C + bias[N]
//
// One kernel template serves the fp32 SGEMM (ops.matmul / matmulBias,
// src/core/ops.zig:235-471) and the large-M weight-only quantized GEMMs
// (matmulF32Q8Simd / Q8KSimd / Q4Simd, src/core/quantization.zig:207-957):
// B is read from HBM in its stored format (f32, int8 or packed int4),
// dequantized on the register -> LDS store, and every product runs on
// v_mfma_f32_16x16x4_f32 with fp32 accumulation.
//
// Layout of one workgroup (256 threads = 4 wave64s, arranged 2 x 2):
//   block tile BM x BN, K consumed in BK slices, each slice staged through
//   LDS with two buffers: slice t+1 is fetched from global memory into
//   registers while the waves run the MFMAs of slice t.
//   As[buf][BM][BK+4]  A slice, k contiguous (16-byte reads per lane)
//   Bs[buf][BK][BN+4]  B slice as f32, n contiguous
//   The +4 pads make the per-lane 16-byte A reads and the 4-row-apart B
//   reads of the MFMA operand pattern bank-conflict free.
// MFMA operand mapping (16x16x4 f32, wave64): lane l feeds A[l%16][kk] and
// B[kk][l%16] with kk = l/16, and holds D[4*(l/16)+r][l%16] in register r.
// Within a 16-deep k chunk, step s (0..3) feeds kk = l/16 with the physical
// k = 4*kk + s, so each lane reads its four A values with one ds_read_b128.
//
// Workgroup -> tile: the hardware deals workgroups round-robin over the
// 8 XCDs (each with its own L2); ids are remapped so that consecutive tiles
// run on one XCD, then grouped GROUP_M tile-rows at a time so neighbouring
// workgroups share A rows and B columns in that XCD's L2.
#include "tml_internal.hpp"

namespace tml {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;
constexpr int kNumXcd = 8;

struct GemmKArgs {
    int M, N, K;
    const float *A;
    const void *B;
    const float *scales;
    long long block;
    const float *bias;
    float *C;
    float alpha;
    float beta;
    int tiles_m, tiles_n, group_m;
};

// ---------------------------------------------------------------- B formats
// Elements of B moved per global load ("chunk") in the vector path.
template <int FMT> struct BFmt;
template <> struct BFmt<TML_FMT_F32> { static constexpr int EPC = 4; };
template <> struct BFmt<TML_FMT_Q8_0> { static constexpr int EPC = 8; };
template <> struct BFmt<TML_FMT_Q8_K> { static constexpr int EPC = 8; };
template <> struct BFmt<TML_FMT_Q4_0> { static constexpr int EPC = 8; };

// Raw registers of one B chunk.
struct BRaw {
    uint32_t w[4];
    float s;
};

// Sign-extending field extracts (compile to v_bfe_i32).
__device__ __forceinline__ float sext8(uint32_t word, int byte) {
    return (float)((int32_t)(word << (24 - 8 * byte)) >> 24);
}
__device__ __forceinline__ float sext4(uint32_t word, int nib) {
    return (float)((int32_t)(word << (28 - 4 * nib)) >> 28);
}

// Vector-path chunk load at (k, n); caller guarantees n % EPC == 0.
template <int FMT>
__device__ __forceinline__ void load_b_vec(const GemmKArgs &a, int k, int n, BRaw &r) {
    const bool in = (k < a.K) && (n < a.N);
    const size_t e = (size_t)k * a.N + n;
    if constexpr (FMT == TML_FMT_F32) {
        uint4 v = in ? *(const uint4 *)((const float *)a.B + e) : make_uint4(0, 0, 0, 0);
        r.w[0] = v.x; r.w[1] = v.y; r.w[2] = v.z; r.w[3] = v.w;
    } else if constexpr (FMT == TML_FMT_Q8_0 || FMT == TML_FMT_Q8_K) {
        uint2 v = in ? *(const uint2 *)((const int8_t *)a.B + e) : make_uint2(0, 0);
        r.w[0] = v.x; r.w[1] = v.y;
        if constexpr (FMT == TML_FMT_Q8_K) r.s = in ? a.scales[e / a.block] : 0.0f;
    } else {  // Q4_0: 8 nibbles = 4 bytes starting at byte e/2 (e % 8 == 0)
        r.w[0] = in ? *(const uint32_t *)((const uint8_t *)a.B + e / 2) : 0u;
    }
}

// Generic-path chunk: element-wise with bounds, any alignment.
template <int FMT>
__device__ __forceinline__ float load_b_elem(const GemmKArgs &a, int k, int n) {
    if (k >= a.K || n >= a.N) return 0.0f;
    const size_t e = (size_t)k * a.N + n;
    if constexpr (FMT == TML_FMT_F32) {
        return ((const float *)a.B)[e];
    } else if constexpr (FMT == TML_FMT_Q8_0) {
        return (float)((const int8_t *)a.B)[e];
    } else if constexpr (FMT == TML_FMT_Q8_K) {
        return (float)((const int8_t *)a.B)[e] * a.scales[e / a.block];
    } else {
        const uint32_t byte = ((const uint8_t *)a.B)[e / 2];
        return sext4(byte, (int)(e & 1));
    }
}

// Dequantize a raw chunk into EPC floats.
template <int FMT>
__device__ __forceinline__ void decode_b(const BRaw &r, float *out) {
    if constexpr (FMT == TML_FMT_F32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(r.w[i]);
    } else if constexpr (FMT == TML_FMT_Q8_0) {
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = sext8(r.w[i / 4], i % 4);
    } else if constexpr (FMT == TML_FMT_Q8_K) {
        // Reference dequantization: f32(q) * scale, rounded per element
        // (quantization.zig:598-600).
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = sext8(r.w[i / 4], i % 4) * r.s;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = sext4(r.w[0], i);
    }
}

// ---------------------------------------------------------------- kernel
template <int FMT, int BM, int BN, int BK, int WM, int WN, bool VEC>
__global__ __launch_bounds__(kThreads) void gemm_mfma_kernel(GemmKArgs a) {
    constexpr int WAVES_N = BN / WN;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int EPC = BFmt<FMT>::EPC;
    static_assert((BM / WM) * (BN / WN) == 4, "4 waves per workgroup");
    static_assert(BK % 16 == 0 && WM % 16 == 0 && WN % 16 == 0, "MFMA granularity");
    // A slice: float4 chunks; B slice: EPC-element chunks.
    constexpr int A_CHUNKS = BM * BK / 4;
    constexpr int B_CHUNKS = BK * BN / EPC;
    constexpr int A_PER = (A_CHUNKS + kThreads - 1) / kThreads;
    constexpr int B_PER = (B_CHUNKS + kThreads - 1) / kThreads;
    constexpr int LDA = BK + 4;
    constexpr int LDB = BN + 4;

    __shared__ __attribute__((aligned(16))) float As[2][BM * LDA];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDB];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm0 = (wave / WAVES_N) * WM;
    const int wn0 = (wave % WAVES_N) * WN;

    // XCD-aware remap of the workgroup id, then GROUP_M swizzle.
    const int nblk = gridDim.x;
    const int b = blockIdx.x;
    const int per = nblk / kNumXcd, rem = nblk % kNumXcd;
    const int xcd = b % kNumXcd, idx = b / kNumXcd;
    const int lin = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int group = a.group_m * a.tiles_n;
    const int first_m = (lin / group) * a.group_m;
    const int gsize = min(a.tiles_m - first_m, a.group_m);
    const int tile_m = first_m + (lin % group) % gsize;
    const int tile_n = (lin % group) / gsize;
    const int m0 = tile_m * BM;
    const int n0 = tile_n * BN;

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};

    // Staging registers for the next slice.
    float4 ra[A_PER];
    BRaw rb[B_PER];
    float rbe[VEC ? 1 : B_PER * EPC];  // generic path: already-decoded B

    auto load_slice = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * kThreads;
            if (A_CHUNKS % kThreads == 0 || c < A_CHUNKS) {
                const int row = c / (BK / 4), kq = (c % (BK / 4)) * 4;
                const int gm = m0 + row, gk = k0 + kq;
                if constexpr (VEC) {
                    ra[i] = (gm < a.M && gk < a.K) ? *(const float4 *)(a.A + (size_t)gm * a.K + gk)
                                                   : make_float4(0.f, 0.f, 0.f, 0.f);
                } else {
                    float t[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        t[q] = (gm < a.M && gk + q < a.K) ? a.A[(size_t)gm * a.K + gk + q] : 0.0f;
                    ra[i] = make_float4(t[0], t[1], t[2], t[3]);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * kThreads;
            if (B_CHUNKS % kThreads == 0 || c < B_CHUNKS) {
                const int kr = c / (BN / EPC), nc = (c % (BN / EPC)) * EPC;
                if constexpr (VEC) {
                    load_b_vec<FMT>(a, k0 + kr, n0 + nc, rb[i]);
                } else {
#pragma unroll
                    for (int q = 0; q < EPC; ++q) rbe[i * EPC + q] = load_b_elem<FMT>(a, k0 + kr, n0 + nc + q);
                }
            }
        }
    };

    auto store_slice = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * kThreads;
            if (A_CHUNKS % kThreads == 0 || c < A_CHUNKS) {
                const int row = c / (BK / 4), kq = (c % (BK / 4)) * 4;
                *(float4 *)&As[buf][row * LDA + kq] = ra[i];
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * kThreads;
            if (B_CHUNKS % kThreads == 0 || c < B_CHUNKS) {
                const int kr = c / (BN / EPC), nc = (c % (BN / EPC)) * EPC;
                float v[EPC];
                if constexpr (VEC) {
                    decode_b<FMT>(rb[i], v);
                } else {
#pragma unroll
                    for (int q = 0; q < EPC; ++q) v[q] = rbe[i * EPC + q];
                }
#pragma unroll
                for (int q = 0; q < EPC; q += 4)
                    *(float4 *)&Bs[buf][kr * LDB + nc + q] = make_float4(v[q], v[q + 1], v[q + 2], v[q + 3]);
            }
        }
    };

    const int nk = (a.K + BK - 1) / BK;
    load_slice(0);
    store_slice(0);
    __syncthreads();

    const int lrow = lane & 15;
    const int lk = (lane >> 4) * 4;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load_slice((kt + 1) * BK);
        const float *as = As[cur];
        const float *bs = Bs[cur];
#pragma unroll
        for (int kc = 0; kc < BK; kc += 16) {
            float4 av[TM];
            float bv[TN][4];
#pragma unroll
            for (int i = 0; i < TM; ++i) av[i] = *(const float4 *)&as[(wm0 + i * 16 + lrow) * LDA + kc + lk];
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int s = 0; s < 4; ++s) bv[j][s] = bs[(kc + lk + s) * LDB + wn0 + j * 16 + lrow];
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int i = 0; i < TM; ++i) {
                    const float as_ = s == 0 ? av[i].x : s == 1 ? av[i].y : s == 2 ? av[i].z : av[i].w;
#pragma unroll
                    for (int j = 0; j < TN; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(as_, bv[j][s], acc[i][j], 0, 0, 0);
                }
        }
        if (kt + 1 < nk) store_slice(cur ^ 1);
        __syncthreads();
    }

    // Epilogue: C = alpha * acc + beta * C + bias, bounds-checked.
    const int rq = (lane >> 4) * 4;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn0 + j * 16 + lrow;
            if (col >= a.N) continue;
            const float bcol = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm0 + i * 16 + rq + r;
                if (row < a.M) {
                    float *cp = a.C + (size_t)row * a.N + col;
                    float v = a.alpha * acc[i][j][r];
                    if (a.beta != 0.0f) v += a.beta * *cp;
                    if (a.bias) v += bcol;
                    *cp = v;
                }
            }
        }
}

// ---------------------------------------------------------------- configs
struct TileCfg {
    int bm, bn;
    float eff;  // relative per-tile efficiency used by the picker
};
// Index = config id used by TML_GEMM_TILE (1-based there).
constexpr TileCfg kCfgs[] = {
    {128, 128, 1.00f},
    {128, 64, 0.92f},
    {64, 128, 0.92f},
    {64, 64, 0.85f},
    {32, 64, 0.60f},
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <int FMT, bool VEC>
Status launch_cfg(int cfg, const GemmKArgs &ka, hipStream_t s) {
    dim3 block(kThreads);
    auto grid_of = [&](int bm, int bn) { return dim3((unsigned)(((ka.M + bm - 1) / bm) * ((ka.N + bn - 1) / bn))); };
    if constexpr (!VEC) {
        // The generic (unaligned) path is instantiated for one tile shape.
        gemm_mfma_kernel<FMT, 64, 64, 32, 32, 32, false><<<grid_of(64, 64), block, 0, s>>>(ka);
    } else {
        switch (cfg) {
        case 0: gemm_mfma_kernel<FMT, 128, 128, 16, 64, 64, VEC><<<grid_of(128, 128), block, 0, s>>>(ka); break;
        case 1: gemm_mfma_kernel<FMT, 128, 64, 16, 64, 32, VEC><<<grid_of(128, 64), block, 0, s>>>(ka); break;
        case 2: gemm_mfma_kernel<FMT, 64, 128, 16, 32, 64, VEC><<<grid_of(64, 128), block, 0, s>>>(ka); break;
        case 3: gemm_mfma_kernel<FMT, 64, 64, 32, 32, 32, VEC><<<grid_of(64, 64), block, 0, s>>>(ka); break;
        case 4: gemm_mfma_kernel<FMT, 32, 64, 32, 16, 32, VEC><<<grid_of(32, 64), block, 0, s>>>(ka); break;
        default: return Status::Err(TML_ERR_INVALID_ARG, "bad GEMM tile config");
        }
    }
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

// Pick the tile config with the smallest estimated time: full "rounds" of
// workgroups over the CUs times per-tile work over per-tile efficiency.
int pick_cfg(int64_t M, int64_t N, int cus) {
    int best = 0;
    double best_t = 1e300;
    for (int c = 0; c < kNumCfgs; ++c) {
        const int64_t tiles = ((M + kCfgs[c].bm - 1) / kCfgs[c].bm) * ((N + kCfgs[c].bn - 1) / kCfgs[c].bn);
        const int64_t rounds = (tiles + cus - 1) / cus;
        const double t = (double)rounds * kCfgs[c].bm * kCfgs[c].bn / kCfgs[c].eff;
        if (t < best_t) {
            best_t = t;
            best = c;
        }
    }
    return best;
}

bool aligned(const void *p, size_t n) { return ((uintptr_t)p % n) == 0; }

template <int FMT>
Status launch_fmt(const MatmulArgs &m, hipStream_t s, int cus) {
    GemmKArgs ka;
    ka.M = (int)m.M; ka.N = (int)m.N; ka.K = (int)m.K;
    ka.A = m.A; ka.B = m.B; ka.scales = m.scales; ka.block = m.block;
    ka.bias = m.bias; ka.C = m.C; ka.alpha = m.alpha_eff; ka.beta = m.beta;
    int cfg = env_int("TML_GEMM_TILE", 0) - 1;
    if (cfg < 0 || cfg >= kNumCfgs) cfg = pick_cfg(m.M, m.N, cus);
    constexpr int EPC = BFmt<FMT>::EPC;
    const size_t bbytes = FMT == TML_FMT_F32 ? 16 : (FMT == TML_FMT_Q4_0 ? 4 : 8);
    bool vec = (m.K % 4 == 0) && aligned(m.A, 16) && (m.N % EPC == 0) && aligned(m.B, bbytes);
    if (FMT == TML_FMT_Q8_K) vec = vec && (m.block % 8 == 0);
    if (!vec) cfg = 3;  // the generic path is instantiated for one tile shape
    const int bm = kCfgs[cfg].bm, bn = kCfgs[cfg].bn;
    ka.tiles_m = (int)((m.M + bm - 1) / bm);
    ka.tiles_n = (int)((m.N + bn - 1) / bn);
    ka.group_m = 4;
    return vec ? launch_cfg<FMT, true>(cfg, ka, s) : launch_cfg<FMT, false>(3, ka, s);
}

}  // namespace

Status launch_gemm_mfma(const MatmulArgs &m, hipStream_t s) {
    // Index math in the kernel is 32-bit for dimensions and 64-bit for
    // element offsets; grids are 1-D.
    const int64_t lim = (int64_t)1 << 30;
    if (m.M >= lim || m.N >= lim || m.K >= lim)
        return Status::Err(TML_ERR_INVALID_SHAPE, "GEMM dimension exceeds 2^30");
    static int cus = 0;
    if (cus == 0) {
        int dev = 0;
        TML_HIP_TRY(hipGetDevice(&dev));
        TML_HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
    }
    switch (m.fmt) {
        case TML_FMT_F32: return launch_fmt<TML_FMT_F32>(m, s, cus);
        case TML_FMT_Q8_0: return launch_fmt<TML_FMT_Q8_0>(m, s, cus);
        case TML_FMT_Q8_K: return launch_fmt<TML_FMT_Q8_K>(m, s, cus);
        case TML_FMT_Q4_0: return launch_fmt<TML_FMT_Q4_0>(m, s, cus);
        default: return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    }
}

}  // namespace tml
