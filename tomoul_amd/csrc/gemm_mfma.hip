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
#include <cstdlib>

#include "tml_internal.hpp"

namespace tml {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx2 __attribute__((ext_vector_type(2)));

constexpr int kNumXcd = 8;

struct GemmKArgs {
    int M, N, K;
    const float *A;
    const void *B;
    const float *scales;
    long long block;
    const float *bias;
    const float *colscale;  // [N] per-column factor on A.B, or nullptr
    float *C;
    float alpha;
    float beta;
    int tiles_m, tiles_n, group_m;
    int xcd_remap;
    const void *zero;
    int act;             // TML_ACT_* after the bias
    const float *res;    // [M,N] residual added after the bias, or nullptr
    long long tail0;     // tml_act_tail0(M * N)
    unsigned a_bytes = 0, b_bytes = 0;  // M*K*4 and the bytes of B: buffer-resource sizes (vector path)
};

// Vector-path loads go through buffer resources: the base and byte count
// are uniform (SGPRs), the lane's byte offset is one 32-bit VGPR, and
// offsets at or past the byte count read zeros.  This replaces a 64-bit
// address and a zero-block select per load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *base, unsigned nbytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)nbytes, 0x00020000);
}
__device__ __forceinline__ uintx4 buf_load_b128(const void *base, unsigned nbytes, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b128(buf_rsrc(base, nbytes), off, 0, 0);
}
__device__ __forceinline__ uintx2 buf_load_b64(const void *base, unsigned nbytes, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b64(buf_rsrc(base, nbytes), off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load_b32(const void *base, unsigned nbytes, unsigned off) {
    return __builtin_amdgcn_raw_buffer_load_b32(buf_rsrc(base, nbytes), off, 0, 0);
}
constexpr unsigned kBufOutOfRange = 0x80000000u;

// ---------------------------------------------------------------- B formats
// Elements of B moved per global load ("chunk") in the vector path.
template <int FMT> struct BFmt;
template <> struct BFmt<TML_FMT_F32> { static constexpr int EPC = 4; };
template <> struct BFmt<TML_FMT_Q8_0> { static constexpr int EPC = 8; };
template <> struct BFmt<TML_FMT_Q8_K> { static constexpr int EPC = 8; };
template <> struct BFmt<TML_FMT_Q4_0> { static constexpr int EPC = 8; };
template <> struct BFmt<TML_FMT_F16> { static constexpr int EPC = 8; };

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

// Vector-path chunk load at (k, n); n % EPC == 0.  Branch-free, so the
// compiler keeps every load of a slice in flight together.  Through the
// buffer resource (all formats but Q8_K): k >= K lies past the end of B and
// reads zeros; a chunk at n >= N reads bytes of the next k-row, which only
// feed output columns the epilogue drops.  Q8_K (whose block-scale lookup
// must stay inside the scales) selects the zero block instead.
template <int FMT>
__device__ __forceinline__ void load_b_vec(const GemmKArgs &a, int k, int n, BRaw &r) {
    if constexpr (FMT != TML_FMT_Q8_K) {
        const unsigned e = (unsigned)k * (unsigned)a.N + (unsigned)n;  // element index
        if constexpr (FMT == TML_FMT_F32 || FMT == TML_FMT_F16) {
            const uintx4 v = buf_load_b128(a.B, a.b_bytes, e * (FMT == TML_FMT_F32 ? 4u : 2u));
            r.w[0] = v[0]; r.w[1] = v[1]; r.w[2] = v[2]; r.w[3] = v[3];
        } else if constexpr (FMT == TML_FMT_Q8_0) {
            const uintx2 v = buf_load_b64(a.B, a.b_bytes, e);
            r.w[0] = v[0]; r.w[1] = v[1];
        } else {  // Q4_0: 8 nibbles = 4 bytes starting at byte e/2 (e % 8 == 0)
            r.w[0] = buf_load_b32(a.B, a.b_bytes, e / 2);
        }
        return;
    }
    const bool in = (k < a.K) && (n < a.N);
    const size_t e = (size_t)(in ? k : 0) * a.N + (in ? n : 0);
    if constexpr (FMT == TML_FMT_F32 || FMT == TML_FMT_F16) {
        const void *p = FMT == TML_FMT_F32 ? (const void *)((const float *)a.B + e)
                                           : (const void *)((const uint16_t *)a.B + e);
        const uintx4 v = *(const uintx4 *)(in ? p : a.zero);
        r.w[0] = v[0]; r.w[1] = v[1]; r.w[2] = v[2]; r.w[3] = v[3];
    } else if constexpr (FMT == TML_FMT_Q8_0 || FMT == TML_FMT_Q8_K) {
        const uintx2 v = *(const uintx2 *)(in ? (const void *)((const int8_t *)a.B + e) : a.zero);
        r.w[0] = v[0]; r.w[1] = v[1];
        if constexpr (FMT == TML_FMT_Q8_K) r.s = a.scales[e / a.block];
    } else {  // Q4_0: 8 nibbles = 4 bytes starting at byte e/2 (e % 8 == 0)
        r.w[0] = *(const uint32_t *)(in ? (const void *)((const uint8_t *)a.B + e / 2) : a.zero);
    }
}

// Generic-path chunk: element-wise with bounds, any alignment.
template <int FMT>
__device__ __forceinline__ float load_b_elem(const GemmKArgs &a, int k, int n) {
    if (k >= a.K || n >= a.N) return 0.0f;
    const size_t e = (size_t)k * a.N + n;
    if constexpr (FMT == TML_FMT_F32) {
        return ((const float *)a.B)[e];
    } else if constexpr (FMT == TML_FMT_F16) {
        return tml_half_bits(((const uint16_t *)a.B)[e]);
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
    } else if constexpr (FMT == TML_FMT_F16) {
#pragma unroll
        for (int i = 0; i < 8; ++i) out[i] = tml_half_bits(r.w[i / 2] >> (16 * (i % 2)));
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
template <int FMT, int BM, int BN, int BK, int WM, int WN, int NW, bool VEC>
__global__ __launch_bounds__(NW * 64) void gemm_mfma_kernel(GemmKArgs a) {
    constexpr int kThreads = NW * 64;
    constexpr int WAVES_N = BN / WN;
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int NC = BK / 16;  // 16-deep MFMA chunks per slice
    constexpr int EPC = BFmt<FMT>::EPC;
    static_assert((BM / WM) * (BN / WN) == NW, "one wave per WM x WN sub-tile");
    static_assert(WM % 16 == 0 && WN % 16 == 0, "MFMA granularity");
    static_assert(NC % 2 == 0, "the pipeline below assumes an even number of chunks per slice");
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
    const int lin = !a.xcd_remap ? b
                  : (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
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

    // ---- global -> registers -> LDS staging of one BK slice
    struct Stage {
        floatx4 a[A_PER];
        BRaw b[VEC ? B_PER : 1];
        float be[VEC ? 1 : B_PER * EPC];  // generic path: already decoded
    };
    auto load_slice = [&](Stage &st, int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * kThreads;
            if (A_CHUNKS % kThreads == 0 || c < A_CHUNKS) {
                const int row = c / (BK / 4), kq = (c % (BK / 4)) * 4;
                const int gm = m0 + row, gk = k0 + kq;
                if constexpr (VEC) {
                    // rows >= M lie past the end of A; k >= K inside a row
                    // would read the next row, so it points past the end too
                    const unsigned off = gk < a.K ? ((unsigned)gm * (unsigned)a.K + (unsigned)gk) * 4u : kBufOutOfRange;
                    st.a[i] = __builtin_bit_cast(floatx4, buf_load_b128(a.A, a.a_bytes, off));
                } else {
                    float t[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q)
                        t[q] = (gm < a.M && gk + q < a.K) ? a.A[(size_t)gm * a.K + gk + q] : 0.0f;
                    st.a[i] = floatx4{t[0], t[1], t[2], t[3]};
                }
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * kThreads;
            if (B_CHUNKS % kThreads == 0 || c < B_CHUNKS) {
                const int kr = c / (BN / EPC), nc = (c % (BN / EPC)) * EPC;
                if constexpr (VEC) {
                    load_b_vec<FMT>(a, k0 + kr, n0 + nc, st.b[i]);
                } else {
#pragma unroll
                    for (int q = 0; q < EPC; ++q) st.be[i * EPC + q] = load_b_elem<FMT>(a, k0 + kr, n0 + nc + q);
                }
            }
        }
    };
    auto store_slice = [&](const Stage &st, int buf) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * kThreads;
            if (A_CHUNKS % kThreads == 0 || c < A_CHUNKS) {
                const int row = c / (BK / 4), kq = (c % (BK / 4)) * 4;
                *(floatx4 *)&As[buf][row * LDA + kq] = st.a[i];
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * kThreads;
            if (B_CHUNKS % kThreads == 0 || c < B_CHUNKS) {
                const int kr = c / (BN / EPC), nc = (c % (BN / EPC)) * EPC;
                float v[EPC];
                if constexpr (VEC) {
                    decode_b<FMT>(st.b[i], v);
                } else {
#pragma unroll
                    for (int q = 0; q < EPC; ++q) v[q] = st.be[i * EPC + q];
                }
#pragma unroll
                for (int q = 0; q < EPC; q += 4)
                    *(floatx4 *)&Bs[buf][kr * LDB + nc + q] = floatx4{v[q], v[q + 1], v[q + 2], v[q + 3]};
            }
        }
    };

    // ---- LDS -> register fragments of one 16-deep chunk, and its MFMAs
    struct Frag {
        floatx4 a[TM];
        float b[TN][4];
    };
    const int lrow = lane & 15;
    const int lk = (lane >> 4) * 4;
    auto read_frag = [&](Frag &f, int buf, int chunk) __attribute__((always_inline)) {
        const float *as = As[buf];
        const float *bs = Bs[buf];
        const int kc = chunk * 16;
#pragma unroll
        for (int i = 0; i < TM; ++i) f.a[i] = *(const floatx4 *)&as[(wm0 + i * 16 + lrow) * LDA + kc + lk];
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s) f.b[j][s] = bs[(kc + lk + s) * LDB + wn0 + j * 16 + lrow];
    };
    auto mma = [&](const Frag &f) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const float av = f.a[i][s];
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, f.b[j][s], acc[i][j], 0, 0, 0);
            }
    };

    // ---- pipeline
    // Global loads run two slices ahead of the MFMAs (two register stages),
    // LDS holds two slices, and fragment reads run one chunk ahead; the last
    // chunk's MFMAs of a slice are issued after the barrier so that they
    // cover the first fragment reads of the next slice.
    // Every step below is unconditional (a slice index past the end is
    // clamped to the last slice and its loads/stores are harmless repeats),
    // so the loop body is straight-line code with uniform branches only.
    const int nk = (a.K + BK - 1) / BK;
    if (nk > 0) {
        Stage s0, s1;
        Frag f[2];
        load_slice(s0, 0);
        store_slice(s0, 0);
        load_slice(s1, min(1, nk - 1) * BK);
        __syncthreads();
        read_frag(f[0], 0, 0);

        // sched_barrier(0) fences keep the compiler from sinking the next
        // chunk's LDS reads down to their first use: every read of chunk c+1
        // is issued before the MFMAs of chunk c, so its latency is covered.
        auto step = [&](int kt, Stage &sl, const Stage &ss, int cur) __attribute__((always_inline)) {
            load_slice(sl, min(kt + 2, nk - 1) * BK);  // sl's slice kt is already in LDS
#pragma unroll
            for (int c = 0; c + 1 < NC; ++c) {
                read_frag(f[(c + 1) & 1], cur, c + 1);
                __builtin_amdgcn_sched_barrier(0);
                mma(f[c & 1]);
                __builtin_amdgcn_sched_barrier(0);
            }
            store_slice(ss, cur ^ 1);  // slice kt + 1
            __syncthreads();
            read_frag(f[0], cur ^ 1, 0);
            __builtin_amdgcn_sched_barrier(0);
            mma(f[1]);
            __builtin_amdgcn_sched_barrier(0);
        };
        int kt = 0;
        for (; kt + 1 < nk; kt += 2) {
            step(kt, s0, s1, 0);
            step(kt + 1, s1, s0, 1);
        }
        if (kt < nk) step(kt, s0, s1, 0);
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
            const float acol = a.colscale ? a.alpha * a.colscale[col] : a.alpha;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm0 + i * 16 + rq + r;
                if (row < a.M) {
                    float *cp = a.C + (size_t)row * a.N + col;
                    float v = acol * acc[i][j][r];
                    if (a.beta != 0.0f) v += a.beta * *cp;
                    if (a.bias) v += bcol;
                    const long long flat = (long long)row * a.N + col;
                    if (a.res) v += a.res[flat];
                    tml_store_c(cp, tml_apply_act(v, a.act, flat, a.tail0));
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
    {256, 128, 1.00f},
    {128, 128, 0.80f},
    {128, 128, 0.0f},  // experiments only (eff 0: never picked)
    {128, 64, 0.0f},
    {64, 64, 0.0f},
};
constexpr int kNumCfgs = sizeof(kCfgs) / sizeof(kCfgs[0]);

template <int FMT, bool VEC>
Status launch_cfg(int cfg, const GemmKArgs &ka, hipStream_t s) {
    auto grid_of = [&](int bm, int bn) { return dim3((unsigned)(((ka.M + bm - 1) / bm) * ((ka.N + bn - 1) / bn))); };
    if constexpr (!VEC) {
        // The generic (unaligned) path is instantiated for one tile shape.
        gemm_mfma_kernel<FMT, 64, 64, 32, 32, 32, 4, false><<<grid_of(64, 64), 256, 0, s>>>(ka);
    } else {
        switch (cfg) {
        case 0: gemm_mfma_kernel<FMT, 128, 128, 32, 64, 32, 8, VEC><<<grid_of(128, 128), 512, 0, s>>>(ka); break;
        case 1: gemm_mfma_kernel<FMT, 128, 64, 32, 32, 32, 8, VEC><<<grid_of(128, 64), 512, 0, s>>>(ka); break;
        case 2: gemm_mfma_kernel<FMT, 64, 128, 32, 32, 32, 8, VEC><<<grid_of(64, 128), 512, 0, s>>>(ka); break;
        case 3: gemm_mfma_kernel<FMT, 64, 64, 32, 32, 32, 4, VEC><<<grid_of(64, 64), 256, 0, s>>>(ka); break;
        case 4: gemm_mfma_kernel<FMT, 32, 64, 32, 16, 32, 4, VEC><<<grid_of(32, 64), 256, 0, s>>>(ka); break;
        case 5: gemm_mfma_kernel<FMT, 256, 128, 32, 64, 64, 8, VEC><<<grid_of(256, 128), 512, 0, s>>>(ka); break;
        case 6: gemm_mfma_kernel<FMT, 128, 128, 32, 64, 64, 4, VEC><<<grid_of(128, 128), 256, 0, s>>>(ka); break;
        case 7: gemm_mfma_kernel<FMT, 128, 128, 64, 64, 32, 8, VEC><<<grid_of(128, 128), 512, 0, s>>>(ka); break;
        case 8: gemm_mfma_kernel<FMT, 128, 64, 64, 32, 32, 8, VEC><<<grid_of(128, 64), 512, 0, s>>>(ka); break;
        case 9: gemm_mfma_kernel<FMT, 64, 64, 64, 32, 32, 4, VEC><<<grid_of(64, 64), 256, 0, s>>>(ka); break;
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
        if (kCfgs[c].eff <= 0.0f) continue;
        const double t = (double)rounds * kCfgs[c].bm * kCfgs[c].bn / kCfgs[c].eff;
        if (t < best_t) {
            best_t = t;
            best = c;
        }
    }
    return best;
}

int device_cus() {
    static int cus = 0;
    if (cus == 0) {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) == hipSuccess &&
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0)
            cus = n;
        else
            cus = 256;
    }
    return cus;
}

// Direct-copy fp32 kernel: pick (tile, K splits) with the smallest modelled
// time.  A CU runs its share of the units (tile x split); with one unit per
// CU a slice costs t_one, with several resident at once their slices overlap
// and each costs t_many.  So
//   t = ceil(units / CUs) * slices_per_split * (BK / 32) * t_slice(tile, one / many)
//       + t_fill + (splits > 1 ? t_reduce : 0)
// with t_fill (pipeline fill, epilogue, launch) ~3.5 us and t_reduce (the
// second launch that sums the splits' partials) ~3.6 us plus the partials'
// traffic, splits * M * N * 8 bytes at ~6 TB/s.  The per 32-deep slice costs
// (us, one / several per CU) were fitted on MI355X to a sweep of every tile
// x split (1, 2, 4 over twelve shapes -- the XLM-R layer, the Whisper
// large-v3-turbo and tiny encoder linears, the sentence-transformer
// linears, 128x4096x1024 -- and 3, 6, 8 over the six that split) so that
// the model's pick is the measured best on eleven of them and 0.4 us off on
// the twelfth: 128x128 1.975 / 1.998, 128x64 0.974 / 0.854, 64x64 0.528 /
// 0.504, 256x128 4.05 (not refitted: it spills), 128x64 (BK 64) 1.06 /
// 1.147, 64x64 (BK 64) 0.54 / 0.672, 32x64 0.308 / 0.24, 32x64 (BK 64)
// 0.308 / 0.293, 96x32 0.354 / 0.383 (no int4 variant), 32x64 (BK 64, two
// wave groups along K) 0.226 / 0.282, and 32x32 (BK 64, two wave groups, no
// int4 variant) 0.165 / 0.155 -- fitted later, on ten shapes with few 32x64
// tiles (512x384x384 7.38 -> 5.44 us, 512x1536x384 11.10 -> 9.62,
// 512x384x1536 13.17 -> 11.37, 256x1024x1024 13.81 -> 9.49; F16 0.21 / 0.19:
// 512x384x384 7.74 -> 6.07, 512x1536x384 12.08 -> 10.68), where twice the
// tiles fill the CUs; where a 32x64 tile a CU or the large tiles already do
// (512x1024x1024, 1500x1536x384) it stays unpicked, as measured.  Its Q8_K
// entries, 0.272 / 0.226 (the F16 ones scaled as the 32x64 two-group tile's
// are), agree with Q8_K's own times (512x384x384 6.98 us, 0.29 a slice;
// 512x384x1536 16.54, 0.27; 512x1536x384 12.11, 0.24 with three a CU; the
// next-best plans 8.86 / 16.34 / 13.69).  F16 and Q8_K widen B (and Q8_K
// multiplies its block scales) at every fragment read, which costs each
// tile differently, so they have tables of their own: the medians of a
// sweep of every tile x split (1, 2) over eleven shapes (the
// sentence-transformer linears, 384-1500 x 3840-4096 x 768-1280, 128x4096x1024,
// 2048x768x3072, 1024x4096x1024), 128x128 with one unit a CU taken from
// its worst case; with them the planner considers K splits of 1 and 2
// only.  Against the f32 table's picks (us, F16 / Q8_K):
// 512x4096x768 34.39 / 40.17 -> 32.82 / 37.56, 384x4096x1024 34.93 / 41.19
// -> 33.23 / 37.17, 512x3072x768 Q8_K 32.54 -> 30.85, 1500x3840x1280
// 134.1 / 150.2 -> 130.7 / 142.6.  Q4_0 and Q8_0 keep the f32 table.
void pick_dma(int64_t M, int64_t N, int64_t K, int fmt, GemmPlan *p) {
    static const double f32_one[] = {1.975, 0.974, 0.528, 4.05, 1.06, 0.54, 0.308, 0.308, 0.354, 0.226, 0.165};
    static const double f32_many[] = {1.998, 0.854, 0.504, 4.05, 1.147, 0.672, 0.24, 0.293, 0.383, 0.282, 0.155};
    static const double f16_one[] = {2.40, 1.276, 0.680, 4.66, 1.162, 0.690, 0.418, 0.396, 0.556, 0.359, 0.21};
    static const double f16_many[] = {2.123, 1.152, 0.574, 4.66, 1.180, 0.592, 0.304, 0.318, 0.435, 0.318, 0.19};
    static const double q8k_one[] = {2.70, 1.466, 0.861, 5.06, 1.358, 0.799, 0.571, 0.489, 0.687, 0.465, 0.272};
    static const double q8k_many[] = {2.389, 1.291, 0.659, 5.06, 1.370, 0.666, 0.369, 0.355, 0.477, 0.379, 0.226};
    static_assert(sizeof(f32_one) == sizeof(f32_many) && sizeof(f16_one) == sizeof(f32_one) &&
                      sizeof(f16_many) == sizeof(f32_one) && sizeof(q8k_one) == sizeof(f32_one) &&
                      sizeof(q8k_many) == sizeof(f32_one),
                  "one cost pair per tile config");
    const bool narrow_table = fmt == TML_FMT_F16 || fmt == TML_FMT_Q8_K;
    const double *const t_one = fmt == TML_FMT_F16 ? f16_one : fmt == TML_FMT_Q8_K ? q8k_one : f32_one;
    const double *const t_many = fmt == TML_FMT_F16 ? f16_many : fmt == TML_FMT_Q8_K ? q8k_many : f32_many;
    static const int splits[] = {1, 2, 3, 4, 6, 8};
    constexpr double kFill = 3.5, kReduce = 3.6, kBytesPerUs = 6.0e6;
    // Below 128 rows (f32): the 32-row tiles run alone on their CUs, a slice
    // costs 0.25 us (32x64, BK 32 or 64) or 0.20 (32x64 two groups), the
    // 64-deep tiles fill 0.75 us longer, and the reduce launch costs 1.5 us
    // plus its traffic -- fitted to a sweep of the three 32x64 tiles x K
    // split 1-4 over M = 16, 32, 64, 96 and eight N x K (4096 x 1024 to 384 x
    // 1536); there the planner takes those three tiles only, with >= 3 slices
    // a split.  Measured with the rule on the sweep's 32 shapes: 344.2 ->
    // 332.8 us in sum, against 332.2 for the best measured plan of each (32
    // x 3072 x 768 10.89 -> 8.42, 64 x 4096 x 1024 13.46 -> 11.69 us; 16 x
    // 3840 x 1280 and 96 x 1024 x 4096 lost 0.5 / 0.6 us).  The two-group
    // 32x32 tile, added later, costs 0.09 us a slice there, with K split at
    // most 4 ways (the splits it was measured at): on the same 32 shapes
    // 334.5 -> 312.9 us in sum (16 x 4096 x 1024 10.35 -> 9.11, 64 x 3072 x
    // 768 9.61 -> 7.66, 96 x 1536 x 384 7.68 -> 5.57; 32 x 3840 x 1280 lost
    // 1.5 us, 96 x 1024 x 1024 0.3).
    const bool small = M < 128 && fmt == TML_FMT_F32;
    static const double small_one[] = {0.0, 0.0, 0.0, 0.0, 0.0, 0.0, 0.25, 0.25, 0.0, 0.20, 0.09};
    static const int small_max_split[] = {0, 0, 0, 0, 0, 0, 8, 8, 0, 8, 4};
    static_assert(sizeof(small_one) == sizeof(f32_one), "one small-M entry per tile config");
    static_assert(sizeof(small_max_split) / sizeof(int) == sizeof(f32_one) / sizeof(double),
                  "one small-M split limit per tile config");
    const int cus = device_cus();
    int forced_tile = env_int("TML_GEMM_DMA_TILE", 0) - 1;
    if (!gemm_dma_cfg_ok(forced_tile, fmt)) forced_tile = -1;  // unset, or no kernel for this format
    const int forced_split = env_int("TML_GEMM_SPLIT", 0);
    double best_t = 1e300;
    for (int c = 0; c < gemm_dma_num_cfgs(); ++c) {
        if (c >= (int)(sizeof(f32_one) / sizeof(f32_one[0]))) break;  // no cost model for this config
        if ((forced_tile >= 0 && c != forced_tile) || !gemm_dma_cfg_ok(c, fmt)) continue;
        if (small && forced_tile < 0 && small_one[c] == 0.0) continue;  // the fitted 32-row tiles only
        int bm = 0, bn = 0, bk = 32;
        gemm_dma_tile(c, &bm, &bn, &bk);
        const int64_t nk = (K + bk - 1) / bk;
        const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
        for (int sp : splits) {
            if (forced_split > 0 && sp != forced_split) continue;
            if (sp > 1 && nk < (small && forced_split <= 0 ? 3 : 2) * sp) continue;
            if (small && forced_split <= 0 && sp > small_max_split[c]) continue;
            if (narrow_table && sp > 2 && forced_split <= 0) break;  // the narrow tables were fitted on s <= 2
            const int64_t spl = nk > 0 ? (nk + sp - 1) / sp : 1;
            const int64_t real = nk > 0 ? (nk + spl - 1) / spl : 1;
            const int64_t units = tiles * real;
            const int64_t per_cu = (units + cus - 1) / cus;
            const double red = real > 1 ? (small ? 1.5 : kReduce) + (double)real * M * N * 8.0 / kBytesPerUs : 0.0;
            const double one = small && small_one[c] > 0.0 ? small_one[c] : t_one[c];
            const double ts = per_cu > 1 ? t_many[c] : one;
            const double fill = kFill + (small && bk == 64 ? 0.75 : 0.0);
            const double t = (double)per_cu * (double)spl * (bk / 32.0) * ts + fill + red;
            if (t < best_t) {
                best_t = t;
                p->cfg = c;
                p->nsplit = (int)real;
                p->spl = (int)spl;
                p->tiles = (int)tiles;
            }
        }
    }
    if (best_t == 1e300) {
        // a forced split too deep for this K: run the forced (or first) tile unsplit
        const int c = forced_tile >= 0 ? forced_tile : 0;
        int bm = 0, bn = 0, bk = 32;
        gemm_dma_tile(c, &bm, &bn, &bk);
        const int64_t nk = (K + bk - 1) / bk;
        p->cfg = c;
        p->nsplit = 1;
        p->spl = (int)(nk > 0 ? nk : 1);
        p->tiles = (int)(((M + bm - 1) / bm) * ((N + bn - 1) / bn));
    }
    // Split partials are combined by splitk_reduce_kernel, launched after the
    // GEMM.  TML_GEMM_FUSED=1 combines them inside the GEMM instead (the last
    // split of a tile sums them); on MI355X that measured ~2 us slower per
    // headline step than the extra launch (the agent-scope round trip of the
    // last split costs more than a reduce kernel in a graph), so it is off.
    p->fused = p->nsplit > 1 && env_int("TML_GEMM_FUSED", 0) != 0 && gemm_dma_cfg_fusable(p->cfg);
}

bool aligned(const void *p, size_t n) { return ((uintptr_t)p % n) == 0; }

template <int FMT>
Status launch_fmt(const MatmulArgs &m, hipStream_t s, int cus) {
    GemmKArgs ka;
    ka.M = (int)m.M; ka.N = (int)m.N; ka.K = (int)m.K;
    ka.A = m.A; ka.B = m.B; ka.scales = m.scales; ka.block = m.block;
    ka.bias = m.bias; ka.C = m.C; ka.alpha = m.alpha_eff; ka.beta = m.beta;
    ka.act = m.act; ka.res = m.res; ka.colscale = m.colscale; ka.tail0 = tml_act_tail0((long long)m.M * m.N);
    ka.zero = m.zero;
    int cfg = env_int("TML_GEMM_TILE", 0) - 1;
    if (cfg < 0 || cfg >= kNumCfgs) cfg = pick_cfg(m.M, m.N, cus);
    constexpr int EPC = BFmt<FMT>::EPC;
    const size_t bbytes = (FMT == TML_FMT_F32 || FMT == TML_FMT_F16) ? 16 : (FMT == TML_FMT_Q4_0 ? 4 : 8);
    bool vec = (m.K % 4 == 0) && aligned(m.A, 16) && (m.N % EPC == 0) && aligned(m.B, bbytes);
    if (FMT == TML_FMT_Q8_K) vec = vec && (m.block % 8 == 0);
    // the vector path's buffer offsets stay below 2^31: rows up to M + 256
    // of A, k-rows up to K + 64 of B
    const uint64_t brow = (FMT == TML_FMT_F32) ? (uint64_t)m.N * 4 : (FMT == TML_FMT_F16) ? (uint64_t)m.N * 2
                        : (FMT == TML_FMT_Q4_0) ? (uint64_t)m.N / 2 : (uint64_t)m.N;
    const uint64_t lim = (uint64_t)1 << 31;
    vec = vec && (uint64_t)(m.M + 256) * (uint64_t)m.K * 4u < lim && (uint64_t)(m.K + 64) * brow < lim;
    ka.a_bytes = (unsigned)((uint64_t)m.M * (uint64_t)m.K * 4u);
    ka.b_bytes = (unsigned)((uint64_t)m.K * brow);
    if (!vec) cfg = 3;  // the generic path is instantiated for one tile shape
    const int bm = kCfgs[cfg].bm, bn = kCfgs[cfg].bn;
    ka.tiles_m = (int)((m.M + bm - 1) / bm);
    ka.tiles_n = (int)((m.N + bn - 1) / bn);
    ka.group_m = env_int("TML_GEMM_GROUPM", 4);
    if (ka.group_m < 1) ka.group_m = 1;
    ka.xcd_remap = env_int("TML_GEMM_XCD", 1);
    return vec ? launch_cfg<FMT, true>(cfg, ka, s) : launch_cfg<FMT, false>(3, ka, s);
}

}  // namespace

GemmPlan plan_gemm(const MatmulArgs &m) {
    GemmPlan p;
    // Q8_0 / Q4_0 (per-tensor or per-column scales) past the GEMV rows take
    // the bf16 matrix-core kernel whenever its layout conditions hold
    // (gemm_qbf.hip), unless TML_GEMM_QBF=0 or an override asks for a tile or
    // K split of the fp32-MFMA kernels below (tests of those kernels).
    auto set = [](const char *k) {
        const char *v = std::getenv(k);
        return v != nullptr && *v != '\0';
    };
    const bool fp32_forced = set("TML_GEMM_DMA_Q") || set("TML_GEMM_TILE") || set("TML_GEMM_DMA_TILE") ||
                             set("TML_GEMM_SPLIT");
    if (!fp32_forced && gemm_qbf_supported(m)) {
        p.qbf = true;
        pick_qbf(m, &p);
        return p;
    }
    // f32 B takes the direct-copy kernel whenever its rows allow it.  For
    // the narrow formats both kernels read B through buffer resources and
    // the direct-copy kernel reads two adjacent columns per LDS access;
    // measured on MI355X (us, register-staged / direct-copy):
    //   Q8_0 128x4096x1024 16.8 / 17.2, 512x4096x1024 41.4 / 46.0,
    //        1024x4096x1024 77.0 / 77.3, 1500x3840x1280 130.5 / 138.1;
    //   Q4_0 128x5120x1280 33.4 / 28.0, 512x5120x1280 73.1 / 76-79,
    //        1500x3840x1280 162.4 / 140.8;
    //   F16  512x4096x1024 41.5 / 43.2, 1500x3840x1280 143.3 / 132.2;
    //   Q8_K 1500x3840x1280 150.4 / 148.6.
    // So Q4_0 takes the direct-copy kernel from M = 1024 on and at M <= 128
    // (where the register-staged kernel widens each B element of a tile for
    // few rows of A); Q8_0 keeps the register-staged kernel.  F16 and Q8_K,
    // with their own tile costs in the direct-copy planner (pick_dma), take
    // the direct-copy kernel at every M, except Q8_K from M = 512 with
    // N >= 4096 (us, register-staged / direct-copy on the planner's pick, F16
    // | Q8_K): 512x1152x384 14.83 / 11.48 | 17.05 / 13.09, 512x3072x768
    // 33.74 / 28.08 | 34.78 / 30.85, 384x4096x1024 42.3 / 33.2 | 44.1 / 37.2,
    // 128x4096x1024 18.46 / 16.63 | 23.74 / 20.19, 1500x3840x1280 139.3 /
    // 130.7 | 154.7 / 142.6; 512x4096x1024 42.31 / 41.24 | 44.15 / 47.36,
    // 1024x4096x1024 76.03 / 74.37 | 80.51 / 84.76.  Every narrow format
    // also takes it whenever the register-staged
    // kernel's best tiling leaves most CUs idle (it has no K split): at
    // 256x768x3072 Q8_0 the direct-copy kernel with its split takes 23.1 us
    // against 45.1, at 512x384x1536 16.3 against 24.8, at 256x768x768 10.9
    // against 14.5 (96 register tiles each).  TML_GEMM_DMA_Q=1 / 0 forces it
    // on / off for the narrow formats; TML_GEMM_DMA=0 turns it off.
    const int dma_q = env_int("TML_GEMM_DMA_Q", -1);
    bool few_tiles = false;
    if (m.fmt != TML_FMT_F32) {
        const int cus = device_cus();
        const int c = pick_cfg(m.M, m.N, cus);
        const int64_t tiles = ((m.M + kCfgs[c].bm - 1) / kCfgs[c].bm) * ((m.N + kCfgs[c].bn - 1) / kCfgs[c].bn);
        few_tiles = tiles < cus / 2 || (tiles < cus && m.K >= 2048);
    }
    const bool by_m = m.fmt == TML_FMT_F16 || (m.fmt == TML_FMT_Q8_K && !(m.M >= 512 && m.N >= 4096)) ||
                      (m.fmt == TML_FMT_Q4_0 && (m.M >= 1024 || m.M <= 128));
    const bool narrow_ok = m.fmt == TML_FMT_F32 || dma_q == 1 || (dma_q < 0 && (by_m || few_tiles));
    if (narrow_ok && env_int("TML_GEMM_DMA", 1) != 0 && gemm_dma_supported(m) && m.K > 0) {
        p.dma = true;
        pick_dma(m.M, m.N, m.K, m.fmt, &p);
    }
    return p;
}

void gemm_workspace_need(const MatmulArgs &m, size_t *partial_floats, size_t *counters) {
    const GemmPlan p = plan_gemm(m);
    *partial_floats = 0;
    *counters = 0;
    if (p.qbf && p.nsplit > 1) *partial_floats = (size_t)p.nsplit * (size_t)m.M * (size_t)m.N;
    if (p.dma && p.nsplit > 1) gemm_dma_workspace_need(m, p, partial_floats, counters);
}

// The planner's overrides (experiments and tests: TML_GEMM_DMA_TILE,
// TML_GEMM_SPLIT, TML_GEMM_TILE, TML_GEMM_DMA_Q, TML_GEMM_DMA, TML_GEMM_FUSED,
// TML_GEMM_XCDPART, TML_GEMM_XCD, TML_GEMM_GROUPM) are honoured only up to
// the problem sizes the GPU tests run them at, M*N*K <= 512*1024*4096.  A
// calibration sweep that forced tile x split plans at the Whisper encoder
// shapes (M*N*K ~ 1e10) once ended in a GPU memory fault whose cause was not
// found in these kernels (their address arithmetic over that whole sweep is
// checked on the CPU, tests/test_cpu_emu.py), so forced plans above that size
// are refused rather than run untested.  Default plans are unaffected.
// (The CPU build of tests/cpu_emu raises the limit at compile time to check
// the kernels' addresses under every forced plan at full size.)
#ifndef TML_FORCED_PLAN_MAX_MNK
#define TML_FORCED_PLAN_MAX_MNK (512ull * 1024ull * 4096ull)
#endif
constexpr uint64_t kForcedPlanMaxMNK = TML_FORCED_PLAN_MAX_MNK;

bool plan_forced() {
    static const char *const keys[] = {"TML_GEMM_DMA_TILE", "TML_GEMM_SPLIT", "TML_GEMM_TILE",  "TML_GEMM_DMA_Q",
                                       "TML_GEMM_DMA",      "TML_GEMM_FUSED", "TML_GEMM_XCDPART", "TML_GEMM_XCD",
                                       "TML_GEMM_GROUPM",   "TML_GEMM_QBF_TILE", "TML_GEMM_QBF_SPLIT"};
    for (const char *k : keys) {
        const char *v = std::getenv(k);
        if (v != nullptr && *v != '\0') return true;
    }
    return false;
}

Status launch_gemm_mfma(const MatmulArgs &m, const Workspace &ws, hipStream_t s) {
    // Index math in the kernels is 32-bit for dimensions and 64-bit for
    // element offsets; grids are 1-D.
    const int64_t lim = (int64_t)1 << 30;
    if (m.M >= lim || m.N >= lim || m.K >= lim)
        return Status::Err(TML_ERR_INVALID_SHAPE, "GEMM dimension exceeds 2^30");
    if (plan_forced() && (uint64_t)m.M * (uint64_t)m.N * (uint64_t)m.K > kForcedPlanMaxMNK)
        return Status::Err(TML_ERR_INVALID_ARG,
                           "forced GEMM plans (TML_GEMM_* overrides) are refused above M*N*K = 512*1024*4096, "
                           "the largest size the tests run them at");
    const GemmPlan p = plan_gemm(m);
    // TML_REQUIRE_SPLIT=1 (tests): refuse a plan that does not split K
    if (!((p.qbf || p.dma) && p.nsplit > 1) && env_int("TML_REQUIRE_SPLIT", 0) == 1)
        return Status::Err(TML_ERR_INVALID_ARG, "TML_REQUIRE_SPLIT=1: this call's plan does not split K");
    if (p.qbf) return launch_gemm_qbf(m, p, ws, s);
    if (p.dma) return launch_gemm_f32_dma(m, p, ws, s);
    const int cus = device_cus();
    switch (m.fmt) {
        case TML_FMT_F32: return launch_fmt<TML_FMT_F32>(m, s, cus);
        case TML_FMT_Q8_0: return launch_fmt<TML_FMT_Q8_0>(m, s, cus);
        case TML_FMT_Q8_K: return launch_fmt<TML_FMT_Q8_K>(m, s, cus);
        case TML_FMT_Q4_0: return launch_fmt<TML_FMT_Q4_0>(m, s, cus);
        case TML_FMT_F16: return launch_fmt<TML_FMT_F16>(m, s, cus);
        default: return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    }
}

}  // namespace tml
