// gemv_tm.hip -- decoder GEMV on the matrix cores: M = 2..8 rows of fp32
// activations times a prepared (K-contiguous, see gemv_t.hip) Q8_0 / Q4_0
// weight.
//
//   C[M,N] = alpha * A[M,K] . q[K,N] + beta * C + bias[N]   (q: int8 / int4)
//
// The VALU kernels of gemv_t.hip spend M fused multiply-adds per weight
// element; at M = 4-8 that, and the activations each element needs, cost
// 1.7-2.7x the M = 1 time for 3-5 % more bytes.  Here the products run on
// v_mfma_f32_16x16x32_bf16 instead, with fp32 accumulation:
//   * weights: int8 and int4 values are exact in bf16 (int4 as 16 q, one
//     masked byte per nibble; the 1/16 goes into alpha, a power of two, so
//     exact as well);
//   * activations: each fp32 x is split into two bf16 terms, hi = bf16(x)
//     and lo = bf16(x - hi), round to nearest even both, so
//     |x - hi - lo| <= 2^-17 |x|; the product is (hi . q) + (lo . q), two
//     MFMAs accumulating in fp32.
// The result is the reference's dequantize-then-fp32-accumulate product
// (src/core/quantization.zig:158-314, :778-957) to ~1e-5 relative, inside
// the 1e-3 bar for quantized paths; the per-tensor scale is applied once in
// the epilogue as in every other kernel.
//
// Work split.  A workgroup of NW waves owns 16 output columns (the MFMA's N)
// and all of K, for all M rows or, where the column tiles leave CUs idle, for
// one row part (grid.y).  The MFMA's M is the activation row: rows past the
// part read zeros.
// The row of column n is a sequence of 16-byte chunks (16 int8 or 32 int4
// k); chunk ch goes to lane group g = slot % 4 of wave slot / 4, slot =
// ch % (4 NW).  Lane (c, g) of a wave loads chunk ch of column n0 + c (the
// B operand) and lane (m, g) the activations of row m at the same k (the A
// operand): element groups of four consecutive k, placed by the prepared
// layout's chunk interleave, so a wave's activation loads are contiguous
// runs.  Every load of a round (IT chunks per lane) is issued before any
// conversion.  The NW waves' 16x16 accumulators are added through LDS in
// wave order (deterministic) and wave 0 runs the epilogue.
#include "tml_internal.hpp"

#include <algorithm>

namespace tml {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));
typedef uint32_t uintx2 __attribute__((ext_vector_type(2)));

constexpr unsigned kOutOfRange = 0x80000000u;

struct GemvTmArgs {
    int M, N, K;
    const float *A;
    const uint8_t *Bt;
    long long ldt;          // bytes per prepared row (a multiple of 16)
    const float *bias;
    const float *colscale;  // [N] per-column factor on A.B, or nullptr
    float *C;
    float alpha, beta;      // alpha includes 1/16 for Q4_0
    int nchunk;             // 16-byte chunks per prepared row (= K / elements per chunk)
    int act;
    const float *res;
    long long tail0;
    unsigned wbytes;        // N * ldt
    unsigned xbytes;        // M * K * 4
    int nw;                 // waves per workgroup, 1 .. 16
    int mpart;              // rows of a workgroup: row part blockIdx.y is rows [y mpart, (y + 1) mpart)
};

__device__ __forceinline__ uintx4 tm_load16(const void *base, unsigned nbytes, unsigned off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)nbytes, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}

// Two floats to two bf16 (round to nearest even), a in the low half.
__device__ __forceinline__ uint32_t pk_bf16(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2){a, b}, bf16x2));
}
// hi = bf16(x), lo = bf16(x - hi) for a pair of floats, x first clamped to
// the largest finite bf16 (0x1.fep127) for hi: a finite x above 3.396e38
// would otherwise round to an infinite hi.  An infinite x gets
// hi = +-0x1.fep127 and lo = x - hi = x, so that x . q is inf . q as in the
// reference's fp32 product (a NaN where q = 0, else an infinity); a NaN x
// leaves a NaN residual whatever the clamp returned for it.
__device__ __forceinline__ void split_pair(float a, float b, uint32_t &hi, uint32_t &lo) {
    constexpr float kMax = 0x1.fep127f;
    hi = pk_bf16(__builtin_amdgcn_fmed3f(a, -kMax, kMax), __builtin_amdgcn_fmed3f(b, -kMax, kMax));
    lo = pk_bf16(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}
// Signed byte `i` of w as a float.
__device__ __forceinline__ float sbyte(uint32_t w, int i) { return (float)(int8_t)(w >> (8 * i)); }

// First k of element group q of chunk ch (the prepared layout's chunk
// interleave: 64-chunk superchunks, the last `width` chunks wide).
__device__ __forceinline__ int tm_group_k(int ch, int q, int nchunk, int E) {
    const int sc = ch >> 6, c = ch & 63;
    const int width = min(64, nchunk - (sc << 6));
    return sc * 64 * E + 4 * (q * width + c);
}

// Per-wave staging layout, in dwords: row r (hi rows 0 .. MR - 1, lo rows
// MR .. 2 MR - 1) of k-set st for lane group g of sub-round it at
// it * sub + g * group + st * set + 4 r.  The strides are padded so that a
// wave's 8-byte staging writes spread over the 64 LDS banks with at most
// two dwords a bank per instruction (the least 64 lanes x 2 dwords allow)
// and its 16-byte operand reads with at most four (1 KiB over 256 bytes of
// banks); unpadded, every stride is a multiple of 64 dwords and the writes
// serialise up to 16 ways.  (Found by exhaustive search over the strides.)
struct TmStage {
    int lo, set, group, sub, wave;
};
constexpr TmStage tm_stage_make(int mr, int it, int set, int group, int pad2, int pad4) {
    const int sub = 4 * group + (it == 2 ? pad2 : it == 4 ? pad4 : 0);
    return {4 * mr, set, group, sub, it * sub};
}
template <int FMT, int MR, int IT>
constexpr TmStage tm_stage() {
    if constexpr (FMT == TML_FMT_Q8_0) {
        if constexpr (MR == 2) return tm_stage_make(MR, IT, 16, 48, 8, 4);
        else if constexpr (MR == 4) return tm_stage_make(MR, IT, 32, 80, 8, 4);
        else return tm_stage_make(MR, IT, 64, IT == 1 ? 144 : IT == 2 ? 136 : 132, 0, 0);
    } else {
        if constexpr (MR == 2) return tm_stage_make(MR, IT, 20, 80, 0, 4);
        else if constexpr (MR == 4) return tm_stage_make(MR, IT, 36, 144, 0, 4);
        else return tm_stage_make(MR, IT, 68, 272, 0, 4);
    }
}

// B operand of k-set st of a prepared chunk: 8 bf16 weights (16 q for Q4_0).
template <int FMT>
__device__ __forceinline__ uintx4 tm_weights(const uintx4 &w, int st) {
    uintx4 b;
    if constexpr (FMT == TML_FMT_Q8_0) {
        // k-set st = element groups 2 st, 2 st + 1 (dwords 2 st, 2 st + 1)
        const uint32_t d0 = w[2 * st], d1 = w[2 * st + 1];
        b[0] = pk_bf16(sbyte(d0, 0), sbyte(d0, 1));
        b[1] = pk_bf16(sbyte(d0, 2), sbyte(d0, 3));
        b[2] = pk_bf16(sbyte(d1, 0), sbyte(d1, 1));
        b[3] = pk_bf16(sbyte(d1, 2), sbyte(d1, 3));
    } else {
        // k-set st = dword st = elements 8 st .. 8 st + 7 (element groups
        // 2 st, 2 st + 1), nibble j at bits 4j: even nibbles moved to the top
        // of their byte, odd ones masked in place, each byte then 16 q as a
        // signed byte.  Order: elements 0, 2, 1, 3, 4, 6, 5, 7 of the dword,
        // i.e. (x, z), (y, w) of group 2 st, then of group 2 st + 1.
        const uint32_t d = w[st];
        const uint32_t ev = (d << 4) & 0xF0F0F0F0u, od = d & 0xF0F0F0F0u;
        b[0] = pk_bf16(sbyte(ev, 0), sbyte(ev, 1));
        b[1] = pk_bf16(sbyte(od, 0), sbyte(od, 1));
        b[2] = pk_bf16(sbyte(ev, 2), sbyte(ev, 3));
        b[3] = pk_bf16(sbyte(od, 2), sbyte(od, 3));
    }
    return b;
}

template <int FMT, int IT, int MR, int T, bool PF>
__global__ __launch_bounds__(1024) void gemv_tm_kernel(GemvTmArgs a) {
    constexpr int E = FMT == TML_FMT_Q8_0 ? 16 : 32;  // elements per 16-byte chunk
    constexpr int NQ = E / 4;                          // element groups (float4) per chunk
    constexpr int SETS = NQ / 2;                       // 8-element MFMA k-sets per chunk
    constexpr int R = 4 * IT;                          // chunks of a wave's run per round
    constexpr int TOT = MR * NQ * R;                   // activation float4s a wave stages per round
    constexpr int TASKS = (TOT + 63) / 64;
    constexpr TmStage L = tm_stage<FMT, MR, IT>();
    static_assert(IT == 1 || IT == 2 || IT == 4, "runs of 4, 8 or 16 chunks");
    static_assert(L.lo == 4 * MR && L.set >= 8 * MR && (SETS - 1) * L.set + 8 * MR <= L.group &&
                      4 * L.group <= L.sub && L.wave == IT * L.sub && L.wave % 4 == 0,
                  "staging blocks overlap");
    // [nw][L.wave] staging dwords, then (nw - 1) x T x 64 accumulators
    TML_DYNAMIC_LDS(uint32_t, tm_lds);

    const int nw = a.nw;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;  // B: column n0 + 16 tile + c; A: row c
    const int n0 = blockIdx.x * 16 * T;
    // this workgroup's rows: [row0, row0 + mloc)
    const int row0 = blockIdx.y * a.mpart, mloc = min(a.mpart, a.M - row0);
    bool col_ok[T];
    unsigned wrow[T];
#pragma unroll
    for (int tl = 0; tl < T; ++tl) {
        col_ok[tl] = n0 + 16 * tl + c < a.N;
        wrow[tl] = (unsigned)(n0 + 16 * tl + c) * (unsigned)a.ldt;
    }
    uint32_t *const wst = tm_lds + wave * L.wave;
    // A-operand lane c reads row c % (2 MR): rows past 2 MR repeat staged
    // rows, and row i of the product depends on row i of A alone.
    const int rbase = g * L.group + (c % (2 * MR)) * 4;

    floatx4 acc[T];
#pragma unroll
    for (int tl = 0; tl < T; ++tl) acc[tl] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
    // A round: wave w owns the run of R chunks r0 + w R + [0, R); lane group
    // g of sub-round it takes chunk 4 it + g of the run.
    auto load_round = [&](int r0, uintx4 (&w)[IT][T], floatx4 (&x)[TASKS]) __attribute__((always_inline)) {
        const int base = r0 + wave * R;
#pragma unroll
        for (int it = 0; it < IT; ++it) {
            const int ch = base + 4 * it + g;
#pragma unroll
            for (int tl = 0; tl < T; ++tl)
                w[it][tl] = tm_load16(a.Bt, a.wbytes,
                                      ch < a.nchunk && col_ok[tl] ? wrow[tl] + 16u * (unsigned)ch : kOutOfRange);
        }
        // Staging task j = lane + 64 t: chunk u = j % R of the run, element
        // group q and row m of (j / R) -- consecutive lanes take consecutive
        // chunks, whose element groups q are adjacent float4s of the
        // activation row (the layout's chunk interleave), so each load
        // instruction reads runs of 16 R contiguous bytes.
#pragma unroll
        for (int t = 0; t < TASKS; ++t) {
            const int j = lane + 64 * t;
            const int u = j % R, rest = j / R, q = rest % NQ, m = rest / NQ;
            const int ch = base + u;
            const bool in = j < TOT && ch < a.nchunk && m < mloc;
            const unsigned k = in ? (unsigned)tm_group_k(ch, q, a.nchunk, E) : 0u;
            x[t] = __builtin_bit_cast(floatx4,
                                      tm_load16(a.A, a.xbytes, in ? 4u * ((unsigned)(row0 + m) * (unsigned)a.K + k) : kOutOfRange));
        }
    };
    auto compute_round = [&](const uintx4 (&w)[IT][T], const floatx4 (&x)[TASKS]) __attribute__((always_inline)) {
        // Split and stage: k-set q / 2, dwords 2 (q & 1) and 2 (q & 1) + 1 of
        // row m (the B order below), the lo part in row m + MR.
#pragma unroll
        for (int t = 0; t < TASKS; ++t) {
            const int j = lane + 64 * t;
            if (j < TOT) {
                const int u = j % R, rest = j / R, q = rest % NQ, m = rest / NQ;
                const floatx4 v = x[t];
                uint32_t h0, l0, h1, l1;
                if constexpr (FMT == TML_FMT_Q8_0) {
                    split_pair(v[0], v[1], h0, l0);
                    split_pair(v[2], v[3], h1, l1);
                } else {
                    split_pair(v[0], v[2], h0, l0);
                    split_pair(v[1], v[3], h1, l1);
                }
                uint32_t *const d =
                    wst + (u >> 2) * L.sub + (u & 3) * L.group + (q >> 1) * L.set + 4 * m + 2 * (q & 1);
                *(uintx2 *)d = (uintx2){h0, h1};
                *(uintx2 *)(d + L.lo) = (uintx2){l0, l1};
            }
        }
        // the wave's own LDS writes, read back by other lanes of the wave
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
        for (int it = 0; it < IT; ++it) {
#pragma unroll
            for (int st = 0; st < SETS; ++st) {
                const bf16x8 av = __builtin_bit_cast(bf16x8, *(const uintx4 *)(wst + it * L.sub + rbase + st * L.set));
#pragma unroll
                for (int tl = 0; tl < T; ++tl)
                    acc[tl] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        av, __builtin_bit_cast(bf16x8, tm_weights<FMT>(w[it][tl], st)), acc[tl], 0, 0, 0);
            }
        }
        // every lane's reads done before the next round's writes
        __builtin_amdgcn_wave_barrier();
    };

    const int step = nw * R;
    uintx4 wa[IT][T];
    floatx4 xa[TASKS];
    if constexpr (PF) {
        // Two rounds in flight: the next round's loads are issued before
        // this round's arithmetic, so a wave's memory latency overlaps its
        // own work, not only other waves'.
        uintx4 wb[IT][T];
        floatx4 xb[TASKS];
        load_round(0, wa, xa);
        for (int r0 = 0; r0 < a.nchunk; r0 += 2 * step) {
            if (r0 + step < a.nchunk) load_round(r0 + step, wb, xb);
            compute_round(wa, xa);
            if (r0 + step >= a.nchunk) break;
            if (r0 + 2 * step < a.nchunk) load_round(r0 + 2 * step, wa, xa);
            compute_round(wb, xb);
        }
    } else {
        for (int r0 = 0; r0 < a.nchunk; r0 += step) {
            load_round(r0, wa, xa);
            compute_round(wa, xa);
        }
    }

    // Lane (c, g) holds D[4 g + r][c] of each tile: rows of A, columns of B
    // (outputs n0 + 16 tile + c).  Add the waves' accumulators in wave order,
    // then wave 0 adds the lo row m + MR to the hi row m and writes the
    // outputs.
    if (nw > 1) {
        floatx4 *const red = (floatx4 *)(tm_lds + nw * L.wave);
        if (wave > 0) {
#pragma unroll
            for (int tl = 0; tl < T; ++tl) red[((wave - 1) * T + tl) * 64 + lane] = acc[tl];
        }
        __syncthreads();
        if (wave != 0) return;
        for (int w2 = 0; w2 < nw - 1; ++w2) {
#pragma unroll
            for (int tl = 0; tl < T; ++tl) acc[tl] += red[(w2 * T + tl) * 64 + lane];
        }
    }
#pragma unroll
    for (int tl = 0; tl < T; ++tl) {
        floatx4 v4 = acc[tl];
        if constexpr (MR == 2) {
            v4[0] += v4[2];
            v4[1] += v4[3];
        } else {
#pragma unroll
            for (int r = 0; r < 4; ++r) v4[r] += __shfl_xor(v4[r], 4 * MR);
        }
        const int n = n0 + 16 * tl + c;
        if (n >= a.N) continue;
        const float colf = a.colscale ? a.alpha * a.colscale[n] : a.alpha;
        const float biasn = a.bias ? a.bias[n] : 0.0f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = 4 * g + r;
            if (m < MR && m < mloc) {
                const long long flat = (long long)(row0 + m) * a.N + n;
                float v = colf * v4[r];
                if (a.beta != 0.0f) v += a.beta * a.C[flat];
                if (a.bias) v += biasn;
                if (a.res) v += a.res[flat];
                a.C[flat] = tml_apply_act(v, a.act, flat, a.tail0);
            }
        }
    }
}

template <int FMT, int MR, int IT>
constexpr size_t tm_lds_bytes(int nw, int tiles) {
    return (size_t)nw * tm_stage<FMT, MR, IT>().wave * 4 + (size_t)(nw - 1) * tiles * 64 * sizeof(floatx4);
}

template <int FMT, int IT, int MR, int T>
void launch_tm_pf(const GemvTmArgs &ka, bool pf, unsigned grid, hipStream_t s) {
    const dim3 block((unsigned)ka.nw * 64);
    const size_t lds = tm_lds_bytes<FMT, MR, IT>(ka.nw, T);
    // runs of 16 chunks hold too many registers for two rounds in flight
    if constexpr (IT < 4) {
        if (pf) {
            gemv_tm_kernel<FMT, IT, MR, T, true><<<dim3(grid, (unsigned)((ka.M + ka.mpart - 1) / ka.mpart)), block, lds, s>>>(ka);
            return;
        }
    }
    gemv_tm_kernel<FMT, IT, MR, T, false><<<dim3(grid, (unsigned)((ka.M + ka.mpart - 1) / ka.mpart)), block, lds, s>>>(ka);
}

template <int FMT, int IT, int T>
void launch_tm_mr(const GemvTmArgs &ka, bool pf, unsigned grid, hipStream_t s) {
    if (ka.mpart <= 2) launch_tm_pf<FMT, IT, 2, T>(ka, pf, grid, s);
    else if (ka.mpart <= 4) launch_tm_pf<FMT, IT, 4, T>(ka, pf, grid, s);
    else launch_tm_pf<FMT, IT, 8, T>(ka, pf, grid, s);
}

template <int FMT, int T>
void launch_tm_it(const GemvTmArgs &ka, int it, bool pf, unsigned grid, hipStream_t s) {
    switch (it) {
        case 1: launch_tm_mr<FMT, 1, T>(ka, pf, grid, s); break;
        case 2: launch_tm_mr<FMT, 2, T>(ka, pf, grid, s); break;
        default: launch_tm_mr<FMT, 4, T>(ka, pf, grid, s); break;
    }
}

template <int FMT>
void launch_tm_t(const GemvTmArgs &ka, int it, int tiles, bool pf, unsigned grid, hipStream_t s) {
    if (tiles == 2) launch_tm_it<FMT, 2>(ka, it, pf, grid, s);
    else launch_tm_it<FMT, 1>(ka, it, pf, grid, s);
}

template <int FMT>
size_t tm_lds_need_fmt(int64_t M, int it, int nw, int tiles) {
    const int mr = M <= 2 ? 2 : M <= 4 ? 4 : 8;
    switch (mr * 10 + it) {
        case 21: return tm_lds_bytes<FMT, 2, 1>(nw, tiles);
        case 22: return tm_lds_bytes<FMT, 2, 2>(nw, tiles);
        case 24: return tm_lds_bytes<FMT, 2, 4>(nw, tiles);
        case 41: return tm_lds_bytes<FMT, 4, 1>(nw, tiles);
        case 42: return tm_lds_bytes<FMT, 4, 2>(nw, tiles);
        case 44: return tm_lds_bytes<FMT, 4, 4>(nw, tiles);
        case 81: return tm_lds_bytes<FMT, 8, 1>(nw, tiles);
        case 82: return tm_lds_bytes<FMT, 8, 2>(nw, tiles);
        default: return tm_lds_bytes<FMT, 8, 4>(nw, tiles);
    }
}
// LDS bytes of a launch: staging of nw waves plus the cross-wave sums.
size_t tm_lds_need(int fmt, int64_t M, int it, int nw, int tiles) {
    return fmt == TML_FMT_Q8_0 ? tm_lds_need_fmt<TML_FMT_Q8_0>(M, it, nw, tiles)
                               : tm_lds_need_fmt<TML_FMT_Q4_0>(M, it, nw, tiles);
}
constexpr size_t kTmMaxLds = 160 * 1024;  // LDS of a gfx950 CU

}  // namespace

// M = 3..8, and M = 2 for Q4_0 rows of at most 64 chunks: at M = 2 the
// VALU kernels are faster for Q8_0 (3.51 against 3.82 us at 1024x4096) and
// long Q4_0 rows (5.32 against 5.50 us at 5120x1280), slower for short Q4_0
// rows (4.67 against 4.00 us at 1280x5120).
// What the kernel can run: Q8_0 / Q4_0, M = 1..8, K whole chunks.
bool gemv_tm_capable(int fmt, int64_t M, int64_t K) {
    const int64_t e = fmt == TML_FMT_Q8_0 ? 16 : fmt == TML_FMT_Q4_0 ? 32 : 0;
    return e > 0 && M >= 1 && M <= kPreparedGemvMaxM && K > 0 && K % e == 0 && K < ((int64_t)1 << 30);
}

// M = 1 with at least 32768 columns (a vocabulary projection): Q4_0's int4
// decode makes the VALU kernel instruction-bound there (12.71 against 10.61
// us at 1280x51866), and Q8_0 runs 13.98 against 14.89 us; on the layer
// shapes the VALU kernel is the faster one.
bool gemv_tm_m1_preferred(int fmt, int64_t N, int64_t K) {
    return (fmt == TML_FMT_Q4_0 || fmt == TML_FMT_Q8_0) && N >= 32768 && gemv_tm_capable(fmt, 1, K) &&
           env_int("TML_GEMVTM", 1) != 0;
}

bool gemv_tm_supported(int fmt, int64_t M, int64_t K) {
    const int64_t e = fmt == TML_FMT_Q8_0 ? 16 : 32;
    if (!gemv_tm_capable(fmt, M, K)) return false;
    const int mode = env_int("TML_GEMVTM", 1);  // 0: off; 2: every M (tests)
    if (mode == 0) return false;
    if (mode == 2) return true;
    return M >= 3 || (M == 2 && fmt == TML_FMT_Q4_0 && K / e <= 64);
}

Status launch_gemv_tm(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *Bt, int64_t ldt,
                      const float *bias, const float *res, float *C, float alpha_eff, float beta, int act,
                      long long tail0, const float *colscale, hipStream_t s) {
    if (!gemv_tm_capable(fmt, M, K)) return Status::Err(TML_ERR_INVALID_ARG, "matrix-core GEMV: unsupported");
    const int64_t e = fmt == TML_FMT_Q8_0 ? 16 : 32;
    if (ldt < prepared_row_bytes(fmt, K) || ldt % 16 != 0 || ((uintptr_t)Bt % 16) != 0 || ((uintptr_t)A % 16) != 0)
        return Status::Err(TML_ERR_INVALID_ARG, "matrix-core GEMV: prepared layout or alignment");
    // every buffer offset stays below 2^31 (the out-of-range marker)
    if (N * ldt >= ((int64_t)1 << 31) || M * K * 4 >= ((int64_t)1 << 31) || N >= ((int64_t)1 << 30))
        return Status::Err(TML_ERR_INVALID_SHAPE, "matrix-core GEMV: operand too large");
    GemvTmArgs ka;
    ka.M = (int)M; ka.N = (int)N; ka.K = (int)K;
    ka.A = A; ka.Bt = (const uint8_t *)Bt; ka.ldt = ldt;
    ka.bias = bias; ka.colscale = colscale; ka.C = C;
    ka.alpha = fmt == TML_FMT_Q4_0 ? alpha_eff * 0.0625f : alpha_eff;  // int4 read as 16 q
    ka.beta = beta;
    ka.nchunk = (int)(K / e);
    ka.act = act; ka.res = res; ka.tail0 = tail0;
    ka.wbytes = (unsigned)(N * ldt);
    ka.xbytes = (unsigned)(M * K * 4);
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
    }
    // Two 16-column tiles a workgroup at M > 4 where one tile each would
    // leave some CU two workgroups: each CU then stages the activations once
    // for 32 columns instead of twice for 16 (1280x5120 Q4_0, M = 8: 5.48
    // against 5.77 us; at M <= 4 the second tile's registers cost more than
    // the staging saves: 4.57 against 4.01 us at M = 2).
    // Rows of a workgroup.  Where the column tiles alone give fewer
    // workgroups than CUs, M >= 4 rows are split into row parts (grid.y),
    // up to ceil(CUs / workgroups) of them, 2 (3 from M = 7), and M = 4
    // into two parts below twice the CUs; each part
    // stages only its rows' activations and streams the same weights (from
    // L2 after the first).  Measured (us, unsplit -> split, parts): Q4_0
    // 5120x1280 M = 4 6.67 -> 5.59 (2), M = 8 8.14 -> 6.27 (3; 6.62 with
    // 2, 7.36 with 4); 1280x5120 M = 8 6.02 -> 5.59 (2); Q8_0 4096x1024
    // M = 4 7.36 -> 6.37 (2), M = 8 8.16 -> 7.14 (3).  Where every CU
    // already has a workgroup the weight re-reads cost more: Q8_0
    // 1024x4096 M = 8 4.67 -> 4.99.  TML_GEMVTM_MSPLIT forces the count.
    {
        const int64_t wg0 = M > 4 && (N + 15) / 16 > cus ? (N + 31) / 32 : (N + 15) / 16;
        int parts = 1;
        if (M >= 4 && wg0 < cus)
            parts = (int)std::min<int64_t>((cus + wg0 - 1) / wg0, M >= 7 ? 3 : 2);
        else if (M == 4 && wg0 < 2LL * cus)
            parts = 2;  // two parts of two rows: 1280x5120 Q4_0 4.96 -> 4.71 us, 1024x4096 Q8_0 4.39 -> 4.40
        const int forced_parts = env_int("TML_GEMVTM_MSPLIT", 0);
        if (forced_parts >= 1 && forced_parts <= 8) parts = forced_parts;
        ka.mpart = (int)((M + parts - 1) / parts);
    }
    const int64_t mp = ka.mpart;
    int tiles = mp > 4 && (N + 15) / 16 > cus ? 2 : 1;
    const int forced_t = env_int("TML_GEMVTM_T", 0);
    if (forced_t == 1 || forced_t == 2) tiles = forced_t;
    const int64_t grid = (N + 16 * tiles - 1) / (16 * tiles);
    // Runs of R = 4 it chunks per wave and round, it in {1, 2}, at most ten
    // waves: the fewest rounds, then no idle chunk slots, then the most
    // waves.  Measured on MI355X: 40 chunks (K = 1280 Q4_0) -> 10 waves x 4,
    // 64 (K = 1024 Q8_0) -> 8 x 8, 160 (K = 5120 Q4_0) -> 10 x 8 twice,
    // each within 3 % of the best of 4-16 waves x runs of 4, 8, 16.
    int it = 1, nw = 1;
    {
        int64_t best_rounds = -1, best_waste = 0;
        for (int cit = 1; cit <= 2; ++cit)
            for (int cnw = 1; cnw <= 10; ++cnw) {
                const int64_t per = 4LL * cit * cnw;
                const int64_t rounds = (ka.nchunk + per - 1) / per, waste = rounds * per - ka.nchunk;
                const bool better = best_rounds < 0 || rounds < best_rounds ||
                                    (rounds == best_rounds && (waste < best_waste ||
                                                               (waste == best_waste && cnw > nw)));
                if (better) {
                    best_rounds = rounds;
                    best_waste = waste;
                    it = cit;
                    nw = cnw;
                }
            }
    }
    // With eight or more workgroups a CU (vocabulary-sized N), Q4_0: two
    // waves of runs of four, more workgroups resident per CU hiding more
    // latency (1280x51866, M = 1: 10.61 us, against 11.22 with four waves
    // and 14.57 with ten); Q8_0: five waves of runs of eight with two rounds
    // in flight (13.98 us; 14.22 with four waves, 14.59 with one round).
    bool pf = false;
    if (grid >= 8LL * cus) {
        if (fmt == TML_FMT_Q8_0) {
            it = 2;
            nw = (int)std::min<int64_t>(5, (ka.nchunk + 7) / 8);
            pf = true;
        } else {
            it = 1;
            nw = (int)std::min<int64_t>(2, (ka.nchunk + 3) / 4);
        }
    }
    const int forced_nw = env_int("TML_GEMVTM_NW", 0), forced_it = env_int("TML_GEMVTM_IT", 0);
    if (forced_it == 1 || forced_it == 2 || forced_it == 4) it = forced_it;
    if (forced_nw >= 1 && forced_nw <= 16) nw = forced_nw;
    // at most half the LDS where a CU may get two workgroups
    const size_t lds_cap = forced_nw || grid <= cus ? kTmMaxLds : kTmMaxLds / 2;
    while (nw > 1 && tm_lds_need(fmt, mp, it, nw, tiles) > lds_cap) --nw;
    if (tm_lds_need(fmt, mp, it, nw, tiles) > kTmMaxLds)
        return Status::Err(TML_ERR_INVALID_ARG, "matrix-core GEMV: staging exceeds the LDS");
    ka.nw = nw;
    // Two rounds in flight elsewhere: measured no faster on the decoder
    // shapes (Q4_0 vocabulary 10.64 against 10.61 us), so only on request.
    const int forced_pf = env_int("TML_GEMVTM_PF", -1);
    if (forced_pf == 0 || forced_pf == 1) pf = forced_pf == 1;
    switch (fmt) {
        case TML_FMT_Q8_0: launch_tm_t<TML_FMT_Q8_0>(ka, it, tiles, pf, (unsigned)grid, s); break;
        default: launch_tm_t<TML_FMT_Q4_0>(ka, it, tiles, pf, (unsigned)grid, s); break;
    }
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

}  // namespace tml
