// gemm_qbf.hip -- Q8_0 / Q4_0 weight-only GEMM for M > 8 on the bf16 matrix
// cores, the weights dequantized into LDS.
//
//   C[M,N] = act(alpha * A[M,K] . q[K,N] + beta * C + bias[N] + R)
//   (q: int8, or int4 two per byte, even n in the low nibble; alpha carries
//   the per-tensor scale, colscale the per-column ones of the _PC formats)
//
// The reference multiplies fp32 activations by dequantized weights and
// accumulates in fp32 (src/core/quantization.zig:240-311 Q8_0,
// :829-957 Q4_0).  Here the products run on v_mfma_f32_16x16x32_bf16 with
// fp32 accumulation:
//   * weights: int8 and int4 values are exact in bf16, so B is converted
//     once per workgroup when a slice is staged in LDS;
//   * activations: each fp32 x is split into hi = bf16(x) and lo =
//     bf16(x - hi), round to nearest even both, so |x - hi - lo| <= 2^-17 |x|
//     (an infinite x keeps lo = 0); the product is hi . q + lo . q, two
//     MFMAs into the same fp32 accumulator.
// The result equals the dequantize-then-fp32-accumulate product to ~1e-5
// relative (summation order and the 2^-17 split), inside the 1e-3 bar of the
// quantized paths.  A bf16 MFMA does 16x the work of the fp32 MFMA of the
// other GEMM kernels in half the cycles, so even the two of them per product
// leave the kernel bound by its LDS traffic, not by the matrix cores.
//
// Tiles.  A workgroup of four or eight waves owns a BM x BN tile of C (each
// wave a WM x WN sub-tile of (WM/16) x (WN/16) MFMA tiles, or with two wave
// groups half the k of one; with eight waves, half of them stage A and half
// B, see gemm_qbf_kernel) and walks K in 32- or
// 64-deep slices (BK) through two LDS stages: the next slice's global loads
// are issued before the current slice's MFMAs, converted and written after
// them, one barrier a slice.  LDS holds, per stage, A's hi and lo planes and
// B as bf16, each as rows of BK / 8 16-byte slots (8 k each) -- A by output
// row, B by output column, both k-contiguous as the MFMA operands want them
// -- with slot s of row r stored at s ^ ((r / 4) % 4) for four slots and
// s ^ ((r / 2) % 8) for eight, which keeps the operand reads (16 rows, one
// slot) and the staging writes free of bank conflicts.  The 64-deep slices
// halve the steps (barriers, LDS round trips) over a K range; they pay on
// the small tiles, where the tiles are few (M <= 512).
#include "tml_internal.hpp"

#include <algorithm>
#include <type_traits>

namespace tml {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float floatx2 __attribute__((ext_vector_type(2)));

constexpr int kQbfXcd = 8;  // XCDs of an MI355X: workgroups are dealt to them round robin

struct QbfArgs {
    int M, N, K;
    const float *A;         // [M,K], K % 8 == 0, 16-byte aligned
    const uint8_t *B;       // [K,N]: N bytes a row (int8) or N / 2 (int4)
    int ldb;                // bytes per B row
    const float *bias;      // [N] or nullptr
    const float *colscale;  // [N] per-column factor on A.B, or nullptr
    const float *res;       // [M,N] residual after the bias, or nullptr (may equal C)
    float *C;
    float alpha, beta;
    int act;
    long long tail0;
    unsigned a_bytes, b_bytes;  // M * K * 4, K * ldb
    int tiles_m, tiles_n;
    int nsplit, spl;        // K splits, 32-deep slices per split
    float *ws;              // nsplit > 1: [nsplit][M][N] raw partials
    int vec_epi;            // N % 4 == 0 and C, bias, residual, column scales 16-byte aligned
};

__device__ __forceinline__ uintx4 qbf_load16(const void *base, unsigned nbytes, unsigned off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)nbytes, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t qbf_load2(const void *base, unsigned nbytes, unsigned off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)nbytes, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}
__device__ __forceinline__ uint32_t qbf_load1(const void *base, unsigned nbytes, unsigned off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)nbytes, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b8(r, off, 0, 0);
}

// Two floats to two bf16 (round to nearest even), a in the low half.
__device__ __forceinline__ uint32_t qbf_pk(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2){a, b}, bf16x2));
}
// hi = bf16(x), lo = bf16(x - hi) of a pair, x first clamped to the largest
// finite bf16 (0x1.fep127) for hi.  A finite x past it (above 3.396e38)
// would round to an infinite hi and give inf . 0 = nan where the reference
// has 0; clamped, hi + lo is x again.  An infinite x gets hi = +-0x1.fep127
// and lo = x - hi = x, so x . q is the reference's inf . q (nan at q = 0); a
// NaN x leaves a NaN residual whatever the clamp returned for it.
__device__ __forceinline__ void qbf_split(float a, float b, uint32_t &hi, uint32_t &lo) {
    constexpr float kMax = 0x1.fep127f;
    hi = qbf_pk(__builtin_amdgcn_fmed3f(a, -kMax, kMax), __builtin_amdgcn_fmed3f(b, -kMax, kMax));
    lo = qbf_pk(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xFFFF0000u));
}

// Physical slot of logical slot s (8 k) in LDS row r of SL slots: four
// slots (64-byte rows) swap by (r / 4) mod 4, eight (128-byte rows) by
// (r / 2) mod 8, so that 16 consecutive rows read at one logical slot, and
// the staging writes of consecutive slots, cover the 64 banks evenly.
template <int SL>
__device__ __forceinline__ int qbf_slot(int r, int s) {
    if constexpr (SL == 4) return r * 4 + (s ^ ((r >> 2) & 3));
    else return r * 8 + (s ^ ((r >> 1) & 7));
}

// NW = 8 (eight waves): waves 0-3 stage A and waves 4-7 stage B, so each
// wave does one operand's share of a step's staging, and two waves share
// each SIMD, so one's waits are covered by the other's work.  The eight waves
// either own eight WM x WN sub-tiles (KW = 1) or, with KW = 2, two groups of
// four: group 0 (waves 0-3) multiplies the first 32-k half of every 64-deep
// slice and group 1 (waves 4-7) the second half, each wave of a group on its
// own sub-tile; group 1 hands its accumulators to group 0 through LDS after
// the main loop, and group 0 runs the epilogue.
template <int FMT, int BM, int BN, int WM, int WN, int D, int BK = 32, int KW = 1, int NW = 4 * KW>
__global__ __launch_bounds__(64 * NW) void gemm_qbf_kernel(QbfArgs a) {
    static_assert(BK == 32 || BK == 64, "32- or 64-deep slices");
    static_assert(KW == 1 || (KW == 2 && BK == 64), "two wave groups split 64-deep slices into 32-k halves");
    static_assert(NW == 4 || NW == 8, "four waves, or eight staging A and B in two halves");
    constexpr int SL = BK / 8;  // 16-byte slots (8 k) of an LDS row
    constexpr int NT = 256;     // staging threads of an operand (all 256 take both when NW = 4)
    constexpr int NWS = NW / KW;  // waves per group, one per sub-tile
    constexpr int TM = WM / 16, TN = WN / 16;
    constexpr int WAVES_N = BN / WN;
    static_assert((BM / WM) * (BN / WN) == NWS, "one wave of a group per WM x WN sub-tile");
    static_assert(WM % 16 == 0 && WN % 16 == 0, "whole 16 x 16 MFMA tiles");
    // staging tasks of a slice: A one (row, 8-k slot) each; B one (column
    // pair, 8-k slot) each
    constexpr int TA = BM * SL, TB = (BN / 2) * SL;
    constexpr int PA = (TA + NT - 1) / NT, PB = (TB + NT - 1) / NT;
    static_assert(TA % NT == 0 || TA < NT, "A tasks split evenly");

    __shared__ uintx4 Ah[2][BM * SL], Al[2][BM * SL], Bs[2][BN * SL];

    // tid: the thread's index among the NT threads that stage its operand(s)
    const int tid = threadIdx.x % NT, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6);
    const int kg = KW == 2 ? wave / NWS : 0;  // wave group
    const int sw = wave % NWS;               // sub-tile of the wave
    const int wm0 = (sw / WAVES_N) * WM, wn0 = (sw % WAVES_N) * WN;
    const int c = lane & 15, g = lane >> 4;

    // Workgroup -> (tile, K split): consecutive ids within each XCD (own
    // L2), the splits of a tile adjacent, then groups of four tile rows so
    // that neighbours share A rows and B columns.
    int tile_m, tile_n, split;
    {
        const int nblk = gridDim.x, b = blockIdx.x;
        const int per = nblk / kQbfXcd, rem = nblk % kQbfXcd;
        const int xcd = b % kQbfXcd, idx = b / kQbfXcd;
        const int lin = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
        split = lin % a.nsplit;
        const int tlin = lin / a.nsplit;
        constexpr int GM = 4;
        const int group = GM * a.tiles_n;
        const int first_m = (tlin / group) * GM;
        const int gsize = min(a.tiles_m - first_m, GM);
        tile_m = first_m + (tlin % group) % gsize;
        tile_n = (tlin % group) / gsize;
    }
    const int m0 = tile_m * BM, n0 = tile_n * BN;
    // this split's k range [kbase, kend)
    const int kbase = split * a.spl * 32, kend = min(a.K, kbase + a.spl * 32);

    // ---- staging: global -> registers, D slices ahead -> bf16 in LDS (after
    // the MFMAs of the slice before).  Offsets are formed without branches
    // (a branch around a load makes the compiler wait for every load in
    // flight): rows of A past M and k-rows of B past K lie past the buffer's
    // byte count and read zeros; A slots past the split's end get bit 31 set
    // (past every byte count) so they read zeros instead of the next row or
    // the next split's k (B rows there are finite integers times those
    // zeros); B columns past N read bytes of the next k-row that only feed
    // dropped outputs; tasks past TA / TB (small tiles) repeat a valid task's
    // loads and skip its store.  k0 counts from kbase.
    uintx4 ra[D][PA][2];
    uint32_t rb[D][PB][8];
    auto load = [&](auto opa, auto opb, int d, int k0) __attribute__((always_inline)) {
        if constexpr (decltype(opa)::value) {
#pragma unroll
            for (int p = 0; p < PA; ++p) {
                const int j = (tid + p * NT) % TA;
                const int row = j / SL, k = kbase + k0 + 8 * (j % SL);
                const unsigned past_k = (unsigned)(kend - 1 - k) & 0x80000000u;
                const unsigned off = (((unsigned)(m0 + row) * (unsigned)a.K + (unsigned)k) * 4u) | past_k;
                ra[d][p][0] = qbf_load16(a.A, a.a_bytes, off);
                ra[d][p][1] = qbf_load16(a.A, a.a_bytes, off + 16u);
            }
        }
        if constexpr (decltype(opb)::value) {
#pragma unroll
            for (int p = 0; p < PB; ++p) {
                const int j = (tid + p * NT) % TB;
                const int cp = j % (BN / 2), s = j / (BN / 2);
                const unsigned col_byte =
                    FMT == TML_FMT_Q8_0 ? (unsigned)(n0 + 2 * cp) : (unsigned)((n0 + 2 * cp) / 2);
                const unsigned off0 = (unsigned)(kbase + k0 + 8 * s) * (unsigned)a.ldb + col_byte;
#pragma unroll
                for (int kk = 0; kk < 8; ++kk) {
                    const unsigned off = off0 + (unsigned)kk * (unsigned)a.ldb;
                    rb[d][p][kk] =
                        FMT == TML_FMT_Q8_0 ? qbf_load2(a.B, a.b_bytes, off) : qbf_load1(a.B, a.b_bytes, off);
                }
            }
        }
    };
    auto store = [&](auto opa, auto opb, int d, int st) __attribute__((always_inline)) {
        if constexpr (decltype(opa)::value) {
#pragma unroll
            for (int p = 0; p < PA; ++p) {
                const int j = tid + p * NT;
                if (TA % NT == 0 || j < TA) {
                    const int row = j / SL, s = j % SL;
                    const floatx4 x0 = __builtin_bit_cast(floatx4, ra[d][p][0]);
                    const floatx4 x1 = __builtin_bit_cast(floatx4, ra[d][p][1]);
                    uint32_t h0, h1, h2, h3, l0, l1, l2, l3;
                    qbf_split(x0[0], x0[1], h0, l0);
                    qbf_split(x0[2], x0[3], h1, l1);
                    qbf_split(x1[0], x1[1], h2, l2);
                    qbf_split(x1[2], x1[3], h3, l3);
                    Ah[st][qbf_slot<SL>(row, s)] = (uintx4){h0, h1, h2, h3};
                    Al[st][qbf_slot<SL>(row, s)] = (uintx4){l0, l1, l2, l3};
                }
            }
        }
        if constexpr (decltype(opb)::value) {
#pragma unroll
            for (int p = 0; p < PB; ++p) {
                const int j = tid + p * NT;
                if (TB % NT == 0 || j < TB) {
                    const int cp = j % (BN / 2), s = j / (BN / 2);
                    uintx4 e, o;  // columns 2 cp (even) and 2 cp + 1, k = 8 s .. 8 s + 7
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        uint32_t w0 = rb[d][p][2 * q], w1 = rb[d][p][2 * q + 1];
                        // pin the words here: otherwise the compiler moves part of
                        // the unpacking of a set loaded this step up to the step's
                        // end, where it must wait for every load in flight
                        __asm__ volatile("" : "+v"(w0), "+v"(w1));
                        if constexpr (FMT == TML_FMT_Q8_0) {
                            e[q] = qbf_pk((float)(int8_t)(w0 & 0xFFu), (float)(int8_t)(w1 & 0xFFu));
                            o[q] = qbf_pk((float)(int8_t)(w0 >> 8), (float)(int8_t)(w1 >> 8));
                        } else {
                            e[q] = qbf_pk((float)((int32_t)(w0 << 28) >> 28), (float)((int32_t)(w1 << 28) >> 28));
                            o[q] = qbf_pk((float)((int32_t)(w0 << 24) >> 28), (float)((int32_t)(w1 << 24) >> 28));
                        }
                    }
                    Bs[st][qbf_slot<SL>(2 * cp, s)] = e;
                    Bs[st][qbf_slot<SL>(2 * cp + 1, s)] = o;
                }
            }
        }
    };

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = (floatx4){0.0f, 0.0f, 0.0f, 0.0f};
    // One slice, 32 k at a time: lane (c, g) reads k = 32 h + 8 g .. + 7 of
    // A rows wm0 + 16 i + c (hi and lo) and of B columns wn0 + 16 j + c.  All
    // hi products first, then the lo ones, so no MFMA waits on the one before.
    // With two wave groups, group kg takes the half h = kg.
    auto compute = [&](int st) __attribute__((always_inline)) {
#pragma unroll
        for (int hh = 0; hh < SL / 4 / KW; ++hh) {
            const int h = KW == 2 ? kg : hh;
            bf16x8 ah[TM], al[TM], bv[TN];
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const int slot = qbf_slot<SL>(wm0 + 16 * i + c, 4 * h + g);
                ah[i] = __builtin_bit_cast(bf16x8, Ah[st][slot]);
                al[i] = __builtin_bit_cast(bf16x8, Al[st][slot]);
            }
#pragma unroll
            for (int j = 0; j < TN; ++j)
                bv[j] = __builtin_bit_cast(bf16x8, Bs[st][qbf_slot<SL>(wn0 + 16 * j + c, 4 * h + g)]);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[i], bv[j], acc[i][j], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[i], bv[j], acc[i][j], 0, 0, 0);
        }
    };

    // Register set d holds slice kt with kt % D == d: slices 0 .. D-1 are
    // requested up front, and each step refills the set its slice left (slice
    // kt + D) before the MFMAs, so D slices of loads are in flight while a
    // slice is multiplied.  The step count is rounded up to a multiple of D
    // (D even): steps past K multiply zeros, and every step of the unrolled
    // body is the same straight-line code with its LDS stage fixed.
    static_assert(D % 2 == 0, "LDS stage of step u is u % 2");
    const int nk = ((kend - kbase + BK - 1) / BK + D - 1) / D * D;
    // The main loop for a wave that stages A (opa) and / or B (opb); both
    // groups' loops hold the same barriers.
    auto run = [&](auto opa, auto opb) __attribute__((always_inline)) {
#pragma unroll
        for (int d = 0; d < D; ++d) load(opa, opb, d, d * BK);
        store(opa, opb, 0, 0);
        __syncthreads();
        for (int kt0 = 0; kt0 < nk; kt0 += D) {
#pragma unroll
            for (int u = 0; u < D; ++u) {
                // the scheduler keeps the three phases in this order, so the
                // loads of a set are always older than the D - 1 sets after it
                load(opa, opb, u, (kt0 + u + D) * BK);
                __builtin_amdgcn_sched_barrier(0);
                compute(u & 1);
                __builtin_amdgcn_sched_barrier(0);
                store(opa, opb, (u + 1) % D, (u + 1) & 1);
                __builtin_amdgcn_sched_barrier(0);
                __syncthreads();
            }
        }
    };
    using yes = std::integral_constant<bool, true>;
    using no = std::integral_constant<bool, false>;
    if constexpr (NW == 4) {
        run(yes{}, yes{});
    } else {
        if (wave < 4) run(yes{}, no{});
        else run(no{}, yes{});
    }
    if constexpr (KW == 2) {
        // Group 1's accumulators to group 0 through A's hi stages, or B's
        // where those are larger (free: the loop's last barrier follows every
        // wave's last LDS read), in lane order per (wave, i, j).
        constexpr bool XB = BN > BM;
        static_assert(NWS * TM * TN * 64 <= 2 * (XB ? BN : BM) * SL, "the exchange fits the stages it uses");
        floatx4 *const xch = XB ? (floatx4 *)&Bs[0][0] : (floatx4 *)&Ah[0][0];
        if (kg == 1) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) xch[((sw * TM + i) * TN + j) * 64 + lane] = acc[i][j];
        }
        __syncthreads();
        if (kg == 0) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j) acc[i][j] += xch[((sw * TM + i) * TN + j) * 64 + lane];
        }
    }
    // the waves that hold the tile's final accumulators (group 1 of KW = 2
    // only helps with the staged stores below)
    const bool holds = KW == 1 || kg == 0;

    // Epilogue: lane (c, g) holds rows 4 g + r, column c of each MFMA tile.
    if (a.nsplit > 1) {
        // raw partial of this split; launch_splitk_reduce adds the splits in
        // order and runs the epilogue
        if (!holds) return;
        float *const part = a.ws + (size_t)split * a.M * a.N;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn0 + 16 * j + c;
            if (col >= a.N) continue;
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wm0 + 16 * i + 4 * g + r;
                    if (row < a.M) part[(size_t)row * a.N + col] = acc[i][j][r];
                }
        }
        return;
    }
    constexpr bool SB = BN > BM;
    constexpr int CAP = 2 * (SB ? BN : BM) * SL * 4;  // floats the staging buffer holds
    constexpr int PW0 = CAP / BM < BN ? CAP / BM : BN;
    constexpr int PW = PW0 >= 64 ? 64 : PW0 >= 32 ? 32 : 16;  // a power of two dividing BN
    static_assert(BN % PW == 0 && PW % 16 == 0 && BM * PW <= CAP, "passes of whole 16-column blocks");
    if (BN == PW && a.vec_epi) {
        // Staged: where the C tile fits the staging buffer (A's hi stages, or
        // B's where those are larger; free after the barrier below) in one
        // pass, it goes through LDS and is written as whole 16-byte pieces of
        // C rows, a row's BN floats by consecutive lanes of one store
        // instruction, so the non-temporal stores leave whole cache lines
        // rather than the 64-byte strips of the per-lane path.  Measured
        // against the per-lane path (us, Q8_0): 128x4096x1024 11.21 ->
        // 10.19, 512x4096x1024 21.01 -> 18.74, 256x4096x1024 13.71 -> 12.88.
        // The large tiles, which would need two (64 x 128) or four (128 x 128)
        // passes, keep the per-lane path: staged, 1500x3840x1280 measured
        // 44.79 against 43.64 us and 1500x5120x1280 54.24 against 53.54, for
        // 2-11 % more HBM writes than C on the per-lane path.
        constexpr int CH = PW / 4;  // 16-byte pieces per pass row
        float *const ct = SB ? (float *)&Bs[0][0] : (float *)&Ah[0][0];
#pragma unroll
        for (int pass = 0; pass < BN / PW; ++pass) {
            __syncthreads();
            if (holds) {
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if ((wn0 + 16 * j) / PW != pass) continue;  // uniform over the wave
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            ct[(wm0 + 16 * i + 4 * g + r) * PW + wn0 + 16 * j + c - pass * PW] = acc[i][j][r];
                }
            }
            __syncthreads();
#pragma unroll
            for (int e = (int)threadIdx.x; e < BM * CH; e += NW * 64) {
                const int row = m0 + e / CH, col = n0 + pass * PW + 4 * (e % CH);
                if (row >= a.M || col >= a.N) continue;  // N % 4 == 0: a piece is all in or all out
                const floatx4 v4 = *(const floatx4 *)&ct[(e / CH) * PW + 4 * (e % CH)];
                const size_t o = (size_t)row * a.N + col;
                floatx4 cv = {0.f, 0.f, 0.f, 0.f}, bv = {0.f, 0.f, 0.f, 0.f}, rv = {0.f, 0.f, 0.f, 0.f};
                floatx4 sv = {1.f, 1.f, 1.f, 1.f};
                if (a.beta != 0.0f) cv = *(const floatx4 *)(a.C + o);
                if (a.bias) bv = *(const floatx4 *)(a.bias + col);
                if (a.res) rv = *(const floatx4 *)(a.res + o);
                if (a.colscale) sv = *(const floatx4 *)(a.colscale + col);
                floatx4 out;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    float v = (a.colscale ? a.alpha * sv[q] : a.alpha) * v4[q];
                    if (a.beta != 0.0f) v += a.beta * cv[q];
                    if (a.bias) v += bv[q];
                    if (a.res) v += rv[q];
                    out[q] = tml_apply_act(v, a.act, (long long)o + q, a.tail0);
                }
                tml_store_c(a.C + o, out);
            }
        }
        return;
    }
    if (!holds) return;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int col = n0 + wn0 + 16 * j + c;
        if (col >= a.N) continue;
        const float colf = a.colscale ? a.alpha * a.colscale[col] : a.alpha;
        const float biasc = a.bias ? a.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm0 + 16 * i + 4 * g + r;
                if (row < a.M) {
                    const long long flat = (long long)row * a.N + col;
                    float v = colf * acc[i][j][r];
                    if (a.beta != 0.0f) v += a.beta * a.C[flat];
                    if (a.bias) v += biasc;
                    if (a.res) v += a.res[flat];
                    tml_store_c(a.C + flat, tml_apply_act(v, a.act, flat, a.tail0));
                }
            }
    }
}

struct QbfCfg {
    int bm, bn, bk, kw, nw;  // kw, nw: gemm_qbf_kernel's wave groups and waves
};
// Tile configs (index = TML_GEMM_QBF_TILE - 1): <BM, BN, BK> with four
// waves of BM/2 x BN/2.  The two large tiles keep two 32-deep slices of loads
// in flight (D = 2: 170 / 117 registers with the accumulators in ordinary
// VGPRs, two and four workgroups a CU), the small ones four; at the large
// tiles D = 2 measured as fast as or faster than D = 4, which holds one
// workgroup a CU at 128 x 128.  The last two are the small tiles on 64-deep
// slices with two in flight (half the steps, so half the barriers and LDS
// round trips a K range; 116 / 87 registers): 32 x 64 x 64 is the fastest
// config wherever the tiles are few (M <= 512 at the config shapes), e.g.
// 128x4096x1024 12.6 against 16.4 us, 128x1280x5120 19.4 against 30.4 us;
// at M = 1500 it is slower than 64 x 128 x 32 (QKV 61.8 against 47.8 us:
// 186 registers at 64 x 128 x 64 hold two workgroups a CU, and 32 x 64
// tiles re-read A and B twice as often).  Configs 6 and 7 are the two
// 64-deep tiles with two wave groups (KW = 2, eight waves; 80 / 64
// registers): every M <= 512 shape measured faster with them (us, Q8_0,
// every launch reading its own weight copy out of >= 1 GiB, one / two
// groups): 128x4096x1024 12.28 / 11.13, 512x4096x1024 21.66 / 19.33,
// 128x1280x5120 19.01 / 17.40, 256x4096x1024 14.74 / 13.56, 256x768x3072
// 16.54 / 15.16, 384x1280x1280 13.98 / 13.40; Q4_0 128x4096x1024 12.28 /
// 11.08, 512x4096x1024 21.46 / 19.37.  At M = 1500 they are slower than
// 64 x 128 x 32 (QKV 54.0 against 46.5 us; a 64 x 128 x 64 two-group tile,
// 130 registers, 55.8), so the large tiles keep one group.  Configs 8 and
// 9 are the large tiles with eight waves instead (NW = 8, one group: 32 x 32
// / 64 x 32 sub-tiles, waves 0-3 staging A and 4-7 B; 72 / 95 registers, so
// three / two workgroups a CU): the planner takes them for every shape past
// the small-tile rules (us, Q8_0, four / eight waves: 1500x3840x1280 at
// 64 x 128 48.9 / 45.2, 1500x5120x1280 at 128 x 128 62.9 / 53.5,
// 3000x3840x1280 at 128 x 128 105.5 / 80.4).  Config 10 is config 7 with
// four 64-deep slices of loads in flight (D = 4), which the planner takes
// where each unit has a CU to itself and K rounds to whole groups of four.
constexpr QbfCfg kQbfCfgs[] = {{128, 128, 32, 1, 4}, {64, 128, 32, 1, 4}, {64, 64, 32, 1, 4}, {32, 64, 32, 1, 4},
                               {64, 64, 64, 1, 4},   {32, 64, 64, 1, 4},  {64, 64, 64, 2, 8}, {32, 64, 64, 2, 8},
                               {64, 128, 32, 1, 8},  {128, 128, 32, 1, 8}, {32, 64, 64, 2, 8}};
constexpr int kQbfNumCfgs = (int)(sizeof(kQbfCfgs) / sizeof(kQbfCfgs[0]));

template <int FMT>
void launch_qbf_cfg(int cfg, unsigned grid, const QbfArgs &a, hipStream_t s) {
    switch (cfg) {
        case 0: gemm_qbf_kernel<FMT, 128, 128, 64, 64, 2><<<grid, 256, 0, s>>>(a); break;
        case 1: gemm_qbf_kernel<FMT, 64, 128, 32, 64, 2><<<grid, 256, 0, s>>>(a); break;
        case 2: gemm_qbf_kernel<FMT, 64, 64, 32, 32, 4><<<grid, 256, 0, s>>>(a); break;
        case 3: gemm_qbf_kernel<FMT, 32, 64, 16, 32, 4><<<grid, 256, 0, s>>>(a); break;
        case 4: gemm_qbf_kernel<FMT, 64, 64, 32, 32, 2, 64><<<grid, 256, 0, s>>>(a); break;
        case 5: gemm_qbf_kernel<FMT, 32, 64, 16, 32, 2, 64><<<grid, 256, 0, s>>>(a); break;
        case 6: gemm_qbf_kernel<FMT, 64, 64, 32, 32, 2, 64, 2><<<grid, 512, 0, s>>>(a); break;
        case 7: gemm_qbf_kernel<FMT, 32, 64, 16, 32, 2, 64, 2><<<grid, 512, 0, s>>>(a); break;
        case 8: gemm_qbf_kernel<FMT, 64, 128, 32, 32, 2, 32, 1, 8><<<grid, 512, 0, s>>>(a); break;
        case 9: gemm_qbf_kernel<FMT, 128, 128, 64, 32, 2, 32, 1, 8><<<grid, 512, 0, s>>>(a); break;
        default: gemm_qbf_kernel<FMT, 32, 64, 16, 32, 4, 64, 2><<<grid, 512, 0, s>>>(a); break;
    }
}

}  // namespace

// Tile and K split: forced by TML_GEMM_QBF_TILE / TML_GEMM_QBF_SPLIT, else
//   * up to M = 512, where 32x64 tiles number at most four a CU: 64x64x64
//     or 32x64x64 with two wave groups and K split s in 1..4 of least
//     modelled time (see pick_qbf), fitted to a sweep of both tiles at
//     s = 1..4 over 45 shapes (M = 128, 192, 256, 384, 512; N x K = 4096 x
//     1024, 1024 x 4096, 768 x 3072, 3072 x 768, 1280 x 1280, 5120 x 1280,
//     1280 x 5120, 1536 x 384, 384 x 1536; every launch reading its own
//     weight copy; the 41 under the forced-plan size cap): its picks sum to
//     564.0 us against 553.9 for the best of each shape and 591.6 for the
//     rule before (the fewest splits giving every CU a unit); measured on
//     all 45 afterwards 677 against 723 us, e.g. 256x1024x4096 19.24 ->
//     16.46, 256x1280x5120 26.87 -> 21.81, 384x768x3072 18.73 -> 15.92,
//     512x1280x5120 46.34 -> 30.88 us (128x384x1536 9.08 -> 9.56 and
//     512x1280x1280 15.57 -> 16.74 the two that lost);
//   * else the eight-wave 64x128 or 128x128 tile (configs 8, 9) and K split
//     s in 1..4 (at least eight 32-deep slices a split; s > 1 only where the
//     tiles number fewer than the CUs) of least modelled time
//       t = u * ceil(slices / s) * c + 5.3 us + 1.7 us * (s - 1),
//       u = ceil(tiles s / CUs) units a CU,
//     c = 0.42 / 0.335 us a slice-unit at 64x128 for u = 1 / u >= 2 (three
//     workgroups share a CU), 0.78 / 0.59 at 128x128 (two share a CU), the
//     last term the partials and the reduce launch.  Fitted to a tile x
//     split sweep on MI355X (us, Q8_0, every launch reading its own weight
//     copy, 64x128 / 128x128 unsplit unless marked; the four-wave tiles of
//     the same shapes and the plan before in brackets): 1500x3840x1280
//     45.2 / 49.3 (48.9 / 60.2); 1500x5120x1280 59.7 / 53.5 (60.8 / 62.9);
//     1500x1280x5120 s = 2 62.6, 128x128 s = 4 58.2 (64.3); 1024x4096x1024
//     28.7 / 28.6 (32.0 / 42.0, plan 37.2); 2048x768x3072 64x128 s = 4 35.2
//     (36.5); 768x3072x768 20.7 / 23.3 (26.6); 1500x1536x384 13.3 / 15.5
//     (17.6); 3000x3840x1280 85.8 / 80.4 (88.7 / 105.5).  The model's pick
//     is the measured best on seven of the eight and 0.1 us off on the
//     eighth (1024x4096x1024).  Splitting tiles that already fill the CUs
//     costs far more than the reduce term (the partials' traffic, M N s 8
//     bytes, competes with the main loop): 128 x 128 at s = 2 measured
//     53.1 us at 1500x3840x1280, 67.6 at 1500x5120x1280 and 35.0 at
//     1024x4096x1024, 9-13 us above the model.
void pick_qbf(const MatmulArgs &m, GemmPlan *p) {
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
    }
    const int64_t nk = (m.K + 31) / 32;
    auto tiles_of = [&](int c) {
        return ((m.M + kQbfCfgs[c].bm - 1) / kQbfCfgs[c].bm) * ((m.N + kQbfCfgs[c].bn - 1) / kQbfCfgs[c].bn);
    };
    auto split_ok = [&](int64_t ns) {
        return ns == 1 || nk / ns >= 8;
    };
    int cfg = 8;
    int64_t nsplit = 1;
    // the modelled time of config c at s splits (the plan's own rounding of
    // the slices into whole BK-deep ones per split)
    auto modelled = [&](int c, int64_t ns, double c_one, double c_many, double per_split, double traffic) {
        const int64_t per = kQbfCfgs[c].bk / 32;
        const int64_t spl = ((nk + ns - 1) / ns + per - 1) / per * per;
        const int64_t real = (nk + spl - 1) / spl;
        const int64_t per_cu = (tiles_of(c) * real + cus - 1) / cus;
        double t = (double)per_cu * (double)(spl / per) * (per_cu > 1 ? c_many : c_one) + 5.3;
        if (real > 1) t += per_split * (double)(real - 1) + traffic * (double)real * (double)m.M * (double)m.N * 8.0 / 6.0e6;
        return t;
    };
    if (m.M < 128) {
        // 32 x 64 x 64 tiles with two wave groups (config 7) and the largest
        // K split s <= 4 that keeps tiles x s within the CUs and >= 8 32-deep
        // slices a split: the best plan of a 60-point sweep (M = 16-112 at
        // ten encoder / decoder shapes) within 3 % at all but two points
        // (e.g. 48 x 4096 x 1024 9.9 us, 16 x 4096 x 1024 8.6 us; the fp32
        // kernels took 17.5 and 10.2 us)
        cfg = 7;
        for (int64_t ns = 2; ns <= 4; ++ns)
            if (tiles_of(7) * ns <= cus && split_ok(ns)) nsplit = ns;
    } else if (m.M <= 512 && tiles_of(7) <= 4LL * cus) {
        // 64 x 64 x 64 or 32 x 64 x 64 tiles with two wave groups (configs 6,
        // 7) and K split s in 1..4 of least modelled time, c = 0.60 / 0.45 us
        // a 64-deep slice-unit at 64 x 64 for u = 1 / u >= 2, 0.35 / 0.25 at
        // 32 x 64, plus 1.0 us a split past the first and half the
        // partials' traffic at 6 TB/s
        // (a split that takes the units past the CUs needs >= 24 slices a
        // split: at 128 x 3840 x 1280, Q4_0 128 x 5120 x 1280 and 192 x 3840 x
        // 1280 the model's two splits measured 1.6-1.9 us above one)
        static const double c_one[] = {0.60, 0.35}, c_many[] = {0.45, 0.25};
        double best = 1e300;
        for (int i = 0; i < 2; ++i)
            for (int64_t ns = 1; ns <= 4 && split_ok(ns); ++ns) {
                if (ns > 1 && tiles_of(6 + i) * ns > cus && nk / ns < 24) continue;
                const double t = modelled(6 + i, ns, c_one[i], c_many[i], 1.0, 0.5);
                if (t < best) {
                    best = t;
                    cfg = 6 + i;
                    nsplit = ns;
                }
            }
    } else {
        static const int cand[] = {8, 9};
        static const double c_one[] = {0.42, 0.78}, c_many[] = {0.335, 0.59};
        double best = 1e300;
        for (int i = 0; i < 2; ++i)
            for (int64_t ns = 1; ns <= 4; ++ns) {
                // K splits only where the tiles leave CUs idle
                if (!split_ok(ns) || (ns > 1 && tiles_of(cand[i]) >= cus)) break;
                const double t = modelled(cand[i], ns, c_one[i], c_many[i], 1.7, 0.0);
                if (t < best) {
                    best = t;
                    cfg = cand[i];
                    nsplit = ns;
                }
            }
    }
    if (cfg == 7) {
        // Four 64-deep slices of loads in flight instead of two (config 10)
        // where every unit has a CU to itself and a split's steps fill whole
        // rounds of four, bar one: on a 60-point sweep (M = 16-256) this took
        // 128 x 4096 x 1024 from 10.42 to 9.92 us, 128 x 3840 x 1280 11.90 ->
        // 11.09, Q4_0 16 x 1280 x 5120 14.49 -> 13.84; with two CUs' worth of
        // units, or steps rounded up by two or three, it measured slower
        // (1536 x 384, 6 steps: 6.1 -> 6.5 us).
        const int64_t spl = ((nk + nsplit - 1) / nsplit + 1) / 2 * 2;
        const int64_t n64 = spl / 2, real = (nk + spl - 1) / spl;
        if (tiles_of(7) * real <= cus && n64 >= 7 && (n64 % 4 == 0 || n64 % 4 == 3)) cfg = 10;
    }
    const int forced_tile = env_int("TML_GEMM_QBF_TILE", 0) - 1;
    if (forced_tile >= 0 && forced_tile < kQbfNumCfgs) cfg = forced_tile;
    const int forced = env_int("TML_GEMM_QBF_SPLIT", 0);
    if (forced >= 1) nsplit = std::min<int64_t>(forced, nk);
    // 32-deep slices a split, whole slices of the config's depth
    const int64_t per = kQbfCfgs[cfg].bk / 32;
    int64_t spl = ((nk + nsplit - 1) / nsplit + per - 1) / per * per;
    nsplit = (nk + spl - 1) / spl;  // no split without slices
    p->cfg = cfg;
    p->nsplit = (int)nsplit;
    p->spl = (int)std::max<int64_t>(spl, 1);
    p->tiles = (int)tiles_of(cfg);
}

bool gemm_qbf_supported(const MatmulArgs &m) {
    if (m.fmt != TML_FMT_Q8_0 && m.fmt != TML_FMT_Q4_0) return false;
    if (m.M <= kGemvMaxM || m.K <= 0 || m.K % 8 != 0 || m.N % 2 != 0 || ((uintptr_t)m.A % 16) != 0) return false;
    if (env_int("TML_GEMM_QBF", 1) == 0) return false;
    // every buffer offset below 2^31: A rows up to M + 128, B k-rows up to K + 544
    const uint64_t lim = (uint64_t)1 << 31;
    const uint64_t ldb = m.fmt == TML_FMT_Q8_0 ? (uint64_t)m.N : (uint64_t)m.N / 2;
    // (the loads run up to 2 D slices of BK past K, zero-filled: 512 at D = 4, BK = 64)
    return (uint64_t)(m.M + 128) * (uint64_t)m.K * 4u < lim && (uint64_t)(m.K + 544) * ldb < lim &&
           m.M < ((int64_t)1 << 30) && m.N < ((int64_t)1 << 30);
}

Status launch_gemm_qbf(const MatmulArgs &m, const GemmPlan &p, const Workspace &ws, hipStream_t s) {
    if (!gemm_qbf_supported(m))
        return Status::Err(TML_ERR_INVALID_ARG, "bf16 matrix-core GEMM: needs Q8_0 / Q4_0, M > 8, K % 8 == 0, even N, "
                                                "16-byte aligned A");
    QbfArgs a;
    a.M = (int)m.M; a.N = (int)m.N; a.K = (int)m.K;
    a.A = m.A; a.B = (const uint8_t *)m.B;
    a.ldb = (int)(m.fmt == TML_FMT_Q8_0 ? m.N : m.N / 2);
    a.bias = m.bias; a.colscale = m.colscale; a.res = m.res; a.C = m.C;
    a.alpha = m.alpha_eff; a.beta = m.beta;
    a.act = m.act;
    a.tail0 = tml_act_tail0((long long)m.M * m.N);
    a.a_bytes = (unsigned)((uint64_t)m.M * (uint64_t)m.K * 4u);
    a.b_bytes = (unsigned)((uint64_t)m.K * (uint64_t)a.ldb);
    const int cfg = p.cfg;
    if (cfg < 0 || cfg >= kQbfNumCfgs) return Status::Err(TML_ERR_INVALID_ARG, "bf16 matrix-core GEMM: bad tile config");
    const int64_t nk = (m.K + 31) / 32;
    if (p.nsplit < 1 || p.spl < 1 || (int64_t)p.spl * p.nsplit < nk || (int64_t)p.spl * (p.nsplit - 1) >= nk)
        return Status::Err(TML_ERR_INVALID_ARG, "bf16 matrix-core GEMM: split plan does not cover K");
    if (p.nsplit > 1 && (ws.partials == nullptr || ws.partial_floats < (size_t)p.nsplit * (size_t)m.M * (size_t)m.N))
        return Status::Err(TML_ERR_INVALID_ARG, "bf16 matrix-core GEMM: split-K workspace too small");
    a.tiles_m = (int)((m.M + kQbfCfgs[cfg].bm - 1) / kQbfCfgs[cfg].bm);
    a.tiles_n = (int)((m.N + kQbfCfgs[cfg].bn - 1) / kQbfCfgs[cfg].bn);
    a.nsplit = p.nsplit;
    a.spl = p.spl;
    a.ws = p.nsplit > 1 ? ws.partials : nullptr;
    a.vec_epi = m.N % 4 == 0 && ((uintptr_t)m.C % 16) == 0 && (m.bias == nullptr || ((uintptr_t)m.bias % 16) == 0) &&
                (m.res == nullptr || ((uintptr_t)m.res % 16) == 0) &&
                (m.colscale == nullptr || ((uintptr_t)m.colscale % 16) == 0) && env_int("TML_GEMM_VEC_EPI", 1) != 0;
    const int64_t grid = (int64_t)a.tiles_m * a.tiles_n * p.nsplit;
    if (grid >= ((int64_t)1 << 31)) return Status::Err(TML_ERR_INVALID_SHAPE, "bf16 matrix-core GEMM: grid too large");
    if (m.fmt == TML_FMT_Q8_0) launch_qbf_cfg<TML_FMT_Q8_0>(cfg, (unsigned)grid, a, s);
    else launch_qbf_cfg<TML_FMT_Q4_0>(cfg, (unsigned)grid, a, s);
    TML_HIP_TRY(hipGetLastError());
    if (p.nsplit > 1) TML_TRY(launch_splitk_reduce(ws.partials, p.nsplit, m, s));
    return Status::Ok();
}

}  // namespace tml
