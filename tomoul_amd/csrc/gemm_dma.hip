// gemm_dma.hip -- fp32 SGEMM on gfx950 matrix cores with direct global->LDS
// loads (the ops.matmul / matmulBias path, src/core/ops.zig:235-471).
//
//   C[M,N] = alpha * A[M,K] . B[K,N] + beta * C + bias[N]
//
// Data path.  Each BK-deep slice (32 or 64) of the A and B tiles is copied
// from HBM/L2 straight into LDS with buffer_load_dwordx4 ... lds (no staging
// through VGPRs, no ds_write instructions), each operand through a buffer
// resource: a lane's 32-bit offset is fixed for the loop plus one uniform
// step per slice, and offsets past the operand read zeros.  Three LDS stages:
// while the waves run the MFMAs of slice t, the copies of slices t+1 and t+2
// are in flight.  A wave's copy instruction fills 1 KiB of LDS in lane
// order, so the tiles are stored unpadded and bank conflicts are avoided with
// XOR swizzles instead:
//   A stage [BM][BK]: 16-byte chunk q of row r sits in slot q ^ (r % 8), so the
//     per-lane 16-byte fragment reads of 8 consecutive rows hit 8 distinct
//     bank groups;
//   B stage [BK][BN]: 16-byte chunk c of k-row k sits in slot c ^ 4 when
//     (k / 4) is odd, so the lane groups reading rows k and k + 4 use opposite
//     halves of the banks.
// Synchronisation per slice: each wave waits for its own outstanding copies
// of the next slice (s_waitcnt vmcnt with an exact count), then a raw
// s_barrier makes every wave's copies visible.  __syncthreads() is not used in
// the loop: its release fence would wait for all copies in flight
// (vmcnt(0)) and serialise the pipeline.
//
// Compute: v_mfma_f32_16x16x4_f32, fp32 accumulation; lane l feeds A[l%16][kk]
// and B[kk][l%16] with kk = l/16 and holds D[4*(l/16)+r][l%16] in register r
// (for narrow B the 16 columns of a fragment are every other column of a
// 32-column group, see PAIR below);
// within a 16-deep chunk, step s feeds the physical k = 4*kk + s.  Fragment
// reads run one chunk ahead of the MFMAs and are issued between the two
// halves of the current chunk's MFMAs; the last chunk of a slice is
// multiplied after the barrier so that it covers the first reads of the next.
#include <type_traits>

#include "tml_internal.hpp"

namespace tml {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kNumXcd = 8;

struct DmaArgs {
    int M, N, K;
    const float *A;
    const void *B;        // [K,N] in the kernel's format
    long long ldb;        // bytes per row of B
    const float *bias;
    float *C;
    float alpha, beta;
    int tiles_m, tiles_n, group_m;
    int pm, pn, ps;       // XCD partition of (m-tiles, n-tiles, splits), pm*pn*ps = 8; pm = 0: none
    int nsplit, spl;      // K splits and BK-slices per split
    const float *colscale;  // [N] per-column factor on A.B, or nullptr
    const float *kscales;   // Q8_K: scale of element (k, n) at kscales[k * sld + n / 32]
    int sld;                // Q8_K: scale blocks per k-row (N / 32)
    float *ws;            // split partials: [split][M][N], or per tile in lane order when fused
    unsigned *counters;   // per-tile arrival counters (fused split-K), or nullptr
    const float *zero;
    int act;              // TML_ACT_* after the bias
    const float *res;     // [M,N] residual added after the bias, or nullptr
    long long tail0;      // tml_act_tail0(M * N)
    int vec_epi;          // N % 4 == 0 and C, bias, residual, column scales 16-byte aligned
};

#define TML_GPTR(p) ((__attribute__((address_space(1))) void *)(p))

// Buffer resource word 3 for raw (untyped, unswizzled) loads on gfx9 parts:
// DATA_FORMAT = 32 bits.  A lane offset at or past the resource's byte count
// reads zeros; kBufOutOfRange is such an offset for every resource here.
constexpr int kBufDword3 = 0x00020000;
constexpr unsigned kBufOutOfRange = 0x80000000u;

// 16 bytes at base + off (a buffer of nbytes) into this lane's slot of the
// 1 KiB LDS block at lds.  The resource is built from uniform values, so it
// lives in SGPRs and the compiler keeps it out of the loop.
__device__ __forceinline__ void buffer_copy16(const void *base, unsigned nbytes, unsigned off, void *lds) {
    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0,
                                                                       (int)nbytes, kBufDword3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void *)lds, 16, off, 0, 0, 0);
}
#define TML_LPTR(p) ((__attribute__((address_space(3))) void *)(p))

// s_waitcnt vmcnt(N) with the other counters left alone (gfx9 encoding:
// vmcnt[3:0] in bits 3:0, vmcnt[5:4] in bits 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}
__device__ __forceinline__ void wait_lgkmcnt0() {
    __builtin_amdgcn_s_waitcnt((0xF) | (0x3 << 14) | (0x7 << 4) | (0x0 << 8));
}
// Workgroup barrier without a memory fence; the empty asm with a memory
// clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void raw_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Bytes per B element as a fraction (int4: half a byte).
template <int FMT> struct BBytes;
template <> struct BBytes<TML_FMT_F32> { static constexpr int num = 4, den = 1; };
template <> struct BBytes<TML_FMT_F16> { static constexpr int num = 2, den = 1; };
template <> struct BBytes<TML_FMT_Q8_0> { static constexpr int num = 1, den = 1; };
template <> struct BBytes<TML_FMT_Q8_K> { static constexpr int num = 1, den = 1; };
template <> struct BBytes<TML_FMT_Q4_0> { static constexpr int num = 1, den = 2; };

// KW: wave groups splitting each slice's depth.  With KW = 2 the waves
// [0, NW/2) multiply the first half of every BK slice and [NW/2, NW) the
// second half, each wave on the same WM x WN sub-tile as its partner; the two
// accumulators are added through LDS before the epilogue.  Twice the waves
// per SIMD for the same tile, so one wave's LDS and barrier waits are covered
// by the other's MFMAs.
template <int FMT, int BM, int BN, int BK, int WM, int WN, int NW, int NS, int KW = 1>
__global__ __launch_bounds__(NW * 64) void gemm_dma_kernel(DmaArgs a) {
    static_assert(NS == 3 || NS == 4, "3 or 4 LDS stages");
    static_assert(BK == 32 || BK == 64, "slice depth");
    static_assert(KW == 1 || KW == 2, "one or two wave groups along K");
    constexpr int NC = BK / 16;
    constexpr int NCW = NC / KW;  // chunks of a slice multiplied by one wave
    constexpr int NWS = NW / KW;  // waves per group (one per sub-tile)
    constexpr int WAVES_N = BN / WN;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert((BM / WM) * (BN / WN) == NWS, "one wave of each group per WM x WN sub-tile");
    static_assert(NCW % 2 == 0, "fragment double-buffering alternates two buffers over a wave's chunks");
    static_assert(KW == 1 || BN <= BK, "the groups' accumulators are exchanged through one A stage");
    // 1 KiB copy blocks per stage and their shapes.
    constexpr int SLOTS_A = BK / 4;             // 16-byte slots per A row (8 or 16)
    constexpr int ROWS_A = 64 / SLOTS_A;        // A rows per copy block (8 or 4)
    constexpr int BLKS_A = BM * BK / 256;       // copy blocks per A stage
    constexpr int BNUM = BBytes<FMT>::num, BDEN = BBytes<FMT>::den;
    constexpr int BNB = BN * BNUM / BDEN;       // bytes per B k-row in LDS
    constexpr int SLOTS_B = BNB / 16;           // 16-byte slots per B k-row
    constexpr int ROWS_B = 64 / SLOTS_B;        // B k-rows per copy block
    constexpr int BLKS_B = BK * BNB / 1024;     // copy blocks per B stage
    // Slot XOR for k-rows with odd k/4: the 16 lanes of a group read 16*BNUM/BDEN
    // bytes of one k-row, so shift odd k/4 rows by that many slots (0 for int4,
    // whose 8 bytes per group never collide with the neighbouring group's).
    constexpr int XS = BNUM / BDEN;
    static_assert(SLOTS_A == 8 || SLOTS_A == 16, "A swizzle permutes the low 3 bits of the slot");
    static_assert(SLOTS_B >= 2 && 64 % SLOTS_B == 0 && (BK * BNB) % 1024 == 0, "B stage: whole 1 KiB copy blocks");
    static_assert(BLKS_A % NW == 0, "A copy blocks must split evenly over the waves");
    // B copy blocks go round robin over the waves; when they do not split
    // evenly the first BLKS_B % NW waves copy one more per slice.
    constexpr int BPW = (BLKS_B + NW - 1) / NW;
    constexpr int LPW = BLKS_A / NW + BLKS_B / NW;          // copies per wave per slice
    constexpr int LPW_HI = LPW + (BLKS_B % NW != 0 ? 1 : 0);  // ... for waves with an extra B block
    // Q8_K: the slice's block scales, BK k-rows x BN/32 blocks, stored
    // [block][k] in LDS, copied 4 bytes a lane by the last wave (never one
    // with an extra B block) in SCI instructions.
    constexpr bool KS = FMT == TML_FMT_Q8_K;
    static_assert(!KS || BN % 32 == 0, "Q8_K tiles hold whole 32-column scale blocks");
    constexpr int SCN = KS ? BK * (BN / 32) : 0;
    constexpr int SCI = (SCN + 63) / 64;
    constexpr int LPW_S = LPW + SCI;  // copies per slice of the wave that also copies the scales

    __shared__ __attribute__((aligned(1024))) float As0[BM * BK], As1[BM * BK], As2[BM * BK];
    __shared__ __attribute__((aligned(1024))) float Bs0[BK * BNB / 4], Bs1[BK * BNB / 4], Bs2[BK * BNB / 4];
    __shared__ __attribute__((aligned(1024))) float As3[NS > 3 ? BM * BK : 4], Bs3[NS > 3 ? BK * BNB / 4 : 4];
    __shared__ __attribute__((aligned(16))) float Ss0[KS ? SCI * 64 : 4], Ss1[KS ? SCI * 64 : 4],
        Ss2[KS ? SCI * 64 : 4], Ss3[KS && NS > 3 ? SCI * 64 : 4];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kg = wave / NWS;        // wave group: chunks [kg * NCW, (kg + 1) * NCW) of each slice
    const int sw = wave % NWS;        // sub-tile of the wave
    const int wm0 = (sw / WAVES_N) * WM;
    const int wn0 = (sw % WAVES_N) * WN;
    const int c0 = kg * NCW;

    // Workgroup -> (tile, split).  Workgroups are dispatched to the 8 XCDs
    // round robin (id % 8), each XCD with its own L2.
    const int nblk = gridDim.x;
    const int b = blockIdx.x;
    const int xcd = b % kNumXcd, idx = b / kNumXcd;
    int tile_m, tile_n, split;
    if (a.pm > 0) {
        // XCD partition: XCD x owns one block of (m-tiles x n-tiles x
        // splits), chosen by the host so that the A rows and B columns one
        // XCD reads are as few bytes as possible; every operand byte then
        // crosses into at most the XCDs that need it.
        const int lm = a.tiles_m / a.pm, ln = a.tiles_n / a.pn, ls = a.nsplit / a.ps;
        const int pz = xcd % a.ps, py = (xcd / a.ps) % a.pn, px = xcd / (a.ps * a.pn);
        const int sp = idx / (lm * ln), r = idx % (lm * ln);
        tile_m = px * lm + r % lm;
        tile_n = py * ln + r / lm;
        split = pz * ls + sp;
    } else {
        // Consecutive ids per XCD, then GROUP_M swizzle; the K splits of one
        // tile are adjacent ids, so they run on one XCD.
        const int per = nblk / kNumXcd, rem = nblk % kNumXcd;
        const int lin = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
        split = lin % a.nsplit;
        const int tlin = lin / a.nsplit;
        const int group = a.group_m * a.tiles_n;
        const int first_m = (tlin / group) * a.group_m;
        const int gsize = min(a.tiles_m - first_m, a.group_m);
        tile_m = first_m + (tlin % group) % gsize;
        tile_n = (tlin % group) / gsize;
    }
    const int m0 = tile_m * BM;
    const int n0 = tile_n * BN;

    // ---- per-lane copy sources, see the layout notes above.  A and B are
    // read through buffer resources (base + byte count in SGPRs) with a
    // 32-bit per-lane byte offset fixed for the whole loop; each slice adds
    // one uniform step to it (one v_add per copy).  The hardware returns
    // zeros for offsets at or past the byte count, which covers A rows >= M
    // and B k-rows >= K without a select.  The host keeps every offset
    // below 2^31 (gemm_dma_supported).  Per-slice 64-bit address arithmetic
    // and zero-block selects measured 2-5 us per headline GEMM.
    const unsigned a_bytes = (unsigned)a.M * (unsigned)a.K * 4u, b_bytes = (unsigned)a.K * (unsigned)a.ldb;
    unsigned a_off0[BLKS_A / NW];  // byte offset of the lane's A chunk at k0 = 0
    int a_col[BLKS_A / NW];
#pragma unroll
    for (int i = 0; i < BLKS_A / NW; ++i) {
        const int blk = wave + i * NW;
        const int row = blk * ROWS_A + lane / SLOTS_A;
        const int q = (lane % SLOTS_A) ^ (row % 8);
        a_col[i] = q * 4;
        a_off0[i] = ((unsigned)(m0 + row) * (unsigned)a.K + (unsigned)a_col[i]) * 4u;
    }
    const bool extra_b = (BLKS_B % NW) != 0 && wave < BLKS_B % NW;
    unsigned b_off0[BPW];  // byte offset of the lane's B chunk at k0 = 0
#pragma unroll
    for (int i = 0; i < BPW; ++i) {
        const int blk = wave + i * NW;
        const int krow = blk * ROWS_B + lane / SLOTS_B;
        const int q = (lane % SLOTS_B) ^ (((krow >> 2) & 1) * XS);
        // columns past N (N is a whole number of 16-byte chunks) read bytes
        // of the next k-row: they only feed outputs the epilogue drops
        b_off0[i] = (unsigned)krow * (unsigned)a.ldb + (unsigned)(n0 * BNUM / BDEN) + (unsigned)(q * 16);
    }
    const bool scale_wave = KS && wave == NW - 1;
    auto issue = [&](float *as, float *bs, float *ss, int k0) __attribute__((always_inline)) {
#pragma unroll
        for (int i = 0; i < BLKS_A / NW; ++i) {
            // k >= K inside a row would read the next row: point it past
            // the end instead, so the padded product is 0 * 0, never 0 * inf
            const unsigned off = a_col[i] < a.K - k0 ? a_off0[i] + (unsigned)k0 * 4u : kBufOutOfRange;
            buffer_copy16(a.A, a_bytes, off, as + (wave + i * NW) * 256);
        }
        const unsigned kstep = (unsigned)k0 * (unsigned)a.ldb;
#pragma unroll
        for (int i = 0; i < BPW; ++i) {
            const int blk = wave + i * NW;
            if (BLKS_B % NW == 0 || blk < BLKS_B)  // uniform per wave
                buffer_copy16(a.B, b_bytes, b_off0[i] + kstep, bs + blk * 256);
        }
        if constexpr (KS) {
            if (scale_wave) {
#pragma unroll
                for (int ci = 0; ci < SCI; ++ci) {
                    const int l = lane + 64 * ci;
                    const int nb = l / BK, k = l % BK;
                    const bool in = l < SCN && k0 + k < a.K && n0 / 32 + nb < a.sld;
                    const float *src = in ? a.kscales + (size_t)(k0 + k) * a.sld + n0 / 32 + nb : a.zero;
                    __builtin_amdgcn_global_load_lds(TML_GPTR(src), TML_LPTR(ss + ci * 64), 4, 0, 0);
                }
            }
        }
    };

    // ---- fragments
    // Narrow formats keep the B elements as read from LDS (raw bits) until
    // the chunk that uses them: widening right after the read would make the
    // compiler wait for the LDS reads there, between the two MFMA halves.
    struct Frag {
        floatx4 a[TM];
        float b[TN][4];
        uint32_t braw[TN][4];
        floatx4 sc[KS ? TN : 1];  // Q8_K: the scales of b's four k
    };
    const int lrow = lane & 15;
    const int g = lane >> 4;  // lane group: feeds kk = g
    int a_off[TM];            // float offset of the lane's A row (chunk added per read)
#pragma unroll
    for (int i = 0; i < TM; ++i) a_off[i] = (wm0 + i * 16 + lrow) * BK;
    // Narrow B with an even number of 16-column fragments pairs them:
    // fragments 2p and 2p + 1 take the even and odd columns of the wave's
    // p-th 32-column group, so lane lrow feeds the adjacent columns
    // wn0 + 32p + 2 lrow and + 1, which one LDS read returns (2 bytes of
    // int8, 4 of f16, 1 of int4) instead of two.  The epilogue maps
    // fragment j back to its columns (bcol).
    constexpr bool PAIR = FMT != TML_FMT_F32 && TN % 2 == 0;
    constexpr int NRD = PAIR ? TN / 2 : TN;  // B reads per (k, lane)
    auto bcol = [&](int j) __attribute__((always_inline)) {
        return PAIR ? wn0 + 32 * (j / 2) + 2 * lrow + (j % 2) : wn0 + j * 16 + lrow;
    };
    int b_off[NRD];           // swizzled byte offset of the lane's B element(s) within a k-row
#pragma unroll
    for (int j = 0; j < NRD; ++j) {
        const int nb = (PAIR ? wn0 + 32 * j + 2 * lrow : wn0 + j * 16 + lrow) * BNUM / BDEN;
        b_off[j] = (((nb >> 4) ^ ((g & 1) * XS)) << 4) | (nb & 15);
    }
    const int nib = (lrow & 1) * 4;  // int4 unpaired: odd columns sit in the high nibble (N and n0 are even)
    const int aswz = lrow & 7;
    auto read_frag = [&](Frag &f, const float *as, const float *bs, const float *ss, int chunk)
                         __attribute__((always_inline)) {
        const int q = chunk * 4 + g;
        if constexpr (KS) {
            // fragment j's 16 columns lie in one scale block of 32
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int blk = (PAIR ? wn0 + 32 * (j / 2) : wn0 + j * 16) / 32;
                f.sc[j] = *(const floatx4 *)&ss[blk * BK + chunk * 16 + g * 4];
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i) f.a[i] = *(const floatx4 *)&as[a_off[i] + ((q ^ aswz) << 2)];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int k = chunk * 16 + g * 4 + s;
#pragma unroll
            for (int j = 0; j < NRD; ++j) {
                const uint8_t *bp = (const uint8_t *)bs + k * BNB + b_off[j];
                if constexpr (FMT == TML_FMT_F32) f.b[j][s] = *(const float *)bp;
                else if constexpr (PAIR) {
                    // both columns' raw bits; split in widen()
                    if constexpr (FMT == TML_FMT_F16) f.braw[j][s] = *(const uint32_t *)bp;
                    else if constexpr (FMT == TML_FMT_Q4_0) f.braw[j][s] = *bp;
                    else f.braw[j][s] = *(const uint16_t *)bp;
                } else if constexpr (FMT == TML_FMT_F16) f.braw[j][s] = *(const uint16_t *)bp;
                else if constexpr (FMT == TML_FMT_Q8_0 || FMT == TML_FMT_Q8_K)
                    f.braw[j][s] = (uint32_t)(int32_t)*(const int8_t *)bp;
                else f.braw[j][s] = *bp;
            }
        }
    };
    auto widen = [&](Frag &f) __attribute__((always_inline)) {
        if constexpr (PAIR) {
#pragma unroll
            for (int p = 0; p < NRD; ++p)
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const uint32_t r = f.braw[p][s];
                    float lo, hi;  // the even and the odd column
                    if constexpr (FMT == TML_FMT_F16) {
                        lo = tml_half_bits(r & 0xFFFFu);
                        hi = tml_half_bits(r >> 16);
                    } else if constexpr (FMT == TML_FMT_Q4_0) {
                        lo = (float)((int32_t)(r << 28) >> 28);
                        hi = (float)((int32_t)(r << 24) >> 28);
                    } else {
                        lo = (float)((int32_t)(r << 24) >> 24);
                        hi = (float)((int32_t)(r << 16) >> 24);
                    }
                    if constexpr (FMT == TML_FMT_Q8_K) {
                        // reference dequantization: f32(q) * scale, rounded per element
                        lo *= f.sc[2 * p][s];
                        hi *= f.sc[2 * p + 1][s];
                    }
                    f.b[2 * p][s] = lo;
                    f.b[2 * p + 1][s] = hi;
                }
        } else if constexpr (FMT != TML_FMT_F32) {
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const uint32_t r = f.braw[j][s];
                    if constexpr (FMT == TML_FMT_F16) f.b[j][s] = tml_half_bits(r);
                    else if constexpr (FMT == TML_FMT_Q8_0) f.b[j][s] = (float)(int32_t)r;
                    // reference dequantization: f32(q) * scale, rounded per element
                    else if constexpr (FMT == TML_FMT_Q8_K) f.b[j][s] = (float)(int32_t)r * f.sc[j][s];
                    else f.b[j][s] = (float)((int32_t)(r << (28 - nib)) >> 28);
                }
        }
    };

    floatx4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = floatx4{0.f, 0.f, 0.f, 0.f};
    // Half h of a chunk's MFMAs: k-steps s = 2h, 2h + 1.
    auto mma_half = [&](const Frag &f, int h) __attribute__((always_inline)) {
#pragma unroll
        for (int s = 2 * h; s < 2 * h + 2; ++s)
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(f.a[i][s], f.b[j][s], acc[i][j], 0, 0, 0);
    };

    // Stage buffers are selected at compile time (stage S of a step is a
    // template constant) so the compiler can tell which LDS array each copy
    // writes and never waits for copies into other stages.
    auto stage_a = [&](auto S) -> float * {
        if constexpr (decltype(S)::value == 0) return As0;
        else if constexpr (decltype(S)::value == 1) return As1;
        else if constexpr (decltype(S)::value == 2) return As2;
        else return As3;
    };
    auto stage_b = [&](auto S) -> float * {
        if constexpr (decltype(S)::value == 0) return Bs0;
        else if constexpr (decltype(S)::value == 1) return Bs1;
        else if constexpr (decltype(S)::value == 2) return Bs2;
        else return Bs3;
    };
    auto stage_s = [&](auto S) -> float * {
        if constexpr (decltype(S)::value == 0) return Ss0;
        else if constexpr (decltype(S)::value == 1) return Ss1;
        else if constexpr (decltype(S)::value == 2) return Ss2;
        else return Ss3;
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    using S2 = std::integral_constant<int, 2>;
    using S3 = std::integral_constant<int, 3>;

    // This workgroup's slices: [ks0, ks0 + nk) of the K dimension.
    const int ks0 = split * a.spl;
    const int nk = min((a.K + BK - 1) / BK - ks0, a.spl);
    if (nk > 0) {
        Frag f[2];
        // Prologue: slices 0 .. NS-2 in flight, slice 0 landed.
        issue(As0, Bs0, Ss0, ks0 * BK);
        issue(As1, Bs1, Ss1, (ks0 + min(1, nk - 1)) * BK);
        if constexpr (NS > 3) issue(As2, Bs2, Ss2, (ks0 + min(2, nk - 1)) * BK);
        // own copies of slice 0 landed
        if (extra_b) wait_vmcnt<LPW_HI * (NS - 2)>();
        else if (scale_wave) wait_vmcnt<LPW_S * (NS - 2)>();
        else wait_vmcnt<LPW * (NS - 2)>();
        raw_barrier();                  // everyone's copies of slice 0 landed
        read_frag(f[0], As0, Bs0, Ss0, c0);

        // One slice: stage S holds slice kt; stage S-1 (mod NS, slice kt-1,
        // fully read before the previous barrier) receives slice kt+NS-1.
        // Slice indices past the end are clamped to the last slice (repeat
        // copies into stages nobody reads again), and the MFMAs of steps past
        // the end are skipped, so every step runs the same memory operations.
        auto step = [&](int kt, auto S) __attribute__((always_inline)) {
            constexpr int s = decltype(S)::value;
            using SN = std::integral_constant<int, (s + 1) % NS>;
            using SF = std::integral_constant<int, (s + NS - 1) % NS>;
            const bool live = kt < nk;
            issue(stage_a(SF{}), stage_b(SF{}), stage_s(SF{}), (ks0 + min(kt + NS - 1, nk - 1)) * BK);
            // Chunk c's fragments sit in f[c % 2].  The reads of the next
            // chunk go between the two halves of chunk c's MFMAs: while copies
            // to LDS are in flight the compiler can only wait for LDS reads
            // with lgkmcnt(0), so the next wait must find nothing recent.
#pragma unroll
            for (int c = 0; c < NCW; ++c) {
                Frag &cur = f[c % 2];
                Frag &nxt = f[(c + 1) % 2];
                if (c + 1 == NCW) {
                    // own copies of slice kt+1 landed
                    if (extra_b) wait_vmcnt<LPW_HI * (NS - 2)>();
                    else if (scale_wave) wait_vmcnt<LPW_S * (NS - 2)>();
                    else wait_vmcnt<LPW * (NS - 2)>();
                    wait_lgkmcnt0();               // own reads of slice kt done before anyone overwrites it
                    raw_barrier();
                }
                __builtin_amdgcn_sched_barrier(0);
                widen(cur);
                if (live) mma_half(cur, 0);
                __builtin_amdgcn_sched_barrier(0);
                if (c + 1 < NCW) read_frag(nxt, stage_a(S), stage_b(S), stage_s(S), c0 + c + 1);
                else read_frag(nxt, stage_a(SN{}), stage_b(SN{}), stage_s(SN{}), c0);
                __builtin_amdgcn_sched_barrier(0);
                if (live) mma_half(cur, 1);
                __builtin_amdgcn_sched_barrier(0);
            }
        };
        for (int kt = 0; kt < nk; kt += NS) {
            step(kt, S0{});
            step(kt + 1, S1{});
            step(kt + 2, S2{});
            if constexpr (NS > 3) step(kt + 3, S3{});
        }
        wait_vmcnt<0>();  // no copy may still be landing when the waves retire
    }

    if constexpr (KW > 1) {
        // Group 1 hands its accumulators to group 0 through A stage 0: every
        // wave's copies have landed (vmcnt(0) above) and its reads are done
        // before the barrier, so nobody touches the stages any more.
        float *xb = As0 + sw * (TM * TN * 4 * 64) + lane;
        wait_lgkmcnt0();
        raw_barrier();
        if (kg == 1) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
#pragma unroll
                    for (int r = 0; r < 4; ++r) xb[((i * TN + j) * 4 + r) * 64] = acc[i][j][r];
        }
        wait_lgkmcnt0();
        raw_barrier();
        if (kg != 0) return;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) acc[i][j][r] += xb[((i * TN + j) * 4 + r) * 64];
    }

    const int rq = g * 4;
    if (a.nsplit > 1 && a.counters != nullptr) {
        // Fused split-K: each split stores its raw partial in lane order
        // (store i of every thread is one contiguous NT-float run), the last
        // split to arrive at the tile's counter sums all splits in split
        // order -- the order splitk_reduce_kernel uses, so the result is the
        // same bit for bit -- and runs the epilogue.  The exchange uses
        // agent-scope stores / loads, no device-wide fence.
        constexpr int NT = NW * 64;
        constexpr int TF = TM * TN * 4;
        constexpr int XB = 4;  // splits whose partials are loaded at once
        __shared__ unsigned xslot;
        const int tile = tile_m * a.tiles_n + tile_n;
        float *base = a.ws + (size_t)tile * a.nsplit * (NT * TF);
        float *mine = base + (size_t)split * (NT * TF);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) xchg_store(mine + ((i * TN + j) * 4 + r) * NT + tid, acc[i][j][r]);
        const unsigned arrived = xchg_arrive(a.counters + tile, &xslot);
        if (arrived != (unsigned)(a.nsplit - 1)) return;
        floatx4 sum[TM][TN];
        for (int s0 = 0; s0 < a.nsplit; s0 += XB) {
            float t[XB][TF];
#pragma unroll
            for (int x = 0; x < XB; ++x) {
                const int sp = min(s0 + x, a.nsplit - 1);
                const float *src = base + (size_t)sp * (NT * TF) + tid;
#pragma unroll
                for (int e = 0; e < TF; ++e) t[x][e] = (sp == split) ? 0.0f : xchg_load(src + e * NT);
            }
#pragma unroll
            for (int x = 0; x < XB; ++x) {
                const int sp = s0 + x;
                if (sp >= a.nsplit) break;
#pragma unroll
                for (int i = 0; i < TM; ++i)
#pragma unroll
                    for (int j = 0; j < TN; ++j) {
                        floatx4 v;
#pragma unroll
                        for (int r = 0; r < 4; ++r) v[r] = (sp == split) ? acc[i][j][r] : t[x][(i * TN + j) * 4 + r];
                        if (sp == 0) sum[i][j] = v;
                        else sum[i][j] += v;
                    }
            }
        }
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) acc[i][j] = sum[i][j];
        xchg_reset(a.counters + tile);
    } else if (a.nsplit > 1) {
        // Split-K: store the raw partial of this split into ws[split][M][N];
        // splitk_reduce_kernel (launched next on the same stream) sums the
        // splits in order and applies the epilogue.
        float *part = a.ws + (size_t)split * a.M * a.N;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                const int col = n0 + bcol(j);
                if (col >= a.N) continue;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = m0 + wm0 + i * 16 + rq + r;
                    if (row < a.M) part[(size_t)row * a.N + col] = acc[i][j][r];
                }
            }
        return;
    }

    {
        if (a.vec_epi) {
            // Staged epilogue: the tile goes through LDS (A stage 0, free once
            // every wave has read its last slice) in passes of PW columns (the
            // stage holds BM x BK floats) and is written as whole 16-byte
            // pieces of C rows, a pass's PW floats of a row (128 or 256 bytes:
            // whole cache lines) by consecutive lanes of one store instruction,
            // instead of 4-byte stores of 16-column strips (config 1: 20.34
            // against 20.58 us; with the non-temporal stores the strips left
            // half lines that cost 17 % more HBM writes at the headline).
            // With two wave groups only group 0 is left (group 1 ended after
            // the exchange, and the barriers count the waves still running);
            // BN <= BK there, so the tile is one pass.
            constexpr int PW = BN < BK ? BN : BK;
            static_assert(BN % PW == 0 && PW % 16 == 0, "passes of whole 16-column fragment blocks");
            constexpr int CH = PW / 4;  // 16-byte pieces per pass row
            float *ct = As0;
#pragma unroll
            for (int pass = 0; pass < BN / PW; ++pass) {
                wait_lgkmcnt0();
                raw_barrier();
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    // the fragment's 16- (32- when paired) column block lies
                    // in one pass; the test is uniform over the wave
                    const int cb = PAIR ? wn0 + 32 * (j / 2) : wn0 + 16 * j;
                    if (cb / PW != pass) continue;
#pragma unroll
                    for (int i = 0; i < TM; ++i)
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            ct[(wm0 + i * 16 + rq + r) * PW + bcol(j) - pass * PW] = acc[i][j][r];
                }
                wait_lgkmcnt0();
                raw_barrier();
#pragma unroll
                for (int e = tid; e < BM * CH; e += NWS * 64) {
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
    }

    // Epilogue: C = alpha * acc + beta * C + bias, bounds-checked.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + bcol(j);
            if (col >= a.N) continue;
            const float biasc = a.bias ? a.bias[col] : 0.0f;
            const float acol = a.colscale ? a.alpha * a.colscale[col] : a.alpha;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = m0 + wm0 + i * 16 + rq + r;
                if (row < a.M) {
                    float *cp = a.C + (size_t)row * a.N + col;
                    float v = acol * acc[i][j][r];
                    if (a.beta != 0.0f) v += a.beta * *cp;
                    if (a.bias) v += biasc;
                    const long long flat = (long long)row * a.N + col;
                    if (a.res) v += a.res[flat];
                    tml_store_c(cp, tml_apply_act(v, a.act, flat, a.tail0));
                }
            }
        }
}

// C = act(alpha * sum_s ws[s] + beta * C + bias) over the M*N outputs, the
// splits summed in order (deterministic).  Four outputs per thread when
// aligned.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float *__restrict__ ws, int nsplit, long long mn,
                                                            int n, float *C, float alpha, float beta,
                                                            const float *__restrict__ bias,
                                                            const float *res, const float *colscale, bool vec,
                                                            int act, long long tail0) {
    const long long stride = (long long)gridDim.x * blockDim.x;
    if (vec) {
        for (long long q = (long long)blockIdx.x * blockDim.x + threadIdx.x; q < mn / 4; q += stride) {
            floatx4 acc = *(const floatx4 *)(ws + 4 * q);
            for (int s = 1; s < nsplit; ++s) acc += *(const floatx4 *)(ws + (size_t)s * mn + 4 * q);
            floatx4 v = alpha * acc;
            if (colscale) v = (alpha * *(const floatx4 *)(colscale + (4 * q) % n)) * acc;
            float *cp = C + 4 * q;
            if (beta != 0.0f) v += beta * *(const floatx4 *)cp;
            if (bias) v += *(const floatx4 *)(bias + (4 * q) % n);
            if (res) v += *(const floatx4 *)(res + 4 * q);
            if (act != TML_ACT_NONE)
#pragma unroll
                for (int r = 0; r < 4; ++r) v[r] = tml_apply_act(v[r], act, 4 * q + r, tail0);
            tml_store_c(cp, v);
        }
    } else {
        for (long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x; e < mn; e += stride) {
            float acc = ws[e];
            for (int s = 1; s < nsplit; ++s) acc += ws[(size_t)s * mn + e];
            float v = (colscale ? alpha * colscale[e % n] : alpha) * acc;
            if (beta != 0.0f) v += beta * C[e];
            if (bias) v += bias[e % n];
            if (res) v += res[e];
            tml_store_c(C + e, tml_apply_act(v, act, e, tail0));
        }
    }
}

struct DmaCfg {
    int bm, bn, bk, kw;  // kw: wave groups along K (gemm_dma_kernel's KW)
};
// Tile configs (index = TML_GEMM_DMA_TILE - 1); see launch_gemm_f32_dma for
// the wave tiling and LDS stages of each.
constexpr DmaCfg kDmaCfgs[] = {{128, 128, 32, 1}, {128, 64, 32, 1}, {64, 64, 32, 1}, {256, 128, 32, 1},
                               {128, 64, 64, 1},  {64, 64, 64, 1},  {32, 64, 32, 1}, {32, 64, 64, 1},
                               {96, 32, 32, 1},   {32, 64, 64, 2},  {32, 32, 64, 2}};

}  // namespace

int gemm_dma_num_cfgs() { return (int)(sizeof(kDmaCfgs) / sizeof(kDmaCfgs[0])); }

// Configs whose two wave groups add their accumulators in the workgroup
// cannot take the fused split-K exchange (every thread stores its partial).
bool gemm_dma_cfg_fusable(int cfg) { return cfg >= 0 && cfg < gemm_dma_num_cfgs() && kDmaCfgs[cfg].kw == 1; }

bool gemm_dma_cfg_ok(int cfg, int fmt) {
    if (cfg < 0 || cfg >= gemm_dma_num_cfgs()) return false;
    const int bn = kDmaCfgs[cfg].bn;
    return fmt != TML_FMT_Q4_0 || bn >= 64;  // a k-row of int4 B holds >= 32 bytes
}

void gemm_dma_tile(int cfg, int *bm, int *bn, int *bk) {
    *bm = kDmaCfgs[cfg].bm;
    *bn = kDmaCfgs[cfg].bn;
    *bk = kDmaCfgs[cfg].bk;
}

static size_t weight_row_bytes(int fmt, int64_t N) {
    switch (fmt) {
        case TML_FMT_F32: return (size_t)N * 4;
        case TML_FMT_F16: return (size_t)N * 2;
        case TML_FMT_Q4_0: return (size_t)N / 2;
        default: return (size_t)N;
    }
}

template <int FMT>
static Status launch_dma_cfg(int cfg, dim3 grid, const DmaArgs &a, hipStream_t s) {
    switch (cfg) {
        // <format, BM, BN, BK, WM, WN, waves, LDS stages>
        case 0: gemm_dma_kernel<FMT, 128, 128, 32, 64, 32, 8, 3><<<grid, 512, 0, s>>>(a); break;
        case 1: gemm_dma_kernel<FMT, 128, 64, 32, 32, 32, 8, 3><<<grid, 512, 0, s>>>(a); break;
        case 2: gemm_dma_kernel<FMT, 64, 64, 32, 32, 32, 4, 3><<<grid, 256, 0, s>>>(a); break;
        case 3: gemm_dma_kernel<FMT, 256, 128, 32, 64, 64, 8, 3><<<grid, 512, 0, s>>>(a); break;
        case 4: gemm_dma_kernel<FMT, 128, 64, 64, 32, 32, 8, 3><<<grid, 512, 0, s>>>(a); break;
        case 5: gemm_dma_kernel<FMT, 64, 64, 64, 32, 32, 4, 3><<<grid, 256, 0, s>>>(a); break;
        case 6: gemm_dma_kernel<FMT, 32, 64, 32, 16, 32, 4, 3><<<grid, 256, 0, s>>>(a); break;
        case 7: gemm_dma_kernel<FMT, 32, 64, 64, 16, 32, 4, 3><<<grid, 256, 0, s>>>(a); break;
        case 9: gemm_dma_kernel<FMT, 32, 64, 64, 16, 32, 8, 3, 2><<<grid, 512, 0, s>>>(a); break;
        case 10:
            if constexpr (FMT != TML_FMT_Q4_0) {
                gemm_dma_kernel<FMT, 32, 32, 64, 16, 16, 8, 3, 2><<<grid, 512, 0, s>>>(a);
                break;
            } else {
                return Status::Err(TML_ERR_INVALID_ARG, "dma GEMM tile 32x32 has no int4 variant");
            }
        case 8:
            // 32 int4 columns are 16 bytes a k-row: less than a copy block's two slots
            if constexpr (FMT != TML_FMT_Q4_0) {
                gemm_dma_kernel<FMT, 96, 32, 32, 48, 16, 4, 3><<<grid, 256, 0, s>>>(a);
                break;
            } else {
                return Status::Err(TML_ERR_INVALID_ARG, "dma GEMM tile 96x32 has no int4 variant");
            }
        default: return Status::Err(TML_ERR_INVALID_ARG, "bad dma GEMM config");
    }
    return Status::Ok();
}

// XCD partition for the tile grid: the (pm, pn, ps) with pm * pn * ps = 8
// that divide (tiles_m, tiles_n, nsplit) exactly and minimise the A rows
// plus B columns one XCD reads, weighted by its share of K.  pm = 0 when
// none divides, or when a workgroup's K range is at most 512 (the partition
// serves L2 reuse across a long K loop; at short K the consecutive-id mapping
// measured faster: config 1's 1500x1536x384 18.77 against 19.03 us, three
// runs each, 512x384x384 7.46 against 7.73), or TML_GEMM_XCDPART=0; =1 takes
// it at any K.  The fused split-K exchange keeps its splits on one XCD, so
// ps = 1 there.
void pick_xcd_partition(int tiles_m, int tiles_n, int nsplit, int bm, int bn, bool fused, int64_t k_per_split,
                        int *pm, int *pn, int *ps) {
    *pm = *pn = *ps = 0;
    const int mode = env_int("TML_GEMM_XCDPART", -1);
    if (mode == 0 || (mode < 0 && k_per_split <= 512)) return;
    double best = 1e300;
    for (int x = 1; x <= kNumXcd; x *= 2)
        for (int y = 1; x * y <= kNumXcd; y *= 2) {
            const int z = kNumXcd / (x * y);
            if (tiles_m % x || tiles_n % y || nsplit % z || (fused && z != 1)) continue;
            const double cost = ((double)(tiles_m / x) * bm + (double)(tiles_n / y) * bn) / z;
            if (cost < best) {
                best = cost;
                *pm = x;
                *pn = y;
                *ps = z;
            }
        }
}

void gemm_dma_workspace_need(const MatmulArgs &m, const GemmPlan &p, size_t *partial_floats, size_t *counters) {
    *partial_floats = 0;
    *counters = 0;
    if (p.nsplit <= 1) return;
    const int bm = kDmaCfgs[p.cfg].bm, bn = kDmaCfgs[p.cfg].bn;
    const size_t tiles = (size_t)((m.M + bm - 1) / bm) * (size_t)((m.N + bn - 1) / bn);
    if (p.fused) {
        *partial_floats = tiles * (size_t)p.nsplit * (size_t)bm * bn;
        *counters = tiles;
    } else {
        *partial_floats = (size_t)p.nsplit * m.M * m.N;
    }
}

bool gemm_dma_supported(const MatmulArgs &m) {
    // Every 16-byte copy of a B row must start on a 16-byte boundary and hold
    // whole elements of one row: N a multiple of 4 (f32), 8 (f16), 16 (int8),
    // 32 (int4).  Q8_K needs 32-element blocks that tile each row (N a
    // multiple of 32), so that element (k, n) has the scale (k * N + n) / 32
    // = k * (N / 32) + n / 32.
    int nmul = 0;
    switch (m.fmt) {
        case TML_FMT_F32: nmul = 4; break;
        case TML_FMT_F16: nmul = 8; break;
        case TML_FMT_Q8_0: nmul = 16; break;
        case TML_FMT_Q4_0: nmul = 32; break;
        case TML_FMT_Q8_K:
            if (m.block != 32 || m.scales == nullptr) return false;
            nmul = 32;
            break;
        default: return false;
    }
    // The copies address A and B with 32-bit byte offsets below 2^31
    // (buffer resources, see gemm_dma_kernel): the largest offset a tile
    // can form is below (M + 256) * K * 4 for A and (K + 64) * (bytes per B
    // row) for B.
    const uint64_t lim = (uint64_t)1 << 31;
    if ((uint64_t)(m.M + 256) * (uint64_t)m.K * 4u >= lim || (uint64_t)(m.K + 64) * weight_row_bytes(m.fmt, m.N) >= lim)
        return false;
    return m.K % 4 == 0 && m.N % nmul == 0 && ((uintptr_t)m.A % 16) == 0 && ((uintptr_t)m.B % 16) == 0;
}

Status launch_gemm_f32_dma(const MatmulArgs &m, const GemmPlan &p, const Workspace &ws, hipStream_t s) {
    if (!gemm_dma_supported(m))
        return Status::Err(TML_ERR_INVALID_ARG, "dma GEMM needs f32/f16/Q8_0/Q8_K/Q4_0 B, K % 4 == 0, 16-byte rows, aligned");
    const int cfg = p.cfg;
    if (cfg < 0 || cfg >= gemm_dma_num_cfgs()) return Status::Err(TML_ERR_INVALID_ARG, "bad dma GEMM config");
    if (p.fused && p.nsplit > 1 && !gemm_dma_cfg_fusable(cfg))
        return Status::Err(TML_ERR_INVALID_ARG, "dma GEMM config with two K wave groups has no fused split-K");
    DmaArgs a;
    a.M = (int)m.M; a.N = (int)m.N; a.K = (int)m.K;
    a.A = m.A; a.B = m.B; a.bias = m.bias; a.C = m.C;
    a.ldb = (long long)weight_row_bytes(m.fmt, m.N);
    a.alpha = m.alpha_eff; a.beta = m.beta;
    a.zero = (const float *)m.zero;
    const int bm = kDmaCfgs[cfg].bm, bn = kDmaCfgs[cfg].bn;
    a.tiles_m = (int)((m.M + bm - 1) / bm);
    a.tiles_n = (int)((m.N + bn - 1) / bn);
    a.group_m = 4;
    pick_xcd_partition(a.tiles_m, a.tiles_n, p.nsplit, bm, bn, p.fused, (m.K + p.nsplit - 1) / p.nsplit, &a.pm, &a.pn,
                       &a.ps);
    a.nsplit = p.nsplit;
    a.spl = p.spl;
    a.ws = ws.partials;
    a.counters = p.fused ? ws.counters : nullptr;
    a.act = m.act;
    a.res = m.res;
    a.colscale = m.colscale;
    a.kscales = m.fmt == TML_FMT_Q8_K ? m.scales : nullptr;
    a.sld = (int)(m.N / 32);
    a.tail0 = tml_act_tail0((long long)m.M * m.N);
    const int64_t tiles = (int64_t)a.tiles_m * a.tiles_n;
    if (p.nsplit > 1) {
        size_t need_floats = 0, need_counters = 0;
        gemm_dma_workspace_need(m, p, &need_floats, &need_counters);
        if (ws.partials == nullptr || ws.partial_floats < need_floats ||
            (p.fused && (ws.counters == nullptr || ws.counter_count < need_counters)))
            return Status::Err(TML_ERR_INVALID_ARG, "GEMM split-K workspace too small");
    }
    const int bk = kDmaCfgs[cfg].bk;
    if (p.spl < 1 || (int64_t)p.spl * p.nsplit < (m.K + bk - 1) / bk)
        return Status::Err(TML_ERR_INVALID_ARG, "GEMM split plan does not cover K");
    if (tiles * p.nsplit >= ((int64_t)1 << 31)) return Status::Err(TML_ERR_INVALID_SHAPE, "GEMM grid too large");
    a.vec_epi = m.N % 4 == 0 && ((uintptr_t)m.C % 16) == 0 && (m.bias == nullptr || ((uintptr_t)m.bias % 16) == 0) &&
                (m.res == nullptr || ((uintptr_t)m.res % 16) == 0) &&
                (m.colscale == nullptr || ((uintptr_t)m.colscale % 16) == 0) && env_int("TML_GEMM_VEC_EPI", 1) != 0;
    const dim3 grid((unsigned)(tiles * p.nsplit));
    Status st;
    switch (m.fmt) {
        case TML_FMT_F32: st = launch_dma_cfg<TML_FMT_F32>(cfg, grid, a, s); break;
        case TML_FMT_F16: st = launch_dma_cfg<TML_FMT_F16>(cfg, grid, a, s); break;
        case TML_FMT_Q8_0: st = launch_dma_cfg<TML_FMT_Q8_0>(cfg, grid, a, s); break;
        case TML_FMT_Q8_K: st = launch_dma_cfg<TML_FMT_Q8_K>(cfg, grid, a, s); break;
        default: st = launch_dma_cfg<TML_FMT_Q4_0>(cfg, grid, a, s); break;
    }
    TML_TRY(st);
    TML_HIP_TRY(hipGetLastError());
    if (p.nsplit > 1 && !p.fused) TML_TRY(launch_splitk_reduce(ws.partials, p.nsplit, m, s));
    return Status::Ok();
}

Status launch_splitk_reduce(const float *partials, int nsplit, const MatmulArgs &m, hipStream_t s) {
    const int64_t n4 = (m.M * m.N + 3) / 4;
    const int64_t blocks = (n4 + 255) / 256;
    splitk_reduce_kernel<<<dim3((unsigned)(blocks < 65535 ? blocks : 65535)), 256, 0, s>>>(
        partials, nsplit, m.M * m.N, m.N, m.C, m.alpha_eff, m.beta, m.bias, m.res, m.colscale,
        m.N % 4 == 0 && ((uintptr_t)m.C % 16) == 0 && (m.bias == nullptr || ((uintptr_t)m.bias % 16) == 0) &&
            (m.res == nullptr || ((uintptr_t)m.res % 16) == 0) &&
            (m.colscale == nullptr || ((uintptr_t)m.colscale % 16) == 0),
        m.act, tml_act_tail0((long long)m.M * m.N));
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

}  // namespace tml
