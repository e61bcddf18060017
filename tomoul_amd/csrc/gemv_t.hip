// gemv_t.hip -- decoder GEMV on prepared, K-contiguous weights (M <= 8 for
// f32, <= 4 for Q8_0, <= 2 for Q4_0).
//
//   C[M,N] = alpha * A[M,K] . Bdeq[K,N] + beta * C + bias[N]
//
// with B held as its device-native "prepared" copy Bt[N][ldt]: row n of Bt
// holds column n of B (f32 four bytes per k, f16 two, int8 one; int4 two k
// per byte, the first in the low nibble), zero padded to ldt bytes, a
// multiple of 16.  The row is a sequence of 16-byte chunks (E = 4, 8, 16, 32
// elements each) in groups of 64 ("superchunks", the last one `width`
// chunks wide); element group g (four consecutive k) of chunk c of
// superchunk s holds k = 64*E*s + 4*(g*width + c) .. +3 (tk_group).  Lane c
// of a wave reads chunk c, so the activations of group g that the 64 lanes
// need are one contiguous run of 1 KiB -- each activation load touches 8
// cache lines instead of 64.  For f32 (one group per chunk) the order is
// plain K order.
// Weights are immutable after load in the reference (AttentionWeights owns
// them until deinit, src/core/attention.zig:54-86), so the copy is made once.
//
// Why: at decoder sizes a launch is bound by memory latency (a plain 4 MiB
// read needs ~2 us on MI355X).  In the stored [K,N] layout a GEMV has to
// split K over workgroups to reach every CU, and combining the splits costs
// two more dependent memory round trips.  With K contiguous, each output is
// one contiguous run of bytes: a column group of LK lanes (one wave, or the
// whole workgroup) walks the runs of its CW outputs in 16-byte chunks, every
// load instruction covers LK * 16 contiguous bytes, and no workgroup ever
// needs another's result.
//
// Per lane: the CW * JB weight chunks of a batch and the activations at the
// same k are loaded back to back (activations straight from L1/L2 into
// registers -- staging them in LDS costs a barrier, and the per-lane stride
// of E floats makes LDS reads conflict), dequantized in registers and
// accumulated into CW * MR dot products, which are reduced over the column
// group with a reduce-scatter butterfly (plus LDS across waves when the
// column group spans the workgroup).  Q8_0 / Q4_0 per-tensor scales are
// folded into alpha.
#include "tml_internal.hpp"

namespace tml {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

struct GemvTArgs {
    int M, N, K;
    const float *A;
    const uint8_t *Bt;
    long long ldt;        // bytes per prepared row
    const float *bias;
    const float *colscale;  // [N] per-column factor on A.B, or nullptr
    float *C;
    float alpha, beta;
    int nchunk;           // 16-byte chunks per prepared row
    const void *zero;
    int act;              // TML_ACT_* after the bias
    const float *res;     // [M,N] residual added after the bias, or nullptr
    long long tail0;      // tml_act_tail0(M * N)
    unsigned wbytes = 0;  // N * ldt: byte count of the Bt buffer resource (XM_BUF)
    unsigned xbytes = 0;  // M * K * 4: byte count of the A buffer resource (XM_BUF)
};

// 16 bytes at base + off of a buffer of nbytes, through a buffer resource:
// offsets at or past nbytes read zeros.  The resource is built from uniform
// values (SGPRs); the lane's offset is one 32-bit VGPR.
template <int POLICY = 0>
__device__ __forceinline__ uintx4 buf_load16(const void *base, unsigned nbytes, unsigned off) {
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, (int)nbytes, 0x00020000);
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, POLICY);
}

// How gemv_t_kernel loads its activations:
//   XM_SCALAR  element by element, each checked against K;
//   XM_VEC     16-byte vectors (K % 4 == 0, A 16-byte aligned), checked;
//   XM_BUF     16-byte vectors through buffer resources, unchecked: K is a
//              whole number of chunks, so only chunks past the row (lanes
//              of a partial last batch) are out of range, and their sums
//              are dropped instead (one select per dot product and batch;
//              their weight loads point past the resource and read zeros).
//              Each load's offset is the lane's constant plus a wave-uniform
//              step; the checked paths spend ~1.4 VALU instructions per
//              Q4_0 element on 64-bit addresses and zero-block selects.
constexpr int XM_SCALAR = 0, XM_VEC = 1, XM_BUF = 2;

// C = act((scale*acc + beta*C + bias) + residual) for output (m, n), the
// reference's order.  (Loading the column factor and bias ahead of the main
// loop -- into VGPRs, SGPRs or LDS -- was measured and is slower overall.)
__device__ __forceinline__ void epi_store(const GemvTArgs &a, int m, int n, float acc) {
    if (m < a.M && n < a.N) {
        const long long flat = (long long)m * a.N + n;
        float v = (a.colscale ? a.alpha * a.colscale[n] : a.alpha) * acc;
        if (a.beta != 0.0f) v += a.beta * a.C[flat];
        if (a.bias) v += a.bias[n];
        if (a.res) v += a.res[flat];
        a.C[flat] = tml_apply_act(v, a.act, flat, a.tail0);
    }
}

template <int FMT> struct TElems;
template <> struct TElems<TML_FMT_F32> { static constexpr int value = 4; };
template <> struct TElems<TML_FMT_Q8_0> { static constexpr int value = 16; };
template <> struct TElems<TML_FMT_Q4_0> { static constexpr int value = 32; };
template <> struct TElems<TML_FMT_F16> { static constexpr int value = 8; };

__device__ __forceinline__ float tsext8(uint32_t word, int byte) {
    return (float)((int32_t)(word << (24 - 8 * byte)) >> 24);
}

// 16 times the signed nibble `nib` of a word: the nibble moved to the top
// of its own byte (even nibbles shifted up by 4, odd ones in place) and that
// byte read as a signed byte -- one masked word per parity shared by four
// nibbles, then one byte-select convert each (v_cvt_f32_i32 with an SDWA
// sign-extended byte operand), where extracting the nibble itself costs a
// bit-field extract more per element.
__device__ __forceinline__ float tsext4x16(uint32_t word, int nib) {
    const uint32_t t = (nib & 1) ? (word & 0xF0F0F0F0u) : ((word << 4) & 0xF0F0F0F0u);
    return (float)(int8_t)(t >> (8 * (nib >> 1)));
}

// Element i of a prepared chunk.  With X16, Q4_0 elements come back 16 times
// their value (tsext4x16) and the kernel's alpha carries the 1/16: scaling by
// a power of two is exact, so every product and partial sum is exactly 16
// times the unscaled one and the result is the same bit for bit.  (The
// direct kernel uses it; in the LDS-staged kernel it measured slower at
// M = 4: 7.56 against 6.47 us at 1280x5120.)
template <int FMT, bool X16 = false>
__device__ __forceinline__ float telem(const uintx4 &w, int i) {
    if constexpr (FMT == TML_FMT_F32) return __uint_as_float(w[i]);
    else if constexpr (FMT == TML_FMT_F16) return tml_half_bits(w[i / 2] >> (16 * (i % 2)));
    else if constexpr (FMT == TML_FMT_Q8_0) return tsext8(w[i / 4], i % 4);
    else if constexpr (X16) return tsext4x16(w[i / 8], i % 8);
    else return (float)((int32_t)(w[i / 8] << (28 - 4 * (i % 8))) >> 28);
}
template <int FMT> constexpr float telem_x16_alpha() { return FMT == TML_FMT_Q4_0 ? 0.0625f : 1.0f; }

constexpr int tlog2(int v) { return v <= 1 ? 0 : 1 + tlog2(v / 2); }

// First k of element group g of chunk ch (see the layout notes above).
__device__ __forceinline__ int tk_group(int ch, int g, int nchunk, int E) {
    const int sc = ch >> 6, c = ch & 63;
    const int width = min(64, nchunk - (sc << 6));
    return sc * 64 * E + 4 * (g * width + c);
}

// v of the lane selected by the DPP control CTRL within the 16-lane row.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}



// LK lanes per column group (16: a DPP row, 64: a wave, 256: the
// workgroup), CW outputs
// per column group, JB chunks per lane per batch (two batches in flight).
// XM: how the activations are loaded (XM_SCALAR / XM_VEC / XM_BUF above).
template <int FMT, int MR, int LK, int CW, int JB, int XM>
__global__ __launch_bounds__(kThreads) void gemv_t_kernel(GemvTArgs a) {
    constexpr int E = TElems<FMT>::value;
    constexpr int GROUPS = kThreads / LK;       // column groups per workgroup
    constexpr int V = CW * MR;                  // dot products per lane
    constexpr int LOG_V = tlog2(V);
    static_assert((1 << LOG_V) == V, "power-of-two dot products per lane");
    static_assert(V <= (LK < 64 ? LK : 64), "one published dot product per lane of the group");
    __shared__ float red[kWaves * V];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int grp = tid / LK, lk = tid % LK;
    const int n0 = (blockIdx.x * GROUPS + grp) * CW;
    // the lane that publishes dot product lk % 64 (wave 0 when the group
    // spans the workgroup) owns output (m, n0 + c) of the epilogue

    // One batch = JB chunks per lane: the 16-byte weight chunk of each of
    // the CW outputs plus the E activations of every row m at those k, all
    // loaded back to back before any arithmetic.  The activations come
    // straight from global memory (L1/L2-resident: every workgroup reads the
    // same x) and serve the CW outputs.  A chunk past the row reads the zero
    // block for weights and activations alike (so a padded product is
    // 0 * 0, never 0 * inf); inside the last chunk the weights are zero
    // padded and activations past K are loaded as zeros.
    const int nbat = (a.nchunk + LK * JB - 1) / (LK * JB);
    uintx4 w0[CW][JB], w1[CW][JB];
    floatx4 x0[JB][MR][E / 4], x1[JB][MR][E / 4];
    // XM_BUF: the lane's byte offsets at batch 0.  A wave's lanes hold
    // consecutive chunks of one superchunk (LK divides 64, or a 256-lane
    // group spans four whole superchunk quarters), so a chunk's element
    // groups sit at a wave-uniform k plus 4 * (lane's chunk within the
    // superchunk).
    const int wave_u = __builtin_amdgcn_readfirstlane(wave);
    const unsigned xlane = 16u * (unsigned)(lk % 64);
    unsigned wlane[CW];
#pragma unroll
    for (int c = 0; c < CW; ++c) wlane[c] = (unsigned)(n0 + c) * (unsigned)a.ldt + 16u * (unsigned)lk;
    auto load_batch = [&](uintx4 (*w)[JB], floatx4 (*x)[MR][E / 4], int bt) __attribute__((always_inline)) {
        if constexpr (XM == XM_BUF) {
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int base = (bt * JB + j) * LK;  // first chunk of the group's batch
                // chunks past the row: read nothing (offset past the resource)
                // rather than the next row's bytes, which would cost traffic
                const bool in = base + lk < a.nchunk;
#pragma unroll
                for (int c = 0; c < CW; ++c)
                    w[c][j] = buf_load16<kStreamLoadPolicy>(a.Bt, a.wbytes, in ? wlane[c] + 16u * (unsigned)base : 0x80000000u);
                const int wb = base + (LK > 64 ? 64 * wave_u : 0);  // first chunk of the wave
                const int sc = wb >> 6;
                const int width = min(64, a.nchunk - (sc << 6));
#pragma unroll
                for (int m = 0; m < MR; ++m)
#pragma unroll
                    for (int q = 0; q < E / 4; ++q) {
                        const int ku = sc * 64 * E + 4 * (q * width + (wb & 63));  // k of the wave's first lane
                        const unsigned u = 4u * (unsigned)(m * a.K + ku);
                        x[j][m][q] = __builtin_bit_cast(floatx4, buf_load16(a.A, a.xbytes, xlane + u));
                    }
            }
            return;
        }
#pragma unroll
        for (int c = 0; c < CW; ++c)
#pragma unroll
            for (int j = 0; j < JB; ++j) {
                const int ch = (bt * JB + j) * LK + lk;
                const int n = n0 + c;
                const bool in = ch < a.nchunk && n < a.N;
                const uint8_t *p = in ? a.Bt + (size_t)n * a.ldt + (size_t)ch * 16 : (const uint8_t *)a.zero;
                w[c][j] = __builtin_nontemporal_load((const uintx4 *)p);
            }
#pragma unroll
        for (int j = 0; j < JB; ++j) {
            const int ch = (bt * JB + j) * LK + lk;
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const bool row_ok = ch < a.nchunk && m < a.M;
                const float *xr = a.A + (size_t)m * a.K;
#pragma unroll
                for (int q = 0; q < E / 4; ++q) {
                    const int k = tk_group(ch, q, a.nchunk, E);
                    if constexpr (XM == XM_VEC) {
                        const bool in = row_ok && k < a.K;  // K % 4 == 0: all four in or out
                        x[j][m][q] = *(const floatx4 *)(in ? xr + k : (const float *)a.zero);
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const bool in = row_ok && k + r < a.K;
                            x[j][m][q][r] = *(in ? xr + k + r : (const float *)a.zero);
                        }
                    }
                }
            }
        }
    };

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;
    auto compute_batch = [&](const uintx4 (*w)[JB], const floatx4 (*x)[MR][E / 4], int bt) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < JB; ++j) {
            // XM_BUF loads chunks past the row unchecked: drop their sums
            const bool keep = XM != XM_BUF || (bt * JB + j) * LK + lk < a.nchunk;
#pragma unroll
            for (int c = 0; c < CW; ++c) {
                float wv[E];
#pragma unroll
                for (int e = 0; e < E; ++e) wv[e] = telem<FMT, true>(w[c][j], e);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float s0 = 0.0f, s1 = 0.0f;  // two chains halve the add latency
#pragma unroll
                    for (int e = 0; e < E; e += 2) {
                        s0 += x[j][m][e / 4][e % 4] * wv[e];
                        s1 += x[j][m][(e + 1) / 4][(e + 1) % 4] * wv[e + 1];
                    }
                    acc[c * MR + m] += keep ? s0 + s1 : 0.0f;
                }
            }
        }
    };
    load_batch(w0, x0, 0);
    for (int bt = 0; bt < nbat; bt += 2) {
        if (bt + 1 < nbat) load_batch(w1, x1, bt + 1);
        compute_batch(w0, x0, bt);
        if (bt + 2 < nbat) load_batch(w0, x0, bt + 2);
        if (bt + 1 < nbat) compute_batch(w1, x1, bt + 1);
    }

    // All-reduce the V dot products over the LK lanes of the column group:
    // DPP within the 16-lane row (quad swaps, half mirror, mirror -- one VALU
    // op each), then xor 16 (ds_swizzle) and xor 32 across the rows of the
    // wave, then LDS across the waves when the group spans the workgroup.
    // Each step adds two disjoint partial sums and both partners compute the
    // same a + b, so every lane ends with bitwise identical totals.
#pragma unroll
    for (int i = 0; i < V; ++i) {
        float v = acc[i];
        v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
        v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
        v += dpp_mov<0x141>(v);  // row_half_mirror
        v += dpp_mov<0x140>(v);  // row_mirror
        if constexpr (LK >= 64) {
            v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
            v += __shfl_xor(v, 32);
        }
        acc[i] = v;
    }
    // Lane lk < V of the group publishes dot product lk.
    float val = acc[0];
#pragma unroll
    for (int i = 1; i < V; ++i)
        if (lk % 64 == i) val = acc[i];
    const int idx = lk % 64;
    if constexpr (LK > 64) {
        if (lane < V) red[wave * V + lane] = val;
        __syncthreads();
        if (wave != 0 || lane >= V) return;
#pragma unroll
        for (int w = 1; w < kWaves; ++w) val += red[w * V + lane];
    } else {
        if (idx >= V) return;
    }
    epi_store(a, idx % MR, n0 + idx / MR, val);
}

// ---- prepare: Bt[n][j] from B[K,N] (ROWS = false) or from the rows of
// W = B^T with a stride of ldw bytes (ROWS = true); one thread per output
// 32-bit word, elements placed by tk_group.
template <int FMT, bool ROWS>
__device__ __forceinline__ uint32_t src_elem(const void *B, int N, long long ldw, int k, int n) {
    const uint8_t *b = (const uint8_t *)B;
    if constexpr (FMT == TML_FMT_F32) {
        return ROWS ? *(const uint32_t *)(b + n * ldw + 4LL * k) : ((const uint32_t *)B)[(long long)k * N + n];
    } else if constexpr (FMT == TML_FMT_F16) {
        return ROWS ? *(const uint16_t *)(b + n * ldw + 2LL * k) : ((const uint16_t *)B)[(long long)k * N + n];
    } else if constexpr (FMT == TML_FMT_Q8_0) {
        return ROWS ? b[n * ldw + k] : b[(long long)k * N + n];
    } else {
        // int4: element e of a packed run is nibble e & 1 of byte e / 2
        const long long e = ROWS ? k : (long long)k * N + n;
        const uint32_t byte = ROWS ? b[n * ldw + e / 2] : b[e / 2];
        return (e & 1) ? (byte >> 4) : (byte & 0xF);
    }
}

template <int FMT, bool ROWS>
__global__ __launch_bounds__(256) void prepare_t_kernel(const void *B, int K, int N, long long ldw, long long ldt,
                                                        uint32_t *Bt) {
    constexpr int E = TElems<FMT>::value;
    constexpr int EPW = E / 4;      // elements per 32-bit word
    constexpr int BITS = 32 / EPW;  // bits per element
    const long long words_per_row = ldt / 4;
    const long long total = (long long)N * words_per_row;
    const int nchunk = (int)(words_per_row / 4);
    for (long long i = (long long)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (long long)gridDim.x * blockDim.x) {
        const int n = (int)(i / words_per_row);
        const int wj = (int)(i % words_per_row);
        const int ch = wj / 4;
        uint32_t word = 0;
#pragma unroll
        for (int h = 0; h < EPW; ++h) {
            const int e = (wj % 4) * EPW + h;  // element within the chunk
            const int k = tk_group(ch, e / 4, nchunk, E) + e % 4;
            if (k < K) word |= src_elem<FMT, ROWS>(B, N, ldw, k, n) << (BITS * h);
        }
        Bt[i] = word;
    }
}

// ---- LDS-staged variant, for row counts whose activations do not fit the
// direct kernel's registers (Q8_0 M > 4, Q4_0 M > 2) and wherever it is
// faster.  One wave per column group of CW outputs; the four waves of a
// workgroup share the activations of one superchunk (64 chunks = 64*E
// consecutive k, all MR rows), staged in LDS by the whole workgroup.  Lane c
// owns chunk c of every superchunk; its element group g needs the
// activations at 4*(g*width + c), so the 64 lanes read 64 consecutive
// 16-byte slots -- conflict-free.  The next superchunk's weights are loaded
// while the current one is multiplied.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_mov<0x141>(v);  // row_half_mirror
    v += dpp_mov<0x140>(v);  // row_mirror
    v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    v += __shfl_xor(v, 32);
    return v;
}

template <int FMT, int MR, int CW, bool XVEC>
__global__ __launch_bounds__(kThreads) void gemv_tl_kernel(GemvTArgs a) {
    constexpr int E = TElems<FMT>::value;
    constexpr int SK4 = 16 * E;  // float4 slots per row of a superchunk (64 * E k)
    constexpr int V = CW * MR;
    static_assert(V <= 64, "one published dot product per lane");
    __shared__ floatx4 xs[MR * SK4];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int n0 = (blockIdx.x * kWaves + wave) * CW;
    const int nsc = (a.nchunk + 63) >> 6;

    uintx4 w[CW], wn[CW];
    auto load_w = [&](uintx4 *dst, int sc) __attribute__((always_inline)) {
        const int ch = (sc << 6) + lane;
#pragma unroll
        for (int c = 0; c < CW; ++c) {
            const int n = n0 + c;
            const bool ok = ch < a.nchunk && n < a.N;
            dst[c] = __builtin_nontemporal_load(
                (const uintx4 *)(ok ? a.Bt + (size_t)n * a.ldt + (size_t)ch * 16 : (const uint8_t *)a.zero));
        }
    };
    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;

    load_w(w, 0);
    for (int sc = 0; sc < nsc; ++sc) {
        const int width = min(64, a.nchunk - (sc << 6));
        const int kbase = sc * 64 * E;
        __syncthreads();  // nobody still reads the previous superchunk
        if constexpr (XVEC) {
            // every load of the stage in flight at once, then the LDS stores;
            // out-of-range slots read the zero block (K % 4 == 0: a slot is
            // all in or all out)
            constexpr int TOT = MR * SK4;
            constexpr int ITER = (TOT + kThreads - 1) / kThreads;
            floatx4 t[ITER];
#pragma unroll
            for (int it = 0; it < ITER; ++it) {
                const int i = tid + it * kThreads;
                const int m = i / SK4, k = kbase + 4 * (i % SK4);
                const bool in = i < TOT && m < a.M && k < a.K;
                t[it] = *(const floatx4 *)(in ? a.A + (size_t)m * a.K + k : (const float *)a.zero);
            }
#pragma unroll
            for (int it = 0; it < ITER; ++it)
                if (TOT % kThreads == 0 || tid + it * kThreads < TOT) xs[tid + it * kThreads] = t[it];
        } else {
            for (int i = tid; i < MR * SK4; i += kThreads) {
                const int m = i / SK4, k = kbase + 4 * (i % SK4);
                floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
                if (m < a.M) {
                    const float *xr = a.A + (size_t)m * a.K;
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (k + r < a.K) v[r] = xr[k + r];
                }
                xs[i] = v;
            }
        }
        __syncthreads();
        if (sc + 1 < nsc) load_w(wn, sc + 1);
        // Lanes past the superchunk's width hold zero weights (the zero
        // block) and take zero activations: 0 * 0, never 0 * inf.
        const bool live = lane < width;
#pragma unroll
        for (int gq = 0; gq < E / 4; ++gq) {
            const int slot = gq * width + lane;
            floatx4 xv[MR];
#pragma unroll
            for (int m = 0; m < MR; ++m) xv[m] = live ? xs[m * SK4 + slot] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < CW; ++c) {
                float wv[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) wv[r] = telem<FMT>(w[c], 4 * gq + r);
#pragma unroll
                for (int m = 0; m < MR; ++m)
                    acc[c * MR + m] += (xv[m][0] * wv[0] + xv[m][1] * wv[1]) + (xv[m][2] * wv[2] + xv[m][3] * wv[3]);
            }
        }
        if (sc + 1 < nsc) {
#pragma unroll
            for (int c = 0; c < CW; ++c) w[c] = wn[c];
        }
    }

#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = wave_sum(acc[i]);
    if (lane >= V) return;
    float val = acc[0];
#pragma unroll
    for (int i = 1; i < V; ++i)
        if (lane == i) val = acc[i];
    epi_store(a, lane % MR, n0 + lane / MR, val);
}

template <int FMT, int MR, int CW>
void launch_tl2(const GemvTArgs &ka, unsigned grid, bool xvec, hipStream_t s) {
    if (xvec) gemv_tl_kernel<FMT, MR, CW, true><<<dim3(grid), dim3(kThreads), 0, s>>>(ka);
    else gemv_tl_kernel<FMT, MR, CW, false><<<dim3(grid), dim3(kThreads), 0, s>>>(ka);
}
template <int FMT, int MR>
void launch_tl1(const GemvTArgs &ka, int cw, unsigned grid, bool xvec, hipStream_t s) {
    if (cw >= 4) launch_tl2<FMT, MR, 4>(ka, grid, xvec, s);
    else if (cw >= 2) launch_tl2<FMT, MR, 2>(ka, grid, xvec, s);
    else launch_tl2<FMT, MR, 1>(ka, grid, xvec, s);
}
template <int FMT>
void launch_tl0(const GemvTArgs &ka, int cw, unsigned grid, bool xvec, hipStream_t s) {
    if (ka.M <= 1) launch_tl1<FMT, 1>(ka, cw, grid, xvec, s);
    else if (ka.M <= 2) launch_tl1<FMT, 2>(ka, cw, grid, xvec, s);
    else if (ka.M <= 4) launch_tl1<FMT, 4>(ka, cw, grid, xvec, s);
    else launch_tl1<FMT, 8>(ka, cw, grid, xvec, s);
}

struct TPlan {
    int lk, cw, jb;
};

// Column-group shape, from sweeps on MI355X:
//  * LK: at decoder sizes (latency-bound) every chunk gets its own lane --
//    one wave per group up to two waves' worth of chunks, else the whole
//    workgroup, fewer rows per wave for M > 2; once the weight streams tens
//    of MB (bandwidth-bound, e.g. a vocabulary projection), short rows
//    (<= 96 chunks) go to 16-lane groups, which waste no lanes and reduce
//    with DPP alone (the 80-chunk Q8_0 vocabulary rows would leave 48 of
//    the 128 lane slots of two 64-lane batches idle).
//  * CW: two outputs per group (four for long rows of weights streaming
//    tens of MB), fewer if that leaves a CU without a workgroup, with
//    CW * MR <= 16 dot products per lane.  At decoder sizes two beat four
//    by 2-11 % (e.g. Q4_0 1280x5120 M = 1: 3.99 against 4.34 us, F16 M = 8:
//    9.06 against 10.32 us) and one, by 2-35 %.
//  * JB = 1: one chunk per lane per batch; the batch loop keeps two in
//    flight (larger batches cost registers and occupancy).
TPlan plan_t(int fmt, int64_t M, int64_t N, int64_t nchunk, int cus) {
    TPlan p;
    const int mr = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    const double weight_bytes = (double)N * (double)nchunk * 16.0;
    const bool big = weight_bytes > 32.0e6;
    if (big && nchunk <= 96) p.lk = 16;
    else if (nchunk <= 128 || mr > 2) p.lk = 64;
    else p.lk = 256;
    const int groups = kThreads / p.lk;
    p.cw = (big && p.lk != 16) ? 4 : 2;
    while (p.cw > 1 && (N + (int64_t)groups * p.cw - 1) / ((int64_t)groups * p.cw) < cus) p.cw /= 2;
    while (p.cw > 1 && p.cw * mr > 16) p.cw /= 2;
    p.jb = 1;
    (void)fmt;
    const int forced_lk = env_int("TML_GEMVT_LK", 0), forced_cw = env_int("TML_GEMVT_CW", 0),
              forced_jb = env_int("TML_GEMVT_JB", 0);
    if (forced_lk == 16 || forced_lk == 64 || forced_lk == 256) p.lk = forced_lk;
    if (forced_cw == 1 || forced_cw == 2 || forced_cw == 4) p.cw = forced_cw;
    if (forced_jb == 1 || forced_jb == 2 || forced_jb == 4) p.jb = forced_jb;
    // a 16-lane group publishes at most 16 dot products: CW * MR <= 16
    if (p.lk == 16)
        while (p.cw > 1 && p.cw * mr > 16) p.cw /= 2;
    return p;
}

template <int FMT, int MR, int LK, int CW, int JB>
void launch_t4(const GemvTArgs &ka_in, unsigned grid, int xm, hipStream_t s) {
    GemvTArgs ka = ka_in;
    ka.alpha *= telem_x16_alpha<FMT>();  // the direct kernel widens Q4_0 to 16x its values
    if (xm == XM_BUF) gemv_t_kernel<FMT, MR, LK, CW, JB, XM_BUF><<<dim3(grid), dim3(kThreads), 0, s>>>(ka);
    else if (xm == XM_VEC) gemv_t_kernel<FMT, MR, LK, CW, JB, XM_VEC><<<dim3(grid), dim3(kThreads), 0, s>>>(ka);
    else gemv_t_kernel<FMT, MR, LK, CW, JB, XM_SCALAR><<<dim3(grid), dim3(kThreads), 0, s>>>(ka);
}
// Batches are capped so that the two in-flight batches of activations stay
// within ~128 registers: JB * MR * E <= 64.
template <int FMT, int MR>
constexpr int jb_max() {
    return TElems<FMT>::value * MR <= 16 ? 4 : (TElems<FMT>::value * MR <= 32 ? 2 : 1);
}
template <int FMT, int MR, int LK, int CW>
void launch_t3(const GemvTArgs &ka, const TPlan &p, unsigned grid, int xm, hipStream_t s) {
    constexpr int JM = jb_max<FMT, MR>();
    const int jb = p.jb < JM ? p.jb : JM;
    if (jb >= 4) launch_t4<FMT, MR, LK, CW, (JM >= 4 ? 4 : JM)>(ka, grid, xm, s);
    else if (jb >= 2) launch_t4<FMT, MR, LK, CW, (JM >= 2 ? 2 : 1)>(ka, grid, xm, s);
    else launch_t4<FMT, MR, LK, CW, 1>(ka, grid, xm, s);
}
template <int FMT, int MR, int LK>
void launch_t2(const GemvTArgs &ka, const TPlan &p, unsigned grid, int xm, hipStream_t s) {
    // plan_t keeps CW * MR <= 16 for 16-lane groups
    switch (p.cw) {
        case 1: launch_t3<FMT, MR, LK, 1>(ka, p, grid, xm, s); break;
        case 2:
            if constexpr (LK != 16 || 2 * MR <= 16) launch_t3<FMT, MR, LK, 2>(ka, p, grid, xm, s);
            break;
        default:
            if constexpr (LK != 16 || 4 * MR <= 16) launch_t3<FMT, MR, LK, 4>(ka, p, grid, xm, s);
            break;
    }
}
template <int FMT, int MR>
void launch_t1(const GemvTArgs &ka, const TPlan &p, unsigned grid, int xm, hipStream_t s) {
    if (p.lk == 16) launch_t2<FMT, MR, 16>(ka, p, grid, xm, s);
    else if (p.lk == 64) launch_t2<FMT, MR, 64>(ka, p, grid, xm, s);
    else launch_t2<FMT, MR, 256>(ka, p, grid, xm, s);
}
template <int FMT>
void launch_t0(const GemvTArgs &ka, const TPlan &p, unsigned grid, int xm, hipStream_t s) {
    constexpr int E = TElems<FMT>::value;
    if (ka.M <= 1) launch_t1<FMT, 1>(ka, p, grid, xm, s);
    else if (ka.M <= 2) launch_t1<FMT, 2>(ka, p, grid, xm, s);
    else if constexpr (E * 4 <= 64) {
        if (ka.M <= 4) launch_t1<FMT, 4>(ka, p, grid, xm, s);
        else if constexpr (E * 8 <= 64) launch_t1<FMT, 8>(ka, p, grid, xm, s);
    }
}

int t_elems(int fmt) { return fmt == TML_FMT_F32 ? 4 : fmt == TML_FMT_F16 ? 8 : (fmt == TML_FMT_Q8_0 ? 16 : 32); }

}  // namespace

int64_t prepared_row_bytes(int fmt, int64_t K) {
    const int64_t bytes = packed_row_bytes(fmt, K);
    const int64_t r = (bytes + 15) / 16 * 16;
    return r > 0 ? r : 16;
}

int64_t prepared_gemv_max_m(int fmt) {
    return (fmt == TML_FMT_F32 || fmt == TML_FMT_F16 || fmt == TML_FMT_Q8_0 || fmt == TML_FMT_Q4_0) ? kPreparedGemvMaxM
                                                                                                  : 0;
}

// Measured on MI355X at the decoder shapes (1024x4096 Q8_0 / F16, 1280x5120
// and 5120x1280 Q4_0): the prepared kernels beat the [K,N] GEMV everywhere
// except Q4_0 at M > 4 (15.0 / 19.7 us against 10.4 / 14.3 us), where the
// staged activations of eight rows outweigh the halved weight bytes.
// The matrix-core kernel (gemv_tm.hip) serves Q8_0 / Q4_0 at M >= 3 (and
// M = 2 on short Q4_0 rows) when K is a whole number of chunks, Q4_0 above
// M = 4 included.
bool prepared_gemv_preferred(int fmt, int64_t M, int64_t K) {
    return gemv_tm_supported(fmt, M, K) || !(fmt == TML_FMT_Q4_0 && M > 4);
}

bool prepared_gemv_supported(int fmt, int64_t M, int64_t K) {
    if (fmt != TML_FMT_F32 && fmt != TML_FMT_F16 && fmt != TML_FMT_Q8_0 && fmt != TML_FMT_Q4_0) return false;
    return M >= 1 && M <= kPreparedGemvMaxM && K < ((int64_t)1 << 30);
}

namespace {
template <bool ROWS>
Status launch_prepare(int fmt, int64_t K, int64_t N, const void *B, int64_t ldw, void *Bt, int64_t ldt,
                      hipStream_t s) {
    if (ldt % 16 != 0 || ldt < prepared_row_bytes(fmt, K))
        return Status::Err(TML_ERR_INVALID_ARG, "prepared row stride too small");
    if (K >= ((int64_t)1 << 30) || N >= ((int64_t)1 << 30) || ldt / 64 >= ((int64_t)1 << 30))
        return Status::Err(TML_ERR_INVALID_SHAPE, "prepare: dimension exceeds 2^30");
    const long long words = (long long)N * (ldt / 4);
    const long long blocks = (words + 255) / 256;
    const dim3 grid((unsigned)(blocks < 65535 ? (blocks > 0 ? blocks : 1) : 65535));
    const int k = (int)K, n = (int)N;
    uint32_t *bt = (uint32_t *)Bt;
    switch (fmt) {
        case TML_FMT_F32: prepare_t_kernel<TML_FMT_F32, ROWS><<<grid, 256, 0, s>>>(B, k, n, ldw, ldt, bt); break;
        case TML_FMT_Q8_0: prepare_t_kernel<TML_FMT_Q8_0, ROWS><<<grid, 256, 0, s>>>(B, k, n, ldw, ldt, bt); break;
        case TML_FMT_Q4_0: prepare_t_kernel<TML_FMT_Q4_0, ROWS><<<grid, 256, 0, s>>>(B, k, n, ldw, ldt, bt); break;
        case TML_FMT_F16: prepare_t_kernel<TML_FMT_F16, ROWS><<<grid, 256, 0, s>>>(B, k, n, ldw, ldt, bt); break;
        default: return Status::Err(TML_ERR_INVALID_FORMAT, "prepared layout: format must be F32, F16, Q8_0 or Q4_0");
    }
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}
}  // namespace

Status launch_prepare_t(int fmt, int64_t K, int64_t N, const void *B, void *Bt, int64_t ldt, hipStream_t s) {
    return launch_prepare<false>(fmt, K, N, B, 0, Bt, ldt, s);
}

Status launch_prepare_rows(int fmt, int64_t K, int64_t N, const void *W, int64_t ldw, void *Bt, int64_t ldt,
                           hipStream_t s) {
    return launch_prepare<true>(fmt, K, N, W, ldw, Bt, ldt, s);
}

Status launch_gemv_t(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *Bt, int64_t ldt,
                     const float *bias, const float *res, float *C, float alpha_eff, float beta,
                     const void *zero, int act, long long tail0, const float *colscale, hipStream_t s) {
    if (!prepared_gemv_supported(fmt, M, K)) return Status::Err(TML_ERR_INVALID_ARG, "prepared GEMV: unsupported");
    if (N >= ((int64_t)1 << 30) || K >= ((int64_t)1 << 30))
        return Status::Err(TML_ERR_INVALID_SHAPE, "GEMV dimension exceeds 2^30");
    if (ldt < prepared_row_bytes(fmt, K) || ldt % 16 != 0 || ((uintptr_t)Bt % 16) != 0)
        return Status::Err(TML_ERR_INVALID_ARG, "prepared weight layout");
    // Q8_0 / Q4_0 at M <= 4 with the activations staged per workgroup
    // (gemv_x.hip) where gemv_x_preferred finds it the faster kernel.
    if (gemv_x_preferred(fmt, M, N, K) && ((uintptr_t)A % 16) == 0)
        return launch_gemv_x(fmt, M, N, K, A, Bt, ldt, bias, res, C, alpha_eff, beta, act, tail0, colscale, s);
    if (env_int("TML_GEMVX", 1) == 3)
        return Status::Err(TML_ERR_INVALID_ARG, "TML_GEMVX=3: this call does not take the staged-activation GEMV");
    // Q8_0 / Q4_0 on the matrix cores (gemv_tm.hip) where it is the faster
    // kernel (M >= 3, short Q4_0 rows at M = 2, Q4_0 vocabularies at M = 1) and its
    // operands fit its buffer offsets.
    if ((gemv_tm_supported(fmt, M, K) || (M == 1 && gemv_tm_m1_preferred(fmt, N, K))) && ((uintptr_t)A % 16) == 0 &&
        N * ldt < ((int64_t)1 << 31) && M * K * 4 < ((int64_t)1 << 31))
        return launch_gemv_tm(fmt, M, N, K, A, Bt, ldt, bias, res, C, alpha_eff, beta, act, tail0, colscale, s);
    GemvTArgs ka;
    ka.M = (int)M; ka.N = (int)N; ka.K = (int)K;
    ka.A = A; ka.Bt = (const uint8_t *)Bt; ka.ldt = ldt;
    ka.bias = bias; ka.C = C; ka.alpha = alpha_eff; ka.beta = beta;
    ka.colscale = colscale;
    ka.nchunk = (int)((prepared_row_bytes(fmt, K) + 15) / 16);
    ka.zero = zero;
    ka.act = act;
    ka.res = res;
    ka.tail0 = tail0;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) == hipSuccess && n > 0) cus = n;
    }
    const bool xvec = (K % 4 == 0) && ((uintptr_t)A % 16 == 0);
    // The direct kernel holds a chunk's activations for every row in
    // registers (MR * E <= 64); beyond that, and where TML_GEMVT_LDS=1 asks
    // for it, the activations are staged in LDS.
    const int mr = M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8;
    // Staging wins for Q4_0 at M = 2 (4.9 against 7.0 us) and F16 at M > 4
    // (6.3 against 6.7 us); elsewhere the direct kernel is as fast or faster.
    const int lds_mode = env_int("TML_GEMVT_LDS", -1);
    const bool use_lds = mr * t_elems(fmt) > 64 || lds_mode == 1 ||
                         (lds_mode < 0 && ((fmt == TML_FMT_Q4_0 && mr == 2) || (fmt == TML_FMT_F16 && mr == 8)));
    if (use_lds) {
        // CW outputs per wave: two (four for Q4_0 at M = 3-4: 6.53 against
        // 7.51 us at 1280x5120; two elsewhere, e.g. Q8_0 M = 8: 5.73 against
        // 6.11 us), fewer if that leaves a CU without a workgroup
        int cw = (fmt == TML_FMT_Q4_0 && mr == 4) ? 4 : 2;
        while (cw > 1 && (N + 4LL * cw - 1) / (4LL * cw) < cus) cw /= 2;
        const int forced_cw = env_int("TML_GEMVT_CW", 0);
        if (forced_cw == 1 || forced_cw == 2 || forced_cw == 4) cw = forced_cw;
        const int64_t grid = (N + 4LL * cw - 1) / (4LL * cw);
        if (grid >= ((int64_t)1 << 31)) return Status::Err(TML_ERR_INVALID_SHAPE, "GEMV grid too large");
        switch (fmt) {
            case TML_FMT_F32: launch_tl0<TML_FMT_F32>(ka, cw, (unsigned)grid, xvec, s); break;
            case TML_FMT_Q8_0: launch_tl0<TML_FMT_Q8_0>(ka, cw, (unsigned)grid, xvec, s); break;
            case TML_FMT_F16: launch_tl0<TML_FMT_F16>(ka, cw, (unsigned)grid, xvec, s); break;
            default: launch_tl0<TML_FMT_Q4_0>(ka, cw, (unsigned)grid, xvec, s); break;
        }
        TML_HIP_TRY(hipGetLastError());
        return Status::Ok();
    }
    const TPlan p = plan_t(fmt, M, N, ka.nchunk, cus);
    // Buffer-resource loads when K is a whole number of chunks and every
    // byte offset fits the resources (below 2^31); measured against the
    // checked vector loads: 3-6 % faster for Q8_0 / Q4_0 / F16 at M <= 4
    // and f32 at M = 1 (Q4_0 vocabulary 13.43 -> 12.67 us), 3-4 % slower
    // for f32 at M = 4-8, which keeps the checked loads.
    const bool exact = (int64_t)ka.nchunk * t_elems(fmt) == K && xvec && N * ldt <= ((int64_t)1 << 31) &&
                       M * K * 4 < ((int64_t)1 << 31) && !(fmt == TML_FMT_F32 && M > 2) &&
                       env_int("TML_GEMVT_BUF", 1) != 0;
    ka.wbytes = (unsigned)(N * ldt);
    ka.xbytes = (unsigned)(M * K * 4);
    const int xm = exact ? XM_BUF : xvec ? XM_VEC : XM_SCALAR;
    const int groups = kThreads / p.lk;
    const int64_t outs_per_wg = (int64_t)groups * p.cw;
    const int64_t grid = (N + outs_per_wg - 1) / outs_per_wg;
    if (grid >= ((int64_t)1 << 31)) return Status::Err(TML_ERR_INVALID_SHAPE, "GEMV grid too large");
    switch (fmt) {
        case TML_FMT_F32: launch_t0<TML_FMT_F32>(ka, p, (unsigned)grid, xm, s); break;
        case TML_FMT_Q8_0: launch_t0<TML_FMT_Q8_0>(ka, p, (unsigned)grid, xm, s); break;
        case TML_FMT_F16: launch_t0<TML_FMT_F16>(ka, p, (unsigned)grid, xm, s); break;
        default: launch_t0<TML_FMT_Q4_0>(ka, p, (unsigned)grid, xm, s); break;
    }
    TML_HIP_TRY(hipGetLastError());
    return Status::Ok();
}

}  // namespace tml
