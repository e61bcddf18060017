// gemv.hip -- skinny GEMM / GEMV for M <= 8 (decoder shapes), all formats.
//
//   C[M,N] = alpha * A[M,K] . Bdeq[K,N] + beta * C + bias[N]
//
// At M <= 8 the product streams B once; at the decoder sizes (3-4 MB of
// weights) one launch is bound by memory latency, not bandwidth: a plain
// 4 MiB read kernel needs ~2 us on MI355X however it is shaped, and it gets
// there only when every CU has its whole share of loads in flight at once.
// So the kernel is built for parallelism and few dependent round trips:
//   * B stays in its stored [K,N] layout (N contiguous; src/core/
//     quantization.zig:193-197).  Work is cut into column segments of LPR
//     lanes x LW bytes and row batches; every lane issues its U loads of LW
//     bytes (and the activations of those rows) back to back, branch-free,
//     before it does any arithmetic.  The grid holds as many workgroups as
//     there are (segment, K split) units, typically one to a few per CU.
//   * Rows need not be a whole number of lane chunks (a 51866-token
//     vocabulary): a chunk is then read as the aligned dwords that cover it
//     and funnel-shifted into place (kRagged below).
//   * Dequantization happens in registers (sign-extending bit-field
//     extracts); Q8_0 / Q4_0 per-tensor scales are applied once in the
//     epilogue, Q8_K block scales per chunk.
//   * The RW = 64 / LPR row lanes of a wave that share a column chunk are
//     combined with a reduce-scatter butterfly (each step exchanges half of
//     the remaining values), which costs about one shuffle per value whatever
//     RW is; the 4 waves then add up through LDS.
//   * K splits: each workgroup publishes its partial segment with
//     agent-coherent stores, waits for them to complete, and bumps the
//     segment's counter; the last workgroup to arrive reads the other
//     partials with agent-coherent loads, sums all of them in split order
//     (results do not depend on scheduling) and writes C, then resets the
//     counter.  Only agent-scope atomic loads/stores touch the partials, so
//     no cache-wide write-back or invalidate is needed.
#include "tml_internal.hpp"

namespace tml {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kNumXcd = 8;
typedef uint32_t uintx4 __attribute__((ext_vector_type(4)));
typedef uint32_t uintx2 __attribute__((ext_vector_type(2)));

struct GemvKArgs {
    int M, N, K;
    const float *A;
    const void *B;
    const float *scales;
    long long block;
    const float *bias;
    const float *colscale;  // [N] per-column factor on A.B, or nullptr
    float *C;
    float alpha, beta;
    int nseg;            // column segments
    int nsplit;          // K splits (workgroups per segment)
    int nb;              // row batches per workgroup
    float *ws;           // [nsplit][MR][N] partials when nsplit > 1
    unsigned *counters;  // one per segment, zero between launches
    const void *zero;
    int act;             // TML_ACT_* after the bias
    const float *res;    // [M,N] residual added after the bias, or nullptr
    long long tail0;     // tml_act_tail0(M * N)
    unsigned bbytes;     // byte count of B (kRagged: the buffer resource's range)
};

// How the kernel reads B:
//   kGeneric  element by element, each checked (any N, block, alignment);
//   kAligned  one LW-byte load per chunk (N % E == 0, B LW-byte aligned);
//   kRagged   any N, B 4-byte aligned and under 2 GiB: a chunk starts at
//             any element, so it is assembled from the LW / 4 + 1 aligned
//             dwords that cover it, read through a buffer resource, and
//             funnel-shifted into place.
enum { kGeneric = 0, kAligned = 1, kRagged = 2 };

// Elements of B held in LW bytes.
template <int FMT, int LW> struct Elems;
template <int LW> struct Elems<TML_FMT_F32, LW> { static constexpr int value = LW / 4; };
template <int LW> struct Elems<TML_FMT_Q8_0, LW> { static constexpr int value = LW; };
template <int LW> struct Elems<TML_FMT_Q8_K, LW> { static constexpr int value = LW; };
template <int LW> struct Elems<TML_FMT_Q4_0, LW> { static constexpr int value = 2 * LW; };
template <int LW> struct Elems<TML_FMT_F16, LW> { static constexpr int value = LW / 2; };

// One chunk as loaded: LW / 4 words (kRagged: one more, and the bit shift
// that aligns the chunk, applied when it is used).
template <int LW> struct Raw { uint32_t w[LW / 4 + 1]; float s; unsigned sh; };

// Sign-extending field extracts (compile to v_bfe_i32).
__device__ __forceinline__ float sext8(uint32_t word, int byte) {
    return (float)((int32_t)(word << (24 - 8 * byte)) >> 24);
}
__device__ __forceinline__ float sext4(uint32_t word, int nib) {
    return (float)((int32_t)(word << (28 - 4 * nib)) >> 28);
}

// s_waitcnt vmcnt(0), other counters untouched (gfx9 encoding).
__device__ __forceinline__ void wait_vm0() { __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8)); }

__device__ __forceinline__ void store_agent(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_agent(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Vector path: one LW-byte load of row k at column n.  Branch-free: an
// invalid chunk (row past the split, column past N) reads the zero block
// (the address is selected, not the value).  Host guarantees N % E == 0,
// LW-byte alignment of B and, for Q8_K, N % block == 0 and block % E == 0,
// so a chunk never straddles a row or a scale block.
template <int FMT, int LW>
__device__ __forceinline__ void load_chunk(const GemvKArgs &a, bool in, int k, int n, Raw<LW> &r) {
    const size_t e = (size_t)k * a.N + n;
    const void *p = !in ? a.zero
                  : FMT == TML_FMT_F32 ? (const void *)((const float *)a.B + e)
                  : FMT == TML_FMT_F16 ? (const void *)((const uint16_t *)a.B + e)
                  : FMT == TML_FMT_Q4_0 ? (const void *)((const uint8_t *)a.B + e / 2)
                                        : (const void *)((const int8_t *)a.B + e);
    if constexpr (LW == 16) {
        const uintx4 v = *(const uintx4 *)p;
        r.w[0] = v[0]; r.w[1] = v[1]; r.w[2] = v[2]; r.w[3] = v[3];
    } else if constexpr (LW == 8) {
        const uintx2 v = *(const uintx2 *)p;
        r.w[0] = v[0]; r.w[1] = v[1];
    } else {
        r.w[0] = *(const uint32_t *)p;
    }
    if constexpr (FMT == TML_FMT_Q8_K) r.s = *(in ? a.scales + e / a.block : (const float *)a.zero);
}

template <int FMT> constexpr int kElemBits = FMT == TML_FMT_F32 ? 32 : FMT == TML_FMT_F16 ? 16 : FMT == TML_FMT_Q4_0 ? 4 : 8;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t b_rsrc(const GemvKArgs &a) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(a.B), (short)0, (int)a.bbytes, 0x00020000);
}

// kRagged: the LW bytes of row k at column n, wherever they start.  Element
// e = k*N + n begins at bit b = e * bits of B; the dwords from b / 32 on are
// read (each range-checked on its own: dwords past B read zero, so an
// invalid chunk points at bbytes rounded up); shift_chunk, called once the
// loads are needed, shifts them right by b % 32.
// A chunk running past the end of its row picks up the next row's first
// elements; they only ever reach columns >= N, whose sums are dropped, and
// past the end of B (elements e >= K*N, columns >= N of the last row) it
// reads zeros.
template <int FMT, int LW>
__device__ __forceinline__ void load_chunk_ragged(const GemvKArgs &a, bool in, int k, int n, Raw<LW> &r) {
    constexpr int ND = LW / 4;
    constexpr int NL = FMT == TML_FMT_F32 ? ND : ND + 1;  // f32 chunks start on a dword
    static_assert(FMT != TML_FMT_F32 || LW == 16, "f32 chunks are 16 bytes");
    const unsigned long long bit = ((unsigned long long)k * (unsigned)a.N + (unsigned)n) * kElemBits<FMT>;
    const unsigned far = (a.bbytes + 3u) & ~3u;
    const unsigned off = in ? (unsigned)(bit >> 5) << 2 : far;
    const __amdgpu_buffer_rsrc_t rs = b_rsrc(a);
    if constexpr (LW == 16) {
        const uintx4 v = __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0);
        r.w[0] = v[0]; r.w[1] = v[1]; r.w[2] = v[2]; r.w[3] = v[3];
    } else {
        const uintx2 v = __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0);
        r.w[0] = v[0]; r.w[1] = v[1];
    }
    if constexpr (NL > 2 && NL > ND) r.w[ND] = __builtin_amdgcn_raw_buffer_load_b32(rs, off + 4u * ND, 0, 0);
    if constexpr (FMT != TML_FMT_F32) {
        // B ending inside a dword: that dword is out of range as a whole
        // (it reads zero), but its first bytes are the last elements of B,
        // so the lanes whose chunk covers it rebuild it from byte loads.
        const unsigned tail = a.bbytes & 3u, full = a.bbytes & ~3u;
        if (tail != 0u && full - off < 4u * NL) {
            uint32_t v = 0;
            for (unsigned i = 0; i < tail; ++i)
                v |= (uint32_t)__builtin_amdgcn_raw_buffer_load_b8(rs, full + i, 0, 0) << (8 * i);
#pragma unroll
            for (int i = 0; i < NL; ++i)
                if (off + 4u * i == full) r.w[i] = v;
        }
    }
    r.sh = (unsigned)bit & 31u;
}

template <int FMT, int LW>
__device__ __forceinline__ void shift_chunk(Raw<LW> &r) {
    if constexpr (FMT != TML_FMT_F32) {
#pragma unroll
        for (int i = 0; i < LW / 4; ++i)
            r.w[i] = (uint32_t)((((unsigned long long)r.w[i + 1] << 32) | r.w[i]) >> r.sh);
    }
}

template <int FMT, int LW>
__device__ __forceinline__ void decode_chunk(const Raw<LW> &r, float *w) {
    constexpr int E = Elems<FMT, LW>::value;
    if constexpr (FMT == TML_FMT_F32) {
#pragma unroll
        for (int i = 0; i < E; ++i) w[i] = __uint_as_float(r.w[i]);
    } else if constexpr (FMT == TML_FMT_F16) {
#pragma unroll
        for (int i = 0; i < E; ++i) w[i] = tml_half_bits(r.w[i / 2] >> (16 * (i % 2)));
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

// Generic path: element-wise loads with bounds, any N, block and alignment;
// the values come back dequantized (Q8_K scale applied, Q8_0 / Q4_0 as
// integers).
template <int FMT, int E>
__device__ __forceinline__ void load_elems(const GemvKArgs &a, bool row_ok, int k, int n, float *w) {
    const size_t e = (size_t)k * a.N + n;
#pragma unroll
    for (int i = 0; i < E; ++i) {
        float v = 0.0f;
        if (row_ok && n + i < a.N) {
            const size_t ei = e + i;
            if constexpr (FMT == TML_FMT_F32) v = ((const float *)a.B)[ei];
            else if constexpr (FMT == TML_FMT_F16) v = tml_half_bits(((const uint16_t *)a.B)[ei]);
            else if constexpr (FMT == TML_FMT_Q8_0) v = (float)((const int8_t *)a.B)[ei];
            else if constexpr (FMT == TML_FMT_Q8_K) v = (float)((const int8_t *)a.B)[ei] * a.scales[ei / a.block];
            else v = sext4(((const uint8_t *)a.B)[ei / 2], (int)(ei & 1));
        }
        w[i] = v;
    }
}

constexpr int ilog2(int v) { return v <= 1 ? 0 : 1 + ilog2(v / 2); }

template <int FMT, int MR, int LW, int LPR, int U, int MODE>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvKArgs a) {
    constexpr int E = Elems<FMT, LW>::value;
    constexpr int RW = 64 / LPR;          // row lanes per wave (rows per load instruction)
    constexpr int SC = LPR * E;           // columns per segment
    constexpr int RB = kWaves * RW * U;   // rows per batch of the workgroup
    constexpr int V = MR * E;             // partial sums per lane
    constexpr int LOG_RW = ilog2(RW);
    constexpr int LOG_V = ilog2(V);
    constexpr int NOUT = MR * SC;         // outputs of the segment
    constexpr int OPT = (NOUT + kThreads - 1) / kThreads;
    static_assert((1 << LOG_RW) == RW && (1 << LOG_V) == V, "power-of-two shapes");

    __shared__ __attribute__((aligned(16))) float red[kWaves * NOUT];
    __shared__ unsigned arrived;

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int cl = lane % LPR, rl = lane / LPR;

    // Consecutive work ids run on one XCD (workgroups are dealt to the XCDs
    // round-robin), so segments narrower than a cache line share its L2.
    const int nblk = gridDim.x, bid = blockIdx.x;
    const int per = nblk / kNumXcd, rem = nblk % kNumXcd;
    const int xcd = bid % kNumXcd, idx = bid / kNumXcd;
    const int work = (xcd < rem) ? xcd * (per + 1) + idx : rem * (per + 1) + (xcd - rem) * per + idx;
    const int seg = work % a.nseg;
    const int split = work / a.nseg;
    const int n = seg * SC + cl * E;
    const bool col_in = n < a.N;
    const int kbeg = split * a.nb * RB;
    const int kend = min(a.K, kbeg + a.nb * RB);
    const int nbat = kend > kbeg ? (kend - kbeg + RB - 1) / RB : 0;
    const int lrow = (wave * RW + rl) * U;  // the lane's first row in a batch

    float acc[V];
#pragma unroll
    for (int i = 0; i < V; ++i) acc[i] = 0.0f;

    // One batch = U consecutive rows per lane: B chunks plus the MR
    // activations of each row.  Rows past the split read the zero block.
    Raw<LW> w0[U], w1[U];
    float x0[U][MR], x1[U][MR];
    auto load_batch = [&](Raw<LW> *w, float (*x)[MR], int bt) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = kbeg + bt * RB + lrow + u;
            const bool valid = k < kend;
            if constexpr (MODE == kAligned) load_chunk<FMT, LW>(a, valid && col_in, valid ? k : 0, col_in ? n : 0, w[u]);
            else if constexpr (MODE == kRagged) load_chunk_ragged<FMT, LW>(a, valid && col_in, k, n, w[u]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const bool ok = valid && m < a.M;
                x[u][m] = *(ok ? a.A + (size_t)m * a.K + k : (const float *)a.zero);
            }
        }
    };
    auto compute_batch = [&](const Raw<LW> *w, const float (*x)[MR], int bt) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            float wv[E];
            if constexpr (MODE == kRagged) {
                Raw<LW> c = w[u];
                shift_chunk<FMT, LW>(c);
                decode_chunk<FMT, LW>(c, wv);
            } else if constexpr (MODE == kAligned) {
                decode_chunk<FMT, LW>(w[u], wv);
            } else {
                const int k = kbeg + bt * RB + lrow + u;
                load_elems<FMT, E>(a, k < kend, k < kend ? k : 0, n, wv);
            }
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int e = 0; e < E; ++e) acc[m * E + e] += x[u][m] * wv[e];
        }
    };

    // Stream B with two batches in flight.
    if (nbat > 0) load_batch(w0, x0, 0);
    for (int bt = 0; bt < nbat; bt += 2) {
        if (bt + 1 < nbat) load_batch(w1, x1, bt + 1);
        compute_batch(w0, x0, bt);
        if (bt + 2 < nbat) load_batch(w0, x0, bt + 2);
        if (bt + 1 < nbat) compute_batch(w1, x1, bt + 1);
    }

    // Reduce-scatter over the RW row lanes (lane bits LPR .. 32): at each
    // step the lane pair splits the remaining values in halves, each keeps
    // one half and adds the partner's copy of it.  Once one value is left,
    // the remaining steps are a plain butterfly.  a + b == b + a exactly, so
    // both lanes of a pair produce identical sums.
    int base = 0;  // index of the first value this lane holds
#pragma unroll
    for (int s = 0; s < LOG_RW; ++s) {
        const int o = LPR << s;
        const bool hi = (lane & o) != 0;
        if (s < LOG_V) {
            const int half = V >> (s + 1);
#pragma unroll
            for (int i = 0; i < half; ++i) {
                const float send = hi ? acc[i] : acc[i + half];
                const float keep = hi ? acc[i + half] : acc[i];
                acc[i] = keep + __shfl_xor(send, o);
            }
            if (hi) base += half;
        } else {
            acc[0] += __shfl_xor(acc[0], o);
        }
    }
    constexpr int HELD = LOG_RW < LOG_V ? (V >> LOG_RW) : 1;
    const bool writer = LOG_RW <= LOG_V || (rl >> LOG_V) == 0;
    if (writer) {
#pragma unroll
        for (int j = 0; j < HELD; ++j) {
            const int i = base + j;
            const int m = i / E, e = i % E;
            red[wave * NOUT + m * SC + cl * E + e] = acc[j];
        }
    }
    __syncthreads();

    float pv[OPT];
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
        const int o = tid + j * kThreads;
        float p = 0.0f;
        if (o < NOUT) {
            p = red[o];
#pragma unroll
            for (int w = 1; w < kWaves; ++w) p += red[w * NOUT + o];
        }
        pv[j] = p;
    }

    const int col0 = seg * SC;
    auto epilogue = [&](int o, float p) __attribute__((always_inline)) {
        const int m = o / SC, col = col0 + o % SC;
        float *cp = a.C + (size_t)m * a.N + col;
        float v = (a.colscale ? a.alpha * a.colscale[col] : a.alpha) * p;
        if (a.beta != 0.0f) v += a.beta * *cp;
        if (a.bias) v += a.bias[col];
        const long long flat = (long long)m * a.N + col;
        if (a.res) v += a.res[flat];
        *cp = tml_apply_act(v, a.act, flat, a.tail0);
    };
    auto useful = [&](int o) __attribute__((always_inline)) {
        return o < NOUT && o / SC < a.M && col0 + o % SC < a.N;
    };

    if (a.nsplit == 1) {
#pragma unroll
        for (int j = 0; j < OPT; ++j) {
            const int o = tid + j * kThreads;
            if (useful(o)) epilogue(o, pv[j]);
        }
        return;
    }

    // Split-K exchange (see the header comment).
    const size_t plane = (size_t)MR * a.N;
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
        const int o = tid + j * kThreads;
        if (useful(o)) store_agent(a.ws + split * plane + (size_t)(o / SC) * a.N + col0 + o % SC, pv[j]);
    }
    wait_vm0();  // this thread's partial stores have completed
    __syncthreads();
    if (tid == 0)
        arrived = __hip_atomic_fetch_add(a.counters + seg, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    if (arrived != (unsigned)(a.nsplit - 1)) return;
    // Issue the loads of up to kXB splits at once (each is a memory round
    // trip), then add them in split order.
    constexpr int kXB = 8;
#pragma unroll
    for (int j = 0; j < OPT; ++j) {
        const int o = tid + j * kThreads;
        const bool use = useful(o);
        const float *src = a.ws + (use ? (size_t)(o / SC) * a.N + col0 + o % SC : 0);
        float p = 0.0f;
        for (int s0 = 0; s0 < a.nsplit; s0 += kXB) {
            float t[kXB];
#pragma unroll
            for (int i = 0; i < kXB; ++i) {
                const int s = min(s0 + i, a.nsplit - 1);
                t[i] = use ? load_agent(src + s * plane) : 0.0f;
            }
#pragma unroll
            for (int i = 0; i < kXB; ++i)
                if (s0 + i < a.nsplit) p += (s0 + i == split) ? pv[j] : t[i];
        }
        if (use) epilogue(o, p);
    }
    if (tid == 0) __hip_atomic_store(a.counters + seg, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ---------------------------------------------------------------- host side
struct GemvPlan {
    int mr, lw, e, lpr, u, sc, rb;
    int nseg, nsplit, nb;
    int mode;         // kGeneric / kAligned / kRagged
    unsigned bbytes;  // kRagged: byte count of B
};

constexpr int kU = 4;         // loads per lane per batch
constexpr int kMaxSplit = 8;  // default cap on K splits per segment

int pick_lw(int fmt, int mr) {
    switch (fmt) {
        case TML_FMT_F32:
        case TML_FMT_F16: return 16;
        case TML_FMT_Q8_0:
        case TML_FMT_Q8_K: return mr <= 4 ? 16 : 8;
        default: return mr <= 2 ? 16 : (mr == 4 ? 8 : 4);  // Q4_0
    }
}

int elems_per_lane(int fmt, int lw) {
    return fmt == TML_FMT_F32 ? lw / 4 : fmt == TML_FMT_F16 ? lw / 2 : (fmt == TML_FMT_Q4_0 ? 2 * lw : lw);
}

bool is_aligned(const void *p, size_t n) { return ((uintptr_t)p % n) == 0; }

int gemv_cus() {
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

// Segment width: the narrowest segment of at least one 128-byte line per
// row that wastes little of the last segment; narrower segments mean fewer
// K splits (less partial traffic) at the cost of more shuffle steps.
// Batches per workgroup: one (maximum parallelism, every load issued at
// once) until the grid would exceed a few workgroups per CU.
GemvPlan make_plan(const MatmulArgs &m) {
    GemvPlan p{};
    p.mr = m.M <= 1 ? 1 : m.M <= 2 ? 2 : m.M <= 4 ? 4 : 8;
    p.lw = pick_lw(m.fmt, p.mr);
    p.e = elems_per_lane(m.fmt, p.lw);
    p.u = kU;
    const int64_t bpe_num = m.fmt == TML_FMT_F32 ? 4 : (m.fmt == TML_FMT_F16 ? 2 : 1),
                  bpe_den = m.fmt == TML_FMT_Q4_0 ? 2 : 1;
    const int64_t rowbytes = (m.N * bpe_num + bpe_den - 1) / bpe_den;
    bool aligned = (m.N % p.e == 0) && is_aligned(m.B, (size_t)p.lw);
    if (m.fmt == TML_FMT_Q8_K) aligned = aligned && (m.block % p.e == 0) && (m.N % m.block == 0);
    // Ragged rows (N not a whole number of chunks, e.g. a 51866-token
    // vocabulary): Q8_0 / Q4_0 / f32 1280x51866 M = 1 94.4 / 77.0 / 80.2 us
    // on the element-wise path, 19.4 / 15.8 / 50.3 us on the ragged-row
    // loads.  The buffer resource's 32-bit range bounds B at 2 GiB.
    const int64_t bbytes = (m.K * m.N * bpe_num + bpe_den - 1) / bpe_den;
    const bool ragged_ok = m.fmt != TML_FMT_Q8_K && is_aligned(m.B, 4) && bbytes <= ((int64_t)1 << 31) - 64 &&
                           env_int("TML_GEMV_RAGGED", 1) != 0;
    p.mode = aligned ? kAligned : ragged_ok ? kRagged : kGeneric;
    p.bbytes = (unsigned)(ragged_ok ? bbytes : 0);
    // Segment width per row: 128 bytes (one line) for f32, 64 bytes for
    // quantized B at M <= 2 and 32 bytes at M > 2 -- measured best on MI355X
    // at the decoder shapes (narrower segments scatter the loads over more
    // lines, wider ones need more K splits and, with many partial sums per
    // lane, fewer but costlier reduction steps); rows narrower than that get
    // the narrowest segment that covers them.  Q4_0 at M > 4 (4 bytes per
    // lane) takes 16 bytes, four lanes per row like the other quantized
    // plans at M > 2: 5120x1280 M = 8 14.4 -> 11.3 us, 1280x5120 10.39 ->
    // 10.22 us (a sweep of every segment width and batches per split).
    int seg_bytes = (m.fmt == TML_FMT_F32 || m.fmt == TML_FMT_F16) ? 128
                  : p.mr <= 2                                  ? 64
                  : (m.fmt == TML_FMT_Q4_0 && p.mr > 4)        ? 16
                                                               : 32;
    // Weights streaming 16 MiB or more (vocabulary projections) take wider
    // segments.  At 1280 x 51866: Q8_0 / Q4_0 at M = 1 22.7 / 21.6 us ->
    // 19.4 / 15.8 us with 256 bytes a row, at M = 2 24.9 / 27.5 -> 22.1 /
    // 19.3 us; f32 at M = 1 / 4 54.0 / 61.1 us -> 50.3 / 55.1 us with 1 KiB.
    // F16 at M = 1 32.4 -> 31.3 us with 1 KiB.  Quantized at M = 4 the
    // narrow segments stay best (32.3 against 33.8 us), and so do F16 at
    // M = 4 (39.7 against 51.4 us) and layer-sized weights (3-5 MB).
    if (bbytes >= ((int64_t)16 << 20)) {
        if ((m.fmt == TML_FMT_Q8_0 || m.fmt == TML_FMT_Q4_0) && p.mr <= 2) seg_bytes = 256;
        else if ((m.fmt == TML_FMT_F32 && p.mr <= 4) || (m.fmt == TML_FMT_F16 && p.mr == 1)) seg_bytes = 1024;
    }
    int lpr = seg_bytes / p.lw;
    if (lpr < 4) lpr = 4;
    if (rowbytes < seg_bytes) {
        lpr = 4;
        while (lpr < 64 && (int64_t)lpr * p.lw < rowbytes) lpr *= 2;
    }
    // One lane a row (16 int8 columns a lane) for Q8_0 at M <= 4 when that
    // still gives every CU a segment and K fits one batch: no K split, so no
    // partial-sum exchange.  1024x4096 at M = 1 / 2 / 4: 6.25 / 6.83 / 7.75
    // -> 5.46 / 6.05 / 7.21 us.  Slower at M = 8 (8.3 -> 10.5 us) and for
    // Q4_0 and f32 at their layer shapes.
    if (m.fmt == TML_FMT_Q8_0 && aligned && p.mr <= 4 && m.K <= (int64_t)kWaves * 64 * kU &&
        m.N / p.e >= gemv_cus())
        lpr = 1;
    const int forced_lpr = env_int("TML_GEMV_LPR", 0);
    if (forced_lpr == 4 || forced_lpr == 8 || forced_lpr == 16 || forced_lpr == 32 || forced_lpr == 64)
        lpr = forced_lpr;
    if ((forced_lpr == 1 || forced_lpr == 2) && aligned) lpr = forced_lpr;  // one or two lanes a row
    if (p.mode == kGeneric) lpr = 16;  // the generic path is instantiated for one shape
    p.lpr = lpr;
    p.sc = lpr * p.e;
    p.rb = kWaves * (64 / lpr) * p.u;
    p.nseg = (int)((m.N + p.sc - 1) / p.sc);
    const int64_t tb = m.K > 0 ? (m.K + p.rb - 1) / p.rb : 1;  // batches along K
    // K splits: enough workgroups for about two per CU, but at most
    // kMaxSplit per segment -- every split adds an arrival on the segment's
    // counter, and those atomics serialise.
    const int cus = gemv_cus();
    int64_t nb = 1;
    const int forced_nb = env_int("TML_GEMV_NB", 0);
    if (forced_nb > 0) {
        nb = forced_nb;
    } else {
        const int64_t max_split = env_int("TML_GEMV_MAXSPLIT", kMaxSplit);
        int64_t want = (2 * (int64_t)cus + p.nseg - 1) / p.nseg;
        if (want > max_split) want = max_split;
        if (want < 1) want = 1;
        nb = (tb + want - 1) / want;
    }
    if (nb > tb) nb = tb;
    if (nb < 1) nb = 1;
    p.nb = (int)nb;
    p.nsplit = (int)((tb + nb - 1) / nb);
    return p;
}

template <int FMT, int MR, int LW, int LPR, int MODE>
void launch_one(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    gemv_kernel<FMT, MR, LW, LPR, kU, MODE><<<dim3((unsigned)(p.nseg * p.nsplit)), dim3(kThreads), 0, s>>>(ka);
}

template <int FMT, int MR, int LW, int MODE>
void launch_mode(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    if constexpr (MODE == kAligned) {
        if (p.lpr == 1) return launch_one<FMT, MR, LW, 1, MODE>(ka, p, s);
        if (p.lpr == 2) return launch_one<FMT, MR, LW, 2, MODE>(ka, p, s);
    }
    switch (p.lpr) {
        case 4: launch_one<FMT, MR, LW, 4, MODE>(ka, p, s); break;
        case 8: launch_one<FMT, MR, LW, 8, MODE>(ka, p, s); break;
        case 16: launch_one<FMT, MR, LW, 16, MODE>(ka, p, s); break;
        case 32: launch_one<FMT, MR, LW, 32, MODE>(ka, p, s); break;
        default: launch_one<FMT, MR, LW, 64, MODE>(ka, p, s); break;
    }
}

template <int FMT, int MR, int LW>
void launch_lpr(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    if (p.mode == kGeneric) {
        launch_one<FMT, MR, LW, 16, kGeneric>(ka, p, s);
        return;
    }
    if constexpr (FMT != TML_FMT_Q8_K) {
        if (p.mode == kRagged) {
            launch_mode<FMT, MR, LW, kRagged>(ka, p, s);
            return;
        }
    }
    launch_mode<FMT, MR, LW, kAligned>(ka, p, s);
}

template <int FMT, int MR>
Status launch_mr(const GemvKArgs &ka, const GemvPlan &p, hipStream_t s) {
    constexpr int LW = (FMT == TML_FMT_F32 || FMT == TML_FMT_F16) ? 16
                     : (FMT == TML_FMT_Q4_0 ? (MR <= 2 ? 16 : (MR == 4 ? 8 : 4)) : (MR <= 4 ? 16 : 8));
    if (p.lw != LW) return Status::Err(TML_ERR_INVALID_ARG, "gemv plan/instantiation mismatch");
    launch_lpr<FMT, MR, LW>(ka, p, s);
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
    // TML_GEMV_RAGGED=2 (tests): refuse a call that would not take the
    // ragged-row loads, so a test proves that they ran
    if (p.mode != kRagged && env_int("TML_GEMV_RAGGED", 1) == 2)
        return Status::Err(TML_ERR_INVALID_ARG, "TML_GEMV_RAGGED=2: this call does not take the ragged-row loads");
    // TML_REQUIRE_SPLIT=1 (tests): refuse a plan that does not split K, so a
    // test of the split-K partials and counters proves that they were used
    if (p.nsplit <= 1 && env_int("TML_REQUIRE_SPLIT", 0) == 1)
        return Status::Err(TML_ERR_INVALID_ARG, "TML_REQUIRE_SPLIT=1: this call's plan does not split K");
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
    ka.nseg = p.nseg; ka.nsplit = p.nsplit; ka.nb = p.nb;
    ka.ws = ws.partials; ka.counters = ws.counters;
    ka.zero = m.zero;
    ka.bbytes = p.bbytes;
    ka.act = m.act; ka.res = m.res; ka.colscale = m.colscale; ka.tail0 = tml_act_tail0((long long)m.M * m.N);
    switch (m.fmt) {
        case TML_FMT_F32: return launch_fmt<TML_FMT_F32>(ka, p, s);
        case TML_FMT_Q8_0: return launch_fmt<TML_FMT_Q8_0>(ka, p, s);
        case TML_FMT_Q8_K: return launch_fmt<TML_FMT_Q8_K>(ka, p, s);
        case TML_FMT_Q4_0: return launch_fmt<TML_FMT_Q4_0>(ka, p, s);
        case TML_FMT_F16: return launch_fmt<TML_FMT_F16>(ka, p, s);
        default: return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    }
}

}  // namespace tml
