// Internal declarations shared by the HIP translation units of libtomoul_hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/tomoul_hip.h"

// A kernel's dynamically sized LDS array (the launch's shared-memory bytes).
#ifndef TML_DYNAMIC_LDS
#define TML_DYNAMIC_LDS(T, v) extern __shared__ T v[]
#endif

namespace tml {

// Status carrying a TML_ERR_* code and a message; ok() when code == TML_OK.
struct Status {
    int code = TML_OK;
    std::string msg;
    bool ok() const { return code == TML_OK; }
    static Status Ok() { return {}; }
    static Status Err(int c, std::string m) { return {c, std::move(m)}; }
};

Status hip_status(hipError_t e, const char *what);

#define TML_HIP_TRY(expr)                                              \
    do {                                                               \
        hipError_t _e = (expr);                                        \
        if (_e != hipSuccess) return ::tml::hip_status(_e, #expr);     \
    } while (0)

#define TML_TRY(expr)                                                  \
    do {                                                               \
        ::tml::Status _s = (expr);                                     \
        if (!_s.ok()) return _s;                                       \
    } while (0)

// One GEMM / GEMV problem on device-resident operands:
//   C = alpha_eff * (A . Bdeq) + beta * C + bias
// where Bdeq is the f32 value of B's element (for Q8_0 / Q4_0 the integer
// value; their per-tensor scale is folded into alpha_eff, a per-column scale
// multiplies column n of A.Bdeq: alpha_eff * colscale[n]), then
//   C = act(C + res)
// with an optional [M,N] residual `res` (read before C is written, per
// element, so it may alias C) and activation `act`.
struct MatmulArgs {
    int64_t M, N, K;
    const float *A;        // [M,K] row-major
    const void *B;         // [K,N] row-major in format fmt
    const float *scales;   // Q8_K block scales (device) or nullptr
    int64_t block;         // Q8_K block size
    const float *bias;     // [N] or nullptr
    float *C;              // [M,N] row-major
    float alpha_eff;       // alpha * per-tensor scale
    float beta;
    int fmt;
    const void *zero;      // >= 64 zero bytes of device memory (see below)
    int act = TML_ACT_NONE;  // activation after the bias (TML_ACT_*)
    const float *res = nullptr;  // [M,N] residual added after the bias (may equal C)
    const float *colscale = nullptr;  // [N] per-column factor on A.B (per-channel formats), or nullptr
};

// Activations of the epilogue, restating the reference's CPU code.
// erf: Abramowitz & Stegun 7.1.26 exactly as src/core/ops.zig:2000-2022
// (the published five-term approximation, |error| <= 1.5e-7).
__device__ __forceinline__ float tml_erf_as(float x) {
    const float a1 = 0.254829592f, a2 = -0.284496736f, a3 = 1.421413741f, a4 = -1.453152027f,
                a5 = 1.061405429f, p = 0.3275911f;
    const float sign = x < 0.0f ? -1.0f : 1.0f;
    const float ax = fabsf(x);
    const float t = 1.0f / (1.0f + p * ax);
    const float t2 = t * t, t3 = t2 * t, t4 = t3 * t, t5 = t4 * t;
    const float y = 1.0f - (a1 * t + a2 * t2 + a3 * t3 + a4 * t4 + a5 * t5) * expf(-ax * ax);
    return sign * y;
}
// v -> act(v) for the element at flat index `flat` of C; tail0 = M*N minus
// (M*N) % 8 is where the reference's 8-wide loops hand over to their
// scalar tail (ops.gelu uses exact tanh there, a Pade approximant before).
__device__ __forceinline__ float tml_apply_act(float v, int act, long long flat, long long tail0) {
    if (act == TML_ACT_GELU_ERF) {
        const float inv_sqrt_2 = 0.7071067811865476f;
        return v * 0.5f * (1.0f + tml_erf_as(v * inv_sqrt_2));  // ops.zig:2029-2057
    }
    if (act == TML_ACT_GELU_TANH) {
        const float sqrt_2_over_pi = 0.7978845608f, coeff = 0.044715f;  // ops.zig:1947-1998
        const float inner = sqrt_2_over_pi * (v + coeff * (v * v * v));
        float th;
        if (flat < tail0) {
            const float x2 = inner * inner;
            th = fminf(1.0f, fmaxf(-1.0f, inner * (27.0f + x2) / (27.0f + 9.0f * x2)));
        } else {
            th = tanhf(inner);
        }
        return 0.5f * v * (1.0f + th);
    }
    return v;
}
__host__ __device__ __forceinline__ long long tml_act_tail0(long long mn) { return mn - mn % 8; }

// Final C stores of the GEMM epilogues (a float or a 16-byte vector of them
// at p) are non-temporal: no workgroup of the launch reads C back, so the
// lines stream out to memory while other tiles still compute, instead of
// sitting dirty in the XCD's L2 until the end-of-kernel release writes them
// back in one burst.  Measured on MI355X: 1500x1536x384 with bias 20.5 ->
// 19.5 us, 512x1024x1024 15.5 -> 14.5 us, Q8_0 512x4096x1024 22.5 -> 21.7
// us, the long-K shapes unchanged.
template <typename T>
__device__ __forceinline__ void tml_store_c(float *p, T v) {
    __builtin_nontemporal_store(v, reinterpret_cast<T *>(p));
}

// Cache-policy operand of the buffer loads that stream a decoder GEMV's
// weights (each byte read once per launch): the non-temporal bit (NT, bit 1
// of the gfx940-family cache-policy field); plain-pointer loads get the same
// policy from __builtin_nontemporal_load.  Used only where one load
// instruction covers whole 128-byte lines: the prepared-layout kernels
// (gemv_t.hip, gemv_x.hip) and the read floor (stream_read.hip).  The
// activations, which every workgroup re-reads, keep the default policy, and
// so do kernels whose lanes read parts of a line that later loads complete
// (gemv_tm.hip's 64-byte row pieces, gemv.hip's ragged rows): there it
// measured slower, up to 19.4 -> 22.8 us for the Q8_0 vocabulary on [K,N].
// Measured on MI355X with every launch reading its own copy out of >= 1
// GiB: the plain 4 MB read 2.90 -> 2.65 us; M = 1 Q8_0 1024x4096 3.17 ->
// 2.83 us, Q4_0 1280x5120 3.60 -> 3.27 us, 5120x1280 3.73 -> 3.48 us.
constexpr int kStreamLoadPolicy = 2;

// Kernels load out-of-range chunks from this zeroed block instead of
// branching around the load: the selected address keeps the load
// unconditional, which lets the compiler keep whole batches of global loads
// in flight (a branch around a load makes it wait for all earlier loads).
constexpr size_t kZeroBlockBytes = 64;

// Cross-workgroup exchange of split-K partials.  A device-scope fence
// (__threadfence) on MI355X writes back / invalidates the XCD's whole L2 and
// costs tens of microseconds per launch, so kernels that combine partials
// never use one.  Instead the partials themselves are written and read with
// agent-scope atomic stores / loads (coherent across the XCDs by
// construction), each writer waits for its stores to complete (vmcnt(0))
// before its workgroup bumps the tile's arrival counter, and the last
// workgroup to arrive reads the other partials and finishes the tile.
__device__ __forceinline__ void xchg_store(float *p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float xchg_load(const float *p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// s_waitcnt vmcnt(0) with the other counters left alone (gfx9 encoding).
__device__ __forceinline__ void xchg_wait_stores() { __builtin_amdgcn_s_waitcnt((0x7 << 4) | (0xF << 8)); }
// Bumps *counter once for the workgroup (after every thread has waited for
// its partial stores) and returns, to every thread, the number of
// workgroups that arrived before this one.  `slot` is a __shared__ word.
__device__ __forceinline__ unsigned xchg_arrive(unsigned *counter, unsigned *slot) {
    xchg_wait_stores();
    __syncthreads();
    if (threadIdx.x == 0)
        *slot = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __syncthreads();
    return *slot;
}
__device__ __forceinline__ void xchg_reset(unsigned *counter) {
    if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Split-K workspace handed to kernels that reduce across workgroups.
struct Workspace {
    float *partials = nullptr;      // nsplit * M * N floats
    size_t partial_floats = 0;
    unsigned *counters = nullptr;   // one per output segment, zero between launches
    size_t counter_count = 0;
};

// Kernel-family launchers (asynchronous).  Each validates that the problem
// fits what its kernels assume before launching.
// Tiled GEMM families for M > kGemvMaxM.  The plan (kernel, tile, K splits)
// is a pure function of the problem, so workspace sizing and launch agree.
struct GemmPlan {
    bool dma = false;  // direct-copy fp32 kernel (gemm_dma.hip)
    int cfg = 0;       // tile config of that kernel family
    int nsplit = 1;    // K splits (dma kernel only)
    int spl = 0;       // BK-slices per split
    int tiles = 0;
    bool fused = false;  // split-K partials combined in the GEMM kernel (no reduce launch)
    bool qbf = false;    // Q8_0 / Q4_0 on the bf16 matrix cores (gemm_qbf.hip; cfg, nsplit, spl its plan)
};
GemmPlan plan_gemm(const MatmulArgs &a);
void gemm_workspace_need(const MatmulArgs &a, size_t *partial_floats, size_t *counters);
Status launch_gemm_mfma(const MatmulArgs &a, const Workspace &ws, hipStream_t s);
// fp32 GEMM with direct global->LDS copies (gemm_dma.hip); supported when
// K % 4 == N % 4 == 0 and A, B are 16-byte aligned.
bool gemm_dma_supported(const MatmulArgs &a);
int gemm_dma_num_cfgs();
bool gemm_dma_cfg_ok(int cfg, int fmt);  // the tile config has a kernel for B format fmt
void gemm_dma_tile(int cfg, int *bm, int *bn, int *bk);
bool gemm_dma_cfg_fusable(int cfg);  // the tile config can combine K splits in the kernel
Status launch_gemm_f32_dma(const MatmulArgs &a, const GemmPlan &p, const Workspace &ws, hipStream_t s);
// Q8_0 / Q4_0 weight-only GEMM on the bf16 matrix cores (gemm_qbf.hip):
// M > kGemvMaxM, K % 8 == 0, even N, 16-byte aligned A.  pick_qbf sets
// p->cfg / nsplit / spl; K splits write nsplit * M * N partial floats that
// launch_splitk_reduce sums.
bool gemm_qbf_supported(const MatmulArgs &a);
void pick_qbf(const MatmulArgs &a, GemmPlan *p);
Status launch_gemm_qbf(const MatmulArgs &a, const GemmPlan &p, const Workspace &ws, hipStream_t s);
// C = act(alpha * sum of the nsplit [M,N] partials (in split order) * colscale + beta * C + bias + res).
Status launch_splitk_reduce(const float *partials, int nsplit, const MatmulArgs &a, hipStream_t s);
void gemm_dma_workspace_need(const MatmulArgs &a, const GemmPlan &p, size_t *partial_floats, size_t *counters);
Status launch_gemv(const MatmulArgs &a, const Workspace &ws, hipStream_t s);
// Workspace needed by launch_gemv for this problem.
void gemv_workspace_need(const MatmulArgs &a, size_t *partial_floats, size_t *counters);
Status launch_quantize(int fmt, int64_t n, const float *w, void *q, float *scales, float *tmp_max,
                       hipStream_t s);
size_t quantize_tmp_floats(int fmt, int64_t n);
// Per-output-column Q8_0 / Q4_0 quantizer of W[K,N]: scales[N]; tmp holds N floats.
Status launch_quantize_cols(int fmt, int64_t K, int64_t N, const float *w, void *q, float *scales, float *tmp,
                           hipStream_t s);

// Largest M routed to the GEMV family (skinny decoder shapes).
constexpr int64_t kGemvMaxM = 8;

// Prepared (device-native, K-contiguous) weights for decoder GEMVs
// (gemv_t.hip): row n holds column n of B, zero padded to a multiple of 16
// bytes; int4 keeps two k per byte, even k in the low nibble.
constexpr int64_t kPreparedGemvMaxM = 8;  // every prepared format
int64_t prepared_row_bytes(int fmt, int64_t K);
bool prepared_gemv_supported(int fmt, int64_t M, int64_t K);
// Whether the prepared kernels are the faster choice at M rows (K deep)
// when the [K,N] weight is also at hand.
bool prepared_gemv_preferred(int fmt, int64_t M, int64_t K);
// Matrix-core decoder GEMV on a prepared Q8_0 / Q4_0 weight (gemv_tm.hip):
// K a whole number of chunks (16 int8 / 32 int4 elements); chosen for M =
// 3..8, M = 2 on short Q4_0 rows, and Q4_0 M = 1 on vocabulary-sized N.
bool gemv_tm_supported(int fmt, int64_t M, int64_t K);
bool gemv_tm_m1_preferred(int fmt, int64_t N, int64_t K);
Status launch_gemv_tm(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *Bt, int64_t ldt,
                      const float *bias, const float *res, float *C, float alpha_eff, float beta, int act,
                      long long tail0, const float *colscale, hipStream_t s);
// Staged-activation decoder GEMV on a prepared Q8_0 / Q4_0 weight
// (gemv_x.hip): M = 1 or 2, K a whole number of chunks; preferred below
// vocabulary-sized N.
bool gemv_x_capable(int fmt, int64_t M, int64_t N, int64_t K);
bool gemv_x_preferred(int fmt, int64_t M, int64_t N, int64_t K);
Status launch_gemv_x(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *Bt, int64_t ldt,
                     const float *bias, const float *res, float *C, float alpha_eff, float beta, int act,
                     long long tail0, const float *colscale, hipStream_t s);
// Bytes of one row of K elements of fmt in the reference's packing (Q4_0:
// two per byte), before the 16-byte padding of a prepared row.
inline int64_t packed_row_bytes(int fmt, int64_t K) {
    return fmt == TML_FMT_F32 ? 4 * K : fmt == TML_FMT_F16 ? 2 * K : (fmt == TML_FMT_Q4_0 ? (K + 1) / 2 : K);
}

// binary16 bits -> f32 (exact, as the reference's @floatCast(f16)).
__device__ __forceinline__ float tml_half_bits(uint32_t bits16) {
    return (float)__builtin_bit_cast(_Float16, (unsigned short)bits16);
}
Status launch_prepare_t(int fmt, int64_t K, int64_t N, const void *B, void *Bt, int64_t ldt, hipStream_t s);
// The same layout from W = B^T stored as N rows of K elements, ldw bytes apart
// (Q4_0: K even, each row starting a byte).
Status launch_prepare_rows(int fmt, int64_t K, int64_t N, const void *W, int64_t ldw, void *Bt, int64_t ldt,
                           hipStream_t s);
Status launch_gemv_t(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *Bt, int64_t ldt,
                     const float *bias, const float *res, float *C, float alpha_eff, float beta,
                     const void *zero, int act, long long tail0, const float *colscale, hipStream_t s);
// Largest M the prepared kernel covers for fmt (8 f32, 4 Q8_0, 2 Q4_0).
int64_t prepared_gemv_max_m(int fmt);

// .tl files (tl.hip).
struct TlTensor {
    std::string name;
    std::vector<int64_t> shape;
    uint64_t offset = 0, size = 0;
};
struct TlFile {
    std::vector<uint8_t> owned;  // the file's bytes (tml_tl_open) ...
    const uint8_t *data = nullptr;  // ... or the caller's (tml_tl_open_bytes)
    uint64_t size = 0;
    uint32_t version = 0;
    int format = 0;                  // TML_FMT_*
    std::vector<TlTensor> tensors;   // file order
    std::unordered_map<std::string, size_t> index;  // name -> last entry of that name
};
// A validated payload: `data` (data_bytes), Q8_K `scales` (nscales floats,
// unaligned in the file), Q8_0 / Q4_0 `scale`.
struct TlParts {
    int fmt = 0;
    int64_t numel = 0;
    const uint8_t *data = nullptr;
    uint64_t data_bytes = 0;
    const uint8_t *scales = nullptr;
    uint64_t nscales = 0;
    float scale = 1.0f;
};
Status tl_open_file(const char *path, TlFile **out);
Status tl_open_bytes(const void *data, uint64_t size, TlFile **out);
const TlTensor *tl_find(const TlFile *f, const char *name);
// getter's checks (by_file_format = false) or getTensorDequantized's
// (by_file_format = true: the file's format decides, getter is ignored).
Status tl_parts(const TlFile *f, const char *name, int getter, bool by_file_format, TlParts *p);
Status launch_dequant(int fmt, int64_t n, const void *raw, const float *scales, float scale, float *out,
                      hipStream_t s);
Status launch_dequant_transpose(int fmt, int64_t rows, int64_t cols, const void *raw, const float *scales,
                                float scale, float *out, hipStream_t s);

// The GEMV read floor (stream_read.hip): reads `bytes` of src with
// chunks_per_lane 16-byte loads a lane and writes stream_read_outputs()
// partial values to out.
int64_t stream_read_outputs(int64_t bytes, int chunks_per_lane);
Status launch_stream_read(const void *src, int64_t bytes, int chunks_per_lane, float *out, hipStream_t s);

// Tuning overrides for experiments (0 = heuristic).  Read from the
// TML_GEMM_TILE / TML_GEMV_SPLIT environment variables once.
int env_int(const char *name, int dflt);

}  // namespace tml
