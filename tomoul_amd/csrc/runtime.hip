// runtime.hip -- the C ABI of include/tomoul_hip.h: argument validation,
// per-device state (stream, staging buffers, split-K workspace, registered
// weights) and routing to the kernel families:
//   M <= 8            -> gemv.hip  (B streamed once, HBM-bound)
//   M >  8            -> gemm_mfma.hip (LDS-tiled fp32 MFMA, compute-bound)
// The host-pointer entry points wrap the device-pointer one: upload operands
// (or reuse a registered weight), launch, download C, synchronise.
// tml_hip_gemm_ex_dev_noalloc is the device-pointer entry point for callers
// that cannot allocate: its split-K scratch is a static device array.
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "host_copier.hpp"
#include "tml_internal.hpp"

namespace tml {

Status hip_status(hipError_t e, const char *what) {
    const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? TML_ERR_OUT_OF_MEMORY
                     : (e == hipErrorNoDevice || e == hipErrorInvalidDevice) ? TML_ERR_NO_DEVICE
                                                                              : TML_ERR_HIP;
    return Status::Err(code, std::string(what) + ": " + hipGetErrorString(e));
}

int env_int(const char *name, int dflt) {
    const char *v = std::getenv(name);
    if (v == nullptr || *v == '\0') return dflt;
    return std::atoi(v);
}

namespace {

thread_local std::string g_last_error;

int report(const Status &s) {
    g_last_error = s.ok() ? std::string() : s.msg;
    return s.code;
}

// A device allocation that only grows.
struct DevBuf {
    void *p = nullptr;
    size_t bytes = 0;
    Status ensure(size_t n) {
        if (n <= bytes) return Status::Ok();
        if (p) {
            TML_HIP_TRY(hipFree(p));
            p = nullptr;
            bytes = 0;
        }
        TML_HIP_TRY(hipMalloc(&p, n));
        bytes = n;
        return Status::Ok();
    }
    void release() {
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
};

// Pinned host memory that only grows: the staging of the host-pointer entry
// points.  Their calls are synchronous, so no copy still reads a buffer when
// a later call grows it.
struct PinnedBuf {
    void *p = nullptr;
    size_t bytes = 0;
    Status ensure(size_t n) {
        if (n <= bytes) return Status::Ok();
        if (p) {
            TML_HIP_TRY(hipHostFree(p));
            p = nullptr;
            bytes = 0;
        }
        TML_HIP_TRY(hipHostMalloc(&p, n, hipHostMallocDefault));
        bytes = n;
        return Status::Ok();
    }
    void release() {
        if (p) (void)hipHostFree(p);
        p = nullptr;
        bytes = 0;
    }
};

// Device-native copy of a weight for decoder GEMVs (gemv_t.hip).  `B` is
// the [K,N] weight the copy was made from; it is used for row counts the
// prepared kernel does not cover.
struct Prepared {
    int device = -1;
    int fmt = 0;
    int64_t K = 0, N = 0;
    float scale = 1.0f;
    const void *B = nullptr;   // the [K,N] weight, or null for a rows-prepared weight
    void *Bt = nullptr;
    int64_t ldt = 0;
    bool owns_bt = true;       // false: Bt is the caller's buffer, used in place
    float *colscale = nullptr;  // per-channel formats: device copy of the N column scales
    std::vector<float> host_colscale;  // ... and the host values it was made from (host-pointer path)
};

void free_prepared(Prepared *p) {
    if (p == nullptr) return;
    if (p->owns_bt && p->Bt) (void)hipFree(p->Bt);
    if (p->colscale) (void)hipFree(p->colscale);
    delete p;
}

struct Registered {
    void *dev = nullptr;
    size_t bytes = 0;
    Prepared *prep = nullptr;  // made on the first decoder call that uses this weight
};

// A device allocation that only grows and never frees a buffer a launch
// may still reference: the split-K workspace of the asynchronous "_dev"
// entry points.  Their launches may sit in a queue or in a captured HIP
// graph that is replayed later, so a grown buffer replaces the old one in
// new launches only; the old one is released by tml_hip_shutdown.
struct GrowBuf {
    void *p = nullptr;
    size_t bytes = 0;
    std::vector<void *> retired;
    Status ensure(size_t n) {
        if (n <= bytes) return Status::Ok();
        // Grow by at least half again, so that a sequence of rising sizes
        // (a model load reading tensor after tensor) retires few buffers:
        // the retired ones together stay below twice the live one.
        n = std::max(n, bytes + bytes / 2);
        n = (n + 255) & ~(size_t)255;
        void *q = nullptr;
        TML_HIP_TRY(hipMalloc(&q, n));
        if (p) retired.push_back(p);
        p = q;
        bytes = n;
        return Status::Ok();
    }
    void release() {
        for (void *r : retired) (void)hipFree(r);
        retired.clear();
        if (p) (void)hipFree(p);
        p = nullptr;
        bytes = 0;
    }
};

struct DeviceCtx {
    int device = -1;
    hipStream_t stream = nullptr;
    DevBuf a, b, c, bias, res, scales;   // staging of the host-pointer API (synchronous calls)
    PinnedBuf pin_in, pin_out;           // ... and its pinned host side
    std::vector<hipEvent_t> chunk_done;  // ... and the chunks of its downloads
    GrowBuf qtmp, tl_raw, tl_scales, tr;  // quantizer partials, .tl payload staging, transpose temporary
    GrowBuf ws, counters;                // split-K workspace (gemv, gemm)
    DevBuf zero;                         // kZeroBlockBytes of zeros
    std::unordered_map<const void *, Registered> weights;
};

std::mutex g_mu;
std::unordered_map<int, DeviceCtx *> g_ctx;

Status scratch_setup(hipStream_t s, void **base);

Status current_ctx(DeviceCtx **out) {
    int n = 0;
    hipError_t e = hipGetDeviceCount(&n);
    if (e != hipSuccess || n <= 0) return Status::Err(TML_ERR_NO_DEVICE, "no HIP device available");
    int dev = 0;
    TML_HIP_TRY(hipGetDevice(&dev));
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_ctx.find(dev);
    if (it != g_ctx.end()) {
        *out = it->second;
        return Status::Ok();
    }
    DeviceCtx *c = new DeviceCtx();
    c->device = dev;
    e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        delete c;
        return hip_status(e, "hipStreamCreateWithFlags");
    }
    Status zs = c->zero.ensure(kZeroBlockBytes);
    if (zs.ok()) {
        e = hipMemset(c->zero.p, 0, kZeroBlockBytes);
        if (e != hipSuccess) zs = hip_status(e, "hipMemset");
    }
    if (zs.ok()) {
        void *base = nullptr;
        zs = scratch_setup(c->stream, &base);
    }
    if (!zs.ok()) {
        (void)hipStreamDestroy(c->stream);
        c->zero.release();
        delete c;
        return zs;
    }
    g_ctx[dev] = c;
    *out = c;
    return Status::Ok();
}

// Split-K workspace (partial sums and arrival counters) this problem needs.
void workspace_need(const MatmulArgs &m, size_t *partial_floats, size_t *counters) {
    *partial_floats = 0;
    *counters = 0;
    if (m.M <= kGemvMaxM) gemv_workspace_need(m, partial_floats, counters);
    else gemm_workspace_need(m, partial_floats, counters);
}

// Grow the split-K workspace to what this problem needs; new counters are
// zeroed, and the zeroing waited for, before this call returns (kernels
// leave them zero when they finish), so a later call on any stream finds
// them zero.  Growing allocates, so it is refused while `s` is being
// captured into a graph: run every captured call once eagerly first.
Status ensure_workspace(DeviceCtx *c, const MatmulArgs &m, hipStream_t s, Workspace *ws) {
    size_t pf = 0, nc = 0;
    workspace_need(m, &pf, &nc);
    if (pf > 0) {
        const bool grow_ws = pf * sizeof(float) > c->ws.bytes;
        const bool grow_ctr = nc * sizeof(unsigned) > c->counters.bytes;
        if (grow_ws || grow_ctr) {
            hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
            TML_HIP_TRY(hipStreamIsCapturing(s, &cap));
            if (cap != hipStreamCaptureStatusNone)
                return Status::Err(TML_ERR_INVALID_ARG,
                                   "the split-K workspace must grow during stream capture: run this call once "
                                   "eagerly (outside capture) before capturing it");
        }
        TML_TRY(c->ws.ensure(pf * sizeof(float)));
        if (grow_ctr) {
            TML_TRY(c->counters.ensure(nc * sizeof(unsigned)));
            TML_HIP_TRY(hipMemsetAsync(c->counters.p, 0, c->counters.bytes, s));
            TML_HIP_TRY(hipStreamSynchronize(s));
        }
    }
    ws->partials = (float *)c->ws.p;
    ws->partial_floats = c->ws.bytes / sizeof(float);
    ws->counters = (unsigned *)c->counters.p;
    ws->counter_count = c->counters.bytes / sizeof(unsigned);
    return Status::Ok();
}

bool per_channel(int fmt) { return fmt == TML_FMT_Q8_0_PC || fmt == TML_FMT_Q4_0_PC; }
// The kernels' data format of fmt (per-channel formats store Q8_0 / Q4_0 data).
int data_fmt(int fmt) {
    return fmt == TML_FMT_Q8_0_PC ? TML_FMT_Q8_0 : (fmt == TML_FMT_Q4_0_PC ? TML_FMT_Q4_0 : fmt);
}

bool valid_fmt(int fmt) {
    return fmt == TML_FMT_F32 || fmt == TML_FMT_Q8_0 || fmt == TML_FMT_Q4_0 || fmt == TML_FMT_Q8_K ||
           fmt == TML_FMT_F16 || per_channel(fmt);
}

// Bytes of a K x N weight in format fmt.
size_t weight_bytes(int fmt, int64_t K, int64_t N) {
    const size_t e = (size_t)K * (size_t)N;
    switch (data_fmt(fmt)) {
        case TML_FMT_F32: return e * 4;
        case TML_FMT_F16: return e * 2;
        case TML_FMT_Q4_0: return (e + 1) / 2;
        default: return e;
    }
}

bool valid_act(int act) { return act == TML_ACT_NONE || act == TML_ACT_GELU_ERF || act == TML_ACT_GELU_TANH; }

// Validates a device-pointer matmul and fills its MatmulArgs (zero block
// and workspace excepted).  *empty: nothing to compute (M == 0 or N == 0).
Status matmul_args(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                   const float *scales, int64_t block, const float *bias, float *C, float alpha, float beta,
                   int act, const float *res, MatmulArgs *m, bool *empty) {
    *empty = false;
    if (!valid_fmt(fmt)) return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    if (!valid_act(act)) return Status::Err(TML_ERR_INVALID_ARG, "unknown activation");
    if (M < 0 || N < 0 || K < 0) return Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension");
    if (M == 0 || N == 0) {
        *empty = true;
        return Status::Ok();
    }
    if (C == nullptr || (K > 0 && (A == nullptr || B == nullptr)))
        return Status::Err(TML_ERR_INVALID_ARG, "null matrix pointer");
    if (fmt == TML_FMT_Q8_K && (block <= 0 || (K > 0 && scales == nullptr)))
        return Status::Err(TML_ERR_INVALID_ARG, "Q8_K needs scales and a positive block size");
    if (per_channel(fmt) && scales == nullptr)
        return Status::Err(TML_ERR_INVALID_ARG, "per-channel formats need their N column scales");
    m->M = M; m->N = N; m->K = K;
    m->A = A; m->B = B; m->block = fmt == TML_FMT_Q8_K ? block : 1;
    m->scales = fmt == TML_FMT_Q8_K ? scales : nullptr;
    m->colscale = per_channel(fmt) ? scales : nullptr;
    m->bias = bias; m->C = C; m->beta = beta; m->fmt = data_fmt(fmt);
    m->alpha_eff = (fmt == TML_FMT_Q8_0 || fmt == TML_FMT_Q4_0) ? alpha * scale : alpha;
    m->act = act;
    m->res = res;
    return Status::Ok();
}

Status launch_matmul(const MatmulArgs &m, const Workspace &ws, hipStream_t s) {
    if (m.M <= kGemvMaxM) return launch_gemv(m, ws, s);
    return launch_gemm_mfma(m, ws, s);
}

Status gemm_dev(DeviceCtx *c, int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B,
                float scale, const float *scales, int64_t block, const float *bias, float *C, float alpha,
                float beta, hipStream_t s, int act = TML_ACT_NONE, const float *res = nullptr) {
    MatmulArgs m;
    bool empty = false;
    TML_TRY(matmul_args(fmt, M, N, K, A, B, scale, scales, block, bias, C, alpha, beta, act, res, &m, &empty));
    if (empty) return Status::Ok();
    m.zero = c->zero.p;
    Workspace ws;
    TML_TRY(ensure_workspace(c, m, s, &ws));
    return launch_matmul(m, ws, s);
}

// ---------------------------------------------- allocation-free scratch
// The split-K scratch of tml_hip_gemm_ex_dev_noalloc: a static device array
// (each GPU holds its own copy, at its own address, for the life of the
// process), never allocated or freed by the library.  Layout:
//   [0, 256)                 zero block (kernels point out-of-range loads here; never written)
//   [256, 256 + 64 KiB)      arrival counters, zero between launches
//   [kScratchPartialOff, end) split-K partial sums
// Host code uses the address hipGetSymbolAddress returns for the current
// device, never the array's name.
constexpr size_t kScratchBytes = TML_NOALLOC_SCRATCH_BYTES;
constexpr size_t kScratchCounters = 16384;
constexpr size_t kScratchPartialOff = 256 + kScratchCounters * sizeof(unsigned);
static_assert(kScratchPartialOff % 256 == 0 && kScratchPartialOff < kScratchBytes, "scratch layout");
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxScratchDevices = 64;
struct ScratchSlot {
    void *base = nullptr;  // this device's address of `scratch`
    bool ready = false;
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxScratchDevices];

__global__ void zero_words_kernel(unsigned *p, unsigned long long n) {
    const unsigned long long i = (unsigned long long)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

// Once per device, with that device current: look up the device's address
// of `scratch` and clear its zero block and counters (a fill kernel on `s`,
// waited for).  Allocates nothing.  Refused while `s` is being captured.
Status scratch_setup(hipStream_t s, void **base) {
    int dev = 0;
    TML_HIP_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxScratchDevices)
        return Status::Err(TML_ERR_NO_DEVICE, "device id beyond the static scratch table");
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    ScratchSlot &sl = g_scratch[dev];
    if (!sl.ready) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        TML_HIP_TRY(hipStreamIsCapturing(s, &cap));
        if (cap != hipStreamCaptureStatusNone)
            return Status::Err(TML_ERR_INVALID_ARG,
                               "the static scratch of this device is not set up: call tml_hip_init on the device "
                               "(or make one call outside stream capture) first");
        void *p = nullptr;
        TML_HIP_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        const unsigned long long words = kScratchPartialOff / sizeof(unsigned);
        zero_words_kernel<<<dim3((unsigned)((words + 255) / 256)), dim3(256), 0, s>>>((unsigned *)p, words);
        TML_HIP_TRY(hipGetLastError());
        TML_HIP_TRY(hipStreamSynchronize(s));
        sl.base = p;
        sl.ready = true;
    }
    *base = sl.base;
    return Status::Ok();
}

Status gemm_dev_noalloc(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                        const float *scales, int64_t block, const float *bias, float *C, float alpha, float beta,
                        hipStream_t s, int act, const float *res) {
    MatmulArgs m;
    bool empty = false;
    TML_TRY(matmul_args(fmt, M, N, K, A, B, scale, scales, block, bias, C, alpha, beta, act, res, &m, &empty));
    if (empty) return Status::Ok();
    void *base = nullptr;
    TML_TRY(scratch_setup(s, &base));
    // The plan is the one tml_hip_gemm_ex_dev would run (same kernels, same
    // K splits, same bits); a plan whose partial sums do not fit the static
    // scratch is refused, never replaced by a smaller split.
    const size_t cap_floats = (kScratchBytes - kScratchPartialOff) / sizeof(float);
    size_t pf = 0, nc = 0;
    workspace_need(m, &pf, &nc);
    if (pf > cap_floats || nc > kScratchCounters)
        return Status::Err(TML_ERR_INVALID_SHAPE,
                           "this problem's split-K plan needs " + std::to_string(pf * sizeof(float)) +
                               " bytes of partial sums and " + std::to_string(nc) +
                               " counters; the static scratch holds " + std::to_string(cap_floats * sizeof(float)) +
                               " bytes and " + std::to_string(kScratchCounters) +
                               " counters (TML_NOALLOC_SCRATCH_BYTES): use tml_hip_gemm_ex_dev");
    m.zero = base;
    Workspace ws;
    ws.partials = (float *)((unsigned char *)base + kScratchPartialOff);
    ws.partial_floats = cap_floats;
    ws.counters = (unsigned *)((unsigned char *)base + 256);
    ws.counter_count = kScratchCounters;
    return launch_matmul(m, ws, s);
}

bool preparable_fmt(int fmt) {
    return fmt == TML_FMT_F32 || fmt == TML_FMT_F16 || fmt == TML_FMT_Q8_0 || fmt == TML_FMT_Q4_0 || per_channel(fmt);
}

// Builds the prepared copy of the [K,N] device weight B (asynchronous on s).
Status make_prepared(DeviceCtx *c, int fmt, int64_t K, int64_t N, const void *B, float scale,
                     const float *colscale, hipStream_t s, Prepared **out) {
    if (!preparable_fmt(fmt))
        return Status::Err(TML_ERR_INVALID_FORMAT, "prepare: format must be F32, F16, Q8_0, Q4_0 or their per-channel forms");
    if (per_channel(fmt) && colscale == nullptr && N > 0)
        return Status::Err(TML_ERR_INVALID_ARG, "per-channel formats need their N column scales");
    if (K < 0 || N < 0) return Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension");
    if (K >= ((int64_t)1 << 30) || N >= ((int64_t)1 << 30))
        return Status::Err(TML_ERR_INVALID_SHAPE, "prepare: dimension exceeds 2^30");
    if (B == nullptr && K > 0 && N > 0) return Status::Err(TML_ERR_INVALID_ARG, "null weight pointer");
    Prepared *p = new Prepared();
    p->device = c->device;
    p->fmt = fmt;
    p->K = K;
    p->N = N;
    p->scale = scale;
    p->B = B;
    p->ldt = prepared_row_bytes(data_fmt(fmt), K);
    const size_t bytes = (size_t)(N > 0 ? N : 1) * (size_t)p->ldt;
    auto build = [&]() -> Status {
        TML_HIP_TRY(hipMalloc(&p->Bt, bytes));
        if (per_channel(fmt) && N > 0) {
            TML_HIP_TRY(hipMalloc((void **)&p->colscale, (size_t)N * sizeof(float)));
            TML_HIP_TRY(hipMemcpyAsync(p->colscale, colscale, (size_t)N * sizeof(float), hipMemcpyDeviceToDevice, s));
        }
        return N > 0 ? launch_prepare_t(data_fmt(fmt), K, N, B, p->Bt, p->ldt, s) : Status::Ok();
    };
    Status st = build();
    if (!st.ok()) {
        free_prepared(p);
        return st;
    }
    *out = p;
    return Status::Ok();
}

// C = alpha * A . dequant(B) + beta * C + bias with a prepared weight: the
// K-contiguous decoder kernel when it covers M and K, else the [K,N] path.
Status gemm_prepared(DeviceCtx *c, const Prepared *p, int64_t M, const float *A, const float *bias, float *C,
                     float alpha, float beta, hipStream_t s, int act = TML_ACT_NONE,
                     const float *res = nullptr) {
    if (M < 0) return Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension");
    if (!valid_act(act)) return Status::Err(TML_ERR_INVALID_ARG, "unknown activation");
    if (M == 0 || p->N == 0) return Status::Ok();
    if (C == nullptr || (p->K > 0 && A == nullptr)) return Status::Err(TML_ERR_INVALID_ARG, "null matrix pointer");
    const float alpha_eff = (p->fmt == TML_FMT_Q8_0 || p->fmt == TML_FMT_Q4_0) ? alpha * p->scale : alpha;
    const long long tail0 = tml_act_tail0((long long)M * p->N);
    const int dfmt = data_fmt(p->fmt);
    if (prepared_gemv_supported(dfmt, M, p->K) && (p->B == nullptr || prepared_gemv_preferred(dfmt, M, p->K)))
        return launch_gemv_t(dfmt, M, p->N, p->K, A, p->Bt, p->ldt, bias, res, C, alpha_eff, beta, c->zero.p, act,
                             tail0, p->colscale, s);
    if (p->B != nullptr)
        return gemm_dev(c, p->fmt, M, p->N, p->K, A, p->B, p->scale, p->colscale, 0, bias, C, alpha, beta, s, act,
                        res);
    // Rows-prepared weight (no [K,N] form): the prepared kernel over
    // consecutive blocks of rows.  Each launch reads the whole weight, so
    // this serves short prompts; the activation's flat-index split is kept
    // global by shifting tail0 per block.
    const int64_t mr = prepared_gemv_max_m(dfmt);
    for (int64_t r0 = 0; r0 < M; r0 += mr) {
        const int64_t rows = M - r0 < mr ? M - r0 : mr;
        const size_t off = (size_t)r0 * (size_t)p->N;
        TML_TRY(launch_gemv_t(dfmt, rows, p->N, p->K, A + (size_t)r0 * p->K, p->Bt, p->ldt, bias,
                              res ? res + off : nullptr, C + off, alpha_eff, beta, c->zero.p, act,
                              tail0 - (long long)off, p->colscale, s));
    }
    return Status::Ok();
}

// Resident copy of a registered host buffer of at least `bytes`, or null.
const void *resident(DeviceCtx *c, const void *host, size_t bytes) {
    auto it = c->weights.find(host);
    if (it == c->weights.end() || it->second.bytes < bytes) return nullptr;
    return it->second.dev;
}

// Pinned staging of one host-pointer call's inputs.  Each input is copied
// into the pinned buffer by the host copier in chunks of kStageChunk, each
// sent from there asynchronously, so the host copy of one chunk overlaps the
// transfer of the one before.  A call whose inputs (or output) exceed
// kPinnedStageMax sends them from the caller's memory directly.
constexpr size_t kPinnedStageMax = (size_t)256 << 20;
constexpr size_t kStageChunk = (size_t)4 << 20;
size_t stage_round(size_t n) { return (n + 255) & ~(size_t)255; }
struct Stager {
    char *base = nullptr;  // null: not staged
    size_t off = 0;
};

Status upload(DeviceCtx *c, DevBuf &buf, const void *host, size_t bytes, const void **dev, Stager *st) {
    if (bytes == 0) {
        *dev = nullptr;
        return Status::Ok();
    }
    if (const void *r = resident(c, host, bytes)) {
        *dev = r;
        return Status::Ok();
    }
    TML_TRY(buf.ensure(bytes));
    if (st->base) {
        char *pin = st->base + st->off;
        for (size_t o = 0; o < bytes; o += kStageChunk) {
            const size_t len = std::min(kStageChunk, bytes - o);
            HostCopier::get().copy(pin + o, (const char *)host + o, len);
            TML_HIP_TRY(hipMemcpyAsync((char *)buf.p + o, pin + o, len, hipMemcpyHostToDevice, c->stream));
        }
        st->off += stage_round(bytes);
    } else {
        TML_HIP_TRY(hipMemcpyAsync(buf.p, host, bytes, hipMemcpyHostToDevice, c->stream));
    }
    *dev = buf.p;
    return Status::Ok();
}

// Host-pointer call: stage operands, run, copy C back, wait.
Status host_gemm(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                 const float *scales, int64_t block, const float *bias, float *C, float alpha, float beta,
                 int act = TML_ACT_NONE, const float *res = nullptr) {
    if (!valid_fmt(fmt)) return Status::Err(TML_ERR_INVALID_FORMAT, "unknown weight format");
    if (!valid_act(act)) return Status::Err(TML_ERR_INVALID_ARG, "unknown activation");
    if (M < 0 || N < 0 || K < 0) return Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension");
    if (M == 0 || N == 0) return Status::Ok();
    if (C == nullptr || (K > 0 && (A == nullptr || B == nullptr)))
        return Status::Err(TML_ERR_INVALID_ARG, "null matrix pointer");
    if (fmt == TML_FMT_Q8_K && (block <= 0 || (K > 0 && scales == nullptr)))
        return Status::Err(TML_ERR_INVALID_ARG, "Q8_K needs scales and a positive block size");
    if (per_channel(fmt) && scales == nullptr)
        return Status::Err(TML_ERR_INVALID_ARG, "per-channel formats need their N column scales");
    DeviceCtx *c = nullptr;
    TML_TRY(current_ctx(&c));
    const size_t abytes = (size_t)M * K * sizeof(float), bbytes = weight_bytes(fmt, K, N);
    const size_t sbytes = fmt == TML_FMT_Q8_K && K > 0 ? ((size_t)K * N + block - 1) / block * sizeof(float)
                          : per_channel(fmt)           ? (size_t)N * sizeof(float)
                                                       : 0;
    const size_t cbytes = (size_t)M * N * sizeof(float);
    Stager st;
    {
        auto need = [&](const void *h, size_t n) { return h == nullptr || n == 0 || resident(c, h, n) ? 0 : stage_round(n); };
        const size_t total = need(A, abytes) + need(B, bbytes) + need(scales, sbytes) +
                             need(bias, bias ? (size_t)N * sizeof(float) : 0) + need(res, res ? cbytes : 0) +
                             (beta != 0.0f ? stage_round(cbytes) : 0);
        if (total > 0 && total <= kPinnedStageMax) {
            TML_TRY(c->pin_in.ensure(total));
            st.base = (char *)c->pin_in.p;
        }
    }
    const void *dA = nullptr, *dB = nullptr, *dS = nullptr, *dBias = nullptr;
    TML_TRY(upload(c, c->a, A, abytes, &dA, &st));
    TML_TRY(upload(c, c->b, B, bbytes, &dB, &st));
    if (sbytes) TML_TRY(upload(c, c->scales, scales, sbytes, &dS, &st));
    if (bias) TML_TRY(upload(c, c->bias, bias, (size_t)N * sizeof(float), &dBias, &st));
    const void *dRes = nullptr;
    if (res) TML_TRY(upload(c, c->res, res, cbytes, &dRes, &st));
    TML_TRY(c->c.ensure(cbytes));
    if (beta != 0.0f) {
        const void *src = C;
        if (st.base) {
            HostCopier::get().copy(st.base + st.off, C, cbytes);
            src = st.base + st.off;
        }
        TML_HIP_TRY(hipMemcpyAsync(c->c.p, src, cbytes, hipMemcpyHostToDevice, c->stream));
    }
    // A registered weight used at a decoder row count gets (once) and then
    // uses its prepared, K-contiguous copy.
    Registered *reg = nullptr;
    if (preparable_fmt(fmt) && prepared_gemv_supported(data_fmt(fmt), M, K) &&
        prepared_gemv_preferred(data_fmt(fmt), M, K)) {
        auto it = c->weights.find(B);
        if (it != c->weights.end() && it->second.bytes >= weight_bytes(fmt, K, N)) reg = &it->second;
    }
    if (reg) {
        Prepared *p = reg->prep;
        const bool same_cols = !per_channel(fmt) ||
                               (p && p->host_colscale.size() == (size_t)N &&
                                std::memcmp(p->host_colscale.data(), scales, (size_t)N * sizeof(float)) == 0);
        if (p && (p->fmt != fmt || p->K != K || p->N != N || p->scale != scale || !same_cols)) {
            TML_HIP_TRY(hipStreamSynchronize(c->stream));
            free_prepared(p);
            p = reg->prep = nullptr;
        }
        if (!p) {
            TML_TRY(make_prepared(c, fmt, K, N, reg->dev, scale, (const float *)dS, c->stream, &p));
            if (per_channel(fmt)) p->host_colscale.assign(scales, scales + N);
            reg->prep = p;
        }
        TML_TRY(gemm_prepared(c, p, M, (const float *)dA, (const float *)dBias, (float *)c->c.p, alpha, beta,
                              c->stream, act, (const float *)dRes));
    } else {
        TML_TRY(gemm_dev(c, fmt, M, N, K, (const float *)dA, dB, scale, (const float *)dS, block,
                         (const float *)dBias, (float *)c->c.p, alpha, beta, c->stream, act,
                         (const float *)dRes));
    }
    if (cbytes <= kPinnedStageMax) {
        // C down in chunks, each copied out to the caller while the next is
        // still in transfer
        TML_TRY(c->pin_out.ensure(cbytes));
        const size_t nch = (cbytes + kStageChunk - 1) / kStageChunk;
        while (c->chunk_done.size() < nch) {
            hipEvent_t e;
            TML_HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableTiming));
            c->chunk_done.push_back(e);
        }
        char *const pin = (char *)c->pin_out.p;
        for (size_t i = 0; i < nch; ++i) {
            const size_t o = i * kStageChunk, len = std::min(kStageChunk, cbytes - o);
            TML_HIP_TRY(hipMemcpyAsync(pin + o, (const char *)c->c.p + o, len, hipMemcpyDeviceToHost, c->stream));
            TML_HIP_TRY(hipEventRecord(c->chunk_done[i], c->stream));
        }
        for (size_t i = 0; i < nch; ++i) {
            const size_t o = i * kStageChunk, len = std::min(kStageChunk, cbytes - o);
            TML_HIP_TRY(hipEventSynchronize(c->chunk_done[i]));
            HostCopier::get().copy((char *)C + o, pin + o, len);
        }
        return Status::Ok();
    }
    TML_HIP_TRY(hipMemcpyAsync(C, c->c.p, cbytes, hipMemcpyDeviceToHost, c->stream));
    TML_HIP_TRY(hipStreamSynchronize(c->stream));
    return Status::Ok();
}

Status quantize_dev(DeviceCtx *c, int fmt, int64_t n, const float *w, void *q, float *scales, hipStream_t s) {
    if (fmt != TML_FMT_Q8_0 && fmt != TML_FMT_Q4_0 && fmt != TML_FMT_Q8_K && fmt != TML_FMT_F16)
        return Status::Err(TML_ERR_INVALID_FORMAT, "quantize: format must be Q8_0, Q4_0, Q8_K or F16");
    if (n < 0) return Status::Err(TML_ERR_INVALID_SHAPE, "negative element count");
    if ((scales == nullptr && fmt != TML_FMT_F16) || (n > 0 && (w == nullptr || q == nullptr)))
        return Status::Err(TML_ERR_INVALID_ARG, "null pointer");
    if (fmt == TML_FMT_F16) return launch_quantize(fmt, n, w, q, scales, nullptr, s);
    if (n == 0) {
        // The reference's all-zero rule: an empty Q8_0 / Q4_0 tensor gets
        // scale 1 (max|v| == 0); Q8_K has no blocks.
        if (fmt != TML_FMT_Q8_K) {
            const float one = 1.0f;
            TML_HIP_TRY(hipMemcpyAsync(scales, &one, sizeof one, hipMemcpyHostToDevice, s));
            TML_HIP_TRY(hipStreamSynchronize(s));
        }
        return Status::Ok();
    }
    TML_TRY(c->qtmp.ensure(quantize_tmp_floats(fmt, n) * sizeof(float) + 16));
    return launch_quantize(fmt, n, w, q, scales, (float *)c->qtmp.p, s);
}

Status tl_check_getter(int getter) {
    if (getter < TML_FMT_F32 || getter > TML_FMT_F16) return Status::Err(TML_ERR_INVALID_FORMAT, "unknown getter format");
    return Status::Ok();
}
Status tl_need(const TlParts &p, const void *data, const float *scales, const float *scale) {
    if ((p.data_bytes > 0 && data == nullptr) || (p.nscales > 0 && scales == nullptr) ||
        ((p.fmt == TML_FMT_Q8_0 || p.fmt == TML_FMT_Q4_0) && scale == nullptr))
        return Status::Err(TML_ERR_INVALID_ARG, "null destination");
    return Status::Ok();
}

}  // namespace
}  // namespace tml

using namespace tml;

extern "C" {

int tml_hip_init(void) {
    DeviceCtx *c = nullptr;
    return report(current_ctx(&c));
}

void tml_hip_shutdown(void) {
    std::lock_guard<std::mutex> lk(g_mu);
    for (auto &kv : g_ctx) {
        DeviceCtx *c = kv.second;
        int prev = 0;
        (void)hipGetDevice(&prev);
        (void)hipSetDevice(c->device);
        (void)hipDeviceSynchronize();
        for (auto &w : c->weights) {
            free_prepared(w.second.prep);
            (void)hipFree(w.second.dev);
        }
        c->a.release(); c->b.release(); c->c.release(); c->bias.release(); c->res.release();
        c->scales.release(); c->qtmp.release(); c->ws.release(); c->counters.release();
        c->tl_raw.release(); c->tl_scales.release(); c->tr.release();
        c->pin_in.release(); c->pin_out.release();
        for (hipEvent_t e : c->chunk_done) (void)hipEventDestroy(e);
        c->chunk_done.clear();
        c->zero.release();
        if (c->stream) (void)hipStreamDestroy(c->stream);
        (void)hipSetDevice(prev);
        delete c;
    }
    g_ctx.clear();
}

const char *tml_hip_last_error(void) { return g_last_error.c_str(); }

int tml_hip_device_name(char *buf, size_t len) {
    if (buf == nullptr || len == 0) return report(Status::Err(TML_ERR_INVALID_ARG, "null buffer"));
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, c->device);
    if (e != hipSuccess) return report(hip_status(e, "hipGetDeviceProperties"));
    std::snprintf(buf, len, "%s", prop.name);
    return report(Status::Ok());
}

int tml_hip_sgemm(int64_t M, int64_t N, int64_t K, const float *A, const float *B, float *C, float alpha,
                  float beta) {
    return report(host_gemm(TML_FMT_F32, M, N, K, A, B, 1.0f, nullptr, 0, nullptr, C, alpha, beta));
}

int tml_hip_sgemm_bias(int64_t M, int64_t N, int64_t K, const float *A, const float *B, const float *bias,
                       float *C) {
    if (bias == nullptr && M > 0 && N > 0) return report(Status::Err(TML_ERR_INVALID_ARG, "null bias"));
    return report(host_gemm(TML_FMT_F32, M, N, K, A, B, 1.0f, nullptr, 0, bias, C, 1.0f, 0.0f));
}

int tml_hip_sgemv(int64_t M, int64_t N, const float *A, const float *x, float *y, float alpha, float beta) {
    // y[M] = A[M,N] . x[N] is the GEMM C[M,1] = A[M,K=N] . B[K=N,1] with
    // B = x read as an N x 1 row-major matrix (no copy or transpose needed).
    return report(host_gemm(TML_FMT_F32, M, 1, N, A, x, 1.0f, nullptr, 0, nullptr, y, alpha, beta));
}

int tml_hip_sgemm_q8(int64_t M, int64_t N, int64_t K, const float *A, const int8_t *Bq, float scale, float *C) {
    return report(host_gemm(TML_FMT_Q8_0, M, N, K, A, Bq, scale, nullptr, 0, nullptr, C, 1.0f, 0.0f));
}

int tml_hip_sgemm_q8k(int64_t M, int64_t N, int64_t K, const float *A, const int8_t *Bq, const float *scales,
                      int64_t block, float *C) {
    return report(host_gemm(TML_FMT_Q8_K, M, N, K, A, Bq, 1.0f, scales, block, nullptr, C, 1.0f, 0.0f));
}

int tml_hip_sgemm_q4(int64_t M, int64_t N, int64_t K, const float *A, const uint8_t *Bp, float scale, float *C) {
    return report(host_gemm(TML_FMT_Q4_0, M, N, K, A, Bp, scale, nullptr, 0, nullptr, C, 1.0f, 0.0f));
}

int tml_hip_sgemm_f16(int64_t M, int64_t N, int64_t K, const float *A, const uint16_t *Bh, float *C) {
    return report(host_gemm(TML_FMT_F16, M, N, K, A, Bh, 1.0f, nullptr, 0, nullptr, C, 1.0f, 0.0f));
}

int tml_hip_gemm(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                 const float *scales, int64_t block, const float *bias, float *C) {
    return report(host_gemm(fmt, M, N, K, A, B, scale, scales, block, bias, C, 1.0f, 0.0f));
}

int tml_hip_gemm_act(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                     const float *scales, int64_t block, const float *bias, int act, float *C) {
    return report(host_gemm(fmt, M, N, K, A, B, scale, scales, block, bias, C, 1.0f, 0.0f, act));
}

int tml_hip_gemm_residual(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                          const float *scales, int64_t block, const float *bias, const float *residual, float *C) {
    if (residual == nullptr && M > 0 && N > 0) return report(Status::Err(TML_ERR_INVALID_ARG, "null residual"));
    return report(host_gemm(fmt, M, N, K, A, B, scale, scales, block, bias, C, 1.0f, 0.0f, TML_ACT_NONE, residual));
}

int tml_hip_quantize(int fmt, int64_t n, const float *w, void *q, float *scales) {
    if (fmt != TML_FMT_Q8_0 && fmt != TML_FMT_Q4_0 && fmt != TML_FMT_Q8_K && fmt != TML_FMT_F16)
        return report(Status::Err(TML_ERR_INVALID_FORMAT, "quantize: format must be Q8_0, Q4_0, Q8_K or F16"));
    if (n < 0) return report(Status::Err(TML_ERR_INVALID_SHAPE, "negative element count"));
    if ((scales == nullptr && fmt != TML_FMT_F16) || (n > 0 && (w == nullptr || q == nullptr)))
        return report(Status::Err(TML_ERR_INVALID_ARG, "null pointer"));
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    const size_t qbytes = weight_bytes(fmt, 1, n);
    const size_t nscales = fmt == TML_FMT_F16 ? 0 : fmt == TML_FMT_Q8_K ? (size_t)(n + 31) / 32 : 1;
    auto run = [&]() -> Status {
        TML_TRY(c->a.ensure((size_t)n * sizeof(float) + 16));
        TML_TRY(c->b.ensure(qbytes + 16));
        TML_TRY(c->scales.ensure(nscales * sizeof(float) + 16));
        if (n > 0) TML_HIP_TRY(hipMemcpyAsync(c->a.p, w, (size_t)n * sizeof(float), hipMemcpyHostToDevice, c->stream));
        TML_TRY(quantize_dev(c, fmt, n, (const float *)c->a.p, c->b.p, (float *)c->scales.p, c->stream));
        if (qbytes > 0) TML_HIP_TRY(hipMemcpyAsync(q, c->b.p, qbytes, hipMemcpyDeviceToHost, c->stream));
        if (nscales > 0 && (fmt != TML_FMT_Q8_K || n > 0))
            TML_HIP_TRY(hipMemcpyAsync(scales, c->scales.p, nscales * sizeof(float), hipMemcpyDeviceToHost,
                                       c->stream));
        TML_HIP_TRY(hipStreamSynchronize(c->stream));
        return Status::Ok();
    };
    return report(run());
}

int tml_hip_weight_register(const void *host, size_t bytes) {
    if (host == nullptr || bytes == 0) return report(Status::Err(TML_ERR_INVALID_ARG, "null or empty weight"));
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    auto run = [&]() -> Status {
        auto it = c->weights.find(host);
        if (it != c->weights.end()) {
            // a refreshed weight invalidates its prepared copy
            TML_HIP_TRY(hipStreamSynchronize(c->stream));
            free_prepared(it->second.prep);
            it->second.prep = nullptr;
            if (it->second.bytes != bytes) {
                TML_HIP_TRY(hipFree(it->second.dev));
                c->weights.erase(it);
                it = c->weights.end();
            }
        }
        if (it == c->weights.end()) {
            Registered r;
            TML_HIP_TRY(hipMalloc(&r.dev, bytes));
            r.bytes = bytes;
            it = c->weights.emplace(host, r).first;
        }
        TML_HIP_TRY(hipMemcpyAsync(it->second.dev, host, bytes, hipMemcpyHostToDevice, c->stream));
        TML_HIP_TRY(hipStreamSynchronize(c->stream));
        return Status::Ok();
    };
    return report(run());
}

int tml_hip_weight_release(const void *host) {
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    auto it = c->weights.find(host);
    if (it == c->weights.end()) return report(Status::Err(TML_ERR_INVALID_ARG, "weight not registered"));
    auto run = [&]() -> Status {
        TML_HIP_TRY(hipStreamSynchronize(c->stream));
        free_prepared(it->second.prep);
        TML_HIP_TRY(hipFree(it->second.dev));
        c->weights.erase(it);
        return Status::Ok();
    };
    return report(run());
}

int tml_hip_gemm_dev(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                     const float *scales, int64_t block, const float *bias, float *C, float alpha, float beta,
                     void *stream) {
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    return report(gemm_dev(c, fmt, M, N, K, A, B, scale, scales, block, bias, C, alpha, beta, (hipStream_t)stream));
}

int tml_hip_gemm_ex_dev(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B, float scale,
                        const float *scales, int64_t block, const float *bias, const float *residual, int act,
                        float *C, float alpha, float beta, void *stream) {
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    return report(gemm_dev(c, fmt, M, N, K, A, B, scale, scales, block, bias, C, alpha, beta, (hipStream_t)stream,
                           act, residual));
}

int tml_hip_gemm_ex_dev_noalloc(int fmt, int64_t M, int64_t N, int64_t K, const float *A, const void *B,
                                float scale, const float *scales, int64_t block, const float *bias,
                                const float *residual, int act, float *C, float alpha, float beta, void *stream) {
    return report(gemm_dev_noalloc(fmt, M, N, K, A, B, scale, scales, block, bias, C, alpha, beta,
                                   (hipStream_t)stream, act, residual));
}

int tml_hip_prepare_dev(int fmt, int64_t K, int64_t N, const void *B, float scale, void *stream,
                        tml_prepared_t *out) {
    if (out == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null handle pointer"));
    *out = nullptr;
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    Prepared *p = nullptr;
    s = make_prepared(c, fmt, K, N, B, scale, nullptr, (hipStream_t)stream, &p);
    if (s.ok()) *out = (tml_prepared_t)p;
    return report(s);
}

int tml_hip_prepare_ex_dev(int fmt, int64_t K, int64_t N, const void *B, float scale, const float *scales,
                           void *stream, tml_prepared_t *out) {
    if (out == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null handle pointer"));
    *out = nullptr;
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    Prepared *p = nullptr;
    s = make_prepared(c, fmt, K, N, B, scale, scales, (hipStream_t)stream, &p);
    if (s.ok()) *out = (tml_prepared_t)p;
    return report(s);
}

int tml_hip_prepare_rows_dev(int fmt, int64_t K, int64_t N, const void *W, int64_t ldw, float scale, void *stream,
                             tml_prepared_t *out) {
    if (out == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null handle pointer"));
    *out = nullptr;
    if (!preparable_fmt(fmt) || per_channel(fmt))
        return report(Status::Err(TML_ERR_INVALID_FORMAT, "prepare rows: format must be F32, F16, Q8_0 or Q4_0"));
    if (K < 0 || N < 0) return report(Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension"));
    if (K >= ((int64_t)1 << 30) || N >= ((int64_t)1 << 30))
        return report(Status::Err(TML_ERR_INVALID_SHAPE, "prepare: dimension exceeds 2^30"));
    if (fmt == TML_FMT_Q4_0 && K % 2 != 0)
        return report(Status::Err(TML_ERR_INVALID_SHAPE, "Q4_0 rows need an even K (each row starts a byte)"));
    const int64_t row = packed_row_bytes(fmt, K);
    if (ldw < row) return report(Status::Err(TML_ERR_INVALID_ARG, "row stride shorter than a row"));
    if (W == nullptr && K > 0 && N > 0) return report(Status::Err(TML_ERR_INVALID_ARG, "null weight pointer"));
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    Prepared *p = new Prepared();
    p->device = c->device;
    p->fmt = fmt;
    p->K = K;
    p->N = N;
    p->scale = scale;
    if (fmt == TML_FMT_F32 && K > 0 && row % 16 == 0 && ldw % 16 == 0 && ((uintptr_t)W % 16) == 0) {
        // f32 rows in plain K order are already the prepared layout: use the
        // caller's rows in place.
        p->Bt = const_cast<void *>(W);
        p->ldt = ldw;
        p->owns_bt = false;
        *out = (tml_prepared_t)p;
        return report(Status::Ok());
    }
    p->ldt = prepared_row_bytes(fmt, K);
    const size_t bytes = (size_t)(N > 0 ? N : 1) * (size_t)p->ldt;
    auto build = [&]() -> Status {
        TML_HIP_TRY(hipMalloc(&p->Bt, bytes));
        if (N == 0) return Status::Ok();
        return launch_prepare_rows(fmt, K, N, W, ldw, p->Bt, p->ldt, (hipStream_t)stream);
    };
    s = build();
    if (!s.ok()) {
        free_prepared(p);
        return report(s);
    }
    *out = (tml_prepared_t)p;
    return report(Status::Ok());
}

int tml_hip_gemm_prepared(tml_prepared_t w, int64_t M, const float *A, const float *bias, float *C, float alpha,
                          float beta, void *stream) {
    if (w == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null prepared weight"));
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    const Prepared *p = (const Prepared *)w;
    if (p->device != c->device) return report(Status::Err(TML_ERR_INVALID_ARG, "prepared weight of another device"));
    return report(gemm_prepared(c, p, M, A, bias, C, alpha, beta, (hipStream_t)stream));
}

int tml_hip_gemm_prepared_ex(tml_prepared_t w, int64_t M, const float *A, const float *bias, const float *residual,
                             int act, float *C, float alpha, float beta, void *stream) {
    if (w == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null prepared weight"));
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    const Prepared *p = (const Prepared *)w;
    if (p->device != c->device) return report(Status::Err(TML_ERR_INVALID_ARG, "prepared weight of another device"));
    return report(gemm_prepared(c, p, M, A, bias, C, alpha, beta, (hipStream_t)stream, act, residual));
}

int tml_hip_prepared_free(tml_prepared_t w) {
    if (w == nullptr) return report(Status::Ok());
    Prepared *p = (Prepared *)w;
    const hipError_t e = hipDeviceSynchronize();
    free_prepared(p);
    return report(e == hipSuccess ? Status::Ok() : hip_status(e, "hipDeviceSynchronize"));
}

int tml_hip_stream_read_dev(const void *src, int64_t bytes, int chunks_per_lane, float *out, void *stream) {
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    return report(launch_stream_read(src, bytes, chunks_per_lane, out, (hipStream_t)stream));
}

int tml_hip_quantize_dev(int fmt, int64_t n, const float *w, void *q, float *scales, void *stream) {
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    return report(quantize_dev(c, fmt, n, w, q, scales, (hipStream_t)stream));
}

int tml_hip_quantize_cols_dev(int fmt, int64_t K, int64_t N, const float *w, void *q, float *scales, void *stream) {
    if (!per_channel(fmt))
        return report(Status::Err(TML_ERR_INVALID_FORMAT, "column quantizer: format must be Q8_0_PC or Q4_0_PC"));
    if (K < 0 || N < 0) return report(Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension"));
    if ((N > 0 && scales == nullptr) || (K * N > 0 && (w == nullptr || q == nullptr)))
        return report(Status::Err(TML_ERR_INVALID_ARG, "null pointer"));
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    auto run = [&]() -> Status {
        TML_TRY(c->qtmp.ensure((size_t)(N > 0 ? N : 1) * sizeof(float)));
        return launch_quantize_cols(data_fmt(fmt), K, N, w, q, scales, (float *)c->qtmp.p, (hipStream_t)stream);
    };
    return report(run());
}

int tml_hip_quantize_cols(int fmt, int64_t K, int64_t N, const float *w, void *q, float *scales) {
    if (!per_channel(fmt))
        return report(Status::Err(TML_ERR_INVALID_FORMAT, "column quantizer: format must be Q8_0_PC or Q4_0_PC"));
    if (K < 0 || N < 0) return report(Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension"));
    if ((N > 0 && scales == nullptr) || (K * N > 0 && (w == nullptr || q == nullptr)))
        return report(Status::Err(TML_ERR_INVALID_ARG, "null pointer"));
    if (N == 0) return report(Status::Ok());
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    const size_t n = (size_t)K * (size_t)N;
    const size_t qbytes = weight_bytes(fmt, K, N);
    auto run = [&]() -> Status {
        TML_TRY(c->a.ensure(n * sizeof(float) + 16));
        TML_TRY(c->b.ensure(qbytes + 16));
        TML_TRY(c->scales.ensure((size_t)N * sizeof(float)));
        TML_TRY(c->qtmp.ensure((size_t)N * sizeof(float)));
        if (n > 0) TML_HIP_TRY(hipMemcpyAsync(c->a.p, w, n * sizeof(float), hipMemcpyHostToDevice, c->stream));
        TML_TRY(launch_quantize_cols(data_fmt(fmt), K, N, (const float *)c->a.p, c->b.p, (float *)c->scales.p,
                                     (float *)c->qtmp.p, c->stream));
        if (qbytes > 0) TML_HIP_TRY(hipMemcpyAsync(q, c->b.p, qbytes, hipMemcpyDeviceToHost, c->stream));
        TML_HIP_TRY(hipMemcpyAsync(scales, c->scales.p, (size_t)N * sizeof(float), hipMemcpyDeviceToHost, c->stream));
        TML_HIP_TRY(hipStreamSynchronize(c->stream));
        return Status::Ok();
    };
    return report(run());
}

int tml_hip_transpose_requant_dev(int fmt, int64_t rows, int64_t cols, const void *q, const float *scales,
                                  float scale, void *q_out, float *scales_out, void *stream) {
    if (fmt != TML_FMT_Q8_0 && fmt != TML_FMT_Q4_0 && fmt != TML_FMT_Q8_K)
        return report(Status::Err(TML_ERR_INVALID_FORMAT, "transpose-requantize: format must be Q8_0, Q4_0 or Q8_K"));
    if (rows < 0 || cols < 0) return report(Status::Err(TML_ERR_INVALID_SHAPE, "negative matrix dimension"));
    const int64_t n = rows * cols;
    if (scales_out == nullptr || (n > 0 && (q == nullptr || q_out == nullptr)) ||
        (fmt == TML_FMT_Q8_K && n > 0 && scales == nullptr))
        return report(Status::Err(TML_ERR_INVALID_ARG, "null pointer"));
    DeviceCtx *c = nullptr;
    Status s = current_ctx(&c);
    if (!s.ok()) return report(s);
    auto run = [&]() -> Status {
        const hipStream_t st = (hipStream_t)stream;
        if (n > 0) {
            TML_TRY(c->tr.ensure((size_t)n * sizeof(float)));
            TML_TRY(launch_dequant_transpose(fmt, rows, cols, q, scales, scale, (float *)c->tr.p, st));
        }
        return quantize_dev(c, fmt, n, (const float *)c->tr.p, q_out, scales_out, st);
    };
    return report(run());
}

// ------------------------------------------------------------ .tl files
int tml_tl_open(const char *path, tml_tl_t *out) {
    if (out == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null handle pointer"));
    TlFile *f = nullptr;
    Status s = tl_open_file(path, &f);
    *out = (tml_tl_t)f;
    return report(s);
}

int tml_tl_open_bytes(const void *data, uint64_t size, tml_tl_t *out) {
    if (out == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null handle pointer"));
    TlFile *f = nullptr;
    Status s = tl_open_bytes(data, size, &f);
    *out = (tml_tl_t)f;
    return report(s);
}

int tml_tl_close(tml_tl_t f) {
    delete (TlFile *)f;
    return report(Status::Ok());
}

int tml_tl_format(tml_tl_t f) {
    if (f == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null file"));
    return ((const TlFile *)f)->format;
}

int64_t tml_tl_count(tml_tl_t f) {
    if (f == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null file"));
    return (int64_t)((const TlFile *)f)->index.size();
}

const char *tml_tl_name(tml_tl_t f, int64_t i) {
    if (f == nullptr) return nullptr;
    const TlFile *t = (const TlFile *)f;
    if (i < 0 || (size_t)i >= t->tensors.size()) return nullptr;
    return t->tensors[(size_t)i].name.c_str();
}

int tml_tl_info(tml_tl_t f, const char *name, int64_t *dims, int cap, int *ndim, uint64_t *offset,
                uint64_t *size) {
    if (f == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null file"));
    const TlTensor *t = tl_find((const TlFile *)f, name);
    if (t == nullptr)
        return report(Status::Err(TML_ERR_TENSOR_NOT_FOUND, std::string("no tensor named ") + (name ? name : "")));
    if (ndim) *ndim = (int)t->shape.size();
    for (int i = 0; dims && i < cap && i < (int)t->shape.size(); ++i) dims[i] = t->shape[(size_t)i];
    if (offset) *offset = t->offset;
    if (size) *size = t->size;
    return report(Status::Ok());
}


int tml_tl_read(tml_tl_t f, const char *name, int getter, void *data, float *scales, float *scale) {
    if (f == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null file"));
    auto run = [&]() -> Status {
        TML_TRY(tl_check_getter(getter));
        TlParts p;
        TML_TRY(tl_parts((const TlFile *)f, name, getter, false, &p));
        TML_TRY(tl_need(p, data, scales, scale));
        if (p.data_bytes) std::memcpy(data, p.data, p.data_bytes);
        if (p.nscales) std::memcpy(scales, p.scales, p.nscales * 4);
        if (p.fmt == TML_FMT_Q8_0 || p.fmt == TML_FMT_Q4_0) *scale = p.scale;
        return Status::Ok();
    };
    return report(run());
}

int tml_tl_read_dev(tml_tl_t f, const char *name, int getter, void *data, float *scales, float *scale,
                    void *stream) {
    if (f == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null file"));
    auto run = [&]() -> Status {
        TML_TRY(tl_check_getter(getter));
        TlParts p;
        TML_TRY(tl_parts((const TlFile *)f, name, getter, false, &p));
        TML_TRY(tl_need(p, data, scales, scale));
        DeviceCtx *c = nullptr;
        TML_TRY(current_ctx(&c));
        const hipStream_t st = (hipStream_t)stream;
        if (p.data_bytes)
            TML_HIP_TRY(hipMemcpyAsync(data, p.data, p.data_bytes, hipMemcpyHostToDevice, st));
        if (p.nscales) TML_HIP_TRY(hipMemcpyAsync(scales, p.scales, p.nscales * 4, hipMemcpyHostToDevice, st));
        if (p.fmt == TML_FMT_Q8_0 || p.fmt == TML_FMT_Q4_0) *scale = p.scale;
        return Status::Ok();
    };
    return report(run());
}

int tml_tl_read_dequantized_dev(tml_tl_t f, const char *name, float *out, void *stream) {
    if (f == nullptr) return report(Status::Err(TML_ERR_INVALID_ARG, "null file"));
    auto run = [&]() -> Status {
        TlParts p;
        TML_TRY(tl_parts((const TlFile *)f, name, 0, true, &p));
        if (p.numel > 0 && out == nullptr) return Status::Err(TML_ERR_INVALID_ARG, "null destination");
        if (p.numel == 0) return Status::Ok();
        DeviceCtx *c = nullptr;
        TML_TRY(current_ctx(&c));
        const hipStream_t st = (hipStream_t)stream;
        if (p.fmt == TML_FMT_F32) {
            TML_HIP_TRY(hipMemcpyAsync(out, p.data, p.data_bytes, hipMemcpyHostToDevice, st));
            return Status::Ok();
        }
        TML_TRY(c->tl_raw.ensure(p.data_bytes + 16));
        TML_HIP_TRY(hipMemcpyAsync(c->tl_raw.p, p.data, p.data_bytes, hipMemcpyHostToDevice, st));
        if (p.nscales) {
            TML_TRY(c->tl_scales.ensure(p.nscales * 4));
            TML_HIP_TRY(hipMemcpyAsync(c->tl_scales.p, p.scales, p.nscales * 4, hipMemcpyHostToDevice, st));
        }
        return launch_dequant(p.fmt, p.numel, c->tl_raw.p, (const float *)c->tl_scales.p, p.scale, out, st);
    };
    return report(run());
}

}  // extern "C"
