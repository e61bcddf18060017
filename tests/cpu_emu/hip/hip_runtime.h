// CPU emulation of the HIP runtime and of the gfx950 builtins that the
// sources of libtomoul_hip use -- test infrastructure for a bounds-checked
// CPU build of the whole library (tests/cpu_emu/build.py).
//
// The library's own .hip files are compiled for the host with this header in
// place of <hip/hip_runtime.h>, under AddressSanitizer and UBSan.  A kernel
// launch runs the kernel body once per (block, thread) of the grid, one
// thread after another, with the real index arithmetic of the source.  Every
// global-memory access is a host access to an allocation of exactly the
// size the runtime asked hipMalloc for, so ASan reports any access outside
// it; LDS arrays are static arrays and a launch's dynamic LDS is a heap
// block of the size the launch asked for, so an access outside either is
// reported as well.  Buffer loads implement the hardware's range check (a dword at or
// past the resource's byte count reads zero, no access is made) and
// report -- as an error -- a resource whose byte count exceeds the
// allocation it points into.  LDS-DMA copies write lane `l`'s bytes at
// lds + l * size, as the hardware does.
//
// What is NOT emulated: cross-lane data (DPP, swizzles and shuffles return
// the lane's own value), the contents other threads leave in LDS, and the
// matrix-core arithmetic.  Results are therefore meaningless; only the
// addresses are checked.  Control flow depends on the arguments only
// (plus the split-K arrival counters, which behave as on the device when
// the blocks run one after another).
#pragma once

#include <algorithm>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <type_traits>
#include <vector>

#define __global__
#define __device__
#define __host__
#define __shared__ static
#define __forceinline__ inline __attribute__((always_inline))
#define __launch_bounds__(...)
#define __align__(n) __attribute__((aligned(n)))
#define HIP_SYMBOL(x) (&(x))

#ifndef __HIP_MEMORY_SCOPE_AGENT
#define __HIP_MEMORY_SCOPE_WAVEFRONT 2
#define __HIP_MEMORY_SCOPE_WORKGROUP 3
#define __HIP_MEMORY_SCOPE_AGENT 4
#define __HIP_MEMORY_SCOPE_SYSTEM 5
#endif

struct dim3 {
    unsigned x, y, z;
    constexpr dim3(unsigned x_ = 1, unsigned y_ = 1, unsigned z_ = 1) : x(x_), y(y_), z(z_) {}
};
struct tml_emu_index {
    unsigned x = 0, y = 0, z = 0;
};
inline tml_emu_index threadIdx, blockIdx;
inline dim3 blockDim, gridDim;

// ------------------------------------------------------------ runtime API
enum hipError_t {
    hipSuccess = 0,
    hipErrorInvalidValue = 1,
    hipErrorOutOfMemory = 2,
    hipErrorMemoryAllocation = 2,
    hipErrorNoDevice = 100,
    hipErrorInvalidDevice = 101,
    hipErrorInvalidSymbol = 13,
    hipErrorStreamCaptureUnsupported = 900,
};
enum hipMemcpyKind { hipMemcpyHostToHost, hipMemcpyHostToDevice, hipMemcpyDeviceToHost, hipMemcpyDeviceToDevice,
                     hipMemcpyDefault };
enum hipDeviceAttribute_t { hipDeviceAttributeMultiprocessorCount = 1 };
enum hipStreamCaptureStatus { hipStreamCaptureStatusNone = 0, hipStreamCaptureStatusActive = 1 };
struct ihipStream_t {
    int id;
};
typedef ihipStream_t *hipStream_t;
constexpr unsigned hipStreamNonBlocking = 1;
struct hipDeviceProp_t {
    char name[256];
    int multiProcessorCount;
};

// Allocations made through hipMalloc, for the buffer-resource size check.
inline std::map<uintptr_t, size_t> &tml_emu_allocs() {
    static std::map<uintptr_t, size_t> m;
    return m;
}
// Non-zero makes hipStreamIsCapturing report an active capture.
inline int tml_emu_capturing = 0;
inline long long tml_emu_launches = 0;

inline const char *hipGetErrorString(hipError_t e) { return e == hipSuccess ? "no error" : "emulated HIP error"; }
inline hipError_t hipGetLastError() { return hipSuccess; }
inline hipError_t hipPeekAtLastError() { return hipSuccess; }
inline hipError_t hipGetDeviceCount(int *n) {
    *n = 1;
    return hipSuccess;
}
inline hipError_t hipGetDevice(int *d) {
    *d = 0;
    return hipSuccess;
}
inline hipError_t hipSetDevice(int) { return hipSuccess; }
inline hipError_t hipDeviceGetAttribute(int *v, hipDeviceAttribute_t, int) {
    *v = 256;
    return hipSuccess;
}
inline hipError_t hipGetDeviceProperties(hipDeviceProp_t *p, int) {
    std::snprintf(p->name, sizeof p->name, "CPU emulation of gfx950");
    p->multiProcessorCount = 256;
    return hipSuccess;
}
inline hipError_t hipStreamCreateWithFlags(hipStream_t *s, unsigned) {
    static ihipStream_t st{1};
    *s = &st;
    return hipSuccess;
}
inline hipError_t hipStreamDestroy(hipStream_t) { return hipSuccess; }
inline hipError_t hipStreamSynchronize(hipStream_t) { return hipSuccess; }
inline hipError_t hipDeviceSynchronize() { return hipSuccess; }
inline hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus *st) {
    *st = tml_emu_capturing ? hipStreamCaptureStatusActive : hipStreamCaptureStatusNone;
    return hipSuccess;
}
inline hipError_t hipMalloc(void **p, size_t n) {
    void *q = nullptr;
    if (posix_memalign(&q, 256, n ? n : 1) != 0) return hipErrorOutOfMemory;
    *p = q;
    tml_emu_allocs()[(uintptr_t)q] = n;
    return hipSuccess;
}
template <typename T>
inline hipError_t hipMalloc(T **p, size_t n) {
    return hipMalloc((void **)p, n);
}
inline hipError_t hipFree(void *p) {
    if (p) {
        tml_emu_allocs().erase((uintptr_t)p);
        std::free(p);
    }
    return hipSuccess;
}
// Pinned host memory: plain host memory of exactly the asked size.
constexpr unsigned hipHostMallocDefault = 0;
inline hipError_t hipHostMalloc(void **p, size_t n, unsigned) {
    void *q = std::malloc(n ? n : 1);
    if (q == nullptr) return hipErrorOutOfMemory;
    *p = q;
    return hipSuccess;
}
inline hipError_t hipHostFree(void *p) {
    std::free(p);
    return hipSuccess;
}
// Events: work runs when it is issued, so every event has completed.
typedef struct tml_emu_event *hipEvent_t;
constexpr unsigned hipEventDisableTiming = 2;
inline hipError_t hipEventCreateWithFlags(hipEvent_t *e, unsigned) {
    *e = (hipEvent_t)std::malloc(1);
    return *e ? hipSuccess : hipErrorOutOfMemory;
}
inline hipError_t hipEventRecord(hipEvent_t, hipStream_t = nullptr) { return hipSuccess; }
inline hipError_t hipEventSynchronize(hipEvent_t) { return hipSuccess; }
inline hipError_t hipEventDestroy(hipEvent_t e) {
    std::free(e);
    return hipSuccess;
}
inline hipError_t hipMemset(void *p, int v, size_t n) {
    std::memset(p, v, n);
    return hipSuccess;
}
inline hipError_t hipMemsetAsync(void *p, int v, size_t n, hipStream_t = nullptr) { return hipMemset(p, v, n); }
inline hipError_t hipMemcpy(void *d, const void *s, size_t n, hipMemcpyKind) {
    if (n) std::memcpy(d, s, n);
    return hipSuccess;
}
inline hipError_t hipMemcpyAsync(void *d, const void *s, size_t n, hipMemcpyKind k, hipStream_t = nullptr) {
    return hipMemcpy(d, s, n, k);
}
inline hipError_t hipGetSymbolAddress(void **p, const void *sym) {
    *p = const_cast<void *>(sym);
    return hipSuccess;
}

// ------------------------------------------------------------- launches
// Dynamic LDS of the running launch: a heap block of exactly the bytes the
// launch asked for, so an access past it is an ASan report.
inline std::vector<char> *&tml_emu_dyn_buf() {
    static std::vector<char> *b = nullptr;
    return b;
}
inline void *tml_emu_dyn_lds() { return tml_emu_dyn_buf() ? tml_emu_dyn_buf()->data() : nullptr; }
#define TML_DYNAMIC_LDS(T, v) T *const v = (T *)tml_emu_dyn_lds()

template <typename... P>
struct tml_emu_launcher {
    void (*k)(P...);
    dim3 g, b;
    size_t shmem;
    template <typename... A>
    void operator()(A &&...args) const {
        ++tml_emu_launches;
        gridDim = g;
        blockDim = b;
        std::vector<char> dyn(shmem);
        tml_emu_dyn_buf() = shmem ? &dyn : nullptr;
        for (unsigned bz = 0; bz < g.z; ++bz)
            for (unsigned by = 0; by < g.y; ++by)
                for (unsigned bx = 0; bx < g.x; ++bx) {
                    blockIdx.x = bx; blockIdx.y = by; blockIdx.z = bz;
                    for (unsigned tz = 0; tz < b.z; ++tz)
                        for (unsigned ty = 0; ty < b.y; ++ty)
                            for (unsigned tx = 0; tx < b.x; ++tx) {
                                threadIdx.x = tx; threadIdx.y = ty; threadIdx.z = tz;
                                k(args...);
                            }
                }
        tml_emu_dyn_buf() = nullptr;
    }
};
template <typename... P>
tml_emu_launcher<P...> tml_emu_launch(void (*k)(P...), dim3 g, dim3 b, size_t shmem = 0, hipStream_t = nullptr) {
    return {k, g, b, shmem};
}

// ------------------------------------------------------------- device side
inline void __syncthreads() {}
template <typename A, typename B>
inline std::common_type_t<A, B> min(A a, B b) {
    return a < b ? a : b;
}
template <typename A, typename B>
inline std::common_type_t<A, B> max(A a, B b) {
    return a < b ? b : a;
}
inline float __uint_as_float(uint32_t u) { return __builtin_bit_cast(float, u); }
inline uint32_t __float_as_uint(float f) { return __builtin_bit_cast(uint32_t, f); }
inline int __float_as_int(float f) { return __builtin_bit_cast(int, f); }
inline float __int_as_float(int i) { return __builtin_bit_cast(float, i); }
inline unsigned tml_emu_lane() { return threadIdx.x & 63u; }

template <typename T>
inline T __shfl_xor(T v, int, int = 64) {
    return v;
}
template <typename T>
inline void tml_emu_atomic_store(T *p, T v) {
    *p = v;
}
template <typename T>
inline T tml_emu_atomic_load(const T *p) {
    return *p;
}
template <typename T, typename U>
inline T tml_emu_atomic_fetch_add(T *p, U v) {
    const T o = *p;
    *p = o + (T)v;
    return o;
}
#define __hip_atomic_store(p, v, order, scope) tml_emu_atomic_store((p), (v))
#define __hip_atomic_load(p, order, scope) tml_emu_atomic_load((p))
#define __hip_atomic_fetch_add(p, v, order, scope) tml_emu_atomic_fetch_add((p), (v))

typedef float tml_emu_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t tml_emu_u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t tml_emu_u32x2 __attribute__((ext_vector_type(2)));

inline void __builtin_amdgcn_s_waitcnt(int) {}
inline void __builtin_amdgcn_s_barrier() {}
inline void __builtin_amdgcn_sched_barrier(int) {}
inline void __builtin_amdgcn_wave_barrier() {}
inline void __builtin_amdgcn_fence(int, const char *) {}
template <typename T>
inline T __builtin_amdgcn_readfirstlane(T v) {
    return v;
}
inline tml_emu_f32x4 __builtin_amdgcn_mfma_f32_16x16x4f32(float, float, tml_emu_f32x4 c, int, int, int) { return c; }
typedef __bf16 tml_emu_bf16x8 __attribute__((ext_vector_type(8)));
inline tml_emu_f32x4 __builtin_amdgcn_mfma_f32_16x16x32_bf16(tml_emu_bf16x8, tml_emu_bf16x8, tml_emu_f32x4 c, int, int,
                                                            int) {
    return c;
}
inline float __builtin_amdgcn_fmed3f(float a, float b, float c) { return a < b ? b : (a > c ? c : a); }
inline int __builtin_amdgcn_update_dpp(int, int src, int, int, int, bool) { return src; }
inline int __builtin_amdgcn_ds_swizzle(int v, int) { return v; }

// Buffer resources: base, byte count.
struct tml_emu_rsrc {
    const char *base;
    uint32_t num;
};
typedef tml_emu_rsrc __amdgpu_buffer_rsrc_t;

// A resource may only describe bytes of one allocation: a byte count past
// its end would let in-range offsets touch memory the kernel does not own.
inline void tml_emu_check_rsrc(const tml_emu_rsrc &r) {
    if (r.num == 0) return;
    auto &m = tml_emu_allocs();
    auto it = m.upper_bound((uintptr_t)r.base);
    if (it == m.begin()) {
        std::fprintf(stderr, "EMU ERROR: buffer resource base %p is not in any hipMalloc allocation\n", (void *)r.base);
        std::abort();
    }
    --it;
    const uintptr_t end = it->first + it->second;
    if ((uintptr_t)r.base + r.num > end) {
        std::fprintf(stderr, "EMU ERROR: buffer resource [%p, +%u) runs %llu bytes past its allocation\n",
                     (void *)r.base, r.num, (unsigned long long)((uintptr_t)r.base + r.num - end));
        std::abort();
    }
}
inline tml_emu_rsrc __builtin_amdgcn_make_buffer_rsrc(void *p, short, int num, int) {
    tml_emu_rsrc r{(const char *)p, (uint32_t)num};
    tml_emu_check_rsrc(r);
    return r;
}
// One dword at byte offset off: zero when off + 4 is past the byte count.
inline uint32_t tml_emu_buf_dword(const tml_emu_rsrc &r, uint64_t off) {
    if (off + 4 > r.num) return 0u;
    uint32_t v;
    std::memcpy(&v, r.base + off, 4);
    return v;
}
inline tml_emu_u32x4 __builtin_amdgcn_raw_buffer_load_b128(tml_emu_rsrc r, unsigned off, int soff, int) {
    const uint64_t o = (uint64_t)off + (uint64_t)soff;
    return tml_emu_u32x4{tml_emu_buf_dword(r, o), tml_emu_buf_dword(r, o + 4), tml_emu_buf_dword(r, o + 8),
                         tml_emu_buf_dword(r, o + 12)};
}
inline tml_emu_u32x2 __builtin_amdgcn_raw_buffer_load_b64(tml_emu_rsrc r, unsigned off, int soff, int) {
    const uint64_t o = (uint64_t)off + (uint64_t)soff;
    return tml_emu_u32x2{tml_emu_buf_dword(r, o), tml_emu_buf_dword(r, o + 4)};
}
inline uint32_t __builtin_amdgcn_raw_buffer_load_b32(tml_emu_rsrc r, unsigned off, int soff, int) {
    return tml_emu_buf_dword(r, (uint64_t)off + (uint64_t)soff);
}
// 2- and 1-byte loads: zero when the bytes run past the byte count.
inline unsigned short __builtin_amdgcn_raw_buffer_load_b16(tml_emu_rsrc r, unsigned off, int soff, int) {
    const uint64_t o = (uint64_t)off + (uint64_t)soff;
    if (o + 2 > r.num) return 0;
    unsigned short v;
    std::memcpy(&v, r.base + o, 2);
    return v;
}
inline unsigned char __builtin_amdgcn_raw_buffer_load_b8(tml_emu_rsrc r, unsigned off, int soff, int) {
    const uint64_t o = (uint64_t)off + (uint64_t)soff;
    if (o + 1 > r.num) return 0;
    return (unsigned char)r.base[o];
}
// LDS DMA: lane l's `size` bytes land at lds + l * size.
inline void __builtin_amdgcn_raw_ptr_buffer_load_lds(tml_emu_rsrc r, __attribute__((address_space(3))) void *lds,
                                                     int size, unsigned off, int soff, int imm, int) {
    char *dst = (char *)lds + (size_t)tml_emu_lane() * (size_t)size;
    const uint64_t o = (uint64_t)off + (uint64_t)soff + (uint64_t)imm;
    for (int i = 0; i < size; i += 4) {
        const uint32_t v = tml_emu_buf_dword(r, o + (uint64_t)i);
        std::memcpy(dst + i, &v, 4);
    }
}
inline void __builtin_amdgcn_global_load_lds(__attribute__((address_space(1))) void *src,
                                             __attribute__((address_space(3))) void *lds, int size, int imm, int) {
    char *dst = (char *)lds + (size_t)tml_emu_lane() * (size_t)size;
    std::memcpy(dst, (const char *)src + imm, (size_t)size);
}
