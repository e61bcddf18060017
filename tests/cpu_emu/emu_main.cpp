// Driver of the bounds-checked CPU build (tests/cpu_emu/build.py): reads one
// case per line from stdin and runs it through the library's C ABI with
// operands allocated (through the emulated hipMalloc) at exactly the sizes
// the header documents.  ASan / UBSan abort the process on the first bad
// access; the case line is printed (and flushed) before it runs, so the
// report names it.
//
// Case line:  <op> <fmt> <M> <N> <K> <flags> [NAME=VALUE ...]
//   op     gemm     tml_hip_gemm_ex_dev
//          prep     tml_hip_prepare_ex_dev + tml_hip_gemm_prepared_ex
//          rows     tml_hip_prepare_rows_dev (W = B^T, N rows of K) + gemm_prepared_ex
//          host     tml_hip_gemm_act (host-pointer path, staging and copies)
//          quant    tml_hip_quantize_dev over K*N elements (cols: tml_hip_quantize_cols_dev)
//          treq     tml_hip_transpose_requant_dev of a [K, N] tensor
//          noalloc  tml_hip_gemm_ex_dev_noalloc
//          tlfile   the .tl file named by the flags field: open it, list it, and
//                   read every tensor with every getter to host memory, to the
//                   device and dequantized (errors are expected for most)
//   flags  any of: b bias, r residual, e GELU (erf), t GELU (tanh), B beta != 0; "-" for none;
//          S allocates B 16 bytes short of its size (a planted mistake: the
//          harness must report it)
//   NAME=VALUE  environment for this case only (the library's tuning overrides)
// Output: "ok <line>" or "err <code> <message> <line>" per case; exit 0.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <sstream>
#include <string>
#include <vector>

#include "hip/hip_runtime.h"
#include "tomoul_hip.h"

namespace {

size_t weight_bytes(int fmt, int64_t K, int64_t N) {
    const size_t e = (size_t)K * (size_t)N;
    switch (fmt) {
        case TML_FMT_F32: return 4 * e;
        case TML_FMT_F16: return 2 * e;
        case TML_FMT_Q4_0:
        case TML_FMT_Q4_0_PC: return (e + 1) / 2;
        default: return e;
    }
}

// A device buffer of exactly n bytes (at least one allocation byte, as
// hipMalloc(0) still returns a pointer) filled with small finite floats or
// bytes.
void *dev(size_t n, bool floats) {
    void *p = nullptr;
    hipMalloc(&p, n);
    if (floats) {
        float *f = (float *)p;
        for (size_t i = 0; i < n / 4; ++i) f[i] = 0.25f * (float)((i * 7) % 9) - 1.0f;
    } else {
        unsigned char *b = (unsigned char *)p;
        for (size_t i = 0; i < n; ++i) b[i] = (unsigned char)(i * 37 + 11);
    }
    return p;
}

int act_of(const std::string &f) {
    if (f.find('e') != std::string::npos) return TML_ACT_GELU_ERF;
    if (f.find('t') != std::string::npos) return TML_ACT_GELU_TANH;
    return TML_ACT_NONE;
}

int run_case(const std::string &op, int fmt, int64_t M, int64_t N, int64_t K, const std::string &flags) {
    const bool has_bias = flags.find('b') != std::string::npos;
    const bool has_res = flags.find('r') != std::string::npos;
    const float beta = flags.find('B') != std::string::npos ? 0.5f : 0.0f;
    const int act = act_of(flags);
    const bool pc = fmt == TML_FMT_Q8_0_PC || fmt == TML_FMT_Q4_0_PC;
    const size_t nscales = fmt == TML_FMT_Q8_K ? ((size_t)K * N + 31) / 32 : pc ? (size_t)N : 0;
    std::vector<void *> bufs;
    auto mk = [&](size_t n, bool floats) {
        void *p = dev(n, floats);
        bufs.push_back(p);
        return p;
    };
    int rc = 0;
    if (op == "tlfile") {
        tml_tl_t f = nullptr;
        rc = tml_tl_open(flags.c_str(), &f);
        if (rc != 0) return rc;
        const int64_t n = tml_tl_count(f);
        (void)tml_tl_format(f);
        for (int64_t i = 0;; ++i) {
            const char *name = tml_tl_name(f, i);
            if (name == nullptr) break;
            int64_t dims[8];
            int ndim = 0;
            uint64_t off = 0, size = 0;
            if (tml_tl_info(f, name, dims, 8, &ndim, &off, &size) != 0) continue;
            // destinations sized from what the getters can copy: a payload
            // inside the file (anything else is CorruptedFile)
            FILE *fp = std::fopen(flags.c_str(), "rb");
            std::fseek(fp, 0, SEEK_END);
            const uint64_t fsize = (uint64_t)std::ftell(fp);
            std::fclose(fp);
            const size_t cap = (size_t)(size < fsize ? size : fsize) + 64;
            for (int getter = 0; getter <= 4; ++getter) {
                void *data = mk(cap, false);
                float *scales = (float *)mk(cap, false);
                float scale = 0.0f;
                std::vector<unsigned char> host(cap);
                std::vector<float> hscales(cap / 4 + 1);
                (void)tml_tl_read(f, name, getter, host.data(), hscales.data(), &scale);
                (void)tml_tl_read_dev(f, name, getter, data, scales, &scale, nullptr);
            }
            float *out = (float *)mk(8 * cap + 64, true);
            (void)tml_tl_read_dequantized_dev(f, name, out, nullptr);
        }
        (void)n;
        tml_tl_close(f);
        for (void *p : bufs) hipFree(p);
        return 0;
    }
    if (op == "quant") {
        const int64_t n = K * N;
        float *w = (float *)mk((size_t)n * 4, true);
        void *q = mk(weight_bytes(fmt, K, N), false);
        float *s = (float *)mk((fmt == TML_FMT_Q8_K ? ((size_t)n + 31) / 32 : pc ? (size_t)N : 1) * 4, true);
        rc = pc ? tml_hip_quantize_cols_dev(fmt, K, N, w, q, s, nullptr) : tml_hip_quantize_dev(fmt, n, w, q, s, nullptr);
    } else if (op == "treq") {
        void *q = mk(weight_bytes(fmt, K, N), false);
        float *s = (float *)mk((fmt == TML_FMT_Q8_K ? ((size_t)K * N + 31) / 32 : 1) * 4, true);
        void *qo = mk(weight_bytes(fmt, K, N), false);
        float *so = (float *)mk((fmt == TML_FMT_Q8_K ? ((size_t)K * N + 31) / 32 : 1) * 4, true);
        rc = tml_hip_transpose_requant_dev(fmt, K, N, q, s, 0.01f, qo, so, nullptr);
    } else {
        float *A = (float *)mk((size_t)M * K * 4, true);
        const size_t bb = weight_bytes(fmt, K, N);
        const bool short_b = flags.find('S') != std::string::npos;
        void *B = mk(short_b && bb > 16 ? bb - 16 : bb, fmt == TML_FMT_F32);
        float *S = nscales ? (float *)mk(nscales * 4, true) : nullptr;
        float *bias = has_bias ? (float *)mk((size_t)N * 4, true) : nullptr;
        float *res = has_res ? (float *)mk((size_t)M * N * 4, true) : nullptr;
        float *C = (float *)mk((size_t)M * N * 4, true);
        if (op == "gemm") {
            rc = tml_hip_gemm_ex_dev(fmt, M, N, K, A, B, 0.01f, S, 32, bias, res, act, C, 1.0f, beta, nullptr);
        } else if (op == "noalloc") {
            rc = tml_hip_gemm_ex_dev_noalloc(fmt, M, N, K, A, B, 0.01f, S, 32, bias, res, act, C, 1.0f, beta, nullptr);
        } else if (op == "prep" || op == "rows") {
            tml_prepared_t h = nullptr;
            if (op == "prep") {
                rc = tml_hip_prepare_ex_dev(fmt, K, N, B, 0.01f, S, nullptr, &h);
            } else {
                const int64_t row = fmt == TML_FMT_F32 ? 4 * K : fmt == TML_FMT_F16 ? 2 * K
                                  : fmt == TML_FMT_Q4_0 ? (K + 1) / 2 : K;
                void *W = mk((size_t)N * row, fmt == TML_FMT_F32);
                rc = tml_hip_prepare_rows_dev(fmt, K, N, W, row, 0.01f, nullptr, &h);
            }
            if (rc == 0) {
                rc = tml_hip_gemm_prepared_ex(h, M, A, bias, res, act, C, 1.0f, beta, nullptr);
                tml_hip_prepared_free(h);
            }
        } else if (op == "host") {
            std::vector<float> hA((size_t)M * K, 0.5f), hC((size_t)M * N, 0.0f), hbias((size_t)N, 0.1f),
                hS(nscales ? nscales : 1, 0.01f);
            std::vector<unsigned char> hB(weight_bytes(fmt, K, N), 3);
            rc = tml_hip_gemm_act(fmt, M, N, K, hA.data(), hB.data(), 0.01f, nscales ? hS.data() : nullptr, 32,
                                  has_bias ? hbias.data() : nullptr, act, hC.data());
        } else {
            std::fprintf(stderr, "unknown op %s\n", op.c_str());
            std::exit(2);
        }
    }
    for (void *p : bufs) hipFree(p);
    return rc;
}

}  // namespace

int main() {
    std::string line;
    char buf[4096];
    long n = 0;
    while (std::fgets(buf, sizeof buf, stdin)) {
        line = buf;
        while (!line.empty() && (line.back() == '\n' || line.back() == '\r')) line.pop_back();
        if (line.empty() || line[0] == '#') continue;
        std::istringstream is(line);
        std::string op, flags;
        int fmt = 0;
        long long M = 0, N = 0, K = 0;
        is >> op >> fmt >> M >> N >> K >> flags;
        std::vector<std::string> env;
        for (std::string kv; is >> kv;) env.push_back(kv);
        for (auto &kv : env) {
            const size_t eq = kv.find('=');
            setenv(kv.substr(0, eq).c_str(), kv.substr(eq + 1).c_str(), 1);
        }
        std::fprintf(stdout, "run %s\n", line.c_str());
        std::fflush(stdout);
        const long long launches0 = tml_emu_launches;
        const int rc = run_case(op, fmt, M, N, K, flags);
        for (auto &kv : env) unsetenv(kv.substr(0, kv.find('=')).c_str());
        if (rc == 0)
            std::fprintf(stdout, "ok %lld %s\n", tml_emu_launches - launches0, line.c_str());
        else
            std::fprintf(stdout, "err %d [%s] %s\n", rc, tml_hip_last_error(), line.c_str());
        std::fflush(stdout);
        ++n;
    }
    tml_hip_shutdown();
    std::fprintf(stdout, "done %ld\n", n);
    return 0;
}
