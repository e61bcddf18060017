// Exercises tml::HostCopier (tomoul_amd/csrc/host_copier.hpp), the parallel
// host memcpy behind the host-pointer entry points, for tests/test_host_copier.py
// under ThreadSanitizer: sizes on both sides of the single-thread cutoff and
// of the part size, odd lengths and offsets, back-to-back jobs, and jobs
// requested from several threads at once.  Every copy is checked byte for
// byte.  Exit status 0 on success.
#include <cstdio>
#include <cstdlib>
#include <thread>
#include <vector>

#include "host_copier.hpp"

namespace {

unsigned long long rng_state = 0x9E3779B97F4A7C15ull;
unsigned next_rand() {
    rng_state ^= rng_state << 13;
    rng_state ^= rng_state >> 7;
    rng_state ^= rng_state << 17;
    return (unsigned)rng_state;
}

bool one_copy(size_t n, size_t src_off, size_t dst_off, unsigned seed) {
    std::vector<unsigned char> src(n + src_off), dst(n + dst_off + 64, 0xAB);
    for (size_t i = 0; i < src.size(); ++i) src[i] = (unsigned char)(i * 131u + seed);
    tml::HostCopier::get().copy(dst.data() + dst_off, src.data() + src_off, n);
    for (size_t i = 0; i < n; ++i)
        if (dst[dst_off + i] != src[src_off + i]) {
            std::fprintf(stderr, "mismatch at %zu of %zu\n", i, n);
            return false;
        }
    for (size_t i = 0; i < dst_off; ++i)
        if (dst[i] != 0xAB) return false;
    for (size_t i = dst_off + n; i < dst.size(); ++i)
        if (dst[i] != 0xAB) {
            std::fprintf(stderr, "write past the end at %zu (n %zu)\n", i, n);
            return false;
        }
    return true;
}

}  // namespace

int main() {
    const size_t sizes[] = {0, 1, 4095, (size_t)512 << 10, ((size_t)512 << 10) - 1, ((size_t)1 << 20) + 7,
                            (size_t)4 << 20, ((size_t)9 << 20) + 333};
    for (size_t n : sizes)
        for (size_t off = 0; off < 3; ++off)
            if (!one_copy(n, off, 2 * off, (unsigned)n)) return 1;
    for (int i = 0; i < 40; ++i) {
        const size_t n = (next_rand() % (6u << 20)) + 1;
        if (!one_copy(n, next_rand() % 64, next_rand() % 64, (unsigned)i)) return 1;
    }
    // several requesting threads: jobs are serialised, each still exact
    std::vector<std::thread> ts;
    std::vector<int> ok(4, 1);
    for (int t = 0; t < 4; ++t)
        ts.emplace_back([t, &ok] {
            for (int i = 0; i < 10; ++i)
                if (!one_copy(((size_t)(t + 1) << 20) + (size_t)i * 4099, (size_t)t, (size_t)i, (unsigned)(t * 100 + i)))
                    ok[t] = 0;
        });
    for (auto &th : ts) th.join();
    for (int v : ok)
        if (!v) return 1;
    std::puts("host copier ok");
    return 0;
}
