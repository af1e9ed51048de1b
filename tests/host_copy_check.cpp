// Driver for tests/test_host_copy.py: exercises dhx::parallel_copy and
// dhx::Copier (dinov3-loom_amd/csrc/host_copy.cpp) on the host, built with
// ThreadSanitizer or AddressSanitizer + UndefinedBehaviorSanitizer. Prints
// "ok <checks>" and exits 0 when every check holds; exits 1 on the first
// mismatch (the sanitizers report races and memory errors themselves).
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>

#include "host_copy.hpp"

namespace {

int g_checks = 0;

void expect(bool ok, const char* what, uint64_t a = 0, uint64_t b = 0) {
    ++g_checks;
    if (!ok) {
        std::printf("FAILED: %s (%llu, %llu)\n", what, (unsigned long long)a, (unsigned long long)b);
        std::fflush(stdout);
        std::exit(1);
    }
}

std::vector<unsigned char> random_bytes(std::mt19937_64& rng, uint64_t n) {
    std::vector<unsigned char> v(n);
    for (uint64_t i = 0; i < n; i += 8) {
        const uint64_t r = rng();
        std::memcpy(v.data() + i, &r, std::min<uint64_t>(8, n - i));
    }
    return v;
}

// parallel_copy at sizes around its 4 MiB split unit and its 16-thread cap.
void check_parallel_copy(std::mt19937_64& rng) {
    const uint64_t mib = 1ull << 20;
    const uint64_t sizes[] = {0, 1, 7, 4 * mib - 1, 4 * mib, 4 * mib + 1, 9 * mib + 3, 64 * mib + 13, 80 * mib + 5};
    for (uint64_t n : sizes) {
        const std::vector<unsigned char> src = random_bytes(rng, n);
        std::vector<unsigned char> dst(n + 64, 0xa5);  // guard bytes past the end stay untouched
        dhx::parallel_copy(dst.data(), src.data(), n);
        expect(n == 0 || std::memcmp(dst.data(), src.data(), n) == 0, "parallel_copy data", n);
        bool guard = true;
        for (int i = 0; i < 64; ++i) guard &= dst[n + i] == 0xa5;
        expect(guard, "parallel_copy wrote past n", n);
    }
}

// Copies of random sizes between distinct buffers; the main thread reads
// each destination right after waiting for its ticket (the pattern of the
// forward pipeline), and chained copies (a -> b, then b -> c) prove that
// copies run in submission order.
void check_copier(std::mt19937_64& rng, bool threaded) {
    const int jobs = 96;
    std::vector<std::vector<unsigned char>> src(jobs), mid(jobs), dst(jobs);
    for (int i = 0; i < jobs; ++i) {
        const uint64_t n = (i % 7 == 0) ? (rng() % (24ull << 20)) : (rng() % (3ull << 20));
        src[i] = random_bytes(rng, n);
        mid[i].assign(n, 0);
        dst[i].assign(n, 0);
    }
    dhx::Copier copier(threaded);
    std::vector<uint64_t> first(jobs), second(jobs);
    for (int i = 0; i < jobs; ++i) {
        first[i] = copier.submit(mid[i].data(), src[i].data(), src[i].size());
        second[i] = copier.submit(dst[i].data(), mid[i].data(), mid[i].size());
        expect(first[i] == 2ull * i && second[i] == 2ull * i + 1, "tickets count from 0 in order", first[i], second[i]);
        if (i >= 3) {  // wait a few jobs behind, as the pipeline does
            copier.wait(second[i - 3]);
            expect(dst[i - 3] == src[i - 3], "chained copy after wait", (uint64_t)i - 3);
        }
    }
    copier.wait(second[jobs - 1]);
    for (int i = 0; i < jobs; ++i) expect(dst[i] == src[i], "chained copy", (uint64_t)i);
}

// Destroying a copier with copies still queued runs them all first.
void check_drain_on_destruction(std::mt19937_64& rng) {
    const int jobs = 24;
    std::vector<std::vector<unsigned char>> src(jobs), dst(jobs);
    for (int i = 0; i < jobs; ++i) {
        src[i] = random_bytes(rng, (1ull << 20) + rng() % (8ull << 20));
        dst[i].assign(src[i].size(), 0);
    }
    {
        dhx::Copier copier(true);
        for (int i = 0; i < jobs; ++i) copier.submit(dst[i].data(), src[i].data(), src[i].size());
    }
    for (int i = 0; i < jobs; ++i) expect(dst[i] == src[i], "queued copy ran before destruction", (uint64_t)i);
}

}  // namespace

int main() {
    std::mt19937_64 rng(20261202);
    check_parallel_copy(rng);
    check_copier(rng, true);
    check_copier(rng, false);
    check_drain_on_destruction(rng);
    std::printf("ok %d\n", g_checks);
    return 0;
}
