// Compares the restated expf (chatterbox.cpp_amd/csrc/cbx_expf.h, compiled
// here as host code: the branching form, the branch-free form, and for x <= 0
// the non-positive form) with the host libm expf over every binary32 bit
// pattern
// in [lo_bits, hi_bits).  Prints "<mismatches> <count>" and the first few
// mismatching inputs.  usage: expf_exhaustive lo_bits hi_bits n_threads
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

#include "../../chatterbox.cpp_amd/csrc/cbx_expf.h"

int main(int argc, char** argv) {
    if (argc != 4) return 2;
    const uint64_t lo = strtoull(argv[1], nullptr, 0), hi = strtoull(argv[2], nullptr, 0);
    const int nt = atoi(argv[3]);
    std::vector<uint64_t> bad(nt, 0);
    std::vector<uint32_t> first(nt, 0);
    std::vector<std::thread> th;
    for (int t = 0; t < nt; ++t) {
        th.emplace_back([&, t] {
            const uint64_t a = lo + (hi - lo) * t / nt, b = lo + (hi - lo) * (t + 1) / nt;
            for (uint64_t u = a; u < b; ++u) {
                const uint32_t bits = (uint32_t)u;
                float x;
                std::memcpy(&x, &bits, 4);
                const float r = std::exp(x), m = cbx::expf_libm(x);
                const float b = cbx::expf_libm_branchless(x);
                const bool nonpos = x <= 0.0f;  // -inf included, NaN not
                const float p = nonpos ? cbx::expf_nonpos(x) : r;
                uint32_t rb, mb, bb, pb;
                std::memcpy(&rb, &r, 4);
                std::memcpy(&mb, &m, 4);
                std::memcpy(&bb, &b, 4);
                std::memcpy(&pb, &p, 4);
                if (rb != mb || rb != bb || rb != pb) {
                    if (!bad[t]) first[t] = bits;
                    ++bad[t];
                }
            }
        });
    }
    uint64_t total = 0;
    for (int t = 0; t < nt; ++t) {
        th[t].join();
        total += bad[t];
    }
    printf("%llu %llu\n", (unsigned long long)total, (unsigned long long)(hi - lo));
    for (int t = 0; t < nt; ++t)
        if (bad[t]) printf("first mismatch 0x%08x\n", first[t]);
    return 0;
}
