// TEST INFRASTRUCTURE ONLY: compares the device restatements of expf and log1pf
// (snapdragon-engine_amd/csrc/oxe_libm.h, compiled here for the host) with this host's C library,
// bit for bit, over every float input from `lo` to `hi` (hex, inclusive-exclusive).
// Usage: libm_check <fn: 0 expf, 1 log1pf> <lo> <hi> <threads>; prints "<mismatches> <first>".
#include "oxe_libm.h"
#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <thread>
#include <vector>

int main(int argc, char **argv) {
    if (argc < 5) return 2;
    const int fn = atoi(argv[1]);
    const uint64_t lo = strtoull(argv[2], nullptr, 16), hi = strtoull(argv[3], nullptr, 16);
    const int nt = atoi(argv[4]);
    std::atomic<uint64_t> bad{0}, first{~0ull};
    std::vector<std::thread> th;
    for (int t = 0; t < nt; t++)
        th.emplace_back([&, t] {
            const uint64_t a = lo + (hi - lo) * t / nt, b = lo + (hi - lo) * (t + 1) / nt;
            uint64_t nb = 0;
            for (uint64_t i = a; i < b; i++) {
                const uint32_t u = (uint32_t)i;
                float x;
                memcpy(&x, &u, 4);
                const float want = fn == 0 ? expf(x) : log1pf(x);
                const float got = fn == 0 ? oxe_libm::expf_c(x) : oxe_libm::log1pf_c(x);
                uint32_t uw, ug;
                memcpy(&uw, &want, 4);
                memcpy(&ug, &got, 4);
                if (uw != ug && !(std::isnan(want) && std::isnan(got))) {
                    nb++;
                    uint64_t f = first.load();
                    while (i < f && !first.compare_exchange_weak(f, i)) {
                    }
                }
            }
            bad += nb;
        });
    for (auto &x : th) x.join();
    printf("%llu %llx\n", (unsigned long long)bad.load(), (unsigned long long)first.load());
    return 0;
}
