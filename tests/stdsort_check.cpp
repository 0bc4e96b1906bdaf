// TEST INFRASTRUCTURE ONLY: the device's std::sort restatement (snapdragon-engine_amd/csrc/
// oxe_stdsort.h, compiled here for the host) against this host's libstdc++ std::sort with the
// reference's comparator x[a] > x[b] (oxe_ops.cpp:157-164), on seeded tie-heavy rows.
// Usage: stdsort_check <rows> <seed>; prints "<mismatching rows> <first bad row>".
#include "oxe_stdsort.h"
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <random>
#include <vector>

int main(int argc, char **argv) {
    if (argc < 3) return 2;
    const int rows = atoi(argv[1]);
    std::mt19937_64 rng(strtoull(argv[2], nullptr, 10));
    int bad = 0, first = -1;
    const int sizes[] = {2, 3, 15, 16, 17, 31, 64, 100, 256, 257, 1000, 2048};
    for (int r = 0; r < rows; r++) {
        const int n = sizes[r % (sizeof(sizes) / sizeof(sizes[0]))];
        // values from a small set (many ties), a few distinct values, or sorted runs with ties
        const int kind = (r / 12) % 5;
        const int levels = kind == 0 ? 1 : kind == 1 ? 2 : kind == 2 ? 7 : kind == 3 ? 40 : n;
        std::vector<float> v(n);
        for (int i = 0; i < n; i++) v[i] = (float)(rng() % (uint64_t)levels) * 0.125f;
        if (r % 7 == 3) std::sort(v.begin(), v.end());              // ascending runs
        if (r % 7 == 4) std::sort(v.begin(), v.end(), std::greater<float>());
        std::vector<int32_t> a(n), b(n);
        std::vector<uint8_t> c(n);
        for (int i = 0; i < n; i++) a[i] = b[i] = i;
        std::sort(a.begin(), a.end(), [&](int32_t x, int32_t y) { return v[x] > v[y]; });
        oxe_sort::Range st[OXE_SORT_STACK];
        oxe_sort::sort_desc(b.data(), v.data(), n, st);
        bool ok = a == b;
        if (n <= 256) {   // the device sorts 8-bit indices of 256 experts
            for (int i = 0; i < n; i++) c[i] = (uint8_t)i;
            oxe_sort::sort_desc(c.data(), v.data(), n, st);
            for (int i = 0; i < n; i++) ok &= a[i] == c[i];
        }
        if (!ok) {
            bad++;
            if (first < 0) first = r;
        }
    }
    // McIlroy's adversary ("A killer adversary for quicksort", 1999): values fixed lazily during a
    // std::sort so that every pivot is bad; the finished assignment drives the introsort past its
    // depth limit into the heap-sort branch
    for (int n : {64, 256, 1000, 2048}) {
        std::vector<int> val(n, n), idx(n);
        int nsolid = 0, cand = 0;
        for (int i = 0; i < n; i++) idx[i] = i;
        std::sort(idx.begin(), idx.end(), [&](int x, int y) {
            if (val[x] == n && val[y] == n) {
                if (x == cand) val[x] = nsolid++;
                else val[y] = nsolid++;
            }
            if (val[x] == n) cand = x;
            else if (val[y] == n) cand = y;
            return val[x] < val[y];
        });
        std::vector<float> v(n);
        for (int i = 0; i < n; i++) v[i] = -(float)val[i];     // descending comparator == the adversary's ascending one
        std::vector<int32_t> a(n), b(n);
        for (int i = 0; i < n; i++) a[i] = b[i] = i;
        std::sort(a.begin(), a.end(), [&](int32_t x, int32_t y) { return v[x] > v[y]; });
        oxe_sort::Range st[OXE_SORT_STACK];
        oxe_sort::sort_desc(b.data(), v.data(), n, st);
        if (a != b) {
            bad++;
            if (first < 0) first = 1000000 + n;
        }
    }
    printf("%d %d\n", bad, first);
    return 0;
}
