// The order libstdc++'s std::sort leaves equal elements in, restated for one thread (host or device).
//
// The reference's top-k (crates/kernels-sys/csrc/oxe_ops.cpp:157-164) falls back to
//   std::sort(idx, idx + n, [x](int a, int b) { return x[a] > x[b]; })
// whenever the k + 1 largest values are not strictly distinct. std::sort is not stable, so the
// order of tied experts (and with it the chosen top 8) is whatever libstdc++'s algorithm produces.
// This is that algorithm (libstdc++ bits/stl_algo.h and bits/stl_heap.h, unchanged in substance
// since GCC 4.8): introsort with depth limit 2 floor(log2 n); the median of (first + 1, mid,
// last - 1) moved to the front as the pivot; the unguarded Hoare partition of [first + 1, last);
// recursion on the right part, iteration on the left; heap sort of a range once the depth limit is
// spent; then insertion sort of the first 16 elements and unguarded insertion of the rest.
// Processing order of disjoint ranges does not change the result; the recursion is an explicit
// stack whose depth is bounded by the depth limit (stack[] holds OXE_SORT_STACK entries).
//
// With a NaN among the values the comparator is not a strict weak ordering and libstdc++'s
// unguarded loops may leave the range; here every loop stays inside [0, n) instead.
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define OXE_SFN __host__ __device__ static inline
#else
#define OXE_SFN static inline
#endif

#define OXE_SORT_STACK 24   // > 2 floor(log2 n) + 1 for n <= 2048

namespace oxe_sort {

struct Range {
    int16_t first, last, depth;
};

// comp(a, b): value of index a > value of index b
template <class I>
OXE_SFN bool comp(const float *v, I a, I b) { return v[a] > v[b]; }

template <class I>
OXE_SFN void swap_at(I *x, int a, int b) {
    const I t = x[a];
    x[a] = x[b];
    x[b] = t;
}

template <class I>
OXE_SFN void move_median_to_first(I *x, const float *v, int result, int a, int b, int c) {
    if (comp(v, x[a], x[b])) {
        if (comp(v, x[b], x[c])) swap_at(x, result, b);
        else if (comp(v, x[a], x[c])) swap_at(x, result, c);
        else swap_at(x, result, a);
    } else if (comp(v, x[a], x[c])) {
        swap_at(x, result, a);
    } else if (comp(v, x[b], x[c])) {
        swap_at(x, result, c);
    } else {
        swap_at(x, result, b);
    }
}

// Hoare partition of [first, last) around the element at pivot (outside the range)
template <class I>
OXE_SFN int unguarded_partition(I *x, const float *v, int first, int last, int pivot) {
    const int lo = first, hi = last;
    while (true) {
        while (first < hi - 1 && comp(v, x[first], x[pivot])) ++first;
        --last;
        while (last > lo && comp(v, x[pivot], x[last])) --last;
        if (!(first < last)) return first;
        swap_at(x, first, last);
        ++first;
    }
}

template <class I>
OXE_SFN void push_heap(I *x, const float *v, int first, int hole, int top, I value) {
    int parent = (hole - 1) / 2;
    while (hole > top && comp(v, x[first + parent], value)) {
        x[first + hole] = x[first + parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    x[first + hole] = value;
}

template <class I>
OXE_SFN void adjust_heap(I *x, const float *v, int first, int hole, int len, I value) {
    const int top = hole;
    int second = hole;
    while (second < (len - 1) / 2) {
        second = 2 * (second + 1);
        if (comp(v, x[first + second], x[first + second - 1])) second--;
        x[first + hole] = x[first + second];
        hole = second;
    }
    if ((len & 1) == 0 && second == (len - 2) / 2) {
        second = 2 * (second + 1);
        x[first + hole] = x[first + second - 1];
        hole = second - 1;
    }
    push_heap(x, v, first, hole, top, value);
}

// std::__partial_sort(first, last, last): make_heap, then sort_heap
template <class I>
OXE_SFN void heap_sort(I *x, const float *v, int first, int last) {
    const int len = last - first;
    if (len >= 2) {
        for (int parent = (len - 2) / 2;; parent--) {
            adjust_heap(x, v, first, parent, len, x[first + parent]);
            if (parent == 0) break;
        }
    }
    while (last - first > 1) {
        --last;
        const I value = x[last];
        x[last] = x[first];
        adjust_heap(x, v, first, 0, last - first, value);
    }
}

// element i moved left past every element it compares greater than (stops at lo)
template <class I>
OXE_SFN void linear_insert(I *x, const float *v, int i, int lo) {
    const I val = x[i];
    int j = i;
    while (j > lo && comp(v, val, x[j - 1])) {
        x[j] = x[j - 1];
        j--;
    }
    x[j] = val;
}

template <class I>
OXE_SFN void insertion_sort(I *x, const float *v, int first, int last) {
    for (int i = first + 1; i < last; i++) {
        if (comp(v, x[i], x[first])) {
            const I val = x[i];
            for (int j = i; j > first; j--) x[j] = x[j - 1];
            x[first] = val;
        } else {
            linear_insert(x, v, i, first);
        }
    }
}

// std::sort(x, x + n, comp) with comp(a, b) = v[a] > v[b]; stack: OXE_SORT_STACK entries of scratch
template <class I>
OXE_SFN void sort_desc(I *x, const float *v, int n, Range *stack) {
    if (n < 2) return;
    int lg = 0;
    while ((2 << lg) <= n) lg++;
    int sp = 0;
    stack[sp++] = Range{0, (int16_t)n, (int16_t)(2 * lg)};
    while (sp > 0) {
        const Range r = stack[sp - 1];
        int first = r.first, last = r.last, depth = r.depth;
        if (last - first <= 16) {
            sp--;
            continue;
        }
        if (depth == 0) {
            heap_sort(x, v, first, last);
            sp--;
            continue;
        }
        depth--;
        const int mid = first + (last - first) / 2;
        move_median_to_first(x, v, first, first + 1, mid, last - 1);
        const int cut = unguarded_partition(x, v, first + 1, last, first);
        // the loop goes on with [first, cut); the recursive call takes [cut, last) first
        stack[sp - 1] = Range{(int16_t)first, (int16_t)cut, (int16_t)depth};
        if (sp < OXE_SORT_STACK) stack[sp++] = Range{(int16_t)cut, (int16_t)last, (int16_t)depth};
    }
    // __final_insertion_sort
    if (n > 16) {
        insertion_sort(x, v, 0, 16);
        for (int i = 16; i < n; i++) linear_insert(x, v, i, 0);
    } else {
        insertion_sort(x, v, 0, n);
    }
}

}  // namespace oxe_sort
