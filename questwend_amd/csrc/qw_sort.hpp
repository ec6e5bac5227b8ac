// qw_sort.hpp -- an exact replay of the reference's argsort for tie cases.
//
// ggml's ARGSORT (ggml/src/ggml-cpu/ops.cpp:8332-8382) orders indices with
// std::sort and the comparator data[a] > data[b].  std::sort is not stable, so
// when equal probabilities reach into the top-k the selected ids depend on the
// exact steps of the C++ library's introsort.  The reference CPU path is built
// against GCC's libstdc++ (the toolchain in this image: introsort with a depth
// limit of 2*floor(log2 n), median-of-three pivot moved to the front, an
// unguarded Hoare partition, 16-element threshold, heapsort fallback, then a
// final insertion sort).  The routine below performs those same steps, in code
// of its own, so the permutation it produces is the one std::sort produces.
// It runs on one GPU thread and only when a tie is detected (see router.hip);
// it is also callable on the host so CPU tests can check it against std::sort.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qw {

struct DescByValue {
    const float* v;
    __host__ __device__ bool operator()(int32_t a, int32_t b) const { return v[a] > v[b]; }
};

template <typename Cmp>
__host__ __device__ inline void sift_up_(int32_t* a, int hole, int top, int32_t value, const Cmp& less) {
    int parent = (hole - 1) / 2;
    while (hole > top && less(a[parent], value)) {
        a[hole] = a[parent];
        hole = parent;
        parent = (hole - 1) / 2;
    }
    a[hole] = value;
}

template <typename Cmp>
__host__ __device__ inline void sift_down_(int32_t* a, int hole, int len, int32_t value, const Cmp& less) {
    const int top = hole;
    int child = hole;
    while (child < (len - 1) / 2) {
        child = 2 * (child + 1);
        if (less(a[child], a[child - 1])) child--;
        a[hole] = a[child];
        hole = child;
    }
    if ((len & 1) == 0 && child == (len - 2) / 2) {
        child = 2 * (child + 1);
        a[hole] = a[child - 1];
        hole = child - 1;
    }
    sift_up_(a, hole, top, value, less);
}

template <typename Cmp>
__host__ __device__ inline void heap_pop_into_(int32_t* first, int len, int32_t* result, const Cmp& less) {
    const int32_t value = *result;
    *result = first[0];
    sift_down_(first, 0, len, value, less);
}

template <typename Cmp>
__host__ __device__ inline void heap_sort_range_(int32_t* first, int n, const Cmp& less) {
    // build heap
    if (n >= 2) {
        for (int parent = (n - 2) / 2;; --parent) {
            sift_down_(first, parent, n, first[parent], less);
            if (parent == 0) break;
        }
    }
    // heap-select over [n, n) is empty; then sort the heap
    for (int last = n; last > 1;) {
        --last;
        heap_pop_into_(first, last, first + last, less);
    }
}

template <typename Cmp>
__host__ __device__ inline void median_to_front_(int32_t* r, int32_t* a, int32_t* b, int32_t* c, const Cmp& less) {
    int32_t* pick;
    if (less(*a, *b)) {
        if (less(*b, *c)) pick = b;
        else if (less(*a, *c)) pick = c;
        else pick = a;
    } else if (less(*a, *c)) {
        pick = a;
    } else if (less(*b, *c)) {
        pick = c;
    } else {
        pick = b;
    }
    const int32_t t = *r;
    *r = *pick;
    *pick = t;
}

template <typename Cmp>
__host__ __device__ inline int32_t* hoare_unguarded_(int32_t* lo, int32_t* hi, const int32_t* pivot, const Cmp& less) {
    for (;;) {
        while (less(*lo, *pivot)) ++lo;
        --hi;
        while (less(*pivot, *hi)) --hi;
        if (!(lo < hi)) return lo;
        const int32_t t = *lo;
        *lo = *hi;
        *hi = t;
        ++lo;
    }
}

template <typename Cmp>
__host__ __device__ inline void insert_guarded_(int32_t* first, int32_t* last, const Cmp& less) {
    if (first == last) return;
    for (int32_t* i = first + 1; i != last; ++i) {
        const int32_t val = *i;
        if (less(val, *first)) {
            for (int32_t* p = i; p != first; --p) *p = *(p - 1);
            *first = val;
        } else {
            int32_t* hole = i;
            int32_t* prev = i - 1;
            while (less(val, *prev)) {
                *hole = *prev;
                hole = prev;
                --prev;
            }
            *hole = val;
        }
    }
}

template <typename Cmp>
__host__ __device__ inline void insert_unguarded_(int32_t* first, int32_t* last, const Cmp& less) {
    for (int32_t* i = first; i != last; ++i) {
        const int32_t val = *i;
        int32_t* hole = i;
        int32_t* prev = i - 1;
        while (less(val, *prev)) {
            *hole = *prev;
            hole = prev;
            --prev;
        }
        *hole = val;
    }
}

// Pending right-hand ranges: at most one per level, and there are at most
// 2*floor(log2 n) + 1 levels before the heapsort fallback takes over.
constexpr int SORT_STACK = 66;
struct SortRange { int first, last, depth; };

// Sorts idx[0..n) so that the order equals libstdc++ std::sort(idx, idx+n, less).
// `stack` holds SORT_STACK entries (LDS on the device, so it never spills).
template <typename Cmp>
__host__ __device__ inline void libstdcxx_sort(int32_t* idx, int n, const Cmp& less, SortRange* stack) {
    if (n <= 1) return;
    constexpr int kThreshold = 16;
    int lg = 0;
    while ((2 << lg) <= n) ++lg;  // floor(log2 n)
    int sp = 0;
    stack[sp++] = {0, n, 2 * lg};
    while (sp > 0) {
        const SortRange r = stack[--sp];
        int32_t* first = idx + r.first;
        int32_t* last = idx + r.last;
        int depth = r.depth;
        while (last - first > kThreshold) {
            if (depth == 0) {
                heap_sort_range_(first, (int) (last - first), less);
                break;
            }
            --depth;
            int32_t* mid = first + (last - first) / 2;
            median_to_front_(first, first + 1, mid, last - 1, less);
            int32_t* cut = hoare_unguarded_(first + 1, last, first, less);
            // the right part is sorted independently of the left one, so the order
            // in which the two are processed does not change the result
            if (sp < SORT_STACK) stack[sp++] = {(int) (cut - idx), (int) (last - idx), depth};
            last = cut;
        }
    }
    if (n > kThreshold) {
        insert_guarded_(idx, idx + kThreshold, less);
        insert_unguarded_(idx + kThreshold, idx + n, less);
    } else {
        insert_guarded_(idx, idx + n, less);
    }
}

__host__ __device__ inline void libstdcxx_sort_desc(int32_t* idx, int n, const float* values, SortRange* stack) {
    libstdcxx_sort(idx, n, DescByValue{values}, stack);
}

}  // namespace qw
