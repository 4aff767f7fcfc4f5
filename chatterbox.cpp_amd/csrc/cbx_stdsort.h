// cbx_stdsort.h -- the order std::sort gives equal scores, replayed on one lane.
//
// The reference ranks the finite scores for top-p with
//   std::sort(sorted.begin(), sorted.end(),
//             [](const IS& a, const IS& b) { return a.s > b.s; })
// over {id, score} pairs gathered in id order (src/main.cpp:752-755).
// std::sort is not stable, so when equal scores straddle the top-p cutoff
// which of their ids the reference keeps is decided by the exact sequence of
// moves its std::sort makes.  The reference is built with libstdc++ (GCC 11,
// the toolchain its build names); its std::sort is an introsort whose steps
// are restated here for one thread over (score, id) arrays, comparator
// "a.s > b.s":
//
//   bits/stl_algo.h  __sort: __introsort_loop with depth limit 2*floor(log2 n),
//                    then __final_insertion_sort
//                    __introsort_loop: while more than 16 elements, partition
//                    around the median of (first+1, mid, last-1) moved to
//                    first, recurse on the right part, loop on the left; at
//                    depth 0 heap-sort the range (__partial_sort)
//                    __unguarded_partition, __move_median_to_first,
//                    __insertion_sort, __unguarded_linear_insert,
//                    __unguarded_insertion_sort, __final_insertion_sort
//   bits/stl_heap.h  __make_heap, __adjust_heap, __push_heap, __pop_heap,
//                    __sort_heap
//
// The recursion on the right part becomes an explicit stack: the ranges it
// sorts are disjoint and each is sorted by its own steps, so the order in
// which they are taken does not change the result.  Same comparisons, same
// element moves, hence the same final order (pinned against libstdc++'s
// std::sort itself on tied, random and adversarial inputs:
// tests/native/stdsort_replay.cpp).  Rows with NaN scores are outside this
// (the comparator is then not a strict weak order and std::sort's unguarded
// scans are undefined).
#pragma once

#include <stdint.h>

#if defined(__HIPCC__)
#define CBX_SORT_HD __host__ __device__ inline
#else
#define CBX_SORT_HD inline
#endif

namespace cbx {

// The sequence being sorted: element i is (s[i], id[i]).
template <typename Id>
struct SortSeq {
    float* s;
    Id* id;
    struct El {
        float s;
        Id id;
    };
    CBX_SORT_HD El get(int i) const { return {s[i], id[i]}; }
    CBX_SORT_HD void put(int i, El e) const {
        s[i] = e.s;
        id[i] = e.id;
    }
    CBX_SORT_HD void swap(int i, int j) const {
        const El t = get(i);
        put(i, get(j));
        put(j, t);
    }
};

// comp(a, b) of the reference: a.s > b.s.
CBX_SORT_HD bool sort_comp(float a, float b) { return a > b; }

template <typename Id>
CBX_SORT_HD void stdsort_push_heap(const SortSeq<Id>& q, int first, int hole, int top,
                                   typename SortSeq<Id>::El v) {
    int parent = (hole - 1) / 2;
    while (hole > top && sort_comp(q.s[first + parent], v.s)) {
        q.put(first + hole, q.get(first + parent));
        hole = parent;
        parent = (hole - 1) / 2;
    }
    q.put(first + hole, v);
}

template <typename Id>
CBX_SORT_HD void stdsort_adjust_heap(const SortSeq<Id>& q, int first, int hole, int len,
                                     typename SortSeq<Id>::El v) {
    const int top = hole;
    int second = hole;
    while (second < (len - 1) / 2) {
        second = 2 * (second + 1);
        if (sort_comp(q.s[first + second], q.s[first + second - 1])) second--;
        q.put(first + hole, q.get(first + second));
        hole = second;
    }
    if ((len & 1) == 0 && second == (len - 2) / 2) {
        second = 2 * (second + 1);
        q.put(first + hole, q.get(first + second - 1));
        hole = second - 1;
    }
    stdsort_push_heap(q, first, hole, top, v);
}

// __partial_sort(first, last, last): __make_heap, then __sort_heap.
template <typename Id>
CBX_SORT_HD void stdsort_heap_sort(const SortSeq<Id>& q, int first, int last) {
    const int len = last - first;
    if (len >= 2) {
        int parent = (len - 2) / 2;
        while (true) {
            stdsort_adjust_heap(q, first, parent, len, q.get(first + parent));
            if (parent == 0) break;
            parent--;
        }
    }
    while (last - first > 1) {
        --last;
        const typename SortSeq<Id>::El v = q.get(last);
        q.put(last, q.get(first));
        stdsort_adjust_heap(q, first, 0, last - first, v);
    }
}

template <typename Id>
CBX_SORT_HD void stdsort_median_to_first(const SortSeq<Id>& q, int r, int a, int b, int c) {
    const float sa = q.s[a], sb = q.s[b], sc = q.s[c];
    if (sort_comp(sa, sb)) {
        if (sort_comp(sb, sc)) q.swap(r, b);
        else if (sort_comp(sa, sc)) q.swap(r, c);
        else q.swap(r, a);
    } else if (sort_comp(sa, sc)) {
        q.swap(r, a);
    } else if (sort_comp(sb, sc)) {
        q.swap(r, c);
    } else {
        q.swap(r, b);
    }
}

// __unguarded_partition_pivot: the median of three moved to first, then the
// unguarded partition of [first + 1, last) around it; returns the cut.
template <typename Id>
CBX_SORT_HD int stdsort_partition_pivot(const SortSeq<Id>& q, int first, int last) {
    const int mid = first + (last - first) / 2;
    stdsort_median_to_first(q, first, first + 1, mid, last - 1);
    const float pv = q.s[first];  // the pivot stays at first throughout
    int lo = first + 1, hi = last;
    while (true) {
        while (sort_comp(q.s[lo], pv)) ++lo;
        --hi;
        while (sort_comp(pv, q.s[hi])) --hi;
        if (!(lo < hi)) return lo;
        q.swap(lo, hi);
        ++lo;
    }
}

template <typename Id>
CBX_SORT_HD void stdsort_linear_insert(const SortSeq<Id>& q, int last) {
    const typename SortSeq<Id>::El v = q.get(last);
    int next = last - 1;
    while (sort_comp(v.s, q.s[next])) {
        q.put(last, q.get(next));
        last = next;
        --next;
    }
    q.put(last, v);
}

template <typename Id>
CBX_SORT_HD void stdsort_insertion_sort(const SortSeq<Id>& q, int first, int last) {
    if (first == last) return;
    for (int i = first + 1; i != last; ++i) {
        if (sort_comp(q.s[i], q.s[first])) {
            const typename SortSeq<Id>::El v = q.get(i);
            for (int j = i; j > first; --j) q.put(j, q.get(j - 1));
            q.put(first, v);
        } else {
            stdsort_linear_insert(q, i);
        }
    }
}

constexpr int kStdSortThreshold = 16;  // _S_threshold

constexpr int kStdSortMaxN = 65535;   // ranges packed in 16-bit halves

// std::sort of [0, n), n <= kStdSortMaxN.  Returns the number of ranges that
// reached the depth limit and were heap-sorted (0 for almost every input;
// for the tests).
template <typename Id>
CBX_SORT_HD int stdsort_replay(const SortSeq<Id>& q, int n) {
    if (n <= 0 || n > kStdSortMaxN) return 0;
    int lg = 0;
    while ((n >> (lg + 1)) != 0) ++lg;  // floor(log2 n) <= 15
    // Ranges waiting for __introsort_loop, as (first | last << 16, depth).
    // Every range on the stack has a smaller depth than the one below it
    // (a popped range pushes only depths below its own), so it never holds
    // more than 2 * 15 + 1 entries.
    uint32_t st_range[32];
    uint8_t st_depth[32];
    st_range[0] = (uint32_t)n << 16;
    st_depth[0] = (uint8_t)(2 * lg);
    int top = 1;
    int heaped = 0;
    while (top > 0) {
        --top;
        const int first = (int)(st_range[top] & 0xffffu);
        int last = (int)(st_range[top] >> 16);
        int depth = st_depth[top];
        while (last - first > kStdSortThreshold) {
            if (depth == 0) {
                stdsort_heap_sort(q, first, last);
                ++heaped;
                break;
            }
            --depth;
            const int cut = stdsort_partition_pivot(q, first, last);
            st_range[top] = (uint32_t)cut | ((uint32_t)last << 16);
            st_depth[top] = (uint8_t)depth;
            ++top;
            last = cut;
        }
    }
    // __final_insertion_sort
    if (n > kStdSortThreshold) {
        stdsort_insertion_sort(q, 0, kStdSortThreshold);
        for (int i = kStdSortThreshold; i < n; ++i) stdsort_linear_insert(q, i);
    } else {
        stdsort_insertion_sort(q, 0, n);
    }
    return heaped;
}

}  // namespace cbx
