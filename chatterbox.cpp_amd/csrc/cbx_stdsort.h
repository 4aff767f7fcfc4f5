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

// The sequence being sorted.  SortSeq: element i is (s[i], id[i]) with the
// score itself as key (float: comp is a > b) or, where memory is short, the
// score's rank among the distinct scores in descending order (uint16_t: comp
// is a < b), which orders and ties exactly as the scores do.  PackedSeq: one
// word per element, (rank << 16) | id.  The steps below read keys with
// key(i) / key_of(element) and move whole elements.
template <typename Id, typename Key = float>
struct SortSeq {
    Key* s;
    Id* id;
    struct El {
        Key s;
        Id id;
    };
    CBX_SORT_HD El get(int i) const { return {s[i], id[i]}; }
    CBX_SORT_HD void put(int i, El e) const {
        s[i] = e.s;
        id[i] = e.id;
    }
    CBX_SORT_HD Key key(int i) const { return s[i]; }
    CBX_SORT_HD static Key key_of(const El& e) { return e.s; }
    CBX_SORT_HD void swap(int i, int j) const {
        const El t = get(i);
        put(i, get(j));
        put(j, t);
    }
};

struct PackedSeq {
    uint32_t* w;
    using El = uint32_t;
    CBX_SORT_HD El get(int i) const { return w[i]; }
    CBX_SORT_HD void put(int i, El e) const { w[i] = e; }
    CBX_SORT_HD uint16_t key(int i) const { return (uint16_t)(w[i] >> 16); }
    CBX_SORT_HD static uint16_t key_of(El e) { return (uint16_t)(e >> 16); }
    CBX_SORT_HD void swap(int i, int j) const {
        const El t = w[i];
        w[i] = w[j];
        w[j] = t;
    }
};

// comp(a, b) of the reference: a.s > b.s.
CBX_SORT_HD bool sort_comp(float a, float b) { return a > b; }
CBX_SORT_HD bool sort_comp(uint16_t rank_a, uint16_t rank_b) { return rank_a < rank_b; }

template <class Seq>
CBX_SORT_HD void stdsort_push_heap(const Seq& q, int first, int hole, int top,
                                   typename Seq::El v) {
    int parent = (hole - 1) / 2;
    while (hole > top && sort_comp(q.key(first + parent), Seq::key_of(v))) {
        q.put(first + hole, q.get(first + parent));
        hole = parent;
        parent = (hole - 1) / 2;
    }
    q.put(first + hole, v);
}

template <class Seq>
CBX_SORT_HD void stdsort_adjust_heap(const Seq& q, int first, int hole, int len,
                                     typename Seq::El v) {
    const int top = hole;
    int second = hole;
    while (second < (len - 1) / 2) {
        second = 2 * (second + 1);
        if (sort_comp(q.key(first + second), q.key(first + second - 1))) second--;
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
template <class Seq>
CBX_SORT_HD void stdsort_heap_sort(const Seq& q, int first, int last) {
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
        const typename Seq::El v = q.get(last);
        q.put(last, q.get(first));
        stdsort_adjust_heap(q, first, 0, last - first, v);
    }
}

template <class Seq>
CBX_SORT_HD void stdsort_median_to_first(const Seq& q, int r, int a, int b, int c) {
    const auto sa = q.key(a), sb = q.key(b), sc = q.key(c);
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
template <class Seq>
CBX_SORT_HD int stdsort_partition_pivot(const Seq& q, int first, int last) {
    const int mid = first + (last - first) / 2;
    stdsort_median_to_first(q, first, first + 1, mid, last - 1);
    const auto pv = q.key(first);  // the pivot stays at first throughout
    int lo = first + 1, hi = last;
    while (true) {
        while (sort_comp(q.key(lo), pv)) ++lo;
        --hi;
        while (sort_comp(pv, q.key(hi))) --hi;
        if (!(lo < hi)) return lo;
        q.swap(lo, hi);
        ++lo;
    }
}

template <class Seq>
CBX_SORT_HD void stdsort_linear_insert(const Seq& q, int last) {
    const typename Seq::El v = q.get(last);
    int next = last - 1;
    while (sort_comp(Seq::key_of(v), q.key(next))) {
        q.put(last, q.get(next));
        last = next;
        --next;
    }
    q.put(last, v);
}

template <class Seq>
CBX_SORT_HD void stdsort_insertion_sort(const Seq& q, int first, int last) {
    if (first == last) return;
    for (int i = first + 1; i != last; ++i) {
        if (sort_comp(q.key(i), q.key(first))) {
            const typename Seq::El v = q.get(i);
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
template <class Seq>
CBX_SORT_HD int stdsort_replay(const Seq& q, int n) {
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

// ---------------------------------------------------------------------------
// The same sort, reduced to what top-p needs and restated with prefix counts
// so that a wavefront can run it in parallel.
//
// Elements are packed words (rank << 16) | id, rank = the score's rank among
// the distinct scores (descending), so comp(a, b) is rank(a) < rank(b).
//
// 1. Only the order of the elements tied at the cutoff, rank kT, matters:
//    __final_insertion_sort is a stable insertion sort, and after the
//    introsort loop every element of a range it left (<= 16 elements, or
//    heap-sorted) is no less than every element of the ranges after it, so the
//    tied elements end in the order the introsort loop left them.  Ranges
//    holding no element of rank kT are therefore not sorted at all.
// 2. __unguarded_partition around pivot v (at first, moved there by
//    __move_median_to_first) stops its left scan at the elements with
//    !(comp(x, v)) and its right scan at those with !(comp(v, x)); nothing
//    between the two scans has moved yet, so the k-th left stop L_k and the
//    k-th right stop R_k (counted from the right) are swapped exactly while
//    L_k < R_k.  With lb(p) = left stops before p and ra(p) = right stops
//    after p: a left stop p is swapped iff ra(p) > lb(p), with partner rank
//    lb(p); a right stop q iff lb(q) > ra(q), with partner rank ra(q).  The
//    returned cut is the first unswapped left stop or the leftmost swapped
//    right stop, whichever comes first (or last: the range's end).
// Pinned against the serial restatement above and against std::sort itself
// (tests/native/stdsort_replay.cpp).

CBX_SORT_HD uint32_t pk_rank(uint32_t w) { return w >> 16; }

// __unguarded_partition_pivot of [f, l) (l - f > 16) by prefix counts; tmp
// holds l - f words.  Returns the cut.
CBX_SORT_HD int stdsort_partition_counts(uint32_t* w, uint32_t* tmp, int f, int l) {
    const int m = l - f, mid = f + m / 2;
    stdsort_median_to_first(PackedSeq{w}, f, f + 1, mid, l - 1);
    const uint32_t pv = pk_rank(w[f]);
    const int half = (m + 1) / 2;
    uint32_t* tl = tmp;
    uint32_t* tr = tmp + half;
    int n_r = 0;
    for (int p = f + 1; p < l; ++p) n_r += !(pv < pk_rank(w[p])) ? 1 : 0;
    int lb = 0, rb = 0, cut = l;
    for (int p = f + 1; p < l; ++p) {
        const uint32_t k = pk_rank(w[p]);
        const bool is_l = !(k < pv), is_r = !(pv < k);
        const int ra = n_r - rb - (is_r ? 1 : 0);
        if (is_l) {
            if (ra > lb) tl[lb] = w[p];
            else if (p < cut) cut = p;
        }
        if (is_r && lb > ra) {
            tr[ra] = w[p];
            if (p < cut) cut = p;
        }
        lb += is_l ? 1 : 0;
        rb += is_r ? 1 : 0;
    }
    lb = 0;
    rb = 0;
    for (int p = f + 1; p < l; ++p) {
        const uint32_t k = pk_rank(w[p]);
        const bool is_l = !(k < pv), is_r = !(pv < k);
        const int ra = n_r - rb - (is_r ? 1 : 0);
        const int lbp = lb;
        lb += is_l ? 1 : 0;
        rb += is_r ? 1 : 0;
        if (is_l && ra > lbp) w[p] = tr[lbp];
        else if (is_r && lbp > ra) w[p] = tl[ra];
    }
    return cut;
}

// The ids of the elements of rank kT in the order std::sort leaves them
// (written to ids[0 ..]); returns their count.  w[0, n) is the sequence in
// the reference's input order (id order); it is permuted in place; tmp
// holds n words.  Serial form of what a wavefront does in the sampler.
CBX_SORT_HD int stdsort_tied_order(uint32_t* w, uint32_t* tmp, int n, uint32_t kT, uint16_t* ids) {
    if (n <= 0 || n > kStdSortMaxN) return 0;
    int lg = 0;
    while ((n >> (lg + 1)) != 0) ++lg;
    uint32_t st_range[32];
    uint8_t st_depth[32];
    st_range[0] = (uint32_t)n << 16;
    st_depth[0] = (uint8_t)(2 * lg);
    int top = 1;
    while (top > 0) {
        --top;
        const int f = (int)(st_range[top] & 0xffffu);
        int l = (int)(st_range[top] >> 16);
        int depth = st_depth[top];
        while (l - f > kStdSortThreshold) {
            bool has = false;
            for (int p = f; p < l; ++p) has = has || pk_rank(w[p]) == kT;
            if (!has) break;
            if (depth == 0) {  // __partial_sort: rare (adversarial inputs)
                stdsort_heap_sort(PackedSeq{w}, f, l);
                break;
            }
            --depth;
            const int cut = stdsort_partition_counts(w, tmp, f, l);
            st_range[top] = (uint32_t)cut | ((uint32_t)l << 16);
            st_depth[top] = (uint8_t)depth;
            ++top;
            l = cut;
        }
    }
    int m = 0;
    for (int p = 0; p < n; ++p)
        if (pk_rank(w[p]) == kT) ids[m++] = (uint16_t)(w[p] & 0xffffu);
    return m;
}

}  // namespace cbx
