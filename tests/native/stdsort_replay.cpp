// The one-lane std::sort restatement (chatterbox.cpp_amd/csrc/cbx_stdsort.h,
// compiled here as host code) against libstdc++'s own std::sort on the
// reference's element type and comparator (src/main.cpp:752-755): struct
// {int idx; float s;}, pairs built in id order, comp a.s > b.s.  The final
// orders must be identical element for element, ids included, which pins the
// order std::sort gives equal scores.  The same holds with the scores
// replaced by their 16-bit ranks among the distinct scores (the form used
// where LDS is short), and for the prefix-count form that follows only the
// ranges holding one rank (stdsort_tied_order, the form a wavefront runs):
// the ids of each rank come out in std::sort's order.
//
// Inputs: sizes 0..600 and a few large ones, values drawn from small sets
// (many ties), from wide sets (few ties), all equal, sorted both ways, and
// inputs built by McIlroy's adversary against std::sort itself (median-of-3
// killers that drive the introsort to its heap-sort fallback).  Prints
// "<cases> <mismatches> <heap-sorted ranges seen>"; exit status 1 on a
// mismatch.
#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "../../chatterbox.cpp_amd/csrc/cbx_stdsort.h"

namespace {

struct IS {
    int idx;
    float s;
};

int g_heaped = 0;

bool same_as_std(const std::vector<float>& scores) {
    std::vector<IS> ref;
    for (int i = 0; i < (int)scores.size(); ++i) ref.push_back({i, scores[i]});
    std::sort(ref.begin(), ref.end(), [](const IS& a, const IS& b) { return a.s > b.s; });
    std::vector<float> s(scores);
    std::vector<uint16_t> id(scores.size());
    for (size_t i = 0; i < id.size(); ++i) id[i] = (uint16_t)i;
    cbx::SortSeq<uint16_t> q{s.data(), id.data()};
    g_heaped += cbx::stdsort_replay(q, (int)s.size());
    for (size_t i = 0; i < ref.size(); ++i)
        if (ref[i].idx != (int)id[i] || ref[i].s != s[i]) return false;
    // the same sort on 16-bit ranks of the distinct scores (descending)
    std::vector<float> dist(scores);
    std::sort(dist.begin(), dist.end(), [](float a, float b) { return a > b; });
    std::vector<uint16_t> rk(scores.size()), id2(scores.size());
    for (size_t i = 0; i < scores.size(); ++i) {
        const auto it = std::lower_bound(dist.begin(), dist.end(), scores[i],
                                         [](float a, float b) { return a > b; });
        rk[i] = (uint16_t)(it - dist.begin());
        id2[i] = (uint16_t)i;
    }
    const std::vector<uint16_t> rank_of_id(rk);
    cbx::SortSeq<uint16_t, uint16_t> q2{rk.data(), id2.data()};
    (void)cbx::stdsort_replay(q2, (int)rk.size());
    for (size_t i = 0; i < ref.size(); ++i)
        if (ref[i].idx != (int)id2[i]) return false;
    // the tied-order form: for every rank present, the ids of that rank in
    // std::sort's final order (prefix-count partitions of the ranges that hold
    // the rank, no final insertion sort)
    const int n = (int)scores.size();
    std::vector<uint32_t> base(n), w(n), tmp(n + 1);
    for (int i = 0; i < n; ++i) base[i] = ((uint32_t)rank_of_id[i] << 16) | (uint32_t)i;
    std::vector<uint16_t> got(n);
    for (int start = 0; start < n;) {
        const uint32_t kT = (uint32_t)(std::lower_bound(dist.begin(), dist.end(), ref[start].s,
                                                        [](float a, float b) { return a > b; }) -
                                       dist.begin());
        int end = start;
        while (end < n && ref[end].s == ref[start].s) ++end;
        w = base;
        const int m = cbx::stdsort_tied_order(w.data(), tmp.data(), n, kT, got.data());
        if (m != end - start) return false;
        for (int i = 0; i < m; ++i)
            if ((int)got[i] != ref[start + i].idx) return false;
        // only a few ranks of large inputs (time)
        start = (n > 700 && end - start < 3) ? end + n / 7 : end;
        while (start < n && start > 0 && ref[start].s == ref[start - 1].s) ++start;
    }
    // one prefix-count partition of the whole sequence against the serial one
    if (n > cbx::kStdSortThreshold) {
        std::vector<uint32_t> a(base), b(base);
        const int c1 = cbx::stdsort_partition_pivot(cbx::PackedSeq{a.data()}, 0, n);
        const int c2 = cbx::stdsort_partition_counts(b.data(), tmp.data(), 0, n);
        if (c1 != c2 || a != b) return false;
    }
    return true;
}

// McIlroy, "A killer adversary for quicksort" (1999): values are frozen
// lazily while std::sort runs, so that its pivots are as bad as possible;
// the frozen values are then a fixed input.  Sorting ascending by val here is
// the reference's descending sort of s = -val.
std::vector<float> adversary(int n) {
    const int gas = n;
    std::vector<int> val(n, gas);
    int nsolid = 0, candidate = 0;
    std::vector<IS> v;
    for (int i = 0; i < n; ++i) v.push_back({i, 0.0f});
    std::sort(v.begin(), v.end(), [&](const IS& a, const IS& b) {
        const int x = a.idx, y = b.idx;
        if (val[x] == gas && val[y] == gas) {
            if (x == candidate) val[x] = nsolid++;
            else val[y] = nsolid++;
        }
        if (val[x] == gas) candidate = x;
        else if (val[y] == gas) candidate = y;
        return val[x] < val[y];
    });
    std::vector<float> s(n);
    for (int i = 0; i < n; ++i) s[i] = -(float)val[i];
    return s;
}

}  // namespace

int main() {
    std::mt19937 rng(20261202);
    int cases = 0, bad = 0;
    auto run = [&](const std::vector<float>& s) {
        ++cases;
        if (!same_as_std(s)) {
            ++bad;
            if (bad <= 5) std::printf("mismatch at n=%zu\n", s.size());
        }
    };
    std::vector<int> sizes;
    for (int n = 0; n <= 600; ++n) sizes.push_back(n);
    for (int n : {1000, 1023, 1024, 1025, 2048, 4097, 8194, 16384, 32768}) sizes.push_back(n);
    for (int n : sizes) {
        for (int distinct : {1, 2, 3, 7, 50, 1 << 20}) {
            std::uniform_int_distribution<int> d(0, distinct - 1);
            std::vector<float> s(n);
            for (float& x : s) x = 0.25f * (float)d(rng) - 3.0f;
            run(s);
        }
        std::vector<float> up(n), down(n);
        for (int i = 0; i < n; ++i) {
            up[i] = (float)(i / 3);
            down[i] = (float)((n - i) / 3);
        }
        run(up);
        run(down);
        if (n >= 2 && (n < 200 || n % 97 == 0 || n >= 1000)) run(adversary(n));
    }
    std::printf("%d %d %d\n", cases, bad, g_heaped);
    return bad ? 1 : 0;
}
