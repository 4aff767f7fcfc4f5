// The one-lane std::sort restatement (chatterbox.cpp_amd/csrc/cbx_stdsort.h,
// compiled here as host code) against libstdc++'s own std::sort on the
// reference's element type and comparator (src/main.cpp:752-755): struct
// {int idx; float s;}, pairs built in id order, comp a.s > b.s.  The final
// orders must be identical element for element, ids included, which pins the
// order std::sort gives equal scores.
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
