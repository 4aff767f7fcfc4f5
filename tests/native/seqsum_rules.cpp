// Host check of the segment-scan rules in chatterbox.cpp_amd/csrc/cbx_seqsum.h:
// 64 simulated lanes run the same segment procedure as the device scan
// (chunk tables, exclusive scan, the walk of the lane holding the segment's
// end, one ordinary add for the term that leaves the binade) and every case
// is compared with the plain left-to-right binary32 loop.
//   usage: seqsum_rules <cases> <seed>      prints "<bad_sum> <bad_hit> <cases> <segments>"
#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "../../chatterbox.cpp_amd/csrc/cbx_seqsum.h"

using namespace cbx;

static long g_segments = 0;

// Left-to-right sum P + t[i0] + ... (and first index reaching thr > 0).
static float scan_sum(const float* t, int n, float P, int i0, float thr, int* hit) {
    const int L = 64;
    *hit = -1;
    while (i0 < n) {
        ++g_segments;
        const int e = seq_unit_exp(P);
        const int N0 = (int)ldexpf(P, -e);
        const int p0 = N0 & 1;
        int nthr = kSeqSat;
        if (thr > 0.0f) nthr = (int)ceilf(fminf(ldexpf(thr, -e), kSeqClamp));
        const int target = std::min(nthr, 1 << 24);
        const int C = (n - i0 + L - 1) / L;
        std::vector<SeqTab> incl(L);
        for (int l = 0; l < L; ++l) {
            SeqTab T = seq_identity();
            for (int k = 0; k < C; ++k) {
                const int i = i0 + l * C + k;
                if (i < n) T = seq_push(T, seq_step(t[i], e));
            }
            incl[l] = l ? seq_compose(incl[l - 1], T) : T;
        }
        int L0 = -1;
        for (int l = 0; l < L; ++l)
            if (N0 + (p0 ? incl[l].d1 : incl[l].d0) >= target) { L0 = l; break; }
        if (L0 < 0) return ldexpf((float)(N0 + (p0 ? incl[L - 1].d1 : incl[L - 1].d0)), e);
        const SeqTab X = L0 ? incl[L0 - 1] : seq_identity();
        int d = p0 ? X.d1 : X.d0, c = p0 ? (X.q >> 1) & 1 : X.q & 1;
        int kind = 0, idx = 0, nprev = 0;
        for (int k = 0; k < C; ++k) {
            const int i = i0 + L0 * C + k;
            if (i >= n) break;
            const int nb = N0 + d;
            seq_apply(d, c, seq_step(t[i], e));
            if (N0 + d >= (1 << 24)) { kind = 1; idx = i; nprev = nb; break; }
            if (N0 + d >= nthr) { kind = 2; idx = i; break; }
        }
        if (kind == 2) { *hit = idx; return P; }
        if (kind == 0) { std::printf("walk found nothing\n"); std::exit(2); }
        P = ldexpf((float)nprev, e) + t[idx];
        if (thr > 0.0f && P >= thr) { *hit = idx; return P; }
        i0 = idx + 1;
    }
    return P;
}

int main(int argc, char** argv) {
    const int cases = argc > 1 ? atoi(argv[1]) : 20000;
    std::mt19937_64 rng(argc > 2 ? strtoull(argv[2], nullptr, 0) : 1);
    std::normal_distribution<double> nd;
    std::uniform_real_distribution<double> ud(0, 1);
    long bad_sum = 0, bad_hit = 0;
    for (int tc = 0; tc < cases; ++tc) {
        const int n = 1 + (int)(rng() % 2100);
        const int mode = (int)(rng() % 7);
        std::vector<float> s(n);
        const double sig = 0.5 + 6 * ud(rng);
        for (int i = 0; i < n; ++i) {
            switch (mode) {
            case 0: s[i] = (float)(nd(rng) * sig); break;
            case 1: s[i] = (float)(std::floor(nd(rng) * 4) / 4); break;      // many equal terms
            case 2: s[i] = (float)(-(double)(rng() % 64) * 0.6931471805599453); break;
            case 3: s[i] = (float)(nd(rng) * 0.01); break;                     // near-equal
            case 4: s[i] = (float)(-ud(rng) * 100); break;                      // wide range
            case 5: s[i] = (float)(-(double)(rng() % 8)); break;
            default: s[i] = (float)(nd(rng) * 3); break;
            }
        }
        std::sort(s.begin(), s.end(), std::greater<float>());
        std::vector<float> t(n);
        for (int i = 0; i < n; ++i) t[i] = expf(s[i] - s[0]);
        if (mode >= 5 && (tc & 1)) std::shuffle(t.begin(), t.end(), rng);  // unsorted order
        if (mode == 6 && (tc & 2)) for (float& v : t) v = ldexpf(v, -100); // tiny terms
        float ref = t[0];
        for (int i = 1; i < n; ++i) ref += t[i];
        int hit;
        const float got = scan_sum(t.data(), n, t[0], 1, 0.0f, &hit);
        if (std::memcmp(&ref, &got, 4) != 0) {
            if (bad_sum < 5) std::printf("sum mismatch case %d n=%d mode=%d %a %a\n", tc, n, mode, ref, got);
            ++bad_sum;
        }
        // first index with running sum of q_i = t_i / ref >= p
        std::vector<float> q(n);
        for (int i = 0; i < n; ++i) q[i] = t[i] / ref;
        const float p = (tc % 7 == 0) ? 1.0f : (float)(0.05 + 0.95 * ud(rng));
        int href = -1;
        float acc = 0.0f;
        for (int i = 0; i < n; ++i) { acc += q[i]; if (acc >= p) { href = i; break; } }
        int hgot = 0;
        if (!(q[0] >= p)) scan_sum(q.data(), n, q[0], 1, p, &hgot);
        if (href != hgot) {
            if (bad_hit < 5) std::printf("hit mismatch case %d n=%d mode=%d p=%a %d %d\n", tc, n, mode, p, href, hgot);
            ++bad_hit;
        }
    }
    std::printf("%ld %ld %d %ld\n", bad_sum, bad_hit, cases, g_segments);
    return 0;
}
