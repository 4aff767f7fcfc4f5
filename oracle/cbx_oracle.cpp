// cbx_oracle.cpp -- CPU oracle (test infrastructure, never shipped).
//
// A fresh restatement of the chatterbox.cpp T3 sampler,
// tts_cpp::chatterbox::detail::sample_next_token_ex (src/main.cpp:726-801),
// stage by stage, keeping each float operation, its order and precision:
//
//   combine   [extension]  CFG  l = c + w*(c-u), three roundings, no FMA
//   mask      [extension]  allowed bitmask / forced stop -> -inf
//   stage 1   main.cpp:735-738  temperature: s *= (1.0f/temp)
//   stage 2   main.cpp:740-748  top-k on the (k+1)-th largest, -1e-10f quirk
//   stage 3   main.cpp:750-772  top-p in descending std::sort order
//   stage 3b  [extension]  min-p: drop expf(s - max) < min_p (ratio form)
//   stage 4   main.cpp:774-781  repetition penalty, once per distinct id
//   stage 5   main.cpp:783-793  float softmax, sequential sum in index order
//   stage 6   main.cpp:795-800  greedy argmax, or discrete_distribution draw
//             (libstdc++ random.tcc:2657-2677 CDF build, :2697-2712 lookup)
//
// Compiled with -O3 -ffp-contract=off (oracle/Makefile) so no expression is fused.
#include "cbx_oracle.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstring>
#include <numeric>
#include <random>
#include <thread>
#include <vector>

namespace {

constexpr float kNegInf = -INFINITY;

struct Row {
    std::vector<float> s;   // working scores
    uint32_t info = 0;
};

// Extension: CFG combine on raw logits, before anything else.  Upstream
// Chatterbox's form cond + w * (cond - uncond); each operation rounds once.
float cfg_combine(float c, float u, float w) {
    volatile float d = c - u;
    volatile float t = w * d;
    return c + t;
}

// main.cpp:735-738: the reciprocal is formed once in float and multiplied in.
void stage_temperature(Row& r, float temp) {
    if (temp > 0.0f && temp != 1.0f) {
        const float inv_t = 1.0f / temp;
        for (float& v : r.s) v *= inv_t;
    }
}

// main.cpp:740-748: the threshold is the value at position k of a descending
// partial order (the (k+1)-th largest); survivors are strictly above it unless
// fewer than k are, in which case it is nudged down by 1e-10f (in float).
void stage_top_k(Row& r, int32_t top_k) {
    const int n = (int)r.s.size();
    if (!(top_k > 0 && top_k < n)) return;
    std::vector<float> tmp(r.s);
    std::nth_element(tmp.begin(), tmp.begin() + top_k, tmp.end(), std::greater<float>());
    float thr = tmp[top_k];
    int above = 0;
    for (float v : r.s) above += (v > thr) ? 1 : 0;
    if (above < top_k) thr -= 1e-10f;
    for (float& v : r.s)
        if (v <= thr) v = kNegInf;
}

struct Ranked { int idx; float s; };

// Rank the non -inf scores exactly as main.cpp:752-755 does: build in index
// order, then std::sort with a strict "greater score" comparator.  std::sort
// is unstable; using the same library routine on the same sequence gives the
// reference's tie order.
std::vector<Ranked> rank_descending(const Row& r) {
    std::vector<Ranked> v;
    v.reserve(r.s.size());
    for (int i = 0; i < (int)r.s.size(); ++i)
        if (r.s[i] != kNegInf) v.push_back({i, r.s[i]});
    std::sort(v.begin(), v.end(), [](const Ranked& a, const Ranked& b) { return a.s > b.s; });
    return v;
}

// main.cpp:750-772.
void stage_top_p(Row& r, float top_p) {
    if (!(top_p < 1.0f)) return;
    const std::vector<Ranked> sorted = rank_descending(r);
    const float mx = sorted.empty() ? 0.0f : sorted[0].s;
    std::vector<float> pr(sorted.size());
    float psum = 0.0f;
    for (size_t i = 0; i < sorted.size(); ++i) {
        pr[i] = std::exp(sorted[i].s - mx);
        psum += pr[i];
    }
    for (float& x : pr) x /= psum;
    std::vector<char> keep(r.s.size(), 0);
    float cum = 0.0f;
    size_t last = 0;
    bool any = false;
    for (size_t i = 0; i < sorted.size(); ++i) {
        cum += pr[i];
        keep[sorted[i].idx] = 1;
        last = i;
        any = true;
        if (cum >= top_p) break;
    }
    // (main.cpp:770 "keep_set.empty() && !sorted.empty()" cannot fire: the loop
    // above always keeps sorted[0] when sorted is non-empty.)
    if (any && last + 1 < sorted.size() && sorted[last + 1].s == sorted[last].s)
        r.info |= CBX_ORACLE_INFO_TOPP_TIE;
    for (size_t i = 0; i < r.s.size(); ++i)
        if (!keep[i]) r.s[i] = kNegInf;
}

// Extension (after top-p, before the penalty, on the same scores): drop
// survivors whose ratio expf(s - max) to the best survivor is below min_p.
// The best survivor has ratio exactly 1, so at least one always remains.
void stage_min_p(Row& r, float min_p) {
    if (!(min_p > 0.0f)) return;
    float mx = kNegInf;
    bool any = false;
    for (float v : r.s)
        if (v != kNegInf) { mx = any ? std::max(mx, v) : v; any = true; }
    if (!any) return;
    for (float& v : r.s)
        if (v != kNegInf && std::exp(v - mx) < min_p) v = kNegInf;
}

// main.cpp:774-781: each distinct history id once; ids outside [0, n) and
// filtered (-inf) scores are skipped; positive scores divide, others multiply.
void stage_penalty(Row& r, const int32_t* hist, int32_t n_hist, float pen) {
    if (!(pen != 1.0f) || n_hist <= 0) return;
    const int n = (int)r.s.size();
    std::vector<char> seen(n, 0);
    for (int32_t j = 0; j < n_hist; ++j) {
        const int32_t t = hist[j];
        if (t >= 0 && t < n) seen[t] = 1;
    }
    for (int t = 0; t < n; ++t) {
        if (!seen[t] || r.s[t] == kNegInf) continue;
        r.s[t] = r.s[t] > 0 ? r.s[t] / pen : r.s[t] * pen;
    }
}

// main.cpp:783-793.  Returns false for the psum == 0 exit (token 0).
bool stage_softmax(const Row& r, std::vector<float>& probs) {
    const int n = (int)r.s.size();
    float mx = kNegInf;
    for (float v : r.s)
        if (v != kNegInf) mx = std::max(mx, v);
    probs.assign(n, 0.0f);
    float psum = 0.0f;
    for (int i = 0; i < n; ++i) {
        probs[i] = (r.s[i] == kNegInf) ? 0.0f : std::exp(r.s[i] - mx);
        psum += probs[i];
    }
    if (psum == 0.0f) return false;
    for (float& x : probs) x /= psum;
    return true;
}

// std::discrete_distribution<int>(probs)(u) as libstdc++ 11 computes it
// (random.tcc:2657-2677 builds the CDF: double weights, accumulate from 0.0,
// divide each by the sum, partial_sum, force the last entry to 1.0; then
// :2697-2712 returns lower_bound(cdf, u)).  Fewer than two weights: no CDF,
// result 0 and no draw.
int32_t draw_from_cdf(const std::vector<float>& probs, double u) {
    const size_t n = probs.size();
    if (n < 2) return 0;
    std::vector<double> w(probs.begin(), probs.end());
    const double sum = std::accumulate(w.begin(), w.end(), 0.0);
    for (double& x : w) x = x / sum;
    std::vector<double> cdf(n);
    double acc = 0.0;
    for (size_t i = 0; i < n; ++i) { acc = (i == 0) ? w[0] : acc + w[i]; cdf[i] = acc; }
    cdf[n - 1] = 1.0;
    return (int32_t)(std::lower_bound(cdf.begin(), cdf.end(), u) - cdf.begin());
}

bool has_nonfinite(const std::vector<float>& s) {
    for (float v : s)
        if (std::isnan(v) || v == INFINITY) return true;
    return false;
}

// Stages up to and including the softmax; shared by the u-injected and the
// mt19937 front-ends.  Returns false for an EMPTY row.
bool run_filters(Row& r, const float* logits, const float* uncond, int32_t n_vocab,
                 const int32_t* hist, int32_t n_hist, const cbx_oracle_params& p,
                 const uint32_t* allowed, int32_t force_stop, int32_t stop_token,
                 std::vector<float>& probs) {
    r.s.assign(logits, logits + n_vocab);                       // main.cpp:733
    if (uncond)
        for (int i = 0; i < n_vocab; ++i) r.s[i] = cfg_combine(logits[i], uncond[i], p.cfg_weight);
    if (allowed)
        for (int i = 0; i < n_vocab; ++i)
            if (!((allowed[i >> 5] >> (i & 31)) & 1u)) r.s[i] = kNegInf;
    if (force_stop)
        for (int i = 0; i < n_vocab; ++i)
            if (i != stop_token) r.s[i] = kNegInf;
    stage_temperature(r, p.temp);
    if (has_nonfinite(r.s)) r.info |= CBX_ORACLE_INFO_NONFINITE;
    stage_top_k(r, p.top_k);
    stage_top_p(r, p.top_p);
    stage_min_p(r, p.min_p);
    stage_penalty(r, hist, n_hist, p.repeat_penalty);
    return stage_softmax(r, probs);
}

int32_t first_argmax(const std::vector<float>& probs) {
    return (int32_t)(std::max_element(probs.begin(), probs.end()) - probs.begin());
}

int32_t count_kept(const std::vector<float>& probs) {
    int32_t k = 0;
    for (float x : probs) k += (x != 0.0f) ? 1 : 0;
    return k;
}

}  // namespace

extern "C" {

int32_t cbx_oracle_sample_row(const float* logits, const float* logits_uncond,
                              int32_t n_vocab, const int32_t* history,
                              int32_t n_history, const cbx_oracle_params* p,
                              const uint32_t* allowed, int32_t force_stop,
                              int32_t stop_token, double u, uint32_t* info,
                              float* probs_out, int32_t* kept_out) {
    Row r;
    std::vector<float> probs;
    int32_t tok;
    const bool ok = run_filters(r, logits, logits_uncond, n_vocab, history, n_history, *p,
                                allowed, force_stop, stop_token, probs);
    if (!ok) {
        r.info |= CBX_ORACLE_INFO_EMPTY;
        tok = 0;
        probs.assign(n_vocab, 0.0f);
    } else if (p->temp <= 0.0f) {
        r.info |= CBX_ORACLE_INFO_GREEDY;
        tok = first_argmax(probs);
    } else {
        if (n_vocab >= 2) r.info |= CBX_ORACLE_INFO_DREW;
        tok = draw_from_cdf(probs, u);
    }
    if (info) *info = r.info;
    if (probs_out) std::memcpy(probs_out, probs.data(), sizeof(float) * (size_t)n_vocab);
    if (kept_out) *kept_out = count_kept(probs);
    return tok;
}

void cbx_oracle_run_mt19937(const float* logits, int32_t n_steps, int32_t n_vocab,
                            const int32_t* history, int32_t n_history,
                            int32_t grow_history, const cbx_oracle_params* p,
                            uint32_t seed, int32_t* tokens_out, double* u_out) {
    std::mt19937 rng(seed);                                      // engine.cpp:326
    std::vector<int32_t> generated(history, history + n_history);
    for (int32_t t = 0; t < n_steps; ++t) {
        Row r;
        std::vector<float> probs;
        const float* row = logits + (size_t)t * n_vocab;
        const bool ok = run_filters(r, row, nullptr, n_vocab, generated.data(),
                                    (int32_t)generated.size(), *p, nullptr, 0, 0, probs);
        int32_t tok;
        double used = -1.0;
        if (!ok) {
            tok = 0;
        } else if (p->temp <= 0.0f) {
            tok = first_argmax(probs);
        } else {
            // The library routine itself, on the caller's engine (main.cpp:799-800).
            std::mt19937 peek = rng;
            used = std::generate_canonical<double, std::numeric_limits<double>::digits>(peek);
            std::discrete_distribution<int> dist(probs.begin(), probs.end());
            tok = dist(rng);
            if (n_vocab < 2) used = -1.0;
        }
        tokens_out[t] = tok;
        if (u_out) u_out[t] = used;
        if (grow_history) generated.push_back(tok);             // engine.cpp:352
    }
}

int32_t cbx_oracle_cdf_draw(const float* probs, int32_t n, double u) {
    return draw_from_cdf(std::vector<float>(probs, probs + n), u);
}

namespace {
// A UniformRandomBitGenerator over [0, 2^32) that replays two fixed words.
struct TwoWords {
    using result_type = uint32_t;
    uint32_t w[2];
    int i = 0;
    static constexpr result_type min() { return 0u; }
    static constexpr result_type max() { return 0xFFFFFFFFu; }
    result_type operator()() { return w[(i++) & 1]; }
};
}  // namespace

int32_t cbx_oracle_stdlib_draw(const float* probs, int32_t n, uint32_t x0, uint32_t x1) {
    TwoWords g{{x0, x1}};
    std::discrete_distribution<int> dist(probs, probs + n);
    return dist(g);
}

void cbx_oracle_mt_canonical(uint32_t seed, uint64_t discard, int32_t n, double* out) {
    std::mt19937 rng(seed);
    rng.discard(discard);
    for (int32_t i = 0; i < n; ++i)
        out[i] = std::generate_canonical<double, std::numeric_limits<double>::digits>(rng);
}

uint32_t cbx_oracle_mt_10000th(void) {
    std::mt19937 rng;
    rng.discard(9999);
    return (uint32_t)rng();
}

// Philox4x32-10, written from Salmon, Moraes, Dror, Shaw, "Parallel random
// numbers: as easy as 1, 2, 3" (SC'11), section 4: two 32x32->64 multiplies per
// round with multipliers 0xD2511F53 / 0xCD9E8D57, Weyl key schedule
// 0x9E3779B9 / 0xBB67AE85, ten rounds, key bumped between rounds.
void cbx_oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t x0 = ctr[0], x1 = ctr[1], x2 = ctr[2], x3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int round = 0; round < 10; ++round) {
        if (round) { k0 += 0x9E3779B9u; k1 += 0xBB67AE85u; }
        const uint64_t p0 = (uint64_t)0xD2511F53u * x0;
        const uint64_t p1 = (uint64_t)0xCD9E8D57u * x2;
        const uint32_t y0 = (uint32_t)(p1 >> 32) ^ x1 ^ k0;
        const uint32_t y1 = (uint32_t)p1;
        const uint32_t y2 = (uint32_t)(p0 >> 32) ^ x3 ^ k1;
        const uint32_t y3 = (uint32_t)p0;
        x0 = y0; x1 = y1; x2 = y2; x3 = y3;
    }
    out[0] = x0; out[1] = x1; out[2] = x2; out[3] = x3;
}

double cbx_oracle_philox_uniform(uint64_t seed, uint64_t stream, uint64_t step) {
    const uint32_t ctr[4] = {(uint32_t)step, (uint32_t)(step >> 32), (uint32_t)stream,
                             (uint32_t)(stream >> 32)};
    const uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    cbx_oracle_philox4x32_10(ctr, key, o);
    // Matsumoto & Nishimura's genrand_res53 construction (27 + 26 bits).
    const double a = (double)(o[0] >> 5), b = (double)(o[1] >> 6);
    return (a * 67108864.0 + b) * (1.0 / 9007199254740992.0);
}

double cbx_oracle_sample_batch(const float* logits, const float* logits_uncond,
                               int64_t ld, int32_t n_rows, int32_t n_vocab,
                               const int32_t* history, int64_t ld_hist,
                               const int32_t* hist_len,
                               const cbx_oracle_params* params,
                               const uint32_t* allowed, int64_t ld_allowed,
                               const uint8_t* force_stop, int32_t stop_token,
                               const double* u, int32_t n_threads,
                               int32_t* tokens_out, uint32_t* info_out) {
    auto work = [&](int32_t r0, int32_t r1) {
        for (int32_t r = r0; r < r1; ++r) {
            uint32_t info = 0;
            tokens_out[r] = cbx_oracle_sample_row(
                logits + (size_t)r * ld, logits_uncond ? logits_uncond + (size_t)r * ld : nullptr,
                n_vocab, history ? history + (size_t)r * ld_hist : nullptr,
                hist_len ? hist_len[r] : 0, &params[r],
                allowed ? allowed + (size_t)r * ld_allowed : nullptr,
                force_stop ? force_stop[r] : 0, stop_token, u[r], &info, nullptr, nullptr);
            if (info_out) info_out[r] = info;
        }
    };
    const auto t0 = std::chrono::steady_clock::now();
    if (n_threads <= 1) {
        work(0, n_rows);
    } else {
        std::vector<std::thread> th;
        for (int32_t t = 0; t < n_threads; ++t) {
            const int32_t a = (int32_t)((int64_t)n_rows * t / n_threads);
            const int32_t b = (int32_t)((int64_t)n_rows * (t + 1) / n_threads);
            th.emplace_back(work, a, b);
        }
        for (auto& x : th) x.join();
    }
    const auto t1 = std::chrono::steady_clock::now();
    return std::chrono::duration<double>(t1 - t0).count();
}

// IEEE binary16 -> binary32 (exact).
static float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    uint32_t bits;
    if (e == 0) {
        if (m == 0) {
            bits = sign;
        } else {  // subnormal: m * 2^-24
            float f = (float)m * 5.9604644775390625e-8f;
            std::memcpy(&bits, &f, 4);
            bits |= sign;
        }
    } else if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else {
        bits = sign | ((e + 112) << 23) | (m << 13);
    }
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}

// binary32 -> binary16, round to nearest even (finite inputs in range).
static uint16_t float_to_half(float f) {
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int32_t e = (int32_t)((x >> 23) & 0xff) - 127 + 15;
    uint32_t m = x & 0x7fffffu;
    if (((x >> 23) & 0xff) == 0xff) return (uint16_t)(sign | 0x7c00u | (m ? 0x200u : 0u));
    if (e >= 31) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)sign;
        m |= 0x800000u;
        const int shift = 14 - e;
        uint32_t hm = m >> shift;
        const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (hm & 1u))) ++hm;
        return (uint16_t)(sign | hm);
    }
    uint32_t hm = m >> 13;
    const uint32_t rem = m & 0x1fffu;
    uint32_t out = sign | ((uint32_t)e << 10) | hm;
    if (rem > 0x1000u || (rem == 0x1000u && (hm & 1u))) ++out;
    return (uint16_t)out;
}

static size_t block_bytes(int32_t wtype) {
    return wtype == 2 ? 18 : wtype == 6 ? 22 : 34;
}

// The formats' values (ggml's block layouts: ggml-common.h block_q4_0,
// block_q5_0, block_q8_0 -- a third-party dependency the reference links and
// does not vendor; the layouts are the GGUF format's).
void cbx_oracle_dequant_row(const uint8_t* blocks, int32_t wtype, int32_t n_embd, float* out) {
    const int nb = n_embd / 32;
    const size_t bsz = block_bytes(wtype);
    for (int b = 0; b < nb; ++b) {
        const uint8_t* blk = blocks + (size_t)b * bsz;
        uint16_t dh;
        std::memcpy(&dh, blk, 2);
        const float d = half_to_float(dh);
        if (wtype == 2) {  // Q4_0: d, 16 bytes of nibbles
            for (int j = 0; j < 16; ++j) {
                out[b * 32 + j] = (float)((int)(blk[2 + j] & 0x0f) - 8) * d;
                out[b * 32 + j + 16] = (float)((int)(blk[2 + j] >> 4) - 8) * d;
            }
        } else if (wtype == 6) {  // Q5_0: d, qh (little-endian u32), 16 bytes of nibbles
            const uint32_t qh = (uint32_t)blk[2] | (uint32_t)blk[3] << 8 |
                                (uint32_t)blk[4] << 16 | (uint32_t)blk[5] << 24;
            for (int j = 0; j < 16; ++j) {
                const int q0 = (blk[6 + j] & 0x0f) | (int)((qh >> j) & 1u) << 4;
                const int q1 = (blk[6 + j] >> 4) | (int)((qh >> (16 + j)) & 1u) << 4;
                out[b * 32 + j] = (float)(q0 - 16) * d;
                out[b * 32 + j + 16] = (float)(q1 - 16) * d;
            }
        } else {  // Q8_0: d, 32 int8
            for (int j = 0; j < 32; ++j) out[b * 32 + j] = (float)(int8_t)blk[2 + j] * d;
        }
    }
}

// The quantizer of the reference's converter, gguf-py 0.18's
// gguf.quants.quantize (scripts/convert-t3-turbo-to-gguf.py:78-104), per
// block of 32: Q4_0 / Q5_0 take the signed value of largest magnitude mx,
// d = mx / -8 (-16), id = 1 / d (0 for d = 0), q = trunc(float(double(x) *
// double(id) + 8.5 (16.5))) clipped to [0, 15] ([0, 31]) -- the product
// exact in binary64, one rounding to binary64 and one to binary32 before the
// truncation; Q8_0 d = max|x| / 127, q = round half away from zero of x * id
// in binary32.  d is stored as binary16 (round to nearest even).
void cbx_oracle_quantize(const float* w, int32_t n_rows, int32_t n_embd, int32_t wtype,
                         uint8_t* blocks_out) {
    const int nb = n_embd / 32;
    const size_t bsz = block_bytes(wtype);
    for (int32_t r = 0; r < n_rows; ++r) {
        for (int b = 0; b < nb; ++b) {
            const float* x = w + (size_t)r * n_embd + b * 32;
            uint8_t* blk = blocks_out + ((size_t)r * nb + b) * bsz;
            std::memset(blk, 0, bsz);
            if (wtype == 2 || wtype == 6) {
                const int qmax = wtype == 2 ? 15 : 31;
                const float half = wtype == 2 ? 8.0f : 16.0f;
                float amax = 0.0f, mx = 0.0f;
                for (int j = 0; j < 32; ++j)
                    if (amax < std::fabs(x[j])) { amax = std::fabs(x[j]); mx = x[j]; }
                const float d = mx / -half;
                const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
                const uint16_t dh = float_to_half(d);
                std::memcpy(blk, &dh, 2);
                int q[32];
                for (int j = 0; j < 32; ++j) {
                    const double t = (double)x[j] * (double)id + ((double)half + 0.5);
                    q[j] = std::min(qmax, std::max(0, (int)std::trunc((float)t)));
                }
                uint8_t* qs = blk + (wtype == 2 ? 2 : 6);
                for (int j = 0; j < 16; ++j) qs[j] = (uint8_t)((q[j] & 15) | (q[16 + j] & 15) << 4);
                if (wtype == 6) {
                    uint32_t qh = 0;
                    for (int j = 0; j < 32; ++j) qh |= (uint32_t)(q[j] >> 4) << j;
                    for (int i = 0; i < 4; ++i) blk[2 + i] = (uint8_t)(qh >> (8 * i));
                }
            } else {
                float amax = 0.0f;
                for (int j = 0; j < 32; ++j) amax = std::max(amax, std::fabs(x[j]));
                const float d = amax / 127.0f;
                const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
                const uint16_t dh = float_to_half(d);
                std::memcpy(blk, &dh, 2);
                for (int j = 0; j < 32; ++j) blk[2 + j] = (uint8_t)(int8_t)std::lround(x[j] * id);
            }
        }
    }
}

void cbx_oracle_head_f64(const uint8_t* W, int32_t wtype, const float* bias,
                         const float* hidden, int32_t n_rows, int32_t n_vocab,
                         int32_t n_embd, double* out) {
    const size_t row_bytes = (size_t)(n_embd / 32) * block_bytes(wtype);
    std::vector<float> wrow(n_embd);
    for (int32_t v = 0; v < n_vocab; ++v) {
        cbx_oracle_dequant_row(W + (size_t)v * row_bytes, wtype, n_embd, wrow.data());
        for (int32_t r = 0; r < n_rows; ++r) {
            double acc = 0.0;
            const float* h = hidden + (size_t)r * n_embd;
            for (int32_t j = 0; j < n_embd; ++j) acc += (double)wrow[j] * (double)h[j];
            out[(size_t)r * n_vocab + v] = acc + (bias ? (double)bias[v] : 0.0);
        }
    }
}

void cbx_oracle_expf(const float* in, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = std::exp(in[i]);
}

int64_t cbx_oracle_expf_mismatch(uint32_t first_bits, int64_t n, const float* out,
                                 int32_t n_threads) {
    if (n_threads < 1) n_threads = 1;
    std::vector<int64_t> bad(n_threads, 0);
    auto work = [&](int t) {
        const int64_t a = n * t / n_threads, b = n * (t + 1) / n_threads;
        int64_t c = 0;
        for (int64_t i = a; i < b; ++i) {
            const uint32_t bits = first_bits + (uint32_t)i;
            float x;
            std::memcpy(&x, &bits, 4);
            const float ref = std::exp(x);
            uint32_t rb, ob;
            std::memcpy(&rb, &ref, 4);
            std::memcpy(&ob, &out[i], 4);
            c += (rb != ob) ? 1 : 0;
        }
        bad[t] = c;
    };
    std::vector<std::thread> th;
    for (int t = 0; t < n_threads; ++t) th.emplace_back(work, t);
    for (auto& x : th) x.join();
    int64_t total = 0;
    for (int64_t c : bad) total += c;
    return total;
}

}  // extern "C"
