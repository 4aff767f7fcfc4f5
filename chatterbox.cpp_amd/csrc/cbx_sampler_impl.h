// cbx_sampler_impl.h -- gfx950 kernels for the T3 logits->token sampler
// (templates; each cbx_sampler_v*.hip instantiates one vocabulary class so
// the variants compile in parallel).
//
// One workgroup samples one (step, stream) row; a launch covers
// n_steps x n_rows rows.  The row's scores arrive in registers (EPT per lane,
// element i = j*BLOCK + tid, so every global load and store is coalesced).
// Stage order and arithmetic follow sample_next_token_ex (src/main.cpp:726-801):
//
//   load + CFG combine + masks + temperature   (main.cpp:733-738)
//   top-k (main.cpp:740-748): the (k+1)-th largest score is found by one
//          histogram over value bins spanning [min, max] -- a monotone map, so
//          the bin holding rank k is exact -- and an exact selection among
//          the few scores in that bin; rows with non-finite scores use a
//          12+12+8-bit radix select instead.  Then the -1e-10f nudge.
//   fast path (<= 2048 survivors): the survivors move to a register list;
//          top-p sorts it with a bitonic network (lane shuffles in a wave,
//          LDS across waves), min-p and the penalty work on the list
//   general path (more survivors): scores stay per element, top-p sorts
//          (score, id) pairs in LDS
//   top-p (main.cpp:750-772), min-p [extension], repetition penalty from an
//          LDS bitmap of the history (main.cpp:774-781), softmax with the
//          binary32 running sum in id order (main.cpp:783-793), greedy argmax
//          or the libstdc++ discrete_distribution CDF (main.cpp:795-800;
//          random.tcc:2657-2712)
//
// Exactness.  The binary32 running sums take the reference's values: one
// wave holds a run of consecutive terms per lane and evaluates the sum by
// binade segments (finite terms; chain_segments_x) or by sweep chains of
// dependent IEEE adds over the lanes, so every partial sum is the
// reference's.
// The binary64 CDF is located in parallel with a certified margin: the
// parallel cumulative values differ from the reference's sequential ones by
// < 1.5e-11, so when the uniform lies more than 1e-9 from both neighbouring
// boundaries the token is the reference's; otherwise (about 4e-9 of draws)
// one lane replays the reference's sequential CDF exactly.
// Arithmetic uses explicitly rounded intrinsics (__fadd_rn, ...), and the
// library is built with -ffp-contract=off as well.
#pragma once

#include <hip/hip_runtime.h>

#include "cbx_expf.h"
#include "cbx_internal.h"
#include "cbx_philox.h"
#include "cbx_stdsort.h"

// Stage timestamps for a profiling build (CBX_STAGE_CLOCKS defined, one
// translation unit): wave 0 of each of the first 16384 workgroups records the
// shader clock at each marker (0 .. 63, 64 slots per workgroup).  Compiled
// out otherwise.
#if defined(CBX_STAGE_CLOCKS)
__device__ unsigned long long cbx_stage_clock[16384 * 64];
#define CBX_STAMP(n)                                                      \
    do {                                                                  \
        static_assert((n) >= 0 && (n) < 64, "stage marker out of range"); \
        if (threadIdx.x == 0 && blockIdx.x < 16384)                       \
            cbx_stage_clock[blockIdx.x * 64 + (n)] = clock64();           \
    } while (0)
#else
#define CBX_STAMP(n) ((void)0)
#endif

namespace cbx {
namespace {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();
constexpr int kFastMax = 2048;    // survivors handled on the register-list path
constexpr int kValueBins = 2048;  // value histogram of the top-k select
constexpr int kCandMax = 512;     // scores in the selected bin
constexpr int kRadixBins = 4096;  // 12-bit digits of the fallback radix select
constexpr int kSortBins = 2048;   // value bins of the survivor counting sort
constexpr int kSortBinMax = 64;   // largest bin the counting sort ranks directly
constexpr int kKeyBins = 4096;    // value bins of the general path's key sort
constexpr int kKeyBinMax = 255;   // largest bin it ranks directly (8-bit slots)
// Relative distance from u to a located CDF boundary beyond which the draw
// on the binary64 prefix of the exp terms is certain (the reference's values
// are within 2^-23 relative of it).
constexpr double kDrawMargin = 3e-7;
// Word 3 of a raw buffer resource on gfx9-family parts (data format 32-bit,
// no swizzle): loads past num_records return 0.
constexpr int kBufferWord3 = 0x00020000;

// ---------------------------------------------------------------- helpers

// Monotone map float -> uint32 (ascending float order = ascending key).
__device__ __forceinline__ uint32_t okey(float f) {
    const uint32_t b = __builtin_bit_cast(uint32_t, f);
    return b ^ ((b & 0x80000000u) ? 0xFFFFFFFFu : 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
    const uint32_t b = k ^ ((k & 0x80000000u) ? 0x80000000u : 0xFFFFFFFFu);
    return __builtin_bit_cast(float, b);
}
// Composite sort key: ascending order = descending score, then ascending id.
__device__ __forceinline__ uint64_t desc_key(float s, uint32_t idx) {
    return ((uint64_t)(~okey(s)) << 32) | idx;
}
__device__ __forceinline__ float desc_key_value(uint64_t k) { return okey_inv(~(uint32_t)(k >> 32)); }

// Values that are the same in every lane, kept in scalar registers so that
// the branches they control are scalar branches.
__device__ __forceinline__ int uni(int v) { return __builtin_amdgcn_readfirstlane(v); }
// An opaque copy of a wave-uniform double in scalar registers: its
// computation stays where it is written (not sunk to its use).
__device__ __forceinline__ double fresh_d(double v) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    int lo = __builtin_amdgcn_readfirstlane((int)(uint32_t)b);
    int hi = __builtin_amdgcn_readfirstlane((int)(uint32_t)(b >> 32));
    asm volatile("" : "+s"(lo), "+s"(hi));
    return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}
__device__ __forceinline__ float unif(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ int wave_min_i(int x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o, 64));
    return x;
}

__device__ __forceinline__ double wave_incl_scan_f64(double x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const double t = __shfl_up(x, o, 64);
        if (lane >= o) x = __dadd_rn(x, t);
    }
    return x;
}

// Bytes of the LDS region after the three bitmaps (seen, keptw, woff) for a
// survivor capacity: the largest of its uses (radix histogram, value bins and
// candidates, the counting sort's offsets and list, the sorted scores or F).
__host__ __device__ inline size_t region_bytes(int32_t cap) {
    size_t region = (size_t)kRadixBins * 4;
    const size_t bins = (size_t)kValueBins * 4 + (size_t)kCandMax * 4;
    if (bins > region) region = bins;
    const size_t list = (size_t)(cap < kFastMax ? (cap < 64 ? 64 : cap) : kFastMax);
    const size_t fast = (size_t)(kSortBins + 4) * 4 + 8 * list;
    if (fast > region) region = fast;
    // general path: the keys, then the key sort's bin offsets
    if (cap > kFastMax && (size_t)cap * 4 + (size_t)(kKeyBins + 4) * 4 > region)
        region = (size_t)cap * 4 + (size_t)(kKeyBins + 4) * 4;
    return region;
}

struct Shared {
    // the block reductions' per-wave slots, two sets used in turn (the
    // row's phase ph): one barrier per reduction (see block_excl_scan)
    int red_i[2][16];
    float red_f[2][16];
    float red_f2[2][16];
    uint32_t sel_digit, sel_above;
    int bin, above_bins, n_cand, above;
    float thr;
    float psum;        // broadcast of a running sum
    float mx;          // broadcast of the top survivor score
    int n_kept;        // survivors after top-p
    float tie[2];      // scores at the top-p cutoff and just after it
    uint32_t flags;
    uint32_t mxk;      // okey of the largest kept score (an LDS maximum)
};

__device__ __forceinline__ int wave_incl_scan_dpp(int x);
__device__ __forceinline__ int wave_sum_dpp(int x);
__device__ __forceinline__ float wave_max_dpp(float x);
__device__ __forceinline__ float wave_min_dpp(float x);
__device__ __forceinline__ int wave_min_i_dpp(int x);

// Exclusive block scan of one int per lane; `total` receives the block sum.
// The wave steps are DPP operations (no LDS round trip per step), as in every
// block reduction below.  Each reduction takes one barrier: its waves' slots
// are set ph of the reduction slots, and consecutive reductions of a row use
// the two sets in turn (ph, 0 at the row's start in every thread, flips per
// reduction).  A wave that writes set ph again has passed the barrier of the
// reduction in between, which no wave reaches before it has read set ph.
template <int BLOCK>
__device__ __forceinline__ int block_excl_scan(int v, Shared& sh, int& total, int& ph) {
    constexpr int NW = BLOCK / 64;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int incl = wave_incl_scan_dpp(v);
    int* const slot = sh.red_i[ph];
    ph ^= 1;
    if (lane == 63) slot[wid] = incl;
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const int t = slot[w];
        before += (w < wid) ? t : 0;
        tot += t;
    }
    total = uni(tot);
    return before + incl - v;
}

template <int BLOCK>
__device__ __forceinline__ int block_sum(int v, Shared& sh, int& ph) {
    int total;
    (void)block_excl_scan<BLOCK>(v, sh, total, ph);
    return total;
}

template <int BLOCK>
__device__ __forceinline__ float block_max(float v, Shared& sh, int& ph) {
    constexpr int NW = BLOCK / 64;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_max_dpp(v);
    float* const slot = sh.red_f[ph];
    ph ^= 1;
    if (lane == 0) slot[wid] = v;
    __syncthreads();
    float m = slot[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, slot[w]);
    return unif(m);
}


// min and max of the finite scores and whether any score is NaN / +inf.
template <int BLOCK>
__device__ __forceinline__ void block_minmax(float lo, float hi, int bad, Shared& sh, float& blo,
                                             float& bhi, int& bbad, int& ph) {
    constexpr int NW = BLOCK / 64;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    lo = wave_min_dpp(lo);
    hi = wave_max_dpp(hi);
    bad = wave_sum_dpp(bad != 0 ? 1 : 0);
    float* const sl = sh.red_f[ph];
    float* const sh2 = sh.red_f2[ph];
    int* const sb = sh.red_i[ph];
    ph ^= 1;
    if (lane == 0) { sl[wid] = lo; sh2[wid] = hi; sb[wid] = bad; }
    __syncthreads();
    float l = sl[0], h = sh2[0];
    int b = sb[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) {
        l = fminf(l, sl[w]);
        h = fmaxf(h, sh2[w]);
        b |= sb[w];
    }
    blo = unif(l);
    bhi = unif(h);
    bbad = uni(b);
}

// --------------------------------------------------------- top-k selection

// One radix-select pass over BITS bits at SHIFT of the keys matching `prefix`
// under `pmask`; finds the digit holding the element with `rem` larger
// matching keys (descending) and narrows prefix / pmask / rem.
template <int BLOCK, int EPT, int SHIFT, int BITS>
__device__ __forceinline__ void radix_pass(const float (&s)[EPT], int n_valid, uint32_t& prefix,
                                           uint32_t& pmask, uint32_t& rem, uint32_t* hist,
                                           Shared& sh, int& ph) {
    constexpr int NB = 1 << BITS;
    constexpr int BPT = NB >= BLOCK ? NB / BLOCK : 1;  // bins per lane
    constexpr int NT = NB / BPT;                        // lanes holding bins
    const int tid = threadIdx.x;
    for (int i = tid; i < NB; i += BLOCK) hist[i] = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = j * BLOCK + tid;
        const uint32_t k = okey(s[j]);
        if (i < n_valid && (k & pmask) == prefix) atomicAdd(&hist[(k >> SHIFT) & (NB - 1)], 1u);
    }
    __syncthreads();
    uint32_t c[BPT];
    int tot = 0;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
        c[q] = (tid < NT) ? hist[NB - 1 - (tid * BPT + q)] : 0u;
        tot += (int)c[q];
    }
    int all;
    uint32_t excl = (uint32_t)block_excl_scan<BLOCK>(tot, sh, all, ph);
    if (tid < NT && excl <= rem && rem < excl + (uint32_t)tot) {
#pragma unroll
        for (int q = 0; q < BPT; ++q) {
            if (excl + c[q] > rem) {
                sh.sel_digit = (uint32_t)(NB - 1 - (tid * BPT + q));
                sh.sel_above = excl;
                break;
            }
            excl += c[q];
        }
    }
    __syncthreads();
    prefix |= (uint32_t)uni((int)sh.sel_digit) << SHIFT;
    pmask |= (uint32_t)(NB - 1) << SHIFT;
    rem -= (uint32_t)uni((int)sh.sel_above);
    __syncthreads();
}

// The (rank+1)-th largest key among the first n_valid elements (rank 0-based).
template <int BLOCK, int EPT>
__device__ __forceinline__ uint32_t radix_select_desc(const float (&s)[EPT], int n_valid, int rank,
                                      uint32_t* hist, Shared& sh, int& ph) {
    uint32_t prefix = 0, pmask = 0, rem = (uint32_t)rank;
    radix_pass<BLOCK, EPT, 20, 12>(s, n_valid, prefix, pmask, rem, hist, sh, ph);
    radix_pass<BLOCK, EPT, 8, 12>(s, n_valid, prefix, pmask, rem, hist, sh, ph);
    radix_pass<BLOCK, EPT, 0, 8>(s, n_valid, prefix, pmask, rem, hist, sh, ph);
    return prefix;
}

// Top-k threshold by value bins.  bin(v) = min(NB-1, int((v - lo) * scale))
// is non-decreasing in v (each rounded operation is monotone), so every
// score in a higher bin is strictly larger than every score in a lower one:
// the bin holding rank k is found from the histogram and the threshold is the
// exact (rem+1)-th largest among that bin's scores.  Returns false (the
// caller falls back to the radix select) when the bin width is not a finite
// positive number or the bin holds more than kCandMax scores.  On success thr
// is the (k+1)-th largest score (-inf when at most k scores are finite) and
// `above` the number of scores strictly larger.
template <int BLOCK, int EPT>
__device__ __forceinline__ bool topk_value_bins(const float (&s)[EPT], int k, float lo, float hi, uint32_t* hist,
                                float* cand, Shared& sh, float& thr, int& above, int& ph) {
    constexpr int NB = kValueBins;
    constexpr int BPT = NB / BLOCK >= 1 ? NB / BLOCK : 1;
    constexpr int NT = NB / BPT;
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const float scale = __fdiv_rn((float)NB, __fsub_rn(hi, lo));
    if (!(scale < kPosInf) || !(scale > 0.0f)) return false;
    for (int i = tid; i < NB; i += BLOCK) hist[i] = 0u;
    if (tid == 0) sh.n_cand = 0;
    __syncthreads();
    // bin of a score (recomputed where needed rather than held per element)
    auto bin_of = [&](float v) { return min(NB - 1, (int)__fmul_rn(__fsub_rn(v, lo), scale)); };
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if (s[j] != kNegInf) atomicAdd(&hist[bin_of(s[j])], 1u);
    __syncthreads();
    // bins in descending order: lane t owns NB-1-t*BPT .. NB-BPT-t*BPT
    uint32_t c[BPT];
    int tot = 0;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
        c[q] = (tid < NT) ? hist[NB - 1 - (tid * BPT + q)] : 0u;
        tot += (int)c[q];
    }
    int n_fin;
    int excl = block_excl_scan<BLOCK>(tot, sh, n_fin, ph);
    if (n_fin <= k) {  // the (k+1)-th largest is -inf: nothing is removed
        thr = kNegInf;
        above = n_fin;
        return true;
    }
    if (tid < NT && excl <= k && k < excl + tot) {
#pragma unroll
        for (int q = 0; q < BPT; ++q) {
            if (excl + (int)c[q] > k) {
                sh.bin = NB - 1 - (tid * BPT + q);
                sh.above_bins = excl;
                break;
            }
            excl += (int)c[q];
        }
    }
    __syncthreads();
    const int bsel = uni(sh.bin);
    const int above_bins = uni(sh.above_bins);
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        if (s[j] != kNegInf && bin_of(s[j]) == bsel) {
            const int at = atomicAdd(&sh.n_cand, 1);
            if (at < kCandMax) cand[at] = s[j];
        }
    }
    __syncthreads();
    const int n_c = uni(sh.n_cand);
    if (n_c > kCandMax) return false;
    const int rem = k - above_bins;  // 0 <= rem < n_c
    if (wid == 0) {
        if (n_c <= 64) {
            // one candidate per lane, ranked against the others by readlane
            // (no LDS round trip per comparison)
            const float v = lane < n_c ? cand[lane] : kNegInf;
            int gt = 0, ge = 0;
            for (int t = 0; t < n_c; ++t) {
                const float w = __builtin_bit_cast(
                    float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), t));
                gt += (w > v) ? 1 : 0;
                ge += (w >= v) ? 1 : 0;
            }
            if (lane < n_c && gt <= rem && rem < ge) {  // equal candidates all write the same
                sh.thr = v;
                sh.above = above_bins + gt;
            }
        } else {
            for (int c0 = lane; c0 < n_c; c0 += 64) {
                const float v = cand[c0];
                int gt = 0, ge = 0;
                for (int t = 0; t < n_c; ++t) {
                    const float w = cand[t];
                    gt += (w > v) ? 1 : 0;
                    ge += (w >= v) ? 1 : 0;
                }
                if (gt <= rem && rem < ge) {  // equal candidates all write the same
                    sh.thr = v;
                    sh.above = above_bins + gt;
                }
            }
        }
    }
    __syncthreads();
    thr = unif(sh.thr);
    above = uni(sh.above);
    return true;
}

// ------------------------------------------------------------------ sorting

// Value of lane (lane ^ J) of the wave, J < 64: DPP quad permutes for J = 1, 2,
// ds_swizzle (xor mode, within 32 lanes) for J = 4..16, ds_bpermute for 32.
template <int J>
__device__ __forceinline__ uint32_t xlane(uint32_t v) {
    if constexpr (J == 1) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
    } else if constexpr (J == 2) {
        return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
    } else if constexpr (J < 32) {
        return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x1F | (J << 10));
    } else {
        return (uint32_t)__builtin_amdgcn_ds_bpermute((int)(((threadIdx.x & 63) ^ 32) << 2), (int)v);
    }
}
template <int J>
__device__ __forceinline__ uint64_t xlane64(uint64_t v) {
    return ((uint64_t)xlane<J>((uint32_t)(v >> 32)) << 32) | xlane<J>((uint32_t)v);
}

// One stage (block size K, partner distance J) of an ascending bitonic
// network over NR*BLOCK keys held at positions r*BLOCK + tid.
template <int BLOCK, int NR, int K, int J>
__device__ __forceinline__ void bitonic_stage(uint64_t (&x)[NR], uint64_t* xbuf) {
    const int tid = threadIdx.x;
    if constexpr (J >= BLOCK) {  // partner in the same lane, another row
        constexpr int JR = J / BLOCK;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            if ((r & JR) == 0) {
                const int i = r * BLOCK + tid;
                const bool up = (i & K) == 0;
                const uint64_t p = x[r], q = x[r | JR];
                const bool sw = (p > q) == up;
                x[r] = sw ? q : p;
                x[r | JR] = sw ? p : q;
            }
        }
    } else if constexpr (J >= 64) {  // partner in another wave: through LDS
#pragma unroll
        for (int r = 0; r < NR; ++r) xbuf[r * BLOCK + tid] = x[r];
        __syncthreads();
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const uint64_t o = xbuf[r * BLOCK + (tid ^ J)];
            const int i = r * BLOCK + tid;
            const bool keep_min = ((i & J) == 0) == ((i & K) == 0);
            x[r] = keep_min ? (x[r] < o ? x[r] : o) : (x[r] > o ? x[r] : o);
        }
        __syncthreads();
    } else {  // partner in the same wave
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const uint64_t o = xlane64<J>(x[r]);
            const int i = r * BLOCK + tid;
            const bool keep_min = ((i & J) == 0) == ((i & K) == 0);
            x[r] = keep_min ? (x[r] < o ? x[r] : o) : (x[r] > o ? x[r] : o);
        }
    }
}

template <int BLOCK, int NR, int K, int J>
__device__ __forceinline__ void bitonic_stages_j(uint64_t (&x)[NR], uint64_t* xbuf) {
    if constexpr (J > 0) {
        bitonic_stage<BLOCK, NR, K, J>(x, xbuf);
        bitonic_stages_j<BLOCK, NR, K, J / 2>(x, xbuf);
    }
}
template <int BLOCK, int NR, int K, int N>
__device__ __forceinline__ void bitonic_stages_k(uint64_t (&x)[NR], uint64_t* xbuf) {
    if constexpr (K <= N) {
        bitonic_stages_j<BLOCK, NR, K, K / 2>(x, xbuf);
        bitonic_stages_k<BLOCK, NR, K * 2, N>(x, xbuf);
    }
}

// Ascending bitonic sort of the first N positions (N a power of two, at
// least 64, at most NR*BLOCK; positions >= N hold the maximum key and stay
// put), fully unrolled: the network is fixed at compile time.
template <int BLOCK, int NR, int N>
__device__ __forceinline__ void sort_static(uint64_t (&x)[NR], uint64_t* xbuf) {
    bitonic_stages_k<BLOCK, NR, 2, N>(x, xbuf);
}

// Sort dispatch for a register list of NR rows holding n2 positions
// (n2 = max(64, pow2ceil(survivors)), the same in every lane).  A 64-key
// network runs on wave 0 alone.
template <int BLOCK, int NR>
__device__ __forceinline__ void sort_list(uint64_t (&x)[NR], int n2, uint64_t* xbuf) {
    const int wid = threadIdx.x >> 6;
    if constexpr (NR == 1) {
        if (n2 == 64) {
            if (wid == 0) sort_static<BLOCK, 1, 64>(x, xbuf);
        } else if (n2 == 128) {
            sort_static<BLOCK, 1, 128>(x, xbuf);
        } else if (n2 == 256) {
            sort_static<BLOCK, 1, 256>(x, xbuf);
        } else if constexpr (BLOCK >= 1024) {
            if (n2 == 512) sort_static<BLOCK, 1, 512>(x, xbuf);
            else sort_static<BLOCK, 1, 1024>(x, xbuf);
        }
    } else {
        sort_static<BLOCK, NR, NR * BLOCK>(x, xbuf);
    }
}

// Counting sort of the register list (positions r*BLOCK + tid, n keys, the
// rest ~0) into ascending key order (descending score, ascending id).
// bin(v) = min(NB-1, int((v - blo) * scale)) is non-decreasing in v, so keys
// order first by descending bin; a key's place inside its bin is the number of
// smaller keys in the bin.  Every score must lie in [blo, hi].  Returns false,
// with the list untouched, when the bins cannot be formed or one bin holds more
// than kSortBinMax keys; the caller then sorts with the bitonic network.
// LDS: start offsets u32[NB + 4], then the keys u64[n].
template <int BLOCK, int NR>
__device__ __forceinline__ bool bin_sort(uint64_t (&x)[NR], int n, float blo, float hi,
                                         uint8_t* region, Shared& sh, int& ph) {
    constexpr int NB = kSortBins;
    constexpr int BPT = NB / BLOCK;  // bins per lane in the scan
    const int tid = threadIdx.x;
    uint32_t* start = reinterpret_cast<uint32_t*>(region);
    uint64_t* tmp = reinterpret_cast<uint64_t*>(region + (NB + 4) * 4);
    const float range = __fsub_rn(hi, blo);
    const float scale = __fdiv_rn((float)NB, range);
    if (!(range > 0.0f) || !(scale < kPosInf)) return false;
    for (int b = tid; b < NB + 4; b += BLOCK) start[b] = 0u;
    __syncthreads();
    int rb[NR], slot[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        if (r * BLOCK + tid < n) {
            const float v = desc_key_value(x[r]);
            const int b = min(NB - 1, (int)__fmul_rn(__fsub_rn(v, blo), scale));
            rb[r] = NB - 1 - b;  // ascending rb = descending score
            slot[r] = (int)atomicAdd(&start[rb[r]], 1u);
        }
    }
    __syncthreads();
    uint32_t c[BPT];
    int local = 0;
    uint32_t big = 0;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
        c[q] = start[tid * BPT + q];
        local += (int)c[q];
        big = max(big, c[q]);
    }
    int total;
    int base = block_excl_scan<BLOCK>(local, sh, total, ph);
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
        start[tid * BPT + q] = (uint32_t)base;
        base += (int)c[q];
    }
    if (tid == 0) start[NB] = (uint32_t)n;
    if (__syncthreads_or(big > (uint32_t)kSortBinMax)) return false;
#pragma unroll
    for (int r = 0; r < NR; ++r)
        if (r * BLOCK + tid < n) tmp[start[rb[r]] + slot[r]] = x[r];
    __syncthreads();
    int fin[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        if (r * BLOCK + tid < n) {
            const int s0 = (int)start[rb[r]], s1 = (int)start[rb[r] + 1];
            int rank = 0;
            for (int k = s0; k < s1; ++k) rank += (tmp[k] < x[r]) ? 1 : 0;
            fin[r] = s0 + rank;
        }
    }
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NR; ++r)
        if (r * BLOCK + tid < n) tmp[fin[r]] = x[r];
    __syncthreads();
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int i = r * BLOCK + tid;
        x[r] = (i < n) ? tmp[i] : ~0ull;
    }
    return true;
}

// Counting sort of the survivors' keys ~okey(s) (ascending = descending
// score) from the registers (s[j] != -inf: a survivor, every one in [lo, hi])
// into key32[0, n).  bin(v) = min(NB-1, int((v - lo) * scale)) does not
// decrease with v, so the keys order first by descending bin; bin offsets come
// from a block scan, and a key's place inside its bin is the number of smaller
// keys there plus the equal keys in earlier slots.  Keys carry no ids: equal
// keys are the same score, so every order among them is the sorted order.
// Slots are kept in 8 bits, four to a register, and final places in 16 bits.
// Returns false when the bins cannot be formed or one holds more than
// kKeyBinMax keys (key32 then holds nothing useful); the caller sorts with the
// bitonic network.  LDS: key32[n], start u32[kKeyBins + 4].
template <int BLOCK, int EPT>
__device__ __forceinline__ bool bin_sort_keys(const float (&s)[EPT], int n, float lo, float hi,
                                              uint32_t* key32, uint32_t* start, Shared& sh,
                                              int& ph) {
    constexpr int NB = kKeyBins;
    constexpr int BPT = NB / BLOCK;  // bins per lane in the scan
    const int tid = threadIdx.x;
    const float range = __fsub_rn(hi, lo);
    const float scale = __fdiv_rn((float)NB, range);
    if (!(range > 0.0f) || !(scale < kPosInf)) return false;
    auto rbin = [&](float v) {  // ascending rb = descending score
        return NB - 1 - min(NB - 1, (int)__fmul_rn(__fsub_rn(v, lo), scale));
    };
    for (int b = tid; b < NB + 4; b += BLOCK) start[b] = 0u;
    __syncthreads();
    uint32_t slot4[(EPT + 3) / 4];
#pragma unroll
    for (int q = 0; q < (EPT + 3) / 4; ++q) slot4[q] = 0u;
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if (s[j] != kNegInf) {
            const uint32_t sl = atomicAdd(&start[rbin(s[j])], 1u);
            slot4[j >> 2] |= min(sl, 255u) << (8 * (j & 3));
        }
    __syncthreads();
    uint32_t c[BPT];
    int local = 0;
    uint32_t big = 0;
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
        c[q] = start[tid * BPT + q];
        local += (int)c[q];
        big = max(big, c[q]);
    }
    int total;
    int base = block_excl_scan<BLOCK>(local, sh, total, ph);
#pragma unroll
    for (int q = 0; q < BPT; ++q) {
        start[tid * BPT + q] = (uint32_t)base;
        base += (int)c[q];
    }
    if (tid == 0) start[NB] = (uint32_t)n;
    if (__syncthreads_or(big > (uint32_t)kKeyBinMax)) return false;
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if (s[j] != kNegInf)
            key32[start[rbin(s[j])] + ((slot4[j >> 2] >> (8 * (j & 3))) & 255u)] = ~okey(s[j]);
    __syncthreads();
    uint32_t fin2[(EPT + 1) / 2];
#pragma unroll
    for (int q = 0; q < (EPT + 1) / 2; ++q) fin2[q] = 0u;
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if (s[j] != kNegInf) {
            const int rb = rbin(s[j]);
            const int s0 = (int)start[rb], s1 = (int)start[rb + 1];
            const int me = s0 + (int)((slot4[j >> 2] >> (8 * (j & 3))) & 255u);
            const uint32_t key = ~okey(s[j]);
            int rank = 0;
            for (int k = s0; k < s1; ++k) {
                const uint32_t v = key32[k];
                rank += (v < key || (v == key && k < me)) ? 1 : 0;
            }
            fin2[j >> 1] |= (uint32_t)(s0 + rank) << (16 * (j & 1));
        }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if (s[j] != kNegInf) key32[(fin2[j >> 1] >> (16 * (j & 1))) & 0xffffu] = ~okey(s[j]);
    __syncthreads();
    return true;
}

// Ascending bitonic sort of keys [0, n2) in LDS (n2 a power of two).
template <int BLOCK>
__device__ __forceinline__ void bitonic_sort_keys(uint32_t* key, int n2) {
    n2 = uni(n2);
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int t = threadIdx.x; t < (n2 >> 1); t += BLOCK) {
                const int i = ((t & ~(j - 1)) << 1) | (t & (j - 1));
                const int p = i + j;
                const bool up = (i & k) == 0;
                const uint32_t ka = key[i], kb = key[p];
                if ((ka > kb) == up) { key[i] = kb; key[p] = ka; }
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------ reference-order sums


template <int CTRL, int RM>
__device__ __forceinline__ int dpp_i(int old, int x) {
    return __builtin_amdgcn_update_dpp(old, x, CTRL, RM, 0xf, false);
}
template <int CTRL, int RM>
__device__ __forceinline__ float dpp_f(float old, float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                                 __builtin_bit_cast(int, x), CTRL,
                                                                 RM, 0xf, false));
}

// Reductions and scans over the wave by DPP: row shifts 1, 2, 4, 8 inside
// rows of 16 lanes, then row broadcasts of lanes 15 and 31.  Lane 63 ends
// with the total (inclusive scans: every lane its prefix).
__device__ __forceinline__ int wave_incl_scan_dpp(int x) {
    x += dpp_i<0x111, 0xf>(0, x);
    x += dpp_i<0x112, 0xf>(0, x);
    x += dpp_i<0x114, 0xf>(0, x);
    x += dpp_i<0x118, 0xf>(0, x);
    x += dpp_i<0x142, 0xa>(0, x);
    x += dpp_i<0x143, 0xc>(0, x);
    return x;
}
__device__ __forceinline__ int wave_excl_scan_i(int v, int& total) {
    const int incl = wave_incl_scan_dpp(v);
    total = __builtin_amdgcn_readlane(incl, 63);
    return incl - v;
}
__device__ __forceinline__ int wave_sum_dpp(int x) {
    return __builtin_amdgcn_readlane(wave_incl_scan_dpp(x), 63);
}
__device__ __forceinline__ float wave_max_dpp(float x) {
    x = fmaxf(x, dpp_f<0x111, 0xf>(kNegInf, x));
    x = fmaxf(x, dpp_f<0x112, 0xf>(kNegInf, x));
    x = fmaxf(x, dpp_f<0x114, 0xf>(kNegInf, x));
    x = fmaxf(x, dpp_f<0x118, 0xf>(kNegInf, x));
    x = fmaxf(x, dpp_f<0x142, 0xa>(kNegInf, x));
    x = fmaxf(x, dpp_f<0x143, 0xc>(kNegInf, x));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}
__device__ __forceinline__ float wave_sum_f_dpp(float x) {
    x += dpp_f<0x111, 0xf>(0.0f, x);
    x += dpp_f<0x112, 0xf>(0.0f, x);
    x += dpp_f<0x114, 0xf>(0.0f, x);
    x += dpp_f<0x118, 0xf>(0.0f, x);
    x += dpp_f<0x142, 0xa>(0.0f, x);
    x += dpp_f<0x143, 0xc>(0.0f, x);
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}
__device__ __forceinline__ float wave_min_dpp(float x) {
    x = fminf(x, dpp_f<0x111, 0xf>(kPosInf, x));
    x = fminf(x, dpp_f<0x112, 0xf>(kPosInf, x));
    x = fminf(x, dpp_f<0x114, 0xf>(kPosInf, x));
    x = fminf(x, dpp_f<0x118, 0xf>(kPosInf, x));
    x = fminf(x, dpp_f<0x142, 0xa>(kPosInf, x));
    x = fminf(x, dpp_f<0x143, 0xc>(kPosInf, x));
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), 63));
}
__device__ __forceinline__ int wave_min_i_dpp(int x) {
    x = min(x, dpp_i<0x111, 0xf>(0x7fffffff, x));
    x = min(x, dpp_i<0x112, 0xf>(0x7fffffff, x));
    x = min(x, dpp_i<0x114, 0xf>(0x7fffffff, x));
    x = min(x, dpp_i<0x118, 0xf>(0x7fffffff, x));
    x = min(x, dpp_i<0x142, 0xa>(0x7fffffff, x));
    x = min(x, dpp_i<0x143, 0xc>(0x7fffffff, x));
    return __builtin_amdgcn_readlane(x, 63);
}

template <int CTRL, int RM>
__device__ __forceinline__ double dpp_d(double x) {
    const uint64_t b = __builtin_bit_cast(uint64_t, x);
    const uint32_t lo = (uint32_t)dpp_i<CTRL, RM>(0, (int)(uint32_t)b);
    const uint32_t hi = (uint32_t)dpp_i<CTRL, RM>(0, (int)(uint32_t)(b >> 32));
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}
// Inclusive scan of doubles over the wave (lanes without a source add +0).
__device__ __forceinline__ double wave_incl_scan_f64_dpp(double x) {
    x = __dadd_rn(x, dpp_d<0x111, 0xf>(x));
    x = __dadd_rn(x, dpp_d<0x112, 0xf>(x));
    x = __dadd_rn(x, dpp_d<0x114, 0xf>(x));
    x = __dadd_rn(x, dpp_d<0x118, 0xf>(x));
    x = __dadd_rn(x, dpp_d<0x142, 0xa>(x));
    x = __dadd_rn(x, dpp_d<0x143, 0xc>(x));
    return x;
}

__device__ __forceinline__ double readlane_f64(double v, int l) {
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)b, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(b >> 32), l);
    return __builtin_bit_cast(double, ((uint64_t)hi << 32) | lo);
}

// The binary32 running sum acc0 + t_0 + t_1 + ... in order, where lane l holds
// terms l*C .. l*C + C - 1 in t[0, C) (zeros past the last term), by sweeps
// of the wave: a sweep adds each lane's terms, one after the other, to the
// sum carried in from the lane below (a wave_shr:1 DPP operand; lane 0 starts
// from acc0), so after sweep s the sums of lanes 0..s are final.  These are the
// reference's adds in the reference's order (NaN and infinities included);
// a sweep costs C + 1 instructions.  nl: lanes holding terms (1..64).
// Returns the final sum of lane nl - 1.  With THR, stops once a lane's final
// sum reaches thr: `hit` is then the first term index whose running sum is
// >= thr (otherwise -1).
template <int C, bool THR, int CM, bool ACC = false>
__device__ __forceinline__ float chain_sweeps(const float (&t)[CM], int nl, float thr, int& hit,
                                             float acc0 = 0.0f) {
    static_assert(C <= CM, "terms per lane");
    const int lane = threadIdx.x & 63;
    hit = -1;
    float s = 0.0f;
    for (int sw = 0; sw < nl; ++sw) {
        float in = __builtin_bit_cast(
            float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, s), 0x138, 0xf, 0xf, true));
        if constexpr (ACC) in = lane == 0 ? acc0 : in;  // else lane 0 reads 0 (bound_ctrl)
        float acc = __fadd_rn(in, t[0]);
#pragma unroll
        for (int k = 1; k < C; ++k) acc = __fadd_rn(acc, t[k]);
        s = acc;
        if (THR && ((__ballot(s >= thr) >> sw) & 1ull)) {
            // lane sw holds the first crossing: walk its terms from its start
            float w = in;
            int first = C;
#pragma unroll
            for (int k = 0; k < C; ++k) {
                w = __fadd_rn(w, t[k]);
                first = (first == C && w >= thr) ? k : first;
            }
            hit = sw * C + __builtin_amdgcn_readlane(first, sw);
            return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), sw));
        }
    }
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s), nl - 1));
}

// The same sum 0 + t_0 + t_1 + ... (finite terms >= 0, t_0 > 0) with fewer
// dependent steps, for long lanes.  While the running sum P = N*u stays in
// one binade [2^b, 2^(b+1)) (u = 2^(b-23), N an integer), each add moves N by
// an amount that depends on the term and on N's parity only (round to nearest
// even).  A lane's whole run of terms is therefore a two-entry table
// (increment from an even N, from an odd N), read off two real float chains
// started at 2^b and 2^b + u; tables compose, so one DPP scan gives every
// lane's exact starting N.  The first lane whose run leaves the binade then
// adds its terms from that exact start as the reference does (any number of
// binade changes inside), and the next round starts after it.  Lane 0 begins
// from 0 directly.  Exactly the reference's adds' results.
template <int C, int CM>
__device__ __forceinline__ float chain_segments(const float (&t)[CM], int nl, float acc0 = 0.0f) {
    static_assert(C <= CM, "terms per lane");
    const int lane = threadIdx.x & 63;
    constexpr int kSat = 1 << 24;
    float a = acc0;
#pragma unroll
    for (int k = 0; k < C; ++k) a = __fadd_rn(a, t[k]);
    float P = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 0));
    int lstart = 1;
    while (lstart < nl) {
        if (!(P >= 0x1p-100f)) {  // tiny sums (not seen for softmax terms): one add each
            int unused;
            return chain_sweeps<C, false, CM, true>(t, nl, 0.0f, unused, acc0);
        }
        const uint32_t pb = __builtin_bit_cast(uint32_t, P);
        const uint32_t bb = pb & 0x7f800000u;  // bits of 2^b
        const float base = __builtin_bit_cast(float, bb);
        const float lim = __builtin_bit_cast(float, bb + 0x00800000u);  // 2^(b+1)
        const int N0 = (int)((pb & 0x7fffffu) | 0x800000u);            // P / u
        const int p0 = N0 & 1;
        float A0 = base, A1 = __builtin_bit_cast(float, bb + 1u);  // N = 2^23, 2^23 + 1
#pragma unroll
        for (int k = 0; k < C; ++k) {
            A0 = __fadd_rn(A0, t[k]);
            A1 = __fadd_rn(A1, t[k]);
        }
        // increments in units of u (same binade: the bit difference), or saturated
        int d0 = A0 < lim ? (int)(__builtin_bit_cast(uint32_t, A0) - bb) : kSat;
        int d1 = A1 < lim ? (int)(__builtin_bit_cast(uint32_t, A1) - bb) - 1 : kSat;
        d0 = lane < lstart ? 0 : d0;  // lanes already summed: identity
        d1 = lane < lstart ? 0 : d1;
        // inclusive scan; composing an earlier table a with this lane's:
        // from an even start the parity after a is a0 & 1, from an odd one
        // (1 + a1) & 1
        auto step = [&](int a0, int a1) {
            const int n0 = a0 + ((a0 & 1) ? d1 : d0);
            const int n1 = a1 + ((a1 & 1) ? d0 : d1);
            d0 = n0;
            d1 = n1;
        };
        step(dpp_i<0x111, 0xf>(0, d0), dpp_i<0x111, 0xf>(0, d1));  // row_shr:1
        step(dpp_i<0x112, 0xf>(0, d0), dpp_i<0x112, 0xf>(0, d1));  // row_shr:2
        step(dpp_i<0x114, 0xf>(0, d0), dpp_i<0x114, 0xf>(0, d1));  // row_shr:4
        step(dpp_i<0x118, 0xf>(0, d0), dpp_i<0x118, 0xf>(0, d1));  // row_shr:8
        step(dpp_i<0x142, 0xa>(0, d0), dpp_i<0x142, 0xa>(0, d1));  // row_bcast:15
        step(dpp_i<0x143, 0xc>(0, d0), dpp_i<0x143, 0xc>(0, d1));  // row_bcast:31
        const int x0 = dpp_i<0x138, 0xf>(0, d0), x1 = dpp_i<0x138, 0xf>(0, d1);  // exclusive
        const int din = p0 ? x1 : x0, dout = p0 ? d1 : d0;
        const uint64_t reach = __ballot(N0 + dout >= (1 << 24));
        if (reach == 0) {
            // no lane leaves the binade: the total is N0 + the last increment
            return __builtin_bit_cast(float, pb + (uint32_t)__builtin_amdgcn_readlane(dout, 63));
        }
        const int L = (int)__builtin_ctzll(reach);
        float w = __builtin_bit_cast(float, pb + (uint32_t)din);  // lane's exact start
#pragma unroll
        for (int k = 0; k < C; ++k) w = __fadd_rn(w, t[k]);
        P = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), L));
        lstart = L + 1;
    }
    return P;
}

// chain_segments with a threshold: the running sum acc0 + t_0 + t_1 + ... of
// finite terms >= 0 (lane l holding terms l*C .. l*C + C - 1, nl lanes) and,
// with THR, `hit`: the first term index of this layout whose running sum is
// >= thr, else -1 (the value returned is then the full sum, otherwise
// meaningless).  In every round each lane whose exact start is known -- the
// lanes of the current binade up to and including the one that leaves it --
// walks its own terms from that start with the reference's adds, so the
// first lane reaching thr is found in the same pass as the sum.
template <int C, bool THR, int CM>
__device__ __forceinline__ float chain_segments_x(const float (&t)[CM], int nl, float acc0, float thr,
                                                  int& hit) {
    static_assert(C <= CM, "terms per lane");
    const int lane = threadIdx.x & 63;
    hit = -1;
    float a = acc0;
    int fa = C;
#pragma unroll
    for (int k = 0; k < C; ++k) {
        a = __fadd_rn(a, t[k]);
        if constexpr (THR) fa = (fa == C && a >= thr) ? k : fa;
    }
    if constexpr (THR) {
        const int f0 = __builtin_amdgcn_readlane(fa, 0);
        if (f0 < C) {
            hit = f0;
            return acc0;
        }
    }
    float P = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, a), 0));
    int lstart = 1;
    while (lstart < nl) {
        if (!(P >= 0x1p-100f))  // tiny sums: one add each, from the start
            return chain_sweeps<C, THR, CM, true>(t, nl, thr, hit, acc0);
        const uint32_t pb = __builtin_bit_cast(uint32_t, P);
        const uint32_t bb = pb & 0x7f800000u;  // bits of 2^b
        const float base = __builtin_bit_cast(float, bb);
        const float lim = __builtin_bit_cast(float, bb + 0x00800000u);  // 2^(b+1)
        const int N0 = (int)((pb & 0x7fffffu) | 0x800000u);            // P / u
        const int p0 = N0 & 1;
        float A0 = base, A1 = __builtin_bit_cast(float, bb + 1u);  // N = 2^23, 2^23 + 1
#pragma unroll
        for (int k = 0; k < C; ++k) {
            A0 = __fadd_rn(A0, t[k]);
            A1 = __fadd_rn(A1, t[k]);
        }
        int d0 = A0 < lim ? (int)(__builtin_bit_cast(uint32_t, A0) - bb) : (1 << 24);
        int d1 = A1 < lim ? (int)(__builtin_bit_cast(uint32_t, A1) - bb) - 1 : (1 << 24);
        d0 = lane < lstart ? 0 : d0;
        d1 = lane < lstart ? 0 : d1;
        auto step = [&](int a0, int a1) {
            const int n0 = a0 + ((a0 & 1) ? d1 : d0);
            const int n1 = a1 + ((a1 & 1) ? d0 : d1);
            d0 = n0;
            d1 = n1;
        };
        step(dpp_i<0x111, 0xf>(0, d0), dpp_i<0x111, 0xf>(0, d1));  // row_shr:1
        step(dpp_i<0x112, 0xf>(0, d0), dpp_i<0x112, 0xf>(0, d1));  // row_shr:2
        step(dpp_i<0x114, 0xf>(0, d0), dpp_i<0x114, 0xf>(0, d1));  // row_shr:4
        step(dpp_i<0x118, 0xf>(0, d0), dpp_i<0x118, 0xf>(0, d1));  // row_shr:8
        step(dpp_i<0x142, 0xa>(0, d0), dpp_i<0x142, 0xa>(0, d1));  // row_bcast:15
        step(dpp_i<0x143, 0xc>(0, d0), dpp_i<0x143, 0xc>(0, d1));  // row_bcast:31
        const int x0 = dpp_i<0x138, 0xf>(0, d0), x1 = dpp_i<0x138, 0xf>(0, d1);  // exclusive
        const int din = p0 ? x1 : x0, dout = p0 ? d1 : d0;
        const uint64_t reach = __ballot(N0 + dout >= (1 << 24));
        const int L = reach ? (int)__builtin_ctzll(reach) : 64;
        // lanes lstart..min(L, nl - 1) start exactly at P + din units
        float w = __builtin_bit_cast(float, pb + (uint32_t)din);
        int fw = C;
#pragma unroll
        for (int k = 0; k < C; ++k) {
            w = __fadd_rn(w, t[k]);
            if constexpr (THR) fw = (fw == C && w >= thr) ? k : fw;
        }
        if constexpr (THR) {
            const uint64_t hm = __ballot(lane >= lstart && lane <= L && lane < nl && fw < C);
            if (hm) {
                const int l = (int)__builtin_ctzll(hm);
                hit = l * C + __builtin_amdgcn_readlane(fw, l);
                return P;
            }
        }
        if (reach == 0)  // every remaining lane ends inside the binade
            return __builtin_bit_cast(float, pb + (uint32_t)__builtin_amdgcn_readlane(dout, 63));
        P = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, w), L));
        lstart = L + 1;
    }
    return P;
}

// The running sum acc + term(0) + ... + term(n-1) (binary32, index order) by
// one wave, in chunks of 64*C terms (lane l: terms l*C .. l*C + C - 1 of a
// chunk; odd C reads distinct LDS banks), and with THR the first index whose
// running sum is >= thr (`hit`, else -1).  finite: every term finite and >= 0
// and acc finite -- binade segments for C >= 5 or more than 8 lanes of terms
// (a sweep chain is one dependent add and lane shift per lane, the segments a
// few scans whatever the length), sweeps otherwise (and for non-finite
// terms, exact for NaN and infinities too).  DESC: the terms do
// not increase, so once fl(acc + term(base)) == acc at a chunk's start every
// later add leaves acc unchanged (rounding is monotone) and the rest of the
// sum is skipped; no threshold is crossed after that point either.  The test
// uses 2*term(base), so that a later term up to twice as large (an exp or a
// quotient of a slightly smaller score, off by an ulp) is covered too.
template <int C, bool THR, bool DESC, class Term>
__device__ __forceinline__ float wave_run(Term&& term, int n, float acc, float thr, int& hit,
                                          bool finite) {
    const int lane = threadIdx.x & 63;
    hit = -1;
    for (int base = 0; base < n; base += 64 * C) {
        if (DESC && finite) {
            const float t0 = unif(term(base));
            if (__fadd_rn(acc, __fmul_rn(2.0f, t0)) == acc) return acc;
        }
        float t[C];
#pragma unroll
        for (int q = 0; q < C; ++q) {
            const int i = base + lane * C + q;
            t[q] = i < n ? term(i) : 0.0f;
        }
        const int nl = min(64, (n - base + C - 1) / C);
        int h = -1;
        float end;
        if ((C >= 5 || nl > 8) && finite) end = chain_segments_x<C, THR>(t, nl, acc, thr, h);
        else end = chain_sweeps<C, THR, C, true>(t, nl, thr, h, acc);
        if (THR && h >= 0) {
            hit = base + h;
            return end;
        }
        acc = end;
    }
    return acc;
}

// wave_run with C picked from n (at most NMAX): 1, 5, 17 or 33 terms per lane.
template <int NMAX, bool THR, bool DESC, class Term>
__device__ __forceinline__ float wave_run_sum(Term&& term, int n, float acc, float thr, int& hit,
                                              bool finite) {
    n = uni(n);
    if (NMAX <= 64 || n <= 64) return wave_run<1, THR, DESC>(term, n, acc, thr, hit, finite);
    if constexpr (NMAX > 64) {
        if (NMAX <= 320 || n <= 320) return wave_run<5, THR, DESC>(term, n, acc, thr, hit, finite);
        if constexpr (NMAX > 320) {
            if (NMAX <= 1088 || n <= 1088)
                return wave_run<17, THR, DESC>(term, n, acc, thr, hit, finite);
            if constexpr (NMAX > 1088) return wave_run<33, THR, DESC>(term, n, acc, thr, hit, finite);
        }
    }
    return acc;  // not reached
}

// Largest per-lane run (64*C terms per chunk) the one-wave sums and draws of
// a BLOCK-lane kernel are compiled for: 1024-lane kernels (128 registers per
// lane) stop at 17 terms per lane and take longer lists in more chunks.
template <int BLOCK>
constexpr int run_bound(int n) {
    return BLOCK >= 1024 && n > 1088 ? 1088 : n;
}

// The top-p cutoff without forming the q's, when it is certain: the first
// index i whose running sum cum_i = q_0 + ... + q_i (q_j = fl(e_j / psum),
// binary32 adds in order) is >= top_p, for sorted finite terms e_j >= 0 and
// the exact binary32 psum.  With Y_i = (e_0 + ... + e_i) / psum in binary64,
// |cum_i - Y_i| <= i half-ulps of cum_i (one rounding per add) + 2^-24 Y_i
// (the rounding of each q_j); each lane bounds this for its run of C terms by
// its last index and the binade of its last Y (raised by 2^-12), doubled on
// the second term, plus 1e-12 for the binary64 arithmetic.  Where Y -/+ that
// bound puts the first crossing at one index the answer is certain (`last`,
// n - 1 when the sum never reaches top_p); otherwise returns false and the
// caller sums the q's, of which the first `upto` hold the crossing (the sum
// of the first upto q's is certainly >= top_p; n when no index is certain).
// One wave, chunks of 64*C terms.
template <int C, class Term>
__device__ __forceinline__ bool certified_cut_c(Term&& term, int n, float psum, float top_p,
                                                int& last, int& upto) {
    const int lane = threadIdx.x & 63;
    const double p = (double)top_p;
    const double inv = __ddiv_rn(1.0, (double)psum);
    double xb = 0.0;  // the terms before the chunk
    for (int base = 0; base < n; base += 64 * C) {
        float ev[C];
#pragma unroll
        for (int q = 0; q < C; ++q) {
            const int i = base + lane * C + q;
            ev[q] = i < n ? term(i) : 0.0f;
        }
        double part = 0.0;
#pragma unroll
        for (int q = 0; q < C; ++q) part = __dadd_rn(part, (double)ev[q]);
        const double incl = wave_incl_scan_f64_dpp(part);
        const double x0 = __dadd_rn(xb, __dsub_rn(incl, part));
        const double yl = __dmul_rn(__dadd_rn(x0, part), inv);
        const double cm = __dmul_rn(yl, 1.0 + 0x1p-12);
        const int b = __builtin_amdgcn_frexp_exp(cm) - 1;  // cm in [2^b, 2^(b+1))
        const double err = __dadd_rn(
            __dadd_rn(__dmul_rn((double)(base + lane * C + C - 1), ldexp(1.0, max(b, -126) - 24)),
                      __dmul_rn(yl, 0x1p-23)),
            1e-12);
        const double lo_thr = __dsub_rn(p, err), hi_thr = __dadd_rn(p, err);
        // y does not decrease: the first index meeting a bound is the count
        // of the lane's terms before it
        int n_hi = 0, n_lo = 0;
        double x = x0;
#pragma unroll
        for (int q = 0; q < C; ++q) {
            x = __dadd_rn(x, (double)ev[q]);
            const double y = __dmul_rn(x, inv);
            n_hi += y < lo_thr ? 1 : 0;
            n_lo += y < hi_thr ? 1 : 0;
        }
        const int c_hi = min(wave_min_i_dpp(n_hi < C ? base + lane * C + n_hi : 0x7fffffff), n);
        const int c_lo = min(wave_min_i_dpp(n_lo < C ? base + lane * C + n_lo : 0x7fffffff), n);
        if (c_hi < n) {  // the earliest possible crossing is here
            if (c_lo != c_hi) {
                upto = c_lo < n ? c_lo + 1 : n;
                return false;
            }
            last = c_hi;
            return true;
        }
        xb = __dadd_rn(xb, readlane_f64(incl, 63));
    }
    last = n - 1;  // Y stays below top_p - err: the sum never reaches top_p
    return true;
}

// certified_cut_c with C picked from n (at most NMAX): 1, 5, 17 or 33.
template <int NMAX, class Term>
__device__ __forceinline__ bool certified_cut(Term&& term, int n, float psum, float top_p,
                                              int& last, int& upto) {
    n = uni(n);
    upto = n;
    if (NMAX <= 64 || n <= 64) return certified_cut_c<1>(term, n, psum, top_p, last, upto);
    if constexpr (NMAX > 64) {
        if (NMAX <= 320 || n <= 320) return certified_cut_c<5>(term, n, psum, top_p, last, upto);
        if constexpr (NMAX > 320) {
            if (NMAX <= 1088 || n <= 1088) return certified_cut_c<17>(term, n, psum, top_p, last, upto);
            if constexpr (NMAX > 1088) return certified_cut_c<33>(term, n, psum, top_p, last, upto);
        }
    }
    return false;  // not reached
}

// acc + v[0] + ... + v[n-1] in index order, binary32, by one wave, in chunks
// of 64 x 17 terms (lane l holding terms l*17 .. l*17 + 16 of a chunk: odd
// strides, distinct banks).  finite: every term finite and >= 0 and acc
// finite, so the binade segments apply (chain_segments); otherwise sweeps,
// exact for NaN and infinities too.
// The terms come from term(i) (a load, or a value formed on the spot).
constexpr int kChainC = 17;
template <class Term>
__device__ __forceinline__ float wave_chain_sum_of(Term&& term, int n, float acc,
                                                   bool finite = true) {
    const int lane = threadIdx.x & 63;
    n = uni(n);
    for (int base = 0; base < n; base += 64 * kChainC) {
        float t[kChainC];
#pragma unroll
        for (int q = 0; q < kChainC; ++q) {
            const int i = base + lane * kChainC + q;
            t[q] = i < n ? term(i) : 0.0f;
        }
        const int nl = min(64, (n - base + kChainC - 1) / kChainC);
        if (finite) {
            acc = chain_segments<kChainC>(t, nl, acc);
        } else {
            int unused;
            acc = chain_sweeps<kChainC, false, kChainC, true>(t, nl, 0.0f, unused, acc);
        }
    }
    return acc;
}

__device__ __forceinline__ float wave_chain_sum(const float* v, int n, float acc, bool finite = true) {
    return wave_chain_sum_of([&](int i) { return v[i]; }, n, acc, finite);
}

// First i with (0 + v[0] + ... + v[i]) >= thr (binary32, index order), or
// n-1 when the running sum never reaches thr.  One wave.  Terms are
// non-negative, so the running sum never decreases: a chunk is searched only
// when its end value reaches thr.  The terms come from term(i).
template <class Term>
__device__ __forceinline__ int wave_chain_cross_of(Term&& term, int n, float thr,
                                                   bool finite = true) {
    const int lane = threadIdx.x & 63;
    n = uni(n);
    float acc = 0.0f;
    for (int base = 0; base < n; base += 64 * kChainC) {
        float t[kChainC];
#pragma unroll
        for (int q = 0; q < kChainC; ++q) {
            const int i = base + lane * kChainC + q;
            t[q] = i < n ? term(i) : 0.0f;
        }
        const int nl = min(64, (n - base + kChainC - 1) / kChainC);
        int hit = -1;
        float end;
        if (finite) {
            end = chain_segments<kChainC>(t, nl, acc);
        } else {
            int unused;
            end = chain_sweeps<kChainC, false, kChainC, true>(t, nl, 0.0f, unused, acc);
        }
        if (end >= thr) {
            (void)chain_sweeps<kChainC, true, kChainC, true>(t, nl, thr, hit, acc);
            if (hit >= 0) return base + hit;
        }
        acc = end;
    }
    return n - 1;
}
__device__ __forceinline__ int wave_chain_cross(const float* v, int n, float thr, bool finite = true) {
    return wave_chain_cross_of([&](int i) { return v[i]; }, n, thr, finite);
}

// --------------------------------------------------------------- bitmaps

__device__ __forceinline__ int pow2ceil(int n) {
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}

__device__ __forceinline__ bool bit_of(const uint32_t* words, int i) {
    return (words[i >> 5] >> (i & 31)) & 1u;
}

__device__ __forceinline__ int rank_of(const uint32_t* keptw, const uint32_t* woff, int i) {
    const uint32_t wb = keptw[i >> 5];
    return (int)woff[i >> 5] + __popc(wb & ((1u << (i & 31)) - 1u));
}


// Exclusive prefix counts of the kept bitmap's words; returns the count.
template <int BLOCK>
__device__ __forceinline__ int bitmap_offsets(const uint32_t* keptw, uint32_t* woff, int W, Shared& sh,
                                              int& ph) {
    constexpr int WPT = (kMaxVocab / 32 + BLOCK - 1) / BLOCK;  // words per lane
    const int tid = threadIdx.x;
    int cnt[WPT];
    int local = 0;
#pragma unroll
    for (int q = 0; q < WPT; ++q) {
        const int w = tid * WPT + q;
        cnt[q] = (w < W) ? __popc(keptw[w]) : 0;
        local += cnt[q];
    }
    int n;
    int base = block_excl_scan<BLOCK>(local, sh, n, ph);
#pragma unroll
    for (int q = 0; q < WPT; ++q) {
        const int w = tid * WPT + q;
        if (w < W) woff[w] = (uint32_t)base;
        base += cnt[q];
    }
    __syncthreads();
    return n;
}

// ------------------------------------------------ std::sort order of a tie
//
// The wavefront form of stdsort_tied_order (cbx_stdsort.h): the ids of the
// elements of rank kT in the order the reference's std::sort leaves them.
// Each partition is one pass counting the right stops and two passes over
// the range in 64-element chunks, where ballots give every element its
// left-stop and right-stop ranks, so a partition of m elements costs about
// 3m/64 steps instead of m dependent steps on one lane.

// LDS writes made visible to the wavefront's later reads.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int mbcnt64(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// __unguarded_partition_pivot of [f, l) (l - f > 16) over packed words
// (rank << 16 | id) by one wavefront; tmp holds l - f words.  Returns the
// cut and whether [f, cut) and [cut, l) hold an element of rank kT.
__device__ __forceinline__ int wave_partition_counts(uint32_t* w, uint32_t* tmp, int f, int l,
                                                     uint32_t kT, bool& has_lo, bool& has_hi) {
    const int lane = threadIdx.x & 63;
    const int m = l - f, half = (m + 1) / 2;
    if (lane == 0) stdsort_median_to_first(PackedSeq{w}, f, f + 1, f + m / 2, l - 1);
    wave_lds_sync();
    const uint32_t pv = (uint32_t)uni((int)(w[f] >> 16));
    int n_r = 0;  // right stops: !(pv < rank)
    for (int p0 = f + 1; p0 < l; p0 += 64) {
        const int p = p0 + lane;
        n_r += __popcll(__ballot(p < l && !(pv < (w[min(p, l - 1)] >> 16))));
    }
    int lb0 = 0, rb0 = 0, cut = l;
    for (int p0 = f + 1; p0 < l; p0 += 64) {
        const int p = p0 + lane;
        const bool in = p < l;
        const uint32_t x = w[min(p, l - 1)], k = x >> 16;
        const bool is_l = in && !(k < pv), is_r = in && !(pv < k);
        const uint64_t ml = __ballot(is_l), mr = __ballot(is_r);
        const int lb = lb0 + mbcnt64(ml);
        const int ra = n_r - (rb0 + mbcnt64(mr) + (is_r ? 1 : 0));
        int c = 0x7fffffff;
        if (is_l) {
            if (ra > lb) tmp[lb] = x;  // swapped left stop, partner rank lb
            else c = p;                // unswapped left stop
        }
        if (is_r && lb > ra) {         // swapped right stop, partner rank ra
            tmp[half + ra] = x;
            c = p;
        }
        cut = min(cut, wave_min_i(c));
        lb0 += __popcll(ml);
        rb0 += __popcll(mr);
    }
    cut = uni(cut);
    wave_lds_sync();
    bool lo_t = (pv == kT), hi_t = false;  // the pivot stays at f < cut
    lb0 = 0;
    rb0 = 0;
    for (int p0 = f + 1; p0 < l; p0 += 64) {
        const int p = p0 + lane;
        const bool in = p < l;
        const uint32_t x = w[min(p, l - 1)], k = x >> 16;
        const bool is_l = in && !(k < pv), is_r = in && !(pv < k);
        const uint64_t ml = __ballot(is_l), mr = __ballot(is_r);
        const int lb = lb0 + mbcnt64(ml);
        const int ra = n_r - (rb0 + mbcnt64(mr) + (is_r ? 1 : 0));
        uint32_t nx = x;
        if (is_l && ra > lb) nx = tmp[half + lb];
        else if (is_r && lb > ra) nx = tmp[ra];
        if (in) {
            w[p] = nx;
            if ((nx >> 16) == kT) {
                lo_t = lo_t || p < cut;
                hi_t = hi_t || p >= cut;
            }
        }
        lb0 += __popcll(ml);
        rb0 += __popcll(mr);
    }
    has_lo = __ballot(lo_t) != 0;
    has_hi = __ballot(hi_t) != 0;
    wave_lds_sync();
    return cut;
}

// The ids of rank kT, in the reference's std::sort order, written to tied[]
// (which may alias tmp); returns their count.  w[0, n): the survivors as
// (rank << 16 | id) in id order, permuted in place; tmp: n words.  One
// wavefront; the pending ranges live in lanes 0..31 of two registers.
__device__ __forceinline__ int wave_tied_order(uint32_t* w, uint32_t* tmp, int n, uint32_t kT,
                                               uint16_t* tied) {
    const int lane = threadIdx.x & 63;
    int lg = 0;
    while ((n >> (lg + 1)) != 0) ++lg;
    // lane j of st_range / st_depth: stack entry j (range first | last << 16)
    int st_range = lane == 0 ? (int)((uint32_t)n << 16) : 0;
    int st_depth = lane == 0 ? 2 * lg : 0;
    int top = 1;
    while (top > 0) {
        --top;
        const uint32_t rg = (uint32_t)__builtin_amdgcn_readlane(st_range, top);
        const int f = (int)(rg & 0xffffu);
        int l = (int)(rg >> 16);
        int depth = __builtin_amdgcn_readlane(st_depth, top);
        bool has = true;  // ranges are pushed only when they hold rank kT
        while (has && l - f > kStdSortThreshold) {
            if (depth == 0) {  // __partial_sort: rare (adversarial inputs)
                if (lane == 0) stdsort_heap_sort(PackedSeq{w}, f, l);
                wave_lds_sync();
                break;
            }
            --depth;
            bool lo_t, hi_t;
            const int cut = wave_partition_counts(w, tmp, f, l, kT, lo_t, hi_t);
            if (hi_t) {
                st_range = lane == top ? (int)((uint32_t)cut | ((uint32_t)l << 16)) : st_range;
                st_depth = lane == top ? depth : st_depth;
                ++top;
            }
            l = cut;
            has = lo_t;
        }
    }
    // the tied elements in array order
    int m = 0;
    for (int p0 = 0; p0 < n; p0 += 64) {
        const int p = p0 + lane;
        const uint32_t x = p < n ? w[p] : 0u;
        const bool t = p < n && (x >> 16) == kT;
        const uint64_t mt = __ballot(t);
        if (t) tied[m + mbcnt64(mt)] = (uint16_t)(x & 0xffffu);
        m += __popcll(mt);
    }
    wave_lds_sync();
    return m;
}

// ----------------------------------------------------------------- the draw

// The draw by one wave (main.cpp:795-800; random.tcc:2665-2676, :2708-2712):
// the reference builds double weights from the float probabilities in id
// order, divides each by their double sum, takes running partial sums, forces
// the last entry (id V-1) to 1.0 and returns the first id whose cumulative
// value is >= u (ids before the first kept one have cumulative 0: u == 0
// gives id 0).  Here the cumulative values are located on the binary64
// prefix of the unnormalised exp terms F[0, n) (kept ids in id order; lane l
// holds the runs [base + l*C, base + l*C + C), odd C in distinct banks): the
// ratio differs from the reference's value by less than 2^-23 relative
// whatever its float normaliser, so a rank whose neighbouring boundaries are
// more than kDrawMargin (relative) from u is certain.  Returns the rank, or -1
// when it is not certain (the caller replays the reference's arithmetic).
template <int C>
__device__ __forceinline__ int draw_rank_c(const float* F, int n, double u, bool last_kept) {
    const int lane = threadIdx.x & 63;
    const bool one = n <= 64 * C;  // one chunk: the total comes with the prefix
    double total = 0.0;
    if (!one) {
        for (int base = 0; base < n; base += 64 * C) {
            double part = 0.0;
#pragma unroll
            for (int q = 0; q < C; ++q) {
                const int i = base + lane * C + q;
                part = __dadd_rn(part, (double)(i < n ? F[i] : 0.0f));
            }
            total = __dadd_rn(total, readlane_f64(wave_incl_scan_f64_dpp(part), 63));
        }
    }
    double xb = 0.0;
    for (int base = 0; base < n; base += 64 * C) {
        float f[C];
#pragma unroll
        for (int q = 0; q < C; ++q) {
            const int i = base + lane * C + q;
            f[q] = i < n ? F[i] : 0.0f;
        }
        double part = 0.0;
#pragma unroll
        for (int q = 0; q < C; ++q) part = __dadd_rn(part, (double)f[q]);
        const double incl = wave_incl_scan_f64_dpp(part);
        if (one) total = readlane_f64(incl, 63);
        const double target = __dmul_rn(u, total);
        double cp = __dadd_rn(xb, __dsub_rn(incl, part));  // exclusive
        double blo = 0.0, bhi = 0.0;
        int found = 0x7fffffff;
        bool got = false;
#pragma unroll
        for (int q = 0; q < C; ++q) {
            const double before = cp;
            cp = __dadd_rn(cp, (double)f[q]);
            const bool hit = !got && cp >= target && base + lane * C + q < n;
            blo = hit ? before : blo;
            bhi = hit ? cp : bhi;
            found = hit ? base + lane * C + q : found;
            got = got || hit;
        }
        const int rank = wave_min_i_dpp(found);
        if (rank != 0x7fffffff) {
            const int L = __builtin_ctzll(__ballot(found == rank));
            const double inv = __ddiv_rn(1.0, total);
            const double clo = __dmul_rn(readlane_f64(blo, L), inv);
            const double chi = __dmul_rn(readlane_f64(bhi, L), inv);
            const bool lo_ok = rank == 0 || __dsub_rn(u, clo) > kDrawMargin * clo + 1e-30;
            const bool hi_ok = (rank == n - 1 && last_kept) ||
                               __dsub_rn(chi, u) > kDrawMargin * chi + 1e-30;
            return (lo_ok && hi_ok) ? rank : -1;
        }
        xb = __dadd_rn(xb, readlane_f64(incl, 63));
    }
    return -1;
}

// draw_rank_c with C picked from n (at most NMAX): the smallest of the odd
// run lengths 1, 3, 5, 9, 17, 33 whose one chunk holds n (each lane's run is
// a serial chain of binary64 adds, so a row drawing among few ids should not
// walk a long run of zeros).
template <int NMAX>
__device__ __forceinline__ int draw_rank(const float* F, int n, double u, bool last_kept) {
    n = uni(n);
    if (NMAX <= 64 || n <= 64) return draw_rank_c<1>(F, n, u, last_kept);
    if constexpr (NMAX > 64) {
        if (n <= 192) return draw_rank_c<3>(F, n, u, last_kept);
        if (NMAX <= 320 || n <= 320) return draw_rank_c<5>(F, n, u, last_kept);
        if constexpr (NMAX > 320) {
            if (n <= 576) return draw_rank_c<9>(F, n, u, last_kept);
            if (NMAX <= 1088 || n <= 1088) return draw_rank_c<17>(F, n, u, last_kept);
            if constexpr (NMAX > 1088) return draw_rank_c<33>(F, n, u, last_kept);
        }
    }
    return -1;  // not reached
}

// Softmax over the kept entries (val[q], id[q] for bit q of `kept`), then
// greedy or draw with the row's uniform u_draw; writes token, info and, if
// asked, the probability row, and returns the token (in thread 0).
// Shared by both paths.  Every wave takes part in three steps -- the kept
// bitmap and the maximum kept score (each wave's maximum into an LDS
// maximum), then (wave 0) the bitmap's word offsets, then the exp terms F in
// id order -- after which wave 0 alone forms the id-order binary32 sum
// (main.cpp:786-790) and the token, with no workgroup barrier; the other
// waves are done, or wait once for the sum when probabilities are written.
template <int BLOCK, int EPT, int N>
__device__ __forceinline__ int finish_row(float (&val)[N], const int (&id)[N], uint64_t kept,
                           const KernelArgs& a, const cbx_params& P, int64_t rs, double u_draw,
                           uint32_t flags, uint32_t* keptw, uint32_t* woff, float* F,
                           const uint64_t* tab, Shared& sh) {
    constexpr int WMAX = (BLOCK * EPT + 31) / 32;  // bitmap words of the largest vocabulary
    constexpr int WPL = (WMAX + 63) / 64;          // of them per lane of wave 0
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int V = a.n_vocab;
    const int W = (V + 31) >> 5;
    for (int w = tid; w < W; w += BLOCK) keptw[w] = 0u;
    if (tid == 0) sh.mxk = 0u;
    __syncthreads();
    float m = kNegInf;
#pragma unroll
    for (int q = 0; q < N; ++q)
        if ((kept >> q) & 1u) {
            atomicOr(&keptw[id[q] >> 5], 1u << (id[q] & 31));
            m = fmaxf(m, val[q]);
        }
    m = wave_max_dpp(m);
    if (lane == 0) atomicMax(&sh.mxk, okey(m));
    __syncthreads();
    // wave 0: word offsets; each lane keeps its words' counts for id lookups
    int cw[WPL];
    int loc = 0, wbase = 0, n_final = 0;
    int token = 0;
    if (wid == 0) {
#pragma unroll
        for (int q = 0; q < WPL; ++q) {
            const int w = lane * WPL + q;
            cw[q] = (w < W) ? __popc(keptw[w]) : 0;
            loc += cw[q];
        }
        wbase = wave_excl_scan_i(loc, n_final);
        int run = wbase;
#pragma unroll
        for (int q = 0; q < WPL; ++q) {
            const int w = lane * WPL + q;
            if (w < W) woff[w] = (uint32_t)run;
            run += cw[q];
        }
    }
    __syncthreads();
    CBX_STAMP(9);
    // softmax terms (main.cpp:783-785) in id order
    const float mx2 = okey_inv(uni((int)sh.mxk));
#pragma unroll
    for (int q = 0; q < N; ++q)
        if ((kept >> q) & 1u)
            F[rank_of(keptw, woff, id[q])] = expf_libm_branchless(__fsub_rn(val[q], mx2), tab);
    __syncthreads();
    if (wid == 0) {
        // the id of id-order rank `rank` (0 <= rank < n_final): the lane whose
        // words hold it finds the word; lanes 0..31 then count the word's set
        // bits below their own bit
        auto id_of_rank_w = [&](int rank) -> int {
            const int L = __builtin_ctzll(__ballot(wbase <= rank && rank < wbase + loc));
            int run = wbase, wq = 0, kq = 0;
            bool got = false;
#pragma unroll
            for (int q = 0; q < WPL; ++q) {
                const bool in = !got && rank < run + cw[q];
                wq = in ? lane * WPL + q : wq;
                kq = in ? rank - run : kq;
                got = got || in;
                run += cw[q];
            }
            const int w = __builtin_amdgcn_readlane(wq, L);
            const int kb = __builtin_amdgcn_readlane(kq, L);
            const uint32_t bits = keptw[w];
            const bool hit = lane < 32 && ((bits >> (lane & 31)) & 1u) &&
                             (int)__builtin_amdgcn_mbcnt_lo(bits, 0u) == kb;
            return w * 32 + __builtin_ctzll(__ballot(hit));
        };
        // The id-order binary32 sum (main.cpp:786-790) is formed only where it
        // is read: greedy rows, a draw that is not certain, probabilities.
        // A kept row is never empty: the largest kept score's term is
        // expf(0) = 1, or NaN when the row holds NaN or +inf.
        const bool fin = !(flags & CBX_INFO_NONFINITE);
        const bool empty = n_final == 0;
        float psum2 = 0.0f;
        bool have_psum2 = false;
        auto exact_psum2 = [&]() {
            if (!have_psum2) {
                int unused;
                psum2 = wave_run_sum<run_bound<BLOCK>(BLOCK * EPT), false, false>(
                    [&](int i) { return F[i]; }, n_final, 0.0f, 0.0f, unused, fin);
                have_psum2 = true;
            }
            return psum2;
        };
        CBX_STAMP(10);
        if (empty) {
            flags |= CBX_INFO_EMPTY;
        } else if (P.temp <= 0.0f) {
            // first argmax of p_i = e_i / psum over ids (zeros elsewhere);
            // only NaN probabilities: no maximum, id 0
            const float ps = exact_psum2();
            float best = -1.0f;
            int first = 0x7fffffff;
            for (int i = lane; i < n_final; i += 64) {
                const float p = __fdiv_rn(F[i], ps);
                if (p > best) { best = p; first = i; }  // ascending i: keeps the first
            }
            const float b = wave_max_dpp(best);
            const int rk = wave_min_i_dpp(best == b ? first : 0x7fffffff);
            token = rk == 0x7fffffff ? 0 : id_of_rank_w(rk);
            flags |= CBX_INFO_GREEDY;
        } else if (V >= 2) {
            flags |= CBX_INFO_DREW;
            const double u = u_draw;
            const bool last_kept = bit_of(keptw, V - 1);
            int rank = -1;
            if (!(u > 0.0)) {
                token = 0;  // lower_bound of 0 is the first entry
            } else {
                rank = draw_rank<run_bound<BLOCK>(BLOCK * EPT)>(F, n_final, u, last_kept);
                if (rank < 0) {
                    // the reference's arithmetic: float probabilities, double
                    // CDF, on one lane (rare)
                    const float ps = exact_psum2();
                    int rk = -1;
                    if (lane == 0) {
                        double sum = 0.0;
                        for (int r = 0; r < n_final; ++r)
                            sum = __dadd_rn(sum, (double)__fdiv_rn(F[r], ps));
                        double acc = 0.0;
                        for (int r = 0; r < n_final; ++r) {
                            acc = __dadd_rn(acc, __ddiv_rn((double)__fdiv_rn(F[r], ps), sum));
                            const double c = (r == n_final - 1 && last_kept) ? 1.0 : acc;
                            if (c >= u) { rk = r; break; }
                        }
                    }
                    rank = __builtin_amdgcn_readlane(rk, 0);
                    if (rank < 0) token = V - 1;
                }
                if (rank >= 0) token = id_of_rank_w(rank);
            }
            CBX_STAMP(11);
        }
        CBX_STAMP(12);
        const float ps_out = (a.probs && !empty) ? exact_psum2() : 0.0f;
        if (lane == 0) {
            a.tokens[rs] = token;
            if (a.info) a.info[rs] = flags | sh.flags;
            sh.psum = ps_out;
        }
    }
    if (a.probs) {
        __syncthreads();
        const float ps = unif(sh.psum);
        float* prow = a.probs + rs * a.ld_probs;
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int i = j * BLOCK + tid;
            if (i < V)
                prow[i] = (ps != 0.0f && bit_of(keptw, i)) ? __fdiv_rn(F[rank_of(keptw, woff, i)], ps)
                                                          : 0.0f;
        }
    }
    return token;
}

// ------------------------------------------------------------------ kernel

// The rest of a row whose n_surv <= NR*BLOCK survivors sit in the LDS list
// xbuf[0, n_surv) as composite keys: each lane holds positions r*BLOCK + tid.
// Returns the token (in thread 0).
template <int BLOCK, int EPT, int NR>
__device__ __forceinline__ int fast_path(const KernelArgs& a, const cbx_params& P, int64_t rs,
                                          double u_draw, uint32_t flags, int n_surv,
                                          float blo, float bhi,
                                          bool use_topp, bool use_pen, const uint32_t* seen,
                                          uint32_t* keptw, uint32_t* woff, uint8_t* region,
                                          const uint64_t* tab, Shared& sh, int& ph) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    uint64_t* xbuf = reinterpret_cast<uint64_t*>(region);
    float* E = reinterpret_cast<float*>(region);
    float* F = reinterpret_cast<float*>(region);
    const int n2 = uni(max(64, pow2ceil(n_surv)));
    uint64_t x[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        const int i = r * BLOCK + tid;
        x[r] = (i < n_surv) ? xbuf[i] : ~0ull;
    }
    __syncthreads();
    uint64_t kept = 0;  // bit r: list entry r kept
    float mx_surv = kNegInf;
    // ---- top-p (main.cpp:750-772) ----
    if (use_topp) {
        if (!bin_sort<BLOCK, NR>(x, n_surv, blo, bhi, region, sh, ph)) sort_list<BLOCK, NR>(x, n2, xbuf);
        CBX_STAMP(4);
        if (tid == 0) sh.mx = desc_key_value(x[0]);
        __syncthreads();
        mx_surv = unif(sh.mx);
        // E (the bin sort's offsets area) does not overlap the keys still read
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int i = r * BLOCK + tid;
            if (i < n_surv)
                E[i] = expf_libm_branchless(__fsub_rn(desc_key_value(x[r]), mx_surv), tab);
        }
        __syncthreads();
        CBX_STAMP(5);
        if (wid == 0) {
            // psum = 0 + e_0 + e_1 + ... (e_0 = 1), then with q_i = e_i / psum
            // the first i with q_0 + ... + q_i >= top_p.  Rows holding NaN or
            // +inf take the term-by-term chains (the segment scan needs finite
            // terms).  The sorted terms do not increase: the sums stop once
            // the adds are no-ops.
            const bool fin = !(flags & CBX_INFO_NONFINITE);
            auto e_at = [&](int i) { return E[i]; };
            int hit;
            const float psum =
                wave_run_sum<run_bound<BLOCK>(NR * BLOCK), false, true>(e_at, n_surv, 0.0f, 0.0f, hit, fin);
            CBX_STAMP(6);
            int last, upto = n_surv;
            if (!(fin && certified_cut<run_bound<BLOCK>(NR * BLOCK)>(e_at, n_surv, psum, P.top_p, last, upto))) {
                // q_i = e_i / psum formed as the sum reads them: a run's
                // loads and divisions are in flight together.  Only the
                // first upto q's can hold the crossing; the whole list is
                // summed if they do not reach top_p after all.
                auto q_at = [&](int i) { return __fdiv_rn(E[i], psum); };
                (void)wave_run_sum<run_bound<BLOCK>(NR * BLOCK), true, true>(q_at, upto, 0.0f, P.top_p, hit, fin);
                if (hit < 0 && upto < n_surv)
                    (void)wave_run_sum<run_bound<BLOCK>(NR * BLOCK), true, true>(q_at, n_surv, 0.0f, P.top_p, hit, fin);
                last = hit < 0 ? n_surv - 1 : hit;
            }
            if (lane == 0) sh.n_kept = last + 1;
        }
        __syncthreads();
        CBX_STAMP(7);
        const int n_kept = uni(sh.n_kept);
#pragma unroll
        for (int r = 0; r < NR; ++r) {
            const int i = r * BLOCK + tid;
            if (i < n_kept) kept |= (uint64_t)1 << r;
            if (i == n_kept - 1) sh.tie[0] = desc_key_value(x[r]);
            if (i == n_kept && i < n_surv) sh.tie[1] = desc_key_value(x[r]);
        }
        __syncthreads();
        const bool tie = n_kept < n_surv && sh.tie[0] == sh.tie[1];
        if (tid == 0 && tie) sh.flags |= CBX_INFO_TOPP_TIE;
        if (tie && !(flags & CBX_INFO_NONFINITE)) {
            // Equal scores straddle the cutoff.  The survivors become words
            // (rank << 16 | id) in id order -- rank: the first sorted position
            // of the score, found in the sorted scores; position: from a
            // bitmap of the ids -- and wave 0 replays the reference's
            // std::sort over the ranges holding the tied score
            // (wave_tied_order); of the tied ids the first n_kept - kT are kept.
            const float T = sh.tie[0];
            float* vals = reinterpret_cast<float*>(region);
            const int W = (a.n_vocab + 31) >> 5;
#pragma unroll
            for (int r = 0; r < NR; ++r)
                if (r * BLOCK + tid < n_surv) {
                    vals[r * BLOCK + tid] = desc_key_value(x[r]);
                    const uint32_t i = (uint32_t)x[r];
                    atomicOr(&keptw[i >> 5], 1u << (i & 31));
                }
            __syncthreads();
            (void)bitmap_offsets<BLOCK>(keptw, woff, W, sh, ph);
            // first sorted position of v: the count of scores above it
            auto above = [&](float v) {
                int lo = 0, hi = n_surv;
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (vals[mid] > v) lo = mid + 1;
                    else hi = mid;
                }
                return lo;
            };
            const int kT = above(T);
            uint32_t wd[NR];
            int at[NR];
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                at[r] = -1;
                wd[r] = 0u;
                if (r * BLOCK + tid < n_surv) {
                    const uint32_t i = (uint32_t)x[r];
                    wd[r] = ((uint32_t)above(desc_key_value(x[r])) << 16) | i;
                    at[r] = rank_of(keptw, woff, (int)i);
                }
            }
            __syncthreads();  // the scores are read: the storage takes the words
            uint32_t* wv = reinterpret_cast<uint32_t*>(region);
            uint32_t* tmp = wv + n_surv;
#pragma unroll
            for (int r = 0; r < NR; ++r)
                if (at[r] >= 0) wv[at[r]] = wd[r];
            for (int w = tid; w < W; w += BLOCK) keptw[w] = 0u;
            __syncthreads();
            uint16_t* tied = reinterpret_cast<uint16_t*>(tmp);
            if (wid == 0) (void)wave_tied_order(wv, tmp, n_surv, (uint32_t)kT, tied);
            __syncthreads();
            for (int i = tid; i < n_kept - kT; i += BLOCK)
                atomicOr(&keptw[tied[i] >> 5], 1u << (tied[i] & 31));
            __syncthreads();
            kept = 0;
#pragma unroll
            for (int r = 0; r < NR; ++r) {
                const float v = desc_key_value(x[r]);
                if (r * BLOCK + tid < n_surv &&
                    (v > T || (v == T && bit_of(keptw, (int)(uint32_t)x[r]))))
                    kept |= (uint64_t)1 << r;
            }
            __syncthreads();  // finish_row clears the bitmap again
        }
    } else {
#pragma unroll
        for (int r = 0; r < NR; ++r)
            if (r * BLOCK + tid < n_surv) kept |= (uint64_t)1 << r;
    }
    float val[NR];
    int id[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
        val[r] = desc_key_value(x[r]);
        id[r] = (int)(uint32_t)x[r];
    }
    // ---- min-p [extension]: drop expf(s - s_max) < min_p ----
    if (P.min_p > 0.0f) {
        float m = kNegInf;
#pragma unroll
        for (int r = 0; r < NR; ++r) m = ((kept >> r) & 1u) ? fmaxf(m, val[r]) : m;
        const float mx_kept = use_topp ? mx_surv : block_max<BLOCK>(m, sh, ph);
#pragma unroll
        for (int r = 0; r < NR; ++r)
            if (((kept >> r) & 1u) &&
                expf_libm_branchless(__fsub_rn(val[r], mx_kept), tab) < P.min_p)
                kept &= ~((uint64_t)1 << r);
    }
    // ---- repetition penalty (main.cpp:774-781), seen bitmap built at load ----
    if (use_pen) {
#pragma unroll
        for (int r = 0; r < NR; ++r)
            if (((kept >> r) & 1u) && bit_of(seen, id[r]))
                val[r] = val[r] > 0.0f ? __fdiv_rn(val[r], P.repeat_penalty)
                                       : __fmul_rn(val[r], P.repeat_penalty);
    }
    __syncthreads();  // E and xbuf are done with; F takes the region
    CBX_STAMP(8);
    return finish_row<BLOCK, EPT, NR>(val, id, kept, a, P, rs, u_draw, flags, keptw, woff, F, tab,
                                      sh);
}

// MAXNR: the largest register list (rows per lane) compiled in; GENERAL: the
// per-element path for more survivors is compiled in (the launch picks the
// variant from the survivor capacity, so lean variants carry no unused code).
// One workgroup samples row-step g of the launch and returns its token (in
// thread 0; -1 for a row put on the redo list).  DEC: a decode step, whose
// stream state `dec_state` (read by the caller) is checked once the row's
// loads are in flight; an ended stream returns kEndedRow from every thread.
constexpr int kEndedRow = -2;
template <int BLOCK, int EPT, int MAXNR, bool GENERAL, bool DEC = false>
__device__ __forceinline__ int sample_row_wg(const KernelArgs& a, int64_t g, Shared& sh,
                                             uint64_t* tab, uint8_t* smem, int32_t dec_state = 0) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    const int step = (int)(g / a.n_rows), row = (int)(g % a.n_rows);
    const int V = a.n_vocab;
    const int cap = a.cap;
    const int W = (V + 31) >> 5;
    const int Wp = (W + 3) & ~3;

    // LDS: seen[Wp] | keptw[Wp] | woff[Wp] | region, whose use changes:
    //   top-k:        value histogram u32[2048] + candidates f32[512], or the
    //                 radix histogram u32[4096]
    //   fast path:    xbuf u64[2048] (list, cross-wave exchanges), then E f32
    //   general path: key32 u32[cap] (sorted scores), then the key sort's bin
    //                 offsets u32[kKeyBins + 4], after the sort the exp terms
    //                 f32[n_surv] right after the keys when the region holds
    //                 them; for a tie at the top-p cutoff, words u32[n_surv]
    //                 (rank << 16 | id) and their partition scratch in its place
    //   finish:       F f32[n_final]
    uint32_t* seen = reinterpret_cast<uint32_t*>(smem);
    uint32_t* keptw = seen + Wp;
    uint32_t* woff = keptw + Wp;
    uint8_t* region = reinterpret_cast<uint8_t*>(woff + Wp);
    uint32_t* hist = reinterpret_cast<uint32_t*>(region);
    float* cand = reinterpret_cast<float*>(region + kValueBins * 4);
    uint64_t* xbuf = reinterpret_cast<uint64_t*>(region);
    uint32_t* key32 = reinterpret_cast<uint32_t*>(region);
    float* F = reinterpret_cast<float*>(region);

    const cbx_params P = a.params[row];
    const int64_t rs = (int64_t)step * a.n_rows + row;  // row-step linear id
    int ph = 0;  // the block reductions' slot set (block_excl_scan)
    CBX_STAMP(0);

    // ---- load (all loads first), combine, mask, temperature (main.cpp:733-738) ----
    // Buffer loads bounded by a resource of V*4 bytes: one lane offset, the
    // j*BLOCK stride in a scalar offset, ids >= V read 0 (masked below);
    // non-temporal (cache policy nt): each row's logits are read once.
    const float* lrow = a.logits + rs * a.ld_logits;
    const int32_t* hrow = a.history ? a.history + (int64_t)row * a.ld_history : nullptr;
    float s[EPT];
    {
        const __amdgpu_buffer_rsrc_t rl = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(lrow), (short)0, V * 4, kBufferWord3);
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            s[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(
                                                 rl, tid * 4, j * BLOCK * 4, 2));
    }
    // the history's first kHistPre*BLOCK ids, issued right behind the row so
    // that one wait covers both.  They are bounded by the history's row
    // stride, not its length: the length is a load of its own, and waiting
    // for it would put a second memory round trip before these.  Ids past the
    // length are masked below; loads past the stride read 0.
    constexpr int kHistPre = 4;
    int32_t hid[kHistPre];
    const int hpre = a.history ? (int)min(a.ld_history, (int64_t)(kHistPre * BLOCK)) : 0;
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(hrow), (short)0, hpre * 4, kBufferWord3);
    if (a.history) {
#pragma unroll
        for (int q = 0; q < kHistPre; ++q)
            hid[q] = __builtin_amdgcn_raw_buffer_load_b32(rh, tid * 4, q * BLOCK * 4, 0);
    }
    if constexpr (DEC) {
        // an ended stream is not sampled (its row's loads are simply dropped)
        if (dec_state != CBX_DECODE_RUNNING) {
            if (tid == 0) {
                a.tokens[row] = a.stop_token;
                if (a.info) a.info[row] = CBX_INFO_ENDED;
            }
            return kEndedRow;
        }
    }
    // the draw's uniform and the force-stop flag, while the loads are in
    // flight (scalar work and loads: the draw at the row's end need not wait)
    double u_draw = 0.0;
    if (a.draw_mode == CBX_DRAW_PHILOX) {
        const uint64_t sid = a.stream_ids ? a.stream_ids[row] : (uint64_t)row;
        u_draw = philox_uniform(a.seed, sid, a.step0 + (uint64_t)step);
    } else if (a.uniforms) {
        u_draw = a.uniforms[rs];
    }
    u_draw = fresh_d(u_draw);
    const bool fstop = a.force_stop && a.force_stop[rs];
    const int hlen = a.history ? (int)min((int64_t)a.history_len[row], a.ld_history) : 0;
    const bool use_pen = P.repeat_penalty != 1.0f && hlen > 0;
    if (a.uncond) {
        const __amdgpu_buffer_rsrc_t ru = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.uncond + rs * a.ld_logits), (short)0, V * 4, kBufferWord3);
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const float un = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(ru, tid * 4, j * BLOCK * 4, 2));
            s[j] = __fadd_rn(s[j], __fmul_rn(P.cfg_weight, __fsub_rn(s[j], un)));
        }
    }
    if (tid < 32) tab[tid] = kExp2TabDev.t[tid];
    // the allowed row, staged in the region (free until the top-k pass) so
    // the mask pass reads its words from LDS; history ids -> seen bitmap
    const uint32_t* arow = a.allowed ? a.allowed + (int64_t)row * a.ld_allowed : nullptr;
    uint32_t* const mrow = reinterpret_cast<uint32_t*>(region);
    for (int w = tid; w < W; w += BLOCK) {
        keptw[w] = 0u;
        seen[w] = 0u;
        if (arow) mrow[w] = arow[w];
    }
    if (tid == 0) sh.flags = 0u;
    __syncthreads();
    if (use_pen) {
#pragma unroll
        for (int q = 0; q < kHistPre; ++q) {
            const int32_t t = hid[q];
            if (q * BLOCK + tid < hlen && t >= 0 && t < V) atomicOr(&seen[t >> 5], 1u << (t & 31));
        }
        for (int j = kHistPre * BLOCK + tid; j < hlen; j += BLOCK) {
            const int32_t t = hrow[j];
            if (t >= 0 && t < V) atomicOr(&seen[t >> 5], 1u << (t & 31));
        }
    }
    const bool scale = P.temp > 0.0f && P.temp != 1.0f;
    const float inv_t = __fdiv_rn(1.0f, P.temp);
    int nonfinite = 0;
    float lo = kPosInf, hi = kNegInf;
    // element j of this lane is id j*BLOCK + tid: valid for j < n_mine; its
    // allowed bit is bit (tid & 31) of word j*BLOCK/32 + tid/32
    const int n_mine = (V - tid + BLOCK - 1) / BLOCK;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        float v = s[j];
        bool masked = j >= n_mine;
        if (arow) {
            // word j*BLOCK/32 + tid/32 (words past the row: the element is past V)
            const int w = j * (BLOCK / 32) + (tid >> 5);
            const uint32_t word = w < W ? mrow[w] : 0u;
            masked = masked || !((word >> (tid & 31)) & 1u);
        }
        if (fstop) masked = masked || (j * BLOCK + tid) != a.stop_token;
        v = masked ? kNegInf : v;
        if (scale) v = __fmul_rn(v, inv_t);
        nonfinite |= (v != v || v == kPosInf) ? 1 : 0;
        lo = (v != kNegInf) ? fminf(lo, v) : lo;
        hi = (v != kNegInf) ? fmaxf(hi, v) : hi;
        s[j] = v;
    }
    int bad;
    block_minmax<BLOCK>(lo, hi, nonfinite, sh, lo, hi, bad, ph);
    CBX_STAMP(1);
    const uint32_t flags = bad ? CBX_INFO_NONFINITE : 0u;

    // ---- top-k (main.cpp:740-748) ----
    const bool use_topk = P.top_k > 0 && P.top_k < V;
    float sblo = lo;  // every survivor lies in [sblo, hi]
    if (use_topk) {
        float thr;
        int above;
        if (!bad && !(hi > lo)) {
            // every finite score equal (or none): the (k+1)-th largest is that
            // score when more than k are finite, else -inf; none is above it
            int mine_f = 0;
#pragma unroll
            for (int j = 0; j < EPT; ++j) mine_f += (s[j] != kNegInf) ? 1 : 0;
            const int n_fin = block_sum<BLOCK>(mine_f, sh, ph);
            thr = n_fin > P.top_k ? lo : kNegInf;
            above = n_fin > P.top_k ? 0 : n_fin;
        } else if (bad ||
                   !topk_value_bins<BLOCK, EPT>(s, P.top_k, lo, hi, hist, cand, sh, thr, above, ph)) {
            thr = okey_inv(radix_select_desc<BLOCK, EPT>(s, V, P.top_k, hist, sh, ph));
            int n_above = 0;
#pragma unroll
            for (int j = 0; j < EPT; ++j) n_above += (s[j] > thr) ? 1 : 0;
            above = block_sum<BLOCK>(n_above, sh, ph);
        }
        if (above < P.top_k) thr = __fsub_rn(thr, 1e-10f);
        sblo = fmaxf(thr, lo);
#pragma unroll
        for (int j = 0; j < EPT; ++j) s[j] = (s[j] <= thr) ? kNegInf : s[j];
    }

    // ---- survivors (score != -inf): count and compaction offsets ----
    CBX_STAMP(2);
    int mine = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) mine += (s[j] != kNegInf) ? 1 : 0;
    int n_surv;
    int off = block_excl_scan<BLOCK>(mine, sh, n_surv, ph);
    if (n_surv > cap) {
        if (tid == 0) {
            a.tokens[rs] = -1;
            if (a.info) a.info[rs] = flags | CBX_INFO_OVERFLOW;
            if (a.redo) {  // the redo pass samples the row again at full capacity
                const int i = atomicAdd(&a.redo[0], 1);
                if (i < a.redo_max) a.redo[2 + i] = (int32_t)rs;
            }
        }
        if (a.probs) {
            float* prow = a.probs + rs * a.ld_probs;
            for (int i = tid; i < V; i += BLOCK) prow[i] = 0.0f;
        }
        return -1;
    }
    const bool use_topp = P.top_p < 1.0f && n_surv > 0;

    if (n_surv <= MAXNR * BLOCK) {
        // ================= fast path: survivors in a register list =================
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (s[j] != kNegInf) xbuf[off++] = desc_key(s[j], (uint32_t)(j * BLOCK + tid));
        __syncthreads();
        CBX_STAMP(3);
        const int rows_needed = uni((max(64, pow2ceil(n_surv)) + BLOCK - 1) / BLOCK);
        if (rows_needed <= 1) {
            return fast_path<BLOCK, EPT, 1>(a, P, rs, u_draw, flags, n_surv, sblo, hi, use_topp,
                                            use_pen, seen, keptw, woff, region, tab, sh, ph);
        } else if constexpr (MAXNR >= 2) {
            if (rows_needed == 2) {
                return fast_path<BLOCK, EPT, 2>(a, P, rs, u_draw, flags, n_surv, sblo, hi, use_topp,
                                                use_pen, seen, keptw, woff, region, tab, sh, ph);
            } else if constexpr (MAXNR >= 4) {
                if (rows_needed <= 4) {
                    return fast_path<BLOCK, EPT, 4>(a, P, rs, u_draw, flags, n_surv, sblo, hi,
                                                    use_topp, use_pen, seen, keptw, woff, region,
                                                    tab, sh, ph);
                } else if constexpr (MAXNR >= 8) {
                    return fast_path<BLOCK, EPT, 8>(a, P, rs, u_draw, flags, n_surv, sblo, hi,
                                                    use_topp, use_pen, seen, keptw, woff, region,
                                                    tab, sh, ph);
                }
            }
        }
        return -1;  // not reached: rows_needed <= MAXNR
    }
    if constexpr (!GENERAL) {
        return -1;  // not reached: the launch capacity never exceeds MAXNR*BLOCK here
    } else {
    // ================= general path: scores per element =================
    // ---- top-p (main.cpp:750-772) ----
    // The survivors' scores alone are sorted (keys ~okey(s), ascending =
    // descending score: 4 bytes each, so every id of a 32768 vocabulary fits
    // the LDS).  The cutoff is then a score T: the kept ids are those above
    // T and, of the ids scoring exactly T, the ones std::sort puts first.
    float T = kNegInf;
    bool tie = false;
    if (use_topp) {
        // counting sort by value bins (finite rows), else the bitonic network
        if (bad || !bin_sort_keys<BLOCK, EPT>(s, n_surv, sblo, hi, key32, key32 + cap, sh, ph)) {
#pragma unroll
            for (int j = 0; j < EPT; ++j)
                if (s[j] != kNegInf) key32[off++] = ~okey(s[j]);
            const int n2 = uni(max(64, pow2ceil(n_surv)));
            for (int i = n_surv + tid; i < n2; i += BLOCK) key32[i] = 0xFFFFFFFFu;
            __syncthreads();
            CBX_STAMP(13);
            bitonic_sort_keys<BLOCK>(key32, n2);
        }
        CBX_STAMP(14);
        const float mx_surv = unif(okey_inv(~key32[0]));
        // The exp terms in sorted order: formed by every lane into the LDS
        // after the keys when it holds them, else where the sums read them.
        // The sums (wave 0) stop once their adds are no-ops.
        float* const eg = reinterpret_cast<float*>(key32 + n_surv);
        const bool e_lds = (size_t)n_surv * 8 <= region_bytes(cap);
        auto e_form = [&](int i) {
            return expf_libm_branchless(__fsub_rn(okey_inv(~key32[i]), mx_surv), tab);
        };
        if (e_lds) {
            for (int i = tid; i < n_surv; i += BLOCK) eg[i] = e_form(i);
            __syncthreads();
        }
        auto e_of = [&](int i) { return e_lds ? eg[i] : e_form(i); };
        constexpr int NG = run_bound<BLOCK>(BLOCK * EPT);
        if (wid == 0) {
            int unused;
            const float ps = wave_run_sum<NG, false, true>(e_of, n_surv, 0.0f, 0.0f, unused, !bad);
            if (lane == 0) sh.psum = ps;
        }
        __syncthreads();
        CBX_STAMP(15);
        const float psum = unif(sh.psum);
        // the cutoff: certified in binary64 where it can be, else the q's summed
        int last = -1, upto = n_surv;
        if (wid == 0 && !bad && !certified_cut<NG>(e_of, n_surv, psum, P.top_p, last, upto)) last = -1;
        if (wid == 0 && lane == 0) {
            sh.n_kept = last + 1;
            sh.n_cand = upto;  // the q's that hold the crossing
        }
        __syncthreads();
        if (uni(sh.n_kept) == 0) {  // not certain (or NaN / +inf rows)
            if (e_lds) {
                for (int i = tid; i < n_surv; i += BLOCK) eg[i] = __fdiv_rn(eg[i], psum);
                __syncthreads();
            }
            if (wid == 0) {
                int hit;
                auto q_of = [&](int i) { return e_lds ? eg[i] : __fdiv_rn(e_form(i), psum); };
                const int nq = bad ? n_surv : uni(sh.n_cand);
                (void)wave_run_sum<NG, true, true>(q_of, nq, 0.0f, P.top_p, hit, !bad);
                if (hit < 0 && nq < n_surv)
                    (void)wave_run_sum<NG, true, true>(q_of, n_surv, 0.0f, P.top_p, hit, !bad);
                if (lane == 0) sh.n_kept = (hit < 0 ? n_surv - 1 : hit) + 1;
            }
            __syncthreads();
        }
        const int n_kept = uni(sh.n_kept);
        T = unif(okey_inv(~key32[n_kept - 1]));
        tie = n_kept < n_surv && unif(okey_inv(~key32[n_kept])) == T;
        if (tid == 0) {
            sh.mx = mx_surv;  // min-p reference: the best survivor
            if (tie) sh.flags |= CBX_INFO_TOPP_TIE;
        }
        if (tie && !bad) {
            // Equal scores straddle the cutoff.  Each survivor becomes a word
            // (rank << 16 | id) -- rank: the first sorted position of its
            // score (same order, same ties, 16 bits) -- in id order (positions
            // from a bitmap of the survivor ids).  Wave 0 replays the
            // reference's std::sort over the ranges holding the tied score
            // (wave_tied_order) when the LDS holds a second array of the same
            // size, else lane 0 replays the whole sort; the first n_kept - kT
            // tied ids are kept.
            const int kT = uni([&] {  // sorted positions scoring above T
                const uint32_t key = ~okey(T);
                int lo = 0, hi = n_surv;
                while (lo < hi) {
                    const int mid = (lo + hi) >> 1;
                    if (key32[mid] < key) lo = mid + 1;
                    else hi = mid;
                }
                return lo;
            }());
            uint32_t rk2[(EPT + 1) / 2];  // two 16-bit ranks per register
#pragma unroll
            for (int q = 0; q < (EPT + 1) / 2; ++q) rk2[q] = 0u;
#pragma unroll
            for (int j = 0; j < EPT; ++j) {
                if (s[j] != kNegInf) {
                    const uint32_t key = ~okey(s[j]);
                    int lo = 0, hi = n_surv;  // first position with key32 >= key
                    while (lo < hi) {
                        const int mid = (lo + hi) >> 1;
                        if (key32[mid] < key) lo = mid + 1;
                        else hi = mid;
                    }
                    rk2[j >> 1] |= (uint32_t)lo << (16 * (j & 1));
                }
            }
            uint32_t* wv = reinterpret_cast<uint32_t*>(region);
            for (int w = tid; w < W; w += BLOCK) keptw[w] = 0u;
            __syncthreads();  // the sorted keys are read: their storage takes the words
#pragma unroll
            for (int j = 0; j < EPT; ++j)
                if (s[j] != kNegInf) {
                    const int i = j * BLOCK + tid;
                    atomicOr(&keptw[i >> 5], 1u << (i & 31));
                }
            __syncthreads();
            (void)bitmap_offsets<BLOCK>(keptw, woff, W, sh, ph);
#pragma unroll
            for (int j = 0; j < EPT; ++j)
                if (s[j] != kNegInf) {
                    const int i = j * BLOCK + tid;
                    wv[rank_of(keptw, woff, i)] = ((rk2[j >> 1] >> (16 * (j & 1))) << 16) | (uint32_t)i;
                }
            __syncthreads();  // every position is read from the bitmap
            for (int w = tid; w < W; w += BLOCK) keptw[w] = 0u;
            __syncthreads();
            if ((size_t)n_surv * 8 <= region_bytes(cap)) {
                uint16_t* tied = reinterpret_cast<uint16_t*>(wv + n_surv);
                if (wid == 0) (void)wave_tied_order(wv, wv + n_surv, n_surv, (uint32_t)kT, tied);
                __syncthreads();
                for (int i = tid; i < n_kept - kT; i += BLOCK)
                    atomicOr(&keptw[tied[i] >> 5], 1u << (tied[i] & 31));
            } else {
                if (tid == 0) (void)stdsort_replay(PackedSeq{wv}, n_surv);
                __syncthreads();
                for (int i = tid; i < n_kept; i += BLOCK) {
                    const uint32_t id = wv[i] & 0xffffu;
                    atomicOr(&keptw[id >> 5], 1u << (id & 31));
                }
            }
        }
        __syncthreads();
    }

    // kept predicate per register element: above the cutoff score, or at it
    // among the ids the replayed sort kept
    uint64_t kept = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = j * BLOCK + tid;
        const bool at_cut = (tie && !bad) ? (s[j] > T || (s[j] == T && bit_of(keptw, i)))
                                          : s[j] >= T;
        const bool k = s[j] != kNegInf && (!use_topp || at_cut);
        kept |= (uint64_t)k << j;
    }

    // ---- min-p [extension]: drop expf(s - s_max) < min_p ----
    if (P.min_p > 0.0f) {
        float m = kNegInf;
#pragma unroll
        for (int j = 0; j < EPT; ++j) m = ((kept >> j) & 1u) ? fmaxf(m, s[j]) : m;
        const float mx_kept = use_topp ? unif(sh.mx) : block_max<BLOCK>(m, sh, ph);
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (((kept >> j) & 1u) && expf_libm_branchless(__fsub_rn(s[j], mx_kept), tab) < P.min_p)
                kept &= ~((uint64_t)1 << j);
    }

    // ---- repetition penalty (main.cpp:774-781), seen bitmap built at load ----
    if (use_pen) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int i = j * BLOCK + tid;
            if (((kept >> j) & 1u) && bit_of(seen, i))
                s[j] = s[j] > 0.0f ? __fdiv_rn(s[j], P.repeat_penalty)
                                   : __fmul_rn(s[j], P.repeat_penalty);
        }
    }
    __syncthreads();  // every read of the top-p bitmap and lists is done
    int id[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) id[j] = j * BLOCK + tid;
    return finish_row<BLOCK, EPT, EPT>(s, id, kept, a, P, rs, u_draw, flags, keptw, woff, F, tab, sh);
    }
}

// The row-step a workgroup samples.  Workgroups are handed to the 8 XCDs in
// turn (workgroup b to XCD b % 8), and inside an XCD again in turn to its
// parts, while consecutive row-steps of a launch are the streams of one step,
// each with its own knobs (and so its own cost: a top_k of 1000 costs about
// twice a top_k of 50).  Taken in launch order, XCD x would sample only the
// streams r = x mod 8 (and its parts narrower classes still), and the part
// holding the costliest streams would set the launch's time.  Instead each
// XCD takes a contiguous eighth of the launch's row-steps and, when that
// eighth is whole steps, walks it stream by stream (the steps of one stream
// in turn): every part sees every stream alike, and a stream's history is
// re-read from the XCD's L2.  Measured on the headline workload (B=256
// streams with top_k of 50, 250 or 1000 each): 1.92 -> 1.66 ms per
// 1024-step launch.
__device__ __forceinline__ int64_t xcd_spread(int64_t b, int64_t n, int64_t n_rows) {
    if (n % 8) return b;
    const int64_t m = n / 8, k = b / 8;
    if (m % n_rows) return (b % 8) * m + k;
    const int64_t steps = m / n_rows;
    return (b % 8) * m + (k % steps) * n_rows + k / steps;
}

template <int BLOCK, int EPT, int MAXNR, bool GENERAL>
__global__ __launch_bounds__(BLOCK) void sample_rows_kernel(KernelArgs a) {
    __shared__ Shared sh;
    __shared__ uint64_t tab[32];
    extern __shared__ __align__(16) uint8_t smem[];
    sample_row_wg<BLOCK, EPT, MAXNR, GENERAL>(a, xcd_spread(blockIdx.x, gridDim.x, a.n_rows), sh, tab,
                                              smem);
}

// The rows a launch put on its redo list (more ids survived top-k than its
// capacity held), sampled again here at the vocabulary's capacity:
// workgroup b takes list entry b, or leaves at once when the list is
// shorter.  One row per workgroup and no loop around the row's code: in a
// loop the compiler's allocation of the row's registers spills.  The last of
// the working workgroups clears the list for the next launch (no memset, so
// the pair of launches can be captured in a graph).  A workgroup that reads
// the count after that clear finds 0 and leaves, which is right: every
// workgroup with a row to do read the count before adding itself to `done`.
template <int BLOCK, int EPT, int MAXNR>
__global__ __launch_bounds__(BLOCK) void redo_rows_kernel(KernelArgs a) {
    __shared__ Shared sh;
    __shared__ uint64_t tab[32];
    __shared__ int32_t head[2];
    extern __shared__ __align__(16) uint8_t smem[];
    int32_t* const list = a.redo;
    if (threadIdx.x == 0) {
        const int n = min(list[0], a.redo_max);
        head[0] = n;
        head[1] = (int)blockIdx.x < n ? list[2 + blockIdx.x] : -1;
    }
    __syncthreads();
    const int n = uni(head[0]), row = uni(head[1]);
    if (row < 0) return;
    a.redo = nullptr;  // full capacity: nothing more to hand on
    sample_row_wg<BLOCK, EPT, MAXNR, true>(a, row, sh, tab, smem);
    if (threadIdx.x == 0) {
        __threadfence();
        if (atomicAdd(&list[1], 1) == n - 1) {
            list[0] = 0;
            list[1] = 0;
            __threadfence();
        }
    }
}

// One decode step (cbx_decode_step): workgroup r takes stream r (one step, so
// the row-step is the row) at full capacity, where no row overflows.  A
// stream that has ended is not sampled; a running one is sampled by the
// plain row code, after which thread 0 -- the thread that stored the row's
// token, which the row code returns to it -- applies the engine loop's update
// (chatterbox_engine.cpp:345-353): the stop token ends the stream, any other
// id is pushed onto its history (which the row read, [0, len), for its
// penalty), written as the next step's input, and ends the stream at its
// length limit.  The other kernels carry none of this.
template <int BLOCK, int EPT, int MAXNR>
__global__ __launch_bounds__(BLOCK) void decode_rows_kernel(KernelArgs a) {
    __shared__ Shared sh;
    __shared__ uint64_t tab[32];
    extern __shared__ __align__(16) uint8_t smem[];
    const int row = blockIdx.x;
    // the stream's state, length and limit, read while the row loads (no
    // memory round trip of their own before or after the row)
    const int32_t state = a.dec_state[row];
    const int32_t len0 = a.dec_len[row];
    const int32_t max0 = a.dec_max ? a.dec_max[row] : 0;
    const int32_t token = sample_row_wg<BLOCK, EPT, MAXNR, true, true>(a, row, sh, tab, smem, state);
    if (token == kEndedRow) return;
    if (threadIdx.x == 0) {  // the thread that stored the token
        if (token == a.stop_token) {
            a.dec_state[row] = CBX_DECODE_STOP;
            return;
        }
        const int64_t lim = a.dec_max ? min((int64_t)max0, a.ld_history) : a.ld_history;
        int32_t len = max(len0, 0);
        if (len < lim) {
            a.dec_history[(int64_t)row * a.ld_history + len] = token;
            a.dec_len[row] = ++len;
        }
        if (a.dec_next) a.dec_next[row] = token;
        if (len >= lim) a.dec_state[row] = CBX_DECODE_LIMIT;
    }
}

// LDS a workgroup kernel declares besides its dynamic share (the redo
// kernel's row list included).
constexpr size_t kStaticLds = sizeof(Shared) + 32 * 8 + 64;

template <int BLOCK, int EPT, int MAXNR, bool GENERAL>
hipError_t launch_cfg(const KernelArgs& a, hipStream_t stream) {
    const size_t lds = lds_bytes_for(a.cap, a.n_vocab);
    // Dynamic LDS beyond 64 KiB has to be granted per kernel; remember the
    // largest grant so repeated launches skip the call.
    static size_t granted = 64 * 1024 - kStaticLds;
    if (lds > granted) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&sample_rows_kernel<BLOCK, EPT, MAXNR, GENERAL>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        granted = lds;
    }
    const int64_t rows = (int64_t)a.n_steps * a.n_rows;
    hipLaunchKernelGGL((sample_rows_kernel<BLOCK, EPT, MAXNR, GENERAL>), dim3((unsigned)rows),
                       dim3(BLOCK), lds, stream, a);
    return hipGetLastError();
}

template <int BLOCK, int EPT, int MAXNR>
hipError_t launch_redo_cfg(const KernelArgs& a, hipStream_t stream) {
    const size_t lds = lds_bytes_for(a.cap, a.n_vocab);
    static size_t granted = 64 * 1024 - kStaticLds;
    if (lds > granted) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&redo_rows_kernel<BLOCK, EPT, MAXNR>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        granted = lds;
    }
    hipLaunchKernelGGL((redo_rows_kernel<BLOCK, EPT, MAXNR>), dim3((unsigned)a.redo_max),
                       dim3(BLOCK), lds, stream, a);
    return hipGetLastError();
}

// A decode step at capacity a.cap (every row of the vocabulary).
template <int BLOCK, int EPT>
hipError_t launch_decode_for(const KernelArgs& a, hipStream_t stream) {
    constexpr int NRMAX = kFastMax / BLOCK;
    const size_t lds = lds_bytes_for(a.cap, a.n_vocab);
    static size_t granted = 64 * 1024 - kStaticLds;
    if (lds > granted) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&decode_rows_kernel<BLOCK, EPT, NRMAX>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        granted = lds;
    }
    hipLaunchKernelGGL((decode_rows_kernel<BLOCK, EPT, NRMAX>), dim3((unsigned)a.n_rows),
                       dim3(BLOCK), lds, stream, a);
    return hipGetLastError();
}

// The redo pass at capacity a.cap (every row of the vocabulary, on gfx950).
template <int BLOCK, int EPT>
hipError_t launch_redo_for(const KernelArgs& a, hipStream_t stream) {
    return launch_redo_cfg<BLOCK, EPT, kFastMax / BLOCK>(a, stream);
}

// Variant by survivor capacity: the smallest register list that holds `cap`
// survivors, or the full kernel when cap exceeds the register lists (the
// lists hold at most kFastMax survivors: kFastMax / BLOCK rows per lane).
template <int BLOCK, int EPT>
hipError_t launch_for(const KernelArgs& a, hipStream_t stream) {
    constexpr int NRMAX = kFastMax / BLOCK;
    static_assert(NRMAX >= 1 && NRMAX * BLOCK == kFastMax, "register list rows");
    if (a.cap <= BLOCK) return launch_cfg<BLOCK, EPT, 1, false>(a, stream);
    if constexpr (NRMAX > 4) {
        if (a.cap <= 4 * BLOCK) return launch_cfg<BLOCK, EPT, 4, false>(a, stream);
    }
    if (a.cap <= kFastMax) return launch_cfg<BLOCK, EPT, NRMAX, false>(a, stream);
    return launch_cfg<BLOCK, EPT, NRMAX, true>(a, stream);
}

}  // namespace
}  // namespace cbx
