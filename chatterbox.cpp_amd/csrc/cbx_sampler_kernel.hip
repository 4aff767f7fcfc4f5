// cbx_sampler_kernel.hip -- gfx950 kernels for the T3 logits->token sampler.
//
// One workgroup samples one (step, stream) row; a launch covers
// n_steps x n_rows rows.  The row's scores stay in registers for the whole
// kernel (EPT per lane, element i = j*BLOCK + tid, so every global load and
// store is coalesced); LDS holds only what must be ordered: the survivors
// sorted for top-p (6 bytes each) and then the kept scores in id order
// (4 bytes each), plus id bitmaps.  Stage order and arithmetic follow
// sample_next_token_ex (src/main.cpp:726-801):
//
//   load + CFG combine + masks + temperature   (main.cpp:733-738)
//   top-k: LDS radix select of the (k+1)-th largest, 8 bits per pass
//          (main.cpp:740-748, including the -1e-10f nudge)
//   top-p: survivors compacted to LDS, bitonic sort (descending score,
//          ascending id), glibc-exact expf, the two binary32 running sums in
//          sorted order (main.cpp:750-772)
//   min-p [extension], in registers
//   repetition penalty from an LDS bitmap of the history (main.cpp:774-781)
//   softmax: binary32 running sum in id order (main.cpp:783-793)
//   greedy argmax, or the libstdc++ discrete_distribution CDF walked in id
//   order in binary64 (main.cpp:795-800; random.tcc:2657-2712)
//
// The running sums are evaluated in the reference's order with IEEE binary32
// / binary64 adds, so every intermediate value is the reference's value.
// Arithmetic uses explicitly rounded intrinsics (__fadd_rn, ...), and the
// library is built with -ffp-contract=off as well.
#include <hip/hip_runtime.h>

#include "cbx_expf.h"
#include "cbx_internal.h"
#include "cbx_philox.h"

namespace cbx {
namespace {

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kPosInf = __builtin_huge_valf();

// Monotone map float -> uint32 (ascending float order = ascending key).
__device__ __forceinline__ uint32_t okey(float f) {
    const uint32_t b = __builtin_bit_cast(uint32_t, f);
    return b ^ ((b & 0x80000000u) ? 0xFFFFFFFFu : 0x80000000u);
}
__device__ __forceinline__ float okey_inv(uint32_t k) {
    const uint32_t b = k ^ ((k & 0x80000000u) ? 0x80000000u : 0xFFFFFFFFu);
    return __builtin_bit_cast(float, b);
}

__device__ __forceinline__ int wave_incl_scan(int x, int lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(x, o, 64);
        if (lane >= o) x += t;
    }
    return x;
}
__device__ __forceinline__ float wave_max(float x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = fmaxf(x, __shfl_xor(x, o, 64));
    return x;
}
__device__ __forceinline__ int wave_min(int x) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) x = min(x, __shfl_xor(x, o, 64));
    return x;
}

struct Shared {
    uint32_t hist[256];
    int red_i[16];
    float red_f[16];
    uint32_t sel_digit, sel_above;
    float psum;        // broadcast of a running sum
    int n_kept;        // survivors after top-p
    int token;
    float tie[2];      // scores at the top-p cutoff and just after it
    uint32_t flags;
};

// Exclusive block scan of one int per lane; `total` receives the block sum.
template <int BLOCK>
__device__ __forceinline__ int block_excl_scan(int v, Shared& sh, int& total) {
    constexpr int NW = BLOCK / 64;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    const int incl = wave_incl_scan(v, lane);
    if (lane == 63) sh.red_i[wid] = incl;
    __syncthreads();
    int before = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
        const int t = sh.red_i[w];
        before += (w < wid) ? t : 0;
        tot += t;
    }
    __syncthreads();
    total = tot;
    return before + incl - v;
}

template <int BLOCK>
__device__ __forceinline__ int block_sum(int v, Shared& sh) {
    int total;
    (void)block_excl_scan<BLOCK>(v, sh, total);
    return total;
}

template <int BLOCK>
__device__ __forceinline__ float block_max(float v, Shared& sh) {
    constexpr int NW = BLOCK / 64;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_max(v);
    if (lane == 0) sh.red_f[wid] = v;
    __syncthreads();
    float m = sh.red_f[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, sh.red_f[w]);
    __syncthreads();
    return m;
}

template <int BLOCK>
__device__ __forceinline__ int block_min(int v, Shared& sh) {
    constexpr int NW = BLOCK / 64;
    const int lane = threadIdx.x & 63, wid = threadIdx.x >> 6;
    v = wave_min(v);
    if (lane == 0) sh.red_i[wid] = v;
    __syncthreads();
    int m = sh.red_i[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = min(m, sh.red_i[w]);
    __syncthreads();
    return m;
}

// The (rank+1)-th largest key among the first n_valid elements (rank is
// 0-based), by 4 passes of an 8-bit LDS histogram over the bucket that still
// contains it.
template <int BLOCK, int EPT>
__device__ uint32_t radix_select_desc(const float (&s)[EPT], int n_valid, int rank, Shared& sh) {
    const int tid = threadIdx.x, lane = tid & 63, wid = tid >> 6;
    uint32_t prefix = 0, pmask = 0;
    uint32_t rem = (uint32_t)rank;
    for (int pass = 0; pass < 4; ++pass) {
        const int shift = 24 - 8 * pass;
        for (int i = tid; i < 256; i += BLOCK) sh.hist[i] = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int i = j * BLOCK + tid;
            if (i < n_valid) {
                const uint32_t k = okey(s[j]);
                if ((k & pmask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 0xFFu], 1u);
            }
        }
        __syncthreads();
        if (wid == 0) {
            // Lane l owns digits 255-4l .. 252-4l (descending).
            const uint32_t c0 = sh.hist[255 - 4 * lane], c1 = sh.hist[254 - 4 * lane];
            const uint32_t c2 = sh.hist[253 - 4 * lane], c3 = sh.hist[252 - 4 * lane];
            const int tot = (int)(c0 + c1 + c2 + c3);
            const uint32_t incl = (uint32_t)wave_incl_scan(tot, lane);
            const uint32_t excl = incl - (uint32_t)tot;
            const uint64_t hit = __ballot(incl > rem);
            const int L = __ffsll((unsigned long long)hit) - 1;
            if (lane == L) {
                uint32_t d, above;
                if (excl + c0 > rem) { d = 255 - 4 * lane; above = excl; }
                else if (excl + c0 + c1 > rem) { d = 254 - 4 * lane; above = excl + c0; }
                else if (excl + c0 + c1 + c2 > rem) { d = 253 - 4 * lane; above = excl + c0 + c1; }
                else { d = 252 - 4 * lane; above = excl + c0 + c1 + c2; }
                sh.sel_digit = d;
                sh.sel_above = above;
            }
        }
        __syncthreads();
        prefix |= sh.sel_digit << shift;
        pmask |= 0xFFu << shift;
        rem -= sh.sel_above;
        __syncthreads();
    }
    return prefix;
}

// Ascending bitonic sort of (key, id) pairs [0, n2) (n2 a power of two) in
// LDS, ordered by key then id.
template <int BLOCK>
__device__ void bitonic_sort_pairs(uint32_t* key, uint16_t* id, int n2) {
    for (int k = 2; k <= n2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int t = threadIdx.x; t < (n2 >> 1); t += BLOCK) {
                const int i = ((t & ~(j - 1)) << 1) | (t & (j - 1));
                const int p = i + j;
                const bool up = (i & k) == 0;
                const uint32_t ka = key[i], kb = key[p];
                const uint16_t ia = id[i], ib = id[p];
                const bool a_gt_b = (ka > kb) || (ka == kb && ia > ib);
                if (a_gt_b == up) { key[i] = kb; key[p] = ka; id[i] = ib; id[p] = ia; }
            }
            __syncthreads();
        }
    }
}

// Sequential binary32 sum of v[0, n) in index order (one lane).
__device__ __forceinline__ float seq_sum_f32(const float* v, int n) {
    float acc = 0.0f;
    int i = 0;
    for (; i + 4 <= n; i += 4) {
        const float4 q = *reinterpret_cast<const float4*>(v + i);
        acc = __fadd_rn(acc, q.x);
        acc = __fadd_rn(acc, q.y);
        acc = __fadd_rn(acc, q.z);
        acc = __fadd_rn(acc, q.w);
    }
    for (; i < n; ++i) acc = __fadd_rn(acc, v[i]);
    return acc;
}

__device__ __forceinline__ int pow2ceil(int n) {
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}

__device__ __forceinline__ bool bit_of(const uint32_t* words, int i) {
    return (words[i >> 5] >> (i & 31)) & 1u;
}

template <int BLOCK, int EPT>
__global__ __launch_bounds__(BLOCK) void sample_rows_kernel(KernelArgs a) {
    __shared__ Shared sh;
    extern __shared__ __align__(16) uint8_t smem[];

    const int tid = threadIdx.x;
    const int64_t g = blockIdx.x;
    const int step = (int)(g / a.n_rows), row = (int)(g % a.n_rows);
    const int V = a.n_vocab;
    const int cap = a.cap;
    const int W = (V + 31) >> 5;
    const int Wp = (W + 3) & ~3;

    // LDS: seen[Wp] | kept[Wp] | woff[Wp] | list region (6*cap bytes):
    //   top-p:  key32[cap] | id16[cap]   (key32 later reused as E / p values)
    //   final:  F[cap] f32 (kept scores -> exp -> probabilities, id order)
    uint32_t* seen = reinterpret_cast<uint32_t*>(smem);
    uint32_t* keptw = seen + Wp;
    uint32_t* woff = keptw + Wp;
    uint32_t* key32 = woff + Wp;
    float* E = reinterpret_cast<float*>(key32);
    uint16_t* id16 = reinterpret_cast<uint16_t*>(key32 + cap);
    float* F = reinterpret_cast<float*>(key32);

    const cbx_params P = a.params[row];
    const int64_t rs = (int64_t)step * a.n_rows + row;  // row-step linear id

    // ---- load, combine, mask, temperature (main.cpp:733-738) ----
    const float* lrow = a.logits + rs * a.ld_logits;
    const float* urow = a.uncond ? a.uncond + rs * a.ld_logits : nullptr;
    const uint32_t* arow = a.allowed ? a.allowed + (int64_t)row * a.ld_allowed : nullptr;
    const bool fstop = a.force_stop && a.force_stop[rs];
    const bool scale = P.temp > 0.0f && P.temp != 1.0f;
    const float inv_t = __fdiv_rn(1.0f, P.temp);
    float s[EPT];
    int nonfinite = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = j * BLOCK + tid;
        float v = kNegInf;
        if (i < V) {
            v = lrow[i];
            if (urow) v = __fadd_rn(v, __fmul_rn(P.cfg_weight, __fsub_rn(v, urow[i])));
            if (arow && !bit_of(arow, i)) v = kNegInf;
            if (fstop && i != a.stop_token) v = kNegInf;
            if (scale) v = __fmul_rn(v, inv_t);
            nonfinite |= (v != v || v == kPosInf) ? 1 : 0;
        }
        s[j] = v;
    }
    if (tid == 0) sh.flags = 0u;

    // ---- top-k (main.cpp:740-748) ----
    if (P.top_k > 0 && P.top_k < V) {
        const uint32_t kth = radix_select_desc<BLOCK, EPT>(s, V, P.top_k, sh);
        float thr = okey_inv(kth);
        int above = 0;
#pragma unroll
        for (int j = 0; j < EPT; ++j) above += (j * BLOCK + tid < V && s[j] > thr) ? 1 : 0;
        above = block_sum<BLOCK>(above, sh);
        if (above < P.top_k) thr = __fsub_rn(thr, 1e-10f);
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (s[j] <= thr) s[j] = kNegInf;
    }

    // ---- survivors (score != -inf): count and id-order offsets ----
    int mine = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) mine += (j * BLOCK + tid < V && s[j] != kNegInf) ? 1 : 0;
    int n_surv;
    int off = block_excl_scan<BLOCK>(mine, sh, n_surv);
    nonfinite = block_sum<BLOCK>(nonfinite, sh);
    uint32_t flags = nonfinite ? CBX_INFO_NONFINITE : 0u;
    if (n_surv > cap) {
        if (tid == 0) {
            a.tokens[rs] = -1;
            if (a.info) a.info[rs] = flags | CBX_INFO_OVERFLOW;
        }
        if (a.probs) {
            float* prow = a.probs + rs * a.ld_probs;
            for (int i = tid; i < V; i += BLOCK) prow[i] = 0.0f;
        }
        return;
    }

    for (int w = tid; w < W; w += BLOCK) { keptw[w] = 0u; seen[w] = 0u; }
    __syncthreads();

    // ---- top-p (main.cpp:750-772) ----
    const bool use_topp = P.top_p < 1.0f && n_surv > 0;
    float mx_surv = kNegInf;  // largest survivor score (sorted[0].s)
    if (use_topp) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int i = j * BLOCK + tid;
            if (i < V && s[j] != kNegInf) {
                key32[off] = ~okey(s[j]);
                id16[off] = (uint16_t)i;
                ++off;
            }
        }
        const int n2 = pow2ceil(n_surv);
        for (int i = n_surv + tid; i < n2; i += BLOCK) { key32[i] = 0xFFFFFFFFu; id16[i] = 0xFFFFu; }
        __syncthreads();
        bitonic_sort_pairs<BLOCK>(key32, id16, n2);
        mx_surv = okey_inv(~key32[0]);
        __syncthreads();
        for (int i = tid; i < n_surv; i += BLOCK)
            E[i] = expf_libm(__fsub_rn(okey_inv(~key32[i]), mx_surv));
        __syncthreads();
        if (tid == 0) sh.psum = seq_sum_f32(E, n_surv);
        __syncthreads();
        const float psum = sh.psum;
        for (int i = tid; i < n_surv; i += BLOCK) E[i] = __fdiv_rn(E[i], psum);
        __syncthreads();
        if (tid == 0) {
            float cum = 0.0f;
            int last = n_surv - 1;
            for (int i = 0; i < n_surv; ++i) {
                cum = __fadd_rn(cum, E[i]);
                if (cum >= P.top_p) { last = i; break; }
            }
            sh.n_kept = last + 1;
        }
        __syncthreads();
        const int n_kept = sh.n_kept;
        for (int i = tid; i < n_kept; i += BLOCK) {
            const uint32_t idx = id16[i];
            atomicOr(&keptw[idx >> 5], 1u << (idx & 31));
        }
        // equal scores straddling the cutoff: read both ids' scores back
        if (n_kept < n_surv) {
            const int ia = id16[n_kept - 1], ib = id16[n_kept];
#pragma unroll
            for (int j = 0; j < EPT; ++j) {
                const int i = j * BLOCK + tid;
                if (i == ia) sh.tie[0] = s[j];
                if (i == ib) sh.tie[1] = s[j];
            }
        }
        __syncthreads();
        if (tid == 0 && n_kept < n_surv && sh.tie[0] == sh.tie[1]) sh.flags |= CBX_INFO_TOPP_TIE;
    }

    // kept predicate per register element
    uint64_t kept = 0;
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = j * BLOCK + tid;
        const bool k = (i < V) && s[j] != kNegInf && (!use_topp || bit_of(keptw, i));
        kept |= (uint64_t)k << j;
    }

    // ---- min-p [extension]: drop expf(s - s_max) < min_p ----
    if (P.min_p > 0.0f) {
        float m = kNegInf;
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if ((kept >> j) & 1u) m = fmaxf(m, s[j]);
        const float mx_kept = use_topp ? mx_surv : block_max<BLOCK>(m, sh);
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (((kept >> j) & 1u) && expf_libm(__fsub_rn(s[j], mx_kept)) < P.min_p)
                kept &= ~((uint64_t)1 << j);
    }

    // ---- repetition penalty (main.cpp:774-781) from a bitmap of the history ----
    // a history longer than its row stride is read only up to the stride
    const int hlen = a.history ? (int)min((int64_t)a.history_len[row], a.ld_history) : 0;
    const bool use_pen = P.repeat_penalty != 1.0f && hlen > 0;
    if (use_pen) {
        const int32_t* hrow = a.history + (int64_t)row * a.ld_history;
        for (int j = tid; j < hlen; j += BLOCK) {
            const int32_t t = hrow[j];
            if (t >= 0 && t < V) atomicOr(&seen[t >> 5], 1u << (t & 31));
        }
    }
    __syncthreads();  // seen complete; top-p lists no longer read
    if (use_pen) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int i = j * BLOCK + tid;
            if (((kept >> j) & 1u) && bit_of(seen, i))
                s[j] = s[j] > 0.0f ? __fdiv_rn(s[j], P.repeat_penalty)
                                   : __fmul_rn(s[j], P.repeat_penalty);
        }
    }

    // ---- final kept bitmap and id-order ranks ----
    for (int w = tid; w < W; w += BLOCK) keptw[w] = 0u;
    __syncthreads();
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if ((kept >> j) & 1u) {
            const int i = j * BLOCK + tid;
            atomicOr(&keptw[i >> 5], 1u << (i & 31));
        }
    __syncthreads();
    int n_final;
    {
        constexpr int WPT = (kMaxVocab / 32 + BLOCK - 1) / BLOCK;  // words per lane
        int cnt[WPT];
        int local = 0;
#pragma unroll
        for (int q = 0; q < WPT; ++q) {
            const int w = tid * WPT + q;
            cnt[q] = (w < W) ? __popc(keptw[w]) : 0;
            local += cnt[q];
        }
        int base = block_excl_scan<BLOCK>(local, sh, n_final);
#pragma unroll
        for (int q = 0; q < WPT; ++q) {
            const int w = tid * WPT + q;
            if (w < W) woff[w] = (uint32_t)base;
            base += cnt[q];
        }
    }
    __syncthreads();

    // ---- softmax (main.cpp:783-793) ----
    float m = kNegInf;
#pragma unroll
    for (int j = 0; j < EPT; ++j)
        if ((kept >> j) & 1u) m = fmaxf(m, s[j]);
    const float mx2 = block_max<BLOCK>(m, sh);
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int i = j * BLOCK + tid;
        if ((kept >> j) & 1u) {
            s[j] = expf_libm(__fsub_rn(s[j], mx2));
            const uint32_t wb = keptw[i >> 5];
            F[woff[i >> 5] + __popc(wb & ((1u << (i & 31)) - 1u))] = s[j];
        }
    }
    __syncthreads();
    if (tid == 0) sh.psum = seq_sum_f32(F, n_final);
    __syncthreads();
    const float psum2 = sh.psum;
    const bool empty = (psum2 == 0.0f);
    if (!empty) {
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int i = j * BLOCK + tid;
            if ((kept >> j) & 1u) {
                s[j] = __fdiv_rn(s[j], psum2);
                const uint32_t wb = keptw[i >> 5];
                F[woff[i >> 5] + __popc(wb & ((1u << (i & 31)) - 1u))] = s[j];
            }
        }
    }
    __syncthreads();

    // ---- greedy or draw (main.cpp:795-800) ----
    int32_t token = 0;
    if (empty) {
        flags |= CBX_INFO_EMPTY;
    } else if (P.temp <= 0.0f) {
        // first argmax over the full probability vector (zeros elsewhere)
        float best = -1.0f;
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if ((kept >> j) & 1u) best = fmaxf(best, s[j]);
        best = block_max<BLOCK>(best, sh);
        int first = 0x7fffffff;
#pragma unroll
        for (int j = 0; j < EPT; ++j)
            if (((kept >> j) & 1u) && s[j] == best) first = min(first, j * BLOCK + tid);
        token = block_min<BLOCK>(first, sh);
        if (token == 0x7fffffff) token = 0;  // only NaN probabilities: no maximum
        flags |= CBX_INFO_GREEDY;
    } else if (V >= 2) {
        flags |= CBX_INFO_DREW;
        if (tid == 0) {
            double u;
            if (a.draw_mode == CBX_DRAW_PHILOX) {
                const uint64_t sid = a.stream_ids ? a.stream_ids[row] : (uint64_t)row;
                u = philox_uniform(a.seed, sid, a.step0 + (uint64_t)step);
            } else {
                u = a.uniforms[rs];
            }
            // random.tcc:2665-2676: double weights summed from 0.0 in id order,
            // each divided by the sum, running partial sums, last entry 1.0;
            // :2708-2712: the first id whose cumulative value is >= u.
            double sum = 0.0;
            for (int r = 0; r < n_final; ++r) sum = __dadd_rn(sum, (double)F[r]);
            int rank = -1;  // -1: past every kept id -> the forced last entry
            if (!(u > 0.0)) {
                rank = -2;  // u == 0: cumulative value of id 0 (>= 0) already >= u
            } else {
                double acc = 0.0;
                for (int r = 0; r < n_final; ++r) {
                    acc = __dadd_rn(acc, __ddiv_rn((double)F[r], sum));
                    if (acc >= u) { rank = r; break; }
                }
            }
            int tok;
            if (rank == -2) {
                tok = 0;
            } else if (rank == -1) {
                tok = V - 1;
            } else {
                // id of the rank-th kept entry: word by offsets, bit by popcount
                int w = 0;
                while (w + 1 < W && (int)woff[w + 1] <= rank) ++w;
                uint32_t bits = keptw[w];
                for (int k = rank - (int)woff[w]; k > 0; --k) bits &= bits - 1u;
                tok = w * 32 + __ffs(bits) - 1;
            }
            sh.token = tok;
        }
        __syncthreads();
        token = sh.token;
    }

    if (tid == 0) {
        a.tokens[rs] = token;
        if (a.info) a.info[rs] = flags | sh.flags;
    }
    if (a.probs) {
        float* prow = a.probs + rs * a.ld_probs;
#pragma unroll
        for (int j = 0; j < EPT; ++j) {
            const int i = j * BLOCK + tid;
            if (i < V) prow[i] = (!empty && ((kept >> j) & 1u)) ? s[j] : 0.0f;
        }
    }
}

__global__ void debug_expf_kernel(const float* in, float* out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = expf_libm(in[i]);
}

__global__ void debug_philox_kernel(uint64_t seed, const uint64_t* sid, uint64_t step, int32_t n,
                                    double* out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = philox_uniform(seed, sid ? sid[i] : (uint64_t)i, step);
}

template <int BLOCK, int EPT>
hipError_t launch_cfg(const KernelArgs& a, hipStream_t stream) {
    const size_t lds = lds_bytes_for(a.cap, a.n_vocab);
    // Dynamic LDS beyond 64 KiB has to be granted per kernel; remember the
    // largest grant so repeated launches skip the call.
    static size_t granted = 64 * 1024 - sizeof(Shared);
    if (lds > granted) {
        hipError_t e = hipFuncSetAttribute(
            reinterpret_cast<const void*>(&sample_rows_kernel<BLOCK, EPT>),
            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess) return e;
        granted = lds;
    }
    const int64_t rows = (int64_t)a.n_steps * a.n_rows;
    hipLaunchKernelGGL((sample_rows_kernel<BLOCK, EPT>), dim3((unsigned)rows), dim3(BLOCK), lds,
                       stream, a);
    return hipGetLastError();
}

}  // namespace

size_t lds_bytes_for(int32_t cap, int32_t n_vocab) {
    const size_t Wp = (size_t)(((n_vocab + 31) / 32 + 3) & ~3);
    return 3 * Wp * 4 + (size_t)cap * 6;
}

int32_t max_cap_for_lds(int32_t n_vocab, size_t lds_bytes) {
    int32_t cap = 1 << 16;
    while (cap > 64 && lds_bytes_for(cap, n_vocab) + sizeof(Shared) > lds_bytes) cap >>= 1;
    return cap;
}

hipError_t launch_sample(const KernelArgs& a, hipStream_t stream) {
    if (a.n_vocab <= 256 * 32) return launch_cfg<256, 32>(a, stream);
    return launch_cfg<1024, 32>(a, stream);
}

hipError_t launch_debug_expf(const float* in, float* out, int64_t n, hipStream_t stream) {
    const int64_t blocks = (n + 255) / 256;
    hipLaunchKernelGGL(debug_expf_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, in, out, n);
    return hipGetLastError();
}

hipError_t launch_debug_philox(uint64_t seed, const uint64_t* stream_ids, uint64_t step,
                               int32_t n, double* out, hipStream_t stream) {
    const int blocks = (n + 255) / 256;
    hipLaunchKernelGGL(debug_philox_kernel, dim3(blocks), dim3(256), 0, stream, seed, stream_ids,
                       step, n, out);
    return hipGetLastError();
}

}  // namespace cbx
