// cbx_sampler_wave.h -- the one-wavefront-per-row sampler (vocabularies up to
// 256*Q ids, at most kWaveCap survivors after top-k).
//
// A row of a few thousand logits is small: one 64-lane wave holds it in
// registers (4*Q scores per lane, loaded as 16-byte vectors: element 4j + c of
// lane l is id 256j + 4l + c), and every reduction, scan and compaction is a
// wave operation (DPP, ballot/mbcnt) with no workgroup barrier.  Each
// workgroup is a single wave, so a CU keeps many rows in flight while others
// wait on HBM.  Stage order and arithmetic follow sample_next_token_ex
// (src/main.cpp:726-801), exactly as the workgroup kernel in
// cbx_sampler_impl.h does:
//
//   load + CFG combine + masks + temperature (main.cpp:733-738)
//   top-k (main.cpp:740-748): value-bin histogram over [min, max] (a monotone
//          map), exact selection among the scores of the bin holding rank k;
//          rows with NaN/+inf or degenerate ranges use an 8-bit radix select
//   survivors -> LDS list of (descending score, ascending id) keys; counting
//          sort by value bin, each key placed by its rank inside its bin
//   top-p (main.cpp:750-772): the binary32 running sums psum and cum by
//          binade segments or sweep chains; min-p [extension]; repetition
//          penalty from an LDS bitmap of the history (main.cpp:774-781)
//   softmax + draw (main.cpp:783-800): the kept exp terms in id order; the
//          token is located on the parallel binary64 prefix of the exp terms
//          when the uniform is more than kDrawMargin (relative) from both
//          neighbouring boundaries -- the reference's cumulative values differ
//          from that prefix ratio by less than 2^-23 relative, whatever its
//          float normaliser -- otherwise, and for greedy rows or when
//          probabilities are requested, the reference's float normaliser is
//          summed term by term and its double CDF replayed.
//
// Per-element work is written without branches (spare histogram bins and
// list slots take what is dropped): the unrolled element loops would
// otherwise keep one exec mask per element alive.
#pragma once

#include <type_traits>

#include "cbx_sampler_impl.h"

namespace cbx {
namespace {

constexpr int kWaveBins = 1024;   // value bins: top-k select, survivor sort
constexpr int kWaveCand = 256;    // scores in the selected top-k bin
constexpr int kWaveSortMax = 64;  // largest bin the counting sort ranks directly
constexpr int kWaveRows = kWaveCap / 64;

// Waves per SIMD the register allocation aims for (the row's scores take
// 4*Q registers; the rest of the kernel is kept within the same budget).
#ifndef WAVE_WPE
#define WAVE_WPE 4
#endif

// LDS of one row (9.9 KB at Q = 26, allocated in 512-byte granules as
// 10 KB: 16 rows per CU, as many as the 128-register budget allows).  Phases
// reuse storage:
//   list:  the top-k histogram (u32 bins) until the survivors are written;
//          the survivor entries; the top-k bin's candidates while the
//          entries are in registers; the sort's bin counters and offsets
//          while the entries are in registers; the sorted keys; the kept exp
//          terms F in id order at the end
//   keptw: the allowed row of masked rows at the start; the kept bitmap at
//          the end
//   h:     the history bitmap until the penalty pass has read it; then the
//          kept bitmap's word offsets
template <int Q>
struct WaveSmem {
    uint64_t tab[32];
    uint32_t keptw[8 * Q];  // kept ids after every filter
    union {
        uint32_t seen[8 * Q];  // history ids (penalty)
        uint32_t woff[8 * Q];  // kept ids before each word
    } h;
    alignas(16) uint64_t list[kWaveCap + 4];  // survivors (+ padding: maximum keys)
    int rk;

    __device__ float* cand() { return reinterpret_cast<float*>(list); }  // scores of the top-k bin
    __device__ uint64_t* candk() { return list; }  // (score bits << 32 | id), same bin
    __device__ uint32_t* khist() { return reinterpret_cast<uint32_t*>(list); }
    __device__ float* F() { return reinterpret_cast<float*>(list); }
};

// ------------------------------------------------------------ wave helpers


// Four consecutive words of a raw buffer (one 16-byte load).  The vector is
// copied out as bytes: subscripting the builtin's vector result directly
// makes this compiler emit a single-word load.
__device__ __forceinline__ void load4(const __amdgpu_buffer_rsrc_t& r, int voff, int soff,
                                      float* out) {
    // non-temporal (cache policy nt): each row's logits are read once
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 2);
    __builtin_memcpy(out, &v, 16);
}

// Position of this lane's item among the lanes whose bit is set in m.
__device__ __forceinline__ int ballot_rank(uint64_t m) {
    return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(m >> 32),
                                          __builtin_amdgcn_mbcnt_lo((uint32_t)m, 0u));
}

// LDS byte offset of a shared-memory object (the low word of its generic
// address is its offset in the LDS aperture).
template <typename T>
__device__ __forceinline__ uint32_t lds_offset(const T* p) {
    return (uint32_t)(uintptr_t)p;
}

// LDS stores and ORs made by the lanes of `mask` only (a ballot, so a subset
// of the active lanes): the other lanes are switched off for the one
// instruction instead of being sent to spare slots by a per-lane select.
// s_and_saveexec narrows exec to the lanes of the mask that are active and
// keeps the caller's exec, which is put back after the store, so the
// helpers are right in divergent code too (at the cost of the two scalar
// instructions any exec switch takes).
//   pair: w0 at byte offset addr, w1 at addr + 4 (two data registers, so no
//   register pair is assembled for it)
__device__ __forceinline__ void lds_store_pair_lanes(uint32_t addr, uint32_t w0, uint32_t w1,
                                                     uint64_t mask) {
    uint64_t save;
    asm volatile(
        "s_and_saveexec_b64 %0, %4\n\t"
        "ds_write2_b32 %1, %2, %3 offset1:1\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(save)
        : "v"(addr), "v"(w0), "v"(w1), "s"(mask)
        : "memory", "scc");
}
__device__ __forceinline__ void lds_store_b64_lanes(uint32_t addr, uint64_t v, uint64_t mask) {
    uint64_t save;
    asm volatile(
        "s_and_saveexec_b64 %0, %3\n\t"
        "ds_write_b64 %1, %2\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(save)
        : "v"(addr), "v"(v), "s"(mask)
        : "memory", "scc");
}
__device__ __forceinline__ void lds_store_b32_lanes(uint32_t addr, uint32_t v, uint64_t mask) {
    uint64_t save;
    asm volatile(
        "s_and_saveexec_b64 %0, %3\n\t"
        "ds_write_b32 %1, %2\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(save)
        : "v"(addr), "v"(v), "s"(mask)
        : "memory", "scc");
}
// One step of an append: the lanes whose score v is >= b0 store (id, v) at
// consecutive 8-byte slots from byte offset sb in lane order, and sb moves
// past them.  v_cmp writes the lane mask to VCC (inactive lanes 0); when no
// lane passes, the rest is branched over (most vectors of a row with a small
// top_k hold no survivor); else s_and_saveexec narrows exec to it and keeps
// the caller's exec, which is restored after the store.
__device__ __forceinline__ uint32_t append_ge(uint32_t sb, float b0, float v, uint32_t id) {
    uint32_t t, cnt;
    uint64_t save;
    asm volatile(
        "v_cmp_le_f32 vcc, %[b0], %[v]\n\t"
        "s_cbranch_vccz 1f\n\t"
        "s_and_saveexec_b64 %[save], vcc\n\t"
        "v_mbcnt_lo_u32_b32 %[t], vcc_lo, 0\n\t"
        "v_mbcnt_hi_u32_b32 %[t], vcc_hi, %[t]\n\t"
        "v_lshl_add_u32 %[t], %[t], 3, %[sb]\n\t"
        "ds_write2_b32 %[t], %[id], %[v] offset1:1\n\t"
        "s_mov_b64 exec, %[save]\n\t"
        "s_bcnt1_i32_b64 %[cnt], vcc\n\t"
        "s_lshl3_add_u32 %[sb], %[cnt], %[sb]\n"
        "1:"
        : [t] "=&v"(t), [cnt] "=&s"(cnt), [sb] "+s"(sb), [save] "=&s"(save)
        : [b0] "s"(b0), [v] "v"(v), [id] "v"(id)
        : "vcc", "scc", "memory");
    return sb;
}
__device__ __forceinline__ void lds_or_b32_lanes(uint32_t addr, uint32_t v, uint64_t mask) {
    uint64_t save;
    asm volatile(
        "s_and_saveexec_b64 %0, %3\n\t"
        "ds_or_b32 %1, %2\n\t"
        "s_mov_b64 exec, %0"
        : "=&s"(save)
        : "v"(addr), "v"(v), "s"(mask)
        : "memory", "scc");
}

// An opaque copy of a uniform value: predicates built on it in one pass are
// not merged with (and kept alive for) those of another pass.
__device__ __forceinline__ int fresh(int v) {
    asm volatile("" : "+s"(v));
    return v;
}
// The same for a float (held in a vector register: values derived from it
// are recomputed where used).
__device__ __forceinline__ float fresh_v(float v) {
    asm volatile("" : "+v"(v));
    return v;
}


// What turns a row's logits into its scores (main.cpp:733-738 and the
// extensions): CFG combine, allowed mask, forced stop, temperature.
struct RowScores {
    __amdgpu_buffer_rsrc_t rl, ru, ra;
    bool uncond, masked_ids, fstop, scale;
    float cfg_w, inv_t;
    int V, stop;

    // CFG combine of raw logits v with the unconditional ones.
    __device__ __forceinline__ void combine4(float* v, const float* un) const {
#pragma unroll
        for (int c = 0; c < 4; ++c) v[c] = __fadd_rn(v[c], __fmul_rn(cfg_w, __fsub_rn(v[c], un[c])));
    }
    // Scores of ids 256j + 4*lane + c (c < 4) from combined logits.
    __device__ __forceinline__ void finish4(int j, int lane, float* v, int Vm) const {
        uint32_t word = 0xffffffffu;
        if (masked_ids)
            word = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(ra, (8 * j + (lane >> 3)) * 4,
                                                                  0, 0);
        finish4w(j, lane, v, Vm, word);
    }
    // The same with the allowed word of this lane's 4 ids given (all ones for
    // rows without a mask).
    __device__ __forceinline__ void finish4w(int j, int lane, float* v, int Vm, uint32_t word) const {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float x = v[c];
            const int id = 256 * j + 4 * lane + c;
            const bool m = (id >= Vm) | !((word >> (4 * (lane & 7) + c)) & 1u) |
                           (fstop & (id != stop));
            x = m ? kNegInf : x;
            if (scale) x = __fmul_rn(x, inv_t);
            v[c] = x;
        }
    }
    // The same scores again, reloaded (for the rare passes that would
    // otherwise keep a second copy of the row in registers).
    __device__ __forceinline__ void reload4(int j, int lane, float* v, int Vm) const {
        load4(rl, lane * 16, j * 1024, v);
        if (uncond) {
            float un[4];
            load4(ru, lane * 16, j * 1024, un);
            combine4(v, un);
        }
        finish4(j, lane, v, Vm);
    }
};

// One 8-bit radix pass of the (rem+1)-th largest okey among ids < V, over
// scores reloaded vector by vector.
template <int Q>
__device__ __forceinline__ void wave_radix_pass(const RowScores& rsc, int shift, uint32_t& prefix,
                                                uint32_t& pmask, uint32_t& rem, uint32_t* hist) {
    const int lane = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 4; ++q) hist[lane * 4 + q] = 0u;
    if (lane == 0) hist[256] = 0u;
    __syncthreads();
#pragma unroll 1
    for (int j = 0; j < Q; ++j) {
        float v[4];
        rsc.reload4(j, lane, v, rsc.V);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int id = 256 * j + 4 * lane + c;
            const uint32_t k = okey(v[c]);
            const bool in = (id < rsc.V) & ((k & pmask) == prefix);
            atomicAdd(&hist[in ? (k >> shift) & 255u : 256u], 1u);  // 256: spare
        }
    }
    __syncthreads();
    uint32_t cnt[4];
    int tot = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        cnt[q] = hist[255 - (lane * 4 + q)];  // descending digits
        tot += (int)cnt[q];
    }
    int all;
    const uint32_t excl = (uint32_t)wave_excl_scan_i(tot, all);
    int digit = 0;
    uint32_t above = 0;
    const bool mine = excl <= rem && rem < excl + (uint32_t)tot;
    if (mine) {
        uint32_t run = excl;
        bool found = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (!found && run + cnt[q] > rem) {
                digit = 255 - (lane * 4 + q);
                above = run;
                found = true;
            }
            run += cnt[q];
        }
    }
    const int L = __builtin_ctzll(__ballot(mine));
    digit = __builtin_amdgcn_readlane(digit, L);
    above = (uint32_t)__builtin_amdgcn_readlane((int)above, L);
    prefix |= (uint32_t)digit << shift;
    pmask |= 255u << shift;
    rem -= above;
    __syncthreads();
}


// Calls f(std::integral_constant<int, C>) for the odd C in [c, CM] equal to
// the run-time C (terms per lane are odd, so lane-strided LDS reads of the
// sorted list fall in distinct banks).
template <int c, int CM, typename F>
__device__ __forceinline__ void with_odd_c(int C, F&& f) {
    if constexpr (c <= CM) {
        if (C == c) {
            f(std::integral_constant<int, c>{});
            return;
        }
        with_odd_c<c + 2, CM>(C, f);
    }
}

// f(rows) for each group of four list rows g = 0, 4, .. N - 4 that holds
// entries (g < n): f takes the group's first row and its row count (1 when
// the group's first row is the last one, else 4) as compile-time values.
template <int G, int N, class F>
__device__ __forceinline__ void for_row_groups(int n, F&& f) {
    if constexpr (G < N) {
        if (G < n) {
            if (G + 1 == n) f(std::integral_constant<int, G>{}, std::integral_constant<int, 1>{});
            else f(std::integral_constant<int, G>{}, std::integral_constant<int, 4>{});
        }
        for_row_groups<G + 4, N>(n, f);
    }
}

// Inclusive max-scan over the wavefront.
__device__ __forceinline__ int wave_incl_max_scan(int x) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const int t = __shfl_up(x, o, 64);
        if (lane >= o) x = max(x, t);
    }
    return x;
}

// The kept entries of a row whose top-p cutoff falls inside equal scores,
// in the order the reference's std::sort leaves them.  In: the list holds the
// n_surv survivors as sorted keys (descending score, ascending id) and the
// first n_kept are kept.  Out: the list's first n_kept entries are the
// survivors scoring above the tied score T and, of those scoring T, the ones
// std::sort puts first.  Steps: each survivor's rank (the first sorted
// position of its score) and id-order position (from a bitmap of the
// survivor ids in `keptw`, free at this point); the (rank << 16 | id) words
// in id order in the list's storage, then wave_tied_order; the entries above
// T gathered again from the row's scores.
template <int Q>
__device__ __forceinline__ void tie_order_wave(WaveSmem<Q>& sm, const RowScores& rsc, int n_surv,
                                            int n_kept, int V) {
    constexpr int R = kWaveRows;
    constexpr int WPL = (8 * Q + 63) / 64;
    const int lane = threadIdx.x;
    const int nr = (n_surv + 63) >> 6;
    const float T = desc_key_value(sm.list[n_kept - 1]);
    // ranks, ids and the bitmap of survivor ids
    for (int w = lane; w < 8 * Q; w += 64) sm.keptw[w] = 0u;
    wave_lds_sync();
    uint32_t word[R];
    int carry = 0, kT = 0;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        word[r] = 0u;
        if (r < nr) {
            const int i = r * 64 + lane;
            const bool in = i < n_surv;
            const uint64_t key = sm.list[min(i, n_surv - 1)];
            const float v = desc_key_value(key);
            const float prev = desc_key_value(sm.list[max(i - 1, 0)]);
            const bool start = in && (i == 0 || v != prev);
            const int rank = max(carry, wave_incl_max_scan(start ? i : 0));
            carry = __builtin_amdgcn_readlane(rank, 63);
            const uint32_t id = (uint32_t)key;
            word[r] = ((uint32_t)rank << 16) | id;
            kT += __popcll(__ballot(in && v > T));
            if (in) atomicOr(&sm.keptw[id >> 5], 1u << (id & 31));
        }
    }
    wave_lds_sync();
    // id-order position: survivors in the words before the id's, then in its
    // word below it; lane L holds the prefix counts of words L*WPL ..
    int base[WPL];
    {
        int loc = 0;
#pragma unroll
        for (int q = 0; q < WPL; ++q) {
            const int w = lane * WPL + q;
            base[q] = loc;
            loc += w < 8 * Q ? __popc(sm.keptw[w]) : 0;
        }
        int all;
        const int off = wave_excl_scan_i(loc, all);
#pragma unroll
        for (int q = 0; q < WPL; ++q) base[q] += off;
    }
    int pos[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        pos[r] = -1;
        if (r < nr) {
            const uint32_t id = word[r] & 0xffffu;
            const int wd = (int)(id >> 5), owner = wd / WPL, slot = wd - owner * WPL;
            int b = 0;
#pragma unroll
            for (int q = 0; q < WPL; ++q) {
                const int bq = __builtin_amdgcn_ds_bpermute(owner << 2, base[q]);
                b = q == slot ? bq : b;
            }
            const int p = b + __popc(sm.keptw[wd] & ((1u << (id & 31)) - 1u));
            pos[r] = r * 64 + lane < n_surv ? p : -1;
        }
    }
    wave_lds_sync();  // every key is read: the storage takes the words
    uint32_t* w = reinterpret_cast<uint32_t*>(sm.list);
    uint32_t* tmp = w + n_surv;
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r < nr && pos[r] >= 0) w[pos[r]] = word[r];
    wave_lds_sync();
    uint16_t* tied = reinterpret_cast<uint16_t*>(tmp);
    (void)wave_tied_order(w, tmp, n_surv, (uint32_t)kT, tied);
    // the first n_kept - kT tied ids are kept
    const int m_keep = n_kept - kT;
    uint32_t tk[R];
#pragma unroll
    for (int r = 0; r < R; ++r) tk[r] = r * 64 + lane < m_keep ? tied[r * 64 + lane] : 0u;
    wave_lds_sync();
    // the list again: the kT survivors above T from the row's scores, then
    // the kept tied ids
    int n = 0;
#pragma unroll 1
    for (int j = 0; j < Q; ++j) {
        float v[4];
        rsc.reload4(j, lane, v, V);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const bool keep = v[c] > T;
            const uint64_t m = __ballot(keep);
            if (keep) sm.list[n + mbcnt64(m)] = desc_key(v[c], (uint32_t)(256 * j + 4 * lane + c));
            n += __popcll(m);
        }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r * 64 + lane < m_keep) sm.list[kT + r * 64 + lane] = desc_key(T, tk[r]);
    wave_lds_sync();
}

// f(g, 4) for each group of four list rows g = 0, 4, .. N - 4 that holds
// entries (g < n); rows of the last group past n are the callee's to skip.
template <int G, int N, class F>
__device__ __forceinline__ void for_row_groups4(int n, F&& f) {
    if constexpr (G < N) {
        if (G < n) f(std::integral_constant<int, G>{}, std::integral_constant<int, 4>{});
        for_row_groups4<G + 4, N>(n, f);
    }
}
// ------------------------------------------------ top-p by value bins
//
// The common case of top-p (main.cpp:750-772) without sorting the survivors.
// Bins: the sort's monotone value map (descending scores -> ascending bins),
// kLeanBins of them.  The exp terms e_i = expf(s_i - mx) are placed in bin
// order by a counting sort with no order inside a bin, and the last position
// of each bin is marked.  At a bin's last position the binary64 prefix P of
// the terms is the prefix in sorted order whatever the order inside the bins
// (equal scores share a bin).  The reference's float running sum cum_i of
// q_j = fl(e_j / psum), psum its float sum in sorted order, differs from
// Y_i = P_i / S (S the binary64 total) by at most: i half-ulps of cum_i (the
// adds), 2^-24 Y_i (the divisions), and Y_i * gamma for psum itself: the
// classical bound of a recursive float sum of n non-negative terms in any
// order, (n - 1) 2^-24 / (1 - (n - 1) 2^-24), or where smaller (n - 1) half
// ulps of the binade that bound puts the float sum in, over S.  When every bin's last
// position lies certainly below or certainly at/above top_p, the crossing
// lies in the bin between the last "below" and the first "above"; that bin's
// few survivors are ranked (descending score, ascending id: std::sort's order
// for distinct scores) and certified one by one the same way.  The kept
// survivors are written to list[0, n_kept) as raw entries (score bits << 32 |
// id), in any order.  Returns false (the list restored as it was) when a
// bound straddles top_p, when equal scores straddle the cutoff, or when the
// crossing bin holds more survivors than one row: the caller then sorts and
// sums exactly.
constexpr int kLeanBins = 768;
constexpr int kLeanSpare = kLeanBins + 8;            // a spare counter per lane (past the list)
constexpr int kLeanE = kLeanSpare + 64;              // word offset of the terms
constexpr int kLeanEMax = 64 * (kWaveRows + 1) + 64; // terms read (64 lanes x C <= 17,
                                                     // in groups of 4) and the zeros past them
static_assert(kLeanE % 4 == 0, "16-byte aligned terms");
static_assert(kLeanE + kLeanEMax <= 2 * (kWaveCap + 4), "terms fit the list area");
static_assert(kLeanBins % 256 == 0, "whole uint4 groups of bins per lane");

__device__ __forceinline__ uint64_t readlane_u64(uint64_t v, int l) {
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), l);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ int wave_max_i_dpp(int x) { return -wave_min_i_dpp(-x); }

// Keeps a uniformly guarded block a branch: its instructions are not
// speculated into straight-line code that every row would then execute.
__device__ __forceinline__ void keep_branch() { asm volatile(""); }

template <int Q>
__device__ __forceinline__ bool lean_topp(WaveSmem<Q>& sm, int n_surv, float mx, float sxs,
                                          float sxc, float top_p, int& n_kept) {
    constexpr int R = kWaveRows;
    constexpr int CM = R + 1;
    constexpr int BPL = kLeanBins / 64;  // bins per lane in the scan
    // the crossing bin's survivors, ranked in keptw (8 Q words): keys, then terms
    constexpr int NBMAX = 3 * 64 <= 8 * Q ? 64 : 32;
    static_assert(3 * NBMAX <= 8 * Q, "crossing bin fits keptw");
    const int lane = threadIdx.x;
    const int nr = uni((n_surv + 63) >> 6);
    const int nv = fresh(n_surv);
    uint32_t* const cnt = reinterpret_cast<uint32_t*>(sm.list);
    uint32_t* const E = reinterpret_cast<uint32_t*>(sm.list) + kLeanE;  // term bits
    uint64_t w[R];
    // per entry: its bin (past the list: this lane's spare counter), then
    // also its slot in the bin (bits 16..), then its position in bin order
    int pos[R];
    for_row_groups4<0, R>(nr, [&](auto gc, auto cc) {
        constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
        for (int r = g; r < g + rows; ++r) {
            const int i = r * 64 + lane;
            w[r] = sm.list[i];
            const float v = __builtin_bit_cast(float, (uint32_t)(w[r] >> 32));
            const float xq = fmaxf(__fmaf_rn(v, -sxs, sxc), 0.0f);
            const float y = __fmaf_rn(__fmul_rn(__fmul_rn(xq, xq), xq), (float)(kLeanBins - 4),
                                      0x1p23f + 2.0f);
            pos[r] = i < nv ? (int)(__builtin_bit_cast(uint32_t, y) - 0x4B000000u)
                            : kLeanSpare + lane;
        }
    });
    // the list as it was, for the exact path
    auto restore = [&]() -> bool {
        __syncthreads();
        for_row_groups4<0, R>(nr, [&](auto gc, auto cc) {
            constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
            for (int r = g; r < g + rows; ++r)
                lds_store_b64_lanes(lds_offset(&sm.list[0]) + 8u * (uint32_t)(r * 64 + lane), w[r],
                                    __ballot(r * 64 + lane < nv));
        });
        __syncthreads();
        return false;
    };
    CBX_STAMP(40);
    __syncthreads();  // entries read: the list area takes the counters and the terms
    {
        uint4* c4 = reinterpret_cast<uint4*>(cnt) + (BPL / 4) * lane;
#pragma unroll
        for (int i = 0; i < BPL / 4; ++i) c4[i] = make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    CBX_STAMP(41);
    for_row_groups4<0, R>(nr, [&](auto gc, auto cc) {
        constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
        for (int r = g; r < g + rows; ++r)
            pos[r] |= (int)atomicAdd(&cnt[pos[r]], 1u) << 16;
    });
    __syncthreads();
    CBX_STAMP(42);
    // bin counts -> exclusive offsets in place; cnt[kLeanBins] = n_surv
    {
        uint4* c4 = reinterpret_cast<uint4*>(cnt) + (BPL / 4) * lane;
        uint4 w4[BPL / 4];
        uint32_t loc = 0;
#pragma unroll
        for (int i = 0; i < BPL / 4; ++i) {
            w4[i] = c4[i];
            loc += (w4[i].x + w4[i].y) + (w4[i].z + w4[i].w);
        }
        int all;
        uint32_t run = (uint32_t)wave_excl_scan_i((int)loc, all);
#pragma unroll
        for (int i = 0; i < BPL / 4; ++i) {
            uint4 o;
            o.x = run; run += w4[i].x;
            o.y = run; run += w4[i].y;
            o.z = run; run += w4[i].z;
            o.w = run; run += w4[i].w;
            c4[i] = o;
        }
        if (lane == 63) cnt[kLeanBins] = run;
    }
    __syncthreads();
    // the terms in bin order, the last position of each bin with its sign bit
    // set (a term is >= 0); zeros past the list
    E[nv + lane] = 0u;
    E[nv + 64 + lane] = 0u;
    for_row_groups4<0, R>(nr, [&](auto gc, auto cc) {
        constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
        for (int r = g; r < g + rows; ++r) {
            if (r >= nr) {  // (last group: rows past the list)
                pos[r] = 0x7fffffff;
                continue;
            }
            keep_branch();
            const bool in = r * 64 + lane < nv;
            const int b = pos[r] & 0xffff;
            const int o0 = (int)cnt[b], o1 = (int)cnt[b + 1];
            const int p = o0 + (pos[r] >> 16);
            const float v = __builtin_bit_cast(float, (uint32_t)(w[r] >> 32));
            const uint32_t eb =
                __builtin_bit_cast(uint32_t, expf_nonpos(__fsub_rn(v, mx), sm.tab));
            lds_store_b32_lanes(lds_offset(E) + 4u * (uint32_t)(in ? p : 0),
                                eb | (p + 1 == o1 ? 0x80000000u : 0u), __ballot(in));
            pos[r] = in ? p : 0x7fffffff;
        }
    });
    __syncthreads();
    CBX_STAMP(43);
    // lane l: positions [l*C, l*C + C), C odd (distinct banks), read in
    // groups of 4 (positions past C are another lane's: zeroed here)
    const int C = uni(((n_surv + 63) >> 6) | 1);
    const int b0 = lane * C;
    const uint32_t* El = E + b0;
    float t[CM];
    uint32_t mk = 0;  // bit q: position b0 + q ends a bin
    double part = 0.0;
#pragma unroll
    for (int g = 0; g < CM; g += 4) {
#pragma unroll
        for (int q = g; q < g + 4 && q < CM; ++q) t[q] = 0.0f;
        if (g < C) {
            uint32_t raw[4];
#pragma unroll
            for (int q = 0; q < 4 && g + q < CM; ++q) raw[q] = El[g + q];
#pragma unroll
            for (int q = g; q < g + 4 && q < CM; ++q) {
                const uint32_t rq = q < C ? raw[q - g] : 0u;
                t[q] = __builtin_bit_cast(float, rq & 0x7fffffffu);
                mk |= (rq >> 31) << q;
                part = __dadd_rn(part, (double)t[q]);
            }
        }
    }
    const double incl = wave_incl_scan_f64_dpp(part);
    const double S = readlane_f64(incl, 63);
    const double x0 = __dsub_rn(incl, part);
    CBX_STAMP(44);
    const double p = (double)top_p;
    // psum's relative rounding: each of its n - 1 adds of non-negative terms
    // is off by at most half an ulp of its result, whose binade is at most
    // that of the float sum, itself at most S (1 + n 2^-24 (1 + 2^-10)) (the
    // textbook bound of a recursive sum, Higham §4.2): (n - 1) 2^(E - 24) / S
    // with 2^E <= that bound's binade, at most the textbook n 2^-24
    const double inv = __ddiv_rn(1.0, S);
    const double gam_t = (double)n_surv * 0x1p-24 * (1.0 + 0x1p-10);
    const int es = __builtin_amdgcn_frexp_exp(__dmul_rn(S, 1.0 + gam_t)) - 1;
    const double gam = fmin(gam_t, __dmul_rn(__dmul_rn((double)(n_surv - 1), ldexp(1.0, es - 24)),
                                             __dmul_rn(inv, 1.0 + 0x1p-10)));
    // this lane's bound (its last index and the binade of its last Y); the
    // thresholds scaled by S (their rounding is inside the 1e-12)
    const double yl = __dmul_rn(__dadd_rn(x0, part), inv);
    const int be = __builtin_amdgcn_frexp_exp(__dmul_rn(yl, 1.0 + 0x1p-12)) - 1;
    const double err = __dadd_rn(
        __dadd_rn(__dmul_rn((double)(b0 + C - 1), ldexp(1.0, max(be, -126) - 24)),
                  __dmul_rn(yl, 0x1p-23 + gam)),
        1e-12);
    const double loP = __dmul_rn(__dsub_rn(p, err), S), hiP = __dmul_rn(__dadd_rn(p, err), S);
    // prefixes increase with the position: positions q < nlo lie certainly
    // below top_p, q >= nhi certainly at or above it (the zero terms past C
    // only repeat the last prefix: their counts fall on unmarked positions)
    int nlo = 0, nhi = 0;
    double x = x0;
#pragma unroll
    for (int g = 0; g < CM; g += 4) {
        if (g < C) {
            keep_branch();
#pragma unroll
            for (int q = g; q < g + 4 && q < CM; ++q) {
                x = __dadd_rn(x, (double)t[q]);
                nlo += x < loP ? 1 : 0;
                nhi += x < hiP ? 1 : 0;
            }
        }
    }
    const uint32_t below = mk & ((1u << nlo) - 1u);
    const uint32_t above = mk & ~((1u << nhi) - 1u);
    const bool unc = (mk & ~below & ~above) != 0u;
    if (__ballot(unc) != 0) return restore();
    const int jA = below ? b0 + 31 - (int)__builtin_clz(below) : -1;
    const int jB = above ? b0 + (int)__builtin_ctz(above) : 0x7fffffff;
    const int JA = wave_max_i_dpp(jA), JB = wave_min_i_dpp(jB);
    // (the last bin ends at Y = 1 > top_p: some bin end is certainly at or
    // above top_p unless top_p lies within the bound of 1)
    if (JB == 0x7fffffff) return restore();
    CBX_STAMP(45);
    const int s0 = JA + 1, s1 = JB + 1;
    const int nb = s1 - s0;
    uint64_t kc = 0;  // kept in the crossing bin: keys <= kc
    if (nb == 1) {
        n_kept = s1;  // below at JA, at or above at JB
    } else {
        if (nb > NBMAX) return restore();
        // the prefix at JA, summed again by its lane
        double pa = x0;
#pragma unroll
        for (int g = 0; g < CM; g += 4) {
            if (g < C) {
                keep_branch();
#pragma unroll
                for (int q = g; q < g + 4 && q < CM; ++q)
                    pa = __dadd_rn(pa, b0 + q <= JA ? (double)t[q] : 0.0);
            }
        }
        const double PA = JA >= 0 ? readlane_f64(pa, JA / C) : 0.0;
        // the bin's entries into one row (keptw: keys, then terms)
        uint64_t* bk = reinterpret_cast<uint64_t*>(sm.keptw);
        uint32_t* be4 = sm.keptw + 2 * NBMAX;
        int nbin = 0;
        for_row_groups4<0, R>(nr, [&](auto gc, auto cc) {
            constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
            for (int r = g; r < g + rows; ++r) {
                const bool inb = pos[r] >= s0 && pos[r] < s1;
                const uint64_t m = __ballot(inb);
                if (m != 0) {
                    const int at = inb ? nbin + mbcnt64(m) : 0;
                    const float v = __builtin_bit_cast(float, (uint32_t)(w[r] >> 32));
                    lds_store_b64_lanes(lds_offset(bk) + 8u * (uint32_t)at,
                                        desc_key(v, (uint32_t)w[r]), m);
                    lds_store_b32_lanes(lds_offset(be4) + 4u * (uint32_t)at,
                                        E[inb ? pos[r] : 0] & 0x7fffffffu, m);
                    nbin += __popcll(m);
                }
            }
        });
        __syncthreads();
        const bool mine = lane < nb;
        const uint64_t key = mine ? bk[lane] : ~0ull;
        const uint32_t em = mine ? be4[lane] : 0u;
        int rank = 0;
        for (int tt = 0; tt < nb; ++tt) rank += readlane_u64(key, tt) < key ? 1 : 0;
        __syncthreads();  // read: the row takes rank order
        lds_store_b64_lanes(lds_offset(bk) + 8u * (uint32_t)(mine ? rank : 0), key,
                            __ballot(mine));
        lds_store_b32_lanes(lds_offset(be4) + 4u * (uint32_t)(mine ? rank : 0), em,
                            __ballot(mine));
        __syncthreads();
        const uint64_t kr = mine ? bk[lane] : ~0ull;
        const double er = mine ? (double)__builtin_bit_cast(float, be4[lane]) : 0.0;
        const double y = __dmul_rn(__dadd_rn(PA, wave_incl_scan_f64_dpp(er)), inv);
        const int bi = __builtin_amdgcn_frexp_exp(__dmul_rn(y, 1.0 + 0x1p-12)) - 1;
        const double erri = __dadd_rn(
            __dadd_rn(__dmul_rn((double)(s0 + lane), ldexp(1.0, max(bi, -126) - 24)),
                      __dmul_rn(y, 0x1p-23 + gam)),
            1e-12);
        const uint64_t mlo = __ballot(mine && y < __dsub_rn(p, erri));
        const uint64_t mhi = __ballot(mine && y >= __dadd_rn(p, erri));
        const int f = __builtin_ctzll(~mlo);  // first position not certainly below
        if (f >= nb || !((mhi >> f) & 1ull)) return restore();
        // equal scores straddling the cutoff: std::sort's order decides
        if (f + 1 < nb && desc_key_value(readlane_u64(kr, f)) ==
                              desc_key_value(readlane_u64(kr, f + 1)))
            return restore();
        kc = readlane_u64(kr, f);
        n_kept = s0 + f + 1;
    }
    CBX_STAMP(46);
    __syncthreads();  // terms and counters read: the list takes the kept entries
    int nk = 0;
    for_row_groups4<0, R>(nr, [&](auto gc, auto cc) {
        constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
        for (int r = g; r < g + rows; ++r) {
            // kept: positions before the crossing bin, and of that bin its
            // one survivor or those up to the cutoff key
            bool kp = pos[r] < (nb == 1 ? s1 : s0);
            if (nb > 1 && pos[r] >= s0 && pos[r] < s1) {
                const float v = __builtin_bit_cast(float, (uint32_t)(w[r] >> 32));
                kp = desc_key(v, (uint32_t)w[r]) <= kc;
            }
            const uint64_t m = __ballot(kp);
            lds_store_b64_lanes(lds_offset(&sm.list[0]) + 8u * (uint32_t)(nk + mbcnt64(m)), w[r], m);
            nk += __popcll(m);
        }
    });
    __syncthreads();
    return true;
}

// ------------------------------------------------- chunked rows (V > 8448)
//
// Rows too long to hold in registers (V <= 256 Q with Q = 128: 32768 ids) are
// read once, in chunks of kChunkV vectors (256 kChunkV ids) streamed through
// registers, the next chunk's loads in flight while one is scanned.  A lower
// bound tau of the top-k threshold rises as the row is read: every finite
// score >= tau goes on the list (raw entries, in the scan order the one-pass
// kernel lists its survivors in), and when the list has no room for the next
// vector's candidates, tau rises to the smallest entry of the bin holding the
// list's (k+1)-th largest, less 1e-10 (so it stays at or below the row's
// (k+1)-th largest, and below that threshold's nudge), and the entries below
// it leave the list.  At the end the list holds every score >= tau, hence
// the row's (k+1)-th largest: the threshold is taken on it as the reference
// takes it (nth_element, keep s > thr, the -1e-10 nudge when fewer than k are
// above; main.cpp:741-748), and the entries above it are the survivors.
// Rows holding NaN or +inf, and rows whose candidates do not fit the list,
// are marked to overflow (the redo pass samples them at full capacity).
constexpr int kChunkV = 8;
constexpr int kChunkBins = 256;

// W2: the row's chunks split over two waves of one workgroup (smv: their two
// WaveSmem, wv: this wave).  Wave 1 scans the second half into its own list
// with wave-local synchronisation, publishes its count, maximum and flags and
// meets wave 0 at the row's one workgroup barrier, then leaves (n_surv = -1:
// the caller returns); wave 0 scans the first half, merges wave 1's entries
// at or above its running bound tau (the global top k + 1 scores are among
// them: each half's tau is at most that half's (k+1)-th largest score, so at
// most the row's), and goes on alone.  Every early return of either wave
// comes after that barrier.
template <int Q, bool W2 = false>
__device__ __forceinline__ void chunk_front(WaveSmem<Q>& sm, const RowScores& rsc, int lane,
                                            int k, bool use_topk, float (&cur)[4 * kChunkV],
                                            float& hi, float& lo, bool& have_lo, bool& bad,
                                            float& thr, int& n_surv, WaveSmem<Q>* smv = nullptr,
                                            int wv = 0) {
    static_assert(kChunkBins == 4 * 64, "four bins per lane");
    static_assert(8 * Q >= kWaveCap, "the list's values fit the kept-bitmap words");
    const int V = rsc.V;
    const int nch = (V + 256 * kChunkV - 1) / (256 * kChunkV);
    // this wave's chunks [cb, ce)
    const int cb = W2 && wv == 1 ? (nch + 1) / 2 : 0;
    const int ce = W2 && wv == 0 ? (nch + 1) / 2 : nch;
    // LDS ordering among this wave's lanes (one wave per workgroup: the
    // workgroup barrier; two: a wave-local fence, the other wave's storage
    // being its own)
    auto sync = [&]() {
        if constexpr (W2) wave_lds_sync();
        else __syncthreads();
    };
    const uint32_t list0 = lds_offset(&sm.list[0]);
    uint32_t* const hist = sm.keptw;  // free until the filters: bins, then candidates
    auto val = [](uint64_t w) { return __builtin_bit_cast(float, (uint32_t)(w >> 32)); };
    float tau = kNegInf;
    int cnt = 0;
    bool over = false;
    bool nfb = false;  // a NaN or +inf score seen by this lane
    hi = kNegInf;
    thr = kNegInf;
    if (rsc.fstop) {
        // forced stop: every id but the stop token is -inf (as the one-pass
        // kernel's masks make it), so that token's score alone decides; the
        // chunks already requested are not read (and wave 1 has nothing to do)
        if constexpr (W2) {
            if (wv == 1) {
                n_surv = -1;
                return;
            }
        }
        float x = kNegInf;
        if (rsc.stop >= 0 && rsc.stop < V) {
            x = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsc.rl, rsc.stop * 4, 0, 0));
            const uint32_t w = rsc.masked_ids
                                   ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsc.ra, (rsc.stop >> 5) * 4, 0, 0)
                                   : 0xffffffffu;
            x = ((w >> (rsc.stop & 31)) & 1u) ? x : kNegInf;
            if (rsc.scale) x = __fmul_rn(x, rsc.inv_t);
        }
        hi = x;
        bad = x != x || x == kPosInf;
        if (bad) {
            n_surv = kWaveCap + 1;
            return;
        }
        const bool fin = x != kNegInf;
        if (lane == 0 && fin)
            sm.list[0] = ((uint64_t)__builtin_bit_cast(uint32_t, x) << 32) | (uint32_t)rsc.stop;
        lo = fin ? x : kPosInf;
        have_lo = true;
        n_surv = fin ? 1 : 0;
        sync();
        return;
    }
    const uint32_t shl = 4u * (uint32_t)(lane & 7);  // this lane's 4 ids in its mask word
    // bins of the list's values over [lmn, lmx]: bin(v) = floor(fma(v, bs, nb)),
    // monotone in v; the bin holding rank k from the top, and the entries above it
    auto rank_bin = [&](float bs, float nb, int& bsel, int& above_bins) {
        auto bin = [&](float v) {
            return (int)__builtin_amdgcn_fmed3f(__fmaf_rn(v, bs, nb), 0.0f, (float)(kChunkBins - 1));
        };
#pragma unroll
        for (int q = 0; q < 4; ++q) hist[4 * lane + q] = 0u;
        sync();
        for (int i = lane; i < cnt; i += 64) atomicAdd(&hist[bin(val(sm.list[i]))], 1u);
        sync();
        uint32_t c4[4];
        int tot = 0;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            c4[q] = hist[kChunkBins - 1 - (4 * lane + q)];  // descending bins
            tot += (int)c4[q];
        }
        int all;
        const int excl = wave_excl_scan_i(tot, all);
        const bool mine = excl <= k && k < excl + tot;
        int b = 0, ab = 0, run = excl;
        bool found = false;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (mine && !found && run + (int)c4[q] > k) {
                b = kChunkBins - 1 - (4 * lane + q);
                ab = run;
                found = true;
            }
            run += (int)c4[q];
        }
        const int L = __builtin_ctzll(__ballot(mine));
        bsel = __builtin_amdgcn_readlane(b, L);
        above_bins = __builtin_amdgcn_readlane(ab, L);
        sync();  // bin counts read
    };
    auto list_range = [&](float& lmn, float& lmx) {
        float a0 = kPosInf, a1 = kNegInf;
        for (int i = lane; i < cnt; i += 64) {
            const float v = val(sm.list[i]);
            a0 = fminf(a0, v);
            a1 = fmaxf(a1, v);
        }
        lmn = wave_min_dpp(a0);
        lmx = wave_max_dpp(a1);
    };
    // entries v with keep(v) moved down in place, in order
    auto compact = [&](auto&& keep) {
        int nn = 0;
        for (int base = 0; base < cnt; base += 64) {
            const int i = base + lane;
            const uint64_t w = i < cnt ? sm.list[i] : 0ull;
            const uint64_t m = __ballot(i < cnt && keep(val(w)));
            lds_store_b64_lanes(list0 + 8u * (uint32_t)(nn + ballot_rank(m)), w, m);
            nn += __popcll(m);
        }
        cnt = nn;
        sync();
    };
    // tau raised as far as the list's bins allow; false when it cannot rise
    auto prune = [&]() -> bool {
        if (!use_topk || cnt <= k) return false;
        float lmn, lmx;
        list_range(lmn, lmx);
        const float bs = __fdiv_rn((float)kChunkBins, __fsub_rn(lmx, lmn));
        if (!(lmx > lmn) || !(bs < kPosInf)) return false;
        const float nb = -__fmul_rn(lmn, bs);
        int bsel, above_bins;
        rank_bin(bs, nb, bsel, above_bins);
        float mn = kPosInf;
        for (int i = lane; i < cnt; i += 64) {
            const float v = val(sm.list[i]);
            const int b = (int)__builtin_amdgcn_fmed3f(__fmaf_rn(v, bs, nb), 0.0f,
                                                       (float)(kChunkBins - 1));
            if (b >= bsel) mn = fminf(mn, v);
        }
        const float tn = __fsub_rn(wave_min_dpp(mn), 1e-10f);
        if (!(tn > tau)) return false;
        tau = tn;
        compact([&](float v) { return v >= tn; });
        return true;
    };
    // a ring of kRing chunks: kRing - 1 in flight (scores and mask words)
    // while one is scanned, the slot refilled as soon as it is scanned
    constexpr int kRing = 3;
    float buf[kRing][4 * kChunkV];
    uint32_t mw[kRing][kChunkV];
    auto issue = [&](int c, float (&bv)[4 * kChunkV], uint32_t (&wv)[kChunkV]) {
        if (c >= ce) return;
#pragma unroll
        for (int j = 0; j < kChunkV; ++j) load4(rsc.rl, lane * 16, (c * kChunkV + j) * 1024, &bv[4 * j]);
        if (rsc.masked_ids) {
#pragma unroll
            for (int j = 0; j < kChunkV; ++j)
                wv[j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                    rsc.ra, (8 * (c * kChunkV + j) + (lane >> 3)) * 4, 0, 0);
        }
    };
    auto scan = [&](int c, float (&bv)[4 * kChunkV], const uint32_t (&wv)[kChunkV]) {
#pragma unroll
        for (int j = 0; j < kChunkV; ++j) {
            // masks, padding (the last vectors only), temperature: finish4's
            // operations with the lane's mask bits shifted once per vector
            const int jj = c * kChunkV + j;
            uint32_t bits = rsc.masked_ids ? (wv[j] >> shl) : 0xfu;
            // ids past V: the low min(4, max(0, V - id0)) bits stay (one
            // mask per vector, not a compare per score)
            const int nin = min(max(V - (256 * jj + 4 * lane), 0), 4);
            bits &= (1u << nin) - 1u;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                // bit q of `bits` as an all-ones or zero word, then a bitwise
                // select with -inf (no per-score condition register)
                const uint32_t m = (uint32_t)((int32_t)(bits << (31 - q)) >> 31);
                float x = __builtin_bit_cast(
                    float, (__builtin_bit_cast(uint32_t, bv[4 * j + q]) & m) | (0xff800000u & ~m));
                if (rsc.scale) x = __fmul_rn(x, rsc.inv_t);
                bv[4 * j + q] = x;
                nfb = nfb || __builtin_amdgcn_classf(x, 0x203);  // NaN or +inf
                hi = fmaxf(hi, x);
            }
        }
#pragma unroll
        for (int j = 0; j < kChunkV; ++j) {
            if (cnt + 256 > kWaveCap && (!prune() || cnt + 256 > kWaveCap)) {
                over = true;
                break;
            }
            // finite scores >= tau (-inf and NaN never pass)
            const float t2 = tau == kNegInf ? -3.40282347e38f : tau;
            const int id0 = 256 * (c * kChunkV + j) + 4 * lane;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float v = bv[4 * j + q];
                const uint64_t m = __ballot(v >= t2);
                if (m) {
                    lds_store_b64_lanes(
                        list0 + 8u * (uint32_t)(cnt + ballot_rank(m)),
                        ((uint64_t)__builtin_bit_cast(uint32_t, v) << 32) | (uint32_t)(id0 + q), m);
                    cnt += __popcll(m);
                }
            }
        }
    };
#pragma unroll
    for (int e = 0; e < 4 * kChunkV; ++e) buf[0][e] = cur[e];  // chunk cb, loaded by the caller
    if (rsc.masked_ids) {
#pragma unroll
        for (int j = 0; j < kChunkV; ++j)
            mw[0][j] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                rsc.ra, (8 * (cb * kChunkV + j) + (lane >> 3)) * 4, 0, 0);
    }
#pragma unroll
    for (int r = 1; r < kRing; ++r) issue(cb + r, buf[r], mw[r]);
#pragma unroll 1
    for (int c0 = cb; c0 < ce && !over; c0 += kRing) {
#pragma unroll
        for (int r = 0; r < kRing; ++r) {
            if (c0 + r < ce && !over) {
                scan(c0 + r, buf[r], mw[r]);
                issue(c0 + r + kRing, buf[r], mw[r]);
            }
        }
    }
    sync();
    bad = __ballot(nfb) != 0;
    hi = wave_max_dpp(hi);
    if constexpr (W2) {
        // wave 1 publishes (its list stays in its own storage), both waves
        // meet once, wave 1 leaves; wave 0 takes the second half's entries
        // at or above its tau into its list, pruning as it fills
        WaveSmem<Q>& s1 = smv[1];
        if (wv == 1 && lane == 0) {
            s1.h.seen[0] = over ? 0xffffffffu : (uint32_t)cnt;
            s1.h.seen[1] = __builtin_bit_cast(uint32_t, hi);
            s1.h.seen[2] = bad ? 1u : 0u;
        }
        __syncthreads();
        if (wv == 1) {
            n_surv = -1;
            return;
        }
        const uint32_t c1w = s1.h.seen[0];
        hi = fmaxf(hi, __builtin_bit_cast(float, s1.h.seen[1]));
        bad = bad || s1.h.seen[2] != 0u;
        over = over || c1w == 0xffffffffu;
        if (!bad && !over) {
            const int c1 = (int)c1w;
            for (int base = 0; base < c1; base += 64) {
                if (cnt + 64 > kWaveCap && (!prune() || cnt + 64 > kWaveCap)) {
                    over = true;
                    break;
                }
                const int i = base + lane;
                const uint64_t w = i < c1 ? s1.list[i] : 0ull;
                const float t2 = tau == kNegInf ? -3.40282347e38f : tau;
                const uint64_t m = __ballot(i < c1 && val(w) >= t2);
                lds_store_b64_lanes(list0 + 8u * (uint32_t)(cnt + ballot_rank(m)), w, m);
                cnt += __popcll(m);
            }
            sync();
        }
    }
    if (bad || over) {
        n_surv = kWaveCap + 1;  // more than any capacity: the redo pass takes the row
        return;
    }
    if (use_topk && cnt > k) {
        // the (k+1)-th largest: its bin, then that bin's entries ranked
        float lmn, lmx;
        list_range(lmn, lmx);
        const float bs = __fdiv_rn((float)kChunkBins, __fsub_rn(lmx, lmn));
        const bool binned = lmx > lmn && bs < kPosInf;
        const float nb = binned ? -__fmul_rn(lmn, bs) : 0.0f;
        int bsel = 0, above_bins = 0;
        if (binned) rank_bin(bs, nb, bsel, above_bins);
        float* const cand = reinterpret_cast<float*>(hist);
        int nc = 0;
        for (int base = 0; base < cnt; base += 64) {
            const int i = base + lane;
            const float v = i < cnt ? val(sm.list[i]) : 0.0f;
            const int b = binned ? (int)__builtin_amdgcn_fmed3f(__fmaf_rn(v, bs, nb), 0.0f,
                                                                (float)(kChunkBins - 1))
                                 : 0;
            const bool in = i < cnt && b == bsel;
            const uint64_t m = __ballot(in);
            if (in) cand[nc + ballot_rank(m)] = v;
            nc += __popcll(m);
        }
        sync();
        const int rem = k - above_bins;  // 0 <= rem < nc
        float tv = kNegInf;
        int tgt = 0;
        bool hit = false;
        for (int c0 = lane; c0 < nc; c0 += 64) {
            const float v = cand[c0];
            int gt = 0, ge = 0;
            for (int t = 0; t < nc; ++t) {
                const float w = cand[t];
                gt += (w > v) ? 1 : 0;
                ge += (w >= v) ? 1 : 0;
            }
            if (gt <= rem && rem < ge) {
                tv = v;
                tgt = gt;
                hit = true;
            }
        }
        const int L2 = __builtin_ctzll(__ballot(hit));
        thr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, tv), L2));
        const int above = above_bins + __builtin_amdgcn_readlane(tgt, L2);
        if (above < k) thr = __fsub_rn(thr, 1e-10f);
        sync();  // candidates read
        const float th = thr;
        compact([&](float v) { return v > th; });
    } else {
        // every finite score of the row is on the list (tau never rose):
        // all of them survive (at most k, or no top-k), and the smallest is lo
        float lmx;
        list_range(lo, lmx);
        have_lo = true;
    }
    n_surv = cnt;
}

// ------------------------------------------------------------------ kernel

template <int Q, int JT, bool CH = false, bool W2 = false>
__global__ __launch_bounds__(W2 ? 128 : 64) __attribute__((amdgpu_waves_per_eu(WAVE_WPE))) void sample_rows_wave(
    KernelArgs a) {
    static_assert(!W2 || CH, "two waves per row: chunked rows only");
    // W2: two waves per row, each with its own storage (chunk_front)
    __shared__ WaveSmem<Q> smv[W2 ? 2 : 1];
    // (readfirstlane: the compiler then knows it is the same across the wave,
    // so branches on it are uniform)
    const int wv = W2 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;
    WaveSmem<Q>& sm = smv[wv];
    constexpr int EPL = 4 * Q;  // scores per lane
    constexpr int R = kWaveRows;
    const int lane = W2 ? (int)(threadIdx.x & 63u) : (int)threadIdx.x;
    const int64_t g = xcd_spread(blockIdx.x, gridDim.x, a.n_rows);
    const int step = (int)(g / a.n_rows), row = (int)(g % a.n_rows);
    const int V = a.n_vocab;
    const int W = (V + 31) >> 5;
    const int cap = min(a.cap, kWaveCap);
    const cbx_params P = a.params[row];
    const int64_t rs = (int64_t)step * a.n_rows + row;
    CBX_STAMP(0);

    // ---- load: 16-byte buffer loads bounded at V floats (main.cpp:733) ----
    // The range check of a raw buffer load is per dword, so the vector that
    // straddles V returns its in-range words and zeros (masked below).
    const uint32_t* arow = a.allowed ? a.allowed + (int64_t)row * a.ld_allowed : nullptr;
    RowScores rsc;
    rsc.rl = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(a.logits + rs * a.ld_logits),
                                               (short)0, V * 4, kBufferWord3);
    rsc.uncond = a.uncond != nullptr;
    rsc.ru = rsc.rl;
    if (rsc.uncond)
        rsc.ru = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(a.uncond + rs * a.ld_logits), (short)0, V * 4, kBufferWord3);
    rsc.masked_ids = arow != nullptr;
    rsc.ra = rsc.rl;
    if (arow)
        rsc.ra = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(arow), (short)0, W * 4,
                                                   kBufferWord3);
    rsc.fstop = a.force_stop && a.force_stop[rs];
    rsc.scale = P.temp > 0.0f && P.temp != 1.0f;
    rsc.cfg_w = P.cfg_weight;
    rsc.inv_t = __fdiv_rn(1.0f, P.temp);
    rsc.V = V;
    rsc.stop = a.stop_token;
    const int hlen = a.history ? (int)min((int64_t)a.history_len[row], a.ld_history) : 0;
    const bool use_pen = P.repeat_penalty != 1.0f && hlen > 0;
    const int32_t* hrow = a.history + (int64_t)row * a.ld_history;
    // Loads in the order they are needed (memory reads return in order): the
    // exp table's words, the row, then the history's first 1024 ids, so no
    // wait comes between them and one wait covers the row and the ids.
    const uint64_t tabv = kExp2TabDev.t[lane & 31];
    float s[CH ? 1 : EPL];
    float cur[CH ? 4 * kChunkV : 1];  // chunked rows: the chunk being read
    if constexpr (!CH) {
#pragma unroll
        for (int j = 0; j < Q; ++j) load4(rsc.rl, lane * 16, j * 1024, &s[4 * j]);
        if (rsc.uncond) {
            // CFG rows: the uncond vectors stream through a ring of UD register
            // quads, UD - 1 loads ahead of the combine (the waits are in order)
            constexpr int UD = 3;
            float un[UD][4];
#pragma unroll
            for (int j = 0; j < UD - 1; ++j) load4(rsc.ru, lane * 16, j * 1024, un[j]);
#pragma unroll
            for (int j = 0; j < Q; ++j) {
                if (j + UD - 1 < Q) load4(rsc.ru, lane * 16, (j + UD - 1) * 1024, un[(j + UD - 1) % UD]);
                rsc.combine4(&s[4 * j], un[j % UD]);
            }
        }
    } else {
        // the wave's first chunk (chunk 0: ids 0 .. 256 kChunkV - 1; wave 1 of
        // two: the second half's first); the rest stream in as it is scanned
        const int nch = (V + 256 * kChunkV - 1) / (256 * kChunkV);
        const int cb = W2 && wv == 1 ? (nch + 1) / 2 : 0;
#pragma unroll
        for (int j = 0; j < kChunkV; ++j) load4(rsc.rl, lane * 16, (cb * kChunkV + j) * 1024, &cur[4 * j]);
    }
    // ---- history ids -> seen bitmap (main.cpp:775) ----
    // Loads past the history read 0 and are masked out.
    constexpr int HB = 16;  // ids per lane per batch: 1024 per pass
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<int32_t*>(hrow), (short)0, hlen * 4, kBufferWord3);
    int hid[HB];
    const bool build_seen = use_pen && wv == 0;  // (wave 1 of two only scans)
    if (build_seen) {
#pragma unroll
        for (int u = 0; u < HB; ++u)
            hid[u] = __builtin_amdgcn_raw_buffer_load_b32(rh, (u * 64 + lane) * 4, 0, 0);
    }
    // the draw's uniform, while the loads are in flight (scalar work)
    double u_draw = 0.0;
    if (a.draw_mode == CBX_DRAW_PHILOX) {
        const uint64_t sid = a.stream_ids ? a.stream_ids[row] : (uint64_t)row;
        u_draw = philox_uniform(a.seed, sid, a.step0 + (uint64_t)step);
    } else {
        u_draw = a.uniforms[rs];
    }
    u_draw = fresh_d(u_draw);
    if (lane < 32) sm.tab[lane] = tabv;
    for (int w = lane; w < 8 * Q; w += 64) sm.h.seen[w] = 0u;
    if (build_seen) {
        for (int b0 = 0; b0 < hlen; b0 += HB * 64) {
            if (b0 > 0) {
#pragma unroll
                for (int u = 0; u < HB; ++u)
                    hid[u] = __builtin_amdgcn_raw_buffer_load_b32(rh, (b0 + u * 64 + lane) * 4, 0, 0);
            }
#pragma unroll
            for (int u = 0; u < HB; ++u) {
                const int t = hid[u];
                const bool ok = b0 + u * 64 + lane < hlen && t >= 0 && t < V;
                if (b0 + u * 64 < hlen)  // uniform: batches past the history are skipped
                    lds_or_b32_lanes(lds_offset(&sm.h.seen[0]) + ((uint32_t)(t >> 5) << 2),
                                     1u << (t & 31), __ballot(ok));
            }
        }
    }
    // ---- masks and temperature (main.cpp:735-738) ----
    CBX_STAMP(1);
    // Masked rows first set the ids the mask drops to -inf (the allowed row
    // is staged in LDS, in the kept-bitmap words that are cleared again after).
    // Then every row takes the same pass: only ids >= V are padding, which
    // this instantiation meets in vectors j >= JT alone (V > 256*JT); the
    // others need 4 operations per score and no predicate.
    [[maybe_unused]] const bool plain = !rsc.masked_ids && !rsc.fstop;
    // lo, the smallest finite score, is taken only where a path needs it
    // (have_lo): the common one bins from the mean of vector 0 and sorts
    // from the top-k threshold
    float lo = kPosInf, hi = kNegInf;
    bool have_lo = false;
    [[maybe_unused]] float msum = 0.0f;  // this lane's 4 scores of vector 0 (padding-free when JT >= 1)
    bool bad = false;                     // NaN/+inf seen
    [[maybe_unused]] bool neg_inf = false;  // -inf among unmasked scores
    uint32_t flags = 0u;
    // The scores again, reloaded four at a time, for the passes after the
    // fast top-k path (so the register copy of the row need not stay live).
    auto each_score = [&](auto&& f) {
#pragma unroll 1
        for (int j = 0; j < Q; ++j) {
            float v[4];
            rsc.reload4(j, lane, v, V);
#pragma unroll
            for (int c = 0; c < 4; ++c) f(v[c], 256 * j + 4 * lane + c);
        }
    };

    // lo from scores reloaded (where the registers have been given up, and
    // for chunked rows)
    auto lo_from_memory = [&]() {
        if (have_lo) return;
        float m = kPosInf;
        each_score([&](float v, int) { m = fminf(m, v == kNegInf ? kPosInf : v); });
        lo = wave_min_dpp(m);
        have_lo = true;
    };

    // ---- top-k (main.cpp:740-748) ----
    const int k = P.top_k;
    const bool use_topk = k > 0 && k < V;
    float thr = kNegInf;  // survivors: s > thr
    int n_surv = -1;      // >= 0 once the survivor list is built
    if constexpr (!CH) {
        if (!plain) {
            if (rsc.masked_ids)
                for (int w = lane; w < W; w += 64)
                    sm.keptw[w] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rsc.ra, w * 4, 0, 0);
            __syncthreads();
#pragma unroll
            for (int j = 0; j < Q; ++j) {
                const uint32_t word = rsc.masked_ids ? sm.keptw[8 * j + (lane >> 3)] : 0xffffffffu;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int id = 256 * j + 4 * lane + c;
                    const bool m = !((word >> (4 * (lane & 7) + c)) & 1u) |
                                   (rsc.fstop & (id != rsc.stop));
                    s[4 * j + c] = m ? kNegInf : s[4 * j + c];
                }
            }
            __syncthreads();
        }
        {
            // acc = sum of the products of score pairs: finite while every
            // unmasked score is finite, NaN or infinite once one is NaN or
            // infinite (or, for huge scores, when the sum overflows: the check
            // below then finds no such score).  Vectors j >= JT may hold padding.
            float acc = 0.0f;
            const int Vm = fresh(V);
            auto pass = [&](auto scaled) {
                msum = 0.0f;
#pragma unroll
                for (int j = 0; j < Q; ++j) {
                    float w[4];
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        w[c] = s[4 * j + c];
                        if (decltype(scaled)::value) w[c] = __fmul_rn(w[c], rsc.inv_t);
                    }
                    if (j < JT) {
                        if (j == 0) msum = __fadd_rn(__fadd_rn(w[0], w[1]), __fadd_rn(w[2], w[3]));
                        acc = __fmaf_rn(w[0], w[1], acc);
                        acc = __fmaf_rn(w[2], w[3], acc);
                        // running value first: one 3-input max per pair
                        hi = fmaxf(fmaxf(hi, w[0]), w[1]);
                        hi = fmaxf(fmaxf(hi, w[2]), w[3]);
                    } else {
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            const bool pad = 256 * j + 4 * lane + c >= Vm;
                            acc = __fmaf_rn(pad ? 0.0f : w[c], 0.0f, acc);
                            w[c] = pad ? kNegInf : w[c];
                            hi = fmaxf(hi, w[c]);
                        }
                    }
#pragma unroll
                    for (int c = 0; c < 4; ++c) s[4 * j + c] = w[c];
                }
            };
            if (rsc.scale) pass(std::true_type{});
            else pass(std::false_type{});
            const bool spec = __ballot(!(__builtin_fabsf(acc) < kPosInf)) != 0;
            if (spec) {
                // rare: tell NaN/+inf (reported) from -inf logits, and take the
                // minimum over finite scores only
                int nf = 0, ni = 0;
                lo = kPosInf;
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const float v = s[e];
                    const bool pad = (e >> 2) >= JT && 256 * (e >> 2) + 4 * lane + (e & 3) >= Vm;
                    nf |= (!pad && (v != v || v == kPosInf)) ? 1 : 0;
                    ni |= (!pad && v == kNegInf) ? 1 : 0;
                    lo = fminf(lo, v == kNegInf ? kPosInf : v);
                }
                bad = wave_sum_dpp(nf) != 0;
                neg_inf = wave_sum_dpp(ni) != 0;
                lo = wave_min_dpp(lo);
                have_lo = true;
            }
        }
        hi = wave_max_dpp(hi);
        flags = bad ? CBX_INFO_NONFINITE : 0u;
        CBX_STAMP(2);
        // lo from the scores in registers (every unmasked score finite here:
        // rows holding -inf, NaN or +inf took it above) ...
        auto lo_from_registers = [&]() {
            if (have_lo) return;
            float m = kPosInf;
#pragma unroll
            for (int e = 0; e < EPL; ++e) m = fminf(m, s[e] == kNegInf ? kPosInf : s[e]);  // padding
            lo = wave_min_dpp(m);
            have_lo = true;
        };
        if (use_topk) {
            int above = 0;
            bool done = false;
            // Plain rows: y(v) = fma(v, bs, c0) lands in [2^23, 2^23 + NB) for
            // every score in [lo, hi] (checked at both ends; y is monotone), where
            // a float is an integer: bin(v) = bits(y) - bits(2^23) is
            // non-decreasing in v and costs two operations per score.  The
            // V..256Q padding (-inf) is raised to bin 0 and taken off its count.
            // The bins cover [hlo, hi]: for k < V/4 the (k+1)-th largest score
            // lies, for any ordinary row, above the mean of the 256 scores of
            // vector 0, so the bins start there (half the atomics, bins twice as
            // fine).  Scores below hlo land in bins 0..1 (some, within two bins
            // of hlo) or in a dump word of their own lane below the histogram
            // (y below 2^23, where floats step by 1/2: y = 2^23 - (l + 1)/2 has
            // bits(y) - bits(2^23) = -(l + 1)), as does the padding (-inf).  So
            // the counts of bins >= 2 are exact, and a row whose rank-k bin is
            // below 2 (or holding fewer than k + 1 binned scores) takes the
            // full-range pass further down.
            const bool partial = JT >= 1 && 4 * k < V && !bad && !neg_inf;
            if (!partial) lo_from_registers();
            const float hlo = partial ? __fmul_rn(wave_sum_f_dpp(msum), 1.0f / 256.0f) : lo;
            const float hrange = __fsub_rn(hi, hlo);
            const float bs = __fdiv_rn((float)(kWaveBins - 4), hrange);
            const float c0 = __fsub_rn(0x1p23f + 2.0f, __fmul_rn(hlo, bs));
            const bool bins_fit = __fmaf_rn(hlo, bs, c0) >= 0x1p23f &&
                                  __fmaf_rn(hi, bs, c0) <= 0x1p23f + (float)(kWaveBins - 1);
            if (!bad && !neg_inf && hrange > 0.0f && bs < kPosInf && bins_fit) {
                uint32_t* hist = sm.khist() + 64;  // words -64..-1: the lanes' dump words
                const float dump_y = 0x1p23f - 0.5f * (float)(lane + 1);
#pragma unroll
                for (int q = 0; q < kWaveBins / 64; ++q) hist[lane * (kWaveBins / 64) + q] = 0u;
                __syncthreads();
#pragma unroll
                for (int e = 0; e < EPL; ++e) {
                    const float y = fmaxf(__fmaf_rn(s[e], bs, c0), dump_y);
                    atomicAdd(&hist[(int)(__builtin_bit_cast(uint32_t, y) - 0x4B000000u)], 1u);
                }
                __syncthreads();
                CBX_STAMP(16);
                // Lane l owns the 16 bins kWaveBins-1-16l .. kWaveBins-16-16l
                // (descending scores), contiguous in LDS: their total from four
                // 16-byte reads.
                static_assert(kWaveBins == 1024, "16 bins per lane");
                int tot;
                {
                    const uint4* h4 = reinterpret_cast<const uint4*>(hist) + (kWaveBins / 4 - 4 - 4 * lane);
                    uint32_t sum = 0;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const uint4 w = h4[i];
                        sum += (w.x + w.y) + (w.z + w.w);
                    }
                    tot = (int)sum;
                }
                int n_fin;
                const int excl = wave_excl_scan_i(tot, n_fin);
                if (n_fin <= k) {
                    if (!partial) {
                        thr = kNegInf;  // at most k finite scores: nothing is removed
                        above = n_fin;
                        done = true;
                    }  // else fewer than k + 1 scores above hlo: the full-range pass
                } else {
                    // the lane whose bins hold rank k; lanes 0..15 take its bins
                    // (q-th largest first) and scan their counts
                    const int L = __builtin_ctzll(__ballot(excl <= k && k < excl + tot));
                    const int exclL = __builtin_amdgcn_readlane(excl, L);
                    const int bq = kWaveBins - 1 - (16 * L + (lane & 15));
                    const int cq = (int)hist[bq];
                    int inc = cq;  // inclusive scan inside lanes 0..15 (row 0)
                    inc += dpp_i<0x111, 0xf>(0, inc);
                    inc += dpp_i<0x112, 0xf>(0, inc);
                    inc += dpp_i<0x114, 0xf>(0, inc);
                    inc += dpp_i<0x118, 0xf>(0, inc);
                    const int Qh = __builtin_ctzll(__ballot(lane < 16 && exclL + inc > k));
                    const int bsel = kWaveBins - 1 - (16 * L + Qh);
                    const int nsel = __builtin_amdgcn_readlane(cq, Qh);
                    const int above_bins = exclL + __builtin_amdgcn_readlane(inc, Qh) - nsel;
                    // Score boundaries of the selected bin: B0 = least float with
                    // bin >= bsel, B1 = least float with bin >= bsel + 1 (+inf past
                    // the top bin).  bin(v) >= b  <=>  fma(v, bs, c0) >= 2^23 + b,
                    // which (the fma rounding to integers) holds from about
                    // v*bs + c0 = 2^23 + b - 1/2 on; probed over 64 consecutive
                    // floats around that root.
                    auto boundary = [&](int b, float& B) -> bool {
                        const float tb = 0x1p23f + (float)b;
                        const float v0 = (float)(((double)tb - 0.5 - (double)c0) / (double)bs);
                        const float v = okey_inv(okey(v0) + (uint32_t)(lane - 32));
                        const uint64_t m = __ballot(__fmaf_rn(v, bs, c0) >= tb);
                        if (m == 0 || m == ~0ull) return false;
                        const int L0 = __builtin_ctzll(m);
                        if (m != (~0ull << L0)) return false;
                        B = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                          __builtin_bit_cast(int, v), L0));
                        return true;
                    };
                    CBX_STAMP(17);
                    float B0 = kNegInf, B1 = kPosInf;
                    const bool have_b = bsel >= (partial ? 2 : 1) && nsel <= kWaveCand &&
                                        boundary(bsel, B0) &&
                                        (bsel == kWaveBins - 1 || boundary(bsel + 1, B1));
                    __syncthreads();  // histogram reads done: the candidates reuse it
                    CBX_STAMP(18);
                    if (have_b && above_bins + nsel <= kWaveCap) {
                        // One pass: every score >= B0 (the survivors >= B1 and the
                        // selected bin's candidates) joins the list, in (vector,
                        // element, lane) order.
                        auto val_of = [](uint64_t pk) {
                            return __builtin_bit_cast(float, (uint32_t)(pk >> 32));
                        };
                        // sb: byte offset of the next free slot (a running scalar)
                        const uint32_t lbase = lds_offset(&sm.list[0]);
                        uint32_t sb = lbase;
#pragma unroll
                        for (int j = 0; j < Q; ++j) {
#pragma unroll
                            for (int c = 0; c < 4; ++c)
                                sb = append_ge(sb, B0, s[4 * j + c], (uint32_t)(256 * j + 4 * lane + c));
                        }
                        const int n = (int)((sb - lbase) >> 3);
                        __syncthreads();
                        CBX_STAMP(19);
                        const int nr0 = (n + 63) >> 6;
                        int nc = 0;
                        uint64_t x[kWaveRows];  // the list, read once
#pragma unroll
                        for (int g = 0; g < kWaveRows; g += 4) {
                            if (g < nr0) {
#pragma unroll
                                for (int r = g; r < g + 4; ++r) x[r] = sm.list[r * 64 + lane];
                            }
                        }
                        if (n == above_bins + nsel) {
                            // the candidates: list entries below B1
#pragma unroll
                            for (int r = 0; r < kWaveRows; ++r) {
                                if (r < nr0) {
                                    const int i = r * 64 + lane;
                                    const bool inb = i < n && val_of(x[r]) < B1;
                                    const uint64_t m = __ballot(inb);
                                    const int at = ballot_rank(m) + nc;
                                    // (more than the array holds: the count check below fails)
                                    if (nc + __popcll(m) <= kWaveCand)
                                        lds_store_b64_lanes(lds_offset(sm.candk()) + 8u * (uint32_t)at,
                                                            x[r], m);
                                    nc += __popcll(m);
                                }
                            }
                        }
                        __syncthreads();
                        CBX_STAMP(20);
                        if (n == above_bins + nsel && nc == nsel) {
                            const int rem = k - above_bins;  // 0 <= rem < nc
                            float tv = kNegInf;
                            int tgt = 0;
                            bool hitc = false;
                            for (int c0 = lane; c0 < nc; c0 += 64) {
                                const float v = val_of(sm.candk()[c0]);
                                int gt = 0, ge = 0;
                                for (int t = 0; t < nc; ++t) {
                                    const float w = val_of(sm.candk()[t]);
                                    gt += (w > v) ? 1 : 0;
                                    ge += (w >= v) ? 1 : 0;
                                }
                                if (gt <= rem && rem < ge) { tv = v; tgt = gt; hitc = true; }
                            }
                            const int L2 = __builtin_ctzll(__ballot(hitc));
                            thr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                                 __builtin_bit_cast(int, tv), L2));
                            above = above_bins + __builtin_amdgcn_readlane(tgt, L2);
                            if (above < k) thr = __fsub_rn(thr, 1e-10f);
                            CBX_STAMP(21);
                            if (!(thr < B0)) {
                                // survivors: entries > thr, compacted in place
                                int n2 = 0;
#pragma unroll
                                for (int r = 0; r < kWaveRows; ++r) {
                                    if (r < nr0) {
                                        const bool keep = r * 64 + lane < n && val_of(x[r]) > thr;
                                        const uint64_t m = __ballot(keep);
                                        const int at = ballot_rank(m) + n2;
                                        lds_store_b64_lanes(lds_offset(&sm.list[0]) + 8u * (uint32_t)at,
                                                            x[r], m);
                                        n2 += __popcll(m);
                                    }
                                }
                                n_surv = n2;
                            }
                            done = true;  // thr < B0 (nudge past the bin): the full pass below
                        }
                        __syncthreads();
                    }
                }
            }
            if (!done) lo_from_memory();
            const float range = __fsub_rn(hi, lo);
            const float bscale = __fdiv_rn((float)kWaveBins, range);
            const float nlo = -__fmul_rn(lo, bscale);
            if (!done && !bad && range > 0.0f && bscale < kPosInf) {
                // bins with -inf sent to the spare bin NB (masked rows, -inf logits)
                auto bin_of = [&](float v) -> int {
                    const int b = (int)__builtin_amdgcn_fmed3f(__fmaf_rn(v, bscale, nlo), 0.0f,
                                                               (float)(kWaveBins - 1));
                    return v == kNegInf ? kWaveBins : b;
                };
                uint32_t* hist = sm.khist();
#pragma unroll
                for (int q = 0; q < kWaveBins / 64; ++q) hist[lane * (kWaveBins / 64) + q] = 0u;
                if (lane == 0) hist[kWaveBins] = 0u;
                __syncthreads();
                each_score([&](float v, int) { atomicAdd(&hist[bin_of(v)], 1u); });
                __syncthreads();
                constexpr int BPL = kWaveBins / 64;
                uint32_t cnt[BPL];
                int tot = 0;
#pragma unroll
                for (int q = 0; q < BPL; ++q) {
                    cnt[q] = hist[kWaveBins - 1 - (lane * BPL + q)];  // descending bins
                    tot += (int)cnt[q];
                }
                int n_fin;
                const int excl = wave_excl_scan_i(tot, n_fin);
                if (n_fin <= k) {
                    thr = kNegInf;  // at most k finite scores: nothing is removed
                    above = n_fin;
                    done = true;
                } else {
                    const bool mine = excl <= k && k < excl + tot;
                    int bsel = 0, above_bins = 0;
                    if (mine) {
                        int run = excl;
                        bool found = false;
#pragma unroll
                        for (int q = 0; q < BPL; ++q) {
                            if (!found && run + (int)cnt[q] > k) {
                                bsel = kWaveBins - 1 - (lane * BPL + q);
                                above_bins = run;
                                found = true;
                            }
                            run += (int)cnt[q];
                        }
                    }
                    const int L = __builtin_ctzll(__ballot(mine));
                    bsel = __builtin_amdgcn_readlane(bsel, L);
                    above_bins = __builtin_amdgcn_readlane(above_bins, L);
                    __syncthreads();  // histogram reads done: the candidates reuse it
                    int nc = 0;
                    each_score([&](float v, int) {
                        const bool in = bin_of(v) == bsel;
                        const uint64_t m = __ballot(in);
                        const int at = nc + ballot_rank(m);
                        if (nc + __popcll(m) <= kWaveCand)  // else nc > kWaveCand: not used
                            lds_store_b32_lanes(lds_offset(sm.cand()) + 4u * (uint32_t)at,
                                                __builtin_bit_cast(uint32_t, v), m);
                        nc += __popcll(m);
                    });
                    __syncthreads();
                    if (nc <= kWaveCand) {
                        const int rem = k - above_bins;  // 0 <= rem < nc
                        float tv = kNegInf;
                        int tgt = 0;
                        bool hitc = false;
                        for (int c0 = lane; c0 < nc; c0 += 64) {
                            const float v = sm.cand()[c0];
                            int gt = 0, ge = 0;
                            for (int t = 0; t < nc; ++t) {
                                const float w = sm.cand()[t];
                                gt += (w > v) ? 1 : 0;
                                ge += (w >= v) ? 1 : 0;
                            }
                            if (gt <= rem && rem < ge) { tv = v; tgt = gt; hitc = true; }
                        }
                        const int L2 = __builtin_ctzll(__ballot(hitc));
                        thr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(
                                                             __builtin_bit_cast(int, tv), L2));
                        above = above_bins + __builtin_amdgcn_readlane(tgt, L2);
                        done = true;
                    }
                }
                if (done) {
                    if (above < k) thr = __fsub_rn(thr, 1e-10f);
                }
            }
            if (!done && !bad && !(range > 0.0f)) {
                // every finite score equal (or none; forced-stop rows): the
                // (k+1)-th largest is that score when more than k are finite,
                // else -inf, and no score is above it
                int nf = 0;
                each_score([&](float v, int) { nf += (v != kNegInf) ? 1 : 0; });
                const int n_fin = wave_sum_dpp(nf);
                thr = n_fin > k ? lo : kNegInf;
                above = n_fin > k ? 0 : n_fin;
                if (above < k) thr = __fsub_rn(thr, 1e-10f);
                done = true;
            }
            if (!done) {
                // 8-bit radix select over all ids (NaN / inf rows)
                uint32_t prefix = 0, pmask = 0, rem = (uint32_t)k;
                wave_radix_pass<Q>(rsc, 24, prefix, pmask, rem, sm.khist());
                wave_radix_pass<Q>(rsc, 16, prefix, pmask, rem, sm.khist());
                wave_radix_pass<Q>(rsc, 8, prefix, pmask, rem, sm.khist());
                wave_radix_pass<Q>(rsc, 0, prefix, pmask, rem, sm.khist());
                thr = okey_inv(prefix);
                int n_above = 0;
                each_score([&](float v, int) { n_above += (v > thr) ? 1 : 0; });
                above = wave_sum_dpp(n_above);
                if (above < k) thr = __fsub_rn(thr, 1e-10f);
            }
        }
        CBX_STAMP(3);

        // ---- survivors -> LDS list of (score bits << 32 | id) ----
        // keep = score != -inf and not (top-k and score <= thr); without NaN that
        // is score > thr (thr = -inf when nothing is cut).  Only kept items that
        // fit the list are stored.
        if (n_surv < 0) {
            int n = 0;
            each_score([&](float v, int id) {
                const bool keep = bad ? (v != kNegInf && !(v <= thr)) : (v > thr);
                const uint64_t m = __ballot(keep);
                const int at = n + ballot_rank(m);
                // past the list: the row overflows and its list is not used
                lds_store_b64_lanes(lds_offset(&sm.list[0]) + 8u * (uint32_t)at,
                                    ((uint64_t)__builtin_bit_cast(uint32_t, v) << 32) | (uint32_t)id,
                                    __ballot(keep && at < kWaveCap));
                n += __popcll(m);
            });
            n_surv = n;
        }
    } else {
        chunk_front<Q, W2>(sm, rsc, lane, k, use_topk, cur, hi, lo, have_lo, bad, thr, n_surv, smv,
                           wv);
        if constexpr (W2) {
            if (wv == 1) return;  // its half is merged into wave 0's list
        }
        flags = bad ? CBX_INFO_NONFINITE : 0u;
    }
    CBX_STAMP(4);
    if (n_surv > cap) {
        if (lane == 0) {
            a.tokens[rs] = -1;
            if (a.info) a.info[rs] = flags | CBX_INFO_OVERFLOW;
            if (a.redo) {  // the redo pass samples the row again at full capacity
                const int i = atomicAdd(&a.redo[0], 1);
                if (i < a.redo_max) a.redo[2 + i] = (int32_t)rs;
            }
        }
        if (a.probs) {
            float* prow = a.probs + rs * a.ld_probs;
            for (int i = lane; i < V; i += 64) prow[i] = 0.0f;
        }
        return;
    }
    __syncthreads();
    const int nr = (n_surv + 63) >> 6;
    uint32_t rflags = flags;
    const bool use_topp = P.top_p < 1.0f && n_surv > 0;
    int n_kept = n_surv;  // kept: list positions [0, n_kept)
    float mx_surv = hi;
    // top-p sorts by a counting sort over [min survivor, max] where it can
    // (a threshold below lo only widens the range)
    if (!(use_topk && thr > kNegInf)) lo_from_memory();
    const float slo = use_topk && thr > kNegInf ? (have_lo ? fmaxf(thr, lo) : thr) : lo;
    const float srange = __fsub_rn(hi, slo);
    // descending sort bins, finer where survivors crowd (just above the
    // threshold): with x = max(0, (hi - v) / range) in [0, ~1], bin =
    // bits(fma(x^3, NB - 4, 2^23 + 2)) - bits(2^23).  Every step is a
    // correctly rounded monotone operation, so the bin never decreases as v
    // falls; the range is checked at both ends.
    const float sxs = __fdiv_rn(1.0f, srange);
    const float sxc = __fmul_rn(hi, sxs);
    auto sort_bin_y = [&](float v) {
        const float xq = fmaxf(__fmaf_rn(v, -sxs, sxc), 0.0f);
        return __fmaf_rn(__fmul_rn(__fmul_rn(xq, xq), xq), (float)(kWaveBins - 4), 0x1p23f + 2.0f);
    };
    const bool csort = use_topp && !bad && srange > 0.0f && sxs < kPosInf &&
                       sort_bin_y(hi) >= 0x1p23f &&
                       sort_bin_y(slo) <= 0x1p23f + (float)(kWaveBins - 1);
    // The common top-p case without the sort (lean_topp); the rows it cannot
    // certify take the sort and the exact sums below.
    bool lean = use_topp && csort;
    if (lean) {
        int nk_l = 0;
        lean = lean_topp<Q>(sm, n_surv, hi, sxs, sxc, P.top_p, nk_l);
        if (lean) n_kept = nk_l;
    }
    // raw entries -> composite keys (descending score, ascending id), in place;
    // positions [n_surv, 64*nr) become the maximum key (the counting sort
    // converts in registers instead).
    // Rows of the list are handled 4 at a time under one uniform branch, so
    // their LDS accesses overlap; rows past the list only touch unused slots.
    if (!csort && use_topp) {
#pragma unroll
        for (int g = 0; g < R; g += 4) {
            if (g < nr) {
#pragma unroll
                for (int r = g; r < g + 4; ++r) {
                    const int i = r * 64 + lane;
                    const uint64_t w = sm.list[i];
                    const uint64_t key =
                        desc_key(__builtin_bit_cast(float, (uint32_t)(w >> 32)), (uint32_t)w);
                    sm.list[i] = (i < n_surv) ? key : ~0ull;
                }
            }
        }
        __syncthreads();
    }
    CBX_STAMP(5);

    if (use_topp && !lean) {
        rflags |= CBX_INFO_TOPP_SORTED;
        // ---- counting sort of the keys by value bin over [min survivor, max] ----
        // Every survivor is read into registers first, so the counters and
        // offsets can use the list's own storage until the keys go back to
        // their sorted places; each key's bin bounds stay in registers.
        bool sorted = false;
        if (n_surv <= 64) {
            // one row of entries: each lane's key ranked against the others
            // by readlane (no LDS round trips), then one store each; the
            // lanes past the list write the maximum key in place.  Keys are
            // distinct (the ids are), so the ranks are 0 .. n_surv - 1.
            const uint64_t w = sm.list[lane];  // raw entry, or its key (!csort)
            uint64_t key = w;
            if (csort)
                key = lane < n_surv
                          ? desc_key(__builtin_bit_cast(float, (uint32_t)(w >> 32)), (uint32_t)w)
                          : ~0ull;
            // four lanes per step (lanes past the list hold the maximum key,
            // which is never below another)
            auto key_of = [&](int t) -> uint64_t {
                return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(key >> 32), t)
                        << 32) |
                       (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)key, t);
            };
            int rank = 0;
            for (int t = 0; t < n_surv; t += 4) {
                const uint64_t k0 = key_of(t), k1 = key_of(t + 1), k2 = key_of(t + 2),
                               k3 = key_of(t + 3);
                rank += ((k0 < key) ? 1 : 0) + ((k1 < key) ? 1 : 0) + ((k2 < key) ? 1 : 0) +
                        ((k3 < key) ? 1 : 0);
            }
            __syncthreads();  // every entry read: the sorted keys take the list
            sm.list[lane < n_surv ? rank : lane] = key;
            sorted = true;
        } else if (csort) {
            // descending bins rb(v) = bits(sort_bin_y(v)) - bits(2^23), in
            // [0, NB) for v in [slo, hi] (csort checked both ends)
            uint64_t x[R];
            int rb[R], slot[R], s0[R], s1[R];
            uint32_t* cnt = reinterpret_cast<uint32_t*>(sm.list);  // NB counters, then per-lane spares
            constexpr int kSpare = kWaveBins + 8;
            const int nv = fresh(n_surv);
#pragma unroll
            for (int g = 0; g < R; g += 4) {
                if (g < nr) {
#pragma unroll
                    for (int r = g; r < g + 4; ++r) {
                        const int i = r * 64 + lane;
                        const uint64_t w = sm.list[i];  // raw (score bits << 32 | id)
                        const float v = __builtin_bit_cast(float, (uint32_t)(w >> 32));
                        x[r] = (i < nv) ? desc_key(v, (uint32_t)w) : ~0ull;
                        const int b = (int)(__builtin_bit_cast(uint32_t, sort_bin_y(v)) - 0x4B000000u);
                        rb[r] = (i < nv) ? b : kSpare + lane;  // past the list: a spare counter
                    }
                }
            }
            __syncthreads();  // the list is in registers: its storage takes the counters
#pragma unroll
            for (int q = 0; q < kWaveBins / 64; ++q) cnt[lane * (kWaveBins / 64) + q] = 0u;
            if (lane < 8) cnt[kWaveBins + lane] = 0u;
            __syncthreads();
#pragma unroll
            for (int g = 0; g < R; g += 4)
                if (g < nr) {
#pragma unroll
                    for (int r = g; r < g + 4; ++r) slot[r] = (int)atomicAdd(&cnt[rb[r]], 1u);
                }
            __syncthreads();
            CBX_STAMP(13);
            // lane l: bins 16l .. 16l + 15 -> exclusive offsets in place
            uint32_t big = 0;
            {
                uint4* c4 = reinterpret_cast<uint4*>(cnt) + 4 * lane;
                uint4 w4[4];
                uint32_t loc = 0;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    w4[i] = c4[i];
                    big = max(big, max(max(w4[i].x, w4[i].y), max(w4[i].z, w4[i].w)));
                    loc += (w4[i].x + w4[i].y) + (w4[i].z + w4[i].w);
                }
                int all;
                uint32_t run = (uint32_t)wave_excl_scan_i((int)loc, all);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint4 o;
                    o.x = run; run += w4[i].x;
                    o.y = run; run += w4[i].y;
                    o.z = run; run += w4[i].z;
                    o.w = run; run += w4[i].w;
                    c4[i] = o;
                }
                if (lane == 63) cnt[kWaveBins] = run;  // end of the last bin (= n_surv)
            }
            if (__ballot(big > (uint32_t)kWaveSortMax) == 0) {
                __syncthreads();
#pragma unroll
                for (int g = 0; g < R; g += 4)
                    if (g < nr) {
#pragma unroll
                        for (int r = g; r < g + 4; ++r) {  // lanes past the list: empty bins
                            const bool in = r * 64 + lane < nv;
                            const int a0 = (int)cnt[rb[r]], a1 = (int)cnt[rb[r] + 1];
                            s0[r] = in ? a0 : n_surv;
                            s1[r] = in ? a1 : n_surv;
                        }
                    }
                __syncthreads();  // offsets read: the keys take their bins
                CBX_STAMP(14);
#pragma unroll
                for (int g = 0; g < R; g += 4)
                    if (g < nr) {
#pragma unroll
                        for (int r = g; r < g + 4; ++r)
                            lds_store_b64_lanes(lds_offset(&sm.list[0]) + 8u * (uint32_t)(s0[r] + slot[r]),
                                                x[r], __ballot(r * 64 + lane < nv));
                    }
                // keys after the survivors: the maximum key (4 slots, for the
                // reads past a bin's end below)
                if (lane < 4) sm.list[n_surv + lane] = ~0ull;
                __syncthreads();
                CBX_STAMP(15);
                // Rank inside the bin: the keys of the bin below x.  Reads past
                // the bin's end see later bins (lower scores: larger keys) or
                // the maximum key, which never count.  The first four keys of
                // the bins of four rows are read together (most bins hold at
                // most four); longer bins loop on.
                int fin[R];
#pragma unroll
                for (int g = 0; g < R; g += 4) {
                    if (g < nr) {
                        uint64_t kk[4][4];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
#pragma unroll
                            for (int q = 0; q < 4; ++q) kk[u][q] = sm.list[s0[g + u] + q];
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const uint64_t xr = x[g + u];
                            int rank = (kk[u][0] < xr) + (kk[u][1] < xr) + (kk[u][2] < xr) +
                                       (kk[u][3] < xr);
                            for (int t = s0[g + u] + 4; t < s1[g + u]; t += 4) {
                                const uint64_t k0 = sm.list[t];
                                const uint64_t k1 = sm.list[t + 1];
                                const uint64_t k2 = sm.list[t + 2];
                                const uint64_t k3 = sm.list[t + 3];
                                rank += (k0 < xr) + (k1 < xr) + (k2 < xr) + (k3 < xr);
                            }
                            fin[g + u] = s0[g + u] + rank;
                        }
                    }
                }
                __syncthreads();
#pragma unroll
                for (int g = 0; g < R; g += 4)
                    if (g < nr) {
#pragma unroll
                        for (int r = g; r < g + 4; ++r)
                            lds_store_b64_lanes(lds_offset(&sm.list[0]) + 8u * (uint32_t)fin[r], x[r],
                                                __ballot(r * 64 + lane < nv));
                    }
                sorted = true;
            } else {
                // crowded bins: the keys go back in place for the bitonic sort
                __syncthreads();
#pragma unroll
                for (int g = 0; g < R; g += 4)
                    if (g < nr) {
#pragma unroll
                        for (int r = g; r < g + 4; ++r) sm.list[r * 64 + lane] = x[r];
                    }
            }
        }
        if (!sorted) {
            // bitonic sort of the list in LDS (NaN rows, crowded bins)
            const int n2 = max(64, pow2ceil(n_surv));
            __syncthreads();
            for (int i = n_surv + lane; i < n2; i += 64) sm.list[i] = ~0ull;
            __syncthreads();
            for (int kk = 2; kk <= n2; kk <<= 1) {
                for (int jj = kk >> 1; jj > 0; jj >>= 1) {
                    for (int i = lane; i < n2; i += 64) {
                        const int p = i ^ jj;
                        if (p > i) {
                            const uint64_t ka = sm.list[i], kb = sm.list[p];
                            const bool up = (i & kk) == 0;
                            if ((ka > kb) == up) { sm.list[i] = kb; sm.list[p] = ka; }
                        }
                    }
                    __syncthreads();
                }
            }
        }
        __syncthreads();
        // ---- top-p (main.cpp:750-772) ----
        CBX_STAMP(6);
        mx_surv = desc_key_value(sm.list[0]);  // sorted[0]
        // e_i in registers, lane l holding sorted positions [l*C, l*C + C)
        // (C odd: the strided LDS reads fall in distinct banks).  The stage
        // is compiled per C, so its loops unroll without run-time guards and
        // every read of a lane's run is in flight at once.
        constexpr int CM = kWaveRows + 1;
        const int C = uni(((n_surv + 63) >> 6) | 1);
        const int nl = uni((n_surv + C - 1) / C);  // lanes holding terms
        int last = n_surv - 1;
        with_odd_c<1, CM>(C, [&](auto cc) {
            constexpr int CC = decltype(cc)::value;
            float ev[CM];
            // (every index is inside the list and its spare slots; x <= 0 and
            // not NaN for rows without NaN / +inf)
            float xs[CC];
#pragma unroll
            for (int q = 0; q < CC; ++q)
                xs[q] = __fsub_rn(desc_key_value(sm.list[min(lane * CC + q, kWaveCap)]), mx_surv);
            if (!bad) {
#pragma unroll
                for (int q = 0; q < CC; ++q) ev[q] = expf_nonpos(xs[q], sm.tab);
            } else {
#pragma unroll
                for (int q = 0; q < CC; ++q) ev[q] = expf_libm_branchless(xs[q], sm.tab);
            }
#pragma unroll
            for (int q = 0; q < CC; ++q) ev[q] = lane * CC + q < n_surv ? ev[q] : 0.0f;
            CBX_STAMP(7);
            // psum = 0 + e_0 + e_1 + ... (binary32, sorted order), term by term
            int unused;
            float psum;
            if constexpr (CC >= 7) psum = bad ? chain_sweeps<CC, false>(ev, nl, 0.0f, unused)
                                              : chain_segments<CC>(ev, nl);
            else psum = chain_sweeps<CC, false>(ev, nl, 0.0f, unused);
            CBX_STAMP(8);
            // First i with cum_i = q_0 + ... + q_i >= top_p, q_j = e_j / psum
            // (binary32, in order).  With Y_i = (e_0 + ... + e_i) / psum in
            // binary64, |cum_i - Y_i| <= i half-ulps of cum_i (one rounding
            // per add) + 2^-24 Y_i (the rounding of each q_j): a lane bounds
            // this for its terms by its last index and the binade of its last
            // Y.  Where Y_i -/+ that bound puts the first crossing at one index
            // the answer is certain; otherwise (and for rows holding NaN or
            // +inf) the q's are formed and summed as the reference does.
            bool certain = false;
            if (!bad) {
                const double p = (double)P.top_p;
                const double inv = __ddiv_rn(1.0, (double)psum);
                double part = 0.0;
#pragma unroll
                for (int q = 0; q < CC; ++q) part = __dadd_rn(part, (double)ev[q]);
                const double x0 = __dsub_rn(wave_incl_scan_f64_dpp(part), part);
                const double yl = __dmul_rn(__dadd_rn(x0, part), inv);
                const double cm = __dmul_rn(yl, 1.0 + 0x1p-12);
                const int b = __builtin_amdgcn_frexp_exp(cm) - 1;  // cm in [2^b, 2^(b+1))
                const double err = __dadd_rn(
                    __dadd_rn(__dmul_rn((double)(lane * CC + CC - 1),
                                        ldexp(1.0, max(b, -126) - 24)),
                              __dmul_rn(yl, 0x1p-23)),
                    1e-12);
                const double lo_thr = __dsub_rn(p, err), hi_thr = __dadd_rn(p, err);
                // y is non-decreasing: the first index meeting a bound is the
                // count of the lane's terms before it
                int n_hi = 0, n_lo = 0;
                double x = x0;
#pragma unroll
                for (int q = 0; q < CC; ++q) {
                    x = __dadd_rn(x, (double)ev[q]);
                    const double y = __dmul_rn(x, inv);
                    n_hi += y < lo_thr ? 1 : 0;
                    n_lo += y < hi_thr ? 1 : 0;
                }
                int c_hi = n_hi < CC ? lane * CC + n_hi : 0x7fffffff;
                int c_lo = n_lo < CC ? lane * CC + n_lo : 0x7fffffff;
                c_hi = min(wave_min_i_dpp(c_hi), n_surv);  // n_surv: never
                c_lo = min(wave_min_i_dpp(c_lo), n_surv);
                if (c_hi == c_lo) {
                    certain = true;
                    last = c_hi == n_surv ? n_surv - 1 : c_hi;
                }
            }
            if (!certain) {
#pragma unroll
                for (int q = 0; q < CC; ++q) ev[q] = __fdiv_rn(ev[q], psum);  // 0 stays 0
                int hit;
                if constexpr (CC >= 7) {
                    if (!bad) (void)chain_segments_x<CC, true>(ev, nl, 0.0f, P.top_p, hit);
                    else (void)chain_sweeps<CC, true>(ev, nl, P.top_p, hit);
                } else {
                    (void)chain_sweeps<CC, true>(ev, nl, P.top_p, hit);
                }
                last = hit < 0 ? n_surv - 1 : hit;
            }
        });
        n_kept = uni(last + 1);
        CBX_STAMP(9);
        if (n_kept < n_surv &&
            desc_key_value(sm.list[n_kept - 1]) == desc_key_value(sm.list[n_kept])) {
            rflags |= CBX_INFO_TOPP_TIE;
            // Equal scores straddle the cutoff: which of them the reference
            // keeps is decided by its std::sort's order.  The running sums,
            // hence n_kept, do not depend on that order; the kept ids of the
            // tied score do, and are replayed here (wave_tied_order).
            if (!bad) {
                tie_order_wave<Q>(sm, rsc, n_surv, n_kept, V);
            }
        }
        __syncthreads();
        // the kept keys back to raw entries (score bits << 32 | id) for the
        // stages below
        const int nkr = (n_kept + 63) >> 6;
        for_row_groups<0, R>(nkr, [&](auto gc, auto cc) {
            constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
            for (int r = g; r < g + rows; ++r) {
                const int i = r * 64 + lane;
                const uint64_t key = sm.list[i];
                sm.list[i] = ((uint64_t)__builtin_bit_cast(uint32_t, desc_key_value(key)) << 32) |
                             (uint32_t)key;
            }
        });
        __syncthreads();
    }

    // ---- min-p [extension], repetition penalty (main.cpp:774-781) ----
    // kept entries: list positions [0, n_kept); per entry in registers
    for (int w = lane; w < 8 * Q; w += 64) sm.keptw[w] = 0u;
    __syncthreads();
    const int nk = (n_kept + 63) >> 6;
    float val[R];
    int idr[R];
    uint32_t kept = 0;
    {
        const int nkv = fresh(n_kept);
        const float mx_kept = mx_surv;  // the best kept score before the penalty
#pragma unroll
        for (int r = 0; r < R; ++r) {
            val[r] = kNegInf;
            idr[r] = 0;
        }
        for_row_groups<0, R>(nk, [&](auto gc, auto cc) {
            constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
            for (int r = g; r < g + rows; ++r) {
                const int i = r * 64 + lane;
                const uint64_t key = sm.list[i];  // raw: score bits << 32 | id
                bool kp = i < nkv;
                float v = __builtin_bit_cast(float, (uint32_t)(key >> 32));
                const int id = kp ? (int)(uint32_t)key : 0;
                if (P.min_p > 0.0f) {
                    const float x = __fsub_rn(v, mx_kept);
                    kp = kp && !((bad ? expf_libm_branchless(x, sm.tab)
                                      : expf_nonpos(x, sm.tab)) < P.min_p);
                }
                if (use_pen) {
                    const bool hit = kp && bit_of(sm.h.seen, id);
                    const float pv = v > 0.0f ? __fdiv_rn(v, P.repeat_penalty)
                                              : __fmul_rn(v, P.repeat_penalty);
                    v = hit ? pv : v;
                }
                val[r] = v;
                idr[r] = id;
                kept |= (kp ? 1u : 0u) << r;
                lds_or_b32_lanes(lds_offset(&sm.keptw[0]) + ((uint32_t)(id >> 5) << 2),
                                 1u << (id & 31), __ballot(kp));
            }
        });
    }
    // ---- softmax (main.cpp:783-793) ----
    float m2 = kNegInf;
#pragma unroll
    for (int r = 0; r < R; ++r)
        if (r < ((nk + 3) & ~3)) m2 = ((kept >> r) & 1u) ? fmaxf(m2, val[r]) : m2;
    const float mx2 = wave_max_dpp(m2);
    CBX_STAMP(10);
    __syncthreads();
    // id-order ranks of the kept ids: word offsets
    constexpr int WPL = (8 * Q + 63) / 64;
    int n_final;
    int cw[WPL];  // kept ids in the lane's words lane*WPL .. lane*WPL + WPL - 1
    int loc = 0, wbase;
    {
#pragma unroll
        for (int q = 0; q < WPL; ++q) {
            const int w = lane * WPL + q;
            cw[q] = (w < W) ? __popc(sm.keptw[w]) : 0;
            loc += cw[q];
        }
        wbase = wave_excl_scan_i(loc, n_final);
        int basew = wbase;
#pragma unroll
        for (int q = 0; q < WPL; ++q) {
            const int w = lane * WPL + q;
            if (w < W) sm.h.woff[w] = (uint32_t)basew;
            basew += cw[q];
        }
    }
    // Id of the kept id of id-order rank `rank` (0 <= rank < n_final): the
    // lane whose words hold it finds the word; lanes 0..31 then count the
    // word's set bits below their own bit (mbcnt) to find the bit.
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
        const uint32_t bits = sm.keptw[w];
        const bool hit = lane < 32 && ((bits >> (lane & 31)) & 1u) &&
                         (int)__builtin_amdgcn_mbcnt_lo(bits, 0u) == kb;
        return w * 32 + __builtin_ctzll(__ballot(hit));
    };
    __syncthreads();
    // val - mx2 <= 0 and not NaN once mx2 is finite and the row holds no NaN
    auto f_terms = [&](auto nonpos) {
        for_row_groups<0, R>(nk, [&](auto gc, auto cc) {
            constexpr int g = decltype(gc)::value, rows = decltype(cc)::value;
#pragma unroll
            for (int r = g; r < g + rows; ++r) {
                const bool kp = (kept >> r) & 1u;
                const int at = rank_of(sm.keptw, sm.h.woff, idr[r]);  // kept lanes
                const float x = __fsub_rn(val[r], mx2);
                const float e = decltype(nonpos)::value ? expf_nonpos(x, sm.tab)
                                                        : expf_libm_branchless(x, sm.tab);
                lds_store_b32_lanes(lds_offset(sm.F()) + 4u * (uint32_t)at,
                                    __builtin_bit_cast(uint32_t, e), __ballot(kp));
            }
        });
    };
    if (!bad && __builtin_fabsf(mx2) < kPosInf) f_terms(std::true_type{});
    else f_terms(std::false_type{});
    __syncthreads();
    CBX_STAMP(11);

    // ---- greedy or draw (main.cpp:795-800) ----
    int token = 0;
    uint32_t oflags = rflags;
    const bool empty = n_final == 0;  // else psum >= expf(0) = 1
    float psum2 = 0.0f;
    bool have_psum2 = false;
    auto exact_psum2 = [&]() {
        if (!have_psum2) {
            psum2 = wave_chain_sum(sm.F(), n_final, 0.0f, !bad);
            have_psum2 = true;
        }
        return psum2;
    };
    if (empty) {
        oflags |= CBX_INFO_EMPTY;
    } else if (P.temp <= 0.0f) {
        // first argmax of p_i = e_i / psum over ids (main.cpp:795-797)
        const float ps = exact_psum2();
        float best = -1.0f;
        int first = 0x7fffffff;
        for (int i = lane; i < n_final; i += 64) {
            const float p = __fdiv_rn(sm.F()[i], ps);
            if (p > best) { best = p; first = i; }  // ascending i: keeps the first
        }
        const float b = wave_max_dpp(best);
        const int rk = wave_min_i_dpp(best == b ? first : 0x7fffffff);
        token = rk == 0x7fffffff ? 0 : id_of_rank_w(rk);
        oflags |= CBX_INFO_GREEDY;
    } else if (V >= 2) {
        oflags |= CBX_INFO_DREW;
        const double u = u_draw;
        const bool last_kept = bit_of(sm.keptw, V - 1);
        // binary64 prefix of the exp terms in id order: lane l holds the odd
        // run [l*C, l*C + C) in registers (compiled per C, reads in flight
        // together, distinct banks)
        constexpr int CM = kWaveRows + 1;
        const int C = uni(((n_final + 63) >> 6) | 1);
        double total = 0.0, blo = 0.0, bhi = 0.0;
        int found = 0x7fffffff;
        with_odd_c<1, CM>(C, [&](auto cc) {
            constexpr int CC = decltype(cc)::value;
            float f[CC];
#pragma unroll
            for (int q = 0; q < CC; ++q) {
                const int r = lane * CC + q;  // inside the list's float view
                const float v = sm.F()[r];
                f[q] = r < n_final ? v : 0.0f;
            }
            double part = 0.0;
#pragma unroll
            for (int q = 0; q < CC; ++q) part = __dadd_rn(part, (double)f[q]);
            double cp = wave_incl_scan_f64(part, lane);
            total = readlane_f64(cp, 63);
            cp = __dsub_rn(cp, part);  // exclusive
            const double target = __dmul_rn(u, total);
            bool got = false;
#pragma unroll
            for (int q = 0; q < CC; ++q) {
                const double before = cp;
                cp = __dadd_rn(cp, (double)f[q]);
                const bool hit = !got && cp >= target && lane * CC + q < n_final;
                blo = hit ? before : blo;
                bhi = hit ? cp : bhi;
                found = hit ? lane * CC + q : found;
                got = got || hit;
            }
        });
        const int rank = wave_min_i_dpp(found);
        bool certain = false;
        if (!(u > 0.0)) {
            token = 0;  // lower_bound of 0 is the first entry
            certain = true;
        } else if (rank != 0x7fffffff) {
            const int L = __builtin_ctzll(__ballot(found == rank));
            const double inv = __ddiv_rn(1.0, total);
            const double clo = __dmul_rn(readlane_f64(blo, L), inv);
            const double chi = __dmul_rn(readlane_f64(bhi, L), inv);
            const bool lo_ok = rank == 0 || __dsub_rn(u, clo) > kDrawMargin * clo + 1e-30;
            const bool hi_ok = (rank == n_final - 1 && last_kept) ||
                               __dsub_rn(chi, u) > kDrawMargin * chi + 1e-30;
            certain = lo_ok && hi_ok;
            token = id_of_rank_w(rank);
        }
        if (!certain) {
            // the reference's arithmetic: float normaliser, double CDF (rare)
            const float ps = exact_psum2();
            if (lane == 0) {
                double sum = 0.0;
                for (int r = 0; r < n_final; ++r)
                    sum = __dadd_rn(sum, (double)__fdiv_rn(sm.F()[r], ps));
                double acc = 0.0;
                int rk = -1;
                for (int r = 0; r < n_final; ++r) {
                    acc = __dadd_rn(acc, __ddiv_rn((double)__fdiv_rn(sm.F()[r], ps), sum));
                    const double c = (r == n_final - 1 && last_kept) ? 1.0 : acc;
                    if (c >= u) { rk = r; break; }
                }
                sm.rk = rk;
            }
            __syncthreads();
            const int rk = sm.rk;
            token = rk < 0 ? V - 1 : id_of_rank_w(rk);
        }
    }
    CBX_STAMP(12);
    if (lane == 0) {
        a.tokens[rs] = token;
        if (a.info) a.info[rs] = oflags;
    }
    if (a.probs) {
        const float ps = empty ? 0.0f : exact_psum2();
        float* prow = a.probs + rs * a.ld_probs;
        for (int i = lane; i < V; i += 64)
            prow[i] = (!empty && bit_of(sm.keptw, i))
                          ? __fdiv_rn(sm.F()[rank_of(sm.keptw, sm.h.woff, i)], ps)
                          : 0.0f;
    }
}

// Q: scores per lane / 4 (V <= 256*Q); JT: V > 256*JT for every launch; CH:
// the row read in chunks (no CFG rows).
template <int Q, int JT, bool CH = false, bool W2 = false>
hipError_t launch_wave(const KernelArgs& a, hipStream_t stream) {
    const int64_t rows = (int64_t)a.n_steps * a.n_rows;
    hipLaunchKernelGGL((sample_rows_wave<Q, JT, CH, W2>), dim3((unsigned)rows), dim3(W2 ? 128 : 64), 0,
                       stream, a);
    return hipGetLastError();
}

}  // namespace
}  // namespace cbx
