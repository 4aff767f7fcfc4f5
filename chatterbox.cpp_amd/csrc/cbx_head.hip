// cbx_head.hip -- the T3 speech_head projection:
// logits[r][v] = sum_k W[v][k] * h[r][k] + b[v]   (src/main.cpp:577; the weights
// and bias are chatterbox/speech_head(_bias), main.cpp:394-395), for F16, Q4_0,
// Q5_0 and Q8_0 weights in ggml's layout (ne = [n_embd, n_vocab]: row v holds
// the n_embd weights of vocab id v; Q4_0 blocks are an fp16 scale d and 16
// bytes of nibbles, element j < 16 in the low nibble of byte j and element
// j + 16 in its high nibble, w = (q - 8) d; Q5_0 blocks are d, a 32-bit
// little-endian word qh whose bit j is the fifth bit of element j, and the
// nibbles as Q4_0's, w = (q - 16) d; Q8_0 blocks are d and 32 int8, w = q d).
//
// 16 rows and more run on the fp16 matrix cores in two launches:
//  * head_split: each activation row r is scaled by a power of two 2^s_r (its
//    largest magnitude to [2^14, 2^15)) and written as two fp16 parts,
//    x 2^s = hi + lo + e with |e| <= 2^-23 |x 2^s| + 2^-25 (hi and lo rounded
//    to nearest; the 2^-25 is lo's subnormal step, 2^-39 of the row's largest
//    value), together with 2^-s_r, in the matrix-core operand order: for
//    each 16-row tile and 32-weight block, the 64 lanes' 16 bytes of hi parts,
//    then their 16 bytes of lo parts, so each operand load reads 1 KB
//    contiguous (loads of 64-byte pieces of 16 rows were the kernel's limit).
//  * head_mfma: a workgroup of KS waves computes 32 vocab ids x NT row tiles
//    of 16 rows with v_mfma_f32_16x16x32_f16, A = the activation parts, B =
//    the weights: F16 weights as they are, Q4_0 / Q5_0 / Q8_0 as their
//    integers (n - 8, q - 16 or q, exact in fp16) with each block's product scaled by its d
//    in fp32.  Products of fp16 values are exact in fp32; sums are the
//    matrix core's fp32.  Wave w takes the w-th of KS runs of 32-weight
//    blocks along n_embd, and the KS partial tiles are added in wave order
//    through LDS (a fixed order: results do not depend on scheduling); the
//    sum is scaled back by 2^-s_r (exact) and the bias added.
// Lane l feeds A[l%16][8(l/16) ..] and B[8(l/16) ..][l%16] (the same k on
// both operands, so a tile's products are sums over every k) and holds
// D[4(l/16)+i][l%16]: hidden row 4(l/16)+i of the tile, vocab id l%16.
// Rows v >= n_vocab and r >= n_rows read zeros through the buffer
// descriptors' ranges and store nothing.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cbx_internal.h"
#include "cbx_split.h"

namespace cbx {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef uint32_t u4v __attribute__((ext_vector_type(4)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
constexpr int32_t kBufWord3 = 0x00020000;  // raw buffer: 32-bit data format

__device__ __forceinline__ float half_bits_to_float(uint32_t hb) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
}

// Bytes of one block of 32 weights (F16: 32 halves).
template <int WT>
constexpr int block_bytes() {
    return WT == CBX_WTYPE_F16 ? 64 : WT == CBX_WTYPE_Q4_0 ? 18 : WT == CBX_WTYPE_Q5_0 ? 22 : 34;
}

// Bits 0..3 of x to bit 4 of bytes 0..3 (the four products x << 7i land in
// disjoint bit ranges: no carries).
__device__ __forceinline__ uint32_t spread4(uint32_t x) {
    return ((x * 0x00204081u) & 0x01010101u) << 4;
}

// ------------------------------------------------------------ activation split
constexpr int kSplitThreads = 256;

// One thread per group of 8 activations of the padded rows p = 16 T + m of
// the row tiles T (the tiles of hidden0's n_rows rows, then those of
// hidden1's), in row order: thread i takes group j = i mod ng of row
// p = i / ng.  The 4 groups of a block are 4 consecutive lanes, which share
// the block's scale (cbx_split.h); rows past a set's n_rows are zeros.
__global__ __launch_bounds__(kSplitThreads) void head_split(const float* hidden0,
                                                            const float* hidden1, int64_t ld_hidden,
                                                            int n_rows, int n_embd, int R,
                                                            uint32_t* parts, float* inv) {
    const int ng = n_embd / 8, nball = n_embd / 32;
    const int64_t i = (int64_t)blockIdx.x * kSplitThreads + threadIdx.x;
    const bool in = i < (int64_t)R * ng;  // a whole wave's blocks are in or out together
    const int p = in ? (int)(i / ng) : 0, j = in ? (int)(i % ng) : 0;
    const int tps = (n_rows + 15) / 16, T = p / 16, m = p % 16;
    const int rr = (T % tps) * 16 + m;
    const bool real = in && rr < n_rows;
    const float* src = (T < tps ? hidden0 : hidden1) + (int64_t)(real ? rr : 0) * ld_hidden;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(src), (short)0, real ? n_embd * 4 : 0, kBufWord3);
    const f4 a = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, 32 * j, 0, 0));
    const f4 c = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, 32 * j + 16, 0, 0));
    float x[8];
    float mx = 0.0f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        x[e] = a[e];
        x[4 + e] = c[e];
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(x[e]));
    mx = split_block_max4(mx);
    if (!in) return;
    float sc, sinv;
    split_scale(mx, sc, sinv);
    split_store(parts, T, m, nball, j, x, sc);
    if ((j & 3) == 0) inv[split_inv_index(T, m, nball, j >> 2)] = sinv;
}

// --------------------------------------------------------------- matrix cores
// Raw bytes of the 8 weights k = 8g .. 8g + 7 of one block of a vocab row,
// from the row's chunk staged in LDS: F16 four dwords; Q4_0 / Q5_0 / Q8_0 the
// fp16 scale in q[4] and the 8 bytes of nibbles or int8 in q[0..1], Q5_0's
// high-bit word qh in q[2].  Blocks are 18, 22 or 34 bytes, so only 2-byte
// alignment holds: `off` (the block's byte offset in the staged row) is read
// as dwords shifted into place.
template <int WT>
__device__ __forceinline__ void lds_w(const uint32_t* srow, int off, int g, uint32_t* q) {
    if constexpr (WT == CBX_WTYPE_F16) {
        const int b = off + 16 * g;
        const uint32_t* p = srow + (b >> 2);
        const uint32_t sh = 8u * (uint32_t)(b & 3);
        const uint32_t t0 = p[0], t1 = p[1], t2 = p[2], t3 = p[3], t4 = p[4];
        q[0] = __builtin_amdgcn_alignbit(t1, t0, sh);
        q[1] = __builtin_amdgcn_alignbit(t2, t1, sh);
        q[2] = __builtin_amdgcn_alignbit(t3, t2, sh);
        q[3] = __builtin_amdgcn_alignbit(t4, t3, sh);
    } else {
        q[4] = (srow[off >> 2] >> (8 * (off & 3))) & 0xffffu;
        const int qoff = off + (WT == CBX_WTYPE_Q5_0 ? 6 : 2) +
                         (WT == CBX_WTYPE_Q8_0 ? 8 * g : 8 * (g & 1));
        const uint32_t* p = srow + (qoff >> 2);
        const uint32_t sh = 8u * (uint32_t)(qoff & 3);
        const uint32_t t0 = p[0], t1 = p[1], t2 = p[2];
        q[0] = __builtin_amdgcn_alignbit(t1, t0, sh);
        q[1] = __builtin_amdgcn_alignbit(t2, t1, sh);
        if constexpr (WT == CBX_WTYPE_Q5_0) {
            const int hoff = off + 2;
            const uint32_t* ph = srow + (hoff >> 2);
            q[2] = __builtin_amdgcn_alignbit(ph[1], ph[0], 8u * (uint32_t)(hoff & 3));
        }
    }
}

__device__ __forceinline__ float ubyte(uint32_t x, int i) { return (float)((x >> (8 * i)) & 0xffu); }

// Two bytes b0, b1 of x (bytes sel0, sel1) as fp16 (b - off): the byte under
// the high byte 0x64 is the fp16 1024 + b, exactly, and the packed fp16
// subtraction of 1024 + off leaves b - off (an integer of at most 8 bits:
// exact).
__device__ __forceinline__ uint32_t bytes_f16(uint32_t x, uint32_t sel, _Float16 off) {
    const uint32_t v = __builtin_amdgcn_perm(0x64646464u, x, sel);
    const h2 r = __builtin_bit_cast(h2, v) - h2{off, off};
    return __builtin_bit_cast(uint32_t, r);
}

// The 8 integer weights of lds_w's bytes as fp16: Q4_0 n - 8, Q5_0 q - 16
// (q = n | the element's qh bit << 4), Q8_0 q; and the block's scale d.
template <int WT>
__device__ __forceinline__ u4v int_weights(const uint32_t* q, int g, float& d) {
    d = half_bits_to_float(q[4]);
    uint32_t x0, x1;
    _Float16 off;
    if constexpr (WT == CBX_WTYPE_Q4_0) {
        const int sh = g < 2 ? 0 : 4;
        x0 = (q[0] >> sh) & 0x0f0f0f0fu;
        x1 = (q[1] >> sh) & 0x0f0f0f0fu;
        off = (_Float16)1032.0f;
    } else if constexpr (WT == CBX_WTYPE_Q5_0) {
        // lane group g holds elements 8g .. 8g + 7: qh bits 8g .. 8g + 7
        const int sh = g < 2 ? 0 : 4;
        const uint32_t hb = q[2] >> (8 * g);
        x0 = ((q[0] >> sh) & 0x0f0f0f0fu) | spread4(hb & 15u);
        x1 = ((q[1] >> sh) & 0x0f0f0f0fu) | spread4((hb >> 4) & 15u);
        off = (_Float16)1040.0f;
    } else {
        x0 = q[0] ^ 0x80808080u;
        x1 = q[1] ^ 0x80808080u;
        off = (_Float16)1152.0f;
    }
    // selector bytes: 0-3 the bytes of x, 4 the constant's 0x64
    return u4v{bytes_f16(x0, 0x04010400u, off), bytes_f16(x0, 0x04030402u, off),
               bytes_f16(x1, 0x04010400u, off), bytes_f16(x1, 0x04030402u, off)};
}

__device__ __forceinline__ f4 mfma_f16(const u4v& a, const u4v& b, const f4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, a),
                                                  __builtin_bit_cast(h8, b), c, 0, 0, 0);
}

constexpr int KS = 4;  // waves per workgroup (runs of blocks along n_embd)
// NT row tiles of 16 per workgroup (a template argument): each weight block
// feeds the products of NT tiles, so weight loads and conversions are shared
// by 16 NT rows.  Measured at 128 rows, V = 6563, n_embd = 1024 (us, 4 / 2
// tiles): Q4_0 15.3 / 13.9, Q8_0 15.6 / 17.7, F16 17.6 / 23.7; at 16 rows 2
// tiles is faster for all three (one workgroup per CU either way).
// Register sets for the activation parts of RING consecutive blocks: the
// loads of block kb + RING - 1 are issued as block kb's products start (4
// sets measured no faster than 2).
constexpr int RING = 2;

// parts, inv: the split activations of the n_tiles row tiles (those of
// hidden0, then those of hidden1), cbx_split.h's layout; each block's
// products are scaled back by its rows' 2^-s (exact) as they are added.
// K split over workgroups (gridDim.z > 1): workgroup z takes blocks
// [nball z / Z, nball (z + 1) / Z) and writes its partial products to
// out0 + z * zstride (the bias in slab 0 only); the caller adds the slabs.
// Split output (out_parts set, one row set, no K split): the outputs, gelu
// applied when gelu_out, are written as the next product's split activations
// (rows of n_vocab values: this workgroup's 32 outputs are block blockIdx.x
// of each of its rows) instead of fp32 rows.
template <int WT, int NT>
__global__ __launch_bounds__(64 * KS) __attribute__((amdgpu_waves_per_eu(WT == CBX_WTYPE_Q4_0 ? 4 : 1))) void head_mfma(const void* W, const float* bias,
                                                     const uint32_t* parts, const float* inv,
                                                     int n_tiles, float* out0, float* out1,
                                                     int64_t ld_out, int n_rows, int n_vocab,
                                                     int n_embd, int64_t zstride, int gelu_out,
                                                     uint32_t* out_parts, float* out_inv) {
    constexpr int BB = block_bytes<WT>();
    // Weights are staged per wave in chunks of CB blocks: for each of the 32
    // vocab rows the chunk's CB * BB bytes are contiguous, so whole-row dword
    // loads touch two or three lines each (the per-block loads of the 18-byte
    // pieces of 16 rows 576 bytes apart touched up to 32 lines each, and the
    // texture-address path was the measured limit).  RSW dwords per staged
    // row: the bytes from the dword holding the first, plus one.
    constexpr int CB = WT == CBX_WTYPE_F16 ? 4 : 8;
    static_assert(CB % RING == 0, "a chunk holds whole rings of blocks");
    constexpr int RSW = (CB * BB + 6) / 4 + 1;
    __shared__ uint32_t stage[KS][32 * RSW];
    __shared__ f4 part[KS - 1][2 * NT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int v0 = blockIdx.x * 32;
    const int64_t wbytes = (int64_t)n_vocab * (n_embd / 32) * BB;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(W), (short)0, (int)wbytes, kBufWord3);
    const int pbytes = n_tiles * 16 * n_embd * 4;
    const __amdgpu_buffer_rsrc_t rp = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint32_t*>(parts), (short)0, pbytes, kBufWord3);
    const int sbytes = n_tiles * 16 * (n_embd / 32) * 4;
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(inv), (short)0, sbytes, kBufWord3);
    const int va = v0 + m, vb = v0 + 16 + m;
    // rows past the table read zeros (byte offsets past the range)
    const int va_c = va < n_vocab ? va : n_vocab, vb_c = vb < n_vocab ? vb : n_vocab;
    // Row tile T = blockIdx.y * NT + t of the tiles of both row sets (those
    // of hidden0, then those of hidden1): set T / tps, rows 16 (T % tps) ...
    const int tps = (n_rows + 15) / 16;
    const int nball = n_embd / 32;
    uint32_t hoff[NT], soff[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int T = blockIdx.y * NT + t;
        hoff[t] = T < n_tiles ? (uint32_t)(T * nball * 512 + 4 * lane) * 4u : (uint32_t)pbytes;
        // the scales of rows 4g .. 4g + 3 (the rows of this lane's outputs)
        soff[t] = T < n_tiles ? (uint32_t)split_inv_index(T, 4 * g, nball, 0) * 4u : (uint32_t)sbytes;
    }
    f4 acc0[NT], acc1[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc0[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        acc1[t] = acc0[t];
    }
    const int z0 = nball * (int)blockIdx.z / (int)gridDim.z;
    const int zn = nball * ((int)blockIdx.z + 1) / (int)gridDim.z - z0;
    const int kb0 = z0 + zn * wave / KS, kb1 = z0 + zn * (wave + 1) / KS;
    // The activation parts of RING consecutive blocks are in flight in RING
    // register sets (block kb in set (kb - kb0) % RING).  The loads are
    // unconditional (past a wave's run they read the next run's parts, or
    // zeros past the buffer) and the block loop is unrolled by RING, so no
    // register copies (and no waits for the loads just issued) join the sets.
    u4v ph[RING][NT], pl[RING][NT];
    f4 sv[RING][NT];
    auto load = [&](int kb, int r) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint32_t o = hoff[t] + (uint32_t)kb * 2048u;
            ph[r][t] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rp, o, 0, 0));
            pl[r][t] = __builtin_bit_cast(u4v, __builtin_amdgcn_raw_buffer_load_b128(rp, o + 1024, 0, 0));
            sv[r][t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rs, soff[t] + (uint32_t)kb * 64u, 0, 0));
        }
    };
#pragma unroll
    for (int r = 0; r + 1 < RING; ++r) load(kb0 + r, r);
    uint32_t* const sw = stage[wave];
    // one block: its weights from the staged chunk, the next block's parts
    // requested, then the products
    auto block = [&](int kb, int kbc, int sha, int shb, int r) {
        const u4v* const ch = ph[r];
        const u4v* const cl = pl[r];
        const f4* const sc = sv[r];
        uint32_t qa[5], qb[5];
        lds_w<WT>(sw + m * RSW, sha + (kb - kbc) * BB, g, qa);
        lds_w<WT>(sw + (16 + m) * RSW, shb + (kb - kbc) * BB, g, qb);
        load(kb + RING - 1, (r + RING - 1) % RING);
        if constexpr (WT == CBX_WTYPE_F16) {
            const u4v wa = u4v{qa[0], qa[1], qa[2], qa[3]}, wb = u4v{qb[0], qb[1], qb[2], qb[3]};
            f4 pa[NT], pb[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const f4 z = f4{0.0f, 0.0f, 0.0f, 0.0f};
                pa[t] = mfma_f16(cl[t], wa, z);
                pb[t] = mfma_f16(cl[t], wb, z);
                pa[t] = mfma_f16(ch[t], wa, pa[t]);
                pb[t] = mfma_f16(ch[t], wb, pb[t]);
            }
#pragma unroll
            for (int t = 0; t < NT; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc0[t][i] = __fmaf_rn(pa[t][i], sc[t][i], acc0[t][i]);
                    acc1[t][i] = __fmaf_rn(pb[t][i], sc[t][i], acc1[t][i]);
                }
            }
        } else {
            float da, db;
            const u4v ia = int_weights<WT>(qa, g, da), ib = int_weights<WT>(qb, g, db);
            f4 pa[NT], pb[NT];
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const f4 z = f4{0.0f, 0.0f, 0.0f, 0.0f};
                pa[t] = mfma_f16(cl[t], ia, z);
                pb[t] = mfma_f16(cl[t], ib, z);
                pa[t] = mfma_f16(ch[t], ia, pa[t]);
                pb[t] = mfma_f16(ch[t], ib, pb[t]);
            }
            // d 2^-s: exact (a power of two times a binary16 value)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    acc0[t][i] = __fmaf_rn(pa[t][i], __fmul_rn(da, sc[t][i]), acc0[t][i]);
                    acc1[t][i] = __fmaf_rn(pb[t][i], __fmul_rn(db, sc[t][i]), acc1[t][i]);
                }
            }
        }
    };
#pragma unroll 1
    for (int kbc = kb0; kbc < kb1; kbc += CB) {
        const int nb = min(CB, kb1 - kbc);
        // stage rows v0 .. v0 + 31 (rows past the table read zeros): the NDW
        // dwords from the one holding the chunk's first byte (a shorter last
        // chunk stages as many, the rest unused).  Lane 2 rr + h takes
        // dwords [h H, h H + H) of row rr: one row address per lane, and
        // every load and store at a constant offset from it (computing each
        // dword's row and column was a fifth of the kernel's VALU work).
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        {
            constexpr int NDW = RSW - 1, H = (NDW + 1) / 2;
            const int rr = lane >> 1, hh = lane & 1;
            const int vrow = v0 + rr;
            const uint32_t rb =
                vrow < n_vocab
                    ? (((uint32_t)(vrow * nball + kbc) * (uint32_t)BB) & ~3u) + 4u * H * hh
                    : 0x80000000u;
            uint32_t tv[H];
#pragma unroll
            for (int q = 0; q < H; ++q)
                tv[q] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, rb + 4u * q, 0, 0);
            uint32_t* const dst = sw + rr * RSW + H * hh;
#pragma unroll
            for (int q = 0; q < H; ++q) dst[q] = tv[q];
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const int sha = (int)((((int64_t)va_c * nball + kbc) * BB) & 3);
        const int shb = (int)((((int64_t)vb_c * nball + kbc) * BB) & 3);
        // chunks start a multiple of RING blocks after kb0 (CB is one), and
        // only a wave's last chunk can hold fewer
#pragma unroll 1
        for (int kb = kbc; kb < kbc + nb; kb += RING) {
#pragma unroll
            for (int u = 0; u < RING; ++u)
                if (kb + u < kbc + nb) block(kb + u, kbc, sha, shb, u);
        }
    }
    // the partial tiles of waves 1 .. KS-1 join wave 0's in wave order
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            part[wave - 1][2 * t][lane] = acc0[t];
            part[wave - 1][2 * t + 1][lane] = acc1[t];
        }
    }
    __syncthreads();
    if (wave > 0) return;
#pragma unroll
    for (int w = 0; w < KS - 1; ++w) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const f4 p0 = part[w][2 * t][lane], p1 = part[w][2 * t + 1][lane];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                acc0[t][i] = __fadd_rn(acc0[t][i], p0[i]);
                acc1[t][i] = __fadd_rn(acc1[t][i], p1[i]);
            }
        }
    }
    // D[4g + i][m]: hidden row 4g + i of the tile, vocab ids va and vb
    const bool with_bias = bias && blockIdx.z == 0;
    const float ba = with_bias && va < n_vocab ? bias[va] : 0.0f;
    const float bb = with_bias && vb < n_vocab ? bias[vb] : 0.0f;
    if (out_parts) {
        // the 32 outputs of each row as block blockIdx.x of the next
        // product's split row: its largest magnitude over the 16 lanes of
        // the row (ids m and 16 + m), then lane (g, m) holds the values of
        // group m / 8 (id m) and group 2 + m / 8 (id 16 + m) at place m % 8;
        // pairs of lanes join their halves into dwords
        const int nb_out = n_vocab / 32;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int T = blockIdx.y * NT + t;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float xa = __fadd_rn(acc0[t][i], ba), xb = __fadd_rn(acc1[t][i], bb);
                if (gelu_out) {
                    xa = t3_gelu_f(xa);
                    xb = t3_gelu_f(xb);
                }
                float mx = fmaxf(fabsf(xa), fabsf(xb));
#pragma unroll
                for (int o = 1; o < 16; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
                float scl, sinv;
                split_scale(mx, scl, sinv);
                const float ya = __fmul_rn(xa, scl), yb = __fmul_rn(xb, scl);
                const _Float16 ha = (_Float16)ya, hb = (_Float16)yb;
                const _Float16 la = (_Float16)__fsub_rn(ya, (float)ha);
                const _Float16 lb = (_Float16)__fsub_rn(yb, (float)hb);
                // the odd lane's halves join the even lane's dword
                const uint32_t hab = (uint32_t)__builtin_bit_cast(uint16_t, ha) |
                                     (uint32_t)__builtin_bit_cast(uint16_t, hb) << 16;
                const uint32_t lab = (uint32_t)__builtin_bit_cast(uint16_t, la) |
                                     (uint32_t)__builtin_bit_cast(uint16_t, lb) << 16;
                const uint32_t hab_o = (uint32_t)__shfl_xor((int)hab, 1);
                const uint32_t lab_o = (uint32_t)__shfl_xor((int)lab, 1);
                const int mrow = 4 * g + i;  // the row's place in its tile
                if (T < n_tiles && (m & 1) == 0) {
                    // dword (m % 8) / 2 of lane 16 gq + mrow's hi (lo) 16 bytes
                    uint32_t* const base = out_parts + ((int64_t)T * nb_out + blockIdx.x) * 512 +
                                           (m & 7) / 2;
                    const int ga = m >> 3, gb = 2 + (m >> 3);
                    base[4 * (16 * ga + mrow)] = (hab & 0xffffu) | (hab_o << 16);
                    base[4 * (16 * ga + mrow) + 256] = (lab & 0xffffu) | (lab_o << 16);
                    base[4 * (16 * gb + mrow)] = (hab >> 16) | (hab_o & 0xffff0000u);
                    base[4 * (16 * gb + mrow) + 256] = (lab >> 16) | (lab_o & 0xffff0000u);
                }
                if (T < n_tiles && m == 0)
                    out_inv[split_inv_index(T, mrow, nb_out, blockIdx.x)] = sinv;
            }
        }
        return;
    }
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int T = blockIdx.y * NT + t;
        if (T >= n_tiles) continue;
        float* const o = (T >= tps ? out1 : out0) + (int64_t)blockIdx.z * zstride;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rr = (T % tps) * 16 + 4 * g + i;
            if (rr < n_rows) {
                float* orow = o + (int64_t)rr * ld_out;
                const float xa = __fadd_rn(acc0[t][i], ba);
                const float xb = __fadd_rn(acc1[t][i], bb);
                if (va < n_vocab) orow[va] = gelu_out ? t3_gelu_f(xa) : xa;
                if (vb < n_vocab) orow[vb] = gelu_out ? t3_gelu_f(xb) : xb;
            }
        }
    }
}

// ----------------------------------------------------------------- mat-vec
// Fewer than 16 projected rows (a CFG pair is 2): no row tile to fill, so
// the weights are read once by plain FMAs.  The R rows of activations are
// staged in LDS with each 32-element block padded to 33 words; LANES lanes
// (16, or 32 / 64 for narrow outputs with long rows) take one vocab row, lane
// s owning blocks s, s + LANES, ... of it, and 32 lanes' reads of one block
// offset then fall in distinct banks (the vocab rows of a wave share the
// addresses: broadcasts).  Each lane's weights come straight from memory
// (the lanes of a vocab row read its contiguous blocks), dequantized to the
// format's exact fp32 values; each lane sums its blocks' products in element
// order, then the lanes add by a fixed tree (16-lane DPP, then exchanges
// across 16 and 32 lanes, each a commutative pair sum), so results do not
// depend on scheduling.
constexpr int kGemvWaves = 4;

// Words of one staged activation row: 33 per 32-element block.
__host__ __device__ inline int gemv_row_words(int n_embd) { return n_embd / 32 * 33; }

// The raw words of block b of vocab row v (zeros past the table): F16 its
// 16 dwords; the quantized formats the dwords covering the block from the one
// holding its first byte, and that byte's bit offset sh in it (0 or 16: rows
// and blocks start at even bytes).
template <int WT>
struct GemvRaw {
    static constexpr int N = WT == CBX_WTYPE_F16 ? 16 : (block_bytes<WT>() + 2 + 3) / 4;
    uint32_t t[N];
    uint32_t sh;
};

template <int WT>
__device__ __forceinline__ void gemv_load(const __amdgpu_buffer_rsrc_t& rw, int v, int nball, int b,
                                          GemvRaw<WT>& r) {
    if constexpr (WT == CBX_WTYPE_F16) {
        const uint32_t off = (uint32_t)(((int64_t)v * nball + b) * 64);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const auto x = __builtin_amdgcn_raw_buffer_load_b128(rw, off + 16u * i, 0, 0);
            __builtin_memcpy(&r.t[4 * i], &x, 16);
        }
        r.sh = 0;
    } else {
        constexpr int BB = block_bytes<WT>();
        const uint32_t off = (uint32_t)(((int64_t)v * nball + b) * BB);  // even
        const uint32_t a0 = off & ~3u;
        r.sh = 8u * (off & 3u);
#pragma unroll
        for (int i = 0; i < GemvRaw<WT>::N; ++i)
            r.t[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, a0 + 4u * i, 0, 0);
    }
}

// The 32 weights of a block from its raw words, exactly as the format defines
// them.
template <int WT>
__device__ __forceinline__ void gemv_decode(const GemvRaw<WT>& r, float* w) {
    if constexpr (WT == CBX_WTYPE_F16) {
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            w[2 * i] = half_bits_to_float(r.t[i] & 0xffffu);
            w[2 * i + 1] = half_bits_to_float(r.t[i] >> 16);
        }
    } else {
        constexpr int ND = GemvRaw<WT>::N;
        const uint32_t sh = r.sh;
        const float d = half_bits_to_float((r.t[0] >> sh) & 0xffffu);
        // the block's bytes after the scale, as dwords: byte 2 of the block first
        uint32_t q[ND - 1];
#pragma unroll
        for (int i = 0; i < ND - 1; ++i)
            q[i] = sh ? r.t[i + 1] : __builtin_amdgcn_alignbit(r.t[i + 1], r.t[i], 16);
        if constexpr (WT == CBX_WTYPE_Q4_0) {
            // element j < 16: low nibble of byte j; element 16 + j: its high nibble
            const float o = __fmul_rn(d, -8.0f);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t by = (q[j >> 2] >> (8 * (j & 3))) & 0xffu;
                w[j] = __fmaf_rn((float)(by & 15u), d, o);
                w[16 + j] = __fmaf_rn((float)(by >> 4), d, o);
            }
        } else if constexpr (WT == CBX_WTYPE_Q5_0) {
            // q[0] = qh; element j < 16: low nibble of byte j of q[1..4] and
            // qh bit j, element 16 + j: its high nibble and qh bit 16 + j;
            // (q - 16) d is exact in fp32, and so is the fma
            const uint32_t qh = q[0];
            const float o = __fmul_rn(d, -16.0f);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t by = (q[1 + (j >> 2)] >> (8 * (j & 3))) & 0xffu;
                w[j] = __fmaf_rn((float)((by & 15u) | (((qh >> j) & 1u) << 4)), d, o);
                w[16 + j] = __fmaf_rn((float)((by >> 4) | (((qh >> (16 + j)) & 1u) << 4)), d, o);
            }
        } else {
            const float o = __fmul_rn(d, -128.0f);
#pragma unroll
            for (int j = 0; j < 32; ++j)
                w[j] = __fmaf_rn(ubyte(q[j >> 2] ^ 0x80808080u, j & 3), d, o);
        }
    }
}

template <int WT, int RMAX, int LANES, bool NORM>
__global__ __launch_bounds__(64 * kGemvWaves) void head_gemv(
    const void* W, const float* bias, const float* hidden0, const float* hidden1,
    int64_t ld_hidden, float* out0, float* out1, int64_t ld_out, int n_rows, int n_vocab,
    int n_embd, int gelu, GemvNorm nm) {
    extern __shared__ float hs[];  // [R][gemv_row_words(n_embd)]
    const int R = hidden1 ? 2 * n_rows : n_rows;  // <= RMAX
    const int nball = n_embd / 32, rw_words = gemv_row_words(n_embd);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int s = lane & (LANES - 1), grp = lane / LANES;
    constexpr int kRowsPerWave = 64 / LANES;
    constexpr int kRowsPerPass = kRowsPerWave * kGemvWaves;
    // the first pass's first PF blocks per lane are requested before the
    // activations are staged, so their latency overlaps the staging instead
    // of following it (measured at one T3 stream with the norm folded in:
    // c_fc 7.9 -> 7.1 us, c_attn 6.8 -> 6.5 us); the kernels for more rows
    // keep their registers for the rows' sums instead
    constexpr int PF = (NORM || RMAX <= 2) ? 2 : 0;
    constexpr int64_t kBB = block_bytes<WT>();
    const int64_t wbytes = (int64_t)n_vocab * nball * kBB;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(W), (short)0, (int)wbytes, kBufWord3);
    // the rows' step flags, requested before the weights: waiting for them
    // then does not wait for the weights too (loads return in order)
    int act_r[RMAX];
    if constexpr (NORM) {
#pragma unroll
        for (int r = 0; r < RMAX; ++r) act_r[r] = r < R ? nm.act[r] : 0;
    }
    GemvRaw<WT> pre[PF > 0 ? PF : 1];
    {
        const int v = blockIdx.x * kRowsPerPass + wave * kRowsPerWave + grp;
        const int vc = v < n_vocab ? v : n_vocab;
#pragma unroll
        for (int p = 0; p < PF; ++p)
            if (s + p * LANES < nball) gemv_load<WT>(rw, vc, nball, s + p * LANES, pre[p]);
    }
    if constexpr (NORM) {
        // the rows' residual add and layer norm (the T3 layer's, same
        // operations in the same order as its norm kernel, block_sum256
        // included), into LDS; workgroup 0 stores the new residual rows
        __shared__ float red[2 * kGemvWaves];
        static_assert(kGemvWaves == 4, "block_sum256 takes 256 threads");
        int ph = 0;
        const int ept = n_embd / (64 * kGemvWaves);  // <= 16
        for (int r = 0; r < R; ++r) {
            const float* xr = nm.x_in + (int64_t)r * n_embd;
            const float* yr = nm.y + (int64_t)r * n_embd;
            float* xo = nm.x_out + (int64_t)r * n_embd;
            float* hr = hs + r * rw_words;
            float xv[16];
            int act = act_r[0];
#pragma unroll
            for (int q = 1; q < RMAX; ++q) act = r == q ? act_r[q] : act;
            if (act == 0) {  // a stream that takes no step: zeros, x kept
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int k = j * 64 * kGemvWaves + tid;
                    if (j < ept) {
                        hr[(k >> 5) * 33 + (k & 31)] = 0.0f;
                        if (blockIdx.x == 0) xo[k] = xr[k];
                    }
                }
                continue;
            }
            // x + y in chunks of 4 values per thread, each chunk's loads
            // first, then its adds (one wait per chunk: one for n_embd 1024)
            float sum = 0.0f;
#pragma unroll
            for (int j0 = 0; j0 < 16; j0 += 4) {
                if (j0 < ept) {
                    // unconditional loads (indices clamped to the row), so
                    // the four are issued before the first add waits
                    float xa[4], ya[4];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int k = min(j0 + q, ept - 1) * 64 * kGemvWaves + tid;
                        xa[q] = xr[k];
                        ya[q] = yr[k];
                    }
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int j = j0 + q;
                        if (j < ept) {
                            xv[j] = __fadd_rn(ya[q], xa[q]);
                            sum = __fadd_rn(sum, xv[j]);
                        }
                    }
                }
            }
            // the first chunk's g and b, requested now: they arrive during
            // the reductions (later chunks' with their stores)
            float g0[4], b0[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int k = min(q, ept - 1) * 64 * kGemvWaves + tid;
                g0[q] = nm.g[k];
                b0[q] = nm.b[k];
            }
            const float mean = __fdiv_rn(block_sum256(sum, red, ph), (float)n_embd);
            float q2 = 0.0f;
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                if (j < ept) {
                    const float d = __fsub_rn(xv[j], mean);
                    q2 = __fadd_rn(q2, __fmul_rn(d, d));
                }
            }
            const float var = __fdiv_rn(block_sum256(q2, red, ph), (float)n_embd);
            const float scale = __fdiv_rn(1.0f, __fsqrt_rn(__fadd_rn(var, nm.eps)));
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                if (j < ept) {
                    const int k = j * 64 * kGemvWaves + tid;
                    const float gj = j < 4 ? g0[j & 3] : nm.g[k];
                    const float bj = j < 4 ? b0[j & 3] : nm.b[k];
                    if (blockIdx.x == 0) xo[k] = xv[j];
                    hr[(k >> 5) * 33 + (k & 31)] = __fadd_rn(
                        __fmul_rn(__fmul_rn(__fsub_rn(xv[j], mean), scale), gj), bj);
                }
            }
        }
    } else {
        // the rows into LDS, kStage values per thread requested together and
        // then written: one memory round trip per batch, not one per value
        constexpr int kStage = 16;
        const int total = R * n_embd;
        for (int i0 = 0; i0 < total; i0 += 64 * kGemvWaves * kStage) {
            float v[kStage];
#pragma unroll
            for (int q = 0; q < kStage; ++q) {
                const int i = i0 + q * 64 * kGemvWaves + tid;
                const int r = i / n_embd, k = i - r * n_embd;
                const float* src = r < n_rows ? hidden0 + (int64_t)r * ld_hidden
                                              : hidden1 + (int64_t)(r - n_rows) * ld_hidden;
                v[q] = i < total ? src[k] : 0.0f;
            }
#pragma unroll
            for (int q = 0; q < kStage; ++q) {
                const int i = i0 + q * 64 * kGemvWaves + tid;
                const int r = i / n_embd, k = i - r * n_embd;
                if (i < total) hs[r * rw_words + (k >> 5) * 33 + (k & 31)] = v[q];
            }
        }
    }
    __syncthreads();
    bool first = true;
    for (int vb = blockIdx.x * kRowsPerPass; vb < n_vocab; vb += gridDim.x * kRowsPerPass) {
        const int v = vb + wave * kRowsPerWave + grp;
        const int vc = v < n_vocab ? v : n_vocab;  // past the table: zeros
        float acc[RMAX];
#pragma unroll
        for (int r = 0; r < RMAX; ++r) acc[r] = 0.0f;
        // block b's products, in block order
        auto block = [&](const GemvRaw<WT>& raw, int b) {
            float w[32];
            gemv_decode<WT>(raw, w);
            const float* hb = hs + b * 33;
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                if (r < R) {
                    const float* h = hb + r * rw_words;
                    float a = acc[r];
#pragma unroll
                    for (int j = 0; j < 32; ++j) a = __fmaf_rn(w[j], h[j], a);
                    acc[r] = a;
                }
            }
        };
        int b = s;
        if (first) {  // the prefetched blocks of this pass's row
#pragma unroll
            for (int p = 0; p < PF; ++p, b += LANES)
                if (b < nball) block(pre[p], b);
            first = false;
        }
        for (; b < nball; b += LANES) {
            GemvRaw<WT> raw;
            gemv_load<WT>(rw, vc, nball, b, raw);
            block(raw, b);
        }
        // the lanes' sums: lane 15 of each 16-lane row ends with its total,
        // then lanes 16 and 32 apart add theirs, so lane LANES - 1 of each
        // group ends with the total
#pragma unroll
        for (int r = 0; r < RMAX; ++r) {
            float a = acc[r];
            a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                           0, __builtin_bit_cast(int, a), 0x111, 0xf, 0xf, false)));
            a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                           0, __builtin_bit_cast(int, a), 0x112, 0xf, 0xf, false)));
            a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                           0, __builtin_bit_cast(int, a), 0x114, 0xf, 0xf, false)));
            a = __fadd_rn(a, __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
                                                           0, __builtin_bit_cast(int, a), 0x118, 0xf, 0xf, false)));
            if constexpr (LANES >= 32) a = __fadd_rn(a, __shfl_xor(a, 16));
            if constexpr (LANES >= 64) a = __fadd_rn(a, __shfl_xor(a, 32));
            acc[r] = a;
        }
        if (s == LANES - 1 && v < n_vocab) {
            const float bv = bias ? bias[v] : 0.0f;
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                if (r < R) {
                    float* o = r < n_rows ? out0 + (int64_t)r * ld_out
                                          : out1 + (int64_t)(r - n_rows) * ld_out;
                    const float x = __fadd_rn(acc[r], bv);
                    o[v] = gelu ? t3_gelu_f(x) : x;
                }
            }
        }
    }
}

template <int WT, int RMAX, int LANES, bool NORM>
hipError_t launch_gemv_l(const void* W, const float* bias, const float* hidden0,
                         const float* hidden1, int64_t ld_hidden, float* out0, float* out1,
                         int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                         hipStream_t stream, int gelu, const GemvNorm& nm) {
    const int R = hidden1 ? 2 * n_rows : n_rows;
    const size_t lds = (size_t)R * gemv_row_words(n_embd) * 4;
    constexpr int kRowsPerPass = 64 / LANES * kGemvWaves;
    const unsigned grid = (unsigned)((n_vocab + kRowsPerPass - 1) / kRowsPerPass);
    hipLaunchKernelGGL((head_gemv<WT, RMAX, LANES, NORM>), dim3(grid), dim3(64 * kGemvWaves),
                       lds, stream, W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out,
                       n_rows, n_vocab, n_embd, gelu, nm);
    return hipGetLastError();
}

// Lanes per vocab row: 16, doubled (to 64 at most) while the grid would hold
// fewer than 256 workgroups and every lane keeps a block (narrow outputs: the
// T3 layers' products at one stream).
template <int WT, int RMAX, bool NORM = false>
hipError_t launch_gemv(const void* W, const float* bias, const float* hidden0, const float* hidden1,
                       int64_t ld_hidden, float* out0, float* out1, int64_t ld_out, int32_t n_rows,
                       int32_t n_vocab, int32_t n_embd, hipStream_t stream, int gelu,
                       const GemvNorm& nm = GemvNorm{}) {
    const int nball = n_embd / 32;
    int lanes = 16;
    while (lanes < 64 && (n_vocab + 64 / lanes * kGemvWaves - 1) / (64 / lanes * kGemvWaves) < 256 &&
           nball >= 2 * lanes)
        lanes *= 2;
    if (lanes == 64)
        return launch_gemv_l<WT, RMAX, 64, NORM>(W, bias, hidden0, hidden1, ld_hidden, out0, out1,
                                                 ld_out, n_rows, n_vocab, n_embd, stream, gelu, nm);
    if (lanes == 32)
        return launch_gemv_l<WT, RMAX, 32, NORM>(W, bias, hidden0, hidden1, ld_hidden, out0, out1,
                                                 ld_out, n_rows, n_vocab, n_embd, stream, gelu, nm);
    return launch_gemv_l<WT, RMAX, 16, NORM>(W, bias, hidden0, hidden1, ld_hidden, out0, out1,
                                             ld_out, n_rows, n_vocab, n_embd, stream, gelu, nm);
}

template <int WT>
hipError_t launch_gemv_r(const void* W, const float* bias, const float* hidden0,
                         const float* hidden1, int64_t ld_hidden, float* out0, float* out1,
                         int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                         hipStream_t stream, int gelu) {
    const int R = hidden1 ? 2 * n_rows : n_rows;
    if (R <= 2)
        return launch_gemv<WT, 2>(W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                                  n_vocab, n_embd, stream, gelu);
    if (R <= 4)
        return launch_gemv<WT, 4>(W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                                  n_vocab, n_embd, stream, gelu);
    if (R <= 8)
        return launch_gemv<WT, 8>(W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                                  n_vocab, n_embd, stream, gelu);
    return launch_gemv<WT, 16>(W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                               n_vocab, n_embd, stream, gelu);
}

template <int WT, int NT>
hipError_t launch_mfma(const void* W, const float* bias, const uint32_t* parts, const float* inv,
                       int n_tiles, float* out0, float* out1, int64_t ld_out, int n_rows,
                       int n_vocab, int n_embd, hipStream_t stream, int kz = 1,
                       int gelu_out = 0, uint32_t* out_parts = nullptr,
                       float* out_inv = nullptr) {
    const dim3 grid((unsigned)((n_vocab + 31) / 32), (unsigned)((n_tiles + NT - 1) / NT),
                    (unsigned)kz);
    hipLaunchKernelGGL((head_mfma<WT, NT>), grid, dim3(64 * KS), 0, stream, W, bias, parts, inv,
                       n_tiles, out0, out1, ld_out, n_rows, n_vocab, n_embd,
                       (int64_t)n_rows * ld_out, gelu_out, out_parts, out_inv);
    return hipGetLastError();
}

// The matrix-core products on split activations: one row tile per workgroup
// where two would leave fewer than 512 workgroups (narrow outputs, few rows:
// the T3 layer products), the K is split or the outputs are split for the
// next product; else two row tiles per workgroup for Q4_0 and for at most
// two tiles.
hipError_t mfma_dispatch(const void* W, int32_t wtype, const float* bias, const uint32_t* parts,
                         const float* inv, int n_tiles, float* out0, float* out1, int64_t ld_out,
                         int32_t n_rows, int32_t n_vocab, int32_t n_embd, hipStream_t stream,
                         int kz, int gelu_out, uint32_t* out_parts = nullptr,
                         float* out_inv = nullptr) {
    if ((int64_t)((n_vocab + 31) / 32) * ((n_tiles + 1) / 2) < 512 || kz > 1 || gelu_out ||
        out_parts) {
        switch (wtype) {
            case CBX_WTYPE_F16:
                return launch_mfma<CBX_WTYPE_F16, 1>(W, bias, parts, inv, n_tiles, out0, out1,
                                                     ld_out, n_rows, n_vocab, n_embd, stream, kz,
                                                     gelu_out, out_parts, out_inv);
            case CBX_WTYPE_Q4_0:
                return launch_mfma<CBX_WTYPE_Q4_0, 1>(W, bias, parts, inv, n_tiles, out0, out1,
                                                      ld_out, n_rows, n_vocab, n_embd, stream, kz,
                                                     gelu_out, out_parts, out_inv);
            case CBX_WTYPE_Q5_0:
                return launch_mfma<CBX_WTYPE_Q5_0, 1>(W, bias, parts, inv, n_tiles, out0, out1,
                                                      ld_out, n_rows, n_vocab, n_embd, stream, kz,
                                                      gelu_out, out_parts, out_inv);
            case CBX_WTYPE_Q8_0:
                return launch_mfma<CBX_WTYPE_Q8_0, 1>(W, bias, parts, inv, n_tiles, out0, out1,
                                                      ld_out, n_rows, n_vocab, n_embd, stream, kz,
                                                     gelu_out, out_parts, out_inv);
            default:
                return hipErrorInvalidValue;
        }
    }
    const bool two = wtype == CBX_WTYPE_Q4_0 || wtype == CBX_WTYPE_Q5_0 || n_tiles <= 2;
    switch (wtype) {
        case CBX_WTYPE_F16:
            return two ? launch_mfma<CBX_WTYPE_F16, 2>(W, bias, parts, inv, n_tiles, out0, out1,
                                                       ld_out, n_rows, n_vocab, n_embd, stream)
                       : launch_mfma<CBX_WTYPE_F16, 4>(W, bias, parts, inv, n_tiles, out0, out1,
                                                       ld_out, n_rows, n_vocab, n_embd, stream);
        case CBX_WTYPE_Q4_0:
            return launch_mfma<CBX_WTYPE_Q4_0, 2>(W, bias, parts, inv, n_tiles, out0, out1, ld_out,
                                                  n_rows, n_vocab, n_embd, stream);
        case CBX_WTYPE_Q5_0:
            return launch_mfma<CBX_WTYPE_Q5_0, 2>(W, bias, parts, inv, n_tiles, out0, out1, ld_out,
                                                  n_rows, n_vocab, n_embd, stream);
        case CBX_WTYPE_Q8_0:
            return two ? launch_mfma<CBX_WTYPE_Q8_0, 2>(W, bias, parts, inv, n_tiles, out0, out1,
                                                        ld_out, n_rows, n_vocab, n_embd, stream)
                       : launch_mfma<CBX_WTYPE_Q8_0, 4>(W, bias, parts, inv, n_tiles, out0, out1,
                                                        ld_out, n_rows, n_vocab, n_embd, stream);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace

bool head_uses_gemv(int32_t n_rows, bool cfg, int32_t n_embd) {
    const int R = cfg ? 2 * n_rows : n_rows;
    return R < 16 && (size_t)R * gemv_row_words(n_embd) * 4 <= 65536;
}

size_t head_scratch_bytes(int32_t n_rows, bool cfg, int32_t n_embd) {
    const int n_tiles = ((n_rows + 15) / 16) * (cfg ? 2 : 1);
    return head_uses_gemv(n_rows, cfg, n_embd) ? 0 : split_bytes(16 * n_tiles, n_embd);
}

hipError_t launch_head(const void* W, int32_t wtype, const float* bias, const float* hidden0,
                       const float* hidden1, int64_t ld_hidden, float* out0, float* out1,
                       int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                       void* scratch, hipStream_t stream) {
    return launch_head_k(W, wtype, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                         n_vocab, n_embd, scratch, stream, 1, false);
}

int head_k_split(int32_t n_rows, int32_t n_vocab, int32_t n_embd) {
    if (head_uses_gemv(n_rows, false, n_embd)) return 1;
    const int64_t wg = (int64_t)((n_vocab + 31) / 32) * ((n_rows + 15) / 16);  // one tile each
    const int nball = n_embd / 32;
    int kz = 1;
    while (kz < 8 && wg * kz < 512 && nball / (2 * kz * KS) >= 4) kz *= 2;
    return kz;
}

hipError_t launch_head_k(const void* W, int32_t wtype, const float* bias, const float* hidden0,
                         const float* hidden1, int64_t ld_hidden, float* out0, float* out1,
                         int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                         void* scratch, hipStream_t stream, int kz, bool gelu_out) {
    // fewer than 16 projected rows: the mat-vec (activations staged in LDS,
    // at most 64 KiB of them), else the split and the 16-row matrix-core tiles
    const bool cfg = hidden1 != nullptr;
    if (kz < 1 || (kz > 1 && (cfg || gelu_out || head_uses_gemv(n_rows, cfg, n_embd))))
        return hipErrorInvalidValue;  // a K split: one row set on the matrix cores, no gelu
    if (head_uses_gemv(n_rows, cfg, n_embd)) {
        switch (wtype) {
            case CBX_WTYPE_F16:
                return launch_gemv_r<CBX_WTYPE_F16>(W, bias, hidden0, hidden1, ld_hidden, out0,
                                                    out1, ld_out, n_rows, n_vocab, n_embd, stream,
                                                    gelu_out ? 1 : 0);
            case CBX_WTYPE_Q4_0:
                return launch_gemv_r<CBX_WTYPE_Q4_0>(W, bias, hidden0, hidden1, ld_hidden, out0,
                                                     out1, ld_out, n_rows, n_vocab, n_embd, stream,
                                                    gelu_out ? 1 : 0);
            case CBX_WTYPE_Q5_0:
                return launch_gemv_r<CBX_WTYPE_Q5_0>(W, bias, hidden0, hidden1, ld_hidden, out0,
                                                     out1, ld_out, n_rows, n_vocab, n_embd, stream,
                                                     gelu_out ? 1 : 0);
            case CBX_WTYPE_Q8_0:
                return launch_gemv_r<CBX_WTYPE_Q8_0>(W, bias, hidden0, hidden1, ld_hidden, out0,
                                                     out1, ld_out, n_rows, n_vocab, n_embd, stream,
                                                    gelu_out ? 1 : 0);
            default:
                return hipErrorInvalidValue;
        }
    }
    if (!scratch) return hipErrorInvalidValue;
    const int n_tiles = ((n_rows + 15) / 16) * (cfg ? 2 : 1), R = 16 * n_tiles;
    uint32_t* parts = static_cast<uint32_t*>(scratch);
    float* inv = reinterpret_cast<float*>(static_cast<char*>(scratch) + split_inv_offset(R, n_embd));
    const int64_t groups = (int64_t)R * (n_embd / 8);
    hipLaunchKernelGGL(head_split, dim3((unsigned)((groups + kSplitThreads - 1) / kSplitThreads)),
                       dim3(kSplitThreads), 0, stream, hidden0, hidden1, ld_hidden, n_rows, n_embd,
                       R, parts, inv);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return mfma_dispatch(W, wtype, bias, parts, inv, n_tiles, out0, out1, ld_out, n_rows, n_vocab,
                         n_embd, stream, kz, gelu_out ? 1 : 0);
}

hipError_t launch_head_presplit(const void* W, int32_t wtype, const float* bias, float* out0,
                                int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                                const void* scratch, hipStream_t stream, int kz, bool gelu_out,
                                void* out_split) {
    if (!scratch || kz < 1 || head_uses_gemv(n_rows, false, n_embd) || (gelu_out && kz > 1) ||
        (out_split && (kz > 1 || n_vocab % 32 != 0)))
        return hipErrorInvalidValue;
    const int n_tiles = (n_rows + 15) / 16, R = 16 * n_tiles;
    const uint32_t* parts = static_cast<const uint32_t*>(scratch);
    const float* inv =
        reinterpret_cast<const float*>(static_cast<const char*>(scratch) + split_inv_offset(R, n_embd));
    uint32_t* out_parts = static_cast<uint32_t*>(out_split);
    float* out_inv = out_split ? reinterpret_cast<float*>(static_cast<char*>(out_split) +
                                                          split_inv_offset(R, n_vocab))
                               : nullptr;
    return mfma_dispatch(W, wtype, bias, parts, inv, n_tiles, out0, nullptr, ld_out, n_rows,
                         n_vocab, n_embd, stream, kz, gelu_out ? 1 : 0, out_parts, out_inv);
}

hipError_t launch_head_gemv_norm(const void* W, int32_t wtype, const float* bias,
                                 const GemvNorm& nm, float* out, int64_t ld_out, int32_t n_rows,
                                 int32_t n_vocab, int32_t n_embd, hipStream_t stream, bool gelu) {
    if (n_rows < 1 || n_rows > 2 || n_embd % (64 * kGemvWaves) != 0 ||
        n_embd > 16 * 64 * kGemvWaves || !head_uses_gemv(n_rows, false, n_embd))
        return hipErrorInvalidValue;
    const int g = gelu ? 1 : 0;
    switch (wtype) {
        case CBX_WTYPE_F16:
            return launch_gemv<CBX_WTYPE_F16, 2, true>(W, bias, nullptr, nullptr, n_embd, out,
                                                       nullptr, ld_out, n_rows, n_vocab, n_embd,
                                                       stream, g, nm);
        case CBX_WTYPE_Q4_0:
            return launch_gemv<CBX_WTYPE_Q4_0, 2, true>(W, bias, nullptr, nullptr, n_embd, out,
                                                        nullptr, ld_out, n_rows, n_vocab, n_embd,
                                                        stream, g, nm);
        case CBX_WTYPE_Q5_0:
            return launch_gemv<CBX_WTYPE_Q5_0, 2, true>(W, bias, nullptr, nullptr, n_embd, out,
                                                        nullptr, ld_out, n_rows, n_vocab, n_embd,
                                                        stream, g, nm);
        case CBX_WTYPE_Q8_0:
            return launch_gemv<CBX_WTYPE_Q8_0, 2, true>(W, bias, nullptr, nullptr, n_embd, out,
                                                        nullptr, ld_out, n_rows, n_vocab, n_embd,
                                                        stream, g, nm);
        default:
            return hipErrorInvalidValue;
    }
}

}  // namespace cbx
