// cbx_head.hip -- the T3 speech_head projection on the matrix cores:
// logits[r][v] = sum_k W[v][k] * h[r][k] + b[v]   (src/main.cpp:577; the weights
// and bias are chatterbox/speech_head(_bias), main.cpp:394-395), for F16, Q4_0
// and Q8_0 weights in ggml's layout (ne = [n_embd, n_vocab]: row v holds the
// n_embd weights of vocab id v; Q4_0 blocks are an fp16 scale d and 16 bytes
// of nibbles, element j < 16 in the low nibble of byte j and element j + 16
// in its high nibble, w = (q - 8) d; Q8_0 blocks are d and 32 int8, w = q d).
//
// A workgroup of KS wavefronts computes 32 vocab ids x NT row tiles of 16
// rows with v_mfma_f32_16x16x4_f32 (two 16x16 accumulators per tile per
// wave); the row tiles run over the tiles of the first (cond) row set, then
// those of the second (uncond), so one workgroup can serve both.  Wave w
// takes the w-th of KS runs of 32-weight blocks along n_embd, and the KS
// partial tiles are added in wave order through LDS (a fixed order: results
// do not depend on scheduling).  Lane l feeds A[l%16][l/16]
// and B[l/16][l%16] and holds D[4(l/16)+i][l%16] in accumulator register i.
// Inside a 32-weight block, step s (0..7) and lane group g = l/16 carry
// k = 8g + s, so each lane dequantizes 8 consecutive weights of one block per
// vocab row (one fp16 scale, 8 bytes of nibbles or int8) and reads 8
// consecutive activations: the same k assignment on both operands makes the
// tile's dot products exact sums over every k.  Weights are dequantized in
// registers to the fp32 value the format defines (exactly representable);
// products and sums are the matrix core's fp32.  Rows v >= n_vocab and
// r >= n_rows read zeros through the buffer descriptors' ranges and store
// nothing.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "cbx_internal.h"

namespace cbx {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
constexpr int32_t kBufWord3 = 0x00020000;  // raw buffer: 32-bit data format

__device__ __forceinline__ float half_bits_to_float(uint32_t hb) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)hb);
}

// Raw bytes of the 8 weights k = 8g .. 8g + 7 of one block of a vocab row,
// from the row's chunk staged in LDS: F16 four dwords; Q4_0 / Q8_0 the fp16
// scale in q[4] and the 8 bytes of nibbles or int8 in q[0..1].  Blocks are
// 18 or 34 bytes, so only 2-byte alignment holds: `off` (the block's byte
// offset in the staged row) is read as dwords shifted into place.
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
        const int qoff = off + 2 + (WT == CBX_WTYPE_Q4_0 ? 8 * (g & 1) : 8 * g);
        const uint32_t* p = srow + (qoff >> 2);
        const uint32_t sh = 8u * (uint32_t)(qoff & 3);
        const uint32_t t0 = p[0], t1 = p[1], t2 = p[2];
        q[0] = __builtin_amdgcn_alignbit(t1, t0, sh);
        q[1] = __builtin_amdgcn_alignbit(t2, t1, sh);
    }
}

__device__ __forceinline__ float ubyte(uint32_t x, int i) { return (float)((x >> (8 * i)) & 0xffu); }

// The fp32 weights the format defines, from lds_w's bytes.  Q4_0: nibble
// n = q + 8 and w = (n - 8) d = fma(n, d, -8d), exact (n d and -8d are exact
// and their sum is representable); Q8_0: u = q + 128 (sign bit flipped) and
// w = fma(u, d, -128d), exact for the same reason.
template <int WT>
__device__ __forceinline__ void dequant(const uint32_t* q, int g, float* w) {
    if constexpr (WT == CBX_WTYPE_F16) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[2 * i] = half_bits_to_float(q[i] & 0xffffu);
            w[2 * i + 1] = half_bits_to_float(q[i] >> 16);
        }
    } else {
        const float d = half_bits_to_float(q[4]);
        uint32_t x0, x1;
        float off;
        if constexpr (WT == CBX_WTYPE_Q4_0) {
            const int sh = g < 2 ? 0 : 4;
            x0 = (q[0] >> sh) & 0x0f0f0f0fu;
            x1 = (q[1] >> sh) & 0x0f0f0f0fu;
            off = __fmul_rn(d, -8.0f);
        } else {
            x0 = q[0] ^ 0x80808080u;
            x1 = q[1] ^ 0x80808080u;
            off = __fmul_rn(d, -128.0f);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = __fmaf_rn(ubyte(x0, i), d, off);
            w[4 + i] = __fmaf_rn(ubyte(x1, i), d, off);
        }
    }
}

constexpr int KS = 4;  // waves per workgroup (runs of blocks along n_embd)
// Row tiles of 16 per workgroup: each dequantized weight feeds the products
// of NT tiles, so weight loads and dequantization are shared by 16*NT rows
// (NT = 4: 37.2 -> 31.7 us at 128 rows, V = 6563; NT = 8 leaves one wave
// per SIMD and ran slower).
constexpr int NT = 4;

template <int WT>
__global__ __launch_bounds__(64 * KS) void head_mfma(const void* W, const float* bias,
                                                     const float* hidden0, const float* hidden1,
                                                     int64_t ld_hidden, float* out0, float* out1,
                                                     int64_t ld_out, int n_rows, int n_vocab,
                                                     int n_embd) {
    constexpr int BB = WT == CBX_WTYPE_F16 ? 64 : (WT == CBX_WTYPE_Q4_0 ? 18 : 34);
    // Weights are staged per wave in chunks of CB blocks: for each of the 32
    // vocab rows the chunk's CB * BB bytes are contiguous, so whole-row dword
    // loads touch two or three lines each (the per-block loads of the 18-byte
    // pieces of 16 rows 576 bytes apart touched up to 32 lines each, and the
    // texture-address path was the measured limit).  RSW dwords per staged
    // row: the bytes from the dword holding the first, plus one.
    constexpr int CB = WT == CBX_WTYPE_F16 ? 4 : 8;
    constexpr int RSW = (CB * BB + 6) / 4 + 1;
    __shared__ uint32_t stage[KS][32 * RSW];
    __shared__ f4 part[KS - 1][2 * NT][64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int m = lane & 15, g = lane >> 4;
    const int v0 = blockIdx.x * 32;
    constexpr int64_t kBlockBytes = WT == CBX_WTYPE_F16 ? 64 : (WT == CBX_WTYPE_Q4_0 ? 18 : 34);
    const int64_t wbytes = (int64_t)n_vocab * (n_embd / 32) * kBlockBytes;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(W), (short)0, (int)wbytes, kBufWord3);
    const int hbytes = (int)(((int64_t)(n_rows - 1) * ld_hidden + n_embd) * 4);
    const __amdgpu_buffer_rsrc_t rh0 =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(hidden0), (short)0, hbytes, kBufWord3);
    const __amdgpu_buffer_rsrc_t rh1 = hidden1 ? __builtin_amdgcn_make_buffer_rsrc(
                                                     const_cast<float*>(hidden1), (short)0, hbytes,
                                                     kBufWord3)
                                               : rh0;
    const int va = v0 + m, vb = v0 + 16 + m;
    // rows past the table read zeros (byte offsets past the range)
    const int va_c = va < n_vocab ? va : n_vocab, vb_c = vb < n_vocab ? vb : n_vocab;
    // Row tile T = blockIdx.y * NT + t of the tiles of both row sets (those
    // of hidden0, then those of hidden1): set T / tps, rows 16 (T % tps) ...
    const int tps = (n_rows + 15) / 16, n_tiles = hidden1 ? 2 * tps : tps;
    int64_t hrow[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int T = blockIdx.y * NT + t;
        const int rr = (T % tps) * 16 + m;
        hrow[t] = (T < n_tiles && rr < n_rows) ? (int64_t)rr * ld_hidden
                                                : ((int64_t)n_rows * ld_hidden + n_embd);
    }
    f4 acc0[NT], acc1[NT];
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        acc0[t] = f4{0.0f, 0.0f, 0.0f, 0.0f};
        acc1[t] = acc0[t];
    }
    const int nball = n_embd / 32;
    const int kb0 = nball * wave / KS, kb1 = nball * (wave + 1) / KS;
    // block kb + 1's loads are in flight while block kb's products run
    // (more blocks in flight measured slower: the loads' throughput, not
    // their latency, is what the products wait for)
    uint32_t qa[5], qb[5];
    f4 h0[NT], h1[NT];
    auto load = [&](int kb) {
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const int T = blockIdx.y * NT + t;
            const __amdgpu_buffer_rsrc_t rh = T >= tps ? rh1 : rh0;
            const uint32_t hoff = (uint32_t)((hrow[t] + kb * 32 + 8 * g) * 4);
            h0[t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rh, hoff, 0, 0));
            h1[t] = __builtin_bit_cast(f4, __builtin_amdgcn_raw_buffer_load_b128(rh, hoff + 16, 0, 0));
        }
    };
    if (kb0 < kb1) load(kb0);
    uint32_t* const sw = stage[wave];
#pragma unroll 1
    for (int kbc = kb0; kbc < kb1; kbc += CB) {
        const int nb = min(CB, kb1 - kbc);
        // stage rows v0 .. v0 + 31 (rows past the table read zeros): the
        // dwords from the one holding the chunk's first byte
        const int ndw = (3 + nb * BB + 3) >> 2;  // <= RSW - 1
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        {
            int rr = lane / ndw, d = lane % ndw;
            const int q64 = 64 / ndw, r64 = 64 % ndw;
            for (int i = lane; i < 32 * ndw; i += 64) {
                const int v = v0 + rr < n_vocab ? v0 + rr : n_vocab;
                const uint32_t a0 = (uint32_t)(((int64_t)v * nball + kbc) * BB) & ~3u;
                sw[rr * RSW + d] =
                    (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, a0 + 4u * (uint32_t)d, 0, 0);
                d += r64;
                rr += q64;
                if (d >= ndw) {
                    d -= ndw;
                    ++rr;
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const int sha = (int)((((int64_t)va_c * nball + kbc) * BB) & 3);
        const int shb = (int)((((int64_t)vb_c * nball + kbc) * BB) & 3);
#pragma unroll 1
    for (int kb = kbc; kb < kbc + nb; ++kb) {
        lds_w<WT>(sw + m * RSW, sha + (kb - kbc) * BB, g, qa);
        lds_w<WT>(sw + (16 + m) * RSW, shb + (kb - kbc) * BB, g, qb);
        float wa[8], wb[8];
        dequant<WT>(qa, g, wa);
        dequant<WT>(qb, g, wb);
        float hv[NT][8];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                hv[t][e] = h0[t][e];
                hv[t][4 + e] = h1[t][e];
            }
        }
        if (kb + 1 < kb1) load(kb + 1);
#pragma unroll
        for (int s = 0; s < 8; ++s) {
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                acc0[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[s], hv[t][s], acc0[t], 0, 0, 0);
                acc1[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(wb[s], hv[t][s], acc1[t], 0, 0, 0);
            }
        }
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
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const int T = blockIdx.y * NT + t;
        const int rr = (T % tps) * 16 + m;
        if (T < n_tiles && rr < n_rows) {
            float* orow = (T >= tps ? out1 : out0) + (int64_t)rr * ld_out;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int v = v0 + 4 * g + i, v2 = v + 16;
                if (v < n_vocab) orow[v] = __fadd_rn(acc0[t][i], bias ? bias[v] : 0.0f);
                if (v2 < n_vocab) orow[v2] = __fadd_rn(acc1[t][i], bias ? bias[v2] : 0.0f);
            }
        }
    }
}

// ----------------------------------------------------------------- mat-vec
// Fewer than 16 projected rows (a CFG pair is 2): no row tile to fill, so
// the weights are read once by plain FMAs.  The R rows of activations are
// staged in LDS with each 32-element block padded to 33 words; 16 lanes take
// one vocab row, lane s owning blocks s, s + 16, ... of it, and the 16 lanes'
// reads of one block offset then fall in distinct banks (the four vocab rows
// of a wave share the addresses: broadcasts).  Each lane's weights come
// straight from memory (the 16 lanes of a vocab row read its contiguous
// blocks), dequantized to the format's exact fp32 values; each lane sums its
// blocks' products in element order, then the 16 lanes add by a fixed DPP
// tree, so results do not depend on scheduling.
constexpr int kGemvLanes = 16;       // lanes per vocab row
constexpr int kGemvRowsPerWave = 4;  // vocab rows per wave and pass
constexpr int kGemvWaves = 4;

// Words of one staged activation row: 33 per 32-element block.
__host__ __device__ inline int gemv_row_words(int n_embd) { return n_embd / 32 * 33; }

// The 32 weights of block b of vocab row v (zeros past the table).
template <int WT>
__device__ __forceinline__ void gemv_block(const __amdgpu_buffer_rsrc_t& rw, int v, int nball, int b,
                                           float* w) {
    if constexpr (WT == CBX_WTYPE_F16) {
        const uint32_t off = (uint32_t)(((int64_t)v * nball + b) * 64);
        uint32_t t[16];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const auto x = __builtin_amdgcn_raw_buffer_load_b128(rw, off + 16u * i, 0, 0);
            uint32_t y[4];
            __builtin_memcpy(y, &x, 16);
#pragma unroll
            for (int c = 0; c < 4; ++c) t[4 * i + c] = y[c];
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            w[2 * i] = half_bits_to_float(t[i] & 0xffffu);
            w[2 * i + 1] = half_bits_to_float(t[i] >> 16);
        }
    } else {
        constexpr int BB = WT == CBX_WTYPE_Q4_0 ? 18 : 34;
        constexpr int ND = WT == CBX_WTYPE_Q4_0 ? 5 : 9;  // dwords covering the block
        const uint32_t off = (uint32_t)(((int64_t)v * nball + b) * BB);  // even
        const uint32_t a0 = off & ~3u, sh = 8u * (off & 3u);               // sh: 0 or 16
        uint32_t t[ND];
#pragma unroll
        for (int i = 0; i < ND; ++i)
            t[i] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, a0 + 4u * i, 0, 0);
        const float d = half_bits_to_float((t[0] >> sh) & 0xffffu);
        // the block's bytes after the scale, as dwords: byte 2 of the block first
        uint32_t q[ND - 1];
#pragma unroll
        for (int i = 0; i < ND - 1; ++i)
            q[i] = sh ? t[i + 1] : __builtin_amdgcn_alignbit(t[i + 1], t[i], 16);
        if constexpr (WT == CBX_WTYPE_Q4_0) {
            // element j < 16: low nibble of byte j; element 16 + j: its high nibble
            const float o = __fmul_rn(d, -8.0f);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t by = (q[j >> 2] >> (8 * (j & 3))) & 0xffu;
                w[j] = __fmaf_rn((float)(by & 15u), d, o);
                w[16 + j] = __fmaf_rn((float)(by >> 4), d, o);
            }
        } else {
            const float o = __fmul_rn(d, -128.0f);
#pragma unroll
            for (int j = 0; j < 32; ++j)
                w[j] = __fmaf_rn(ubyte(q[j >> 2] ^ 0x80808080u, j & 3), d, o);
        }
    }
}

template <int WT, int RMAX>
__global__ __launch_bounds__(64 * kGemvWaves) void head_gemv(
    const void* W, const float* bias, const float* hidden0, const float* hidden1,
    int64_t ld_hidden, float* out0, float* out1, int64_t ld_out, int n_rows, int n_vocab,
    int n_embd) {
    extern __shared__ float hs[];  // [R][gemv_row_words(n_embd)]
    const int R = hidden1 ? 2 * n_rows : n_rows;  // <= RMAX
    const int nball = n_embd / 32, rw_words = gemv_row_words(n_embd);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int s = lane & (kGemvLanes - 1), grp = lane / kGemvLanes;
    for (int i = tid; i < R * n_embd; i += 64 * kGemvWaves) {
        const int r = i / n_embd, k = i - r * n_embd;
        const float* src = r < n_rows ? hidden0 + (int64_t)r * ld_hidden
                                      : hidden1 + (int64_t)(r - n_rows) * ld_hidden;
        hs[r * rw_words + (k >> 5) * 33 + (k & 31)] = src[k];
    }
    constexpr int64_t kBB = WT == CBX_WTYPE_F16 ? 64 : (WT == CBX_WTYPE_Q4_0 ? 18 : 34);
    const int64_t wbytes = (int64_t)n_vocab * nball * kBB;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(W), (short)0, (int)wbytes, kBufWord3);
    __syncthreads();
    constexpr int kRowsPerPass = kGemvRowsPerWave * kGemvWaves;
    for (int vb = blockIdx.x * kRowsPerPass; vb < n_vocab; vb += gridDim.x * kRowsPerPass) {
        const int v = vb + wave * kGemvRowsPerWave + grp;
        const int vc = v < n_vocab ? v : n_vocab;  // past the table: zeros
        float acc[RMAX];
#pragma unroll
        for (int r = 0; r < RMAX; ++r) acc[r] = 0.0f;
        for (int b = s; b < nball; b += kGemvLanes) {
            float w[32];
            gemv_block<WT>(rw, vc, nball, b, w);
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
        }
        // the 16 lanes' sums: lane 15 of each 16-lane row ends with the total
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
            acc[r] = a;
        }
        if (s == kGemvLanes - 1 && v < n_vocab) {
            const float bv = bias ? bias[v] : 0.0f;
#pragma unroll
            for (int r = 0; r < RMAX; ++r) {
                if (r < R) {
                    float* o = r < n_rows ? out0 + (int64_t)r * ld_out
                                          : out1 + (int64_t)(r - n_rows) * ld_out;
                    o[v] = __fadd_rn(acc[r], bv);
                }
            }
        }
    }
}

template <int WT, int RMAX>
hipError_t launch_gemv(const void* W, const float* bias, const float* hidden0, const float* hidden1,
                       int64_t ld_hidden, float* out0, float* out1, int64_t ld_out, int32_t n_rows,
                       int32_t n_vocab, int32_t n_embd, hipStream_t stream) {
    const int R = hidden1 ? 2 * n_rows : n_rows;
    const size_t lds = (size_t)R * gemv_row_words(n_embd) * 4;
    constexpr int kRowsPerPass = kGemvRowsPerWave * kGemvWaves;
    const unsigned grid = (unsigned)((n_vocab + kRowsPerPass - 1) / kRowsPerPass);
    hipLaunchKernelGGL((head_gemv<WT, RMAX>), dim3(grid), dim3(64 * kGemvWaves), lds, stream, W,
                       bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows, n_vocab,
                       n_embd);
    return hipGetLastError();
}

template <int WT>
hipError_t launch_gemv_r(const void* W, const float* bias, const float* hidden0,
                         const float* hidden1, int64_t ld_hidden, float* out0, float* out1,
                         int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                         hipStream_t stream) {
    const int R = hidden1 ? 2 * n_rows : n_rows;
    if (R <= 2)
        return launch_gemv<WT, 2>(W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                                  n_vocab, n_embd, stream);
    if (R <= 4)
        return launch_gemv<WT, 4>(W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                                  n_vocab, n_embd, stream);
    if (R <= 8)
        return launch_gemv<WT, 8>(W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                                  n_vocab, n_embd, stream);
    return launch_gemv<WT, 16>(W, bias, hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows,
                               n_vocab, n_embd, stream);
}

}  // namespace

hipError_t launch_head(const void* W, int32_t wtype, const float* bias, const float* hidden0,
                       const float* hidden1, int64_t ld_hidden, float* out0, float* out1,
                       int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                       hipStream_t stream) {
    // fewer than 16 projected rows: the mat-vec (activations staged in LDS,
    // at most 64 KiB of them), else the 16-row matrix-core tiles
    const int R = hidden1 ? 2 * n_rows : n_rows;
    if (R < 16 && (size_t)R * gemv_row_words(n_embd) * 4 <= 65536) {
        switch (wtype) {
            case CBX_WTYPE_F16:
                return launch_gemv_r<CBX_WTYPE_F16>(W, bias, hidden0, hidden1, ld_hidden, out0,
                                                    out1, ld_out, n_rows, n_vocab, n_embd, stream);
            case CBX_WTYPE_Q4_0:
                return launch_gemv_r<CBX_WTYPE_Q4_0>(W, bias, hidden0, hidden1, ld_hidden, out0,
                                                     out1, ld_out, n_rows, n_vocab, n_embd, stream);
            case CBX_WTYPE_Q8_0:
                return launch_gemv_r<CBX_WTYPE_Q8_0>(W, bias, hidden0, hidden1, ld_hidden, out0,
                                                     out1, ld_out, n_rows, n_vocab, n_embd, stream);
            default:
                return hipErrorInvalidValue;
        }
    }
    const int n_tiles = ((n_rows + 15) / 16) * (hidden1 ? 2 : 1);
    const dim3 grid((unsigned)((n_vocab + 31) / 32), (unsigned)((n_tiles + NT - 1) / NT), 1u);
    switch (wtype) {
        case CBX_WTYPE_F16:
            hipLaunchKernelGGL(head_mfma<CBX_WTYPE_F16>, grid, dim3(64 * KS), 0, stream, W, bias,
                               hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows, n_vocab,
                               n_embd);
            break;
        case CBX_WTYPE_Q4_0:
            hipLaunchKernelGGL(head_mfma<CBX_WTYPE_Q4_0>, grid, dim3(64 * KS), 0, stream, W, bias,
                               hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows, n_vocab,
                               n_embd);
            break;
        case CBX_WTYPE_Q8_0:
            hipLaunchKernelGGL(head_mfma<CBX_WTYPE_Q8_0>, grid, dim3(64 * KS), 0, stream, W, bias,
                               hidden0, hidden1, ld_hidden, out0, out1, ld_out, n_rows, n_vocab,
                               n_embd);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace cbx
