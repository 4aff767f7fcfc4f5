// cbx_split.h -- the matrix-core products' activation split, shared by its
// producers (head_split in cbx_head.hip, the T3 layer norm in cbx_t3.hip).
//
// Each block of 32 values of a row is scaled by 2^s (the block's largest
// magnitude to [2^14, 2^15)) and each value written as two fp16 parts,
// y = x 2^s = hi + lo + e with |e| <= 2^-23 |y| + 2^-25 (hi and lo rounded to
// nearest), next to 2^-s.  A scale per block (not per row) lets any producer
// that holds whole blocks of a row write its split itself (the attention's
// heads hold two blocks each, a product's 32-output tile one).
// Layout for padded row p = 16 T + m (row tile T): group j (values 8j ..
// 8j + 7) is lane 16 (j % 4) + m's operand of block j / 4, its hi parts in
// dwords ((T nball + j/4) 512 + 4 lane) .. + 3 and its lo parts 256 dwords on;
// the scales follow the parts from the next 256-byte boundary, block kb of
// row p at float (T nball + kb) 16 + m (the 16 rows of a tile's block
// together: the lanes holding rows 4g .. 4g + 3 of a product tile read
// theirs as one 16-byte load).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace cbx {

typedef uint32_t split_u4 __attribute__((ext_vector_type(4)));
typedef _Float16 split_h2 __attribute__((ext_vector_type(2)));

// 2^s and 2^-s for a row whose largest magnitude is mx: s = 14 - E for mx in
// [2^E, 2^(E+1)), clamped to [-126, 126] so both are normal floats (a finite
// row never meets the lower clamp, so no part overflows; the upper one binds
// only below 2^-112, where the split's error, 2^-25 scaled back by 2^-126, is
// below the smallest fp32 subnormal); s = 0 for a zero row.
__device__ __forceinline__ void split_scale(float mx, float& sc, float& inv) {
    const int E = (int)(__builtin_bit_cast(uint32_t, mx) >> 23) - 127;
    const int s = mx > 0.0f ? min(max(14 - E, -126), 126) : 0;
    sc = __builtin_bit_cast(float, (uint32_t)(127 + s) << 23);
    inv = __builtin_bit_cast(float, (uint32_t)(127 - s) << 23);
}

// Group j of row (T, m) from its 8 values x, scaled by sc, stored in place.
__device__ __forceinline__ void split_store(uint32_t* parts, int T, int m, int nball, int j,
                                            const float (&x)[8], float sc) {
    split_u4 hi, lo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float y0 = __fmul_rn(x[2 * i], sc), y1 = __fmul_rn(x[2 * i + 1], sc);
        const _Float16 h0 = (_Float16)y0, h1 = (_Float16)y1;
        const _Float16 l0 = (_Float16)__fsub_rn(y0, (float)h0);
        const _Float16 l1 = (_Float16)__fsub_rn(y1, (float)h1);
        hi[i] = __builtin_bit_cast(uint32_t, split_h2{h0, h1});
        lo[i] = __builtin_bit_cast(uint32_t, split_h2{l0, l1});
    }
    uint32_t* const o = parts + (int64_t)T * nball * 512 + 4 * m + (j >> 2) * 512 + 64 * (j & 3);
    *reinterpret_cast<split_u4*>(o) = hi;
    *reinterpret_cast<split_u4*>(o + 256) = lo;
}

// The T3 MLP's gelu, tanh form (Hendrycks and Gimpel; ggml_gelu's):
// 0.5 x (1 + tanh(sqrt(2/pi) x (1 + 0.044715 x^2))), each operation rounded.
__device__ __forceinline__ float t3_gelu_f(float x) {
    const float c = 0.7978845608028654f;  // sqrt(2 / pi)
    const float inner =
        __fmul_rn(__fmul_rn(c, x), __fadd_rn(1.0f, __fmul_rn(__fmul_rn(0.044715f, x), x)));
    return __fmul_rn(__fmul_rn(0.5f, x), __fadd_rn(1.0f, tanhf(inner)));
}

// A DPP lane exchange within each 16-lane row (ctrl a compile-time DPP code).
template <int CTRL>
__device__ __forceinline__ float dpp16(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                                  0xf, 0xf, false));
}

// Sum of v over each 16-lane row, the same in every lane of the row: the
// pairs of lanes 1 apart, then 2 (quad_perm), then the two quads of each 8
// (row_half_mirror: every lane of a quad already holds the quad's sum, so
// the mirror's partner adds what lane i ^ 4 would), then the two 8-lane
// halves (row_mirror): the operations of an xor butterfly over 1, 2, 4, 8,
// each add of a pair the same in either lane, without the LDS-routed
// permutes a general shuffle takes.
__device__ __forceinline__ float sum16_dpp(float v) {
    v = __fadd_rn(v, dpp16<0xB1>(v));   // quad_perm [1, 0, 3, 2]
    v = __fadd_rn(v, dpp16<0x4E>(v));   // quad_perm [2, 3, 0, 1]
    v = __fadd_rn(v, dpp16<0x141>(v));  // row_half_mirror
    return __fadd_rn(v, dpp16<0x140>(v));  // row_mirror
}

// Sum of one value per thread over a workgroup of 256 threads, the same
// value in every thread (the T3 layer norm's mean and variance, in the norm
// kernel and where a product stages the norm itself: both use this, so
// their results agree bit for bit).  Each wave: its 16-lane rows by
// sum16_dpp, then the rows' sums as (r0 + r1) + (r2 + r3); the waves' sums
// the same way through red.  red holds 8 floats and consecutive calls use its
// halves in turn (ph, starting at 0 in every thread): one barrier per call
// suffices, since a wave that writes a half again has passed the barrier of
// the call in between, which no wave reaches before it has read that half.
__device__ __forceinline__ float block_sum256(float v, float* red, int& ph) {
    v = sum16_dpp(v);
    auto lane_v = [&](int l) {
        return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
    };
    const float w = __fadd_rn(__fadd_rn(lane_v(0), lane_v(16)), __fadd_rn(lane_v(32), lane_v(48)));
    float* const h = red + 4 * ph;
    ph ^= 1;
    if ((threadIdx.x & 63) == 0) h[threadIdx.x >> 6] = w;
    __syncthreads();
    return __fadd_rn(__fadd_rn(h[0], h[1]), __fadd_rn(h[2], h[3]));
}

// Byte offset of the scales in a split buffer of R padded rows of n_embd.
__host__ __device__ inline size_t split_inv_offset(int R, int n_embd) {
    return ((size_t)R * n_embd * 4 + 255) / 256 * 256;
}

// Bytes of a split buffer of R padded rows (a multiple of 16) of n_embd.
__host__ __device__ inline size_t split_bytes(int R, int n_embd) {
    return split_inv_offset(R, n_embd) + (size_t)R * (n_embd / 32) * 4;
}

// Index of block kb's scale of row (T, m) among the scales.
__host__ __device__ inline int64_t split_inv_index(int T, int m, int nball, int kb) {
    return ((int64_t)T * nball + kb) * 16 + m;
}

// The largest magnitude over the 4 consecutive lanes (lane & ~3 .. + 3) that
// hold one block's 4 groups.
__device__ __forceinline__ float split_block_max4(float mx) {
    mx = fmaxf(mx, __shfl_xor(mx, 1));
    return fmaxf(mx, __shfl_xor(mx, 2));
}

}  // namespace cbx
