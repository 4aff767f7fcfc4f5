// cbx_head.hip -- the T3 speech_head projection on the matrix cores:
// logits[r][v] = sum_k W[v][k] * h[r][k] + b[v]   (src/main.cpp:577; the weights
// and bias are chatterbox/speech_head(_bias), main.cpp:394-395), for F16, Q4_0
// and Q8_0 weights in ggml's layout (ne = [n_embd, n_vocab]: row v holds the
// n_embd weights of vocab id v; Q4_0 blocks are an fp16 scale d and 16 bytes
// of nibbles, element j < 16 in the low nibble of byte j and element j + 16
// in its high nibble, w = (q - 8) d; Q8_0 blocks are d and 32 int8, w = q d).
//
// One wavefront per workgroup computes a tile of 32 vocab ids x 16 rows with
// v_mfma_f32_16x16x4_f32 (two 16x16 accumulators).  Lane l feeds A[l%16][l/16]
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

__device__ __forceinline__ uint32_t ld_u16(const __amdgpu_buffer_rsrc_t& r, uint32_t off) {
    return (uint32_t)(uint16_t)__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, 0);
}

// The 8 weights k = 8g .. 8g + 7 of block kb of vocab row v.
template <int WT>
__device__ __forceinline__ void weights8(const __amdgpu_buffer_rsrc_t& rw, int v, int kb, int g,
                                         int n_embd, float* w) {
    if constexpr (WT == CBX_WTYPE_F16) {
        const uint32_t off = (uint32_t)(((int64_t)v * n_embd + kb * 32 + 8 * g) * 2);
        const uint32_t u0 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, off, 0, 0);
        const uint32_t u1 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, off + 4, 0, 0);
        const uint32_t u2 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, off + 8, 0, 0);
        const uint32_t u3 = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rw, off + 12, 0, 0);
        const uint32_t u[4] = {u0, u1, u2, u3};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[2 * i] = half_bits_to_float(u[i] & 0xffffu);
            w[2 * i + 1] = half_bits_to_float(u[i] >> 16);
        }
    } else {
        constexpr int BB = WT == CBX_WTYPE_Q4_0 ? 18 : 34;  // bytes per block
        const uint32_t blk = (uint32_t)(((int64_t)v * (n_embd / 32) + kb) * BB);
        const float d = half_bits_to_float(ld_u16(rw, blk));
        // Q4_0: bytes 8(g&1) .. +7 of the nibbles, low nibbles for g < 2;
        // Q8_0: int8 values 8g .. 8g + 7
        const uint32_t qoff = blk + 2 + (WT == CBX_WTYPE_Q4_0 ? 8 * (g & 1) : 8 * g);
        uint32_t p[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) p[i] = ld_u16(rw, qoff + 2 * i);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t byte = (p[i >> 1] >> (8 * (i & 1))) & 0xffu;
            if constexpr (WT == CBX_WTYPE_Q4_0) {
                const int q = (int)(g < 2 ? (byte & 0xfu) : (byte >> 4)) - 8;
                w[i] = __fmul_rn((float)q, d);
            } else {
                w[i] = __fmul_rn((float)(int8_t)byte, d);
            }
        }
    }
}

template <int WT>
__global__ __launch_bounds__(64) void head_mfma(const void* W, const float* bias,
                                                const float* hidden, int64_t ld_hidden,
                                                float* out, int64_t ld_out, int n_rows,
                                                int n_vocab, int n_embd) {
    const int lane = threadIdx.x;
    const int m = lane & 15, g = lane >> 4;
    const int v0 = blockIdx.x * 32, r0 = blockIdx.y * 16;
    constexpr int64_t kRowBytesNum = WT == CBX_WTYPE_F16 ? 64 : (WT == CBX_WTYPE_Q4_0 ? 18 : 34);
    const int64_t wbytes = (int64_t)n_vocab * (n_embd / 32) * kRowBytesNum;
    const __amdgpu_buffer_rsrc_t rw = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<void*>(W), (short)0, (int)wbytes, kBufWord3);
    const __amdgpu_buffer_rsrc_t rh = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(hidden), (short)0,
        (int)(((int64_t)(n_rows - 1) * ld_hidden + n_embd) * 4), kBufWord3);
    const int va = v0 + m, vb = v0 + 16 + m, rr = r0 + m;
    // rows past the table read zeros (byte offsets past the range)
    const int va_c = va < n_vocab ? va : n_vocab, vb_c = vb < n_vocab ? vb : n_vocab;
    const int64_t hrow = rr < n_rows ? (int64_t)rr * ld_hidden : ((int64_t)n_rows * ld_hidden + n_embd);
    f4 acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = acc0;
    const int nb = n_embd / 32;
#pragma unroll 1
    for (int kb = 0; kb < nb; ++kb) {
        float wa[8], wb[8], hv[8];
        weights8<WT>(rw, va_c, kb, g, n_embd, wa);
        weights8<WT>(rw, vb_c, kb, g, n_embd, wb);
        const uint32_t hoff = (uint32_t)((hrow + kb * 32 + 8 * g) * 4);
#pragma unroll
        for (int i = 0; i < 8; ++i)
            hv[i] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rh, hoff + 4 * i, 0, 0));
#pragma unroll
        for (int s = 0; s < 8; ++s) {
            acc0 = __builtin_amdgcn_mfma_f32_16x16x4f32(wa[s], hv[s], acc0, 0, 0, 0);
            acc1 = __builtin_amdgcn_mfma_f32_16x16x4f32(wb[s], hv[s], acc1, 0, 0, 0);
        }
    }
    if (rr >= n_rows) return;
    float* orow = out + (int64_t)rr * ld_out;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int v = v0 + 4 * g + i, v2 = v + 16;
        if (v < n_vocab) orow[v] = __fadd_rn(acc0[i], bias ? bias[v] : 0.0f);
        if (v2 < n_vocab) orow[v2] = __fadd_rn(acc1[i], bias ? bias[v2] : 0.0f);
    }
}

}  // namespace

hipError_t launch_head(const void* W, int32_t wtype, const float* bias, const float* hidden,
                       int64_t ld_hidden, float* out, int64_t ld_out, int32_t n_rows,
                       int32_t n_vocab, int32_t n_embd, hipStream_t stream) {
    const dim3 grid((unsigned)((n_vocab + 31) / 32), (unsigned)((n_rows + 15) / 16));
    switch (wtype) {
        case CBX_WTYPE_F16:
            hipLaunchKernelGGL(head_mfma<CBX_WTYPE_F16>, grid, dim3(64), 0, stream, W, bias, hidden,
                               ld_hidden, out, ld_out, n_rows, n_vocab, n_embd);
            break;
        case CBX_WTYPE_Q4_0:
            hipLaunchKernelGGL(head_mfma<CBX_WTYPE_Q4_0>, grid, dim3(64), 0, stream, W, bias, hidden,
                               ld_hidden, out, ld_out, n_rows, n_vocab, n_embd);
            break;
        case CBX_WTYPE_Q8_0:
            hipLaunchKernelGGL(head_mfma<CBX_WTYPE_Q8_0>, grid, dim3(64), 0, stream, W, bias, hidden,
                               ld_hidden, out, ld_out, n_rows, n_vocab, n_embd);
            break;
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace cbx
