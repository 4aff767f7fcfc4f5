// cbx_internal.h -- shared between the C ABI layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/cbx_sampler.h"
#include "../../include/cbx_t3.h"

namespace cbx {

// Record the message cbx_last_error() returns on this thread; returns code.
int set_error(int code, const char* fmt, ...);

// Device-side view of one cbx_batch launch (all pointers device addresses).
struct KernelArgs {
    int32_t n_rows, n_vocab, n_steps, stop_token;
    const float* logits;
    int64_t ld_logits;
    const float* uncond;
    const cbx_params* params;
    const int32_t* history;
    const int32_t* history_len;
    int64_t ld_history;
    const uint32_t* allowed;
    int64_t ld_allowed;
    const uint8_t* force_stop;
    int32_t draw_mode;
    int32_t cap;  // survivor capacity of the on-chip lists (power of two)
    const double* uniforms;
    uint64_t seed;
    const uint64_t* stream_ids;
    uint64_t step0;
    int32_t* tokens;
    uint32_t* info;
    float* probs;
    int64_t ld_probs;
    // Rows left for the redo pass (more survivors than cap): int32 words
    // [0] count, [1] redo workgroups finished, [2 ..] row-step ids (the first
    // redo_max).  NULL when no redo pass follows the launch.
    int32_t* redo;
    int32_t redo_max;
    // A decode step's stream state (n_steps == 1, so a row-step is its row;
    // dec_state NULL for every other call; only the decode kernel reads
    // these): the writable history and length (the same memory as history
    // and history_len), the optional length limits and next-step input ids.
    int32_t* dec_state;
    int32_t* dec_history;
    int32_t* dec_len;
    const int32_t* dec_max;
    int32_t* dec_next;
};

// Rows one redo pass takes at most (one workgroup each).
constexpr int32_t kRedoMax = 4096;
// int32 words of a redo list.
constexpr int32_t kRedoWords = 2 + kRedoMax;

constexpr int32_t kMaxVocab = 32768;
// Survivors after top-k that the one-wave kernel holds; launches whose
// capacity is at most this (and V <= kWaveMaxVocab, or V <= kMaxVocab without
// CFG rows: the chunked form) use it.
constexpr int32_t kWaveCap = 1024;
// Launches of at most this many rows (two per CU) run the workgroup kernel at
// full survivor capacity: one row's latency, not throughput, sets their time.
constexpr int64_t kLatencyRows = 512;
constexpr int32_t kWaveMaxVocab = 256 * 33;

// Largest survivor capacity whose lists fit `lds_bytes` of LDS for n_vocab.
int32_t max_cap_for_lds(int32_t n_vocab, size_t lds_bytes);
// LDS bytes one workgroup needs for (cap, n_vocab).
size_t lds_bytes_for(int32_t cap, int32_t n_vocab);

// Launch the sampler over n_steps * n_rows rows.  Returns a hipError_t.
hipError_t launch_sample(const KernelArgs& a, hipStream_t stream);
// Whether launch_sample runs the one-wave kernel for these arguments.
bool uses_wave_kernel(const KernelArgs& a);
// One vocabulary class each (lanes x scores per lane), used by launch_sample.
// One-wave kernels, scores per lane 4*Q (V <= 256*Q); the *t forms serve
// V > 256*(Q-1), where only the last vector of each lane holds padding.
hipError_t launch_w16(const KernelArgs& a, hipStream_t stream);
hipError_t launch_w26(const KernelArgs& a, hipStream_t stream);
hipError_t launch_w33(const KernelArgs& a, hipStream_t stream);
hipError_t launch_w16t(const KernelArgs& a, hipStream_t stream);
hipError_t launch_w26t(const KernelArgs& a, hipStream_t stream);
hipError_t launch_w33t(const KernelArgs& a, hipStream_t stream);
// V <= 32768 without CFG rows: the one-wave kernel reading the row in chunks.
hipError_t launch_w128c(const KernelArgs& a, hipStream_t stream);
hipError_t launch_w128c2(const KernelArgs& a, hipStream_t stream);
// Launches of chunked rows (V > 8448) with at most this many row-steps split
// each row over two waves (two per SIMD at this size): a row's time is its
// wave's serial scan, halved; above it, one wave per row.
constexpr int64_t kChunkTwoWaveRows = 2048;
hipError_t launch_v512x8(const KernelArgs& a, hipStream_t stream);
hipError_t launch_v512x13(const KernelArgs& a, hipStream_t stream);
hipError_t launch_v512x16(const KernelArgs& a, hipStream_t stream);
hipError_t launch_v1024x16(const KernelArgs& a, hipStream_t stream);
hipError_t launch_v1024x32(const KernelArgs& a, hipStream_t stream);
// After a launch at capacity below the vocabulary's: sample again, at a.cap,
// the rows it put on its redo list, on the same stream (one workgroup per
// listed row; the last workgroup clears the list for the next launch).
hipError_t launch_redo(const KernelArgs& a, hipStream_t stream);
hipError_t launch_redo_v512x8(const KernelArgs& a, hipStream_t stream);
hipError_t launch_redo_v512x13(const KernelArgs& a, hipStream_t stream);
hipError_t launch_redo_v512x16(const KernelArgs& a, hipStream_t stream);
hipError_t launch_redo_v1024x16(const KernelArgs& a, hipStream_t stream);
hipError_t launch_redo_v1024x32(const KernelArgs& a, hipStream_t stream);
// A decode step (a.dec_state set, one step, a.cap the full capacity): one
// workgroup per stream of the vocabulary class's workgroup kernel.
hipError_t launch_decode(const KernelArgs& a, hipStream_t stream);
hipError_t launch_decode_v512x8(const KernelArgs& a, hipStream_t stream);
hipError_t launch_decode_v512x13(const KernelArgs& a, hipStream_t stream);
hipError_t launch_decode_v512x16(const KernelArgs& a, hipStream_t stream);
hipError_t launch_decode_v1024x16(const KernelArgs& a, hipStream_t stream);
hipError_t launch_decode_v1024x32(const KernelArgs& a, hipStream_t stream);

// The speech_head projection (cbx_head.hip): out0[r][v] = W[v] . hidden0[r] + bias[v]
// for r < n_rows, v < n_vocab, and the same from hidden1 into out1 in the same
// launches when hidden1 is given.  `scratch` is device memory of at least
// head_scratch_bytes(n_rows, hidden1 != NULL, n_embd) bytes (the activations
// split for the matrix cores; 0 bytes, and NULL allowed, below 16 rows).
size_t head_scratch_bytes(int32_t n_rows, bool cfg, int32_t n_embd);
// Bytes per block of 32 weights of a CBX_WTYPE_* (0 for an unknown type).
inline int64_t wtype_block_bytes(int32_t wtype) {
    switch (wtype) {
        case CBX_WTYPE_F16: return 64;
        case CBX_WTYPE_Q4_0: return 18;
        case CBX_WTYPE_Q5_0: return 22;
        case CBX_WTYPE_Q8_0: return 34;
        default: return 0;
    }
}
// Whether launch_head takes the mat-vec (fewer than 16 projected rows whose
// activations fit its LDS) rather than the split and the matrix cores.
bool head_uses_gemv(int32_t n_rows, bool cfg, int32_t n_embd);
// launch_head with the products' K split over kz workgroups (one row set, the
// matrix-core path): slab z of out0 (out0 + z * n_rows * ld_out) holds the
// partial products of the z-th run of blocks, the bias in slab 0 only; the
// caller adds the kz slabs.  head_k_split: the kz that launch would use
// (1 for the mat-vec, else doubled up to 8 while the grid holds fewer than
// 512 workgroups and each wave keeps 4 blocks).
// gelu_out: the T3 MLP's gelu (t3_gelu_f) applied to every output as it is
// stored (no K split then).
int head_k_split(int32_t n_rows, int32_t n_vocab, int32_t n_embd);
hipError_t launch_head_k(const void* W, int32_t wtype, const float* bias, const float* hidden0,
                         const float* hidden1, int64_t ld_hidden, float* out0, float* out1,
                         int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                         void* scratch, hipStream_t stream, int kz, bool gelu_out);
// The matrix-core products of n_rows rows already split into `scratch` by
// their producer (cbx_split.h's layout, n_rows padded to whole 16-row tiles):
// launch_head_k without its split launch (one row set; 16 rows and more).
// out_split set (no K split, n_vocab a multiple of 32): the outputs go there
// split for the next product (rows of n_vocab) instead of to out0.
hipError_t launch_head_presplit(const void* W, int32_t wtype, const float* bias, float* out0,
                                int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                                const void* scratch, hipStream_t stream, int kz,
                                bool gelu_out, void* out_split = nullptr);

// The T3 layer's residual add and layer norm folded into the mat-vec product
// that consumes them (1 or 2 rows of n_embd, a multiple of 256, at most
// 4096): per row r, x_out[r] = x_in[r] + y[r], and the product's input row is
// LN(x_out[r]) * g + b, with the same operations in the same order as the
// separate norm kernel; a row with act[r] == 0 gets a zero input and
// x_out[r] = x_in[r].  Workgroup 0 stores x_out (x_in is only read, so the
// two must differ).
struct GemvNorm {
    const float* x_in;
    float* x_out;
    const float* y;
    const float* g;
    const float* b;
    const int32_t* act;
    float eps;
};
hipError_t launch_head_gemv_norm(const void* W, int32_t wtype, const float* bias,
                                 const GemvNorm& nm, float* out, int64_t ld_out, int32_t n_rows,
                                 int32_t n_vocab, int32_t n_embd, hipStream_t stream, bool gelu);
hipError_t launch_head(const void* W, int32_t wtype, const float* bias, const float* hidden0,
                       const float* hidden1, int64_t ld_hidden, float* out0, float* out1,
                       int64_t ld_out, int32_t n_rows, int32_t n_vocab, int32_t n_embd,
                       void* scratch, hipStream_t stream);

// The T3 decode step (cbx_t3.hip).  t3_shape_ok: the widths the kernels take
// (heads of 64, n_embd a supported multiple of 256); t3_attn_lds: the
// attention kernel's LDS for a cache of n_ctx positions; t3_workspace_bytes:
// the step's device workspace for n_rows streams.
bool t3_shape_ok(int32_t n_embd, int32_t n_head);
size_t t3_attn_lds(int32_t n_ctx);
size_t t3_workspace_bytes(int32_t n_rows, int32_t n_embd);
// slots set: the prefill form (cbx_t3_prefill); positions are not advanced.
hipError_t launch_t3_step(const cbx_t3_model& m, int32_t n_rows, const int32_t* tokens,
                          const float* inputs, int32_t* positions, const int32_t* state,
                          const int32_t* slots, int32_t n_slots, const cbx_t3_cache& c,
                          float* hidden, void* ws, hipStream_t st);

}  // namespace cbx
