/*
 * cbx_oracle.h -- CPU oracle for the T3 logits->token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's CPU-baseline leg may load it.  The
 * product (libcbx_sampler.so) never links, loads or calls anything here.
 *
 * It restates tts_cpp::chatterbox::detail::sample_next_token_ex
 * (src/main.cpp:726-801 of chatterbox.cpp; params struct at
 * src/chatterbox_t3_internal.h:113-118) in fresh C++, keeping every
 * floating-point operation, its order and its precision, and inheriting the
 * last step from libstdc++ 11 (std::discrete_distribution, std::mt19937,
 * std::generate_canonical: /usr/include/c++/11/bits/random.tcc:81-89,
 * 2657-2712, 3348-3375).  The exponential is the host libm's expf, exactly as
 * the reference calls it through std::exp(float).
 *
 * Build-defined extensions (absent from the reference, defined here and
 * mirrored by the GPU path): CFG combine, allowed-token bitmask, forced stop,
 * min-p, Philox4x32-10 draws, Q4_0 / Q8_0 speech_head projection.
 */
#ifndef CBX_ORACLE_H
#define CBX_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same field order and meaning as cbx_params in include/cbx_sampler.h. */
typedef struct cbx_oracle_params {
    int32_t top_k;          /* main.cpp:740  active when 0 < top_k < n_vocab            */
    float   top_p;          /* main.cpp:750  active when top_p < 1                      */
    float   temp;           /* main.cpp:735  scale when temp > 0 && temp != 1; <=0 greedy */
    float   repeat_penalty; /* main.cpp:774  active when != 1 and history non-empty     */
    float   min_p;          /* extension: active when > 0                               */
    float   cfg_weight;     /* extension: used when uncond logits are given             */
} cbx_oracle_params;

/* info bits, identical to CBX_INFO_* in include/cbx_sampler.h */
#define CBX_ORACLE_INFO_DREW       0x01u /* a uniform was consumed by the draw          */
#define CBX_ORACLE_INFO_GREEDY     0x02u /* temp <= 0: argmax, no draw                   */
#define CBX_ORACLE_INFO_EMPTY      0x04u /* every score -inf: token 0 (main.cpp:792)     */
#define CBX_ORACLE_INFO_TOPP_TIE   0x08u /* a tie straddles the top-p cutoff             */
#define CBX_ORACLE_INFO_NONFINITE  0x10u /* NaN or +inf after the combine               */

/*
 * One row, uniform injected: exactly sample_next_token_ex with the draw's
 * generate_canonical value replaced by `u` (0 <= u < 1).
 *   logits_uncond / allowed may be NULL.  allowed: bit (i&31) of word i>>5.
 *   probs_out (may be NULL) receives the post-filter float probabilities
 *   (main.cpp:793) or zeros for an EMPTY row.
 *   kept_out (may be NULL) receives the number of non-zero probabilities.
 * Returns the token id.
 */
int32_t cbx_oracle_sample_row(const float* logits, const float* logits_uncond,
                              int32_t n_vocab, const int32_t* history,
                              int32_t n_history, const cbx_oracle_params* p,
                              const uint32_t* allowed, int32_t force_stop,
                              int32_t stop_token, double u, uint32_t* info,
                              float* probs_out, int32_t* kept_out);

/*
 * The reference exactly as the engine drives it (chatterbox_engine.cpp:326,
 * 338-353): one std::mt19937(seed), one call per step, history growing by each
 * sampled token when grow_history != 0 (otherwise the fixed history is used
 * for every step).  logits: [n_steps][n_vocab].  tokens_out: [n_steps].
 * If u_out is non-NULL it receives, per step, the generate_canonical value the
 * draw consumed (or -1.0 when no draw happened).
 */
void cbx_oracle_run_mt19937(const float* logits, int32_t n_steps, int32_t n_vocab,
                            const int32_t* history, int32_t n_history,
                            int32_t grow_history, const cbx_oracle_params* p,
                            uint32_t seed, int32_t* tokens_out, double* u_out);

/* The draw stage alone.  cbx_oracle_cdf_draw: the restated CDF build and
 * lower_bound at uniform u.  cbx_oracle_stdlib_draw: libstdc++'s own
 * std::discrete_distribution<int>(probs) driven by a 32-bit engine whose
 * next two outputs are x0 then x1 (so u = (x0 + x1*2^32) / 2^64 rounded),
 * which lets tests hit exact u values such as CDF boundaries. */
int32_t cbx_oracle_cdf_draw(const float* probs, int32_t n, double u);
int32_t cbx_oracle_stdlib_draw(const float* probs, int32_t n, uint32_t x0, uint32_t x1);

/* std::generate_canonical<double,53>(mt19937) values: the next n draws of a
 * generator seeded with `seed` after discarding `discard` 32-bit outputs. */
void cbx_oracle_mt_canonical(uint32_t seed, uint64_t discard, int32_t n, double* out);

/* The C++ standard's mt19937 check value: 10000th output of default seed. */
uint32_t cbx_oracle_mt_10000th(void);

/* Philox4x32-10 (Salmon et al., SC'11) of one counter block. */
void cbx_oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);

/* Uniform in [0,1) with 53 random bits keyed by (seed, stream, step):
 * counter {step lo, step hi, stream lo, stream hi}, key {seed lo, seed hi};
 * u = ((x0 >> 5) * 2^26 + (x1 >> 6)) * 2^-53. */
double cbx_oracle_philox_uniform(uint64_t seed, uint64_t stream, uint64_t step);

/* Batched rows (independent), for the CPU baseline and bulk parity.
 * logits [n_rows][ld], params [n_rows], history [n_rows][ld_hist] with
 * hist_len [n_rows], allowed [n_rows][ld_allowed] or NULL, force_stop
 * [n_rows] or NULL, u [n_rows].  n_threads <= 1 runs serially.
 * Returns elapsed wall seconds of the sampling loop only. */
double cbx_oracle_sample_batch(const float* logits, const float* logits_uncond,
                               int64_t ld, int32_t n_rows, int32_t n_vocab,
                               const int32_t* history, int64_t ld_hist,
                               const int32_t* hist_len,
                               const cbx_oracle_params* params,
                               const uint32_t* allowed, int64_t ld_allowed,
                               const uint8_t* force_stop, int32_t stop_token,
                               const double* u, int32_t n_threads,
                               int32_t* tokens_out, uint32_t* info_out);

/* Q4_0 / Q5_0 / Q8_0 blocks of 32 weights (ggml layout: fp16 scale d, then
 * 16 bytes of nibbles -- low nibbles hold elements 0..15, high nibbles
 * 16..31 --; Q5_0 puts a little-endian 32-bit word of fifth bits (bit j for
 * element j) between d and the nibbles; Q8_0 32 int8 values).  Dequantise
 * one row of n_embd weights to fp32: (q - 8) d, (q - 16) d, q d. */
void cbx_oracle_dequant_row(const uint8_t* blocks, int32_t wtype, int32_t n_embd, float* out);

/* Quantise fp32 rows to Q4_0 (wtype 2), Q5_0 (wtype 6) or Q8_0 (wtype 8)
 * with the reference converter's quantizer, gguf-py's (d = the signed value of
 * largest magnitude / -8 or / -16, q = trunc(x / d + 8.5 or 16.5) clipped;
 * Q8_0 d = amax / 127, q rounded half away from zero).  Output rows are
 * n_embd/32 blocks. */
void cbx_oracle_quantize(const float* w, int32_t n_rows, int32_t n_embd, int32_t wtype,
                         uint8_t* blocks_out);

/* fp64-accumulated head: logits[r][v] = sum_j deq(W[v][j]) * h[r][j] + b[v]. */
void cbx_oracle_head_f64(const uint8_t* W, int32_t wtype, const float* bias,
                         const float* hidden, int32_t n_rows, int32_t n_vocab,
                         int32_t n_embd, double* out);

/* Elementwise host libm expf (the function the reference's std::exp(float)
 * resolves to) -- used to check the GPU's restated exponential. */
void cbx_oracle_expf(const float* in, float* out, int64_t n);

/* Count positions where out[i] != expf(x_i) for the contiguous float bit
 * patterns x_i = first_bits + i (i < n), using n_threads threads. */
int64_t cbx_oracle_expf_mismatch(uint32_t first_bits, int64_t n, const float* out,
                                 int32_t n_threads);

#ifdef __cplusplus
}
#endif
#endif
