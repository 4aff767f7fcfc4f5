/*
 * cbx_sampler.h -- C ABI of the MI355X (gfx950) T3 logits->token sampler.
 *
 * Drop-in for the per-step sampler of chatterbox.cpp,
 *   int32_t tts_cpp::chatterbox::detail::sample_next_token_ex(
 *       const std::vector<float>& logits, const std::vector<int32_t>& generated,
 *       const chatterbox_sampling_params& params, std::mt19937& rng)
 * (src/main.cpp:726-801, declared at src/chatterbox_t3_internal.h:144-148),
 * called from src/chatterbox_engine.cpp:338,351 and, through the wrapper at
 * src/chatterbox_cli.cpp:394-405, from chatterbox_cli.cpp:1270,1283,1633,1643.
 *
 * Semantics are the reference's, bit for bit: given the same logits, history,
 * parameters and the same uniform u in [0,1) for the draw, the token id is the
 * one the reference returns.  The draw's uniform is supplied by the caller
 * (CBX_DRAW_UNIFORM; include/cbx_sampler.hpp derives it from the caller's
 * std::mt19937 exactly as std::discrete_distribution does) or generated on the
 * device by Philox4x32-10 keyed (seed, stream, step) (CBX_DRAW_PHILOX).
 *
 * Plain C: every pointer is a plain address, every size an integer; device
 * pointers are HIP device addresses, `stream` is a hipStream_t (NULL = the
 * null stream).  No C++ exception crosses this boundary.
 *
 * Return codes: CBX_OK (0) or a negative CBX_ERR_*; cbx_last_error() gives a
 * thread-local message for the last failing call on the calling thread.
 */
#ifndef CBX_SAMPLER_H
#define CBX_SAMPLER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define CBX_OK               0
#define CBX_ERR_INVALID     (-1)  /* bad argument (null pointer, size out of range) */
#define CBX_ERR_HIP         (-2)  /* a HIP runtime call failed                      */
#define CBX_ERR_UNSUPPORTED (-3)  /* valid request this build does not implement    */
#define CBX_ERR_NOMEM       (-4)  /* device or host allocation failed               */

/* Per-row sampling knobs.  The first four are chatterbox_sampling_params
 * (src/chatterbox_t3_internal.h:113-118; defaults 1000, 0.95, 0.8, 1.2) and
 * keep the reference's activation rules (main.cpp:735, 740, 750, 774). */
typedef struct cbx_params {
    int32_t top_k;          /* active when 0 < top_k < n_vocab                      */
    float   top_p;          /* active when top_p < 1                                */
    float   temp;           /* scale by 1/temp when temp > 0 && temp != 1;
                               temp <= 0 selects the first argmax (no draw)        */
    float   repeat_penalty; /* active when != 1 and the history is non-empty      */
    float   min_p;          /* extension, active when > 0: after top-p, drop ids
                               with expf(s - s_max) < min_p                         */
    float   cfg_weight;     /* extension, used when uncond logits are given:
                               l = c + w * (c - u), each operation rounded once     */
} cbx_params;

/* Per-row result flags. */
#define CBX_INFO_DREW      0x01u /* the uniform was consumed (reference drew from rng) */
#define CBX_INFO_GREEDY    0x02u /* temp <= 0: first argmax of the probabilities       */
#define CBX_INFO_EMPTY     0x04u /* every score was -inf: token 0 (main.cpp:792)       */
#define CBX_INFO_TOPP_TIE  0x08u /* equal scores straddle the top-p cutoff; the kept
                                    ones are those the reference's std::sort puts
                                    first (its order is replayed)                  */
#define CBX_INFO_NONFINITE 0x10u /* NaN or +inf scores: outside the contract           */
#define CBX_INFO_OVERFLOW  0x20u /* more survivors than the launch's capacity:
                                    token -1.  Only past the 4096 row-steps of a
                                    call's redo list (max_survivors set too low);
                                    at full capacity never on gfx950, whose LDS
                                    holds every id of a 32768 vocabulary           */
#define CBX_INFO_TOPP_SORTED 0x80u /* diagnostic, one-wave kernel only: the top-p
                                    cutoff was taken on the sorted survivor list
                                    with exact float running sums, because value
                                    bins could not certify it (the same token
                                    either way; other kernels always sort and do
                                    not set this bit)                              */

#define CBX_DRAW_UNIFORM 0 /* uniforms[step][row] supplied by the caller            */
#define CBX_DRAW_PHILOX  1 /* Philox4x32-10: counter {step lo, step hi, stream lo,
                              stream hi}, key {seed lo, seed hi}; u = ((x0>>5)*2^26 +
                              (x1>>6)) * 2^-53                                        */

typedef struct cbx_sampler cbx_sampler; /* opaque; one per decode thread */

/* Batched request: n_steps independent batches of n_rows streams, step-major.
 * All pointers are device pointers.  Optional ones may be NULL. */
typedef struct cbx_batch {
    int32_t n_rows;             /* streams per step (>= 1)                          */
    int32_t n_vocab;            /* 2 .. cbx_max_vocab()                             */
    int32_t n_steps;            /* >= 1                                             */
    int32_t stop_token;         /* id kept by force_stop rows                       */
    const float*    logits;     /* [n_steps][n_rows][ld_logits]                     */
    int64_t         ld_logits;  /* >= n_vocab                                       */
    const float*    logits_uncond; /* optional CFG uncond rows, same layout         */
    const cbx_params* params;   /* [n_rows]                                         */
    const int32_t*  history;    /* optional [n_rows][ld_history] generated ids      */
    const int32_t*  history_len;/* [n_rows], required with history                  */
    int64_t         ld_history;
    const uint32_t* allowed;    /* optional [n_rows][ld_allowed] bitmask, bit (i&31)
                                   of word i>>5 set = id i allowed                  */
    int64_t         ld_allowed; /* >= ceil(n_vocab/32)                              */
    const uint8_t*  force_stop; /* optional [n_steps][n_rows]: nonzero = every id
                                   but stop_token is masked                        */
    int32_t         draw_mode;  /* CBX_DRAW_UNIFORM or CBX_DRAW_PHILOX              */
    int32_t         max_survivors; /* host hint: bound on ids left by top-k (e.g. the
                                   largest active top_k); 0 = n_vocab.  At most
                                   1024 with n_vocab <= 8448 runs one wavefront
                                   per row (the fastest form for large calls;
                                   small calls: cbx_sampler_set_latency_rows).
                                   Rows with more
                                   survivors (ties at a tiny top-k threshold, top-k
                                   off) are sampled again on the same stream by a
                                   second pass at the capacity of the whole
                                   vocabulary: up to 4096 such row-steps per call;
                                   any beyond keep token -1 and CBX_INFO_OVERFLOW
                                   (a call whose rows may all exceed the bound,
                                   e.g. top-k off, passes 0)                    */
    const double*   uniforms;   /* CBX_DRAW_UNIFORM: [n_steps][n_rows] in [0,1)      */
    uint64_t        seed;       /* CBX_DRAW_PHILOX key                              */
    const uint64_t* stream_ids; /* CBX_DRAW_PHILOX: [n_rows]; NULL = row index      */
    uint64_t        step0;      /* CBX_DRAW_PHILOX: counter of step 0               */
    int32_t*        tokens;     /* out [n_steps][n_rows]                            */
    uint32_t*       info;       /* optional out [n_steps][n_rows] CBX_INFO_* bits   */
    float*          probs;      /* optional out [n_steps][n_rows][ld_probs]:
                                   post-filter probabilities (main.cpp:793)        */
    int64_t         ld_probs;
} cbx_batch;

/* Largest n_vocab this build accepts. */
int32_t cbx_max_vocab(void);

/* Create a handle on HIP device `device` sized for single-row calls of up to
 * max_vocab logits and max_history history ids (its pinned staging and device
 * buffers).  Batched calls use caller memory and need no sizing. */
int cbx_sampler_create(cbx_sampler** out, int32_t device, int32_t max_vocab,
                       int32_t max_history);
int cbx_sampler_destroy(cbx_sampler* s);

/* Launch policy (no counterpart in the reference, which samples one row on
 * the CPU): a call of at most `rows` row-steps (n_rows * n_steps; default
 * 512, two per CU on MI355X) is bound by one row's latency and runs at full
 * survivor capacity, ignoring max_survivors -- a row spread over the waves of
 * a workgroup, and no redo pass.  Larger calls keep max_survivors (one wave
 * per row while the survivors fit).  0 turns the rule off.  Results are the
 * same either way. */
int cbx_sampler_set_latency_rows(cbx_sampler* s, int64_t rows);

/* Single row, host memory in and out, synchronous: the reference call shape
 * (logits, history, params in; token out).  Replaces the body of
 * sample_next_token_ex (main.cpp:726-801); `u` is the draw's uniform. */
int cbx_sample_row(cbx_sampler* s, const float* logits, int32_t n_vocab,
                   const int32_t* history, int32_t n_history,
                   const cbx_params* params, double u,
                   int32_t* token_out, uint32_t* info_out);

/* Single row with the extensions: optional CFG uncond logits, allowed bitmask
 * (ceil(n_vocab/32) words), forced stop, and the post-filter probabilities
 * (n_vocab floats) out.  Host memory, synchronous. */
int cbx_sample_row_ex(cbx_sampler* s, const float* logits, const float* logits_uncond,
                      int32_t n_vocab, const int32_t* history, int32_t n_history,
                      const cbx_params* params, const uint32_t* allowed,
                      int32_t force_stop, int32_t stop_token, double u,
                      int32_t* token_out, uint32_t* info_out, float* probs_out);

/* Batched, device memory, asynchronous on `stream`.  The handle supplies the
 * device and the redo list of a launch with max_survivors set (the rows it
 * samples again): calls on one handle that overlap in time on several
 * streams race on that list, so each stream takes its own handle.
 * Replaces n_steps x n_rows calls of sample_next_token_ex. */
int cbx_sample_batch(cbx_sampler* s, const cbx_batch* b, void* stream);

/* cbx_sample_batch without any device memory of the handle: the rows to
 * sample again (more survivors than max_survivors allows) go on a redo list
 * in a file-scope device array of the library, one per GPU, whose address
 * cbx_sampler_create resolves.  No counterpart in the reference: for callers
 * that cannot allocate or use allocated scratch per call (code under HIP
 * graph capture, tight serving loops).  Allocates nothing and calls no
 * memset.  Limit: with max_survivors below the vocabulary's capacity at most
 * 4096 row-steps (n_rows * n_steps) per call (CBX_ERR_INVALID beyond).  Every
 * call on one GPU shares the array: calls that overlap in time on one GPU
 * (several streams, several handles) race and must not be issued. */
int cbx_sample_batch_static(cbx_sampler* s, const cbx_batch* b, void* stream);

/* Weight formats of the speech_head projection (ggml type ids; rows of n_embd
 * weights, one per vocab id, ggml ne = [n_embd, n_vocab]). */
#define CBX_WTYPE_F16  1 /* 2 bytes per weight                                    */
#define CBX_WTYPE_Q4_0 2 /* 18-byte blocks of 32: fp16 d, 16 bytes of nibbles
                            (element j < 16 low nibble of byte j, j + 16 high);
                            w = (q - 8) * d                                       */
#define CBX_WTYPE_Q5_0 6 /* 22-byte blocks of 32: fp16 d, 32-bit little-endian qh
                            (bit j: fifth bit of element j), 16 bytes of nibbles
                            as Q4_0; w = (q - 16) * d                             */
#define CBX_WTYPE_Q8_0 8 /* 34-byte blocks of 32: fp16 d, 32 int8; w = q * d     */

/* The T3 speech_head projection, logits = W h + b (src/main.cpp:577; weights
 * chatterbox/speech_head and chatterbox/speech_head_bias, main.cpp:394-395,
 * written by scripts/convert-t3-turbo-to-gguf.py:65-104).  Device pointers. */
typedef struct cbx_head {
    const void*  weights;       /* [n_vocab] rows in the wtype layout             */
    int32_t      wtype;         /* CBX_WTYPE_*                                    */
    int32_t      n_embd;        /* 32 .. 16384, a multiple of 32                  */
    const float* bias;          /* optional [n_vocab]                             */
    const float* hidden;        /* [rows][ld_hidden] fp32 (the ln_f output)       */
    const float* hidden_uncond; /* optional CFG uncond rows, same layout          */
    int64_t      ld_hidden;     /* >= n_embd                                      */
    float*       logits;        /* out [rows][ld_logits]                          */
    float*       logits_uncond; /* out, required with hidden_uncond               */
} cbx_head;

/* The projection alone for n_rows rows of hidden (and hidden_uncond) into
 * logits (and logits_uncond), row stride ld_logits >= n_vocab; weights as
 * the format defines them, exact products, fp32 sums.  From 16 projected rows
 * on, the fp16 matrix cores take each activation row scaled by a power of
 * two as two fp16 parts (each activation to 2^-23 relative plus 2^-39 of
 * its row's largest magnitude), held in a device buffer of the
 * handle that a call larger than any before it replaces (waiting for the
 * device): head calls on one handle are ordered on one stream.
 * Replaces the speech_head mul_mat of the T3 step (main.cpp:577).  Async. */
int cbx_head_logits(cbx_sampler* s, const cbx_head* h, int32_t n_rows, int32_t n_vocab,
                    int64_t ld_logits, void* stream);

/* Fused variant of cbx_sample_batch: the projection of the batch's
 * n_steps * n_rows hidden rows into h->logits (row stride b->ld_logits; with
 * hidden_uncond also h->logits_uncond), then the sampler over them, both on
 * `stream`.  b->logits is ignored; b->logits_uncond is used only when
 * h->hidden_uncond is NULL.  Replaces the speech_head mul_mat, the logits
 * hand-off (main.cpp:706-708) and sample_next_token_ex of one T3 step. */
int cbx_head_sample_batch(cbx_sampler* s, const cbx_head* h, const cbx_batch* b, void* stream);

/* Decode state of n_rows streams, kept on the device.  The engine's T3 loop
 * (src/chatterbox_engine.cpp:337-356) pushes each sampled id onto
 * `generated` (the penalty history of the next call), feeds it to the next
 * step graph as its "speech_token" input (main.cpp:697), ends a stream at
 * its stop token (dropped from the result) or after n_predict + 1 ids (or
 * n_ctx), and copies the logits to the host and waits for them every token
 * (main.cpp:706-708).  A decode step updates this state on the device
 * instead, so a loop of steps copies nothing to the host until the caller
 * reads `state`; `history[r][0, history_len[r])` is then stream r's result. */
#define CBX_DECODE_RUNNING 0 /* sampled next step                                  */
#define CBX_DECODE_STOP    1 /* sampled stop_token (not appended): ended           */
#define CBX_DECODE_LIMIT   2 /* history holds max_len ids: ended                   */

#define CBX_INFO_ENDED 0x40u /* decode step: the stream had ended; not sampled, its
                                token is stop_token                                */

typedef struct cbx_decode {
    int32_t*       state;       /* [n_rows] CBX_DECODE_*; streams start RUNNING    */
    int32_t*       history;     /* [n_rows][ld_history] ids sampled so far        */
    int32_t*       history_len; /* [n_rows]                                       */
    int64_t        ld_history;  /* >= 1                                           */
    const int32_t* max_len;     /* optional [n_rows] id limit per stream
                                   (min(n_predict, n_ctx - prompt_len) + 1 for
                                   the engine loop); NULL or above ld_history:
                                   ld_history                                     */
    int32_t*       next_token;  /* optional [n_rows] out: each id appended, for the
                                   next step's input                              */
} cbx_decode;

/* One decode step of b->n_rows streams (b->n_steps must be 1; b's history,
 * history_len and ld_history are ignored: d's are used): each running stream
 * is sampled as cbx_sample_batch does, with b->stop_token as its stop id, at
 * the capacity of the whole vocabulary (max_survivors is ignored: no row
 * overflows); then the stop token ends it (CBX_DECODE_STOP), any other id is
 * appended to its history and written to next_token, and a history of
 * max_len ids ends it (CBX_DECODE_LIMIT).  Streams already ended are not
 * sampled: their token is stop_token, info CBX_INFO_ENDED, their probs row is
 * not written.  One launch, asynchronous on `stream`, on the device alone.
 * Replaces one iteration of the engine's decode loop after its step graph
 * (chatterbox_engine.cpp:345-353) with the logits left on the device. */
int cbx_decode_step(cbx_sampler* s, const cbx_batch* b, const cbx_decode* d, void* stream);

/* cbx_decode_step on logits projected by the speech_head first, as in
 * cbx_head_sample_batch: the step graph's ln_f rows in, the next step's input
 * ids out. */
int cbx_head_decode_step(cbx_sampler* s, const cbx_head* h, const cbx_batch* b,
                         const cbx_decode* d, void* stream);

/* Thread-local description of the last error on this thread ("" if none). */
const char* cbx_last_error(void);

#ifdef __cplusplus
}
#endif
#endif
