/*
 * cbx_t3.h -- the T3 transformer's decode step for many streams on one
 * MI355X: the producer of the rows the fused speech_head and the sampler
 * consume (include/cbx_sampler.h).
 *
 * The reference runs one stream: its step graph (src/main.cpp:617-633) embeds
 * the fed-back speech id and its position, runs the GPT-2 core
 * (build_transformer_core, main.cpp:469-575) over a KV cache of one
 * sequence (main.cpp:419-424) and projects ln_f's output through the
 * speech_head.  cbx_t3_step runs that step for n streams at once, each at its
 * own position with its own KV cache, and stops at ln_f's output: the rows
 * cbx_head_decode_step projects and samples.  With the decode state of
 * cbx_decode_step feeding its ids back (cbx_decode.next_token), a whole
 * batched decode loop stays on the device.
 *
 * Device pointers throughout; fp32 except the four matrices of every layer,
 * which take the speech_head's formats (CBX_WTYPE_F16 / Q4_0 / Q5_0 / Q8_0, rows of
 * n_in weights per output, ggml ne = [n_in, n_out]).
 */
#ifndef CBX_T3_H
#define CBX_T3_H

#include <stdint.h>

#include "cbx_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* One GPT-2 block's tensors (main.cpp:403-416: model/h<i>/...). */
typedef struct cbx_t3_layer {
    const float* ln_1_g;      /* [n_embd]                                        */
    const float* ln_1_b;
    const void*  attn_w;      /* c_attn: [3 n_embd] rows of n_embd (q | k | v)   */
    const float* attn_b;      /* [3 n_embd]                                      */
    const void*  attn_proj_w; /* c_proj: [n_embd] rows of n_embd                */
    const float* attn_proj_b;
    const float* ln_2_g;
    const float* ln_2_b;
    const void*  fc_w;        /* mlp c_fc: [4 n_embd] rows of n_embd             */
    const float* fc_b;
    const void*  fc_proj_w;   /* mlp c_proj: [n_embd] rows of 4 n_embd           */
    const float* fc_proj_b;
} cbx_t3_layer;

/* The model (main.cpp:348-424; hyperparameters main.cpp:356-367). */
typedef struct cbx_t3_model {
    int32_t n_layer;          /* 1 .. 256                                        */
    int32_t n_embd;           /* 64 * n_head, a multiple of 256, <= 4096         */
    int32_t n_head;           /* heads of 64 dimensions                          */
    int32_t n_pos;            /* rows of wpe (the model's n_ctx)                 */
    int32_t n_speech_vocab;   /* rows of speech_emb                              */
    int32_t wtype;            /* CBX_WTYPE_* of every layer's four matrices      */
    float   eps;              /* layer-norm epsilon                              */
    const float* wpe;         /* [n_pos][n_embd] position embeddings             */
    const float* speech_emb;  /* [n_speech_vocab][n_embd]                        */
    const cbx_t3_layer* layers; /* host array of n_layer                         */
    const float* ln_f_g;      /* [n_embd]                                        */
    const float* ln_f_b;
} cbx_t3_model;

/* KV caches of n streams, fp32, the reference's per-layer [HD, n_ctx, n_head]
 * order (main.cpp:480-488) with the stream outermost:
 * k[s][layer][head][pos][64], v the same. */
typedef struct cbx_t3_cache {
    float*  k;
    float*  v;
    int32_t n_ctx;            /* positions per stream, <= n_pos                  */
} cbx_t3_cache;

/* One decode step of n_rows streams.  Stream r's input is speech id
 * tokens[r] (or, with `inputs`, the row inputs[r][0, n_embd), already
 * embedded: a prompt's rows, fed one position per call) at position
 * positions[r]: its k and v are appended to the cache at that position, its
 * attention runs over positions [0, positions[r]], and ln_f's output goes to
 * hidden[r][0, n_embd); then positions[r] is incremented.  A stream is
 * skipped (nothing written to its cache, its hidden row zero, its position
 * unchanged) when state is given and state[r] != CBX_DECODE_RUNNING, when
 * its position is outside [0, cache.n_ctx) or its token outside
 * [0, n_speech_vocab).  Asynchronous on `stream`; the handle holds the
 * step's workspace (grown on demand: calls on one handle are ordered on one
 * stream).  Replaces eval_step (main.cpp:691-710) up to ln_f for every
 * stream at once. */
int cbx_t3_step(cbx_sampler* s, const cbx_t3_model* m, int32_t n_rows,
                const int32_t* tokens, const float* inputs, int32_t* positions,
                const int32_t* state, const cbx_t3_cache* cache, float* hidden,
                void* stream);

/* The prompt pass for many streams: n_rows rows, row r the speech id
 * tokens[r] (or the embedded row inputs[r][0, n_embd): the prompt's rows, as
 * the reference builds them from the speaker projection, the conditioning
 * and text embeddings and the start id, main.cpp:602-611) of the stream in
 * cache slot slots[r] at position positions[r].  Every row's k and v are
 * stored first, then each row attends over its stream's positions
 * [0, positions[r]], so the rows of one stream in one call see each other
 * as the reference's causal prompt graph does (main.cpp:490-497, :673-685);
 * a stream's positions must be distinct within a call, and those below a
 * row's position already in the cache or in the call.  ln_f's rows go to
 * hidden[r]; positions are only read.  Rows whose slot is outside
 * [0, n_slots), position outside [0, cache.n_ctx) or token outside
 * [0, n_speech_vocab) are skipped.  The cache holds n_slots streams.
 * Asynchronous on `stream`.  Replaces eval_prompt (main.cpp:643-689) up to
 * ln_f, for any number of streams at once. */
int cbx_t3_prefill(cbx_sampler* s, const cbx_t3_model* m, int32_t n_rows,
                   const int32_t* slots, int32_t n_slots, const int32_t* tokens,
                   const float* inputs, const int32_t* positions,
                   const cbx_t3_cache* cache, float* hidden, void* stream);

#ifdef __cplusplus
}
#endif
#endif
