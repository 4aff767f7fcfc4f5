/* cbx_gguf.h -- the speech_head, sampling metadata and T3 transformer of a
 * chatterbox T3 GGUF.
 *
 * The reference loads the T3 model with ggml's gguf reader
 * (src/main.cpp:356-399): the speech vocabulary size and the stop token from
 * the keys of src/chatterbox_t3_internal.h:33-40, and the tensors
 * chatterbox/speech_head (ggml ne = [n_embd, n_vocab], F16 by default,
 * Q4_0 / Q5_0 / Q8_0 when converted with --quant, scripts/convert-t3-turbo-to-gguf.py
 * :65-104, :160-163) and chatterbox/speech_head_bias (F32 [n_vocab]).  These
 * entry points read the same items from the file for cbx_head: the parse
 * runs on the host only; the load copies the tensor bytes to device buffers
 * the caller allocated.  The file layout is GGUF version 2 or 3 (ggml's
 * published format: little-endian header, typed key/value pairs, tensor
 * infos, tensor data aligned to general.alignment, default 32).
 *
 * Return codes as in cbx_sampler.h; cbx_last_error() gives the reason.
 * Every size and offset read from the file is checked against the file size
 * before use: a damaged or truncated file is CBX_ERR_INVALID, a head in a
 * format cbx_head does not take (e.g. Q4_1, K-quants) CBX_ERR_UNSUPPORTED. */
#ifndef CBX_GGUF_H
#define CBX_GGUF_H

#include <stdint.h>

#include "cbx_sampler.h"
#include "cbx_t3.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct cbx_head_file {
    int32_t  n_vocab;            /* speech_head ne[1] (rows, one per vocab id)      */
    int32_t  n_embd;             /* speech_head ne[0]; chatterbox.n_embd if present */
    int32_t  wtype;              /* CBX_WTYPE_F16 / _Q4_0 / _Q5_0 / _Q8_0           */
    int32_t  has_bias;           /* 1 if chatterbox/speech_head_bias is present     */
    int32_t  speech_vocab_size;  /* chatterbox.speech_vocab_size, -1 if absent      */
    int32_t  start_speech_token; /* chatterbox.start_speech_token, -1 if absent     */
    int32_t  stop_speech_token;  /* chatterbox.stop_speech_token, -1 if absent      */
    int32_t  gguf_version;       /* 2 or 3                                          */
    uint64_t weight_offset;      /* absolute byte offset of the weights in the file */
    uint64_t weight_bytes;       /* n_vocab rows in the wtype layout                */
    uint64_t bias_offset;        /* absolute byte offset of the bias (if present)   */
    uint64_t bias_bytes;         /* 4 * n_vocab, or 0                               */
} cbx_head_file;

/* Parse the header, key/value pairs and tensor infos of the GGUF at `path`
 * and fill *out.  Host only (no HIP call).  The head must be 2-D with
 * n_embd a multiple of 32 (32 .. 16384) and 1 <= n_vocab <= cbx_max_vocab();
 * a bias must be F32 [n_vocab]; a speech_vocab_size or stop token present in
 * the file must agree with the head (speech_vocab_size == n_vocab,
 * 0 <= stop_speech_token < n_vocab). */
int cbx_gguf_read_head(const char* path, cbx_head_file* out);

/* Copy the head's weight bytes (info->weight_bytes) to d_weights and, when
 * the file has a bias and d_bias is not NULL, the bias to d_bias (device
 * memory of the current HIP device, allocated by the caller).  `info` is
 * what cbx_gguf_read_head returned for the same file; the load checks the
 * file again against it.  Synchronous. */
int cbx_gguf_load_head(const char* path, const cbx_head_file* info, void* d_weights,
                       float* d_bias);

/* The T3 transformer of the same file, for cbx_t3_step: the keys
 * chatterbox.n_embd, n_head, n_layer, n_ctx and layer_norm_eps (required, as
 * the reference's loader requires them, main.cpp:356-367) and the tensors of
 * main.cpp:400-416 as the converter names them (scripts/convert-t3-turbo-to-
 * gguf.py:150-189): model/wpe (F32 [n_embd, n_ctx]), chatterbox/speech_emb
 * (F16 or F32 [n_embd, n_speech_vocab]), model/ln_f/{g,b} and per layer i
 * model/h<i>/ln_1/{g,b}, ln_2/{g,b}, attn/c_attn/{w,b}, attn/c_proj/{w,b},
 * mlp/c_fc/{w,b}, mlp/c_proj/{w,b}: the four matrices F16, Q4_0, Q5_0 or Q8_0 (one
 * type for all), the rest F32. */
typedef struct cbx_t3_file {
    int32_t  n_layer;
    int32_t  n_embd;
    int32_t  n_head;
    int32_t  n_pos;              /* model/wpe rows (chatterbox.n_ctx)               */
    int32_t  n_speech_vocab;     /* chatterbox/speech_emb rows                      */
    int32_t  wtype;              /* CBX_WTYPE_* of the layer matrices               */
    float    eps;                /* chatterbox.layer_norm_eps                       */
    int32_t  start_speech_token; /* -1 if absent                                    */
    int32_t  stop_speech_token;  /* -1 if absent                                    */
    int32_t  gguf_version;
    uint64_t device_bytes;       /* one device buffer of this size holds the model  */
} cbx_t3_file;

/* Parse the T3 tensors and keys of the GGUF at `path` (host only): their
 * names, types, shapes and data ranges are checked, and *out gets the model's
 * shape and the device bytes its tensors take (each at a 256-byte boundary,
 * speech_emb widened to F32). */
int cbx_gguf_read_t3(const char* path, cbx_t3_file* out);

/* Copy every T3 tensor of the file into d_buffer (info->device_bytes of
 * device memory of the current HIP device, allocated by the caller), fill
 * layers[0 .. n_layer) (host memory) with their device addresses and *model
 * with the rest (model->layers = layers), ready for cbx_t3_step.  `info` is
 * what cbx_gguf_read_t3 returned for the same file; the load checks the file
 * again against it.  Synchronous. */
int cbx_gguf_load_t3(const char* path, const cbx_t3_file* info, void* d_buffer,
                     cbx_t3_layer* layers, cbx_t3_model* model);

#ifdef __cplusplus
}
#endif

#endif /* CBX_GGUF_H */
