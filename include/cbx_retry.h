/* cbx_retry.h -- the early-stop retry policy of the T3 segment loop, for a
 * batched engine that draws with Philox keys.
 *
 * The reference's CLI (src/chatterbox_cli.cpp:1597-1683) decodes each text
 * segment as follows: min_tokens = max(8, 5 * text tokens); an attempt that
 * ends on the stop token with fewer than min_tokens speech tokens (the stop
 * token popped) is retried, up to MAX_RETRIES = 3 times, each retry from the
 * segment's RNG snapshot advanced by 1009 * attempt draws
 * (rng.discard(1009 * attempt)); the first attempt that is not cut short
 * (ended by n_predict or the context, or long enough) is kept; when every
 * attempt is short, the longest is kept (the first of equal lengths).
 *
 * With CBX_DRAW_PHILOX a draw is keyed (seed, stream, step), so a retry
 * needs no snapshot: attempt a of stream s draws with the stream id
 * cbx_retry_stream_id(s, a), which is s itself for attempt 0 and lies in a
 * range no other (stream, attempt) pair uses for a > 0 (stream ids below
 * 2^56).  Through the C++ shim (cbx_sampler.hpp) the caller keeps its
 * std::mt19937 and the reference's discard(1009 * attempt) unchanged.
 * Host only; no HIP call. */
#ifndef CBX_RETRY_H
#define CBX_RETRY_H

#include <stdint.h>

#include "cbx_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

#define CBX_RETRY_MAX_RETRIES 3  /* chatterbox_cli.cpp:1615 */

typedef struct cbx_retry {
    int32_t min_tokens;   /* max(8, 5 * n_text_tokens)                               */
    int32_t max_retries;  /* CBX_RETRY_MAX_RETRIES                                   */
    int32_t attempt;      /* the attempt to run next (or the last one run, once done) */
    int32_t done;         /* 1 once an attempt is kept                                */
    int32_t best_attempt; /* longest attempt so far (-1 before the first)             */
    int32_t best_len;     /* its length in speech tokens, stop token popped           */
    int32_t kept_attempt; /* once done: the attempt whose tokens to keep              */
    int32_t kept_len;     /* once done: its length                                    */
} cbx_retry;

/* Start the policy for one segment of n_text_tokens (>= 0) text tokens. */
int cbx_retry_init(cbx_retry* r, int32_t n_text_tokens);

/* Philox stream id of attempt `attempt` (0 .. max_retries) of stream
 * `stream` (< 2^56): stream + attempt * 2^56.  UINT64_MAX for arguments out
 * of range. */
uint64_t cbx_retry_stream_id(uint64_t stream, int32_t attempt);

/* Record the attempt just run: n_tokens speech tokens after popping a final
 * stop token, and the reference's stopped_by_stop_token flag
 * (chatterbox_cli.cpp:1633-1638): nonzero only when the loop found the stop
 * token as the current token at the top of one of its n_predict iterations.
 * A stop token sampled by the last iteration is popped (:1647-1648) but the
 * flag stays 0, so such an attempt is kept however short it is; neither does
 * a loop that ends on a full context set it.  Returns 1 if another attempt
 * should run (r->attempt is then its number), 0 if r->done (r->kept_attempt /
 * kept_len say which tokens to keep), or a negative CBX_ERR_* for a call after
 * done or bad arguments. */
int cbx_retry_record(cbx_retry* r, int32_t n_tokens, int32_t stopped_by_stop_token);

/* The same record from what a decoder counts: n_sampled tokens drawn in the
 * attempt (the prompt's token and one per loop iteration run), the last of
 * them last_token, and the loop's bound n_predict (>= 0).  The loop checks
 * the token drawn before iteration i (i < n_predict) at that iteration's top,
 * so the attempt stopped on the stop token exactly when last_token ==
 * stop_token and n_sampled <= n_predict; n_tokens is n_sampled less the
 * popped stop token. */
int cbx_retry_record_tokens(cbx_retry* r, int32_t n_sampled, int32_t last_token,
                            int32_t stop_token, int32_t n_predict);

#ifdef __cplusplus
}
#endif

#endif /* CBX_RETRY_H */
