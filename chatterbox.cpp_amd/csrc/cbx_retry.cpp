// cbx_retry.cpp -- the T3 segment loop's early-stop retry policy
// (include/cbx_retry.h), following src/chatterbox_cli.cpp:1614-1672: the
// min_tokens floor (:1614), MAX_RETRIES (:1615), the per-attempt RNG offset
// (:1620-1621, here a Philox stream id per attempt), the stop flag of the
// decode loop (:1633-1638) and the pop of a final stop token (:1647-1648),
// the longest-attempt fallback (:1651) and the accept test (:1653-1654).
#include "../../include/cbx_retry.h"
#include "cbx_internal.h"

extern "C" int cbx_retry_init(cbx_retry* r, int32_t n_text_tokens) {
    if (!r || n_text_tokens < 0 || n_text_tokens > (1 << 28))
        return cbx::set_error(CBX_ERR_INVALID, "cbx_retry_init: NULL state or n_text_tokens %d",
                              n_text_tokens);
    const int32_t m = 5 * n_text_tokens;
    r->min_tokens = m > 8 ? m : 8;
    r->max_retries = CBX_RETRY_MAX_RETRIES;
    r->attempt = 0;
    r->done = 0;
    r->best_attempt = -1;
    r->best_len = 0;
    r->kept_attempt = -1;
    r->kept_len = 0;
    return CBX_OK;
}

extern "C" uint64_t cbx_retry_stream_id(uint64_t stream, int32_t attempt) {
    if (stream >> 56 || attempt < 0 || attempt > CBX_RETRY_MAX_RETRIES) return UINT64_MAX;
    return stream + ((uint64_t)attempt << 56);
}

extern "C" int cbx_retry_record(cbx_retry* r, int32_t n_tokens, int32_t stopped_by_stop_token) {
    if (!r || n_tokens < 0) return cbx::set_error(CBX_ERR_INVALID, "cbx_retry_record: bad arguments");
    if (r->done) return cbx::set_error(CBX_ERR_INVALID, "cbx_retry_record: the segment is done");
    // the longest attempt so far (strictly longer replaces: the first of equals stays)
    if (r->best_attempt < 0 || n_tokens > r->best_len) {
        r->best_attempt = r->attempt;
        r->best_len = n_tokens;
    }
    if (!stopped_by_stop_token || n_tokens >= r->min_tokens) {
        r->done = 1;
        r->kept_attempt = r->attempt;
        r->kept_len = n_tokens;
        return 0;
    }
    if (r->attempt < r->max_retries) {
        ++r->attempt;
        return 1;
    }
    r->done = 1;
    r->kept_attempt = r->best_attempt;
    r->kept_len = r->best_len;
    return 0;
}

extern "C" int cbx_retry_record_tokens(cbx_retry* r, int32_t n_sampled, int32_t last_token,
                                       int32_t stop_token, int32_t n_predict) {
    if (!r || n_sampled < 1 || n_predict < 0 || n_sampled > n_predict + 1)
        return cbx::set_error(CBX_ERR_INVALID,
                              "cbx_retry_record_tokens: %d tokens drawn with n_predict %d",
                              n_sampled, n_predict);
    const bool last_is_stop = last_token == stop_token;
    // iteration i (< n_predict) checks the (i+1)-th token drawn
    const int32_t stopped = last_is_stop && n_sampled <= n_predict ? 1 : 0;
    return cbx_retry_record(r, n_sampled - (last_is_stop ? 1 : 0), stopped);
}
