// cbx_capi.cpp -- the extern "C" boundary of libcbx_sampler.so.
//
// Validates arguments, owns the per-handle stream and staging buffers for the
// single-row calls, and forwards to the kernels.  No exception crosses the
// boundary: every entry point returns CBX_OK or a negative CBX_ERR_* and
// leaves a message for cbx_last_error() on the calling thread.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <new>

#include "cbx_internal.h"

struct cbx_sampler {
    int32_t device = 0;
    int32_t max_vocab = 0;
    int32_t max_history = 0;
    size_t lds_limit = 0;
    hipStream_t stream = nullptr;
    // device buffers for single-row calls
    float* d_logits = nullptr;
    float* d_uncond = nullptr;
    int32_t* d_hist = nullptr;
    int32_t* d_hist_len = nullptr;
    cbx_params* d_params = nullptr;
    uint32_t* d_allowed = nullptr;
    uint8_t* d_force = nullptr;
    double* d_u = nullptr;
    int32_t* d_token = nullptr;
    uint32_t* d_info = nullptr;
    float* d_probs = nullptr;
    // redo lists (rows over a launch's survivor capacity): batched calls, and
    // the single-row calls on the handle's own stream
    int32_t* d_redo = nullptr;
    int32_t* d_redo_row = nullptr;
    // the device's address of the file-scope redo list of
    // cbx_sample_batch_static (shared by every handle on the device)
    int32_t* static_redo = nullptr;
    // launches of at most this many row-steps run at full capacity
    int64_t latency_rows = cbx::kLatencyRows;
    // the head's activation split (matrix-core projections), grown on demand
    void* d_head = nullptr;
    size_t head_bytes = 0;
    // the T3 decode step's workspace, grown on demand
    void* d_t3 = nullptr;
    size_t t3_bytes = 0;
    // pinned host staging for the small per-call inputs/outputs
    struct Small {
        cbx_params params;
        double u;
        int32_t hist_len;
        int32_t token;
        uint32_t info;
        uint8_t force;
    }* h_small = nullptr;
};

namespace {

thread_local char g_err[512] = "";

// The redo list of cbx_sample_batch_static: device memory the library never
// allocates, one copy per GPU (a file-scope device array, zero when the
// library is loaded; every redo pass leaves it empty again).  Host code uses
// each device's address of it, from hipGetSymbolAddress with that device
// current, never the array's name.
constexpr int kMaxDevices = 64;
static __device__ __align__(256) int32_t scratch[cbx::kRedoWords];
std::mutex g_scratch_mu;
int32_t* g_scratch_ptr[kMaxDevices] = {};

// The address of `scratch` on `device`, which must be current; resolved once
// per device.
hipError_t static_scratch(int device, int32_t** out) {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        g_scratch_ptr[device] = static_cast<int32_t*>(p);
    }
    *out = g_scratch_ptr[device];
    return hipSuccess;
}

int fail(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}

#define CBX_HIP(call)                                                                     \
    do {                                                                                  \
        hipError_t e_ = (call);                                                           \
        if (e_ != hipSuccess)                                                             \
            return fail(CBX_ERR_HIP, "%s failed: %s", #call, hipGetErrorString(e_));       \
    } while (0)

struct DeviceGuard {
    int prev = -1;
    explicit DeviceGuard(int dev) {
        if (hipGetDevice(&prev) != hipSuccess) prev = -1;
        if (prev != dev) (void)hipSetDevice(dev);
    }
    ~DeviceGuard() {
        int cur = -1;
        if (prev >= 0 && hipGetDevice(&cur) == hipSuccess && cur != prev) (void)hipSetDevice(prev);
    }
};

void release(cbx_sampler* s) {
    DeviceGuard g(s->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    (void)hipFree(s->d_logits);
    (void)hipFree(s->d_uncond);
    (void)hipFree(s->d_hist);
    (void)hipFree(s->d_hist_len);
    (void)hipFree(s->d_params);
    (void)hipFree(s->d_allowed);
    (void)hipFree(s->d_force);
    (void)hipFree(s->d_u);
    (void)hipFree(s->d_token);
    (void)hipFree(s->d_info);
    (void)hipFree(s->d_probs);
    (void)hipFree(s->d_redo);
    (void)hipFree(s->d_redo_row);
    (void)hipFree(s->d_head);
    (void)hipFree(s->d_t3);
    if (s->h_small) (void)hipHostFree(s->h_small);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    delete s;
}

// Survivor capacity for a launch: the smaller of n_vocab and the caller's
// hint, rounded up to a power of two, limited by the device's LDS.
int32_t pick_cap(const cbx_sampler* s, int32_t n_vocab, int32_t hint) {
    int32_t want = (hint > 0 && hint < n_vocab) ? hint : n_vocab;
    int32_t cap = 64;
    while (cap < want) cap <<= 1;
    const int32_t lim = cbx::max_cap_for_lds(n_vocab, s->lds_limit);
    return cap < lim ? cap : lim;
}

// The launch, and after a launch at a survivor capacity below the
// vocabulary's (a caller's max_survivors hint) the redo pass: rows with more
// survivors (ties at a tiny top-k threshold, top-k off, a hint below top_k)
// go on the redo list `redo` and are sampled again, on the same stream, at
// the largest capacity the device's LDS allows -- the whole vocabulary for
// every n_vocab <= 32768 on gfx950.
//
// A launch of at most `latency_rows` rows is bound by one row's latency, not
// by throughput: it runs at full capacity whatever the hint (the workgroup
// kernel, a row spread over several waves, with nothing to redo).
hipError_t launch_with_redo(int32_t full, cbx::KernelArgs a, int32_t* redo, int64_t latency_rows,
                            hipStream_t st) {
    const int64_t rows = (int64_t)a.n_steps * a.n_rows;
    if (rows <= latency_rows) a.cap = full;
    a.redo = a.cap < full ? redo : nullptr;
    a.redo_max = (int32_t)(rows < cbx::kRedoMax ? rows : cbx::kRedoMax);
    hipError_t e = cbx::launch_sample(a, st);
    if (e != hipSuccess || !a.redo) return e;
    a.cap = full;
    return cbx::launch_redo(a, st);
}

bool params_ok(const cbx_params* p) {
    // NaN knobs would make the reference's activation tests meaningless.
    return p->top_p == p->top_p && p->temp == p->temp && p->repeat_penalty == p->repeat_penalty &&
           p->min_p == p->min_p && p->cfg_weight == p->cfg_weight;
}

}  // namespace

namespace cbx {
int set_error(int code, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
    return code;
}
}  // namespace cbx

extern "C" {

const char* cbx_last_error(void) { return g_err; }

int32_t cbx_max_vocab(void) { return cbx::kMaxVocab; }

int cbx_sampler_create(cbx_sampler** out, int32_t device, int32_t max_vocab, int32_t max_history) {
    if (!out) return fail(CBX_ERR_INVALID, "cbx_sampler_create: out is NULL");
    *out = nullptr;
    if (max_vocab < 1 || max_vocab > cbx::kMaxVocab)
        return fail(CBX_ERR_INVALID, "cbx_sampler_create: max_vocab %d outside [1, %d]", max_vocab,
                    cbx::kMaxVocab);
    if (max_history < 0) return fail(CBX_ERR_INVALID, "cbx_sampler_create: max_history < 0");
    int n_dev = 0;
    CBX_HIP(hipGetDeviceCount(&n_dev));
    if (device < 0 || device >= n_dev)
        return fail(CBX_ERR_INVALID, "cbx_sampler_create: device %d of %d", device, n_dev);

    cbx_sampler* s = new (std::nothrow) cbx_sampler();
    if (!s) return fail(CBX_ERR_NOMEM, "cbx_sampler_create: out of host memory");
    s->device = device;
    s->max_vocab = max_vocab;
    s->max_history = max_history;
    DeviceGuard g(device);
    hipDeviceProp_t prop;
    hipError_t e = hipGetDeviceProperties(&prop, device);
    if (e != hipSuccess) {
        release(s);
        return fail(CBX_ERR_HIP, "hipGetDeviceProperties: %s", hipGetErrorString(e));
    }
    s->lds_limit = prop.sharedMemPerBlock > prop.sharedMemPerBlockOptin ? prop.sharedMemPerBlock
                                                                         : prop.sharedMemPerBlockOptin;
    const size_t W = (size_t)(max_vocab + 31) / 32;
    const size_t h = (size_t)(max_history > 0 ? max_history : 1);
    e = hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking);
    if (e == hipSuccess) e = hipMalloc(&s->d_logits, sizeof(float) * max_vocab);
    if (e == hipSuccess) e = hipMalloc(&s->d_uncond, sizeof(float) * max_vocab);
    if (e == hipSuccess) e = hipMalloc(&s->d_hist, sizeof(int32_t) * h);
    if (e == hipSuccess) e = hipMalloc(&s->d_hist_len, sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc(&s->d_params, sizeof(cbx_params));
    if (e == hipSuccess) e = hipMalloc(&s->d_allowed, sizeof(uint32_t) * W);
    if (e == hipSuccess) e = hipMalloc(&s->d_force, 1);
    if (e == hipSuccess) e = hipMalloc(&s->d_u, sizeof(double));
    if (e == hipSuccess) e = hipMalloc(&s->d_token, sizeof(int32_t));
    if (e == hipSuccess) e = hipMalloc(&s->d_info, sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(&s->d_probs, sizeof(float) * max_vocab);
    if (e == hipSuccess) e = hipMalloc(&s->d_redo, sizeof(int32_t) * cbx::kRedoWords);
    if (e == hipSuccess) e = hipMalloc(&s->d_redo_row, sizeof(int32_t) * 3);
    // the lists start empty; each redo pass leaves them empty again
    if (e == hipSuccess) e = hipMemset(s->d_redo, 0, sizeof(int32_t) * cbx::kRedoWords);
    if (e == hipSuccess) e = hipMemset(s->d_redo_row, 0, sizeof(int32_t) * 3);
    if (e == hipSuccess) e = hipHostMalloc((void**)&s->h_small, sizeof(cbx_sampler::Small));
    if (e == hipSuccess) e = static_scratch(device, &s->static_redo);
    if (e != hipSuccess) {
        release(s);
        return fail(e == hipErrorOutOfMemory ? CBX_ERR_NOMEM : CBX_ERR_HIP,
                    "cbx_sampler_create: %s", hipGetErrorString(e));
    }
    *out = s;
    return CBX_OK;
}

int cbx_sampler_set_latency_rows(cbx_sampler* s, int64_t rows) {
    if (!s) return fail(CBX_ERR_INVALID, "cbx_sampler_set_latency_rows: NULL handle");
    if (rows < 0) return fail(CBX_ERR_INVALID, "cbx_sampler_set_latency_rows: rows < 0");
    s->latency_rows = rows;
    return CBX_OK;
}

int cbx_sampler_destroy(cbx_sampler* s) {
    if (!s) return CBX_OK;
    release(s);
    return CBX_OK;
}

int cbx_sample_row_ex(cbx_sampler* s, const float* logits, const float* logits_uncond,
                      int32_t n_vocab, const int32_t* history, int32_t n_history,
                      const cbx_params* params, const uint32_t* allowed, int32_t force_stop,
                      int32_t stop_token, double u, int32_t* token_out, uint32_t* info_out,
                      float* probs_out) {
    if (!s || !logits || !params || !token_out)
        return fail(CBX_ERR_INVALID, "cbx_sample_row: NULL handle, logits, params or token_out");
    if (n_vocab < 1 || n_vocab > s->max_vocab)
        return fail(CBX_ERR_INVALID, "cbx_sample_row: n_vocab %d outside [1, %d]", n_vocab,
                    s->max_vocab);
    if (n_history < 0 || n_history > s->max_history || (n_history > 0 && !history))
        return fail(CBX_ERR_INVALID, "cbx_sample_row: history of %d ids (handle holds %d)",
                    n_history, s->max_history);
    if (!params_ok(params)) return fail(CBX_ERR_INVALID, "cbx_sample_row: NaN parameter");
    if (!(u >= 0.0 && u < 1.0)) return fail(CBX_ERR_INVALID, "cbx_sample_row: u outside [0, 1)");
    DeviceGuard g(s->device);
    hipStream_t st = s->stream;
    cbx_sampler::Small* hs = s->h_small;
    hs->params = *params;
    hs->u = u;
    hs->hist_len = n_history;
    hs->force = force_stop ? 1 : 0;
    const size_t W = (size_t)(n_vocab + 31) / 32;
    CBX_HIP(hipMemcpyAsync(s->d_logits, logits, sizeof(float) * n_vocab, hipMemcpyHostToDevice, st));
    if (logits_uncond)
        CBX_HIP(hipMemcpyAsync(s->d_uncond, logits_uncond, sizeof(float) * n_vocab,
                               hipMemcpyHostToDevice, st));
    if (n_history > 0)
        CBX_HIP(hipMemcpyAsync(s->d_hist, history, sizeof(int32_t) * n_history,
                               hipMemcpyHostToDevice, st));
    if (allowed)
        CBX_HIP(hipMemcpyAsync(s->d_allowed, allowed, sizeof(uint32_t) * W, hipMemcpyHostToDevice, st));
    CBX_HIP(hipMemcpyAsync(s->d_params, &hs->params, sizeof(cbx_params), hipMemcpyHostToDevice, st));
    CBX_HIP(hipMemcpyAsync(s->d_u, &hs->u, sizeof(double), hipMemcpyHostToDevice, st));
    CBX_HIP(hipMemcpyAsync(s->d_hist_len, &hs->hist_len, sizeof(int32_t), hipMemcpyHostToDevice, st));
    CBX_HIP(hipMemcpyAsync(s->d_force, &hs->force, 1, hipMemcpyHostToDevice, st));

    cbx::KernelArgs a{};
    a.n_rows = 1;
    a.n_vocab = n_vocab;
    a.n_steps = 1;
    a.stop_token = stop_token;
    a.logits = s->d_logits;
    a.ld_logits = n_vocab;
    a.uncond = logits_uncond ? s->d_uncond : nullptr;
    a.params = s->d_params;
    a.history = s->d_hist;
    a.history_len = s->d_hist_len;
    a.ld_history = n_history;
    a.allowed = allowed ? s->d_allowed : nullptr;
    a.ld_allowed = (int64_t)W;
    a.force_stop = s->d_force;
    a.draw_mode = CBX_DRAW_UNIFORM;
    a.cap = pick_cap(s, n_vocab, (params->top_k > 0 && params->top_k < n_vocab) ? params->top_k : 0);
    a.uniforms = s->d_u;
    a.tokens = s->d_token;
    a.info = s->d_info;
    a.probs = probs_out ? s->d_probs : nullptr;
    a.ld_probs = n_vocab;
    CBX_HIP(launch_with_redo(pick_cap(s, n_vocab, 0), a, s->d_redo_row, s->latency_rows, st));
    CBX_HIP(hipMemcpyAsync(&hs->token, s->d_token, sizeof(int32_t), hipMemcpyDeviceToHost, st));
    CBX_HIP(hipMemcpyAsync(&hs->info, s->d_info, sizeof(uint32_t), hipMemcpyDeviceToHost, st));
    if (probs_out)
        CBX_HIP(hipMemcpyAsync(probs_out, s->d_probs, sizeof(float) * n_vocab, hipMemcpyDeviceToHost, st));
    CBX_HIP(hipStreamSynchronize(st));
    *token_out = hs->token;
    if (info_out) *info_out = hs->info;
    if (hs->info & CBX_INFO_OVERFLOW)
        return fail(CBX_ERR_UNSUPPORTED,
                    "cbx_sample_row: more survivors after top-k than the on-chip capacity %d", a.cap);
    return CBX_OK;
}

int cbx_sample_row(cbx_sampler* s, const float* logits, int32_t n_vocab, const int32_t* history,
                   int32_t n_history, const cbx_params* params, double u, int32_t* token_out,
                   uint32_t* info_out) {
    return cbx_sample_row_ex(s, logits, nullptr, n_vocab, history, n_history, params, nullptr, 0,
                             0, u, token_out, info_out, nullptr);
}

}  // extern "C"

namespace {
// Checks a batched request and fills the kernel arguments (fn names the
// entry point in messages).
int batch_args(const char* fn, const cbx_sampler* s, const cbx_batch* b, cbx::KernelArgs& a) {
    if (!s || !b) return fail(CBX_ERR_INVALID, "%s: NULL handle or batch", fn);
    if (b->n_rows < 1 || b->n_steps < 1)
        return fail(CBX_ERR_INVALID, "%s: n_rows %d, n_steps %d", fn, b->n_rows, b->n_steps);
    if ((int64_t)b->n_rows * b->n_steps > 0x7fffffffLL)
        return fail(CBX_ERR_INVALID, "%s: n_rows * n_steps exceeds 2^31-1", fn);
    if (b->n_vocab < 1 || b->n_vocab > cbx::kMaxVocab)
        return fail(CBX_ERR_INVALID, "%s: n_vocab %d outside [1, %d]", fn, b->n_vocab,
                    cbx::kMaxVocab);
    if (!b->logits || !b->params || !b->tokens)
        return fail(CBX_ERR_INVALID, "%s: NULL logits, params or tokens", fn);
    if (b->ld_logits < b->n_vocab)
        return fail(CBX_ERR_INVALID, "%s: ld_logits %lld < n_vocab %d", fn,
                    (long long)b->ld_logits, b->n_vocab);
    if (b->history && (!b->history_len || b->ld_history < 0))
        return fail(CBX_ERR_INVALID, "%s: history without history_len/ld_history", fn);
    if (b->allowed && b->ld_allowed < (b->n_vocab + 31) / 32)
        return fail(CBX_ERR_INVALID, "%s: ld_allowed %lld < ceil(n_vocab/32)", fn,
                    (long long)b->ld_allowed);
    if (b->probs && b->ld_probs < b->n_vocab)
        return fail(CBX_ERR_INVALID, "%s: ld_probs %lld < n_vocab", fn, (long long)b->ld_probs);
    if (b->draw_mode == CBX_DRAW_UNIFORM) {
        if (!b->uniforms) return fail(CBX_ERR_INVALID, "%s: uniforms is NULL", fn);
    } else if (b->draw_mode != CBX_DRAW_PHILOX) {
        return fail(CBX_ERR_INVALID, "%s: unknown draw_mode %d", fn, b->draw_mode);
    }
    if (b->max_survivors < 0) return fail(CBX_ERR_INVALID, "%s: max_survivors < 0", fn);
    a = cbx::KernelArgs{};
    a.n_rows = b->n_rows;
    a.n_vocab = b->n_vocab;
    a.n_steps = b->n_steps;
    a.stop_token = b->stop_token;
    a.logits = b->logits;
    a.ld_logits = b->ld_logits;
    a.uncond = b->logits_uncond;
    a.params = b->params;
    a.history = b->history;
    a.history_len = b->history_len;
    a.ld_history = b->ld_history;
    a.allowed = b->allowed;
    a.ld_allowed = b->ld_allowed;
    a.force_stop = b->force_stop;
    a.draw_mode = b->draw_mode;
    a.cap = pick_cap(s, b->n_vocab, b->max_survivors);
    a.uniforms = b->uniforms;
    a.seed = b->seed;
    a.stream_ids = b->stream_ids;
    a.step0 = b->step0;
    a.tokens = b->tokens;
    a.info = b->info;
    a.probs = b->probs;
    a.ld_probs = b->ld_probs;
    return CBX_OK;
}

// A decode step's batch: b with d's history (one step only).
int decode_batch(const char* fn, const cbx_batch* b, const cbx_decode* d, cbx_batch& bb) {
    if (!b || !d) return fail(CBX_ERR_INVALID, "%s: NULL batch or decode state", fn);
    if (b->n_steps != 1)
        return fail(CBX_ERR_INVALID, "%s: n_steps %d (a decode step samples one step)", fn,
                    b->n_steps);
    if (!d->state || !d->history || !d->history_len || d->ld_history < 1)
        return fail(CBX_ERR_INVALID, "%s: NULL state, history or history_len, or ld_history < 1",
                    fn);
    bb = *b;
    bb.history = d->history;
    bb.history_len = d->history_len;
    bb.ld_history = d->ld_history;
    return CBX_OK;
}

// The batched sampler on the handle's redo list, or with d set a decode step:
// its own kernel at the capacity of the whole vocabulary (no row overflows,
// so no redo pass), max_survivors ignored.
int sample(const char* fn, cbx_sampler* s, const cbx_batch* b, const cbx_decode* d,
           hipStream_t st) {
    cbx::KernelArgs a;
    const int rc = batch_args(fn, s, b, a);
    if (rc != CBX_OK) return rc;
    const int32_t full = pick_cap(s, b->n_vocab, 0);
    DeviceGuard g(s->device);
    if (d) {
        if (full < b->n_vocab)
            return fail(CBX_ERR_UNSUPPORTED, "%s: this device's LDS holds %d of %d survivors", fn,
                        full, b->n_vocab);
        a.cap = full;
        a.dec_state = d->state;
        a.dec_history = d->history;
        a.dec_len = d->history_len;
        a.dec_max = d->max_len;
        a.dec_next = d->next_token;
        CBX_HIP(cbx::launch_decode(a, st));
        return CBX_OK;
    }
    CBX_HIP(launch_with_redo(full, a, s->d_redo, s->latency_rows, st));
    return CBX_OK;
}
}  // namespace

extern "C" {

int cbx_sample_batch(cbx_sampler* s, const cbx_batch* b, void* stream) {
    return sample("cbx_sample_batch", s, b, nullptr, (hipStream_t)stream);
}

int cbx_decode_step(cbx_sampler* s, const cbx_batch* b, const cbx_decode* d, void* stream) {
    cbx_batch bb;
    const int rc = decode_batch("cbx_decode_step", b, d, bb);
    if (rc != CBX_OK) return rc;
    return sample("cbx_decode_step", s, &bb, d, (hipStream_t)stream);
}

int cbx_sample_batch_static(cbx_sampler* s, const cbx_batch* b, void* stream) {
    cbx::KernelArgs a;
    const int rc = batch_args("cbx_sample_batch_static", s, b, a);
    if (rc != CBX_OK) return rc;
    const int32_t full = pick_cap(s, b->n_vocab, 0);
    const int64_t rows = (int64_t)b->n_rows * b->n_steps;
    // calls of at most latency_rows row-steps run at full capacity (no redo
    // list is used), whatever their survivor bound
    if (rows > s->latency_rows && a.cap < full && rows > cbx::kRedoMax)
        return fail(CBX_ERR_INVALID,
                    "cbx_sample_batch_static: %lld row-steps with max_survivors %d: its redo list "
                    "holds %d rows (at most %d row-steps per call, or max_survivors 0)",
                    (long long)rows, b->max_survivors, cbx::kRedoMax, cbx::kRedoMax);
    if (!s->static_redo)
        return fail(CBX_ERR_HIP, "cbx_sample_batch_static: no device address of the redo list");
    DeviceGuard g(s->device);
    CBX_HIP(launch_with_redo(full, a, s->static_redo, s->latency_rows, (hipStream_t)stream));
    return CBX_OK;
}

namespace {
int check_head(const char* fn, const cbx_head* h, int32_t n_rows, int32_t n_vocab,
               int64_t ld_logits) {
    if (!h || !h->weights || !h->hidden || !h->logits)
        return fail(CBX_ERR_INVALID, "%s: NULL head, weights, hidden or logits", fn);
    if (cbx::wtype_block_bytes(h->wtype) == 0)
        return fail(CBX_ERR_INVALID, "%s: unknown wtype %d", fn, h->wtype);
    if (h->n_embd < 32 || h->n_embd > 16384 || h->n_embd % 32)
        return fail(CBX_ERR_INVALID, "%s: n_embd %d not a multiple of 32 in [32, 16384]", fn,
                    h->n_embd);
    if (h->ld_hidden < h->n_embd)
        return fail(CBX_ERR_INVALID, "%s: ld_hidden %lld < n_embd %d", fn,
                    (long long)h->ld_hidden, h->n_embd);
    if (h->hidden_uncond && !h->logits_uncond)
        return fail(CBX_ERR_INVALID, "%s: hidden_uncond without logits_uncond", fn);
    if (n_rows < 1 || n_vocab < 1 || n_vocab > cbx::kMaxVocab || ld_logits < n_vocab)
        return fail(CBX_ERR_INVALID, "%s: n_rows %d, n_vocab %d, ld_logits %lld", fn, n_rows,
                    n_vocab, (long long)ld_logits);
    // the kernel's buffer descriptors address the weights and rows in 32 bits
    const int64_t bpb = cbx::wtype_block_bytes(h->wtype);
    if ((int64_t)n_vocab * (h->n_embd / 32) * bpb > 0x7fffffffLL ||
        ((int64_t)n_rows * h->ld_hidden + h->n_embd) * 4 > 0x7fffffffLL ||
        (int64_t)(h->hidden_uncond ? 2 : 1) * (n_rows + 15) * h->n_embd * 4 > 0x7fffffffLL)
        return fail(CBX_ERR_UNSUPPORTED, "%s: weights or hidden rows past 2 GiB", fn);
    return CBX_OK;
}

// The handle's split buffer holds one call's activations at a time: head calls
// on one handle are ordered on one stream (a larger call than any before
// waits for the device while the buffer is replaced).
int run_head(cbx_sampler* s, const cbx_head* h, int32_t n_rows, int32_t n_vocab,
             int64_t ld_logits, hipStream_t st) {
    const size_t need = cbx::head_scratch_bytes(n_rows, h->hidden_uncond != nullptr, h->n_embd);
    if (need > s->head_bytes) {
        CBX_HIP(hipDeviceSynchronize());
        CBX_HIP(hipFree(s->d_head));
        s->d_head = nullptr;
        s->head_bytes = 0;
        CBX_HIP(hipMalloc(&s->d_head, need));
        s->head_bytes = need;
    }
    CBX_HIP(cbx::launch_head(h->weights, h->wtype, h->bias, h->hidden, h->hidden_uncond,
                             h->ld_hidden, h->logits, h->logits_uncond, ld_logits, n_rows,
                             n_vocab, h->n_embd, s->d_head, st));
    return CBX_OK;
}
}  // namespace

int cbx_head_logits(cbx_sampler* s, const cbx_head* h, int32_t n_rows, int32_t n_vocab,
                    int64_t ld_logits, void* stream) {
    if (!s) return fail(CBX_ERR_INVALID, "cbx_head_logits: NULL handle");
    const int rc = check_head("cbx_head_logits", h, n_rows, n_vocab, ld_logits);
    if (rc != CBX_OK) return rc;
    DeviceGuard g(s->device);
    return run_head(s, h, n_rows, n_vocab, ld_logits, (hipStream_t)stream);
}

}  // extern "C"

namespace {
// The projection into h->logits, then the sampler over them (fn names the
// entry point in messages; d set: a decode step).
int head_then_sample(const char* fn, cbx_sampler* s, const cbx_head* h, const cbx_batch* b,
                     const cbx_decode* d, hipStream_t st) {
    if (!s || !b) return fail(CBX_ERR_INVALID, "%s: NULL handle or batch", fn);
    if (b->n_rows < 1 || b->n_steps < 1 || (int64_t)b->n_rows * b->n_steps > 0x7fffffffLL)
        return fail(CBX_ERR_INVALID, "%s: n_rows %d, n_steps %d", fn, b->n_rows, b->n_steps);
    const int32_t rows = b->n_rows * b->n_steps;
    const int rc = check_head(fn, h, rows, b->n_vocab, b->ld_logits);
    if (rc != CBX_OK) return rc;
    cbx_batch bb = *b;
    if (d) {
        const int rd = decode_batch(fn, b, d, bb);
        if (rd != CBX_OK) return rd;
    }
    bb.logits = h->logits;
    if (h->hidden_uncond) bb.logits_uncond = h->logits_uncond;
    {
        DeviceGuard g(s->device);
        const int rh = run_head(s, h, rows, b->n_vocab, b->ld_logits, st);
        if (rh != CBX_OK) return rh;
    }
    return sample(fn, s, &bb, d, st);
}
}  // namespace

extern "C" {

int cbx_head_sample_batch(cbx_sampler* s, const cbx_head* h, const cbx_batch* b, void* stream) {
    return head_then_sample("cbx_head_sample_batch", s, h, b, nullptr, (hipStream_t)stream);
}

int cbx_head_decode_step(cbx_sampler* s, const cbx_head* h, const cbx_batch* b,
                         const cbx_decode* d, void* stream) {
    return head_then_sample("cbx_head_decode_step", s, h, b, d, (hipStream_t)stream);
}

}  // extern "C"

namespace {
// cbx_t3_step and cbx_t3_prefill (slots set): the checks and the launch.
int t3_run(const char* fn, cbx_sampler* s, const cbx_t3_model* m, int32_t n_rows,
           const int32_t* tokens, const float* inputs, int32_t* positions, const int32_t* state,
           const int32_t* slots, int32_t n_slots, const cbx_t3_cache* cache, float* hidden,
           void* stream) {
    if (!s || !m || !cache) return fail(CBX_ERR_INVALID, "%s: NULL handle, model or cache", fn);
    if (n_rows < 1) return fail(CBX_ERR_INVALID, "%s: n_rows %d", fn, n_rows);
    if (m->n_layer < 1 || m->n_layer > 256 || !m->layers)
        return fail(CBX_ERR_INVALID, "%s: n_layer %d or NULL layers", fn, m->n_layer);
    if (m->n_embd < 1 || m->n_embd > 4096 || !cbx::t3_shape_ok(m->n_embd, m->n_head))
        return fail(CBX_ERR_UNSUPPORTED,
                    "%s: n_embd %d, n_head %d (heads of 64, n_embd in {256..1024 by 256, 1536, "
                    "2048, 3072, 4096})", fn, m->n_embd, m->n_head);
    if (cbx::wtype_block_bytes(m->wtype) == 0)
        return fail(CBX_ERR_INVALID, "%s: unknown wtype %d", fn, m->wtype);
    if (!(m->eps >= 0.0f) || !m->wpe || !m->ln_f_g || !m->ln_f_b || m->n_pos < 1 ||
        (!inputs && (!tokens || !m->speech_emb || m->n_speech_vocab < 1)))
        return fail(CBX_ERR_INVALID, "%s: eps, wpe, ln_f, n_pos or the embedding missing", fn);
    for (int l = 0; l < m->n_layer; ++l) {
        const cbx_t3_layer& L = m->layers[l];
        if (!L.ln_1_g || !L.ln_1_b || !L.attn_w || !L.attn_b || !L.attn_proj_w ||
            !L.attn_proj_b || !L.ln_2_g || !L.ln_2_b || !L.fc_w || !L.fc_b || !L.fc_proj_w ||
            !L.fc_proj_b)
            return fail(CBX_ERR_INVALID, "%s: layer %d has a NULL tensor", fn, l);
    }
    if (!cache->k || !cache->v || cache->n_ctx < 1 || cache->n_ctx > m->n_pos)
        return fail(CBX_ERR_INVALID, "%s: cache k/v NULL or n_ctx %d outside [1, n_pos]", fn,
                    cache->n_ctx);
    if (cbx::t3_attn_lds(cache->n_ctx) + 2048 > s->lds_limit)
        return fail(CBX_ERR_UNSUPPORTED, "%s: n_ctx %d: the attention's LDS exceeds the device's",
                    fn, cache->n_ctx);
    if (!positions || !hidden) return fail(CBX_ERR_INVALID, "%s: NULL positions or hidden", fn);
    // the matrix kernels' buffer descriptors address rows in 32 bits
    if ((int64_t)n_rows * 4 * m->n_embd * 4 > 0x7fffffffLL)
        return fail(CBX_ERR_UNSUPPORTED, "%s: %d rows past 2 GiB of activations", fn, n_rows);
    DeviceGuard g(s->device);
    const size_t need = cbx::t3_workspace_bytes(n_rows, m->n_embd);
    if (need > s->t3_bytes) {
        CBX_HIP(hipDeviceSynchronize());
        CBX_HIP(hipFree(s->d_t3));
        s->d_t3 = nullptr;
        s->t3_bytes = 0;
        CBX_HIP(hipMalloc(&s->d_t3, need));
        s->t3_bytes = need;
    }
    CBX_HIP(cbx::launch_t3_step(*m, n_rows, tokens, inputs, positions, state, slots, n_slots,
                                *cache, hidden, s->d_t3, (hipStream_t)stream));
    return CBX_OK;
}
}  // namespace

extern "C" {

int cbx_t3_step(cbx_sampler* s, const cbx_t3_model* m, int32_t n_rows, const int32_t* tokens,
                const float* inputs, int32_t* positions, const int32_t* state,
                const cbx_t3_cache* cache, float* hidden, void* stream) {
    return t3_run("cbx_t3_step", s, m, n_rows, tokens, inputs, positions, state, nullptr, 0,
                  cache, hidden, stream);
}

int cbx_t3_prefill(cbx_sampler* s, const cbx_t3_model* m, int32_t n_rows, const int32_t* slots,
                   int32_t n_slots, const int32_t* tokens, const float* inputs,
                   const int32_t* positions, const cbx_t3_cache* cache, float* hidden,
                   void* stream) {
    if (!slots || n_slots < 1)
        return fail(CBX_ERR_INVALID, "cbx_t3_prefill: NULL slots or n_slots %d", n_slots);
    // positions are read, not advanced, in the prefill form
    return t3_run("cbx_t3_prefill", s, m, n_rows, tokens, inputs, const_cast<int32_t*>(positions),
                  nullptr, slots, n_slots, cache, hidden, stream);
}


}  // extern "C"
