"""chatterbox.cpp_amd -- MI355X (gfx950) T3 logits->token sampler.

Python view of the C ABI in include/cbx_sampler.h (libcbx_sampler.so, built
in-tree by ``make -C chatterbox.cpp_amd``).  The product is the shared library;
this module only loads it with ctypes and passes device pointers (taken from
torch tensors) and the current HIP stream.  There is no Python or CPU fallback:
if the library is missing, importing or calling raises.

The per-row semantics are those of the reference's
``tts_cpp::chatterbox::detail::sample_next_token_ex`` (src/main.cpp:726-801).
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
# The in-tree build; CBX_SAMPLER_LIB names another build of the same library.
LIB_PATH = os.environ.get("CBX_SAMPLER_LIB") or os.path.join(_HERE, "lib", "libcbx_sampler.so")

CBX_OK = 0
CBX_ERR_INVALID = -1
CBX_ERR_HIP = -2
CBX_ERR_UNSUPPORTED = -3
CBX_ERR_NOMEM = -4

CBX_INFO_DREW = 0x01
CBX_INFO_GREEDY = 0x02
CBX_INFO_EMPTY = 0x04
CBX_INFO_TOPP_TIE = 0x08
CBX_INFO_NONFINITE = 0x10
CBX_INFO_OVERFLOW = 0x20
CBX_INFO_TOPP_SORTED = 0x80

CBX_INFO_ENDED = 0x40

CBX_DRAW_UNIFORM = 0
CBX_DRAW_PHILOX = 1

CBX_DECODE_RUNNING = 0
CBX_DECODE_STOP = 1
CBX_DECODE_LIMIT = 2


class Params(ctypes.Structure):
    """cbx_params (include/cbx_sampler.h); the first four fields are
    chatterbox_sampling_params (src/chatterbox_t3_internal.h:113-118)."""

    _fields_ = [
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("temp", ctypes.c_float),
        ("repeat_penalty", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("cfg_weight", ctypes.c_float),
    ]


PARAMS_DTYPE_FIELDS = ("top_k", "top_p", "temp", "repeat_penalty", "min_p", "cfg_weight")


class Batch(ctypes.Structure):
    """cbx_batch (include/cbx_sampler.h)."""

    _fields_ = [
        ("n_rows", ctypes.c_int32),
        ("n_vocab", ctypes.c_int32),
        ("n_steps", ctypes.c_int32),
        ("stop_token", ctypes.c_int32),
        ("logits", ctypes.c_void_p),
        ("ld_logits", ctypes.c_int64),
        ("logits_uncond", ctypes.c_void_p),
        ("params", ctypes.c_void_p),
        ("history", ctypes.c_void_p),
        ("history_len", ctypes.c_void_p),
        ("ld_history", ctypes.c_int64),
        ("allowed", ctypes.c_void_p),
        ("ld_allowed", ctypes.c_int64),
        ("force_stop", ctypes.c_void_p),
        ("draw_mode", ctypes.c_int32),
        ("max_survivors", ctypes.c_int32),
        ("uniforms", ctypes.c_void_p),
        ("seed", ctypes.c_uint64),
        ("stream_ids", ctypes.c_void_p),
        ("step0", ctypes.c_uint64),
        ("tokens", ctypes.c_void_p),
        ("info", ctypes.c_void_p),
        ("probs", ctypes.c_void_p),
        ("ld_probs", ctypes.c_int64),
    ]


CBX_WTYPE_F16, CBX_WTYPE_Q4_0, CBX_WTYPE_Q5_0, CBX_WTYPE_Q8_0 = 1, 2, 6, 8


class Head(ctypes.Structure):
    """cbx_head (include/cbx_sampler.h): the speech_head projection."""

    _fields_ = [
        ("weights", ctypes.c_void_p),
        ("wtype", ctypes.c_int32),
        ("n_embd", ctypes.c_int32),
        ("bias", ctypes.c_void_p),
        ("hidden", ctypes.c_void_p),
        ("hidden_uncond", ctypes.c_void_p),
        ("ld_hidden", ctypes.c_int64),
        ("logits", ctypes.c_void_p),
        ("logits_uncond", ctypes.c_void_p),
    ]


class Decode(ctypes.Structure):
    """cbx_decode (include/cbx_sampler.h): device-resident decode state."""

    _fields_ = [
        ("state", ctypes.c_void_p),
        ("history", ctypes.c_void_p),
        ("history_len", ctypes.c_void_p),
        ("ld_history", ctypes.c_int64),
        ("max_len", ctypes.c_void_p),
        ("next_token", ctypes.c_void_p),
    ]


class T3Layer(ctypes.Structure):
    """cbx_t3_layer (include/cbx_t3.h)."""

    _fields_ = [(f, ctypes.c_void_p) for f in (
        "ln_1_g", "ln_1_b", "attn_w", "attn_b", "attn_proj_w", "attn_proj_b", "ln_2_g", "ln_2_b",
        "fc_w", "fc_b", "fc_proj_w", "fc_proj_b")]


class T3Model(ctypes.Structure):
    """cbx_t3_model (include/cbx_t3.h)."""

    _fields_ = [
        ("n_layer", ctypes.c_int32),
        ("n_embd", ctypes.c_int32),
        ("n_head", ctypes.c_int32),
        ("n_pos", ctypes.c_int32),
        ("n_speech_vocab", ctypes.c_int32),
        ("wtype", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("wpe", ctypes.c_void_p),
        ("speech_emb", ctypes.c_void_p),
        ("layers", ctypes.POINTER(T3Layer)),
        ("ln_f_g", ctypes.c_void_p),
        ("ln_f_b", ctypes.c_void_p),
    ]


class T3Cache(ctypes.Structure):
    """cbx_t3_cache (include/cbx_t3.h)."""

    _fields_ = [("k", ctypes.c_void_p), ("v", ctypes.c_void_p), ("n_ctx", ctypes.c_int32)]


class HeadFile(ctypes.Structure):
    """cbx_head_file (include/cbx_gguf.h): the speech_head of a T3 GGUF."""

    _fields_ = [
        ("n_vocab", ctypes.c_int32),
        ("n_embd", ctypes.c_int32),
        ("wtype", ctypes.c_int32),
        ("has_bias", ctypes.c_int32),
        ("speech_vocab_size", ctypes.c_int32),
        ("start_speech_token", ctypes.c_int32),
        ("stop_speech_token", ctypes.c_int32),
        ("gguf_version", ctypes.c_int32),
        ("weight_offset", ctypes.c_uint64),
        ("weight_bytes", ctypes.c_uint64),
        ("bias_offset", ctypes.c_uint64),
        ("bias_bytes", ctypes.c_uint64),
    ]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


class T3File(ctypes.Structure):
    """cbx_t3_file (include/cbx_gguf.h): the T3 transformer of a T3 GGUF."""

    _fields_ = [
        ("n_layer", ctypes.c_int32),
        ("n_embd", ctypes.c_int32),
        ("n_head", ctypes.c_int32),
        ("n_pos", ctypes.c_int32),
        ("n_speech_vocab", ctypes.c_int32),
        ("wtype", ctypes.c_int32),
        ("eps", ctypes.c_float),
        ("start_speech_token", ctypes.c_int32),
        ("stop_speech_token", ctypes.c_int32),
        ("gguf_version", ctypes.c_int32),
        ("device_bytes", ctypes.c_uint64),
    ]

    def as_dict(self):
        return {f: getattr(self, f) for f, _ in self._fields_}


class Retry(ctypes.Structure):
    """cbx_retry (include/cbx_retry.h): the early-stop retry policy of one segment."""

    _fields_ = [(f, ctypes.c_int32) for f in (
        "min_tokens", "max_retries", "attempt", "done", "best_attempt", "best_len",
        "kept_attempt", "kept_len")]


class CbxError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"cbx error {code}: {msg}")
        self.code = code


_lib = None


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libcbx_sampler.so and declare its prototypes.  Raises if absent."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is not built; run `make -C chatterbox.cpp_amd` (or __graft_entry__.build())")
    # Load torch's HIP runtime first when torch is present, so the library
    # binds to the same runtime instance (same devices, streams and memory)
    # instead of loading a second copy of libamdhip64 into the process.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    lib = ctypes.CDLL(path)
    vp, i32, i64, u64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64
    lib.cbx_max_vocab.restype = i32
    lib.cbx_max_vocab.argtypes = []
    lib.cbx_sampler_create.restype = ctypes.c_int
    lib.cbx_sampler_create.argtypes = [ctypes.POINTER(vp), i32, i32, i32]
    lib.cbx_sampler_destroy.restype = ctypes.c_int
    lib.cbx_sampler_destroy.argtypes = [vp]
    lib.cbx_sampler_set_latency_rows.restype = ctypes.c_int
    lib.cbx_sampler_set_latency_rows.argtypes = [vp, ctypes.c_int64]
    lib.cbx_sample_row.restype = ctypes.c_int
    lib.cbx_sample_row.argtypes = [vp, vp, i32, vp, i32, ctypes.POINTER(Params), ctypes.c_double,
                                   ctypes.POINTER(i32), ctypes.POINTER(ctypes.c_uint32)]
    lib.cbx_sample_row_ex.restype = ctypes.c_int
    lib.cbx_sample_row_ex.argtypes = [vp, vp, vp, i32, vp, i32, ctypes.POINTER(Params), vp, i32,
                                      i32, ctypes.c_double, ctypes.POINTER(i32),
                                      ctypes.POINTER(ctypes.c_uint32), vp]
    lib.cbx_sample_batch.restype = ctypes.c_int
    lib.cbx_sample_batch.argtypes = [vp, ctypes.POINTER(Batch), vp]
    lib.cbx_sample_batch_static.restype = ctypes.c_int
    lib.cbx_sample_batch_static.argtypes = [vp, ctypes.POINTER(Batch), vp]
    lib.cbx_head_logits.restype = ctypes.c_int
    lib.cbx_head_logits.argtypes = [vp, ctypes.POINTER(Head), i32, i32, i64, vp]
    lib.cbx_head_sample_batch.restype = ctypes.c_int
    lib.cbx_head_sample_batch.argtypes = [vp, ctypes.POINTER(Head), ctypes.POINTER(Batch), vp]
    lib.cbx_decode_step.restype = ctypes.c_int
    lib.cbx_decode_step.argtypes = [vp, ctypes.POINTER(Batch), ctypes.POINTER(Decode), vp]
    lib.cbx_head_decode_step.restype = ctypes.c_int
    lib.cbx_head_decode_step.argtypes = [vp, ctypes.POINTER(Head), ctypes.POINTER(Batch),
                                         ctypes.POINTER(Decode), vp]
    lib.cbx_t3_step.restype = ctypes.c_int
    lib.cbx_t3_step.argtypes = [vp, ctypes.POINTER(T3Model), i32, vp, vp, vp, vp,
                                ctypes.POINTER(T3Cache), vp, vp]
    lib.cbx_t3_prefill.restype = ctypes.c_int
    lib.cbx_t3_prefill.argtypes = [vp, ctypes.POINTER(T3Model), i32, vp, i32, vp, vp, vp,
                                   ctypes.POINTER(T3Cache), vp, vp]
    lib.cbx_gguf_read_head.restype = ctypes.c_int
    lib.cbx_gguf_read_head.argtypes = [ctypes.c_char_p, ctypes.POINTER(HeadFile)]
    lib.cbx_gguf_load_head.restype = ctypes.c_int
    lib.cbx_gguf_load_head.argtypes = [ctypes.c_char_p, ctypes.POINTER(HeadFile), vp, vp]
    lib.cbx_gguf_read_t3.restype = ctypes.c_int
    lib.cbx_gguf_read_t3.argtypes = [ctypes.c_char_p, ctypes.POINTER(T3File)]
    lib.cbx_gguf_load_t3.restype = ctypes.c_int
    lib.cbx_gguf_load_t3.argtypes = [ctypes.c_char_p, ctypes.POINTER(T3File), vp,
                                     ctypes.POINTER(T3Layer), ctypes.POINTER(T3Model)]
    lib.cbx_retry_init.restype = ctypes.c_int
    lib.cbx_retry_init.argtypes = [ctypes.POINTER(Retry), i32]
    lib.cbx_retry_stream_id.restype = u64
    lib.cbx_retry_stream_id.argtypes = [u64, i32]
    lib.cbx_retry_record.restype = ctypes.c_int
    lib.cbx_retry_record.argtypes = [ctypes.POINTER(Retry), i32, i32]
    lib.cbx_retry_record_tokens.restype = ctypes.c_int
    lib.cbx_retry_record_tokens.argtypes = [ctypes.POINTER(Retry), i32, i32, i32, i32]
    lib.cbx_last_error.restype = ctypes.c_char_p
    lib.cbx_last_error.argtypes = []
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != CBX_OK:
        raise CbxError(rc, _lib.cbx_last_error().decode(errors="replace"))


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream_ptr():
    import torch
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def read_head_gguf(path) -> HeadFile:
    """cbx_gguf_read_head: parse the speech_head of a T3 GGUF (host only)."""
    lib = load_library()
    info = HeadFile()
    _check(lib.cbx_gguf_read_head(os.fsencode(path), ctypes.byref(info)))
    return info


def load_head_gguf(path, device="cuda"):
    """cbx_gguf_load_head into new device tensors: returns (info, weights as
    uint8 bytes of the wtype layout, bias float32 or None), ready for
    Sampler.head."""
    import torch
    info = read_head_gguf(path)
    w = torch.empty(int(info.weight_bytes), dtype=torch.uint8, device=device)
    b = torch.empty(info.n_vocab, dtype=torch.float32, device=device) if info.has_bias else None
    _check(_lib.cbx_gguf_load_head(os.fsencode(path), ctypes.byref(info),
                                   ctypes.c_void_p(w.data_ptr()), _ptr(b)))
    return info, w, b


def read_t3_gguf(path) -> T3File:
    """cbx_gguf_read_t3: the T3 transformer's shape in the GGUF at `path`."""
    load_library()
    info = T3File()
    _check(_lib.cbx_gguf_read_t3(os.fsencode(path), ctypes.byref(info)))
    return info


def load_t3_gguf(path, device="cuda"):
    """cbx_gguf_load_t3 into one new device buffer: returns (info, model),
    the T3Model ready for Sampler.t3_step (it keeps the buffer alive)."""
    import torch
    info = read_t3_gguf(path)
    buf = torch.empty(int(info.device_bytes), dtype=torch.uint8, device=device)
    layers = (T3Layer * info.n_layer)()
    m = T3Model()
    _check(_lib.cbx_gguf_load_t3(os.fsencode(path), ctypes.byref(info),
                                 ctypes.c_void_p(buf.data_ptr()), layers, ctypes.byref(m)))
    m.layers = layers
    m._keep = (buf, layers)
    return info, m


def retry_start(n_text_tokens) -> Retry:
    """cbx_retry_init: the retry policy for a segment of n_text_tokens."""
    r = Retry()
    _check(load_library().cbx_retry_init(ctypes.byref(r), n_text_tokens))
    return r


def retry_record(r: Retry, n_tokens, stopped_by_stop_token) -> bool:
    """cbx_retry_record: True if another attempt should run (r.attempt)."""
    rc = _lib.cbx_retry_record(ctypes.byref(r), n_tokens, 1 if stopped_by_stop_token else 0)
    if rc < 0:
        _check(rc)
    return rc == 1


def retry_record_tokens(r: Retry, n_sampled, last_token, stop_token, n_predict) -> bool:
    """cbx_retry_record_tokens: the record from the tokens drawn in the
    attempt; True if another attempt should run (r.attempt)."""
    rc = _lib.cbx_retry_record_tokens(ctypes.byref(r), n_sampled, last_token, stop_token,
                                      n_predict)
    if rc < 0:
        _check(rc)
    return rc == 1


def retry_stream_id(stream, attempt) -> int:
    """cbx_retry_stream_id: the Philox stream id of a stream's attempt."""
    return int(load_library().cbx_retry_stream_id(stream, attempt))


def params_tensor(rows, device="cuda"):
    """Pack per-row knobs into a device tensor laid out as cbx_params[n]:
    rows is a sequence of dicts or Params."""
    import numpy as np
    import torch
    n = len(rows)
    arr = (Params * n)()
    for i, r in enumerate(rows):
        if isinstance(r, Params):
            arr[i] = r
        else:
            arr[i] = Params(**r)
    raw = np.frombuffer(bytes(arr), dtype=np.uint8).copy()
    return torch.from_numpy(raw).to(device)


class Sampler:
    """Owns one cbx_sampler handle (include/cbx_sampler.h)."""

    def __init__(self, device: int = 0, max_vocab: int = 32768, max_history: int = 4096):
        self.lib = load_library()
        h = ctypes.c_void_p()
        _check(self.lib.cbx_sampler_create(ctypes.byref(h), device, max_vocab, max_history))
        self.handle = h

    def close(self):
        if getattr(self, "handle", None):
            self.lib.cbx_sampler_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def set_latency_rows(self, rows: int):
        """Calls of at most `rows` row-steps run at full survivor capacity on
        the workgroup kernel (default 512; 0: never)."""
        _check(self.lib.cbx_sampler_set_latency_rows(self.handle, rows))

    # -- single row, host memory (the reference call shape) -------------------
    def sample_row(self, logits, history, params, u, logits_uncond=None, allowed=None,
                   force_stop=False, stop_token=0, want_probs=False):
        import numpy as np
        lg = np.ascontiguousarray(logits, dtype=np.float32)
        hist = np.ascontiguousarray(history if history is not None else [], dtype=np.int32)
        unc = None if logits_uncond is None else np.ascontiguousarray(logits_uncond, dtype=np.float32)
        al = None if allowed is None else np.ascontiguousarray(allowed, dtype=np.uint32)
        probs = np.zeros(lg.size, dtype=np.float32) if want_probs else None
        p = params if isinstance(params, Params) else Params(**params)
        tok = ctypes.c_int32()
        info = ctypes.c_uint32()
        _check(self.lib.cbx_sample_row_ex(
            self.handle, lg.ctypes.data, None if unc is None else unc.ctypes.data, lg.size,
            hist.ctypes.data if hist.size else None, hist.size, ctypes.byref(p),
            None if al is None else al.ctypes.data, 1 if force_stop else 0, stop_token,
            float(u), ctypes.byref(tok), ctypes.byref(info),
            None if probs is None else probs.ctypes.data))
        return (tok.value, info.value, probs) if want_probs else (tok.value, info.value)

    # -- batched, device memory ------------------------------------------------
    def sample_batch(self, logits, params, tokens, *, n_steps=1, uniforms=None,
                     logits_uncond=None, history=None, history_len=None, allowed=None,
                     force_stop=None, stop_token=0, info=None, probs=None,
                     draw_mode=None, seed=0, stream_ids=None, step0=0, max_survivors=0,
                     n_vocab=None, stream=None, head=None, static_scratch=False, decode=None):
        """logits: device float32 [n_steps*n_rows, ld] (or [n_steps, n_rows, ld]);
        params: device uint8 tensor from params_tensor(); tokens: device int32.
        n_vocab defaults to ld (the row stride).  static_scratch: call
        cbx_sample_batch_static (the redo list in the library's device array).
        decode: a Decode from decode_state(): one decode step
        (cbx_decode_step / cbx_head_decode_step), its history in place of
        history/history_len."""
        ld = logits.shape[-1]
        total_rows = logits.numel() // ld
        n_rows = total_rows // n_steps
        n_vocab = ld if n_vocab is None else n_vocab
        b = Batch()
        b.n_rows = n_rows
        b.n_vocab = n_vocab
        b.n_steps = n_steps
        b.stop_token = stop_token
        b.logits = logits.data_ptr()
        b.ld_logits = ld
        b.logits_uncond = None if logits_uncond is None else logits_uncond.data_ptr()
        b.params = params.data_ptr()
        b.history = None if history is None else history.data_ptr()
        b.history_len = None if history_len is None else history_len.data_ptr()
        b.ld_history = 0 if history is None else history.shape[-1]
        b.allowed = None if allowed is None else allowed.data_ptr()
        b.ld_allowed = 0 if allowed is None else allowed.shape[-1]
        b.force_stop = None if force_stop is None else force_stop.data_ptr()
        if draw_mode is None:
            draw_mode = CBX_DRAW_UNIFORM if uniforms is not None else CBX_DRAW_PHILOX
        b.draw_mode = draw_mode
        b.max_survivors = max_survivors
        b.uniforms = None if uniforms is None else uniforms.data_ptr()
        b.seed = seed
        b.stream_ids = None if stream_ids is None else stream_ids.data_ptr()
        b.step0 = step0
        b.tokens = tokens.data_ptr()
        b.info = None if info is None else info.data_ptr()
        b.probs = None if probs is None else probs.data_ptr()
        b.ld_probs = 0 if probs is None else probs.shape[-1]
        st = _stream_ptr() if stream is None else ctypes.c_void_p(stream)
        if decode is not None:
            if head is None:
                _check(self.lib.cbx_decode_step(self.handle, ctypes.byref(b), ctypes.byref(decode),
                                                st))
            else:
                _check(self.lib.cbx_head_decode_step(self.handle, ctypes.byref(head),
                                                     ctypes.byref(b), ctypes.byref(decode), st))
        elif head is None:
            fn = self.lib.cbx_sample_batch_static if static_scratch else self.lib.cbx_sample_batch
            _check(fn(self.handle, ctypes.byref(b), st))
        else:
            _check(self.lib.cbx_head_sample_batch(self.handle, ctypes.byref(head), ctypes.byref(b),
                                                  st))

    @staticmethod
    def decode_state(state, history, history_len, *, max_len=None, next_token=None):
        """A cbx_decode over device int32 tensors: state [n_rows], history
        [n_rows, ld_history], history_len [n_rows], optional max_len and
        next_token [n_rows]."""
        d = Decode()
        d.state = state.data_ptr()
        d.history = history.data_ptr()
        d.history_len = history_len.data_ptr()
        d.ld_history = history.shape[-1]
        d.max_len = None if max_len is None else max_len.data_ptr()
        d.next_token = None if next_token is None else next_token.data_ptr()
        d._tensors = (state, history, history_len, max_len, next_token)
        return d

    @staticmethod
    def t3_model(layers, wpe, speech_emb, ln_f_g, ln_f_b, *, wtype, n_head, eps=1e-5):
        """A cbx_t3_model over device tensors: layers a list of dicts with
        the cbx_t3_layer field names (matrices as uint8 bytes of the wtype
        layout, the rest float32), wpe [n_pos, n_embd], speech_emb
        [V, n_embd]."""
        arr = (T3Layer * len(layers))()
        for i, L in enumerate(layers):
            for f, _ in T3Layer._fields_:
                setattr(arr[i], f, L[f].data_ptr())
        m = T3Model()
        m.n_layer = len(layers)
        m.n_embd = wpe.shape[1]
        m.n_head = n_head
        m.n_pos = wpe.shape[0]
        m.n_speech_vocab = speech_emb.shape[0]
        m.wtype = wtype
        m.eps = eps
        m.wpe = wpe.data_ptr()
        m.speech_emb = speech_emb.data_ptr()
        m.layers = arr
        m.ln_f_g = ln_f_g.data_ptr()
        m.ln_f_b = ln_f_b.data_ptr()
        m._keep = (arr, layers, wpe, speech_emb, ln_f_g, ln_f_b)
        return m

    @staticmethod
    def _check_t3(fn, model, n_rows, n_slots, k_cache, v_cache, hidden, **rows):
        """The C ABI takes the caches and rows as raw addresses: a cache built
        for another layer or head count would be written past its end, so
        the tensors' shapes, dtypes and layout are checked here first."""
        import torch
        want = (n_slots, model.n_layer, model.n_head, k_cache.shape[-2] if k_cache.dim() else 0, 64)
        for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
            if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != want:
                raise ValueError("%s: %s must be contiguous float32 of shape %s, got %s %s%s" % (
                    fn, name, want, t.dtype, tuple(t.shape),
                    "" if t.is_contiguous() else " (not contiguous)"))
        if hidden.dtype != torch.float32 or not hidden.is_contiguous() or \
                tuple(hidden.shape) != (n_rows, model.n_embd):
            raise ValueError("%s: hidden must be contiguous float32 [%d, %d], got %s %s" % (
                fn, n_rows, model.n_embd, hidden.dtype, tuple(hidden.shape)))
        for name, (t, dt, shape) in rows.items():
            if t is None:
                continue
            if t.dtype != dt or not t.is_contiguous() or tuple(t.shape) != shape:
                raise ValueError("%s: %s must be contiguous %s of shape %s, got %s %s" % (
                    fn, name, dt, shape, t.dtype, tuple(t.shape)))

    def t3_step(self, model, positions, k_cache, v_cache, hidden, *, tokens=None, inputs=None,
                state=None, stream=None):
        """cbx_t3_step: one decode step of positions.numel() streams; caches
        [n_rows, n_layer, n_head, n_ctx, 64] float32, hidden [n_rows, n_embd]
        out; positions (int32) advance by one for the streams that step."""
        import torch
        n = positions.numel()
        self._check_t3("t3_step", model, n, n, k_cache, v_cache, hidden,
                       positions=(positions, torch.int32, (n,)),
                       tokens=(tokens, torch.int32, (n,)), state=(state, torch.int32, (n,)),
                       inputs=(inputs, torch.float32, (n, model.n_embd)))
        c = T3Cache()
        c.k = k_cache.data_ptr()
        c.v = v_cache.data_ptr()
        c.n_ctx = k_cache.shape[-2]
        st = _stream_ptr() if stream is None else ctypes.c_void_p(stream)
        _check(self.lib.cbx_t3_step(self.handle, ctypes.byref(model), positions.numel(),
                                    _ptr(tokens), _ptr(inputs), _ptr(positions), _ptr(state),
                                    ctypes.byref(c), _ptr(hidden), st))

    def t3_prefill(self, model, slots, positions, k_cache, v_cache, hidden, *, tokens=None,
                   inputs=None, stream=None):
        """cbx_t3_prefill: rows of (slot, position) in one call (device int32
        slots and positions [n_rows]); caches [n_slots, n_layer, n_head,
        n_ctx, 64]; positions are only read."""
        import torch
        n = slots.numel()
        self._check_t3("t3_prefill", model, n, k_cache.shape[0] if k_cache.dim() else 0, k_cache,
                       v_cache, hidden, slots=(slots, torch.int32, (n,)),
                       positions=(positions, torch.int32, (n,)),
                       tokens=(tokens, torch.int32, (n,)),
                       inputs=(inputs, torch.float32, (n, model.n_embd)))
        c = T3Cache()
        c.k = k_cache.data_ptr()
        c.v = v_cache.data_ptr()
        c.n_ctx = k_cache.shape[-2]
        st = _stream_ptr() if stream is None else ctypes.c_void_p(stream)
        _check(self.lib.cbx_t3_prefill(self.handle, ctypes.byref(model), slots.numel(),
                                       _ptr(slots), k_cache.shape[0], _ptr(tokens), _ptr(inputs),
                                       _ptr(positions), ctypes.byref(c), _ptr(hidden), st))

    def decode_step(self, logits, params, tokens, decode, **kw):
        """cbx_decode_step (head=...: cbx_head_decode_step) of one step."""
        self.sample_batch(logits, params, tokens, decode=decode, **kw)

    @staticmethod
    def head(weights, wtype, n_embd, hidden, logits, *, bias=None, hidden_uncond=None,
             logits_uncond=None):
        """A cbx_head over device tensors: weights (uint8 bytes of the wtype
        layout), hidden [rows, ld] float32, logits [rows, ld] float32 out."""
        h = Head()
        h.weights = weights.data_ptr()
        h.wtype = wtype
        h.n_embd = n_embd
        h.bias = None if bias is None else bias.data_ptr()
        h.hidden = hidden.data_ptr()
        h.hidden_uncond = None if hidden_uncond is None else hidden_uncond.data_ptr()
        h.ld_hidden = hidden.shape[-1]
        h.logits = logits.data_ptr()
        h.logits_uncond = None if logits_uncond is None else logits_uncond.data_ptr()
        # the structure holds raw addresses: keep the tensors alive with it
        h._tensors = (weights, bias, hidden, hidden_uncond, logits, logits_uncond)
        return h

    def head_logits(self, head, n_rows, n_vocab, ld_logits, stream=None):
        st = _stream_ptr() if stream is None else ctypes.c_void_p(stream)
        _check(self.lib.cbx_head_logits(self.handle, ctypes.byref(head), n_rows, n_vocab,
                                        ld_logits, st))

    def head_sample_batch(self, head, logits, params, tokens, **kw):
        """cbx_head_sample_batch: the projection into head.logits (whose
        shape gives the row stride), then sample_batch's sampling."""
        self.sample_batch(logits, params, tokens, head=head, **kw)
