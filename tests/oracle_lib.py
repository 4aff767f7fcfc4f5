"""ctypes view of the CPU oracle (oracle/cbx_oracle.h).

Test infrastructure: the oracle is the checker.  Only tests, the smoke check
and bench.py's CPU-baseline leg load it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_SO = os.path.join(ORACLE_DIR, "_build", "libcbx_oracle.so")


class OParams(ctypes.Structure):
    _fields_ = [
        ("top_k", ctypes.c_int32),
        ("top_p", ctypes.c_float),
        ("temp", ctypes.c_float),
        ("repeat_penalty", ctypes.c_float),
        ("min_p", ctypes.c_float),
        ("cfg_weight", ctypes.c_float),
    ]


INFO_DREW = 0x01
INFO_GREEDY = 0x02
INFO_EMPTY = 0x04
INFO_TOPP_TIE = 0x08
INFO_NONFINITE = 0x10

_lib = None


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", ORACLE_DIR], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(ORACLE_SO):
        build_oracle()
    L = ctypes.CDLL(ORACLE_SO)
    vp, i32, i64, u32, u64, f64 = (ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64,
                                  ctypes.c_uint32, ctypes.c_uint64, ctypes.c_double)
    L.cbx_oracle_sample_row.restype = i32
    L.cbx_oracle_sample_row.argtypes = [vp, vp, i32, vp, i32, ctypes.POINTER(OParams), vp, i32, i32,
                                        f64, ctypes.POINTER(u32), vp, ctypes.POINTER(i32)]
    L.cbx_oracle_run_mt19937.restype = None
    L.cbx_oracle_run_mt19937.argtypes = [vp, i32, i32, vp, i32, i32, ctypes.POINTER(OParams), u32,
                                         vp, vp]
    L.cbx_oracle_mt_canonical.restype = None
    L.cbx_oracle_mt_canonical.argtypes = [u32, u64, i32, vp]
    L.cbx_oracle_mt_10000th.restype = u32
    L.cbx_oracle_mt_10000th.argtypes = []
    L.cbx_oracle_philox4x32_10.restype = None
    L.cbx_oracle_philox4x32_10.argtypes = [vp, vp, vp]
    L.cbx_oracle_philox_uniform.restype = f64
    L.cbx_oracle_philox_uniform.argtypes = [u64, u64, u64]
    L.cbx_oracle_sample_batch.restype = f64
    L.cbx_oracle_sample_batch.argtypes = [vp, vp, i64, i32, i32, vp, i64, vp, vp, vp, i64, vp, i32,
                                          vp, i32, vp, vp]
    L.cbx_oracle_dequant_row.restype = None
    L.cbx_oracle_dequant_row.argtypes = [vp, i32, i32, vp]
    L.cbx_oracle_quantize.restype = None
    L.cbx_oracle_quantize.argtypes = [vp, i32, i32, i32, vp]
    L.cbx_oracle_head_f64.restype = None
    L.cbx_oracle_head_f64.argtypes = [vp, i32, vp, vp, i32, i32, i32, vp]
    L.cbx_oracle_expf.restype = None
    L.cbx_oracle_expf.argtypes = [vp, vp, i64]
    L.cbx_oracle_expf_mismatch.restype = i64
    L.cbx_oracle_expf_mismatch.argtypes = [u32, i64, vp, i32]
    _lib = L
    return L


def params(top_k=1000, top_p=0.95, temp=0.8, repeat_penalty=1.2, min_p=0.0, cfg_weight=0.0):
    return OParams(top_k, top_p, temp, repeat_penalty, min_p, cfg_weight)


def _p(a):
    return None if a is None else a.ctypes.data


def sample_row(logits, history=(), p=None, u=0.5, uncond=None, allowed=None, force_stop=False,
               stop_token=0, want_probs=False):
    """One row through the oracle.  Returns (token, info[, probs, kept])."""
    L = lib()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    hist = np.ascontiguousarray(history, dtype=np.int32)
    unc = None if uncond is None else np.ascontiguousarray(uncond, dtype=np.float32)
    al = None if allowed is None else np.ascontiguousarray(allowed, dtype=np.uint32)
    p = params() if p is None else p
    info = ctypes.c_uint32()
    kept = ctypes.c_int32()
    probs = np.zeros(lg.size, dtype=np.float32) if want_probs else None
    tok = L.cbx_oracle_sample_row(_p(lg), _p(unc), lg.size, _p(hist) if hist.size else None,
                                  hist.size, ctypes.byref(p), _p(al), 1 if force_stop else 0,
                                  stop_token, float(u), ctypes.byref(info), _p(probs),
                                  ctypes.byref(kept))
    if want_probs:
        return tok, info.value, probs, kept.value
    return tok, info.value


def sample_batch(logits, p_list, u, history=None, hist_len=None, uncond=None, allowed=None,
                 force_stop=None, stop_token=0, n_threads=1):
    """Rows of a 2-D logits array; returns (tokens, infos, seconds)."""
    L = lib()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    n_rows, ld = lg.shape
    parr = (OParams * n_rows)(*p_list)
    uu = np.ascontiguousarray(u, dtype=np.float64)
    toks = np.zeros(n_rows, dtype=np.int32)
    infos = np.zeros(n_rows, dtype=np.uint32)
    hist = None if history is None else np.ascontiguousarray(history, dtype=np.int32)
    hl = None if hist_len is None else np.ascontiguousarray(hist_len, dtype=np.int32)
    unc = None if uncond is None else np.ascontiguousarray(uncond, dtype=np.float32)
    al = None if allowed is None else np.ascontiguousarray(allowed, dtype=np.uint32)
    fs = None if force_stop is None else np.ascontiguousarray(force_stop, dtype=np.uint8)
    secs = L.cbx_oracle_sample_batch(
        _p(lg), _p(unc), ld, n_rows, ld, _p(hist), 0 if hist is None else hist.shape[1], _p(hl),
        parr, _p(al), 0 if al is None else al.shape[1], _p(fs), stop_token, _p(uu), n_threads,
        _p(toks), _p(infos))
    return toks, infos, secs


def run_mt19937(logits_steps, history, p, seed, grow_history=True):
    L = lib()
    lg = np.ascontiguousarray(logits_steps, dtype=np.float32)
    n_steps, V = lg.shape
    hist = np.ascontiguousarray(history, dtype=np.int32)
    toks = np.zeros(n_steps, dtype=np.int32)
    us = np.zeros(n_steps, dtype=np.float64)
    L.cbx_oracle_run_mt19937(_p(lg), n_steps, V, _p(hist) if hist.size else None, hist.size,
                             1 if grow_history else 0, ctypes.byref(p), seed, _p(toks), _p(us))
    return toks, us


def mt_canonical(seed, n, discard=0):
    out = np.zeros(n, dtype=np.float64)
    lib().cbx_oracle_mt_canonical(seed, discard, n, out.ctypes.data)
    return out


def philox(ctr, key):
    c = np.ascontiguousarray(ctr, dtype=np.uint32)
    k = np.ascontiguousarray(key, dtype=np.uint32)
    o = np.zeros(4, dtype=np.uint32)
    lib().cbx_oracle_philox4x32_10(c.ctypes.data, k.ctypes.data, o.ctypes.data)
    return o


def philox_uniform(seed, stream, step):
    return lib().cbx_oracle_philox_uniform(seed, stream, step)


def libm_expf(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().cbx_oracle_expf(x.ctypes.data, out.ctypes.data, x.size)
    return out


def cdf_draw(probs, u):
    p = np.ascontiguousarray(probs, dtype=np.float32)
    L = lib()
    L.cbx_oracle_cdf_draw.restype = ctypes.c_int32
    L.cbx_oracle_cdf_draw.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_double]
    return L.cbx_oracle_cdf_draw(p.ctypes.data, p.size, float(u))


def stdlib_draw(probs, x0, x1):
    p = np.ascontiguousarray(probs, dtype=np.float32)
    L = lib()
    L.cbx_oracle_stdlib_draw.restype = ctypes.c_int32
    L.cbx_oracle_stdlib_draw.argtypes = [ctypes.c_void_p, ctypes.c_int32, ctypes.c_uint32,
                                         ctypes.c_uint32]
    return L.cbx_oracle_stdlib_draw(p.ctypes.data, p.size, x0, x1)


# ---- speech_head formats (oracle/cbx_oracle.cpp) ----
WTYPE_F16, WTYPE_Q4_0, WTYPE_Q5_0, WTYPE_Q8_0 = 1, 2, 6, 8
BLOCK_BYTES = {WTYPE_Q4_0: 18, WTYPE_Q5_0: 22, WTYPE_Q8_0: 34}


def quantize(w, wtype):
    """fp32 [rows, n_embd] -> uint8 [rows, n_embd/32 * block bytes] (ggml rules);
    F16 rows are the IEEE binary16 bytes."""
    w = np.ascontiguousarray(w, np.float32)
    rows, n = w.shape
    if wtype == WTYPE_F16:
        return w.astype(np.float16).view(np.uint8).reshape(rows, n * 2).copy()
    out = np.zeros((rows, n // 32 * BLOCK_BYTES[wtype]), np.uint8)
    lib().cbx_oracle_quantize(w.ctypes.data, rows, n, wtype, out.ctypes.data)
    return out


def dequantize(blocks, wtype, n_embd):
    """uint8 [rows, bytes] -> fp32 [rows, n_embd], the values the format defines."""
    blocks = np.ascontiguousarray(blocks, np.uint8)
    rows = blocks.shape[0]
    if wtype == WTYPE_F16:
        return blocks.view(np.float16).reshape(rows, n_embd).astype(np.float32)
    out = np.zeros((rows, n_embd), np.float32)
    for r in range(rows):
        lib().cbx_oracle_dequant_row(blocks[r].ctypes.data, wtype, n_embd,
                                     out[r].ctypes.data)
    return out


def head_f64(blocks, wtype, bias, hidden, n_vocab, n_embd):
    """logits [rows, n_vocab] in binary64: sum_k deq(W[v][k]) h[r][k] + b[v]
    (F16 rows through dequantize and a binary64 product)."""
    hidden = np.ascontiguousarray(hidden, np.float32)
    if wtype == WTYPE_F16:
        wd = dequantize(blocks, wtype, n_embd).astype(np.float64)
        out = hidden.astype(np.float64) @ wd.T
        return out + (0.0 if bias is None else bias.astype(np.float64))
    rows = hidden.shape[0]
    out = np.zeros((rows, n_vocab), np.float64)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib().cbx_oracle_head_f64(np.ascontiguousarray(blocks).ctypes.data, wtype,
                              None if b is None else b.ctypes.data, hidden.ctypes.data, rows,
                              n_vocab, n_embd, out.ctypes.data)
    return out
