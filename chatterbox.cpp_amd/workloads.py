"""Synthetic inputs for the sampler's measured configurations.

Each builder returns host (numpy) arrays, seeded, so the GPU path and the CPU
oracle see identical bytes.  Vocabulary sizes follow the T3 models: 6563
speech ids with stop id 6562 for GPT-2-medium T3 Turbo
(scripts/convert-t3-turbo-to-gguf.py:19-21) and 8194 for the Llama-520M T3.
Knob defaults are chatterbox_sampling_params (chatterbox_t3_internal.h:113-118).
"""
from __future__ import annotations

import numpy as np

V_TURBO = 6563
STOP_TURBO = 6562
V_LLAMA = 8194
PARAM_FIELDS = ("top_k", "top_p", "temp", "repeat_penalty", "min_p", "cfg_weight")


def _spiked_normal(rng, rows, V, sigma, n_spikes, spike):
    x = (rng.standard_normal((rows, V)) * sigma).astype(np.float32)
    for r in range(rows):
        x[r, rng.choice(V, size=n_spikes, replace=False)] = spike
    return x


def single_stream(steps=500, min_p=0.05, seed=0x5EED1):
    """One stream, V=6563: logits ~N(0,3) plus 5 spikes at +12 per step, a fixed
    history of 256 ids uniform in [0, V); k=1000, p=0.95, T=0.8, pen=1.2."""
    rng = np.random.default_rng(seed)
    logits = _spiked_normal(rng, steps, V_TURBO, 3.0, 5, 12.0)
    history = rng.integers(0, V_TURBO, size=256).astype(np.int32)
    params = dict(top_k=1000, top_p=0.95, temp=0.8, repeat_penalty=1.2, min_p=min_p,
                  cfg_weight=0.0)
    return dict(logits=logits, history=history, params=params, V=V_TURBO)


def cfg_pair(steps=1000, seed=0x5EED2):
    """CFG pair, V=8194: cond ~N(0,3), uncond = cond + N(0,1), w=0.5; history
    grows with the sampled ids; pen 1.2, T 0.8, p 0.95, min_p 0.05, top-k off."""
    rng = np.random.default_rng(seed)
    cond = (rng.standard_normal((steps, V_LLAMA)) * 3.0).astype(np.float32)
    uncond = (cond + rng.standard_normal((steps, V_LLAMA))).astype(np.float32)
    params = dict(top_k=0, top_p=0.95, temp=0.8, repeat_penalty=1.2, min_p=0.05, cfg_weight=0.5)
    return dict(cond=cond, uncond=uncond, params=params, V=V_LLAMA)


def batched_streams(B=256, steps=1, seed=0x5EED3, hist_max=1000, V=V_TURBO):
    """B independent streams, V=6563 (or V): logits ~N(0,3) with 5 spikes per
    row at heights U[6,12]; history lengths U[0, hist_max]; per-row
    temperature U[0.5,1.2], top_k from {50, 250, 1000}; top_p 0.9, penalty
    1.2."""
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((steps * B, V)) * 3.0).astype(np.float32)
    for r in range(steps * B):
        idx = rng.choice(V, size=5, replace=False)
        logits[r, idx] = rng.uniform(6.0, 12.0, size=5).astype(np.float32)
    hist_len = rng.integers(0, hist_max + 1, size=B).astype(np.int32)
    history = rng.integers(0, V, size=(B, hist_max)).astype(np.int32)
    temps = rng.uniform(0.5, 1.2, size=B).astype(np.float32)
    ks = rng.choice(np.array([50, 250, 1000]), size=B)
    params = [dict(top_k=int(ks[r]), top_p=0.9, temp=float(temps[r]), repeat_penalty=1.2,
                   min_p=0.0, cfg_weight=0.0) for r in range(B)]
    return dict(logits=logits, history=history, hist_len=hist_len, params=params, V=V, B=B,
                steps=steps)


def masked_stress(B=1024, V=32768, seed=0x5EED5, stop_token=None):
    """B=1024, V=32768 logits ~N(0,4); per-row allowed bitmask with 20% of ids
    set (Bernoulli); forced stop on ~1/16 of rows; history 512 per stream;
    pen 1.3, k 50, p 0.9, min_p 0.02."""
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((B, V)) * 4.0).astype(np.float32)
    allowed_bits = rng.random((B, V)) < 0.2
    stop = V - 1 if stop_token is None else stop_token
    allowed_bits[:, stop] = True
    allowed = pack_bitmask(allowed_bits)
    force_stop = (rng.random(B) < 1.0 / 16).astype(np.uint8)
    history = rng.integers(0, V, size=(B, 512)).astype(np.int32)
    hist_len = np.full(B, 512, dtype=np.int32)
    params = [dict(top_k=50, top_p=0.9, temp=0.8, repeat_penalty=1.3, min_p=0.02,
                   cfg_weight=0.0)] * B
    return dict(logits=logits, allowed=allowed, allowed_bits=allowed_bits, force_stop=force_stop,
                history=history, hist_len=hist_len, params=params, V=V, B=B, stop=stop)


def pack_params(rows) -> np.ndarray:
    """cbx_params[n] as raw bytes (int32 top_k, then five float32)."""
    dt = np.dtype([("top_k", "<i4"), ("top_p", "<f4"), ("temp", "<f4"),
                   ("repeat_penalty", "<f4"), ("min_p", "<f4"), ("cfg_weight", "<f4")])
    arr = np.zeros(len(rows), dtype=dt)
    for i, r in enumerate(rows):
        for f in PARAM_FIELDS:
            arr[i][f] = r[f]
    return arr.view(np.uint8)


def pack_bitmask(bits: np.ndarray) -> np.ndarray:
    """bool [rows, V] -> uint32 [rows, ceil(V/32)] with id i at bit (i & 31) of
    word i >> 5."""
    rows, V = bits.shape
    words = (V + 31) // 32
    padded = np.zeros((rows, words * 32), dtype=bool)
    padded[:, :V] = bits
    return np.packbits(padded, axis=1, bitorder="little").view("<u4").reshape(rows, words).copy()
