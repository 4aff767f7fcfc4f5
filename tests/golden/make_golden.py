"""Writes tests/golden/sampler_cases.npz: small sampler cases (inputs and the
oracle's outputs) covering every stage and knob combination.

The reference keeps no sampler vectors, so these are produced by the oracle
(oracle/cbx_oracle.cpp), after its own pins pass (tests/test_oracle_pins.py,
tests/test_native_pins.py).  They freeze the expected outputs so that the GPU
path and any later change to the oracle are checked against the same bytes.
Run from the repository root:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(HERE))
import oracle_lib as O  # noqa: E402

V = 300
N = 48
HL = 40


def main():
    rng = np.random.default_rng(20261201)
    logits = np.zeros((N, V), np.float32)
    params = np.zeros((N, 6), np.float64)
    u = np.zeros(N)
    history = rng.integers(-3, V + 3, size=(N, HL)).astype(np.int32)
    hist_len = rng.integers(0, HL + 1, size=N).astype(np.int32)
    allowed = np.full((N, (V + 31) // 32), 0xFFFFFFFF, np.uint32)
    for r in range(N):
        kind = r % 8
        x = (rng.standard_normal(V) * rng.uniform(0.5, 5)).astype(np.float32)
        if kind == 1:
            x[rng.choice(V, 5, replace=False)] = 12.0
        if kind == 2:
            x = np.round(x).astype(np.float32)          # many exact ties
        if kind == 3:
            bits = rng.random(V) < 0.3
            words = np.zeros((V + 31) // 32 * 32, bool)
            words[:V] = bits
            allowed[r] = np.packbits(words, bitorder="little").view("<u4")
        if kind == 4:
            x[:] = -np.inf
            x[rng.choice(V, 3, replace=False)] = rng.standard_normal(3)
        logits[r] = x
        params[r] = [rng.choice([0, 1, 7, 50, 299, 300, 1000]),
                     rng.choice([1.0, 0.95, 0.5, 0.0]),
                     rng.choice([0.8, 1.0, 0.0, 0.5, 1.7]),
                     rng.choice([1.0, 1.2, 0.7]),
                     rng.choice([0.0, 0.05]),
                     0.0]
        u[r] = rng.choice([rng.random(), 0.0, np.nextafter(1.0, 0.0)], p=[0.8, 0.1, 0.1])
    tokens = np.zeros(N, np.int32)
    info = np.zeros(N, np.uint32)
    probs = np.zeros((N, V), np.float32)
    for r in range(N):
        p = O.OParams(int(params[r, 0]), *[float(v) for v in params[r, 1:]])
        t, i, pr, _ = O.sample_row(logits[r], history[r, :hist_len[r]], p, u[r],
                                   allowed=allowed[r], want_probs=True)
        tokens[r], info[r], probs[r] = t, i, pr
    np.savez_compressed(os.path.join(HERE, "sampler_cases.npz"), logits=logits, params=params,
                        u=u, history=history, hist_len=hist_len, allowed=allowed, tokens=tokens,
                        info=info, probs=probs)
    print("wrote", N, "cases; tokens", tokens.tolist())


if __name__ == "__main__":
    main()
