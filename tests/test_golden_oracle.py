"""The committed golden cases (tests/golden/sampler_cases.npz) still come out of
the oracle bit for bit: guards the oracle against regressions."""
import os

import numpy as np

import oracle_lib as O

PATH = os.path.join(os.path.dirname(__file__), "golden", "sampler_cases.npz")


def test_oracle_reproduces_golden_cases():
    g = np.load(PATH)
    for r in range(g["logits"].shape[0]):
        pr = g["params"][r]
        p = O.OParams(int(pr[0]), *[float(v) for v in pr[1:]])
        tok, info, probs, _ = O.sample_row(g["logits"][r], g["history"][r, :g["hist_len"][r]], p,
                                           g["u"][r], allowed=g["allowed"][r], want_probs=True)
        assert tok == g["tokens"][r], r
        assert info == g["info"][r], r
        assert np.array_equal(probs.view(np.uint32), g["probs"][r].view(np.uint32)), r
