"""Seeded cases for the exact running-sum scan: term lists (sorted and
shuffled exponentials, ties, near-equal, wide and tiny), thresholds, and the
plain left-to-right binary32 results they must reproduce."""
import numpy as np


def make_cases(n_cases, seed, max_n=2048, with_order=False):
    """with_order: also return, per case, whether its terms do not increase
    (the cases left sorted)."""
    rng = np.random.default_rng(seed)
    terms, offs, thr, exp_sum, exp_hit, desc = [], [0], [], [], [], []
    for c in range(n_cases):
        n = int(rng.integers(1, max_n + 1))
        mode = c % 7
        sig = 0.5 + 6 * rng.random()
        if mode == 0:
            s = rng.standard_normal(n) * sig
        elif mode == 1:
            s = np.floor(rng.standard_normal(n) * 4) / 4
        elif mode == 2:
            s = -rng.integers(0, 64, n) * 0.6931471805599453
        elif mode == 3:
            s = rng.standard_normal(n) * 0.01
        elif mode == 4:
            s = -rng.random(n) * 100
        elif mode == 5:
            s = -rng.integers(0, 8, n).astype(np.float64)
        else:
            s = rng.standard_normal(n) * 3
        s = np.sort(s.astype(np.float32))[::-1]
        t = np.exp((s - s[0]).astype(np.float32)).astype(np.float32)
        if c % 3 == 0:
            t = rng.permutation(t)
        desc.append(c % 3 != 0)
        if c % 5 == 4:
            # normalised terms: the top-p cumulative search
            total = np.add.accumulate(t, dtype=np.float32)[-1]
            t = (t / total).astype(np.float32)
            p = np.float32(0.05 + 0.95 * rng.random()) if c % 10 != 9 else np.float32(1.0)
        else:
            p = np.float32(0.0)
        acc = np.add.accumulate(t, dtype=np.float32)
        terms.append(t)
        offs.append(offs[-1] + n)
        thr.append(p)
        exp_sum.append(acc[-1])
        if p > 0:
            idx = np.nonzero(acc >= p)[0]
            exp_hit.append(int(idx[0]) if idx.size else -1)
        else:
            exp_hit.append(-1)
    out = (np.concatenate(terms).astype(np.float32), np.array(offs, np.int32),
           np.array(thr, np.float32), np.array(exp_sum, np.float32),
           np.array(exp_hit, np.int32))
    return out + (np.array(desc, np.uint8),) if with_order else out
