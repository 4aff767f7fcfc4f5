"""Token / probability comparison between the GPU path and the oracle.

Bar (per row): the token ids are equal.  The only tolerated differences are
counted and reported, never silently passed:
  * filter-boundary ties: equal scores straddle the top-p cutoff
    (CBX_INFO_TOPP_TIE), so the kept id depends on std::sort's tie order;
  * draw-boundary ties: the uniform lies within 1e-6 of a cumulative
    probability boundary of the oracle's CDF.
Probabilities must be bitwise equal on rows without a filter tie (stronger
than the 1e-5 relative bar).
"""
from __future__ import annotations

import numpy as np

INFO_DREW, INFO_GREEDY, INFO_EMPTY, INFO_TOPP_TIE, INFO_NONFINITE, INFO_OVERFLOW = (
    0x01, 0x02, 0x04, 0x08, 0x10, 0x20)
DRAW_TIE_EPS = 1e-6


def _near_cdf_boundary(probs_row, u):
    w = probs_row.astype(np.float64)
    s = w.sum()
    if s <= 0:
        return False
    cdf = np.cumsum(w / s)
    return bool(np.min(np.abs(cdf - u)) < DRAW_TIE_EPS)


class Report:
    def __init__(self, name):
        self.name = name
        self.rows = 0
        self.exact = 0
        self.filter_ties = 0
        self.draw_ties = 0
        self.prob_rows_checked = 0

    def __str__(self):
        return (f"[parity {self.name}] rows={self.rows} exact={self.exact} "
                f"filter_boundary_ties={self.filter_ties} draw_boundary_ties={self.draw_ties} "
                f"prob_rows_bitwise={self.prob_rows_checked}")


def compare(name, tok_gpu, info_gpu, tok_ref, info_ref, u=None, probs_gpu=None, probs_ref=None):
    tok_gpu = np.asarray(tok_gpu).reshape(-1)
    tok_ref = np.asarray(tok_ref).reshape(-1)
    info_gpu = np.asarray(info_gpu).reshape(-1).astype(np.uint32)
    info_ref = np.asarray(info_ref).reshape(-1).astype(np.uint32)
    rep = Report(name)
    rep.rows = tok_ref.size
    assert tok_gpu.shape == tok_ref.shape
    assert not np.any(info_gpu & INFO_OVERFLOW), "GPU rows overflowed the on-chip capacity"
    # outcome class must agree (drew / greedy / empty)
    mask = INFO_DREW | INFO_GREEDY | INFO_EMPTY
    bad_cls = np.nonzero((info_gpu & mask) != (info_ref & mask))[0]
    assert bad_cls.size == 0, f"{name}: outcome flags differ at rows {bad_cls[:10]}"
    tie_gpu = (info_gpu & INFO_TOPP_TIE) != 0
    tie_ref = (info_ref & INFO_TOPP_TIE) != 0
    diff = np.nonzero(tok_gpu != tok_ref)[0]
    hard = []
    for r in diff:
        if tie_ref[r] or tie_gpu[r]:
            rep.filter_ties += 1
        elif u is not None and probs_ref is not None and _near_cdf_boundary(probs_ref[r], u[r]):
            rep.draw_ties += 1
        else:
            hard.append(int(r))
    rep.exact = rep.rows - diff.size
    assert not hard, (f"{name}: {len(hard)} token mismatches outside boundary ties, rows "
                      f"{hard[:10]}: gpu {tok_gpu[hard[:10]]} ref {tok_ref[hard[:10]]}")
    if probs_gpu is not None and probs_ref is not None:
        ok_rows = np.nonzero(~(tie_ref | tie_gpu))[0]
        pg = np.asarray(probs_gpu)[ok_rows]
        pr = np.asarray(probs_ref)[ok_rows]
        neq = np.nonzero(np.any(pg.view(np.uint32) != pr.view(np.uint32), axis=1))[0]
        if neq.size:
            r = int(ok_rows[neq[0]])
            j = np.nonzero(np.asarray(probs_gpu)[r] != np.asarray(probs_ref)[r])[0][:5]
            raise AssertionError(f"{name}: probabilities differ bitwise on {neq.size} rows; "
                                 f"row {r} ids {j}: gpu {np.asarray(probs_gpu)[r][j]} "
                                 f"ref {np.asarray(probs_ref)[r][j]}")
        rep.prob_rows_checked = ok_rows.size
    print(rep, flush=True)
    return rep
