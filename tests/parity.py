"""Token / probability comparison between the GPU path and the oracle.

Bar (per row): the token ids are equal, the outcome flags (drew / greedy /
empty, and the top-p tie flag) agree, and the post-filter probabilities are
bitwise equal (stronger than the 1e-5 relative bar).  Rows whose top-p cutoff
falls inside a run of equal scores are held to the same bar: the GPU replays
the reference's std::sort order for them.

The one tolerated class is a draw within 1e-6 of a cumulative-probability
boundary of the oracle's CDF; such rows are counted, and a test fails when
there are more of them than it expects (0 unless it says otherwise).
"""
from __future__ import annotations

import numpy as np

INFO_DREW, INFO_GREEDY, INFO_EMPTY, INFO_TOPP_TIE, INFO_NONFINITE, INFO_OVERFLOW = (
    0x01, 0x02, 0x04, 0x08, 0x10, 0x20)
INFO_TOPP_SORTED = 0x80  # diagnostic of the one-wave kernel (not compared with the oracle)
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
        self.tie_rows = 0        # rows whose top-p cutoff falls inside equal scores
        self.draw_ties = 0       # token mismatches within 1e-6 of a CDF boundary
        self.prob_rows_checked = 0

    def counts(self):
        return (f"rows={self.rows} exact={self.exact} topp_tie_rows={self.tie_rows} "
                f"draw_boundary_ties={self.draw_ties} prob_rows_bitwise={self.prob_rows_checked}")

    def __str__(self):
        return f"[parity {self.name}] {self.counts()}"


def compare(name, tok_gpu, info_gpu, tok_ref, info_ref, u=None, probs_gpu=None, probs_ref=None,
            max_draw_ties=0):
    tok_gpu = np.asarray(tok_gpu).reshape(-1)
    tok_ref = np.asarray(tok_ref).reshape(-1)
    info_gpu = np.asarray(info_gpu).reshape(-1).astype(np.uint32)
    info_ref = np.asarray(info_ref).reshape(-1).astype(np.uint32)
    rep = Report(name)
    rep.rows = tok_ref.size
    assert tok_gpu.shape == tok_ref.shape
    over = np.nonzero(info_gpu & INFO_OVERFLOW)[0]
    assert over.size == 0, f"{name}: GPU rows {over[:10]} overflowed the on-chip capacity"
    # outcome class and the top-p tie flag must agree
    mask = INFO_DREW | INFO_GREEDY | INFO_EMPTY | INFO_TOPP_TIE
    bad_cls = np.nonzero((info_gpu & mask) != (info_ref & mask))[0]
    assert bad_cls.size == 0, (f"{name}: flags differ at rows {bad_cls[:10]}: gpu "
                               f"{info_gpu[bad_cls[:10]]} ref {info_ref[bad_cls[:10]]}")
    rep.tie_rows = int(np.count_nonzero(info_ref & INFO_TOPP_TIE))
    diff = np.nonzero(tok_gpu != tok_ref)[0]
    hard = []
    for r in diff:
        if u is not None and probs_ref is not None and _near_cdf_boundary(probs_ref[r], u[r]):
            rep.draw_ties += 1
        else:
            hard.append(int(r))
    rep.exact = rep.rows - diff.size
    assert not hard, (f"{name}: {len(hard)} token mismatches outside draw-boundary ties, rows "
                      f"{hard[:10]}: gpu {tok_gpu[hard[:10]]} ref {tok_ref[hard[:10]]}; "
                      f"{rep.counts()}")
    assert rep.draw_ties <= max_draw_ties, (f"{name}: {rep.draw_ties} draw-boundary ties, "
                                            f"{max_draw_ties} expected; {rep.counts()}")
    if probs_gpu is not None and probs_ref is not None:
        pg = np.asarray(probs_gpu)
        pr = np.asarray(probs_ref)
        neq = np.nonzero(np.any(pg.view(np.uint32) != pr.view(np.uint32), axis=1))[0]
        if neq.size:
            r = int(neq[0])
            j = np.nonzero(pg[r] != pr[r])[0][:5]
            raise AssertionError(f"{name}: probabilities differ bitwise on {neq.size} rows; "
                                 f"row {r} ids {j}: gpu {pg[r][j]} ref {pr[r][j]}; "
                                 f"{rep.counts()}")
        rep.prob_rows_checked = pg.shape[0]
    print(rep, flush=True)
    return rep
