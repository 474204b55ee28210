"""Shared parity bars for the sampling path (GPU tests and the CPU emulation
of the kernels compare against the CPU oracle with the same rules).

Bars:
* rows finished by the exact path (<= 1024 candidates after truncation and
  min-p; every top-k row): token, kept count and pick probability bit-exact;
* rows with more candidates (no top-k nucleus): the device sums probabilities
  in f64, the reference sequentially in f32.  Against the reference, tokens
  must match except where u lies within TOL_U of a CDF boundary or top-p's
  cumulative lies within TOL_P of p (counted and reported); probabilities
  within 1e-5 relative / 1e-6 absolute of the exact-arithmetic value.
  Against exact arithmetic throughout (the oracle's f64 view: top-p by f64
  partial sums, the draw over that kept mass), the kept count must match
  unless top_p lies within TOL_EXACT (2e-6, relative) of a cumulative, and
  with the same kept count the token must match unless u * mass lies within
  TOL_EXACT of a boundary;
* logprobs and top-n logprobs within 1e-5 relative / 1e-6 absolute, top-n
  ids bit-exact.
"""
from __future__ import annotations

import numpy as np

from tachyon_amd import workloads as wl

TOL_U = 1e-5
TOL_P = 1e-5
# the device's own arithmetic on rows with more candidates: f64 sums, with the
# mass before the resolved bin from hardware exp2 terms (each within 3e-6)
TOL_EXACT = 2e-6
EXACT_CAP = 1024
REL, ABS = 1e-5, 1e-6


def close(a, b, rel=REL, abs_=ABS):
    return abs(float(a) - float(b)) <= abs_ + rel * abs(float(b))


def check(w, got, ref, label):
    """Asserts the bars row by row; returns (n_exact_rows, n_boundary_exempt,
    n_exact_arithmetic_picks): rows on the exact path, rows whose token differs
    from the reference's inside a boundary exemption, and rows with more
    candidates whose pick was checked against exact arithmetic throughout."""
    from oracle import pyoracle

    exempt = 0
    exact_rows = 0
    exact_picks = 0
    for r in range(w.rows):
        d = ref.diag[r]
        p = w.params[r]
        tag = f"{label} row {r} params={p} diag={d}"
        exact = d["path"] in (pyoracle.PATH_ARGMAX_FAST, pyoracle.PATH_NONE_ALLOWED) or d["survivors"] <= EXACT_CAP
        if exact:
            exact_rows += 1
            assert got["token"][r] == ref.token[r], tag + f" got={got['token'][r]} ref={ref.token[r]}"
            assert got["keep"][r] == ref.keep[r], tag + f" got keep={got['keep'][r]}"
            assert got["prob"][r].tobytes() == ref.prob[r].tobytes(), tag + f" prob {got['prob'][r]} {ref.prob[r]}"
            same_token = True
        else:
            boundary = d["u_gap"] < TOL_U or d["p_gap"] < TOL_P
            same_token = got["token"][r] == ref.token[r]
            if not same_token:
                assert boundary, tag + f" got={got['token'][r]} ref={ref.token[r]}"
                exempt += 1
            if got["keep"][r] != ref.keep[r]:
                assert d["p_gap"] < TOL_P or got["keep"][r] == d["keep_exact"], tag + f" keep {got['keep'][r]}"
            # against exact arithmetic throughout, which is what the device
            # computes: the kept count, then the pick over that kept mass,
            # except where the target lies within TOL_EXACT of a boundary
            if d["pgap_exact"] >= TOL_EXACT:
                assert got["keep"][r] == d["keep_exact"], tag + f" keep {got['keep'][r]} exact {d['keep_exact']}"
            if got["keep"][r] == d["keep_exact"] and d["consumed_u"] and d["ugap_exact"] >= TOL_EXACT:
                assert got["token"][r] == d["token_exact"], tag + f" got={got['token'][r]} exact={d['token_exact']}"
                exact_picks += 1
            if same_token and got["keep"][r] == ref.keep[r]:
                # against the exact-arithmetic probability p_pick / sum(p)
                p_exact = float(ref.prob[r]) * float(d["mass"]) / float(d["mass64"])
                assert close(got["prob"][r], p_exact), tag + f" prob {got['prob'][r]} vs {p_exact}"
        if (p["flags"] & wl.ROW_LOGPROBS) and same_token:
            assert close(got["logprob"][r], ref.logprob[r]), tag + f" lp {got['logprob'][r]} {ref.logprob[r]}"
            n = min(int(p["n_logprobs"]), w.usable, w.top_stride)
            assert got["top_ids"][r, :n].tolist() == ref.top_ids[r, :n].tolist(), tag
            for j in range(n):
                assert close(got["top_lp"][r, j], ref.top_lp[r, j]), tag + f" top lp {j}"
    return exact_rows, exempt, exact_picks


def check_mask_property(w, got):
    """Size-independent property: every pick of a constrained row with a
    non-empty kept set is an allowed id."""
    if w.mask is None:
        return
    for r in range(w.rows):
        if not (w.params["flags"][r] & wl.ROW_CONSTRAINED) or got["keep"][r] == 0:
            continue
        t = int(got["token"][r])
        assert (w.mask[r, t >> 5] >> (t & 31)) & 1, (r, t)


def check_distribution(w, ids, ps, keep, rids, rps, rkeep, label):
    for r in range(w.rows):
        assert keep[r] == rkeep[r], (label, r, keep[r], rkeep[r])
        k = min(int(keep[r]), ids.shape[1])
        assert ids[r, :k].tolist() == rids[r, :k].tolist(), (label, r)
        assert np.array_equal(ps[r, :k], rps[r, :k]), (label, r)


RANDOM_CASES = [
    dict(seed=1, vocab=300),
    dict(seed=2, vocab=300, ties=True),
    dict(seed=3, vocab=300, masked=True),
    dict(seed=4, vocab=300, masked=True, ties=True, mask_frac=0.05),
    dict(seed=5, vocab=1500, masked=True, mask_frac=0.02, rows=12),
    dict(seed=6, vocab=2100, rows=12, mode="nucleus"),
    dict(seed=7, vocab=2100, rows=12, mode="minp", ties=True),
    dict(seed=8, vocab=64, rows=12, stride=80, masked=True, ties=True),
    dict(seed=9, vocab=1200, rows=12, mode="topp", sigma=8.0),
    dict(seed=10, vocab=5, rows=12, masked=True, mask_frac=0.6),
    dict(seed=11, vocab=40000, rows=24, masked=True, mask_frac=0.01),
    dict(seed=12, vocab=40000, rows=24, ties=True, hist_len=300),
    dict(seed=13, vocab=20001, rows=18, stride=20003, masked=True),
    dict(seed=14, vocab=70000, rows=12, mode="nucleus", sigma=1.0),
    dict(seed=15, vocab=70000, rows=12, mode="all", masked=True, mask_frac=0.002),
    # nucleus sets of thousands: equal values beyond one bin's capacity, and a
    # narrow cluster beside a far outlier (value bins split a second time)
    dict(seed=16, vocab=15000, rows=6, mode="nucleus", ties=True),
    dict(seed=17, vocab=15000, rows=6, mode="nucleus", sigma=0.01, outlier=-1.0e4),
    dict(seed=18, vocab=60000, rows=12, mode="nucleus", sigma=0.003, outlier=-50.0, masked=True, mask_frac=0.5),
]

DIST_CASES = [(21, dict(vocab=500, mode="mixed")), (22, dict(vocab=3000, mode="minp")),
              (23, dict(vocab=3000, mode="topk", ties=True))]
