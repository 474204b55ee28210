"""Shared parity bars for the sampling path (GPU tests and the CPU emulation
of the kernels compare against the CPU oracle with the same rules).

Bars:
* every row: token, kept count and pick probability bit-exact with the
  reference's arithmetic (the oracle).  A row whose token or kept count
  differs passes only when the reference itself returns that pair after u
  moves by at most TOL_U and top_p by at most TOL_P: the shifts are measured
  with the reference's own f32 arithmetic (oracle or_reconcile), never
  assumed;
* logprobs and top-n logprobs within 1e-5 relative / 1e-6 absolute, top-n
  ids bit-exact.
"""
from __future__ import annotations

import numpy as np

from tachyon_amd import workloads as wl

TOL_U = 1e-5
TOL_P = 1e-5
REL, ABS = 1e-5, 1e-6


def close(a, b, rel=REL, abs_=ABS):
    """Within the logprob tolerance; NaN matches NaN only (a row holding a
    NaN logit has a NaN logsumexp)."""
    a, b = float(a), float(b)
    if b != b or a != a:
        return a != a and b != b
    return abs(a - b) <= abs_ + rel * abs(b)


def same_f32(a, b):
    """Bit-exact, except that any NaN matches any NaN (the payload of a NaN
    result is not the reference's arithmetic)."""
    if a != a or b != b:
        return a != a and b != b
    return np.float32(a).tobytes() == np.float32(b).tobytes()


def boundary_shift(w, r, token, keep):
    """(du, dp) the reference needs to return (token, keep) on row r, or None
    when no move of u and top_p does."""
    from oracle import pyoracle

    return pyoracle.reconcile(w, r, token, keep)


def check(w, got, ref, label):
    """Asserts the bars row by row; returns (n_rows_bit_exact, n_boundary):
    rows equal to the reference, and rows that differ within the measured
    boundary tolerance."""
    exact_rows = 0
    boundary = 0
    for r in range(w.rows):
        d = ref.diag[r]
        p = w.params[r]
        tag = f"{label} row {r} params={p} diag={d}"
        same_token = got["token"][r] == ref.token[r]
        if same_token and got["keep"][r] == ref.keep[r]:
            exact_rows += 1
            assert same_f32(got["prob"][r], ref.prob[r]), tag + f" prob {got['prob'][r]} {ref.prob[r]}"
        else:
            shift = boundary_shift(w, r, got["token"][r], got["keep"][r])
            assert shift is not None and shift[0] <= TOL_U and shift[1] <= TOL_P, (
                tag + f" got={got['token'][r]} keep={got['keep'][r]} ref={ref.token[r]} keep={ref.keep[r]}"
                f" shift(du, dp)={shift}")
            boundary += 1
        if (p["flags"] & wl.ROW_LOGPROBS) and same_token:
            assert close(got["logprob"][r], ref.logprob[r]), tag + f" lp {got['logprob'][r]} {ref.logprob[r]}"
            n = min(int(p["n_logprobs"]), w.usable, w.top_stride)
            assert got["top_ids"][r, :n].tolist() == ref.top_ids[r, :n].tolist(), tag
            for j in range(n):
                assert close(got["top_lp"][r, j], ref.top_lp[r, j]), tag + f" top lp {j}"
    return exact_rows, boundary


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
    # NaN, +inf and -inf logits (a NaN at id 0, NaNs at random ids, +inf
    # spikes, rows 70% -inf, rows all -inf), on the split-row kernel (12 rows)
    # and the whole-row kernel (20 rows)
    dict(seed=19, vocab=300, rows=12, specials=True),
    dict(seed=20, vocab=3000, rows=20, specials=True, masked=True),
    dict(seed=24, vocab=3000, rows=12, specials=True, mode="topk", masked=True, mask_frac=0.02),
    dict(seed=25, vocab=5000, rows=20, specials=True, mode="nucleus"),
    # rows with NaNs at 3-5% of their ids, where partition_point's probe
    # order decides which ids top_n keeps (the split-row kernel: 12 rows;
    # the whole-row kernel: 20 rows)
    dict(seed=30, vocab=2000, rows=12, nan_frac=0.05, mode="topk"),
    dict(seed=31, vocab=3000, rows=20, nan_frac=0.03, mode="topk", masked=True),
    # histories longer than the LDS history table (2048 ids): penalties
    # applied on re-reads
    dict(seed=26, vocab=3000, rows=20, hist_len=4000),
    # penalties over a vocabulary beyond the history bitmap (262144 ids)
    dict(seed=27, vocab=300000, rows=20, hist_len=64),
    # nucleus rows of ~150k candidates under one dominant value (top-p decided
    # at the first candidate: value bins past the decision stay coarse)
    dict(seed=29, vocab=151936, rows=6, mode="nucleus", sigma=3.0, outlier=18.0),
]

DIST_CASES = [(21, dict(vocab=500, mode="mixed")), (22, dict(vocab=3000, mode="minp")),
              (23, dict(vocab=3000, mode="topk", ties=True)),
              # kept sets beyond the 1024 written entries (DIST_TRUNCATED)
              (28, dict(vocab=6000, mode="nucleus", sigma=0.5))]

# Top-k windows near 1024 over vocabularies a few segments long: with fewer
# finite group maxima than the window needs, every element of a split-row
# segment passes its threshold (more than a segment's candidate area holds)
WINDOW_CASES = [dict(seed=40, vocab=4000), dict(seed=41, vocab=8192, hist_len=8),
                dict(seed=42, vocab=6000, rows=4, hist_len=400, masked=True),
                dict(seed=43, vocab=12000, rows=3, top_k=1000, hist_len=500, repetition_penalty=0.9)]


def dense_cluster_workloads():
    """Nucleus rows (no top-k, T 2-3) whose first third of the vocabulary is
    a dense cluster narrower than one value bin: two rows of the seeded sweep
    (batches 193 and 272) that once ended with INTERNAL (a fine bin beyond a
    census round), and eight synthetic rows of the same kind with other
    top-p and temperatures.  Returns [(label, workload)]."""
    out = []
    for b, r in [(193, 7), (272, 18)]:
        w, _ = wl.sweep_batch(0x5EE0 + b)
        ids = w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]]
        out.append((f"sweep{b} row {r}",
                    wl.Workload(f"sweep{b}r{r}", w.logits[r:r + 1].copy(), w.usable, w.params[r:r + 1].copy(),
                                ids.copy(), np.array([0, len(ids)], np.uint32), None,
                                w.uniforms[r:r + 1].copy(), w.top_stride)))
    w = wl.cluster_case(seed=60, vocab=151936, rows=8)
    w.params["temperature"] = np.array([3, 3, 3, 2, 3, 3, 2.5, 3], np.float32)
    w.params["top_p"] = np.array([1.0, 0.9, 0.99, 1.0, 0.95, 1.0, 0.9, 0.5], np.float32)
    out.append(("cluster60", w))
    return out
