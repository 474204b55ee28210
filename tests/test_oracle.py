"""Pins the CPU oracle (oracle/tachyon_oracle.cpp) before it is trusted as
the parity checker of the GPU path.

* The reference's own known-answer tests, ported from
  /root/reference/src/sampler.rs:328-395 and src/speculative.rs:349-391.
* Closed forms and hand-derived expectations (penalties, log-softmax).
* A mathematical pin of the RNG: the xorshift triple (12, 25, 27) gives a
  full-period generator over GF(2)^64.
* Brute force against oracle/naive.py, an independent full-sort restatement,
  on small and tie-heavy random inputs covering every row kind.
"""
import math
import struct

import numpy as np
import pytest

from oracle import naive
from tachyon_amd import workloads as wl


# --------------------------------------------------------------------------
# sampler.rs:328-395, ported
# --------------------------------------------------------------------------

def test_reference_greedy_and_top_k(oracle):
    logits = [0.1, 3.0, 2.9, -1.0]
    assert oracle.Sampler.greedy().sample(logits, 4) == 1
    s = oracle.Sampler(temperature=1.0, top_k=2, top_p=1.0, repetition_penalty=1.0, seed=3)
    for _ in range(200):
        assert s.sample(logits, 4) in (1, 2)


def test_reference_constraint_and_distribution(oracle):
    logits = [0.1, 3.0, 2.9, -1.0]
    s = oracle.Sampler.greedy()
    allowed = np.array([True, False, True, True])  # |t| t != 1
    mask = wl.pack_mask(allowed[None, :])[0]
    assert s.sample_with(logits, 4, [], mask) == 2
    s = oracle.Sampler(temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0, seed=1)
    d = s.distribution(logits, 4)
    assert d[0][0] == 1
    assert abs(np.float32(sum(np.float32(p) for _, p in d)) - 1.0) < 1e-5


def test_reference_top_n_matches_a_full_sort(oracle):
    x = np.array([((i * 2654435761) & 0xFFFFFFFF) % 10007 for i in range(5000)], np.float32)
    srt = sorted(((float(v), i) for i, v in enumerate(x)), key=lambda t: -t[0])
    vals, _ = oracle.top_n(x, 37)
    assert vals.tolist() == [v for v, _ in srt[:37]]


def test_reference_logprobs_are_log_softmax(oracle):
    lp, top_ids, _, _ = oracle.logprobs([1.0, 2.0, 3.0], 1, 2)
    f = np.float32
    z = f(math.log(float(f(math.exp(1.0)) + f(math.exp(2.0)) + f(math.exp(3.0)))))
    assert abs(lp - (2.0 - z)) < 1e-5
    assert top_ids.tolist() == [2, 1]


def test_reference_penalty_can_flip_the_choice(oracle):
    s = oracle.Sampler.greedy(repetition_penalty=2.0)
    assert s.sample([0.0, 3.0, 2.0], 3, [1]) == 2


# --------------------------------------------------------------------------
# speculative.rs:349-391, ported (draw / uniform / verify)
# --------------------------------------------------------------------------

def test_reference_speculative_sampling_preserves_the_target_distribution(oracle):
    p = [(0, 0.5), (1, 0.3), (2, 0.2)]
    q = [(0, 0.2), (1, 0.6), (2, 0.2)]
    rng = oracle.Sampler(temperature=1.0, top_k=0, top_p=1.0, repetition_penalty=1.0, seed=7)
    trials = 200_000
    counts = [0, 0, 0]
    for _ in range(trials):
        x = rng.draw(q)
        u = rng.uniform()
        verdict, residual = oracle.verify(p, q, x, u)
        t = x if verdict == "accept" else rng.draw(residual)
        counts[t] += 1
    for i, (_, want) in enumerate(p):
        assert abs(counts[i] / trials - want) < 0.01


def test_reference_deterministic_drafts_reduce_to_greedy(oracle):
    p = [(4, 1.0)]
    assert oracle.verify(p, [], 4, 0.99)[0] == "accept"
    v, r = oracle.verify(p, [], 5, 0.0)
    assert v == "resample" and r == [(4, 1.0)]


# --------------------------------------------------------------------------
# RNG (sampler.rs:64, :255-261)
# --------------------------------------------------------------------------

def _gf2_step_matrix(a, b, c):
    """Columns of the GF(2) matrix of x ^= x>>a; x ^= x<<b; x ^= x>>c."""
    M64 = (1 << 64) - 1

    def step(x):
        x ^= x >> a
        x ^= (x << b) & M64
        x ^= x >> c
        return x

    return [step(1 << i) for i in range(64)]


def _gf2_mul(A, B):
    # (A*B) column j = A applied to column j of B
    out = []
    for col in B:
        v = 0
        i = 0
        while col:
            if col & 1:
                v ^= A[i]
            col >>= 1
            i += 1
        out.append(v)
    return out


def _gf2_pow(A, e):
    R = [1 << i for i in range(64)]
    while e:
        if e & 1:
            R = _gf2_mul(A, R)
        A = _gf2_mul(A, A)
        e >>= 1
    return R


def test_rng_xorshift_triple_has_full_period():
    """(12, 25, 27) must make the state map a full-period linear map: order
    exactly 2^64-1.  A wrong shift or direction breaks this."""
    M = _gf2_step_matrix(12, 25, 27)
    ident = [1 << i for i in range(64)]
    n = (1 << 64) - 1
    assert _gf2_pow(M, n) == ident
    for q in (3, 5, 17, 257, 641, 65537, 6700417):
        assert _gf2_pow(M, n // q) != ident
    # a plausible typo is not full period
    assert _gf2_pow(_gf2_step_matrix(12, 25, 26), n) != ident


def test_rng_two_restatements_agree_and_output_grid(oracle):
    assert 0x2545F4914F6CDD1D == 2685821657736338717  # xorshift64* multiplier (Vigna)
    for seed in (0, 1, 3, 7, 0xDEADBEEF, (1 << 64) - 1):
        s = oracle.Sampler(seed=seed)
        st = naive.rng_seed(seed)
        assert s.state == st
        for _ in range(500):
            u, st = naive.rng_next(st)
            v = s.uniform()
            assert v == u
            assert 0.0 <= v < 1.0 and float(v * (1 << 24)).is_integer()
    # uniformity of the output over 2^18 draws (mean and a 64-bin chi-square)
    s = oracle.Sampler(seed=12345)
    us = np.array([s.uniform() for _ in range(1 << 18)])
    assert abs(us.mean() - 0.5) < 3e-3
    h, _ = np.histogram(us, bins=64, range=(0, 1))
    chi2 = float(((h - h.mean()) ** 2 / h.mean()).sum())
    assert chi2 < 120  # 63 dof; p ~ 1e-5 bound


# --------------------------------------------------------------------------
# Closed forms
# --------------------------------------------------------------------------

def test_penalties_hand_derived(oracle):
    x = np.array([2.0, -2.0, 0.0, -0.0, 5.0], np.float32)
    got = oracle.penalize(x, [0, 1, 2, 3, 3, 9], rep=2.0, pres=0.5, freq=0.25)
    # id0: 2/2=1 -> (1-.25)-.5 ; id1: -2*2=-4 -> (-4-.25)-.5 ; id2: 0 is not >0 -> 0*2=0 -> (0-.25)-.5
    # id3 (count 2): -0*2=-0 -> (-0-.5)-.5 ; id4 untouched ; id9 >= n ignored
    assert got.tolist() == [0.25, -4.75, -0.75, -1.0, 5.0]
    # repetition only: count-insensitive (sampler.rs:166-168 dedups)
    got = oracle.penalize(x, [0, 0, 0, 1], rep=2.0)
    assert got.tolist() == [1.0, -4.0, 0.0, -0.0, 5.0]


def test_logprobs_closed_form(oracle):
    rng = np.random.default_rng(5)
    for _ in range(20):
        x = (rng.standard_normal(3000) * 3).astype(np.float32)
        tok = int(rng.integers(0, 3000))
        lp, ids, lps, lse = oracle.logprobs(x, tok, 7)
        exact = float(x.max()) + math.log(math.fsum(math.exp(float(v) - float(x.max())) for v in x))
        assert abs(lse - exact) < 2e-6
        assert abs(lp - (float(x[tok]) - exact)) < 4e-6
        order = np.lexsort((np.arange(3000), -x.astype(np.float64)))[:7]
        assert ids.tolist() == order.tolist()


def test_argmax_first_maximum_and_zeros(oracle):
    assert oracle.argmax([1.0, 3.0, 3.0, 2.0]) == 1
    assert oracle.argmax([-0.0, 0.0, -1.0]) == 0  # -0 == +0: first wins
    assert oracle.argmax([-np.inf, -np.inf]) == 0


def test_top_n_matches_full_sort_with_ties(oracle):
    rng = np.random.default_rng(11)
    for _ in range(30):
        n = int(rng.integers(1, 400))
        x = rng.integers(-3, 4, size=n).astype(np.float32)
        x[rng.random(n) < 0.1] = -0.0
        k = int(rng.integers(0, n + 5))
        vals, ids = oracle.top_n(x, k)
        ref = naive.ieee_rank(x)[:k]
        assert ids.tolist() == ref


# --------------------------------------------------------------------------
# Brute force: C++ oracle vs the naive full-sort restatement
# --------------------------------------------------------------------------

def _naive_batch(w):
    out = []
    for r in range(w.rows):
        p = w.params[r]
        if w.hist_offsets is not None:
            rec = w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]]
        else:
            rec = []
        constrained = bool(p["flags"] & wl.ROW_CONSTRAINED)
        tok, keep, prob = naive.sample_row(
            w.logits[r, :w.usable], p["temperature"], int(p["top_k"]), p["top_p"],
            p["repetition_penalty"], rec, w.mask[r] if constrained else None, w.uniforms[r],
            p["presence_penalty"], p["frequency_penalty"], p["min_p"], constrained)
        lp = None
        if p["flags"] & wl.ROW_LOGPROBS:
            lp = naive.logprobs(w.logits[r, :w.usable], tok, int(p["n_logprobs"]))
        out.append((tok, keep, prob, lp))
    return out


CASES = [
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
]


@pytest.mark.parametrize("case", CASES, ids=[f"s{c['seed']}" for c in CASES])
def test_oracle_matches_naive(oracle, case):
    w = wl.random_case(**case)
    got = oracle.sample_batch(w)
    ref = _naive_batch(w)
    for r, (tok, keep, prob, lp) in enumerate(ref):
        assert int(got.token[r]) == tok, (r, w.params[r])
        assert int(got.keep[r]) == keep, r
        assert struct.pack("<f", got.prob[r]) == struct.pack("<f", np.float32(prob)), r
        if lp is not None:
            assert struct.pack("<f", got.logprob[r]) == struct.pack("<f", np.float32(lp[0])), r
            n = len(lp[1])
            assert got.top_ids[r, :n].tolist() == [i for i, _ in lp[1]]
            assert np.array_equal(got.top_lp[r, :n], np.array([v for _, v in lp[1]], np.float32))


def test_oracle_edge_cases(oracle):
    V = 40
    x = np.linspace(-2, 2, V).astype(np.float32)[None, :]
    base = dict(logits=x, usable=V, hist_ids=None, hist_offsets=None, uniforms=np.array([0.5], np.float32))

    def run(params, mask=None):
        w = wl.Workload("edge", params=params, mask=mask, **base)
        return oracle.sample_batch(w)

    # k > V behaves as k = V
    a = run(wl.make_params(1, temperature=1.0, top_k=1000))
    b = run(wl.make_params(1, temperature=1.0, top_k=V))
    assert a.token[0] == b.token[0]
    # nothing allowed -> argmax of the raw row, keep 0, no uniform consumed
    m = wl.pack_mask(np.zeros((1, V), bool))
    r = run(wl.make_params(1, temperature=1.0, top_k=5, flags=wl.ROW_CONSTRAINED), m)
    assert r.token[0] == V - 1 and r.keep[0] == 0 and r.diag["consumed_u"][0] == 0
    # only low ids allowed: outside the 256-window is impossible here (V < 256),
    # so window = V and the best allowed wins greedily
    allowed = np.zeros((1, V), bool)
    allowed[0, :3] = True
    r = run(wl.make_params(1, temperature=0.0, flags=wl.ROW_CONSTRAINED), wl.pack_mask(allowed))
    assert r.token[0] == 2
    # min_p keeps at least the best candidate
    r = run(wl.make_params(1, temperature=1.0, min_p=1.0))
    assert r.token[0] == V - 1 and r.keep[0] == 1


def test_constrained_window_rule_differs_from_mask_then_topk(oracle):
    """sampler.rs:184-222: rank the 256-wide window of UNMASKED logits, drop
    disallowed ids, then truncate to k.  With 0 < allowed-in-window < k the
    kept set is smaller than mask-then-top-k would give."""
    V = 1000
    x = np.arange(V, dtype=np.float32)[::-1].copy()[None, :] / 10  # id 0 best
    allowed = np.zeros((1, V), bool)
    allowed[0, [5, 600, 601, 602]] = True  # one inside the top-256 window
    w = wl.Workload("win", x, V, wl.make_params(1, temperature=1.0, top_k=3, flags=wl.ROW_CONSTRAINED),
                    None, None, wl.pack_mask(allowed), np.array([0.99], np.float32))
    r = oracle.sample_batch(w)
    assert r.token[0] == 5 and r.keep[0] == 1
    # nothing allowed inside the window -> whole-vocabulary fallback, then top-3
    allowed[0, 5] = False
    w.mask = wl.pack_mask(allowed)
    r = oracle.sample_batch(w)
    assert r.diag["path"][0] == 3 and r.keep[0] == 3 and r.token[0] in (600, 601, 602)


# ---- the measured boundary check (or_reconcile) -------------------------------

def _reference_pick(w, r, u, top_p=None):
    """The reference's (token, keep) for row r with its uniform set to u (and
    top_p, if given): the oracle run on a one-row copy."""
    from oracle import pyoracle

    one = wl.Workload("one", w.logits[r:r + 1].copy(), w.usable, w.params[r:r + 1].copy(), None, None, None,
                      np.array([u], np.float32))
    if top_p is not None:
        one.params["top_p"][0] = top_p
    if w.hist_ids is not None:
        a, b = int(w.hist_offsets[r]), int(w.hist_offsets[r + 1])
        one.hist_ids = w.hist_ids[a:b].copy()
        one.hist_offsets = np.array([0, b - a], np.uint32)
    res = pyoracle.sample_batch(one)
    return int(res.token[0]), int(res.keep[0])


def test_reconcile_matches_a_scan_of_u(oracle):
    """or_reconcile's u-shift against brute force: u swept over a grid of
    2^-16 steps, each value run through the reference's arithmetic; the
    nearest u that returns a given token must lie within one grid step of
    u + du (or u - du)."""
    from oracle import pyoracle

    w = wl.random_case(seed=61, vocab=1500, rows=4, mode="nucleus", logprobs=False, hist_len=0)
    grid = np.arange(0, 1 << 16, dtype=np.float64) / (1 << 16)
    for r in range(w.rows):
        u0 = float(w.uniforms[r])
        _, keep = _reference_pick(w, r, u0)
        picks = {}
        for u in grid[::64]:
            t, k = _reference_pick(w, r, np.float32(u))
            picks.setdefault(t, []).append(u)
        for tok, us in list(picks.items())[:6]:
            du, dp = pyoracle.reconcile(w, r, tok, keep)
            assert dp == 0.0
            nearest = min(abs(u - u0) for u in us)
            # the scan sees the token's interval only at its grid points
            assert du <= nearest + 1e-12, (r, tok, du, nearest)
            assert nearest - du <= 64.0 / (1 << 16), (r, tok, du, nearest)
            # and the reference returns the token at the reconciled u
            if du > 0.0:
                side = 1.0 if min(us, key=lambda u: abs(u - u0)) > u0 else -1.0
                u1 = np.float32(u0 + side * (du + 1e-7))
                assert _reference_pick(w, r, u1)[0] == tok, (r, tok, du)


def test_reconcile_top_p_shift(oracle):
    """The kept count as a step function of top_p: a kept count one off the
    reference's needs the measured shift in top_p, and the reference returns
    that count once top_p moves by it."""
    from oracle import pyoracle

    w = wl.random_case(seed=62, vocab=1500, rows=4, mode="topp", logprobs=False, hist_len=0)
    for r in range(w.rows):
        tok, keep = _reference_pick(w, r, float(w.uniforms[r]))
        assert pyoracle.reconcile(w, r, tok, keep) == (0.0, 0.0)
        if keep < 3:
            continue
        k2 = keep - 1
        res = pyoracle.reconcile(w, r, pyoracle.sample_batch(w).token[r], k2)
        if res is None:  # the token lies beyond k2: a pair no move reaches
            continue
        du, dp = res
        assert dp > 0.0
        p1 = np.float32(float(w.params["top_p"][r]) - dp)
        assert _reference_pick(w, r, float(w.uniforms[r]), top_p=p1)[1] == k2, (r, dp)


def test_boundary_check_rejects_exact_arithmetic_picks(oracle):
    """The parity bar measures the boundary: picks made with exact (f64)
    sums, as an earlier device path made them on c2's temperature-only rows,
    differ from the reference's sequential f32 folds by more than the 1e-5
    the north star allows on rows 8-10, 12, 13 and 15; the check rejects
    them.  The f64 view here is computed independently of the oracle's
    sampler (numpy sort, math.fsum mass, f64 cumulative sums)."""
    from oracle import pyoracle
    from parity import TOL_U, boundary_shift

    w = wl.c2()
    ref = pyoracle.sample_batch(w)
    over = []
    for r in range(8, 16):
        p = w.params[r]
        h = w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]]
        y = pyoracle.penalize(w.logits[r, :w.usable], h, float(p["repetition_penalty"]),
                              float(p["presence_penalty"]), float(p["frequency_penalty"]))
        t = np.float32(p["temperature"])
        cut = np.float32(y.max() - np.float32(30.0) * t)
        ids = np.nonzero(y >= cut)[0]
        ids = ids[np.lexsort((ids, -y[ids].astype(np.float64)))]
        probs = pyoracle.expf_array(((y[ids] - y[ids[0]]) / t).astype(np.float32)).astype(np.float64)
        mass = math.fsum(probs)
        j = int(np.searchsorted(np.cumsum(probs), float(w.uniforms[r]) * mass))
        tok = int(ids[min(j, len(ids) - 1)])
        assert boundary_shift(w, r, ref.token[r], ref.keep[r]) == (0.0, 0.0)
        du, dp = boundary_shift(w, r, tok, len(ids))
        if du > TOL_U:
            over.append(r)
    assert {8, 9, 10, 12, 13, 15} <= set(over), over


def test_nan_and_inf_semantics_hand_derived(oracle):
    """NaN and infinite logits, traced by hand through sampler.rs: top_n's
    insertion with partition_point in the probe order of Rust 1.87.0, the
    reference's pinned toolchain (size = len, base = 0; while size > 1: half
    = size / 2, mid = base + half, base = mid when w >= v holds, size -=
    half; then base + [w(base) >= v]), `v > floor` false for NaN, argmax's
    strict '>', NaN probabilities that no fold step decides, and pick
    falling through to idx[keep - 1] (sampler.rs:139-150, :267-285, :314-322)."""
    nan, inf = np.nan, np.inf
    # argmax: nothing beats a NaN at 0; elsewhere a NaN never wins
    assert oracle.argmax([1.0, nan, 3.0]) == 2
    assert oracle.argmax([nan, 5.0, 7.0]) == 0
    assert oracle.argmax([2.0, nan, 2.0]) == 0
    # [NaN, 1, 2], n=2: NaN enters first; 1 goes before it (NaN >= 1 is
    # false); the list is full with floor NaN, so 2 is never inserted
    v, i = oracle.top_n([nan, 1.0, 2.0], 2)
    assert i.tolist() == [1, 0] and v[0] == 1.0 and np.isnan(v[1])
    # [3, NaN, 1, 5], n=3: [3] -> [NaN, 3] -> [NaN, 3, 1] (probe at 3: 3 >= 1)
    # -> 5 > floor 1: probes 3 >= 5 no, NaN >= 5 no -> [5, NaN, 3]
    v, i = oracle.top_n([3.0, nan, 1.0, 5.0], 3)
    assert i.tolist() == [3, 1, 0] and v[0] == 5.0 and np.isnan(v[1]) and v[2] == 3.0
    # [6, NaN, 7, 9, 6, 5, 6], n=6, where the probe orders differ:
    # [6] -> [NaN, 6] -> 7: probe 6 (no), base NaN (no): [7, NaN, 6]
    # -> 9: probes NaN, NaN, base 7 (no): [9, 7, NaN, 6]
    # -> 6 (id 4): size 4 probes NaN (no), size 2 probes 7 (yes, base 1),
    #    base 7 >= 6: at 2: [9, 7, 6, NaN, 6]
    # -> 5: size 5 probes 6 (yes, base 2), size 3 and 2 probe NaN (no),
    #    base 6 >= 5: at 3: [9, 7, 6, 5, NaN, 6], full, floor 6 (id 0)
    # -> 6 (id 6): 6 > 6 is false, skipped.  (The older halving search puts
    #    5 last, floor 5, and then inserts id 6: [3, 2, 4, 6, 1, 0].)
    v, i = oracle.top_n([6.0, nan, 7.0, 9.0, 6.0, 5.0, 6.0], 6)
    assert i.tolist() == [3, 2, 4, 5, 1, 0] and np.isnan(v[4])
    # [1, NaN, 2, 3, 0.5], n=4: [1] -> [NaN, 1] -> 2: probe 1 (no), base
    # NaN (no): [2, NaN, 1] -> 3: probes NaN, NaN, base 2 (no): at 0:
    # [3, 2, NaN, 1], full, floor 1: 0.5 is never inserted
    v, i = oracle.top_n([1.0, nan, 2.0, 3.0, 0.5], 4)
    assert i.tolist() == [3, 2, 1, 0]
    # [0, inf, 1, inf], n=3: ties of inf keep the lower id first
    v, i = oracle.top_n([0.0, inf, 1.0, inf], 3)
    assert i.tolist() == [1, 3, 2]

    def one(x, **kw):
        x = np.asarray([x], np.float32)
        w = wl.Workload("nan", x, x.shape[1], wl.make_params(1, **kw), None, None, None,
                        np.array([0.25], np.float32))
        return oracle.sample_batch(w)

    # ranked [(1, id 1), (NaN, id 0)]: p = [1, NaN], total NaN: acc never
    # reaches top_p, keep = 2, r = u * NaN never <= 0: the last kept, id 0
    r = one([nan, 1.0, 2.0, 0.5], temperature=1.0, top_k=2, top_p=0.9)
    assert r.token[0] == 0 and r.keep[0] == 2 and np.isnan(r.prob[0])
    # best +inf: p_0 = exp((inf - inf) / t) = NaN, so again the last kept (id 2)
    r = one([0.0, inf, 1.0, inf], temperature=1.0, top_k=3, top_p=0.5)
    assert r.token[0] == 2 and r.keep[0] == 3
    # every logit -inf: top_n keeps id order, p = exp(NaN) = NaN: the last, id 3;
    # sample()'s greedy shortcut is argmax: id 0
    r = one([-inf] * 4, temperature=1.0)
    assert r.token[0] == 3 and r.keep[0] == 4
    r = one([-inf] * 4, temperature=0.0)
    assert r.token[0] == 0
    # a NaN at id 0 and greedy: argmax returns 0 whatever follows
    r = one([nan, 9.0, 1.0], temperature=0.0)
    assert r.token[0] == 0


# ---- JsonObject (constrain.rs), the mask producer's oracle -------------------

JSON_VALID = [  # constrain.rs:315-326: accepted and complete
    b'{}',
    b'{"a": 1}',
    b'{"name": "Ada", "age": 36, "langs": ["en", "fr"], "ok": true, "x": null}',
    '{"n": -0.5e+10, "z": 0, "e": "é\\n\\"q\\""}'.encode(),
    b'{\n  "nested": {"deep": [[1, 2], {"k": false}]}\n}',
]
JSON_PREFIXES = [  # constrain.rs:329-340: accepted, not complete
    b'{"a": "unfinished',
    b'{"a": [1, 2',
    b'{"a": tr',
    b'{"a": 12',
]
JSON_INVALID = [  # constrain.rs:343-361: rejected
    b"[1]", b'"top"', b"{a: 1}", b'{"a" 1}', b'{"a": 01}', b'{"a": 1,}', b'{"a": tru}', b'{"a": "\\x"}',
    b'{"a": [1}', b'{"a": 1}}', b'{"a": "line\nbreak"}', b'{"a": .5}',
]


def test_json_reference_tests(oracle):
    """The reference's own constraint tests (constrain.rs:304-362)."""
    for t in JSON_VALID:
        assert oracle.json_check(t) == (True, True), t
    for t in JSON_PREFIXES:
        assert oracle.json_check(t) == (True, False), t
    for t in JSON_INVALID:
        assert not oracle.json_check(t)[0], t
    assert not oracle.json_check(b"{" + b" " * 40)[0]  # whitespace_is_bounded


def test_json_limits_hand_derived(oracle):
    """Limits traced through constrain.rs: a number's step returns `len < 40`
    with the length before the byte (the first digit is length 1), so 40
    digits pass and the 41st fails; `open` refuses a 33rd container; 16
    whitespace bytes in a row pass and the 17th fails; \\u takes exactly four
    hex digits."""
    assert oracle.json_check(b'{"a": ' + b"1" * 40)[0]
    assert not oracle.json_check(b'{"a": ' + b"1" * 41)[0]
    deep = b'{"a":' + b"[" * 31
    assert oracle.json_check(deep)[0]
    assert not oracle.json_check(deep + b"[")[0]
    assert oracle.json_check(b"{" + b" " * 16)[0]
    assert not oracle.json_check(b"{" + b" " * 17)[0]
    assert oracle.json_check(b'{"a": "\\u00e9"}') == (True, True)
    assert not oracle.json_check(b'{"a": "\\u00g9"}')[0]
    # a number ends at a byte that cannot continue it, which then counts as structure
    assert oracle.json_check(b'{"a": 0}') == (True, True)
    assert oracle.json_check(b'{"a": -0.5e-3 }') == (True, True)
    assert not oracle.json_check(b'{"a": -}')[0]
    assert not oracle.json_check(b'{"a": 1.}')[0]
    # after the object closes nothing follows, not even whitespace
    assert not oracle.json_check(b"{} ")[0]


# ---- the output layer (oracle/lmhead_oracle.cpp) ---------------------------------

def _bf16_bits(a):
    """float32 -> bf16 bit patterns, round to nearest even (no NaNs here)."""
    u = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def _bf16_f64(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def test_rmsnorm_closed_forms(oracle):
    """kernels.rs:522-528: the mean (not the sum) of squares, eps inside the
    square root, then x * inv * g.  A constant row of 0.5 with eps 0 has
    inv exactly 2 and gives g back; with eps = 1 on a row of 3s inv is
    1/sqrt(10); random rows agree with an f64 restatement to f32 rounding."""
    g = np.linspace(-2.0, 3.0, 64).astype(np.float32)
    out = oracle.rmsnorm(np.full((1, 64), 0.5, np.float32), g, 0.0)
    assert np.array_equal(out[0], g)
    out = oracle.rmsnorm(np.full((1, 64), 3.0, np.float32), np.ones(64, np.float32), 1.0)
    assert np.allclose(out[0], 3.0 / math.sqrt(10.0), rtol=2e-7, atol=0)
    rng = np.random.default_rng(5)
    x = rng.normal(0, 2.0, (7, 96)).astype(np.float32)
    w = rng.normal(1.0, 0.3, 96).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-5) * w.astype(np.float64)
    assert np.allclose(oracle.rmsnorm(x, w, 1e-5), ref, rtol=1e-5, atol=1e-6)


def test_matmul_bf16_selects_and_sums_exactly(oracle):
    """weights.rs:230-239 / kernels.rs:1411-1413: out[i][r] = sum_k W[r][k] *
    x[i][k].  One-hot rows of W (row r picks column (3r + 1) mod dim) on
    non-square shapes pin the indexing and the operand order; small integers
    give sums that f32 holds exactly, which must equal numpy's integer
    product."""
    rows, dim, t = 37, 64, 5
    w = np.zeros((rows, dim), np.float32)
    pick = (3 * np.arange(rows) + 1) % dim
    w[np.arange(rows), pick] = 1.0
    rng = np.random.default_rng(6)
    x = rng.normal(0, 1, (t, dim)).astype(np.float32)
    out = oracle.matmul_bf16(_bf16_bits(w), x)
    assert out.shape == (t, rows)
    assert np.array_equal(out, x[:, pick])
    wi = rng.integers(-3, 4, (rows, dim))
    xi = rng.integers(-5, 6, (t, dim))
    out = oracle.matmul_bf16(_bf16_bits(wi.astype(np.float32)), xi.astype(np.float32))
    assert np.array_equal(out, (xi @ wi.T).astype(np.float32))
    # bf16 rounding of W is the reference's (round to nearest even): 1 + 2^-8
    # (a tie) rounds to 1, 1 + 3 * 2^-8 to 1 + 2^-6
    assert _bf16_bits(np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8], np.float32)).tolist() == [0x3F80, 0x3F82]
    assert np.array_equal(_bf16_f64(_bf16_bits(np.array([1.5, -2.25], np.float32))), [1.5, -2.25])


def test_quantize_q8_known_answers(oracle):
    """kernels.rs:84-100: d = max|x| / 127 per 32-value block, q = (x / d)
    rounded half away from zero.  With max|x| = 127 the scale is exactly 1,
    so q is the rounding of x itself: the halves pin the rounding mode (half
    to even would give 0, -2, 2 for 0.5, -2.5, 2.5), and a second block at
    twice the size must give the same values with scale 2.  An all-zero
    block has scale 0 and values 0; a NaN neither sets the block's maximum
    nor survives as a value (`as i8` maps it to 0)."""
    head = [127.0, 0.5, -0.5, 1.5, -2.5, 2.5, 63.49, -63.5, 0.49, -127.0]
    want = [127, 1, -1, 2, -3, 3, 63, -64, 0, -127]
    b0 = np.zeros(32, np.float32)
    b0[:len(head)] = head
    b3 = np.zeros(32, np.float32)
    b3[0], b3[1], b3[2] = np.nan, 12.7, -6.35
    x = np.concatenate([b0, 2 * b0, np.zeros(32, np.float32), b3])
    sc, q = oracle.quantize_q8(x)
    assert sc[:3].tolist() == [1.0, 2.0, 0.0]
    assert np.float32(sc[3]) == np.float32(np.float32(12.7) / np.float32(127.0))
    assert q[:len(want)].tolist() == want and not q[len(want):32].any()
    assert np.array_equal(q[32:64], q[:32])
    assert not q[64:96].any()
    assert q[96:99].tolist() == [0, 127, -64] and not q[99:].any()


def test_f16_scales_match_numpy_for_every_finite_pattern(oracle):
    """f16_finite (kernels.rs:127-131) through the Q8 matmul: one weight row
    per finite f16 bit pattern, holding a single 1 against an activation
    block whose maximum is 127 (scale 1, value 127), so each logit is 127
    times the row's f16 scale, exact in f32.  numpy's float16 conversion is
    the check, normals, subnormals and both zeros alike."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    finite = ((bits >> 10) & 0x1F) != 0x1F
    h = bits[finite].astype(np.uint16)
    wq = np.zeros((h.size, 32), np.int8)
    wq[:, 0] = 1
    x = np.zeros((1, 32), np.float32)
    x[0, 0] = 127.0
    out = oracle.matmul_q8(wq, h[:, None], x)
    want = h.view(np.float16).astype(np.float32) * np.float32(127.0)
    # bit for bit, which also fixes the sign of the two zero logits: Rust's
    # f32 sum starts at -0.0, so -0.0 + (127 * -0.0) stays -0.0 (a sum from
    # +0.0 would give +0.0 there)
    assert np.array_equal(out[0].view(np.uint32), want.view(np.uint32))
    assert np.signbit(out[0][h == 0x8000]).all() and not np.signbit(out[0][h == 0]).any()


def test_matmul_q8_exact_integer_sums(oracle):
    """weights.rs:474-560 with Q8Rows (weights.rs:344-374) and the scalar
    dot_q8_with (kernels.rs:1420-1430): out[i][r] = sum over blocks of the
    block's integer dot * f16 scale * activation scale.  Activation rows
    whose every block reaches 127 are quantized exactly (scale 1), and
    power-of-two weight scales keep every term and sum exact in f32, so the
    result must equal numpy's integer product with the scales applied; a
    wrong block, row or scale index moves whole block dots."""
    rng = np.random.default_rng(11)
    rows, dim, t = 45, 128, 3
    nb = dim // 32
    wq = rng.integers(-127, 128, (rows, dim)).astype(np.int8)
    e = rng.integers(-3, 4, (rows, nb))
    sign = rng.choice([-1.0, 1.0], (rows, nb))
    scale = (sign * np.exp2(e)).astype(np.float16)
    xi = rng.integers(-60, 61, (t, dim))
    xi[:, ::32] = 127  # each block's maximum: the activation scale is 1
    out = oracle.matmul_q8(wq, scale.view(np.uint16), xi.astype(np.float32))
    blocks = (wq.astype(np.int64).reshape(rows, nb, 32)[None] * xi.reshape(t, 1, nb, 32)).sum(-1)
    want = (blocks * scale.astype(np.float64)[None]).sum(-1)
    assert np.array_equal(out.astype(np.float64), want)
    # an activation block of scale 2 doubles that block's share
    x2 = xi.astype(np.float32)
    x2[:, :32] *= 2
    out2 = oracle.matmul_q8(wq, scale.view(np.uint16), x2)
    assert np.array_equal(out2.astype(np.float64), want + blocks[..., 0] * scale[:, 0].astype(np.float64)[None])
