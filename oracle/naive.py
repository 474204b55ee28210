"""Second, deliberately naive CPU restatement of Tachyon's sampler.

TEST INFRASTRUCTURE ONLY: tests/ use it to cross-check the C++ oracle
(oracle/tachyon_oracle.cpp) on small inputs.  It is written independently of
that file and avoids its shortcuts: every ranking is a full sort of the whole
row instead of the reference's one-pass ``top_n``, so a mistake in either
restatement shows up as a disagreement.

Reference: /root/reference/src/sampler.rs (cited per function below) plus the
extension rules (presence/frequency penalty, min-p, packed mask, supplied
uniform) defined for this path.
"""
from __future__ import annotations

import ctypes
import math
import struct

import numpy as np

_libm = ctypes.CDLL("libm.so.6")
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]

F32 = np.float32


def expf(x) -> np.float32:
    """glibc expf, i.e. Rust's f32::exp on linux-gnu (sampler.rs:234)."""
    return F32(_libm.expf(float(x)))


def total_key(v) -> int:
    """f32::total_cmp order as an integer (sampler.rs:207, :220)."""
    (u,) = struct.unpack("<I", struct.pack("<f", float(F32(v))))
    return (~u & 0xFFFFFFFF) if u & 0x80000000 else (u | 0x80000000)


def rng_seed(seed: int) -> int:
    """Sampler::new state (sampler.rs:64)."""
    return ((seed * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF) | 1


def rng_next(state: int) -> tuple[float, int]:
    """Sampler::next_f32 (sampler.rs:255-261) -> (u, new_state)."""
    x = state
    x ^= x >> 12
    x ^= (x << 25) & 0xFFFFFFFFFFFFFFFF
    x ^= x >> 27
    m = (x * 0x2545F4914F6CDD1D) & 0xFFFFFFFFFFFFFFFF
    return float(F32(m >> 40) / F32(1 << 24)), x


def argmax(x) -> int:
    """sampler.rs:314-322: the lowest id among the maxima."""
    best = 0
    for i in range(len(x)):
        if x[i] > x[best]:
            best = i
    return best


def ieee_rank(buf) -> list[int]:
    """All ids, value descending with IEEE equality (-0 == +0), ties by id.

    The first n of this order are exactly what top_n(buf, n) keeps
    (sampler.rs:267-285)."""
    vals = [float(v) for v in buf]
    return sorted(range(len(vals)), key=lambda i: (-vals[i], i))


def total_rank(buf, ids) -> list[int]:
    """`ids` sorted by total_cmp descending, ties by id (sampler.rs:207)."""
    return sorted(ids, key=lambda i: (-total_key(buf[i]), i))


def penalize(x, recent, rep, pres, freq):
    """sampler.rs:165-175 and the presence/frequency extension."""
    buf = np.array(x, dtype=np.float32)
    n = len(buf)
    if len(recent) == 0:
        return buf
    counts: dict[int, int] = {}
    for t in recent:
        counts[int(t)] = counts.get(int(t), 0) + 1
    for t in sorted(counts):
        if t >= n:
            continue
        if F32(rep) != F32(1.0):
            v = buf[t]
            buf[t] = v / F32(rep) if v > 0 else v * F32(rep)
        if F32(pres) != 0 or F32(freq) != 0:
            buf[t] = (buf[t] - F32(freq) * F32(counts[t])) - F32(pres)
    return buf


def allowed(mask_row, i) -> bool:
    return bool((int(mask_row[i >> 5]) >> (i & 31)) & 1)


def sample_row(x, temperature, top_k, top_p, rep, recent=(), mask_row=None,
               u=0.0, pres=0.0, freq=0.0, min_p=0.0, constrained=False):
    """One row of tsm_sample: returns (token, keep, prob).

    sample/sample_with (sampler.rs:77-97) -> pick (:132-151) ->
    candidates (:155-247)."""
    x = np.asarray(x, dtype=np.float32)
    n = len(x)
    t_ = F32(temperature)
    greedy = t_ <= 0
    penal = len(recent) > 0 and (F32(rep) != 1 or F32(pres) != 0 or F32(freq) != 0)
    if not constrained and greedy and not penal:
        return argmax(x), 1, F32(1.0)
    t = F32(1.0) if greedy else t_
    buf = penalize(x, recent, rep, pres, freq)
    want = 1 if greedy else (n if top_k == 0 else min(top_k, n))
    window = min(max(want, 256), n) if constrained else want
    if window <= 1024:
        ranked = ieee_rank(buf)[:window]
    else:
        mx = F32(-np.inf)
        for v in buf:
            mx = F32(max(mx, v)) if not np.isnan(v) else mx
        cutoff = mx - F32(30.0) * t
        ranked = total_rank(buf, [i for i in range(n) if buf[i] >= cutoff])
    if constrained:
        ranked = [i for i in ranked if allowed(mask_row, i)]
        if not ranked:
            ranked = total_rank(buf, [i for i in range(n) if allowed(mask_row, i)])
    ranked = ranked[:want]
    if not ranked:
        return argmax(x), 0, F32(1.0)
    best = buf[ranked[0]]
    probs = [expf((buf[i] - best) / t) for i in ranked]
    if not greedy and F32(min_p) > 0:
        m = 0
        while m < len(probs) and probs[m] >= F32(min_p):
            m += 1
        probs = probs[: max(m, 1)]
    keep = len(probs)
    if not (greedy or F32(top_p) >= 1):
        total = F32(0.0)
        for p in probs:
            total = total + p
        acc = F32(0.0)
        for j, p in enumerate(probs):
            acc = acc + p / total
            if acc >= F32(top_p):
                keep = j + 1
                break
    mass = F32(0.0)
    for p in probs[:keep]:
        mass = mass + p
    r = F32(u) * mass
    pick = keep - 1
    for j in range(keep):
        r = r - probs[j]
        if r <= 0:
            pick = j
            break
    return ranked[pick], keep, probs[pick] / mass


def logprobs(x, token, n):
    """sampler.rs:297-312: (logprob, [(id, lp)...])."""
    x = np.asarray(x, dtype=np.float32)
    mx = F32(-np.inf)
    for v in x:
        mx = F32(max(mx, v))
    s = 0.0
    for v in x:
        s += math.exp(float(F32(v - mx)))
    lse = mx + F32(math.log(s))
    order = ieee_rank(x)[:n]
    return x[token] - lse, [(i, x[i] - lse) for i in order]
