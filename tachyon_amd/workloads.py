"""Synthetic sampling workloads: the benchmark's five configurations (c1-c5)
and small random cases for parity tests.

Each workload holds host (numpy) arrays laid out exactly as the C ABI
expects (include/tachyon_sampler.h): logits [rows][row_stride] f32, per-row
``tsm_row_params`` records, CSR history, packed LSB-first masks and one
uniform per row.  Data is synthetic (there is no model here); its shapes and
distributions follow the benchmark configurations' descriptions.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

ROW_PARAMS_DTYPE = np.dtype(
    [
        ("temperature", "<f4"),
        ("top_k", "<u4"),
        ("top_p", "<f4"),
        ("repetition_penalty", "<f4"),
        ("presence_penalty", "<f4"),
        ("frequency_penalty", "<f4"),
        ("min_p", "<f4"),
        ("flags", "<u4"),
        ("n_logprobs", "<u4"),
        ("reserved", "<u4"),
    ]
)
assert ROW_PARAMS_DTYPE.itemsize == 40

ROW_CONSTRAINED = 1
ROW_LOGPROBS = 2

QWEN_VOCAB = 151936
LLAMA_VOCAB = 128256


@dataclass
class Workload:
    name: str
    logits: np.ndarray          # [rows, row_stride] f32
    usable: int
    params: np.ndarray          # [rows] ROW_PARAMS_DTYPE
    hist_ids: np.ndarray | None
    hist_offsets: np.ndarray | None
    mask: np.ndarray | None     # [rows, mask_stride] u32
    uniforms: np.ndarray        # [rows] f32
    top_stride: int = 0
    meta: dict = field(default_factory=dict)

    @property
    def rows(self) -> int:
        return int(self.logits.shape[0])

    @property
    def row_stride(self) -> int:
        return int(self.logits.shape[1])

    @property
    def mask_stride(self) -> int:
        return 0 if self.mask is None else int(self.mask.shape[1])

    def algorithmic_bytes(self) -> int:
        """Bytes one step must move at least (the headline metric's count): one read
        of every usable logit, the mask words of constrained rows, the history
        ids, the uniforms, and the outputs (token, plus logprob and n top
        (id, logprob) pairs for rows that ask for logprobs)."""
        rows = self.rows
        b = rows * self.usable * 4
        if self.mask is not None:
            nc = int(np.count_nonzero(self.params["flags"] & ROW_CONSTRAINED))
            b += nc * ((self.usable + 31) // 32) * 4
        if self.hist_ids is not None:
            b += self.hist_ids.size * 4
        b += rows * 4 + rows * 4  # uniforms in, tokens out
        nlp = self.params["n_logprobs"].astype(np.int64)
        lp_rows = (self.params["flags"] & ROW_LOGPROBS) != 0
        b += int(np.sum(np.where(lp_rows, 4 + 8 * nlp, 0)))
        return int(b)


def make_params(rows, temperature=0.7, top_k=0, top_p=1.0, repetition_penalty=1.0,
                presence_penalty=0.0, frequency_penalty=0.0, min_p=0.0, flags=0, n_logprobs=0):
    p = np.zeros(rows, ROW_PARAMS_DTYPE)
    p["temperature"] = temperature
    p["top_k"] = top_k
    p["top_p"] = top_p
    p["repetition_penalty"] = repetition_penalty
    p["presence_penalty"] = presence_penalty
    p["frequency_penalty"] = frequency_penalty
    p["min_p"] = min_p
    p["flags"] = flags
    p["n_logprobs"] = n_logprobs
    return p


def uniforms(rng, rows):
    """Per-row u = k / 2^24 with integer k, i.e. exactly the values
    Sampler::next_f32 can produce (sampler.rs:260)."""
    return (rng.integers(0, 1 << 24, size=rows).astype(np.float32) / np.float32(1 << 24)).astype(np.float32)


def zipf_histories(rng, rows, length, vocab, a=1.1):
    """Per-row histories of `length` ids whose ranks follow Zipf(a); rank -> id
    through a seeded permutation of the vocabulary."""
    perm = rng.permutation(vocab).astype(np.uint32)
    ranks = np.empty((rows, length), np.int64)
    filled = 0
    flat = ranks.reshape(-1)
    need = rows * length
    while filled < need:
        z = rng.zipf(a, size=2 * (need - filled))
        z = z[z <= vocab]
        take = min(z.size, need - filled)
        flat[filled:filled + take] = z[:take]
        filled += take
    ids = perm[(ranks - 1) % vocab]
    offsets = (np.arange(rows + 1, dtype=np.uint32) * length).astype(np.uint32)
    return ids.reshape(-1).astype(np.uint32), offsets


def uniform_histories(rng, rows, length, vocab):
    ids = rng.integers(0, vocab, size=rows * length).astype(np.uint32)
    offsets = (np.arange(rows + 1, dtype=np.uint32) * length).astype(np.uint32)
    return ids, offsets


def pack_mask(allowed: np.ndarray) -> np.ndarray:
    """bool [rows, usable] -> u32 [rows, ceil(usable/32)], LSB-first."""
    rows, n = allowed.shape
    words = (n + 31) // 32
    padded = np.zeros((rows, words * 32), bool)
    padded[:, :n] = allowed
    bits = padded.reshape(rows, words, 32).astype(np.uint64)
    w = (bits << np.arange(32, dtype=np.uint64)).sum(axis=2)
    return w.astype(np.uint32)


def gaussian_logits(rng, rows, vocab, sigma):
    x = rng.standard_normal((rows, vocab), dtype=np.float32)
    x *= np.float32(sigma)
    return x


def c1(seed=0x5EED0001) -> Workload:
    """B=1, V=151936, N(0,3^2) + 20 spikes of +8; T=.7 k=40 p=.9 R=1.1/64."""
    rng = np.random.default_rng(seed)
    V = QWEN_VOCAB
    x = gaussian_logits(rng, 1, V, 3.0)
    spikes = rng.choice(V, size=20, replace=False)
    x[0, spikes] += np.float32(8.0)
    ids, off = uniform_histories(rng, 1, 64, V)
    p = make_params(1, temperature=0.7, top_k=40, top_p=0.9, repetition_penalty=1.1)
    return Workload("c1", x, V, p, ids, off, None, uniforms(rng, 1))


def c2(seed=0x5EED0002, rows=32) -> Workload:
    """B=32 mixed rows (greedy / T=1 only / k=50 p=.95 / min_p=.05), N(0,2^2),
    presence .5 frequency .3 over 512-token Zipf(1.1) histories."""
    rng = np.random.default_rng(seed)
    V = QWEN_VOCAB
    x = gaussian_logits(rng, rows, V, 2.0)
    ids, off = zipf_histories(rng, rows, 512, V)
    p = make_params(rows, temperature=1.0, presence_penalty=0.5, frequency_penalty=0.3)
    q = rows // 4
    p["temperature"][:q] = 0.0
    p["top_k"][2 * q:3 * q] = 50
    p["top_p"][2 * q:3 * q] = 0.95
    p["min_p"][3 * q:] = 0.05
    return Workload("c2", x, V, p, ids, off, None, uniforms(rng, rows))


def c3(seed=0x5EED0003, rows=256, vocab=LLAMA_VOCAB) -> Workload:
    """B=256, V=128256, N(0,3^2); per-row mask with allowed fraction
    log-uniform in [0.1%, 60%] (half contiguous ranges, half scattered);
    T=.8 k=40 p=.9; top-20 logprobs."""
    rng = np.random.default_rng(seed)
    V = vocab
    x = gaussian_logits(rng, rows, V, 3.0)
    allowed = np.zeros((rows, V), bool)
    for r in range(rows):
        f = float(np.exp(rng.uniform(np.log(0.001), np.log(0.6))))
        n_allow = max(1, int(round(f * V)))
        if r % 2 == 0:
            nr = int(rng.integers(1, 9))
            lens = rng.multinomial(n_allow, np.ones(nr) / nr)
            for ln in lens:
                if ln == 0:
                    continue
                s = int(rng.integers(0, V - ln + 1))
                allowed[r, s:s + ln] = True
        else:
            allowed[r, rng.choice(V, size=n_allow, replace=False)] = True
    mask = pack_mask(allowed)
    p = make_params(rows, temperature=0.8, top_k=40, top_p=0.9,
                    flags=ROW_CONSTRAINED | ROW_LOGPROBS, n_logprobs=20)
    return Workload("c3", x, V, p, None, None, mask, uniforms(rng, rows), top_stride=20)


def c4(seed=0x5EED0004, rows=256) -> Workload:
    """Headline: B=256, V=151936, N(0,3^2); R=1.1 + presence .4 + frequency .2
    over 1024-token Zipf histories; 30% mask; T=.7 k=64 p=.92 min_p=.02;
    top-5 logprobs."""
    rng = np.random.default_rng(seed)
    V = QWEN_VOCAB
    x = gaussian_logits(rng, rows, V, 3.0)
    ids, off = zipf_histories(rng, rows, 1024, V)
    allowed = rng.random((rows, V), dtype=np.float32) < np.float32(0.3)
    mask = pack_mask(allowed)
    p = make_params(rows, temperature=0.7, top_k=64, top_p=0.92, min_p=0.02,
                    repetition_penalty=1.1, presence_penalty=0.4, frequency_penalty=0.2,
                    flags=ROW_CONSTRAINED | ROW_LOGPROBS, n_logprobs=5)
    return Workload("c4", x, V, p, ids, off, mask, uniforms(rng, rows), top_stride=5)


def c5(seed=0x5EED0005, rows=1024) -> Workload:
    """Worst-case nucleus: B=1024, V=151936, N(0,1); T=1.2, no top-k,
    p=.98, R=1.05 over 256-token histories."""
    rng = np.random.default_rng(seed)
    V = QWEN_VOCAB
    x = gaussian_logits(rng, rows, V, 1.0)
    ids, off = uniform_histories(rng, rows, 256, V)
    p = make_params(rows, temperature=1.2, top_k=0, top_p=0.98, repetition_penalty=1.05)
    return Workload("c5", x, V, p, ids, off, None, uniforms(rng, rows))


CONFIGS = {"c1": c1, "c2": c2, "c3": c3, "c4": c4, "c5": c5}


def random_case(seed, rows=8, vocab=300, stride=None, ties=False, masked=False, mask_frac=0.3,
                logprobs=True, hist_len=16, penalties=True, mode="mixed", sigma=2.0, outlier=None,
                specials=False, nan_frac=0.0):
    """Small random workload for parity tests: mixed per-row settings, optional
    heavy ties (integer-valued logits), masks and histories.  `outlier` sets
    id 0 of every row to that value (a narrow cluster of logits next to one
    far value); `specials` puts NaN, +inf and -inf logits into the rows;
    `nan_frac` makes that fraction of every row's ids NaN."""
    rng = np.random.default_rng(seed)
    stride = stride or vocab
    if ties:
        x = rng.integers(-4, 5, size=(rows, stride)).astype(np.float32)
        x[rng.random((rows, stride)) < 0.05] = -0.0
    else:
        x = (rng.standard_normal((rows, stride)) * sigma).astype(np.float32)
    if outlier is not None:
        x[:, 0] = np.float32(outlier)
    if specials:
        # row r by r % 6: NaNs at 3 random ids, two +inf, 70% -inf, all -inf,
        # a NaN at id 0, one +inf and two NaNs
        srng = np.random.default_rng(seed + 7777)
        for r in range(rows):
            k = r % 6
            if k == 0:
                x[r, srng.integers(0, vocab, 3)] = np.nan
            elif k == 1:
                x[r, srng.integers(0, vocab, 2)] = np.inf
            elif k == 2:
                x[r, :vocab][srng.random(vocab) < 0.7] = -np.inf
            elif k == 3:
                x[r, :vocab] = -np.inf
            elif k == 4:
                x[r, 0] = np.nan
            else:
                x[r, srng.integers(0, vocab, 1)] = np.inf
                x[r, srng.integers(0, vocab, 2)] = np.nan
    if nan_frac > 0.0:
        nrng = np.random.default_rng(seed + 9999)
        x[:, :vocab][nrng.random((rows, vocab)) < nan_frac] = np.nan
    p = make_params(rows)
    for r in range(rows):
        kind = mode if mode != "mixed" else ["greedy", "topk", "topp", "nucleus", "minp", "all"][r % 6]
        t = float(rng.choice([0.0, 0.5, 0.7, 1.0, 1.3])) if kind != "greedy" else 0.0
        if kind != "greedy" and t == 0.0:
            t = 0.8
        p["temperature"][r] = t
        p["top_k"][r] = {"greedy": 1, "topk": int(rng.integers(1, 80)), "topp": int(rng.integers(1, 300)),
                         "nucleus": 0, "minp": 0, "all": int(rng.integers(0, 200))}[kind]
        p["top_p"][r] = {"greedy": 1.0, "topk": 1.0, "topp": float(rng.uniform(0.3, 0.99)),
                         "nucleus": float(rng.uniform(0.5, 1.0)), "minp": 1.0,
                         "all": float(rng.uniform(0.5, 0.99))}[kind]
        p["min_p"][r] = {"minp": float(rng.uniform(0.01, 0.5)), "all": float(rng.uniform(0.0, 0.1))}.get(kind, 0.0)
        if penalties:
            p["repetition_penalty"][r] = float(rng.choice([1.0, 1.1, 0.9, 2.0]))
            p["presence_penalty"][r] = float(rng.choice([0.0, 0.4, -0.3]))
            p["frequency_penalty"][r] = float(rng.choice([0.0, 0.2, 0.5]))
        flags = 0
        if masked and rng.random() < 0.8:
            flags |= ROW_CONSTRAINED
        if logprobs and rng.random() < 0.7:
            flags |= ROW_LOGPROBS
            p["n_logprobs"][r] = int(rng.integers(0, 21))
        p["flags"][r] = flags
    if hist_len > 0:
        lens = rng.integers(0, hist_len + 1, size=rows)
        offs = np.zeros(rows + 1, np.uint32)
        offs[1:] = np.cumsum(lens)
        ids = rng.integers(0, vocab + 3, size=int(offs[-1])).astype(np.uint32)  # a few ids >= usable
    else:
        ids, offs = None, None
    mask = None
    if masked:
        fr = rng.uniform(0.0, mask_frac, size=(rows, 1))
        allowed = rng.random((rows, vocab)) < fr
        mask = pack_mask(allowed)
    top_stride = 20 if logprobs else 0
    return Workload(f"rand{seed}", x, vocab, p, ids, offs, mask, uniforms(rng, rows), top_stride=top_stride)


def window_case(seed, vocab, rows=1, top_k=1024, hist_len=10, repetition_penalty=1.3, masked=False,
                mask_frac=0.5, sigma=2.0):
    """Top-k windows near their 1024 limit over small vocabularies: a
    segment of the split-row kernel then has fewer finite group maxima than
    the window needs, and every one of its elements is a candidate.  Rows
    take top_k, top_k - 24, ... so a batch holds several window sizes; each
    row's history is `hist_len` distinct ids, penalized by
    `repetition_penalty`."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, vocab)) * sigma).astype(np.float32)
    p = make_params(rows, temperature=0.8, top_p=1.0, repetition_penalty=repetition_penalty)
    for r in range(rows):
        p["top_k"][r] = max(1, top_k - 24 * r)
        if masked:
            p["flags"][r] |= ROW_CONSTRAINED
        if r % 2:
            p["flags"][r] |= ROW_LOGPROBS
            p["n_logprobs"][r] = 5
    ids = np.concatenate([rng.choice(vocab, hist_len, replace=False) for _ in range(rows)]).astype(np.uint32)
    offs = (np.arange(rows + 1) * hist_len).astype(np.uint32)
    mask = pack_mask(rng.random((rows, vocab)) < mask_frac) if masked else None
    return Workload(f"window{seed}", x, vocab, p, ids, offs, mask, uniforms(rng, rows), top_stride=8)


def below_window_case(seed, vocab=6000, rows=20):
    """Constrained top-k rows (k = 40, window 256; 20 rows, beyond the
    split kernel's batches) whose allowed ids all lie below the window: the
    other ids sit around 6, the allowed ones (60 to 120 a row) take +0, -0,
    -1 or -2 (even rows) or N(-3, 1) values (odd rows), so the kept list
    comes from the fallback over the whole row (sampler.rs:211-221), where
    f32::total_cmp puts +0 before -0."""
    rng = np.random.default_rng(seed)
    x = (6.0 + rng.standard_normal((rows, vocab))).astype(np.float32)
    allowed = np.zeros((rows, vocab), bool)
    for r in range(rows):
        ids = rng.choice(vocab, int(rng.integers(60, 121)), replace=False)
        allowed[r, ids] = True
        if r % 2 == 0:
            x[r, ids] = rng.choice(np.array([0.0, -0.0, -1.0, -2.0], np.float32), len(ids))
        else:
            x[r, ids] = (rng.standard_normal(len(ids)) - 3.0).astype(np.float32)
    p = make_params(rows, temperature=0.8, top_k=40, top_p=0.9, flags=ROW_CONSTRAINED | ROW_LOGPROBS,
                    n_logprobs=5)
    p["min_p"][1::4] = 0.05
    ids, offs = uniform_histories(rng, rows, 32, vocab)
    p["repetition_penalty"][::3] = 1.2
    return Workload(f"below{seed}", x, vocab, p, ids, offs, pack_mask(allowed), uniforms(rng, rows), top_stride=5)


def cluster_case(seed, vocab=151936, rows=4, width=0.025, temperature=3.0, top_p=0.9, sigma=3.0):
    """Nucleus rows (no top-k) whose first third of the vocabulary sits in a
    dense Gaussian cluster about `width` wide at 3.0, beside N(0, sigma^2)
    logits: at a high temperature every id is a candidate and one value bin
    of the cluster holds thousands of them."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((rows, vocab)) * sigma).astype(np.float32)
    k = vocab // 3
    x[:, :k] = (3.0 + rng.standard_normal((rows, k)) * (width / 6.0)).astype(np.float32)
    p = make_params(rows, temperature=temperature, top_k=0, top_p=top_p)
    p["repetition_penalty"][1::2] = 1.1
    ids, offs = uniform_histories(rng, rows, 64, vocab)
    return Workload(f"cluster{seed}", x, vocab, p, ids, offs, None, uniforms(rng, rows))


def sweep_batch(seed, rows=32):
    """One batch of the seeded GPU sweep: a vocabulary size, a logit
    distribution (Gaussian of several widths, bf16-like quantized values with
    many equal logits, one far outlier per row, a dense cluster over a third
    of the row), per-row temperature, top-k (none, inside and beyond the
    1024-entry window), top-p, min-p, penalties and, for some batches, a mask
    with constrained rows.  Returns (workload, distribution kind)."""
    rng = np.random.default_rng(seed)
    V = int(rng.choice([3000, 20000, 60000, 151936]))
    sig = float(rng.choice([0.3, 1.0, 2.0, 3.0, 6.0]))
    x = (rng.standard_normal((rows, V)) * sig).astype(np.float32)
    kind = int(rng.integers(0, 5))
    if kind == 1:
        x = (np.round(x * 8) / 8).astype(np.float32)
    elif kind == 2:
        x[np.arange(rows), rng.integers(0, V, rows)] += np.float32(rng.uniform(2, 15))
    elif kind == 3:
        x[:, :V // 3] = (x[:, :V // 3] * 0.001 + 3).astype(np.float32)
    p = make_params(rows, temperature=1.0, top_k=0, top_p=1.0)
    p["temperature"] = rng.choice([0.3, 0.7, 1.0, 1.5, 3.0], rows).astype(np.float32)
    p["top_p"] = rng.choice([0.5, 0.9, 0.95, 0.99, 1.0], rows).astype(np.float32)
    p["top_k"] = rng.choice([0, 0, 0, 50, 2000, 5000], rows).astype(np.uint32)
    p["presence_penalty"] = np.where(rng.random(rows) < 0.2, 0.3, 0.0).astype(np.float32)
    p["min_p"] = np.where(rng.random(rows) < 0.2, 0.01, 0.0).astype(np.float32)
    p["repetition_penalty"] = np.where(rng.random(rows) < 0.3, 1.1, 1.0).astype(np.float32)
    ids, off = uniform_histories(rng, rows, 64, V)
    mask = None
    if rng.random() < 0.3:
        mask = pack_mask(rng.random((rows, V)) < rng.uniform(0.05, 0.9))
        p["flags"] = np.where(rng.random(rows) < 0.5, ROW_CONSTRAINED, 0).astype(np.uint32)
    return Workload(f"sweep{seed}", x, V, p, ids, off, mask, uniforms(rng, rows)), kind


# ---- JSON-object constraints (mask producer) ----------------------------------

def _pick_bytes(rng, alphabet, n):
    """n bytes drawn from `alphabet` (a list of byte values)."""
    return bytes(np.asarray(rng.choice(alphabet, n), np.uint8).tolist())


JSON_FRAGMENTS = [
    b"{", b"}", b"[", b"]", b",", b":", b'"', b'{"', b'"}', b'":', b'": ', b'", "', b'",', b'"]', b'["',
    b"[{", b"}]", b"},", b"],", b" {", b" [", b"true", b"false", b"null", b"tru", b"fal", b"nul", b"ue",
    b"se", b"ll", b"0", b"-", b"-0", b"0.", b".5", b"1e", b"e+", b"E-", b"12", b"123", b"3.14", b"1e10",
    b"00", b"01", b"-.", b"\\", b"\\n", b'\\"', b"\\u", b"\\u00", b"00e9", b"\\x", b"ab", b" ", b"  ",
    b"    ", b"\n", b"\n  ", b"\t", b"\r\n", b'  "', b"\xc3\xa9", b"\xe2\x82\xac", b"\x01", b"\x1f",
    b'{"a', b'"a"', b'": "', b'": [', b'": {', b'": 1', b'": -', b'": t', b'": n', b'": f', b"}}",
    b"]]", b"},{", b'", "b', b"1,", b"1}", b"0]", b" 1", b" -", b" :", b": ", b" ,", b" }", b" ]",
]


def json_vocab(n_tokens=151936, seed=0x15A0, n_special=24, n_empty=8):
    """A synthetic tokenizer vocabulary for the mask producer: every single
    byte, JSON fragments, BPE-like words (letters, digits, punctuation, UTF-8,
    a leading space), some long tokens, empty tokens and special tokens.
    Returns (tokens: list of bytes, special_ids)."""
    rng = np.random.default_rng(seed)
    toks = [bytes([b]) for b in range(256)] + list(JSON_FRAGMENTS)
    alpha = b"abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ"
    punct = b"{}[]:,\"\\-+.eE0123456789 \t\n"
    while len(toks) < n_tokens - n_special - n_empty:
        kind = rng.integers(0, 10)
        if kind < 5:      # a word, often with a leading space
            w = _pick_bytes(rng, list(alpha), int(rng.integers(1, 10)))
            toks.append((b" " if rng.random() < 0.5 else b"") + w)
        elif kind < 7:    # digits and number pieces
            toks.append(_pick_bytes(rng, list(b"0123456789.eE+-"), int(rng.integers(1, 7))))
        elif kind < 9:    # punctuation runs, JSON-ish
            toks.append(_pick_bytes(rng, list(punct), int(rng.integers(1, 5))))
        else:             # UTF-8 text or a long token
            if rng.random() < 0.8:
                cps = rng.integers(0xA0, 0x3000, int(rng.integers(1, 4)))
                toks.append("".join(chr(int(c)) for c in cps).encode())
            else:
                toks.append(_pick_bytes(rng, list(alpha + b" "), int(rng.integers(16, 64))))
    toks += [b""] * n_empty
    specials = []
    for k in range(n_special):
        specials.append(len(toks))
        toks.append(b"<|special_%d|>" % k)
    return toks[:n_tokens], [s for s in specials if s < n_tokens]


def json_document(rng, depth=0, max_depth=4):
    """A random JSON value's bytes (the top level an object)."""
    def ws():
        return _pick_bytes(rng, list(b" \n\t"), int(rng.integers(0, 3))) if rng.random() < 0.4 else b""

    def string():
        parts = []
        for _ in range(int(rng.integers(0, 6))):
            r = rng.random()
            if r < 0.1:
                parts.append([b'\\"', b"\\\\", b"\\n", b"\\u00e9", b"\\/"][int(rng.integers(0, 5))])
            elif r < 0.2:
                parts.append("é€".encode())
            else:
                parts.append(_pick_bytes(rng, list(b"abcxyz 0123"), int(rng.integers(1, 5))))
        return b'"' + b"".join(parts) + b'"'

    def value(d):
        r = rng.random()
        if d < max_depth and r < 0.25:
            return obj(d + 1)
        if d < max_depth and r < 0.4:
            items = [ws() + value(d + 1) + ws() for _ in range(int(rng.integers(0, 4)))]
            return b"[" + b",".join(items) + b"]"
        if r < 0.6:
            return string()
        if r < 0.85:
            return [b"0", b"-12", b"3.25", b"1e10", b"-0.5E-3", b"42"][int(rng.integers(0, 6))]
        return [b"true", b"false", b"null"][int(rng.integers(0, 3))]

    def obj(d):
        items = [ws() + string() + ws() + b":" + ws() + value(d) + ws() for _ in range(int(rng.integers(0, 4)))]
        return b"{" + b",".join(items) + b"}"

    return obj(depth)


def json_prefixes(count, seed=0x15A1):
    """`count` random cuts of random JSON-object documents (bytes), from the
    empty prefix to whole documents: the states a constrained sequence
    passes through."""
    rng = np.random.default_rng(seed)
    out = [b""]
    while len(out) < count:
        doc = json_document(rng)
        out.append(doc[:int(rng.integers(0, len(doc) + 1))])
    return out[:count]
