"""ctypes binding of oracle/libtachyon_oracle.so (TEST INFRASTRUCTURE ONLY).

The C++ oracle restates /root/reference/src/sampler.rs; see
oracle/tachyon_oracle.cpp.  Used by tests/, smoke() and bench.py's
cpu_baseline leg as the checker, never by the product path.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from dataclasses import dataclass

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libtachyon_oracle.so")

c_f32p = ctypes.POINTER(ctypes.c_float)
c_u32p = ctypes.POINTER(ctypes.c_uint32)


class OrConfig(ctypes.Structure):
    _fields_ = [
        ("temperature", ctypes.c_float),
        ("top_k", ctypes.c_uint32),
        ("top_p", ctypes.c_float),
        ("repetition_penalty", ctypes.c_float),
        ("seed", ctypes.c_uint64),
        ("presence_penalty", ctypes.c_float),
        ("frequency_penalty", ctypes.c_float),
        ("min_p", ctypes.c_float),
    ]


class OrRowDiag(ctypes.Structure):
    _fields_ = [
        ("path", ctypes.c_uint32),
        ("ranked", ctypes.c_uint32),
        ("survivors", ctypes.c_uint32),
        ("keep", ctypes.c_uint32),
        ("pick", ctypes.c_uint32),
        ("consumed_u", ctypes.c_uint32),
        ("mass", ctypes.c_float),
        ("best", ctypes.c_float),
    ]


DIAG_DTYPE = np.dtype(
    [
        ("path", "<u4"), ("ranked", "<u4"), ("survivors", "<u4"), ("keep", "<u4"),
        ("pick", "<u4"), ("consumed_u", "<u4"), ("mass", "<f4"), ("best", "<f4"),
    ],
    align=True,
)
assert DIAG_DTYPE.itemsize == ctypes.sizeof(OrRowDiag)

PATH_ARGMAX_FAST, PATH_TOP_N, PATH_CUTOFF, PATH_FALLBACK, PATH_NONE_ALLOWED = range(5)

_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.or_rng_seed.restype = ctypes.c_uint64
        L.or_rng_seed.argtypes = [ctypes.c_uint64]
        L.or_rng_next.restype = ctypes.c_float
        L.or_rng_next.argtypes = [ctypes.POINTER(ctypes.c_uint64)]
        L.or_top_n.restype = ctypes.c_size_t
        L.or_top_n.argtypes = [c_f32p, ctypes.c_size_t, ctypes.c_size_t, c_f32p, c_u32p]
        L.or_argmax.restype = ctypes.c_uint32
        L.or_argmax.argtypes = [c_f32p, ctypes.c_size_t]
        L.or_logprobs.restype = ctypes.c_float
        L.or_logprobs.argtypes = [c_f32p, ctypes.c_size_t, ctypes.c_uint32, ctypes.c_size_t,
                                  c_u32p, c_f32p, c_f32p]
        L.or_penalize.restype = None
        L.or_penalize.argtypes = [c_f32p, ctypes.c_size_t, c_u32p, ctypes.c_size_t,
                                  ctypes.c_float, ctypes.c_float, ctypes.c_float]
        L.or_expf_array.restype = None
        L.or_expf_array.argtypes = [c_f32p, c_f32p, ctypes.c_size_t]
        L.or_sampler_new.restype = ctypes.c_void_p
        L.or_sampler_new.argtypes = [ctypes.POINTER(OrConfig)]
        L.or_sampler_free.restype = None
        L.or_sampler_free.argtypes = [ctypes.c_void_p]
        L.or_sampler_state.restype = ctypes.c_uint64
        L.or_sampler_state.argtypes = [ctypes.c_void_p]
        L.or_uniform.restype = ctypes.c_float
        L.or_uniform.argtypes = [ctypes.c_void_p]
        L.or_sample.restype = ctypes.c_uint32
        L.or_sample.argtypes = [ctypes.c_void_p, c_f32p, ctypes.c_size_t, ctypes.c_size_t,
                                c_u32p, ctypes.c_size_t]
        L.or_sample_with.restype = ctypes.c_uint32
        L.or_sample_with.argtypes = [ctypes.c_void_p, c_f32p, ctypes.c_size_t, ctypes.c_size_t,
                                     c_u32p, ctypes.c_size_t, c_u32p]
        L.or_distribution.restype = ctypes.c_size_t
        L.or_distribution.argtypes = [ctypes.c_void_p, c_f32p, ctypes.c_size_t, ctypes.c_size_t,
                                      c_u32p, ctypes.c_size_t, c_u32p, c_f32p, ctypes.c_size_t]
        L.or_draw.restype = ctypes.c_uint32
        L.or_draw.argtypes = [ctypes.c_void_p, c_u32p, c_f32p, ctypes.c_size_t]
        L.or_verify.restype = ctypes.c_int
        L.or_verify.argtypes = [c_u32p, c_f32p, ctypes.c_size_t, c_u32p, c_f32p, ctypes.c_size_t,
                                ctypes.c_uint32, ctypes.c_float, c_u32p, c_f32p,
                                ctypes.POINTER(ctypes.c_size_t)]
        vp = ctypes.c_void_p
        L.or_sample_batch.restype = ctypes.c_int
        L.or_sample_batch.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, vp,
                                      vp, vp, vp, ctypes.c_uint32, vp, vp, vp, vp, vp,
                                      ctypes.c_uint32, vp, vp, vp, ctypes.c_int]
        L.or_distribution_batch.restype = ctypes.c_int
        L.or_distribution_batch.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32,
                                            vp, vp, vp, vp, vp, ctypes.c_uint32, vp, ctypes.c_int]
        L.or_reconcile.restype = ctypes.c_int
        L.or_reconcile.argtypes = [vp, ctypes.c_uint32, vp, vp, ctypes.c_size_t, vp, ctypes.c_float,
                                   ctypes.c_uint32, ctypes.c_uint32, ctypes.POINTER(ctypes.c_double),
                                   ctypes.POINTER(ctypes.c_double)]
        L.or_json_new.restype = vp
        L.or_json_new.argtypes = []
        L.or_json_free.restype = None
        L.or_json_free.argtypes = [vp]
        L.or_json_clone.restype = vp
        L.or_json_clone.argtypes = [vp]
        L.or_json_advance.restype = None
        L.or_json_advance.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t]
        L.or_json_accepts.restype = ctypes.c_int
        L.or_json_accepts.argtypes = [vp, ctypes.c_char_p, ctypes.c_size_t]
        L.or_json_is_complete.restype = ctypes.c_int
        L.or_json_is_complete.argtypes = [vp]
        L.or_json_check.restype = None
        L.or_json_check.argtypes = [ctypes.c_char_p, ctypes.c_size_t, ctypes.POINTER(ctypes.c_int),
                                    ctypes.POINTER(ctypes.c_int)]
        L.or_json_mask.restype = None
        L.or_json_mask.argtypes = [vp, vp, vp, vp, ctypes.c_uint32, ctypes.c_uint32, vp]
        L.or_rmsnorm.restype = None
        L.or_rmsnorm.argtypes = [vp, vp, ctypes.c_uint32, ctypes.c_float, vp]
        L.or_matmul_bf16.restype = None
        L.or_matmul_bf16.argtypes = [vp, ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_uint32, vp,
                                     ctypes.c_uint32]
        L.or_quantize_q8.restype = None
        L.or_quantize_q8.argtypes = [vp, ctypes.c_uint32, vp, vp]
        L.or_matmul_q8.restype = None
        L.or_matmul_q8.argtypes = [vp, vp, ctypes.c_uint32, ctypes.c_uint32, vp, ctypes.c_uint32, vp,
                                   ctypes.c_uint32]
        _lib = L
    return _lib


def _p(a, ct):
    return a.ctypes.data_as(ctypes.POINTER(ct))


def _vp(a):
    return None if a is None else ctypes.c_void_p(a.ctypes.data)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def top_n(x, n):
    x = f32(x)
    v = np.zeros(max(n, 1), np.float32)
    i = np.zeros(max(n, 1), np.uint32)
    k = lib().or_top_n(_p(x, ctypes.c_float), x.size, n, _p(v, ctypes.c_float), _p(i, ctypes.c_uint32))
    return v[:k], i[:k]


def argmax(x):
    x = f32(x)
    return int(lib().or_argmax(_p(x, ctypes.c_float), x.size))


def logprobs(x, token, n):
    x = f32(x)
    ti = np.zeros(max(n, 1), np.uint32)
    tl = np.zeros(max(n, 1), np.float32)
    lse = ctypes.c_float()
    lp = lib().or_logprobs(_p(x, ctypes.c_float), x.size, token, n, _p(ti, ctypes.c_uint32),
                           _p(tl, ctypes.c_float), ctypes.byref(lse))
    k = min(n, x.size)
    return float(lp), ti[:k], tl[:k], float(lse.value)


def penalize(x, recent, rep=1.0, pres=0.0, freq=0.0):
    buf = f32(x).copy()
    r = u32(recent)
    lib().or_penalize(_p(buf, ctypes.c_float), buf.size, _p(r, ctypes.c_uint32), r.size, rep, pres, freq)
    return buf


def expf_array(x):
    x = f32(x)
    y = np.empty_like(x)
    lib().or_expf_array(_p(x, ctypes.c_float), _p(y, ctypes.c_float), x.size)
    return y


class Sampler:
    """The reference's Sampler object (sampler.rs:53-262) on the oracle."""

    def __init__(self, temperature=0.7, top_k=20, top_p=0.8, repetition_penalty=1.05, seed=0,
                 presence_penalty=0.0, frequency_penalty=0.0, min_p=0.0):
        self.cfg = OrConfig(temperature, top_k, top_p, repetition_penalty, seed, presence_penalty,
                            frequency_penalty, min_p)
        self.h = lib().or_sampler_new(ctypes.byref(self.cfg))

    @classmethod
    def greedy(cls, **kw):
        """SamplerConfig::greedy (sampler.rs:33-41)."""
        base = dict(temperature=0.0, top_k=1, top_p=1.0, repetition_penalty=1.0, seed=0)
        base.update(kw)
        return cls(**base)

    def __del__(self):
        if getattr(self, "h", None):
            lib().or_sampler_free(self.h)
            self.h = None

    def sample(self, logits, vocab, recent=()):
        x = f32(logits)
        r = u32(list(recent) or [0])
        return int(lib().or_sample(self.h, _p(x, ctypes.c_float), x.size, vocab, _p(r, ctypes.c_uint32),
                                   len(recent)))

    def sample_with(self, logits, vocab, recent, mask):
        x = f32(logits)
        r = u32(list(recent) or [0])
        m = u32(mask)
        return int(lib().or_sample_with(self.h, _p(x, ctypes.c_float), x.size, vocab,
                                        _p(r, ctypes.c_uint32), len(recent), _p(m, ctypes.c_uint32)))

    def distribution(self, logits, vocab, recent=()):
        x = f32(logits)
        r = u32(list(recent) or [0])
        ids = np.zeros(x.size, np.uint32)
        ps = np.zeros(x.size, np.float32)
        k = lib().or_distribution(self.h, _p(x, ctypes.c_float), x.size, vocab, _p(r, ctypes.c_uint32),
                                  len(recent), _p(ids, ctypes.c_uint32), _p(ps, ctypes.c_float), x.size)
        return list(zip(ids[:k].tolist(), ps[:k].tolist()))

    def draw(self, weighted):
        ids = u32([t for t, _ in weighted] or [0])
        w = f32([p for _, p in weighted] or [0])
        return int(lib().or_draw(self.h, _p(ids, ctypes.c_uint32), _p(w, ctypes.c_float), len(weighted)))

    def uniform(self):
        return float(lib().or_uniform(self.h))

    @property
    def state(self):
        return int(lib().or_sampler_state(self.h))


def verify(p, q, x, u):
    """speculative::verify (speculative.rs:167-189): ('accept', None) or
    ('resample', residual)."""
    pi = u32([t for t, _ in p] or [0])
    pp = f32([v for _, v in p] or [0])
    qi = u32([t for t, _ in q] or [0])
    qp = f32([v for _, v in q] or [0])
    ri = np.zeros(max(len(p), 1), np.uint32)
    rp = np.zeros(max(len(p), 1), np.float32)
    rn = ctypes.c_size_t()
    acc = lib().or_verify(_p(pi, ctypes.c_uint32), _p(pp, ctypes.c_float), len(p), _p(qi, ctypes.c_uint32),
                          _p(qp, ctypes.c_float), len(q), x, u, _p(ri, ctypes.c_uint32),
                          _p(rp, ctypes.c_float), ctypes.byref(rn))
    if acc:
        return "accept", None
    return "resample", list(zip(ri[: rn.value].tolist(), rp[: rn.value].tolist()))


@dataclass
class BatchResult:
    token: np.ndarray
    logprob: np.ndarray
    top_ids: np.ndarray
    top_lp: np.ndarray
    prob: np.ndarray
    keep: np.ndarray
    diag: np.ndarray


def sample_batch(w, nthreads=1) -> BatchResult:
    """tsm_sample() on the oracle for a workload (tachyon_amd.workloads)."""
    rows = w.rows
    top_stride = max(1, w.top_stride)
    token = np.zeros(rows, np.uint32)
    logprob = np.zeros(rows, np.float32)
    top_ids = np.zeros((rows, top_stride), np.uint32)
    top_lp = np.zeros((rows, top_stride), np.float32)
    prob = np.zeros(rows, np.float32)
    keep = np.zeros(rows, np.uint32)
    diag = np.zeros(rows, DIAG_DTYPE)
    lib().or_sample_batch(
        _vp(w.logits), rows, w.row_stride, w.usable, _vp(w.params), _vp(w.hist_ids),
        _vp(w.hist_offsets), _vp(w.mask), w.mask_stride, _vp(w.uniforms), _vp(token),
        _vp(logprob), _vp(top_ids), _vp(top_lp), top_stride, _vp(prob), _vp(keep), _vp(diag),
        nthreads)
    return BatchResult(token, logprob, top_ids, top_lp, prob, keep, diag)


def distribution_batch(w, dist_stride, nthreads=1):
    rows = w.rows
    ids = np.zeros((rows, dist_stride), np.uint32)
    ps = np.zeros((rows, dist_stride), np.float32)
    keep = np.zeros(rows, np.uint32)
    lib().or_distribution_batch(_vp(w.logits), rows, w.row_stride, w.usable, _vp(w.params),
                                _vp(w.hist_ids), _vp(w.hist_offsets), _vp(ids), _vp(ps),
                                dist_stride, _vp(keep), nthreads)
    return ids, ps, keep


def reconcile(w, r, token, keep):
    """How far row r's uniform and top_p must move for the reference to pick
    `token` with kept count `keep`: (du, dp), or None when no move does."""
    x = np.ascontiguousarray(w.logits[r, : w.usable], np.float32)
    prm = np.ascontiguousarray(w.params[r : r + 1])
    rec = None
    nrec = 0
    if w.hist_ids is not None:
        a, b = int(w.hist_offsets[r]), int(w.hist_offsets[r + 1])
        rec = np.ascontiguousarray(w.hist_ids[a:b], np.uint32)
        nrec = b - a
    m = None
    if w.mask is not None and (int(w.params["flags"][r]) & 1):
        m = np.ascontiguousarray(w.mask[r], np.uint32)
    du, dp = ctypes.c_double(), ctypes.c_double()
    rc = lib().or_reconcile(_vp(x), w.usable, _vp(prm), _vp(rec) if nrec else None, nrec, _vp(m),
                            float(w.uniforms[r]), int(token), int(keep), ctypes.byref(du), ctypes.byref(dp))
    return None if rc else (du.value, dp.value)


# ---- JsonObject (constrain.rs), json_oracle.cpp -------------------------------

class JsonOracle:
    """The reference's JsonObject constraint (constrain.rs:88-302)."""

    def __init__(self, _h=None):
        self._h = _h if _h is not None else lib().or_json_new()

    def __del__(self):
        if getattr(self, "_h", None) is not None and _lib is not None:
            _lib.or_json_free(self._h)
            self._h = None

    def clone(self):
        return JsonOracle(lib().or_json_clone(self._h))

    def advance(self, b: bytes):
        lib().or_json_advance(self._h, b, len(b))

    def accepts(self, b: bytes) -> bool:
        return bool(lib().or_json_accepts(self._h, b, len(b)))

    def is_complete(self) -> bool:
        return bool(lib().or_json_is_complete(self._h))

    def mask(self, vocab, usable):
        """allows() for ids [0, usable) as packed u32 words."""
        words = np.zeros((usable + 31) // 32, np.uint32)
        lib().or_json_mask(self._h, _vp(vocab.bytes), _vp(vocab.offsets),
                           None if vocab.special is None else _vp(vocab.special),
                           vocab.n_tokens, usable, _vp(words))
        return words


def json_check(text: bytes):
    """constrain.rs tests' check(): (accepts_bytes, is_complete after advance)."""
    ok, done = ctypes.c_int(), ctypes.c_int()
    lib().or_json_check(text, len(text), ctypes.byref(ok), ctypes.byref(done))
    return bool(ok.value), bool(done.value)


def rmsnorm(x, w, eps):
    """kernels.rs:522-528 per row of x (f32 [t, dim]): the reference's f32 arithmetic."""
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    for i in range(x.shape[0]):
        lib().or_rmsnorm(_vp(x[i]), _vp(w), x.shape[1], float(eps), _vp(out[i]))
    return out


def matmul_bf16(w_bits, x):
    """The Bf16 matmul (weights.rs:230-239): out[i][r] = dot_bf16(W[r], x[i]),
    W as bf16 bit patterns (u16 [rows, dim]), x f32 [t, dim]."""
    w_bits = np.ascontiguousarray(w_bits, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    rows, dim = w_bits.shape
    out = np.empty((x.shape[0], rows), np.float32)
    lib().or_matmul_bf16(_vp(w_bits), rows, dim, _vp(x), x.shape[0], _vp(out), rows)
    return out


def quantize_q8(x):
    """quantize_q8 (kernels.rs:84-100) of one f32 row: (scales f32 [n / 32], values int8 [n])."""
    x = np.ascontiguousarray(x, np.float32)
    sc = np.empty(x.size // 32, np.float32)
    q = np.empty(x.size, np.int8)
    lib().or_quantize_q8(_vp(x), x.size, _vp(sc), _vp(q))
    return sc, q


def matmul_q8(wq, wscale, x):
    """The Q8 matmul (weights.rs:474-560 over Q8Rows): each row of x (f32 [t, dim])
    quantized per 32-value block, then out[i][r] = sum over blocks, in order, of
    (integer block dot) * f16(wscale[r][b]) * xs[i][b].  wq int8 [rows, dim],
    wscale f16 bit patterns u16 [rows, dim / 32]."""
    wq = np.ascontiguousarray(wq, np.int8)
    wscale = np.ascontiguousarray(wscale, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    rows, dim = wq.shape
    out = np.empty((x.shape[0], rows), np.float32)
    lib().or_matmul_q8(_vp(wq), _vp(wscale), rows, dim, _vp(x), x.shape[0], _vp(out), rows)
    return out


def lm_head_q8(x, norm_w, eps, wq, wscale):
    """The output layer of model.rs:700-716 for a Q8 lm_head: rmsnorm, then the Q8 matmul."""
    return matmul_q8(wq, wscale, rmsnorm(x, norm_w, eps))


def lm_head(x, norm_w, eps, w_bits):
    """The output layer of model.rs:700-716 for a Bf16 lm_head: rmsnorm, then the matmul."""
    return matmul_bf16(w_bits, rmsnorm(x, norm_w, eps))
