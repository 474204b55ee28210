"""The JSON-object constraint's automaton of the product library
(tsm_json_init / _advance / _accepts / _is_complete: host functions of the C
ABI, no GPU needed) against the oracle's restatement of constrain.rs, on the
reference's own test texts, the hand-derived limits, random JSON prefixes
and random bytes fed through advance()."""
import numpy as np

from oracle import pyoracle
from tachyon_amd import workloads as wl
from tachyon_amd.constrain import JsonConstraint
from test_oracle import JSON_INVALID, JSON_PREFIXES, JSON_VALID


def product_check(text: bytes):
    c = JsonConstraint()
    ok = c.accepts(text)
    c.advance(text)
    return ok, c.is_complete()


def test_reference_texts():
    for t in JSON_VALID + JSON_PREFIXES + JSON_INVALID + [b"{" + b" " * 40, b'{"a": ' + b"1" * 41]:
        assert product_check(t) == pyoracle.json_check(t), t


def test_states_from_random_prefixes_accept_like_the_oracle():
    toks, _ = wl.json_vocab(4000, seed=3)
    frags = toks[256:]
    rng = np.random.default_rng(5)
    for p in wl.json_prefixes(120, seed=9):
        c, o = JsonConstraint(), pyoracle.JsonOracle()
        c.advance(p)
        o.advance(p)
        assert c.is_complete() == o.is_complete(), p
        for t in [bytes([b]) for b in range(256)] + [frags[i] for i in rng.integers(0, len(frags), 200)]:
            assert c.accepts(t) == o.accepts(t), (p, t)


def test_advance_through_rejected_bytes_matches():
    """advance() keeps stepping past a byte the automaton rejects
    (constrain.rs:292-296): the states must still agree afterwards."""
    rng = np.random.default_rng(11)
    probes = [bytes([b]) for b in range(256)] + [b'"a":1', b"]", b"}", b"1e5", b'\\u12']
    for k in range(300):
        junk = bytes(rng.integers(0, 256, int(rng.integers(1, 30))).astype(np.uint8).tolist())
        if k % 3 == 0:  # mostly JSON bytes
            junk = bytes(rng.choice(list(b'{}[]",:0123456789.eE+- \\utrufalsn'), len(junk)).astype(np.uint8).tolist())
        c, o = JsonConstraint(), pyoracle.JsonOracle()
        for chunk in (b"{", junk):
            c.advance(chunk)
            o.advance(chunk)
        assert c.is_complete() == o.is_complete()
        for t in probes:
            assert c.accepts(t) == o.accepts(t), (junk, t)


def test_mask_set_on_the_cpu_emulation():
    """The mask producer's sources on the CPU emulation (AddressSanitizer):
    tsm_json_masks_fill against tsm_json_mask and the host stepping of
    tsm_json_accepts, over calls that hit, miss and overflow a set keeping 4
    states, a changed vocabulary and a set keeping nothing, with the call
    counts (distinct, kept, evaluated) each call must report."""
    import subprocess

    import emu_harness as E

    exe = E.build("emu_mask")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0 and "ok" in r.stdout, r.stderr[-3000:]
