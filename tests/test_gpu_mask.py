"""GPU: the mask producer (tsm_json_mask) against the oracle's JsonObject
(constrain.rs) token by token, and its masks consumed by tsm_sample.

Bar: every allow-bit equal to `allows(tok, id)` of the reference's automaton
(not special, has bytes, accepts_bytes), bits at or above `usable` zero, and
sampled rows that use a produced mask equal to the oracle's with that mask.
"""
import sys

import numpy as np
import pytest

from tachyon_amd import workloads as wl

pytestmark = pytest.mark.gpu


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def vocab():
    import torch

    assert torch.cuda.is_available(), "no GPU"
    from tachyon_amd.constrain import DeviceVocab, HostVocab

    toks, special = wl.json_vocab(wl.QWEN_VOCAB, seed=0x15A0)
    hv = HostVocab.from_tokens(toks, special)
    return hv, DeviceVocab(hv)


def produce(dv, states, usable, mask_stride):
    import torch

    from tachyon_amd.constrain import json_mask, pack_states

    st = torch.from_numpy(pack_states(states)).cuda()
    mask = torch.full((len(states), mask_stride), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
    json_mask(dv, st, len(states), usable, mask, mask_stride)
    torch.cuda.synchronize()
    return mask.cpu().numpy().view(np.uint32)


def states_for(prefixes):
    from oracle import pyoracle
    from tachyon_amd.constrain import JsonConstraint

    cs, os_ = [], []
    for p in prefixes:
        c, o = JsonConstraint(), pyoracle.JsonOracle()
        c.advance(p)
        o.advance(p)
        cs.append(c)
        os_.append(o)
    return cs, os_


def test_json_mask_matches_the_oracle(vocab):
    """48 random JSON prefixes (seed 0x15A1); TSM_MASK_ROUNDS (environment)
    adds rounds of 48 more, seeds 0x15A1 + 1, ..., for long runs."""
    import os

    hv, dv = vocab
    usable = hv.n_tokens
    stride = (usable + 31) // 32 + 3  # a wider stride: the extra words are not written
    nw = (usable + 31) // 32
    rounds = int(os.environ.get("TSM_MASK_ROUNDS", 1))
    for k in range(rounds):
        prefixes = wl.json_prefixes(48, seed=0x15A1 + k)
        cs, os_ = states_for(prefixes)
        say(f"[gpu] json mask round {k}: {len(cs)} rows x {usable} tokens")
        got = produce(dv, cs, usable, stride)
        for r, o in enumerate(os_):
            ref = o.mask(hv, usable)
            bad = np.nonzero(got[r, :nw] != ref)[0]
            assert bad.size == 0, (k, r, prefixes[r], bad[:5], got[r, bad[:5]], ref[bad[:5]])
            assert (got[r, nw:] == 0x5A5A5A5A).all()
    allowed = [int(np.unpackbits(got[r, :nw].view(np.uint8)).sum()) for r in range(len(cs))]
    say(f"[gpu] json mask: bit-exact; allowed per row min {min(allowed)} max {max(allowed)}")


def test_json_mask_usable_and_tokenizer_length(vocab):
    """usable below the tokenizer's length cuts the row (bits past it zero);
    ids past the tokenizer's length have no bytes and are never allowed."""
    from tachyon_amd.constrain import DeviceVocab, HostVocab

    hv, dv = vocab
    cs, os_ = states_for([b"", b'{"a": "x', b'{"a": [1, 2'])
    for usable in (1, 31, 33, 1000, 4097):
        got = produce(dv, cs, usable, (usable + 31) // 32)
        for r, o in enumerate(os_):
            assert (got[r] == o.mask(hv, usable)).all(), (usable, r)
    toks, special = wl.json_vocab(5000, seed=7)
    hv2 = HostVocab.from_tokens(toks, special)
    dv2 = DeviceVocab(hv2)
    got = produce(dv2, cs, 6000, (6000 + 31) // 32)
    for r, o in enumerate(os_):
        ref = np.zeros((6000 + 31) // 32, np.uint32)
        ref[:(5000 + 31) // 32] = o.mask(hv2, 5000)
        assert (got[r] == ref).all(), r


def test_produced_masks_drive_sampling(vocab):
    """A step of constrained rows whose masks come from the producer: the
    GPU's tokens equal the oracle's with the same masks, and each pick is
    allowed."""
    from oracle import pyoracle
    from parity import check, check_mask_property
    from tachyon_amd.device import SamplerContext, run_workload

    hv, dv = vocab
    prefixes = wl.json_prefixes(32, seed=0x15A2)
    cs, _ = states_for(prefixes)
    V = hv.n_tokens
    masks = produce(dv, cs, V, (V + 31) // 32)
    rng = np.random.default_rng(0x15A3)
    rows = len(cs)
    x = (rng.standard_normal((rows, V)) * 3.0).astype(np.float32)
    p = wl.make_params(rows, temperature=0.8, top_k=40, top_p=0.9, flags=wl.ROW_CONSTRAINED | wl.ROW_LOGPROBS,
                       n_logprobs=3)
    p["top_k"][::4] = 0  # some rows without top-k: the cutoff path with a mask
    w = wl.Workload("jsonmask", x, V, p, None, None, np.ascontiguousarray(masks), wl.uniforms(rng, rows),
                    top_stride=3)
    ctx = SamplerContext(max_rows=rows, max_vocab=V)
    try:
        got = run_workload(ctx, w)
        assert ctx.status() == 0
    finally:
        ctx.close()
    ref = pyoracle.sample_batch(w, nthreads=16)
    exact, _ = check(w, got, ref, "json-mask step")
    check_mask_property(w, got)
    say(f"[gpu] sampling with produced masks: bit-exact rows {exact}/{rows}")


def test_json_mask_rejects_bad_arguments(vocab):
    import torch

    from tachyon_amd import _lib
    from tachyon_amd.constrain import json_mask, pack_states, JsonConstraint

    hv, dv = vocab
    st = torch.from_numpy(pack_states([JsonConstraint()])).cuda()
    mask = torch.zeros(1, 8, dtype=torch.int32, device="cuda")
    with pytest.raises(_lib.TsmError, match="mask_stride"):
        json_mask(dv, st, 1, 1000, mask, 8)
    with pytest.raises(_lib.TsmError, match="rows"):
        json_mask(dv, st, 0, 100, mask, 8)


def state_key(c):
    """A state's identity: its packed bytes without the padding."""
    return c.packed()[:9]


def test_json_mask_set_matches_the_direct_producer(vocab):
    """tsm_json_masks_fill writes every row's mask equal to tsm_json_mask's for
    the same state, over calls that hit, miss and overflow the kept masks:
    first call 80 rows of ~40 states into a set keeping 8 (the first 8
    distinct states get slots, the rest are evaluated straight into their
    rows), then a call of 3 kept states and 5 new ones, then the same rows
    again, a set keeping nothing, and a new vocabulary (nothing reused)."""
    import torch

    from tachyon_amd.constrain import DeviceVocab, JsonConstraint, JsonMaskSet

    hv, dv = vocab
    V = hv.n_tokens
    nw = (V + 31) // 32
    stride = nw + 2
    prefixes = wl.json_prefixes(48, seed=0x15A6)
    cs, _ = states_for(prefixes)
    rng = np.random.default_rng(0x15A7)
    rows1 = [cs[i] for i in rng.integers(0, len(cs), 80)]
    # a state with stray padding bytes is the same state
    odd = JsonConstraint()
    odd.advance(prefixes[5])
    odd.state.pad[0] = 0xAB
    rows1[-1] = odd

    def distinct(rows):
        keys = []
        for c in rows:
            if state_key(c) not in keys:
                keys.append(state_key(c))
        return keys

    def fill(ms, rows, vocab_dev=dv):
        mask = torch.full((len(rows), stride), 0x5A5A5A5A, dtype=torch.int32, device="cuda")
        st = ms.fill(vocab_dev, rows, mask, stride)
        torch.cuda.synchronize()
        return mask.cpu().numpy().view(np.uint32), st

    def check_rows(got, rows):
        ref = produce(dv, rows, V, stride)
        for r in range(len(rows)):
            bad = np.nonzero(got[r, :nw] != ref[r, :nw])[0]
            assert bad.size == 0, (r, bad[:5])
            assert (got[r, nw:] == 0x5A5A5A5A).all(), r

    ms = JsonMaskSet(max_rows=128, capacity=8, usable=V)
    try:
        k1 = distinct(rows1)
        say(f"[gpu] mask set: call 1, {len(rows1)} rows, {len(k1)} states, 8 kept")
        got, st = fill(ms, rows1)
        check_rows(got, rows1)
        assert st == (80, len(k1), 0, len(k1)), st
        # the first 8 distinct states of call 1 hold the slots
        first = {k: next(c for c in rows1 if state_key(c) == k) for k in k1}
        kept = [first[k] for k in k1[:3]]
        others, _ = states_for(wl.json_prefixes(96, seed=0x15A8))
        fresh, seen = [], set(k1)
        for c in others:
            if state_key(c) not in seen:
                seen.add(state_key(c))
                fresh.append(c)
        fresh = fresh[:5]
        assert len(fresh) == 5
        # the kept states first: each new state then takes the slot of one of
        # call 1's states 4-8, the least recently used
        rows2 = [kept[0], kept[1], kept[2], fresh[0], kept[0], fresh[1], fresh[2], fresh[3], fresh[4], fresh[0]]
        say("[gpu] mask set: call 2, 10 rows, 3 kept states and 5 new")
        got, st = fill(ms, rows2)
        check_rows(got, rows2)
        assert st == (10, 8, 3, 5), st
        say("[gpu] mask set: call 3, call 2's rows again")
        got, st = fill(ms, rows2)
        check_rows(got, rows2)
        assert st == (10, 8, 8, 0), st
        # another vocabulary (other device pointers): nothing is reused
        dv2 = DeviceVocab(hv)
        got, st = fill(ms, rows2, dv2)
        check_rows(got, rows2)
        assert st == (10, 8, 0, 8), st
    finally:
        ms.close()
    ms0 = JsonMaskSet(max_rows=128, capacity=0, usable=V)
    try:
        say("[gpu] mask set: capacity 0, call 1's rows")
        got, st = fill(ms0, rows1)
        check_rows(got, rows1)
        assert st == (80, len(k1), 0, len(k1)), st
        got, st = fill(ms0, rows1[:7])
        check_rows(got, rows1[:7])
        assert st[2] == 0, st
    finally:
        ms0.close()


def test_json_mask_set_rejects_bad_arguments(vocab):
    import torch

    from tachyon_amd import _lib
    from tachyon_amd.constrain import JsonConstraint, JsonMaskSet

    hv, dv = vocab
    with pytest.raises(_lib.TsmError, match="max_rows"):
        JsonMaskSet(max_rows=0, capacity=4, usable=100)
    ms = JsonMaskSet(max_rows=4, capacity=4, usable=1000)
    try:
        mask = torch.zeros(8, 40, dtype=torch.int32, device="cuda")
        with pytest.raises(_lib.TsmError, match="rows"):
            ms.fill(dv, [JsonConstraint()] * 5, mask, 40)
        with pytest.raises(_lib.TsmError, match="mask_stride"):
            ms.fill(dv, [JsonConstraint()], mask, 31)
    finally:
        ms.close()
