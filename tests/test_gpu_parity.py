"""GPU parity: the HIP sampling path against the CPU oracle on identical
seeded logits, histories, masks and uniforms, through the C ABI.

Bars (tests/parity.py):
* every row: token, kept count and pick probability bit-exact with the
  reference's arithmetic (rows of more than 1024 candidates included: the
  device reproduces the reference's sequential f32 folds).  A differing row
  would pass only if the reference itself returns it after u moves by at
  most 1e-5 and top_p by at most 1e-5, measured with the oracle's own f32
  arithmetic (or_reconcile);
* logprobs and top-n logprobs within 1e-5 relative / 1e-6 absolute, top-n
  ids bit-exact; NaN matches NaN.
"""
import ctypes
import os
import sys

import numpy as np
import pytest

from tachyon_amd import workloads as wl

pytestmark = pytest.mark.gpu

from parity import DIST_CASES, RANDOM_CASES, WINDOW_CASES, check, check_distribution, check_mask_property


def say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


CTX_VOCAB = 152064


@pytest.fixture(scope="module")
def ctx():
    import torch

    assert torch.cuda.is_available(), "no GPU"
    from tachyon_amd.device import SamplerContext

    c = SamplerContext(max_rows=1024, max_vocab=CTX_VOCAB)
    yield c
    c.close()


def run_case(ctx, w, label, nthreads=16):
    from oracle import pyoracle
    from tachyon_amd.device import run_workload

    say(f"[gpu] {label}: rows={w.rows} V={w.usable} stride={w.row_stride}")
    got = run_workload(ctx, w)
    assert ctx.status() == 0
    ref = pyoracle.sample_batch(w, nthreads=nthreads)
    exact_rows, boundary = check(w, got, ref, label)
    say(f"[gpu] {label}: ok, bit-exact rows {exact_rows}/{w.rows}, within the measured 1e-5 boundary {boundary}")
    return got, ref


# ---------------------------------------------------------------------------

def test_device_expf_matches_glibc(ctx):
    """The device restatement of glibc expf, bit for bit, on a strided sweep of
    every float in [-104, 89], the range edges and special values."""
    import torch

    from oracle import pyoracle

    helper = os.path.join(os.path.dirname(__file__), "helpers", "libtsm_probe.so")
    L = ctypes.CDLL(helper)
    L.tsm_probe_expf.restype = ctypes.c_int
    L.tsm_probe_expf.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_uint32, ctypes.c_void_p]
    neg = np.arange(0x80000000, 0xC2D00000, 97, dtype=np.uint64).astype(np.uint32).view(np.float32)
    pos = np.arange(0, 0x42B20000, 97, dtype=np.uint64).astype(np.uint32).view(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 88.0, -88.0, 88.72283, 88.72284, -103.97208, -103.97207,
                        float.fromhex('0x1.04845ep+5'), float.fromhex('-0x1.f8cbb2p+5'), 1e-30, -1e-30, -87.33655, -87.3366], np.float32)
    x = np.concatenate([neg, pos, special]).astype(np.float32)
    say(f"[gpu] expf sweep over {x.size} inputs")
    xd = torch.from_numpy(x).cuda()
    yd = torch.empty_like(xd)
    assert L.tsm_probe_expf(ctypes.c_void_p(xd.data_ptr()), ctypes.c_void_p(yd.data_ptr()), x.size,
                            ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
    torch.cuda.synchronize()
    got = yd.cpu().numpy()
    ref = pyoracle.expf_array(x)
    bad = np.nonzero(got.view(np.uint32) != ref.view(np.uint32))[0]
    assert bad.size == 0, [(float(x[i]), float(got[i]), float(ref[i])) for i in bad[:5]]


@pytest.mark.parametrize("case", RANDOM_CASES, ids=[f"rand{c['seed']}" for c in RANDOM_CASES])
def test_parity_random(ctx, case):
    from tachyon_amd.device import SamplerContext

    w = wl.random_case(**case)
    if w.usable <= CTX_VOCAB:
        run_case(ctx, w, f"rand{case['seed']}")
        return
    big = SamplerContext(max_rows=w.rows, max_vocab=w.usable)  # vocabularies past the shared context's
    try:
        run_case(big, w, f"rand{case['seed']}")
    finally:
        big.close()


@pytest.mark.parametrize("case", WINDOW_CASES, ids=[f"window{c['seed']}" for c in WINDOW_CASES])
def test_parity_wide_windows(ctx, case):
    """Top-k windows near 1024 over small vocabularies: split-row segments
    whose candidates exceed the segment's area take the exact thresholds."""
    run_case(ctx, wl.window_case(**case), f"window{case['seed']}")


def test_parity_dense_clusters(ctx):
    """Nucleus rows whose dense cluster once overflowed a census round
    (sweep batches 193 and 272) and eight synthetic rows of that kind."""
    from parity import dense_cluster_workloads

    for label, w in dense_cluster_workloads():
        run_case(ctx, w, label)


def test_parity_allowed_below_the_window(ctx):
    """Constrained top-k rows whose allowed ids all rank below the window
    (sampler.rs:211-221: the best allowed ids of the whole row by
    f32::total_cmp), some with +0 and -0 among the kept values."""
    for seed, rows in ((50, 20), (51, 20), (52, 8)):
        run_case(ctx, wl.below_window_case(seed, rows=rows), f"below{seed}")


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4"])
def test_parity_baseline_configs(ctx, name):
    w = wl.CONFIGS[name]()
    got, ref = run_case(ctx, w, name)
    check_mask_property(w, got)


def _rows_of(w, sel, name):
    """The rows `sel` of workload w (with their histories) as a workload."""
    hist_ids = hist_off = None
    if w.hist_offsets is not None:
        lens = np.diff(w.hist_offsets.astype(np.int64))[sel]
        hist_off = np.zeros(len(sel) + 1, np.uint32)
        hist_off[1:] = np.cumsum(lens)
        hist_ids = np.concatenate([w.hist_ids[w.hist_offsets[r]:w.hist_offsets[r + 1]] for r in sel]).astype(np.uint32)
    return wl.Workload(name, np.ascontiguousarray(w.logits[sel]), w.usable, w.params[sel].copy(), hist_ids, hist_off,
                       None if w.mask is None else np.ascontiguousarray(w.mask[sel]), w.uniforms[sel].copy(),
                       top_stride=w.top_stride)


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4"])
@pytest.mark.parametrize("kinds", [True, False], ids=["kinds", "nokinds"])
def test_parity_split_path(ctx, name, kinds):
    """Batches of at most 16 rows take the split-row kernel for their top-k
    rows: the benchmark configurations' shapes at full vocabulary, 16 rows (c2: two of each
    row kind), with the batch's row kinds given and left unknown."""
    from oracle import pyoracle
    from tachyon_amd.device import run_workload

    full = wl.CONFIGS[name]()
    sel = np.arange(0, full.rows, max(1, full.rows // 16))[:16] if name != "c2" else np.array(
        [0, 1, 8, 9, 16, 17, 24, 25])
    w = _rows_of(full, sel, f"{name}s")
    say(f"[gpu] split path {name}: rows={w.rows} kinds={kinds}")
    got = run_workload(ctx, w, kinds=kinds)
    assert ctx.status() == 0
    ref = pyoracle.sample_batch(w, nthreads=16)
    exact_rows, boundary = check(w, got, ref, f"split {name}")
    check_mask_property(w, got)
    say(f"[gpu] split path {name}: ok, bit-exact rows {exact_rows}/{w.rows}, within the boundary {boundary}")


def test_split_path_row_kind_mismatch(ctx):
    """A small batch that names only the split kind but holds a row without
    top-k: that row is not sampled and the status says so; the others are."""
    from oracle import pyoracle
    from tachyon_amd import _lib
    from tachyon_amd.device import Outputs, upload

    w = wl.random_case(seed=41, vocab=3000, rows=6, mode="topk")
    w.params["top_k"][3] = 0  # no top-k: the whole-row kind
    b = upload(w)
    b.row_kinds = _lib.ROWKIND_SPLIT
    out = Outputs(w.rows, w.top_stride)
    ctx.sample(b, out)
    got = out.numpy()
    assert ctx.status() & 16  # TSM_STATUS_ROW_KIND
    ref = pyoracle.sample_batch(w)
    for r in range(w.rows):
        if r != 3:
            assert got["token"][r] == ref.token[r], r


def test_parity_c5_nucleus(ctx):
    w = wl.c5()
    run_case(ctx, w, "c5")


def test_repeat_calls_are_identical(ctx):
    """The context's scratch carries nothing between calls."""
    from tachyon_amd.device import run_workload

    w = wl.c4(rows=64)
    a = run_workload(ctx, w)
    w2 = wl.random_case(seed=99, vocab=w.usable, rows=32, masked=True)
    run_workload(ctx, w2)
    b = run_workload(ctx, w)
    for k in a:
        assert np.array_equal(a[k], b[k]), k


def test_distribution_parity(ctx):
    import torch

    from oracle import pyoracle
    from tachyon_amd.device import upload

    ctx.status()  # clears what earlier calls left
    for seed, kw in DIST_CASES:
        w = wl.random_case(seed=seed, rows=12, **kw)
        say(f"[gpu] distribution seed {seed}")
        b = upload(w)
        ids, ps, keep = ctx.distribution(b, 1024)
        torch.cuda.synchronize()
        ids, ps, keep = ids.cpu().numpy().view(np.uint32), ps.cpu().numpy(), keep.cpu().numpy().view(np.uint32)
        rids, rps, rkeep = pyoracle.distribution_batch(w, 1024)
        check_distribution(w, ids, ps, keep, rids, rps, rkeep, f"dist{seed}")
        # a kept set beyond the written entries is reported
        st = ctx.status()
        assert bool(st & 4) == bool((rkeep > 1024).any()), (seed, st)


@pytest.mark.parametrize("seed,vocab,stride", [(28, 6000, 8192), (32, 40000, 16384), (33, 151936, 4096)])
def test_distribution_parity_whole_kept_set(ctx, seed, vocab, stride):
    """Kept sets of thousands of candidates (nucleus rows over N(0, 0.5^2)
    logits) written whole, best first, up to the stride: every entry equals
    the oracle's Sampler::distribution; the truncation bit is set exactly when
    a kept count exceeds the stride."""
    import torch

    from oracle import pyoracle
    from tachyon_amd.device import upload

    ctx.status()
    w = wl.random_case(seed=seed, rows=6, vocab=vocab, mode="nucleus", sigma=0.5)
    say(f"[gpu] distribution seed {seed}: V={vocab}, stride {stride}")
    ids, ps, keep = ctx.distribution(upload(w), stride)
    torch.cuda.synchronize()
    ids, ps, keep = ids.cpu().numpy().view(np.uint32), ps.cpu().numpy(), keep.cpu().numpy().view(np.uint32)
    rids, rps, rkeep = pyoracle.distribution_batch(w, stride)
    assert (rkeep > 1024).all(), rkeep  # every row's kept set is beyond one chunk
    check_distribution(w, ids, ps, keep, rids, rps, rkeep, f"dist{seed}")
    assert bool(ctx.status() & 4) == bool((rkeep > stride).any()), seed


def test_abi_rejects_bad_arguments(ctx):
    import torch

    from tachyon_amd import _lib
    from tachyon_amd.device import Outputs, upload

    w = wl.random_case(seed=31, vocab=100, rows=4)
    b = upload(w)
    out = Outputs(4, 20)
    ctx.sample(b, out)  # fine
    b.usable = 200  # > row_stride
    with pytest.raises(_lib.TsmError, match="exceeds row_stride"):
        ctx.sample(b, out)
    b.usable = 100
    b.mask = torch.zeros(4, 1, dtype=torch.int32, device="cuda")  # stride 1 < ceil(100/32)
    with pytest.raises(_lib.TsmError, match="mask_stride"):
        ctx.sample(b, out)
