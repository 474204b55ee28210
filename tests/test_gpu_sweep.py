"""GPU: a seeded sweep of mixed settings against the oracle, at the bar of
tests/parity.py.  Each batch draws a vocabulary size, a logit distribution
(Gaussian of several widths, bf16-like quantized values with many equal
logits, one far outlier per row, a dense cluster over a third of the row),
per-row temperature, top-k (none, inside and beyond the 1024-entry window),
top-p, min-p, penalties and, for some batches, a mask with constrained rows.
Nucleus rows of up to 151,936 candidates take the exact f32 folds."""
import sys

import numpy as np
import pytest

from tachyon_amd import workloads as wl

pytestmark = pytest.mark.gpu


def sweep_batch(seed, rows=32):
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
    p = wl.make_params(rows, temperature=1.0, top_k=0, top_p=1.0)
    p["temperature"] = rng.choice([0.3, 0.7, 1.0, 1.5, 3.0], rows).astype(np.float32)
    p["top_p"] = rng.choice([0.5, 0.9, 0.95, 0.99, 1.0], rows).astype(np.float32)
    p["top_k"] = rng.choice([0, 0, 0, 50, 2000, 5000], rows).astype(np.uint32)
    p["presence_penalty"] = np.where(rng.random(rows) < 0.2, 0.3, 0.0).astype(np.float32)
    p["min_p"] = np.where(rng.random(rows) < 0.2, 0.01, 0.0).astype(np.float32)
    p["repetition_penalty"] = np.where(rng.random(rows) < 0.3, 1.1, 1.0).astype(np.float32)
    ids, off = wl.uniform_histories(rng, rows, 64, V)
    mask = None
    if rng.random() < 0.3:
        mask = wl.pack_mask(rng.random((rows, V)) < rng.uniform(0.05, 0.9))
        p["flags"] = np.where(rng.random(rows) < 0.5, wl.ROW_CONSTRAINED, 0).astype(np.uint32)
    return wl.Workload(f"sweep{seed}", x, V, p, ids, off, mask, wl.uniforms(rng, rows)), kind


def test_seeded_sweep_matches_the_oracle():
    import torch

    assert torch.cuda.is_available(), "no GPU"
    from oracle import pyoracle
    from parity import check
    from tachyon_amd.device import SamplerContext, run_workload

    ctx = SamplerContext(max_rows=32, max_vocab=152064)
    try:
        exact = 0
        for k in range(60):
            w, kind = sweep_batch(0x5EE0 + k)
            got = run_workload(ctx, w)
            assert ctx.status() == 0, k
            ref = pyoracle.sample_batch(w, nthreads=16)
            ex, _ = check(w, got, ref, f"sweep batch {k} (V={w.usable}, kind {kind})")
            exact += ex
        print(f"[gpu] sweep: {exact} of {60 * 32} rows bit-exact", flush=True)
        sys.stdout.flush()
    finally:
        ctx.close()
