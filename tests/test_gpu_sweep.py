"""GPU: a seeded sweep of mixed settings against the oracle, at the bar of
tests/parity.py.  Each batch draws a vocabulary size, a logit distribution
(Gaussian of several widths, bf16-like quantized values with many equal
logits, one far outlier per row, a dense cluster over a third of the row),
per-row temperature, top-k (none, inside and beyond the 1024-entry window),
top-p, min-p, penalties and, for some batches, a mask with constrained rows.
Nucleus rows of up to 151,936 candidates take the exact f32 folds.

TSM_SWEEP_FIRST / TSM_SWEEP_LAST (environment) run batches FIRST .. LAST - 1
instead of 0 .. 59, every third one of 12 rows (the split kernel) and the
others of 32: the long runs recorded with the measurements use these."""
import os
import sys

import numpy as np
import pytest

from tachyon_amd.workloads import sweep_batch

pytestmark = pytest.mark.gpu


def test_seeded_sweep_matches_the_oracle():
    import torch

    assert torch.cuda.is_available(), "no GPU"
    from oracle import pyoracle
    from parity import check
    from tachyon_amd.device import SamplerContext, run_workload

    first = int(os.environ.get("TSM_SWEEP_FIRST", 0))
    last = int(os.environ.get("TSM_SWEEP_LAST", 60))
    long_run = "TSM_SWEEP_FIRST" in os.environ or "TSM_SWEEP_LAST" in os.environ
    ctx = SamplerContext(max_rows=32, max_vocab=152064)
    try:
        exact = total = 0
        for k in range(first, last):
            rows = 12 if long_run and k % 3 == 0 else 32
            w, kind = sweep_batch(0x5EE0 + k, rows=rows)
            got = run_workload(ctx, w)
            assert ctx.status() == 0, k
            ref = pyoracle.sample_batch(w, nthreads=16)
            ex, _ = check(w, got, ref, f"sweep batch {k} (V={w.usable}, kind {kind}, rows {rows})")
            exact += ex
            total += rows
            if long_run and k % 500 == 499:
                print(f"[gpu] sweep batch {k}: {exact} of {total} rows bit-exact", flush=True)
        print(f"[gpu] sweep: {exact} of {total} rows bit-exact", flush=True)
        sys.stdout.flush()
    finally:
        ctx.close()
