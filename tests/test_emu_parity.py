"""The HIP kernels' logic on the CPU: the product kernel sources compiled
against the HIP emulation of tests/emu (AddressSanitizer + UBSan, every
"device" array its own exact-size allocation, barriers checked for
divergence), run through the C ABI and held to the same parity bars as the
GPU tests.  This is how a kernel change is checked before it runs on a GPU.
"""
import os

import numpy as np
import pytest

import emu_harness as E
from parity import DIST_CASES, RANDOM_CASES, WINDOW_CASES, check, check_distribution, check_mask_property
from tachyon_amd import workloads as wl

# the small cases run here; the wide ones (vocab >= 20000, and nucleus rows
# over more than 4000 ids, whose exact folds take a minute each on the
# emulation) run with TSM_EMU_ALL=1 -- the GPU suite runs every case
def _wide(c):
    return c["vocab"] >= 20000 or (c.get("mode") == "nucleus" and c["vocab"] > 4000)


FAST = [c for c in RANDOM_CASES if not _wide(c)]
WIDE = [c for c in RANDOM_CASES if _wide(c)]
ALL = os.environ.get("TSM_EMU_ALL") == "1"


@pytest.fixture(scope="module", autouse=True)
def driver():
    return E.build()


def run_case(w, label):
    from oracle import pyoracle

    got = E.emu_sample(w)
    assert got["status"] == 0, got["status"]
    ref = pyoracle.sample_batch(w)
    check(w, got, ref, label)
    check_mask_property(w, got)
    return got, ref


@pytest.mark.parametrize("case", FAST, ids=[f"rand{c['seed']}" for c in FAST])
def test_emu_parity_random(case):
    run_case(wl.random_case(**case), f"emu rand{case['seed']}")


@pytest.mark.skipif(not ALL, reason="wide cases take minutes on the emulation; TSM_EMU_ALL=1 runs them")
@pytest.mark.parametrize("case", WIDE, ids=[f"rand{c['seed']}" for c in WIDE])
def test_emu_parity_random_wide(case):
    run_case(wl.random_case(**case), f"emu rand{case['seed']}")


@pytest.mark.parametrize("case", WINDOW_CASES, ids=[f"window{c['seed']}" for c in WINDOW_CASES])
def test_emu_parity_wide_windows(case):
    """Split-row segments whose candidates would exceed the segment's area
    (regression: such a segment wrote past it, into other segments' entries
    and beyond the scratch) take the exact thresholds instead."""
    run_case(wl.window_case(**case), f"emu window{case['seed']}")


@pytest.mark.parametrize("seed,rows", [(50, 20), (51, 20), (52, 8)])
def test_emu_parity_allowed_below_the_window(seed, rows):
    """Allowed ids only below the window, some valued +0 and -0: the
    fallback's f32::total_cmp order (+0 before -0) against the window's
    (20 rows: the whole-row kernel; 8: the split kernel)."""
    run_case(wl.below_window_case(seed, rows=rows), f"emu below{seed}")


@pytest.mark.parametrize("name,rows", [("c1", 1), ("c2", 8), ("c3", 4), ("c4", 4), ("c5", 4)])
def test_emu_parity_configs(name, rows):
    """The benchmark configurations' shapes at full vocabulary with few rows.  c2's rows come in
    blocks of 8 per kind, so it takes every 4th row of the full batch to
    keep two rows of each kind."""
    if name == "c2":
        full = wl.c2()
        sel = np.arange(0, 32, 4)
        w = wl.Workload("c2s", full.logits[sel], full.usable, full.params[sel], None, None, None,
                        full.uniforms[sel])
        lens = np.diff(full.hist_offsets)[sel]
        off = np.zeros(len(sel) + 1, np.uint32)
        off[1:] = np.cumsum(lens)
        w.hist_ids = np.concatenate([full.hist_ids[full.hist_offsets[r]:full.hist_offsets[r + 1]] for r in sel])
        w.hist_offsets = off
    elif name == "c1":
        w = wl.c1()
    else:
        w = wl.CONFIGS[name](rows=rows)
    run_case(w, f"emu {name}")


def test_emu_distribution():
    from oracle import pyoracle

    for seed, kw in DIST_CASES:
        if not ALL and kw.get("mode") == "nucleus" and kw["vocab"] > 4000:
            continue  # as above: with TSM_EMU_ALL=1
        w = wl.random_case(seed=seed, rows=12, **kw)
        got = E.emu_distribution(w, 1024)
        rids, rps, rkeep = pyoracle.distribution_batch(w, 1024)
        check_distribution(w, got["ids"], got["probs"], got["keep"], rids, rps, rkeep, f"emu dist{seed}")


def test_emu_distribution_whole_kept_set():
    """Kept sets of thousands written whole in chunks of 1024, best first."""
    from oracle import pyoracle

    w = wl.random_case(seed=28, rows=3, vocab=6000, mode="nucleus", sigma=0.5)
    got = E.emu_distribution(w, 8192)
    rids, rps, rkeep = pyoracle.distribution_batch(w, 8192)
    assert (rkeep > 1024).all(), rkeep
    check_distribution(w, got["ids"], got["probs"], got["keep"], rids, rps, rkeep, "emu dist28 whole")
    assert got["status"] & 4 == 0


# Nucleus rows with a dense cluster narrower than a value bin: the fine bins
# of such a coarse bin are laid out from its own sub-histogram, so that no
# fine bin holds more candidates than a census round takes (these rows ended
# with INTERNAL before)
@pytest.mark.parametrize("idx", [0, 1, 2], ids=["sweep193r7", "sweep272r18", "cluster60"])
def test_emu_dense_cluster(idx):
    from oracle import pyoracle

    if idx == 2 and not ALL:
        pytest.skip("eight rows of 151,936 candidates take minutes on the emulation; TSM_EMU_ALL=1 runs them")
    from parity import dense_cluster_workloads

    label, w = dense_cluster_workloads()[idx]
    got = E.emu_sample(w)
    assert got["status"] == 0, got["status"]
    check(w, got, pyoracle.sample_batch(w), f"emu {label}")
