#!/usr/bin/env python3
"""Benchmark of the batched sampling path on one MI355X.

A step is one tsm_sample() call over one batch of synthetic logits already
resident in HBM: one launch of the kernel that takes the batch's rows
(topk_kernel for c3 and c4, whose rows are all of the lean kind;
sample_kernel for c5; both for c2's mixed rows; split_kernel for c1).  The default workload is the benchmark
config c4, the headline: B=256, V=151936, repetition 1.1 + presence 0.4 +
frequency 0.2 over 1024-token Zipf histories, a 30% grammar mask, T=0.7,
top_k=64, top_p=0.92, min_p=0.02 and top-5 logprobs.

Input sets are rotated (3 sets of 161.5 MB > the 256 MB Infinity Cache) so
repeat reads cannot be served from MALL.  GPU time comes from HIP events on
the stream the kernels run on: `value` and `ms_per_step` from K steps with one
event per step (a step then also holds the gap from one launch to the next),
`roofline.achieved` from the same K launches each between two events (the
kernel's own duration, `roofline.kernel_avg_us`).  The CPU baseline is the
oracle restatement of the reference sampler, timed on this host's cores on the
same workload; its results for input set 0 also check the GPU's tokens (after
the timed region).  ``roofline.traffic`` comes from
``profiles/traffic_<config>.json`` (rocprofv3 FETCH_SIZE / WRITE_SIZE passes,
tachyon_amd/traffic.py) only when that file was measured on the library
loaded here (same SHA-256); otherwise it is null.

Prints ONE JSON line.

``--calib-copy-mb N`` instead runs a few device-to-device copies of N MiB
(reads and writes exactly N MiB each): the run that fixes the scale of the
rocprofv3 FETCH_SIZE / WRITE_SIZE counters for tachyon_amd/traffic.py.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "sampled rows/s + HBM GB/s (% of peak), B=256 V=151936 full pipeline"
HBM_PEAK_GBS = 8000.0
SEEDS = {"c1": 0x5EED0001, "c2": 0x5EED0002, "c3": 0x5EED0003, "c4": 0x5EED0004, "c5": 0x5EED0005}
DESCR = {
    "c1": "c1: B=1 V=151936, k=40 p=.9 T=.7 R=1.1/64",
    "c2": "c2: B=32 V=151936 mixed rows, presence .5 frequency .3 over 512 Zipf",
    "c3": "c3: B=256 V=128256 mask log-U(0.1%-60%), k=40 p=.9 T=.8, top-20 logprobs",
    "c4": "c4: B=256 V=151936 full pipeline: R=1.1+pres .4+freq .2 over 1024 Zipf, 30% mask, "
          "T=.7 k=64 p=.92 min_p=.02, top-5 logprobs",
    "c5": "c5: B=1024 V=151936 nucleus p=.98 T=1.2 no top-k, R=1.05/256",
}

# kernels a step launches (batches of up to 16 rows take the split-row kernel
# for their top-k rows)
KERNELS = {
    "c1": "split_kernel (one launch per tsm_sample step)",
    "c2": "topk_kernel + sample_kernel (two launches per tsm_sample step: lean and general rows)",
    "c3": "topk_kernel (one launch per tsm_sample step: every row of the lean kind)",
    "c4": "topk_kernel (one launch per tsm_sample step: every row of the lean kind)",
    "c5": "sample_kernel (one launch per tsm_sample step)",
}


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def cpu_model():
    """The host CPU's model name (/proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def oracle_check(w, got_tokens, threads):
    """Rows of input set 0 whose GPU token equals the oracle's."""
    from oracle import pyoracle

    ref = pyoracle.sample_batch(w, nthreads=threads)
    same = int((ref.token == got_tokens).sum())
    return {"rows": int(w.rows), "token_equal": same}


def cpu_baseline(w, budget_s, threads):
    """Oracle rows/s on host cores (reported baseline, not the target)."""
    from oracle import pyoracle

    pyoracle.sample_batch(w, nthreads=threads)  # warm-up
    t0 = time.perf_counter()
    steps = 0
    while True:
        pyoracle.sample_batch(w, nthreads=threads)
        steps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or steps >= 1000:
            break
    return w.rows * steps / el, steps, el


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="c4", choices=sorted(SEEDS))
    ap.add_argument("--sets", type=int, default=3, help="rotated input sets")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true", help="no CPU baseline")
    ap.add_argument("--no-check", action="store_true", help="no check of set 0's tokens against the oracle")
    ap.add_argument("--json-mask", action="store_true",
                    help="time the mask producer (tsm_json_mask) instead: 256 JsonObject rows over a "
                         "151936-token synthetic vocabulary")
    ap.add_argument("--mask-mode", default="direct", choices=["direct", "dedupe", "cached", "decode"],
                    help="with --json-mask: direct = tsm_json_mask on every row; dedupe = a mask set keeping "
                         "nothing (each distinct state of a step evaluated once); cached = a mask set keeping "
                         "1024 states, the same rows every step; decode = a mask set keeping 1024 states, "
                         "each row advancing through its own document by one 4-byte token per step")
    ap.add_argument("--lm-head", action="store_true",
                    help="time the logits producer (tsm_lm_head) instead: 256 rows, dim 4096, vocab 151936, "
                         "bf16 weights")
    ap.add_argument("--lm-rows", type=int, default=256, help="with --lm-head: logit rows per call (256: the c4 batch)")
    ap.add_argument("--lm-bf16", action="store_true",
                    help="with --lm-head: activations rounded to bf16 (default: the hi/lo split)")
    ap.add_argument("--lm-q8", action="store_true",
                    help="with --lm-head: a Q8 lm_head (tsm_lm_head_q8: int8 weights, an f16 scale per 32)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="run N MiB device copies for counter calibration instead of the bench")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch

    if args.calib_copy_mb:
        n = args.calib_copy_mb << 20
        src = torch.empty(n, dtype=torch.uint8, device="cuda").random_(0, 255)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copied {args.calib_copy_mb} MiB x5")
        return

    if args.lm_head:
        if args.lm_q8:
            bench_lm_head_q8(args)
        else:
            bench_lm_head(args)
        return
    if args.json_mask:
        bench_json_mask(args)
        return

    from tachyon_amd import workloads as wl
    from tachyon_amd.device import Outputs, SamplerContext, upload

    gen = wl.CONFIGS[args.config]
    log(f"[bench] generating {args.sets} input sets of {args.config}")
    sets = [gen(seed=SEEDS[args.config] + 17 * i) for i in range(args.sets)]
    w0 = sets[0]
    rows, vocab = w0.rows, w0.usable
    batches = [upload(w) for w in sets]
    out = Outputs(rows, max(1, w0.top_stride))
    ctx = SamplerContext(rows, vocab)
    torch.cuda.synchronize()

    log(f"[bench] warmup {args.warmup}")
    for i in range(args.warmup):
        ctx.sample(batches[i % len(batches)], out)
    torch.cuda.synchronize()
    assert ctx.status() == 0

    log(f"[bench] timing {args.steps} steps")
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev[0].record()
    for i in range(args.steps):
        ctx.sample(batches[i % len(batches)], out)
        ev[i + 1].record()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    per = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(args.steps))
    total_ms = ev[0].elapsed_time(ev[-1])
    ms_step = total_ms / args.steps
    med_ms = per[len(per) // 2]

    # the kernel's own duration: the same launches, each between two events on
    # its stream (the steps above also hold the gap from one launch to the
    # next); the roofline is priced on this
    log(f"[bench] timing {args.steps} launches between event pairs")
    ea = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    eb = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    torch.cuda.synchronize()
    for i in range(args.steps):
        ea[i].record()
        ctx.sample(batches[i % len(batches)], out)
        eb[i].record()
    torch.cuda.synchronize()
    kern_ms = sum(ea[i].elapsed_time(eb[i]) for i in range(args.steps)) / args.steps

    alg_bytes = w0.algorithmic_bytes()
    achieved = alg_bytes / (kern_ms * 1e-3) / 1e9
    rows_s = rows / (ms_step * 1e-3)

    # outside the timed region: set 0's tokens against the oracle
    check = None
    if not args.no_check:
        ctx.sample(batches[0], out)
        torch.cuda.synchronize()
        assert ctx.status() == 0
        got = out.numpy()["token"]
        log("[bench] checking set 0's tokens against the oracle")
        check = oracle_check(w0, got, min(16, len(os.sched_getaffinity(0))))

    from tachyon_amd import _lib
    from tachyon_amd.traffic import library_sha256

    traffic = None
    traffic_note = None
    lib_sha = library_sha256(_lib.LIB_PATH)
    tfile = os.path.join(ROOT, "profiles", f"traffic_{args.config}.json")
    if os.path.exists(tfile):
        with open(tfile) as fh:
            tj = json.load(fh)
        if tj.get("library_sha256") == lib_sha:
            traffic = tj.get("hbm_bytes_per_step")
        else:
            traffic_note = f"profiles/traffic_{args.config}.json was measured on another build of the library"

    cpu = None
    if not args.no_cpu:
        ref_threads = min((rows + 3) // 4, 4)  # src/scheduler.rs:665-675
        log(f"[bench] cpu baseline: oracle, {ref_threads} threads, ~{args.cpu_seconds}s")
        v, steps, el = cpu_baseline(w0, args.cpu_seconds, ref_threads)
        ncores = len(os.sched_getaffinity(0))
        v_all, steps_all, el_all = cpu_baseline(w0, args.cpu_seconds / 2, ncores)
        cpu = {"value": round(v, 1), "unit": "rows/s", "cores": ref_threads, "kind": "port",
               "cpu_model": cpu_model(),
               "sample": f"{steps} full {args.config} batches ({steps * rows} rows) in {el:.1f}s with the "
                         f"reference's own row parallelism (min(ceil(B/4),4) threads)",
               "all_cores": {"value": round(v_all, 1), "cores": ncores, "sample": f"{steps_all * rows} rows"}}

    rec = {
        "metric": METRIC,
        "value": round(rows_s, 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": DESCR[args.config], "rows": rows, "vocab": vocab, "input_sets": len(sets),
                   "median_ms_per_step": round(med_ms, 5), "wall_s": round(wall, 3)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes_per_step": alg_bytes, "kernel_avg_us": round(kern_ms * 1e3, 2),
                     "kernel": KERNELS[args.config], "library_sha256": lib_sha[:16]},
        "cpu_baseline": cpu,
        "oracle_check": check,
    }
    if traffic_note:
        rec["roofline"]["traffic_note"] = traffic_note
    ctx.close()
    print(json.dumps(rec), flush=True)


def bench_json_mask(args):
    """One step of the mask producer: 256 rows in states from random JSON
    prefixes, every token of a 151936-token synthetic vocabulary; checked
    against the oracle's JsonObject on 8 rows after the timed region."""
    import torch

    from tachyon_amd import workloads as wl
    from tachyon_amd.constrain import DeviceVocab, HostVocab, JsonConstraint, json_mask, pack_states

    import numpy as np

    from tachyon_amd.constrain import JsonMaskSet

    rows, V = 256, wl.QWEN_VOCAB
    toks, special = wl.json_vocab(V, seed=0x15A0)
    hv = HostVocab.from_tokens(toks, special)
    dv = DeviceVocab(hv)
    mode = args.mask_mode
    total = args.warmup + args.steps
    if mode == "decode":
        # each row writes its own document, one 4-byte token per step
        rng = np.random.default_rng(0x15A5)
        docs = [wl.json_document(rng) for _ in range(rows)]
        cur = [JsonConstraint() for _ in range(rows)]
        step_states, step_prefixes = [], []
        for i in range(total):
            step_states.append([c.packed() for c in cur])
            step_prefixes.append([d[:4 * i] for d in docs])
            for r, c in enumerate(cur):
                c.advance(docs[r][4 * i:4 * i + 4])
    else:
        prefixes = wl.json_prefixes(rows, seed=0x15A4)
        cs = []
        for p in prefixes:
            c = JsonConstraint()
            c.advance(p)
            cs.append(c)
        step_states = [[c.packed() for c in cs]] * total
        step_prefixes = [prefixes] * total
    stride = (V + 31) // 32
    mask = torch.zeros(rows, stride, dtype=torch.int32, device="cuda")
    mset = None
    if mode != "direct":
        mset = JsonMaskSet(max_rows=rows, capacity=0 if mode == "dedupe" else 1024, usable=V)
    st_dev = [torch.from_numpy(np.frombuffer(b"".join(ss), np.uint8).copy()).cuda() for ss in step_states[:1]]
    # the host arrays a caller keeps its states in, built before the timed steps
    step_arrays = [JsonMaskSet.pack(ss) for ss in step_states] if mode != "direct" else None
    counts = []
    host_s = 0.0

    def one(i):
        nonlocal host_s
        if mset is None:
            json_mask(dv, st_dev[0], rows, V, mask, stride)
            return
        t0 = time.perf_counter()
        counts.append(mset.fill(dv, step_arrays[i], mask, stride))
        host_s += time.perf_counter() - t0

    for i in range(args.warmup):
        one(i)
    torch.cuda.synchronize()
    counts.clear()
    host_s = 0.0
    ea = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    eb = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    for i in range(args.steps):
        ea[i].record()
        one(args.warmup + i)
        eb[i].record()
    torch.cuda.synchronize()
    us = sum(ea[i].elapsed_time(eb[i]) for i in range(args.steps)) / args.steps * 1e3
    check = None
    if not args.no_check:
        from oracle import pyoracle

        got = mask.cpu().numpy().view(np.uint32)
        last = step_prefixes[total - 1]
        same = 0
        for r in range(0, rows, rows // 8):
            o = pyoracle.JsonOracle()
            o.advance(last[r])
            same += int((got[r] == o.mask(hv, V)).all())
        check = {"rows": 8, "mask_equal": same}
    set_info = None
    if mset is not None:
        c = np.array(counts, dtype=np.float64)
        set_info = {"capacity": 0 if mode == "dedupe" else 1024, "distinct_per_step": round(c[:, 1].mean(), 2),
                    "hits_per_step": round(c[:, 2].mean(), 2), "evaluated_per_step": round(c[:, 3].mean(), 2),
                    "host_us_per_fill": round(host_s / args.steps * 1e6, 1)}
        mset.close()
    alg = int(hv.offsets.nbytes + hv.bytes.nbytes + hv.special.nbytes + rows * stride * 4)
    rec = {"metric": "JsonObject allow-masks per second (rows x 151936 tokens)", "value": round(rows / (us * 1e-6), 1),
           "unit": "rows/s", "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
           "ms_per_step": round(us / 1e3, 5), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "u8", "data": "synthetic",
           "config": {"workload": ("tsm_json_mask: 256 rows, states from random JSON prefixes, synthetic vocab"
                                   if mode != "decode" else
                                   "tsm_json_masks_fill: 256 rows each writing a random JSON document, "
                                   "one 4-byte token per step, synthetic vocab"),
                      "rows": rows, "vocab": V, "mask_mode": mode, "mask_set": set_info},
           "roofline": {"bound": "hbm", "achieved": round(alg / (us * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                        "algorithmic_bytes_per_step": alg, "kernel_avg_us": round(us, 2),
                        "kernel": ("json_mask_kernel (one launch per step)" if mode == "direct" else
                                   "json_mask_kernel over the step's new states + mask_copy_kernel")},
           "cpu_baseline": None, "oracle_check": check}
    print(json.dumps(rec), flush=True)


def bench_lm_head(args):
    """One step of the logits producer at the c4 shape: 256 logit rows, a
    Qwen-class hidden size of 4096 and vocabulary of 151936, random bf16
    weights and f32 activations; the logits are checked against the oracle's
    output layer on a sample after the timed region (the bound of
    tests/test_gpu_lmhead.py)."""
    import torch

    from tachyon_amd.lmhead import lm_head, workspace_bytes

    rows, dim, V = args.lm_rows, 4096, 151936
    split = not args.lm_bf16
    gen = torch.Generator(device="cuda").manual_seed(0x1A4E)
    x = torch.randn(rows, dim, generator=gen, device="cuda", dtype=torch.float32) * 3.0
    g = 1.0 + 0.2 * torch.randn(dim, generator=gen, device="cuda", dtype=torch.float32)
    w = (torch.randn(V, dim, generator=gen, device="cuda", dtype=torch.float32) * 0.02).to(torch.bfloat16)
    out = torch.empty(rows, V, dtype=torch.float32, device="cuda")
    ws = torch.empty(workspace_bytes(rows, dim, split), dtype=torch.uint8, device="cuda")
    for _ in range(args.warmup):
        lm_head(x, g, 1e-6, w, split=split, out=out, workspace=ws)
    torch.cuda.synchronize()
    ea = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    eb = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    for i in range(args.steps):
        ea[i].record()
        lm_head(x, g, 1e-6, w, split=split, out=out, workspace=ws)
        eb[i].record()
    torch.cuda.synchronize()
    us = sum(ea[i].elapsed_time(eb[i]) for i in range(args.steps)) / args.steps * 1e3
    check = None
    if not args.no_check:
        import numpy as np

        from oracle import pyoracle

        rsel = np.unique(np.array([0, rows // 3, (2 * rows) // 3, rows - 1]))
        vsel = np.concatenate([np.arange(0, V - 128, (V - 128) // 512)[:512], np.arange(V - 128, V)])
        rt, vt = torch.from_numpy(rsel).cuda(), torch.from_numpy(vsel).cuda()
        wb = w[vt].view(torch.int16).cpu().numpy().view(np.uint16)
        xs, gs = x[rt].cpu().numpy(), g.cpu().numpy()
        want = pyoracle.lm_head(xs, gs, 1e-6, wb)
        xb = pyoracle.rmsnorm(xs, gs, 1e-6).astype(np.float64)
        s_abs = np.abs(xb) @ np.abs((wb.astype(np.uint32) << 16).view(np.float32).astype(np.float64)).T
        got = out[rt][:, vt].cpu().numpy().astype(np.float64)
        tol = 2.0 ** -16 if split else 2.0 ** -8
        check = {"rows": int(len(rsel)), "ids": int(len(vsel)),
                 "within_bound": int((np.abs(got - want) <= tol * s_abs).sum()), "bound": f"{tol:.3g} * sum|w x|"}
    alg = V * dim * 2 + rows * dim * 4 + dim * 4 + rows * V * 4
    flop = 2.0 * rows * dim * V
    rec = {"metric": "lm_head logit rows/s (rmsnorm + bf16 lm_head, dim 4096, vocab 151936)",
           "value": round(rows / (us * 1e-6), 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(us / 1e3, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "bf16 weights, " + ("bf16 hi+lo activations" if split else "bf16 activations"),
           "data": "synthetic",
           "config": {"workload": f"tsm_lm_head: {rows} rows x dim 4096 x vocab 151936"
                                  + (" (the c4 batch's logits)" if rows == 256 else ""),
                      "rows": rows, "dim": dim, "vocab": V, "split": split},
           "roofline": {"bound": "hbm", "achieved": round(alg / (us * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                        "algorithmic_bytes_per_step": alg, "kernel_avg_us": round(us, 2),
                        "kernel": "lm_prep_kernel + lm_gemm_kernel (one tsm_lm_head call per step)",
                        "mfma_tflops": round(flop * (2 if split else 1) / (us * 1e-6) / 1e12, 1),
                        "mfma_peak_tflops": 2500.0},
           "cpu_baseline": None, "oracle_check": check}
    print(json.dumps(rec), flush=True)


def bench_lm_head_q8(args):
    """One step of the Q8 logits producer at the c4 shape (256 rows, dim
    4096, vocab 151936): random int8 weights with random f16 block scales,
    f32 activations; after the timed region the logits of four rows over
    every id are checked bit for bit against the oracle's Q8 output layer
    (the bar of tests/test_gpu_lmhead_q8.py)."""
    import torch

    from tachyon_amd.lmhead import lm_head_q8, workspace_bytes_q8

    rows, dim, V = args.lm_rows, 4096, 151936
    gen = torch.Generator(device="cuda").manual_seed(0x1A4F)
    x = torch.randn(rows, dim, generator=gen, device="cuda", dtype=torch.float32) * 3.0
    g = 1.0 + 0.2 * torch.randn(dim, generator=gen, device="cuda", dtype=torch.float32)
    wq = torch.randint(-127, 128, (V, dim), generator=gen, device="cuda", dtype=torch.int8)
    wsc = (0.001 * torch.randn(V, dim // 32, generator=gen, device="cuda")).to(torch.float16).view(torch.int16)
    out = torch.empty(rows, V, dtype=torch.float32, device="cuda")
    ws = torch.empty(workspace_bytes_q8(rows, dim), dtype=torch.uint8, device="cuda")
    for _ in range(args.warmup):
        lm_head_q8(x, g, 1e-6, wq, wsc, out=out, workspace=ws)
    torch.cuda.synchronize()
    ea = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    eb = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    for i in range(args.steps):
        ea[i].record()
        lm_head_q8(x, g, 1e-6, wq, wsc, out=out, workspace=ws)
        eb[i].record()
    torch.cuda.synchronize()
    us = sum(ea[i].elapsed_time(eb[i]) for i in range(args.steps)) / args.steps * 1e3
    check = None
    if not args.no_check:
        import numpy as np

        from oracle import pyoracle

        rsel = np.unique(np.array([0, rows // 3, rows - 1]))
        rt = torch.from_numpy(rsel).cuda()
        want = pyoracle.lm_head_q8(x[rt].cpu().numpy(), g.cpu().numpy(), 1e-6, wq.cpu().numpy(),
                                   wsc.cpu().numpy().view(np.uint16))
        got = out[rt].cpu().numpy()
        check = {"rows": int(len(rsel)), "ids": V, "bit_exact": int((got.view(np.uint32) == want.view(np.uint32)).sum())}
    alg = V * dim + V * (dim // 32) * 2 + rows * dim * 4 + dim * 4 + rows * V * 4
    ops = 2.0 * rows * dim * V
    rec = {"metric": "lm_head logit rows/s (rmsnorm + Q8 lm_head, dim 4096, vocab 151936)",
           "value": round(rows / (us * 1e-6), 1), "unit": "rows/s", "n_gpus": 1, "steps": args.steps,
           "warmup": args.warmup, "ms_per_step": round(us / 1e3, 5), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "int8 weights and activations (i32 block dots, f32 scaling)",
           "data": "synthetic",
           "config": {"workload": f"tsm_lm_head_q8: {rows} rows x dim 4096 x vocab 151936"
                                  + (" (the c4 batch's logits)" if rows == 256 else ""),
                      "rows": rows, "dim": dim, "vocab": V},
           "roofline": {"bound": "hbm", "achieved": round(alg / (us * 1e-6) / 1e9, 1), "peak": HBM_PEAK_GBS,
                        "unit": "GB/s", "frac": round(alg / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                        "algorithmic_bytes_per_step": alg, "kernel_avg_us": round(us, 2),
                        "kernel": "lm_q8_prep_kernel + lm_q8_gemm_kernel (one tsm_lm_head_q8 call per step)",
                        "mfma_tops": round(ops / (us * 1e-6) / 1e12, 1), "mfma_peak_tops": 5000.0},
           "cpu_baseline": None, "oracle_check": check}
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
