"""Runs the C ABI on the CPU emulation of the HIP kernels (tests/emu).

TEST INFRASTRUCTURE ONLY.  The product kernel sources are compiled with g++
against a HIP emulation header and AddressSanitizer/UBSan, so that the
kernels' logic (indexing, barriers, selection paths) is checked on the CPU
before anything runs on a GPU.  Nothing in the product imports this.
"""
from __future__ import annotations

import os
import struct
import subprocess
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
EMU_DIR = os.path.join(HERE, "emu")
DRIVER = os.path.join(EMU_DIR, "emu_driver")


def build(target="emu_driver"):
    """make under an exclusive lock (pytest-xdist workers build concurrently)."""
    import fcntl

    with open(os.path.join(EMU_DIR, ".build.lock"), "w") as lock:
        fcntl.flock(lock, fcntl.LOCK_EX)
        jobs = str(max(1, min(5, len(os.sched_getaffinity(0)))))
        subprocess.run(["make", "-s", "-j", jobs, "-C", EMU_DIR, target], check=True)
    return os.path.join(EMU_DIR, target)


def _write_input(path, w, mode, dist_stride=0, kinds=1):
    hist_total = 0xFFFFFFFF if w.hist_ids is None else int(w.hist_ids.size)
    mask_stride = 0 if w.mask is None else int(w.mask.shape[1])
    with open(path, "wb") as fh:
        fh.write(struct.pack("<10I", 0x574D5354, mode, w.rows, w.row_stride, w.usable, mask_stride, hist_total,
                             int(w.top_stride), int(dist_stride), int(kinds)))
        fh.write(np.ascontiguousarray(w.logits, np.float32).tobytes())
        fh.write(np.ascontiguousarray(w.params).tobytes())
        if w.hist_ids is not None:
            fh.write(np.ascontiguousarray(w.hist_offsets, np.uint32).tobytes())
            fh.write(np.ascontiguousarray(w.hist_ids, np.uint32).tobytes())
        if w.mask is not None:
            fh.write(np.ascontiguousarray(w.mask, np.uint32).tobytes())
        fh.write(np.ascontiguousarray(w.uniforms, np.float32).tobytes())


class EmuError(RuntimeError):
    pass


def _run(w, mode, dist_stride=0, driver=None, timeout=900, kinds=1):
    driver = driver or DRIVER
    if not os.path.exists(driver):
        build(os.path.basename(driver))
    with tempfile.TemporaryDirectory() as d:
        fin, fout = os.path.join(d, "in.bin"), os.path.join(d, "out.bin")
        _write_input(fin, w, mode, dist_stride, kinds)
        env = dict(os.environ)
        env.setdefault("ASAN_OPTIONS", "detect_leaks=0:abort_on_error=1")
        r = subprocess.run([driver, fin, fout], capture_output=True, text=True, timeout=timeout, env=env)
        if r.returncode != 0:
            raise EmuError(f"emu_driver exit {r.returncode}\n{r.stderr[-6000:]}")
        raw = open(fout, "rb").read()
    rc, status = struct.unpack_from("<2I", raw, 0)
    if rc != 0:
        raise EmuError(f"rc={rc}: {raw[8:].decode(errors='replace')}")
    off = 8

    def take(dtype, n):
        nonlocal off
        a = np.frombuffer(raw, dtype=dtype, count=n, offset=off).copy()
        off += a.nbytes
        return a

    R = w.rows
    if mode == 0:
        ts = int(w.top_stride)
        out = dict(token=take(np.uint32, R), logprob=take(np.float32, R))
        out["top_ids"] = take(np.uint32, R * ts).reshape(R, ts) if ts else np.zeros((R, 0), np.uint32)
        out["top_lp"] = take(np.float32, R * ts).reshape(R, ts) if ts else np.zeros((R, 0), np.float32)
        out["prob"] = take(np.float32, R)
        out["keep"] = take(np.uint32, R)
    else:
        out = dict(ids=take(np.uint32, R * dist_stride).reshape(R, dist_stride),
                   probs=take(np.float32, R * dist_stride).reshape(R, dist_stride), keep=take(np.uint32, R))
    out["status"] = status
    return out


def emu_sample(w, **kw):
    return _run(w, 0, **kw)


def emu_distribution(w, dist_stride, **kw):
    return _run(w, 1, dist_stride, **kw)
