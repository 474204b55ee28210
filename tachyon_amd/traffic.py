"""HBM traffic of a sampling kernel from rocprofv3 counter passes.

rocprofv3 collects FETCH_SIZE and WRITE_SIZE (KiB per dispatch) in separate
runs: one pair over ``bench.py`` (the sampling kernel) and one pair over
``bench.py --calib-copy-mb N`` (a device-to-device copy of N MiB, which
reads and writes exactly N MiB).  The copy fixes the scale of each counter
on this machine: factor = known bytes / counted bytes.  The kernel's HBM
traffic per launch is then its average count times that factor.

Usage (paths are the ``*_counter_collection.csv`` files rocprofv3 wrote):

    python -m tachyon_amd.traffic --kernel-fetch K_F.csv --kernel-write K_W.csv \\
        --copy-fetch C_F.csv --copy-write C_W.csv --copy-mb 512 \\
        --algorithmic-bytes 161506304 --kernel topk_kernel --out traffic_c4.json

It prints a short text summary and writes the JSON that ``bench.py`` reads
for ``roofline.traffic``.  The JSON carries the SHA-256 of the sampling
library the counters were taken on (``--library``, by default the in-tree
build); ``bench.py`` reports the traffic only when the library it loaded has
the same hash.
"""
from __future__ import annotations

import argparse
import csv
import hashlib
import json
import os
import statistics

KERNEL = "topk_kernel"  # c4's rows all take the lean whole-row kernel
DEFAULT_LIBRARY = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libtachyon_sampler.so")


def library_sha256(path: str) -> str:
    """SHA-256 (hex) of a built library file."""
    h = hashlib.sha256()
    with open(path, "rb") as fh:
        for chunk in iter(lambda: fh.read(1 << 20), b""):
            h.update(chunk)
    return h.hexdigest()


def per_dispatch(path: str, counter: str, name_part: str) -> list[float]:
    """Counter values (summed over the rows of one dispatch) of the dispatches
    whose kernel name contains ``name_part``."""
    acc: dict[int, float] = {}
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] != counter or name_part not in r["Kernel_Name"]:
                continue
            d = int(r["Dispatch_Id"])
            acc[d] = acc.get(d, 0.0) + float(r["Counter_Value"])
    return [acc[d] for d in sorted(acc)]


def copy_kernel_values(path: str, counter: str) -> list[float]:
    """The copy run's dispatches of its largest kernel (the blit that moves
    the buffer; small fills and set-up kernels are left out)."""
    by_name: dict[str, dict[int, float]] = {}
    with open(path, newline="") as fh:
        for r in csv.DictReader(fh):
            if r["Counter_Name"] != counter:
                continue
            by_name.setdefault(r["Kernel_Name"], {})
            d = int(r["Dispatch_Id"])
            by_name[r["Kernel_Name"]][d] = by_name[r["Kernel_Name"]].get(d, 0.0) + float(r["Counter_Value"])
    if not by_name:
        raise SystemExit(f"{path}: no {counter} rows")
    name = max(by_name, key=lambda k: statistics.median(by_name[k].values()))
    return [by_name[name][d] for d in sorted(by_name[name])]


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--kernel-fetch", required=True)
    ap.add_argument("--kernel-write", required=True)
    ap.add_argument("--copy-fetch", required=True)
    ap.add_argument("--copy-write", required=True)
    ap.add_argument("--copy-mb", type=int, required=True)
    ap.add_argument("--algorithmic-bytes", type=int, required=True)
    ap.add_argument("--out", required=True)
    ap.add_argument("--library", default=DEFAULT_LIBRARY, help="the library the counter runs loaded")
    ap.add_argument("--kernel", default=KERNEL, help="a part of the kernel's name (its dispatches are counted)")
    args = ap.parse_args()

    copy_bytes = args.copy_mb << 20
    # medians: the first copy may touch cold pages
    cf = statistics.median(copy_kernel_values(args.copy_fetch, "FETCH_SIZE"))
    cw = statistics.median(copy_kernel_values(args.copy_write, "WRITE_SIZE"))
    f_fetch = copy_bytes / (cf * 1024.0)
    f_write = copy_bytes / (cw * 1024.0)
    kf = per_dispatch(args.kernel_fetch, "FETCH_SIZE", args.kernel)
    kw = per_dispatch(args.kernel_write, "WRITE_SIZE", args.kernel)
    if not kf or not kw:
        raise SystemExit(f"no {args.kernel} dispatches in the counter files")
    fetch_b = statistics.mean(kf) * 1024.0 * f_fetch
    write_b = statistics.mean(kw) * 1024.0 * f_write
    total = fetch_b + write_b
    rec = {
        "library_sha256": library_sha256(args.library),
        "kernel": args.kernel,
        "hbm_bytes_per_step": int(round(total)),
        "fetch_bytes_per_step": int(round(fetch_b)),
        "write_bytes_per_step": int(round(write_b)),
        "algorithmic_bytes_per_step": args.algorithmic_bytes,
        "traffic_over_algorithmic": round(total / args.algorithmic_bytes, 4),
        "kernel_dispatches": {"fetch": len(kf), "write": len(kw)},
        "raw_kib_per_dispatch": {"FETCH_SIZE": round(statistics.mean(kf), 1),
                                 "WRITE_SIZE": round(statistics.mean(kw), 1)},
        "copy_calibration": {"bytes": copy_bytes, "FETCH_SIZE_kib": round(cf, 1), "WRITE_SIZE_kib": round(cw, 1),
                             "fetch_factor": round(f_fetch, 4), "write_factor": round(f_write, 4)},
    }
    with open(args.out, "w") as fh:
        json.dump(rec, fh, indent=1)
        fh.write("\n")
    print(f"{args.kernel}: fetch {fetch_b / 1e6:.2f} MB + write {write_b / 1e6:.3f} MB per launch "
          f"= {total / 1e6:.2f} MB; algorithmic {args.algorithmic_bytes / 1e6:.2f} MB "
          f"(ratio {total / args.algorithmic_bytes:.3f}); copy calibration factors fetch {f_fetch:.3f} "
          f"write {f_write:.3f}")


if __name__ == "__main__":
    main()
