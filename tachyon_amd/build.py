"""Builds the HIP sampling library for gfx950, in tree.

Outputs (next to this file):
  lib/libtachyon_sampler.so       - shared library (ctypes, C++ callers)
  lib/libtachyon_sampler.a        - static archive (what a Rust build.rs links)
  lib/libtachyon_sampler_host.a   - the C++ Sampler API over the C ABI (host/)
and, with build_host_tests(), tests/host/test_sampler_host.

hipcc flags: -O3 for gfx950 only; -ffp-contract=off so every float/double
operation rounds on its own (the sampler's f32 arithmetic is reproduced bit
for bit); packed FP32 instructions disabled.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIBDIR = os.path.join(HERE, "lib")
ROOT = os.path.dirname(HERE)
SOURCES = ["tsm_sample.hip", "tsm_split.hip", "tsm_api.hip", "tsm_mask.hip", "tsm_lmhead.hip"]
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

DEVICE_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-I", os.path.join(ROOT, "include"),
]


def _run(cmd):
    r = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature; that warning is expected
    err = "\n".join(l for l in r.stderr.splitlines() if "packed-fp32-ops" not in l)
    if r.returncode != 0:
        sys.stderr.write(err + "\n")
        raise RuntimeError(f"command failed ({r.returncode}): {' '.join(cmd)}")
    if err.strip():
        sys.stderr.write(err + "\n")


def build(verbose: bool = False) -> str:
    """Compiles every source and links the .so and .a; returns the .so path."""
    os.makedirs(LIBDIR, exist_ok=True)
    objs = []
    for src in SOURCES:
        obj = os.path.join(LIBDIR, src.replace(".hip", ".o"))
        cmd = [HIPCC, *DEVICE_FLAGS, "-c", os.path.join(CSRC, src), "-o", obj]
        if verbose:
            print(" ".join(cmd))
        _run(cmd)
        objs.append(obj)
    so = os.path.join(LIBDIR, "libtachyon_sampler.so")
    tmp = so + ".tmp"
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", tmp, *objs])
    os.replace(tmp, so)
    ar = shutil.which("ar") or "ar"
    a = os.path.join(LIBDIR, "libtachyon_sampler.a")
    if os.path.exists(a):
        os.remove(a)
    _run([ar, "crs", a, *objs])
    return so


def build_test_helpers(verbose: bool = False) -> str:
    """Test-only HIP helper (tests/helpers/libtsm_probe.so)."""
    d = os.path.join(ROOT, "tests", "helpers")
    src = os.path.join(d, "tsm_probe.hip")
    out = os.path.join(d, "libtsm_probe.so")
    cmd = [HIPCC, *DEVICE_FLAGS, "-shared", src, "-o", out + ".tmp"]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


# The C++ layer is host code over the HIP runtime API: g++, no device pass.
CXX = os.environ.get("CXX", "g++")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-D__HIP_PLATFORM_AMD__",
              "-I", os.path.join(ROOT, "include"), "-I", os.path.join(ROCM, "include")]


def build_host(verbose: bool = False) -> str:
    """The C++ Sampler API (host/sampler.cpp) as a static archive."""
    os.makedirs(LIBDIR, exist_ok=True)
    obj = os.path.join(LIBDIR, "sampler_host.o")
    cmd = [CXX, *HOST_FLAGS, "-c", os.path.join(HERE, "host", "sampler.cpp"), "-o", obj]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    a = os.path.join(LIBDIR, "libtachyon_sampler_host.a")
    if os.path.exists(a):
        os.remove(a)
    _run([shutil.which("ar") or "ar", "crs", a, obj])
    return a


def build_host_tests(verbose: bool = False) -> str:
    """tests/host/test_sampler_host: the C++ API's tests, linked with the
    library, its C++ layer and the CPU oracle (the checker)."""
    host_a = build_host(verbose)
    d = os.path.join(ROOT, "tests", "host")
    out = os.path.join(d, "test_sampler_host")
    oracle_dir = os.path.join(ROOT, "oracle")
    cmd = [CXX, *HOST_FLAGS, os.path.join(d, "test_sampler_host.cpp"), host_a,
           "-L", LIBDIR, "-ltachyon_sampler", "-L", oracle_dir, "-ltachyon_oracle",
           "-L", os.path.join(ROCM, "lib"), "-lamdhip64",
           "-Wl,-rpath,$ORIGIN/../../tachyon_amd/lib", "-Wl,-rpath,$ORIGIN/../../oracle",
           f"-Wl,-rpath,{os.path.join(ROCM, 'lib')}", "-o", out + ".tmp"]
    if verbose:
        print(" ".join(cmd))
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
    print(build_test_helpers(verbose="-v" in sys.argv))
