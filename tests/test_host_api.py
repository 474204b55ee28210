"""The C++ Sampler API (tachyon_amd/host/sampler.hpp) through its own test
program, tests/host/test_sampler_host.cpp, which follows the reference's
sampler tests (src/sampler.rs:324-395) and checks whole sequences (tokens and
RNG states) against the CPU oracle."""
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "host", "test_sampler_host")


def _binary():
    if not os.path.exists(BIN):  # host code only: g++, a few seconds
        from tachyon_amd import build as hb

        hb.build_host_tests()
    return BIN


def _run(args, timeout):
    r = subprocess.run([_binary(), *args], capture_output=True, text=True, timeout=timeout)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "FAIL" not in r.stdout


def test_host_api_rng_draw_and_settings():
    """RNG sequence and draw() against the oracle's restatement; settings."""
    _run(["--cpu"], 120)


@pytest.mark.gpu
def test_host_api_on_gpu():
    """The reference's sampler tests and a 12-sequence x 25-step parity run
    (tokens and RNG states) through BatchSampler on the GPU."""
    _run([], 300)
