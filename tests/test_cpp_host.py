"""Runs the C++ host-interface tests (tests/cpp/test_sampler.cpp).

The binary restates the reference's Rust unit tests
(crates/yskn-ref/src/output_head_sampler.rs:256-310) against the C++ mirror of
`SamplingParameters` / `Sampler` / `Selector` in
yasakani-for-mac_amd/host/yskn_sampler.hpp. The CPU run covers only the
parameter rules; the GPU run covers every test.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
BIN = os.path.join(HERE, "cpp", "test_sampler")


def _run(args):
    assert os.path.exists(BIN), f"{BIN} is not built (make -C tests/cpp)"
    r = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "ALL PASSED" in r.stdout


def test_cpp_host_parameters():
    if not os.path.exists(BIN):
        subprocess.run(["make", "-s", "-C", os.path.join(HERE, "cpp")], check=True)
    _run(["--cpu"])


@pytest.mark.gpu
def test_cpp_host_sampler():
    _run([])
