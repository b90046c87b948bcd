"""Runs the C++ host-layer test binary (tests/cpp/host_test.cpp), which
restates the reference's own ctest mains over the device KV cache through the
engine-facing C++ layer (dbinfer_amd/host). The CPU part needs no GPU."""
import os
import subprocess

import pytest

BIN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "cpp", "host_test")


def run(args):
    assert os.path.exists(BIN), "run __graft_entry__.build() first"
    r = subprocess.run([BIN] + args, capture_output=True, text=True, timeout=300)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 checks failed" in r.stdout


def test_host_layer_cpu_parts():
    run(["--cpu-only"])


@pytest.mark.gpu
def test_host_layer_on_device():
    run([])
