"""Runs the C++ port of the reference acceptance tests (tests/cpp/bitlinear_engine_test.cpp),
which drives the nn:: C++ API of libnn-hip.so (HipEngine, BitLinear, RMSNorm, Model::add,
cli::create_engine). Exit codes follow the reference's ctest convention: 0 pass, 1 fail,
77 skip (no device)."""
import os
import subprocess

import pytest

from conftest import ROOT

BIN = os.path.join(ROOT, "tests", "cpp", "bin", "bitlinear_engine_test")


def run():
    assert os.path.exists(BIN), "build it with __graft_entry__.build() (make -C neuralnet.cpp_amd)"
    p = subprocess.run([BIN, os.path.join(ROOT, "tests", "golden")], capture_output=True, text=True, timeout=240)
    print(p.stdout[-6000:], p.stderr[-2000:], flush=True)
    return p


def test_cpp_port_host_sections():
    """Host-only sections pass; without a visible device the binary reports skip (77)."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("device present: covered by the gpu variant")
    p = run()
    assert p.returncode == 77, p.stdout
    assert "[FAIL]" not in p.stdout


@pytest.mark.gpu
def test_cpp_port_on_hip_engine():
    p = run()
    assert p.returncode == 0, p.stdout
    assert "all passed" in p.stdout
