"""The register quantizer's division-free code paths against the exact division they replace,
on the CPU (tests/cpp/quant_math_check.c: every half-integer boundary of sampled token scales,
40 ulps either side, plus uniform and special values). The GPU side of the same property is
test_gpu_parity.py's near-tie and special-value tests through the kernel itself."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(ROOT, "tests", "cpp", "quant_math_check.c")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="gcc not on PATH")
def test_quant_division_free_paths(tmp_path):
    exe = str(tmp_path / "quant_math_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", exe, SRC, "-lm"], check=True)
    out = subprocess.run([exe, "1500"], check=False, capture_output=True, text=True, timeout=300)
    print(out.stdout)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout
