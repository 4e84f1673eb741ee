"""CPU-side checks of the drop-in boundary: libnn-hip.so loads, exports exactly the C ABI
that include/nnhip.h declares (and the Python binding declares every one of them), and
rejects bad arguments with a status code and a message before touching a GPU.
No compute entry point is called here (there is no GPU in this container)."""
import ctypes
import os
import re
import subprocess
import sys

import pytest

from conftest import ROOT

HEADER = os.path.join(ROOT, "include", "nnhip.h")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nnhip_\w+)\s*\(", text)))


def test_library_built(nnhip):
    assert os.path.exists(nnhip.LIB_PATH), "run __graft_entry__.build() first"


def test_exports_match_header(nnhip):
    declared = header_functions()
    assert len(declared) >= 35
    out = subprocess.run(["nm", "-D", "--defined-only", nnhip.LIB_PATH], check=True,
                         capture_output=True, text=True).stdout
    exported = set(re.findall(r"\s[TW]\s+(nnhip_\w+)$", out, flags=re.M))
    missing = [f for f in declared if f not in exported]
    assert not missing, f"declared but not exported: {missing}"
    assert exported <= set(declared), f"exported but not declared: {sorted(exported - set(declared))}"


def test_binding_covers_header(nnhip):
    assert sorted(nnhip.SIGNATURES) == header_functions()
    L = nnhip.lib()
    for name in nnhip.SIGNATURES:
        assert hasattr(L, name)


def test_gfx950_code_object_present(nnhip):
    """The library carries a gfx950 code object (our own build's offload bundle)."""
    data = open(nnhip.LIB_PATH, "rb").read()
    assert b"amdgcn-amd-amdhsa--gfx950" in data


def test_errors_without_a_device(nnhip):
    L = nnhip.lib()
    assert L.nnhip_version().decode().startswith("nnhip")
    # null context -> INVALID_ARG and a message, no HIP call made
    assert L.nnhip_sync(None) == 1
    assert "null context" in L.nnhip_last_error().decode()
    assert L.nnhip_row_absmean(None, None, 4, 4, None) == 1
    # pure size helpers
    assert L.nnhip_repacked_bytes(17, 257) == 32 * 512 // 4
    assert L.nnhip_act_i8_bytes(2560, 3) == 2560 * 3
    assert L.nnhip_act_i8_bytes(17, 2) == 256 * 2


def test_no_cpu_fallback_without_gpu(nnhip):
    """The binding raises instead of computing anything on the host."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    with pytest.raises(nnhip.NNHipError):
        nnhip.Context(0)


def test_fnv1a64_output_hash(nnhip):
    """The bench's output hash uses the reference layer_bench --hash constants
    (src/layer_bench.cpp:732-741): the empty input gives its start value, and every byte is folded
    as h = (h ^ byte) * 1099511628211 mod 2^64 (a host function, no GPU)."""
    import numpy as np
    assert nnhip.fnv1a64(np.zeros(0, np.uint8)) == "%016x" % 1469598103934665603
    data = np.frombuffer(b"BitLinear W1.58A8", np.uint8)
    h = 1469598103934665603
    for byte in data.tolist():
        h = ((h ^ byte) * 1099511628211) % (1 << 64)
    assert nnhip.fnv1a64(data) == "%016x" % h
    # f32 values hash their little-endian bytes
    x = np.array([1.0, -2.5], np.float32)
    assert nnhip.fnv1a64(x) == nnhip.fnv1a64(x.view(np.uint8))


def test_bench_traffic_needs_matching_kernel_sources(tmp_path, monkeypatch, capsys):
    """bench.py's roofline.traffic comes from the committed PMC summary only while the grouped
    GEMV's sources hash to the value the summary records; after any change it is omitted."""
    import shutil
    sys.path.insert(0, ROOT)
    import bench
    assert bench.profiled_traffic() is not None  # the committed summary matches the tree
    (tmp_path / "profiles").mkdir()
    (tmp_path / "neuralnet.cpp_amd" / "csrc").mkdir(parents=True)
    shutil.copy(os.path.join(ROOT, "profiles", "k_gemv_grouped_m1_layerstack_pmc.md"), tmp_path / "profiles")
    for src in ("k_gemv.hip", "gemv_tile.hpp"):
        shutil.copy(os.path.join(ROOT, "neuralnet.cpp_amd", "csrc", src), tmp_path / "neuralnet.cpp_amd" / "csrc")
    monkeypatch.setattr(bench, "ROOT", str(tmp_path))
    assert bench.profiled_traffic() is not None
    with open(tmp_path / "neuralnet.cpp_amd" / "csrc" / "k_gemv.hip", "a") as f:
        f.write("\n// changed\n")
    assert bench.profiled_traffic() is None
    assert "other k_gemv sources" in capsys.readouterr().err
