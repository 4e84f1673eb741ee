"""Shared test setup: the `gpu` marker, loaders for libnn-hip.so's Python binding and the
CPU oracle (test infrastructure), and seeded input helpers."""
import importlib.util
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU (MI355X); runs on the GPU box")


def load_nnhip():
    """Import neuralnet.cpp_amd/__init__.py (the directory name has a dot) as `nnhip_py`."""
    name = "nnhip_py"
    if name in sys.modules:
        return sys.modules[name]
    pkg = os.path.join(ROOT, "neuralnet.cpp_amd")
    spec = importlib.util.spec_from_file_location(name, os.path.join(pkg, "__init__.py"),
                                                  submodule_search_locations=[pkg])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[name] = mod
    spec.loader.exec_module(mod)
    return mod


@pytest.fixture(scope="session")
def nnhip():
    return load_nnhip()


@pytest.fixture(scope="session")
def orc():
    from oracle import nn_oracle
    nn_oracle.lib()
    return nn_oracle


@pytest.fixture(scope="session")
def ctx(nnhip):
    c = nnhip.Context(0)
    yield c
    c.close()


def uniform(shape, seed, lo=-1.0, hi=1.0):
    from oracle import nn_oracle
    n = int(np.prod(shape))
    return nn_oracle.fill_uniform(n, seed, lo, hi).reshape(shape)


def normal(shape, seed, mean=0.0, std=1.0):
    from oracle import nn_oracle
    n = int(np.prod(shape))
    return nn_oracle.fill_normal(n, seed, mean, std).reshape(shape)
