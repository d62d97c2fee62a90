import os
import subprocess
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, os.path.join(ROOT, "stream-_amd"))

GOLDEN = os.path.join(ROOT, "tests", "golden", "ref_vectors.npz")
ENGINE_GOLDEN = os.path.join(ROOT, "tests", "golden", "engine_vectors.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def _ensure_oracle():
    so = os.path.join(ROOT, "oracle", "liboracle.so")
    if not os.path.exists(so):   # built by __graft_entry__.build(); build here only if nothing is there
        subprocess.run(["make", "-C", os.path.join(ROOT, "oracle"), "all"], check=True, capture_output=True)
    return so


@pytest.fixture(scope="session")
def orc():
    _ensure_oracle()
    import oracle as O
    return O.Oracle()


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def engine_golden():
    """route() / rmsnorm() inputs and outputs of the reference engine built from its source (make_engine_golden.py)"""
    with np.load(ENGINE_GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_cases(g, prefix):
    """case names under prefix/ in a golden dict"""
    return sorted({k.split("/")[1] for k in g if k.startswith(prefix + "/")})


@pytest.fixture(scope="session")
def hip():
    """The HIP library through its C-ABI. Fails (not skips) when it is missing: GPU tests must run native code."""
    _ensure_hip_lib()
    import es_hip_quant as E
    lib = E.Lib()
    if not lib.available():
        pytest.fail("es_hip_available() == 0: no usable gfx950 device: " + lib.last_error())
    return lib


def _ensure_hip_lib():
    so = os.path.join(ROOT, "stream-_amd", "libes_hip_quant.so")
    if not os.path.exists(so):   # built by __graft_entry__.build(); build here only if nothing is there
        subprocess.run(["make", "-C", os.path.join(ROOT, "stream-_amd"), "-j4"], check=True, capture_output=True)
    return so


@pytest.fixture(scope="session")
def hiplib():
    """The library loaded without requiring a device (CPU tests of the boundary)."""
    _ensure_hip_lib()
    import es_hip_quant as E
    return E.Lib()
