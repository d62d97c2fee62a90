"""CPU tests of the C-ABI boundary: the library loads, exports every entry point include/es_hip_quant.h declares, reports
format facts like the reference, and refuses to compute without a gfx950 device (no CPU fallback)."""
import ctypes as C
import os
import re

import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "es_hip_quant.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(es_hip_\w+)\s*\(", text)))


def test_header_declares_the_drop_in_surface():
    names = declared_functions()
    for n in ("es_hip_matvec", "es_hip_matvec_multi", "es_hip_matvec_dev", "es_hip_matvec_multi_dev", "es_hip_run_jobs",
              "es_hip_row_bytes", "es_hip_quant_supported", "es_hip_register", "es_hip_available", "es_hip_last_error"):
        assert n in names


def test_library_exports_every_declared_symbol(hiplib):
    missing = [n for n in declared_functions() if not hasattr(hiplib._L, n)]
    assert not missing, missing


def test_exports_are_c_symbols():
    out = os.popen(f"nm -D --defined-only {E.LIB_PATH}").read()
    for n in declared_functions():
        assert re.search(rf"\sT\s{n}$", out, flags=re.M), n   # unmangled, extern "C"


def test_no_other_c_symbols_exported():
    """every unmangled symbol the library defines is a declared es_hip_* entry point (helpers stay internal)"""
    declared = set(declared_functions())
    stray = []
    for line in os.popen(f"nm -D --defined-only {E.LIB_PATH}").read().splitlines():
        parts = line.split()
        if len(parts) != 3 or parts[2].startswith(("_Z", "__hip_cuid_", "_init", "_fini", "_edata", "_end", "__bss",
                                                   "__odr_asan", "__asan")):   # (the last two: sanitizer builds)
            continue
        if parts[2] not in declared:
            stray.append(parts[2])
    assert not stray, stray


@pytest.mark.parametrize("F", ["Q4_0", "Q5_0", "Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"])
def test_row_bytes_match_reference(hiplib, F):
    t = O.TYPES[F]
    assert hiplib._L.es_hip_quant_supported(t) == 1
    for cols in (0, 256, 768, 896 if O.BLOCK_ELEMS[t] == 32 else 1024, 2048, 8192):
        assert hiplib._L.es_hip_row_bytes(t, cols) == O.row_bytes(t, cols)


def test_unsupported_types(hiplib):
    for t in (0, 1, 3, 7, 9, 15, 16, 39):
        assert hiplib._L.es_hip_quant_supported(t) == 0
        assert hiplib._L.es_hip_row_bytes(t, 256) == 0


def test_order_switch(hiplib):
    assert hiplib.get_order() == E.ORDER_X86_CONTRACT   # the reference's default (clang) build
    assert hiplib.set_order(E.ORDER_SCALAR) == E.ORDER_X86_CONTRACT
    assert hiplib.get_order() == E.ORDER_SCALAR
    with pytest.raises(E.EsHipError):
        hiplib.set_order(7)
    hiplib.set_order(E.ORDER_X86_CONTRACT)


def test_no_device_means_no_compute(hiplib):
    """without a gfx950 device every compute entry point fails loudly; nothing runs on the CPU instead"""
    if hiplib.available():
        pytest.skip("a device is present")
    assert "device" in hiplib.last_error().lower()
    with pytest.raises(E.EsHipError) as ei:
        hiplib.matvec_multi_dev(E.Q4_K, 4096, 256, 0, 1, 4096, 0, 1, 4096, 1)
    assert ei.value.code == -1
    assert hiplib._L.es_hip_malloc(16) is None
    # the void drop-in leaves y untouched and reports through es_hip_last_error
    W = np.zeros(144, np.uint8)
    acts = np.zeros((1, 1), O.Q8K)
    y = np.full((1, 1), 7.0, np.float32)
    with pytest.raises(E.EsHipError):
        hiplib.host_matvec_multi(E.Q4_K, W, 256, 0, 1, acts, y)
    assert y[0, 0] == 7.0


def test_q2k_kernel_name_and_switch(hiplib):
    """es_q2k.h's kernel name and scalar switch (src/es_q2k.h:83-86), usable without a device"""
    L = hiplib._L
    assert L.es_hip_q2k_kernel_name() == b"hip-gfx950"
    L.es_hip_q2k_force_scalar(1)
    assert b"scalar" in L.es_hip_q2k_kernel_name()
    L.es_hip_q2k_force_scalar(0)
    assert L.es_hip_q2k_kernel_name() == b"hip-gfx950"
