"""CPU runs under AddressSanitizer and UndefinedBehaviorSanitizer: the oracle (every golden-vector and property test of
tests/test_oracle.py, against oracle/_san/liboracle_san.so built with gcc's sanitizers) and the library's device-free host
code (the C ABI's boundary tests and the expert cache's bookkeeping traces of tests/test_hip_boundary.py and
tests/test_cache.py, against stream-_amd/_build_san/libes_hip_quant_san.so, whose host code clang instrumented). Each
runs in a child Python that preloads the matching sanitizer runtime; any report fails the child."""
import glob
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SAN = os.path.join(ROOT, "oracle", "_san", "liboracle_san.so")
LIB_SAN = os.path.join(ROOT, "stream-_amd", "_build_san", "libes_hip_quant_san.so")
OPTS = {"ASAN_OPTIONS": "detect_leaks=0:abort_on_error=0", "UBSAN_OPTIONS": "halt_on_error=1:print_stacktrace=1"}


def _build(target_dir):
    r = subprocess.run(["make", "-C", target_dir, "san", "-j8"], capture_output=True, text=True)
    if r.returncode:
        pytest.fail("sanitizer build failed:\n" + r.stdout[-2000:] + r.stderr[-2000:])


def _child(preload, env_extra, tests):
    env = dict(os.environ, LD_PRELOAD=preload, **OPTS, **env_extra)
    r = subprocess.run([sys.executable, "-m", "pytest", *tests, "-q", "-x", "-m", "not gpu", "-p", "no:cacheprovider"],
                       cwd=ROOT, env=env, capture_output=True, text=True, timeout=900)
    assert r.returncode == 0, (r.stdout[-3000:] + r.stderr[-3000:])
    assert "ERROR: AddressSanitizer" not in r.stderr and "runtime error:" not in r.stderr, r.stderr[-3000:]
    return r.stdout


def test_oracle_under_asan_ubsan():
    _build(os.path.join(ROOT, "oracle"))
    asan = subprocess.run(["gcc", "-print-file-name=libasan.so"], capture_output=True, text=True).stdout.strip()
    if not os.path.isabs(asan):
        pytest.skip("gcc's libasan is not installed")
    out = _child(asan, {"ESQ_ORACLE_LIB": ORACLE_SAN}, ["tests/test_oracle.py"])
    assert "passed" in out


def test_library_host_code_under_asan_ubsan():
    _build(os.path.join(ROOT, "stream-_amd"))
    rts = sorted(glob.glob("/opt/rocm/llvm/lib/clang/*/lib/linux/libclang_rt.asan-x86_64.so"))
    if not rts:
        pytest.skip("clang's ASan runtime is not installed")
    out = _child(rts[-1], {"ES_HIP_LIB": LIB_SAN}, ["tests/test_hip_boundary.py", "tests/test_cache.py"])
    assert "passed" in out
