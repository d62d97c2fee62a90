"""The device expf (stream-_amd/csrc/es_hip_expf.h) against the host C library's expf, which is what the reference's
SwiGLU and router softmax call (src/es_engine.c:755, 913): the header is compiled for the CPU and compared bit for bit on
every one of the 2^32 float inputs."""
import os
import subprocess

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HDR_DIR = os.path.join(ROOT, "stream-_amd", "csrc")

PROG = r"""
#define ESQ_EXPF_QUAL static inline
#include "es_hip_expf.h"
#include <math.h>
#include <stdio.h>
#include <string.h>
#include <thread>
#include <vector>
#include <atomic>
int main() {
    std::atomic<long> bad{0};
    std::vector<std::thread> th;
    const int nt = 8;
    for (int k = 0; k < nt; k++)
        th.emplace_back([&, k] {
            long b = 0;
            for (uint64_t u = k; u < 0x100000000ull; u += nt) {
                const uint32_t bits = (uint32_t)u;
                float x; memcpy(&x, &bits, 4);
                const float a = expf(x), c = esq_expf(x);
                uint32_t ab, cb; memcpy(&ab, &a, 4); memcpy(&cb, &c, 4);
                if (ab != cb) { if (b < 3) printf("x=%a libm=%a mine=%a\n", x, a, c); b++; }
            }
            bad += b;
        });
    for (auto &t : th) t.join();
    printf("mismatches %ld\n", bad.load());
    return bad.load() != 0;
}
"""


@pytest.fixture(scope="module")
def expf_prog(tmp_path_factory):
    d = tmp_path_factory.mktemp("expf")
    src, exe = d / "chk.cpp", d / "chk"
    src.write_text(PROG)
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-I", HDR_DIR, "-o", str(exe), str(src), "-lm"],
                   check=True)
    return str(exe)


def test_device_expf_equals_libm_on_all_floats(expf_prog):
    r = subprocess.run([expf_prog], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "mismatches 0" in r.stdout


def test_oracle_swiglu_is_the_reference_formula(orc):
    """esq_swiglu restates src/es_engine.c:913 with the host expf: textbook points where the value is known exactly"""
    g = np.array([0.0, -0.0, 100.0, -200.0, 1.0], np.float32)
    u = np.array([3.0, 3.0, 2.0, 5.0, 1.0], np.float32)
    h = orc.swiglu(g, u)
    assert h[0] == 0.0 and h[1] == 0.0                      # 0 / (1 + 1) * u
    assert h[2] == np.float32(200.0)                         # expf(-100) ~ 3.7e-44: 1 + tiny == 1
    assert h[3] == 0.0                                       # -200 / (1 + inf) = -0, times 5
    assert h[4] == np.float32(np.float32(1.0) / (np.float32(1.0) + np.exp(np.float32(-1.0))))
