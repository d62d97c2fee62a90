"""Writes tests/golden/ref_vectors.npz: inputs and outputs of the reference's own kernels, built from its sources.

Run here (where /root/reference exists) after `make -C oracle all ref`:
    python tests/golden/make_golden.py

Every output comes from the reference library (oracle/_ref/libesref_{gcc,clang}.so), never from the oracle. Inputs are
made with the reference's own test recipes (tools/es_mtest.c, tools/es_kbench.c), through the oracle's generators;
the generated inputs are stored, so the fixture does not depend on the generators. Contents, per format F:
    F/mtest_W, F/mtest_x       es_mtest shapes: cols 1024, rows 37, 13 activations (tools/es_mtest.c:17)
    F/gauss_W, F/gauss_x       ~N(0,0.02) weights quantized, ~N(0,1) activations: cols 512, rows 16, 5 activations
    F/{case}_q8                the activation blocks es_act_prepare produced (Q8_0 arena or Q8_K buffer)
    F/{case}_y_{gcc,clang}     es_matvec over rows [3, rows) on the x86 AVX2 path, per compiler
    F/{case}_y_scalar          the same with ES_NO_AVX2=1 (scalar mv_* kernels)
    F/{case}_ymulti_clang      es_matvec_multi (bit-identical to single in the reference: es_mtest's invariant)
    F/{case}_yfloat            es_matvec over rows [3, rows) with activations prepared without blocks (q8 = q80 = NULL):
                               es_dequant_row + dot_f32; checked equal across gcc, clang, scalar and es_matvec_multi
    F/dequant                  es_dequant_row of the first gauss row
plus Q2_K quantizer bytes (es_quantize_q2_K_ref), Q8_K quantizer edge cases, es_fp32_to_fp16 on edge floats and
es_dot_q2_K_q8_K_ref values (the kbench correctness test, tools/es_kbench.c:154-192, at 8 rows).
"""
import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


# name: (seed, slots, layers, experts, k, calls per layer, passes, freq_weight, prefetch)
CACHE_TRACES = {
    "lru": (1, 8, 4, 16, 4, 2, 3, 0.0, "top"),
    "engine": (2, 24, 6, 64, 8, 3, 2, 6.0, "top"),
    "olmoe": (3, 40, 4, 64, 8, 4, 3, 4.0, "top"),
    "wasted": (5, 20, 4, 64, 6, 2, 3, 4.0, "random"),
    "tiny": (4, 6, 3, 16, 8, 1, 2, 1.0, "top"),
    "noprefetch": (6, 12, 5, 32, 4, 3, 2, 2.5, None),
}


def main():
    o = O.Oracle()
    R = {"gcc": O.RefLib("gcc"), "clang": O.RefLib("clang"), "scalar": O.RefLib("gcc", scalar=True)}
    out = {}
    st = np.array([88172645463325252], np.uint64)   # tools/es_mtest.c:9
    for t in (O.Q5_0, O.Q4_0, O.Q4_K, O.Q6_K, O.Q2_K, O.Q8_0, O.Q5_K, O.Q3_K):   # es_mtest's order, then the rest appended
        F = O.NAMES[t]
        cases = {}
        cols, rows, na = 1024, 37, 13
        W = o.mtest_blocks(t, st, rows, cols)
        x = o.mtest_acts(st, cols * na).reshape(na, cols)
        cases["mtest"] = (W, x, cols, rows)
        cols, rows, na = 512, 16, 5
        xw = o.gauss(42 + t, 0.02, rows * cols).reshape(rows, cols)
        W = o.quantize_rows(t, xw)
        x = o.gauss(7 + t, 1.0, na * cols).reshape(na, cols)
        cases["gauss"] = (W, x, cols, rows)
        for name, (W, x, cols, rows) in cases.items():
            out[f"{F}/{name}_W"] = W
            out[f"{F}/{name}_x"] = x
            out[f"{F}/{name}_shape"] = np.array([cols, rows], np.int32)
            _, _, q80, q8 = R["gcc"].prepare(x)
            out[f"{F}/{name}_q8"] = (q8 if O.uses_q8k(t) else q80).view(np.uint8).reshape(x.shape[0], -1)
            for cc, lib in R.items():
                out[f"{F}/{name}_y_{cc}"] = lib.matvec_f32(t, W, cols, rows, x, r0=3)
            out[f"{F}/{name}_ymulti_clang"] = R["clang"].matvec_f32(t, W, cols, rows, x, r0=3, multi=True)
            # the float path (activations without blocks): the same in every build, single and multi
            yf = R["clang"].matvec_float(t, W, cols, rows, x, r0=3)
            for cc, lib in R.items():
                assert np.array_equal(yf.view(np.uint32), lib.matvec_float(t, W, cols, rows, x, r0=3).view(np.uint32))
            assert np.array_equal(yf.view(np.uint32), R["clang"].matvec_float(t, W, cols, rows, x, r0=3, multi=True)
                                  .view(np.uint32))
            out[f"{F}/{name}_yfloat"] = yf
        Wg, _, cols, _ = cases["gauss"]
        out[f"{F}/dequant"] = R["gcc"].dequant(t, Wg[: O.row_bytes(t, cols)], cols)

    # Q2_K test quantizer and reference dot (tools/es_kbench.c:154-192 at 8 rows x 4096)
    s = 42
    w = o.gauss(s, 0.02, 8 * 4096).reshape(8, 4096)
    out["q2k/w"] = w
    out["q2k/W"] = np.concatenate([R["gcc"].quantize_q2_K_ref(w[r]) for r in range(8)])
    xk = o.gauss(7, 1.0, 4096)
    out["q2k/x"] = xk
    out["q2k/xq"] = R["gcc"].quantize_q8_K(xk).view(np.uint8)
    dots = []
    Wb = out["q2k/W"].reshape(8, -1)
    xq = out["q2k/xq"]
    for r in range(8):
        dots.append(R["gcc"].lib.es_dot_q2_K_q8_K_ref(4096, O._p(np.ascontiguousarray(Wb[r])), O._p(xq)))
    out["q2k/dot_ref"] = np.array(dots, np.float32)

    # Q8_K quantizer edge cases: a zero block, exact .5 ties, +-amax, tiny values, one huge value
    e = np.zeros((6, 256), np.float32)
    e[1] = (np.arange(256) - 128) * (127.0 / 128.0)           # ties and near-ties under id = 127/amax
    e[2] = np.where(np.arange(256) % 2, 1.0, -1.0)            # +-amax everywhere
    e[3] = np.linspace(-1e-30, 1e-30, 256, dtype=np.float32)  # tiny
    e[4, 17] = 3e38                                           # one huge value
    e[5] = o.gauss(99, 3.0, 256)
    out["q8k_edge/x"] = e
    out["q8k_edge/q"] = R["gcc"].quantize_q8_K(e).view(np.uint8)
    _, _, q80, _ = R["gcc"].prepare(e)
    out["q80_edge/q"] = q80.view(np.uint8).reshape(6, -1)

    # fp32 -> fp16 rounding of the reference converter
    fl = np.array([0.0, -0.0, 1.0, 65504.0, 65520.0, 1e6, 6.1e-5, 6.0e-8, 2.9e-8, 3.0e-8, 1.0009765625, 1.00048828125,
                   1.000732421875, -2.5e-6, 0.1, 0.001, 1e-10], np.float32)
    out["fp16/f"] = fl
    out["fp16/h"] = np.array([R["gcc"].fp32_to_fp16(float(v)) for v in fl], np.uint16)

    # expert cache traces through the reference's own es_cache.c (oracle/esq_cache_ref.c): engine-like load_experts /
    # prefetch sequences with plain LRU, the engine's frequency weight (1.0 * layers) and others; one with too few slots
    RC = O.RefCache()
    for name, (seed, ns, nl, ne, k, tok, ps, fw, pf) in CACHE_TRACES.items():
        ops = O.make_cache_trace(seed, nl, ne, k, tok, ps, prefetch=pf)
        res, slots, stats = RC.trace(ns, nl, ne, fw, ops)
        out[f"cache/{name}/ops"] = ops
        out[f"cache/{name}/params"] = np.array([ns, nl, ne], np.int32)
        out[f"cache/{name}/freq_weight"] = np.array([fw], np.float64)
        out[f"cache/{name}/res"] = res
        out[f"cache/{name}/slots"] = slots
        out[f"cache/{name}/stats"] = stats

    np.savez_compressed(os.path.join(HERE, "ref_vectors.npz"), **out)
    cc = {}
    for name, exe in (("gcc", "gcc"), ("clang", "/opt/rocm/lib/llvm/bin/clang")):
        try:
            cc[name] = subprocess.run([exe, "--version"], capture_output=True, text=True).stdout.splitlines()[0]
        except OSError:
            cc[name] = "unknown"
    manifest = {
        "source": "reference src/es_quant.c, src/es_q2k.c, src/es_cpu.c built by oracle/Makefile (-O3 -std=c11); "
                  "cache/*: src/es_cache.c, es_io.c, es_cpu.c with oracle/esq_cache_ref.c",
        "compilers": cc,
        "gcc": "x86 AVX2 path, no contraction", "clang": "x86 AVX2 path, -ffp-contract=on (the reference default CC)",
        "scalar": "gcc build with ES_NO_AVX2=1",
        "seeds": {"mtest": 88172645463325252, "gauss_weights": "42+type", "gauss_acts": "7+type"},
        "keys": sorted(out.keys()),
    }
    with open(os.path.join(HERE, "ref_vectors.json"), "w") as f:
        json.dump(manifest, f, indent=1)
    print("wrote", len(out), "arrays,", os.path.getsize(os.path.join(HERE, "ref_vectors.npz")), "bytes")


if __name__ == "__main__":
    main()
