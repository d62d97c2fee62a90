"""Writes tests/golden/engine_vectors.npz: inputs and outputs of the reference engine's own route() (softmax gating) and
rmsnorm() (src/es_engine.c:744-835, 189-194), compiled from its source.

Run here (where /root/reference exists) after `make -C oracle ref`:
    python tests/golden/make_engine_golden.py

Every output comes from oracle/_ref/libesref_engine_clang.so (the reference's default compiler), never from the oracle;
the gcc build must agree bit for bit (checked here before writing). Contents:
    route/{case}/logits, route/{case}/params [k, norm_topk], route/{case}/sel, route/{case}/w
        olmoe      128 tokens x 64 experts, top-8, no renormalisation (config 4's router, src/es_engine.c:1764)
        qwen3      32 tokens x 128 experts, top-8, renormalised (config 5's router, src/es_engine.c:1765)
        ties       repeated and equal logits (first maximum wins), top-8 of 64, both renormalisation settings
        underflow  one dominant logit per token, the rest 60..200 below (expf underflows to subnormals and zero)
        k1, k32    top-1 of 64, and top-32 of 64 (renormalised; 32 is the reference's MAXK, src/es_engine.c:41)
        wide       4 tokens x 1024 experts (route()'s selection buffer limit), top-8, renormalised
    rms/{case}/x, rms/{case}/w (absent: unweighted), rms/{case}/eps, rms/{case}/o
        n896, n2048, n8192 weighted and unweighted; tiny and huge magnitudes
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle as O  # noqa: E402


def route_cases(rng):
    c = {}
    c["olmoe"] = (rng.standard_normal((128, 64)).astype(np.float32), 8, 0)
    c["qwen3"] = (rng.standard_normal((32, 128)).astype(np.float32), 8, 1)
    t = np.zeros((6, 64), np.float32)
    t[1] = np.repeat(np.arange(16, dtype=np.float32) * 0.25, 4)           # groups of four equal logits
    t[2, ::3] = 1.5                                                       # many equal maxima
    t[3] = np.where(np.arange(64) % 2, 0.5, -0.5).astype(np.float32)
    t[4] = rng.integers(-3, 4, 64).astype(np.float32)                     # small-integer logits, many ties
    t[5] = np.float32(7.0)                                                # all equal, non-zero
    c["ties"] = (t, 8, 0)
    c["ties_norm"] = (t.copy(), 8, 1)
    u = -rng.uniform(60.0, 200.0, (8, 64)).astype(np.float32)
    u[np.arange(8), rng.integers(0, 64, 8)] = 0.0
    c["underflow"] = (u, 8, 0)
    c["underflow_norm"] = (u.copy(), 8, 1)
    c["k1"] = (rng.standard_normal((16, 64)).astype(np.float32), 1, 0)
    c["k32"] = (rng.standard_normal((4, 64)).astype(np.float32) * 3, 32, 1)
    c["wide"] = (rng.standard_normal((4, 1024)).astype(np.float32), 8, 1)
    return c


def rms_cases(rng):
    c = {}
    for n in (896, 2048, 8192):
        x = rng.standard_normal((3, n)).astype(np.float32)
        c[f"n{n}_w"] = (x, (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32), 1e-6 if n == 8192 else 1e-5)
        c[f"n{n}"] = (x * np.float32(3.0), None, 1e-5)
    c["tiny"] = ((rng.standard_normal((2, 2048)) * 1e-4).astype(np.float32), None, 1e-6)   # eps comparable to the mean
    c["huge"] = ((rng.standard_normal((2, 2048)) * 1e15).astype(np.float32),
                 (0.5 + rng.random(2048)).astype(np.float32), 1e-5)
    c["zero"] = (np.zeros((1, 896), np.float32), None, 1e-5)
    return c


def main():
    R, G = O.RefEngine("clang"), O.RefEngine("gcc")
    rng = np.random.default_rng(20261202)
    out = {}
    for name, (lg, k, norm) in route_cases(rng).items():
        sel, w = R.route(lg, k, bool(norm))
        sel_g, w_g = G.route(lg, k, bool(norm))
        assert np.array_equal(sel, sel_g) and np.array_equal(w.view(np.uint32), w_g.view(np.uint32)), name
        out[f"route/{name}/logits"] = lg
        out[f"route/{name}/params"] = np.array([k, norm], np.int32)
        out[f"route/{name}/sel"] = sel
        out[f"route/{name}/w"] = w
    for name, (x, w, eps) in rms_cases(rng).items():
        o = R.rmsnorm(x, w, eps)
        assert np.array_equal(o.view(np.uint32), G.rmsnorm(x, w, eps).view(np.uint32)), name
        out[f"rms/{name}/x"] = x
        if w is not None:
            out[f"rms/{name}/w"] = w
        out[f"rms/{name}/eps"] = np.array([eps], np.float32)
        out[f"rms/{name}/o"] = o
    path = os.path.join(HERE, "engine_vectors.npz")
    np.savez_compressed(path, **out)
    print("wrote", len(out), "arrays,", os.path.getsize(path), "bytes")


if __name__ == "__main__":
    main()
