"""GPU parity of the device activation preparation (es_hip_act.hip): es_act_prepare's Q8_0 / Q8_K blocks byte for byte,
and the fused rmsnorm / SwiGLU values bit for bit, against the oracle (whose quantizers are pinned to the reference's own
outputs). Edge cases: zero rows and blocks, ties at .5 under both rounding rules (half away from zero for Q8_0, half to
even for Q8_K), |x| = amax, negative zero, tiny and huge magnitudes, Q8_0-only widths, padded strides."""
import numpy as np
import pytest

import es_hip_quant as E

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def blocks(orc, x, which):
    """the oracle's blocks of each row of x, as bytes [rows, row_bytes]"""
    q = [orc.quantize_q8_0(r) if which == "q80" else orc.quantize_q8_K(r) for r in x]
    return np.stack([b.view(np.uint8).reshape(-1) for b in q])


def edge_rows(cols, rng):
    rows = []
    rows.append(np.zeros(cols, np.float32))                                     # all zero
    r = rng.standard_normal(cols).astype(np.float32)
    r[: min(cols, 256)] = 0.0                                                    # a zero block, then data
    rows.append(r)
    t = np.resize(np.array([2.5, -3.5, 0.5, -0.5, 1.5, 126.5, -127.0, 127.0], np.float32), cols)   # amax 127: d = 1
    rows.append(t)
    rows.append((rng.standard_normal(cols) * 1e-30).astype(np.float32))          # tiny
    rows.append((rng.standard_normal(cols) * 1e30).astype(np.float32))           # huge
    n = rng.standard_normal(cols).astype(np.float32)
    n[::7] = -0.0
    n[3] = -np.abs(n).max() * 1.0                                                 # |x| = amax, negative
    rows.append(n)
    return np.stack(rows)


@pytest.mark.parametrize("cols", [32, 96, 256, 896, 2048, 2080, 8192])
def test_act_prepare_matches_reference_quantizers(hip, orc, cols):
    rng = np.random.default_rng(cols)
    x = np.concatenate([(rng.standard_normal((5, cols)) * s).astype(np.float32) for s in (1e-3, 1.0, 30.0)] +
                       [edge_rows(cols, rng)])
    rows = x.shape[0]
    want80 = blocks(orc, x, "q80")
    k = cols % 256 == 0
    dx = hip.upload(x)
    d80 = hip.alloc(want80.nbytes)
    d8k = hip.alloc(rows * (cols // 256) * 292) if k else None
    hip.act_prepare_dev(dx, 0, rows, cols, d80, 0, d8k, 0)
    assert np.array_equal(hip.download(d80, np.zeros_like(want80)), want80)
    if k:
        want8k = blocks(orc, x, "q8k")
        assert np.array_equal(hip.download(d8k, np.zeros_like(want8k)), want8k)


def test_act_prepare_strides_and_single_output(hip, orc):
    rows, cols = 7, 512
    x = np.random.default_rng(1).standard_normal((rows, cols)).astype(np.float32)
    xs, s80, s8k = cols + 32, (cols // 32) * 36 + 20, (cols // 256) * 292 + 8
    xp = np.zeros((rows, xs), np.float32)
    xp[:, :cols] = x
    d80 = hip.upload(np.full(rows * s80, 0xAB, np.uint8))
    d8k = hip.upload(np.full(rows * s8k, 0xCD, np.uint8))
    dx = hip.upload(xp)
    hip.act_prepare_dev(dx, xs, rows, cols, d80, s80, None, 0)
    hip.act_prepare_dev(dx, xs, rows, cols, None, 0, d8k, s8k)
    g80 = hip.download(d80, np.zeros((rows, s80), np.uint8))
    g8k = hip.download(d8k, np.zeros((rows, s8k), np.uint8))
    assert np.array_equal(g80[:, :(cols // 32) * 36], blocks(orc, x, "q80")) and np.all(g80[:, (cols // 32) * 36:] == 0xAB)
    assert np.array_equal(g8k[:, :(cols // 256) * 292], blocks(orc, x, "q8k")) and np.all(g8k[:, (cols // 256) * 292:] == 0xCD)


@pytest.mark.parametrize("cols,eps,weighted", [(2048, 1e-5, True), (8192, 1e-6, True), (896, 1e-6, False), (16384, 1e-5, True),
                                               (256, 1e-5, False), (96, 1e-6, True)])
def test_rmsnorm_prepare(hip, orc, cols, eps, weighted):
    rng = np.random.default_rng(cols + 1)
    x = np.concatenate([(rng.standard_normal((6, cols)) * s).astype(np.float32) for s in (0.01, 1.0, 50.0)] +
                       [np.zeros((1, cols), np.float32), np.full((1, cols), 0.75, np.float32)])
    rows = x.shape[0]
    w = (1.0 + 0.2 * rng.standard_normal(cols)).astype(np.float32) if weighted else None
    xn_want = orc.rmsnorm(x, w, eps)
    dx, dw = hip.upload(x), (hip.upload(w) if weighted else None)
    dxn = hip.alloc(x.nbytes)
    d80 = hip.alloc(rows * (cols // 32) * 36)
    k = cols % 256 == 0
    d8k = hip.alloc(rows * (cols // 256) * 292) if k else None
    hip.rmsnorm_prepare_dev(dx, 0, dw, eps, rows, cols, dxn, 0, d80, 0, d8k, 0)
    xn = hip.download(dxn, np.zeros_like(x))
    assert np.array_equal(bits(xn), bits(xn_want))
    assert np.array_equal(hip.download(d80, np.zeros((rows, (cols // 32) * 36), np.uint8)), blocks(orc, xn_want, "q80"))
    if k:
        assert np.array_equal(hip.download(d8k, np.zeros((rows, (cols // 256) * 292), np.uint8)), blocks(orc, xn_want, "q8k"))


@pytest.mark.parametrize("ff", [96, 768, 1024, 2048, 8192])
def test_swiglu_prepare(hip, orc, ff):
    rng = np.random.default_rng(ff + 2)
    rows = 9
    gu = (rng.standard_normal((rows, 2 * ff)) * 4.0).astype(np.float32)
    gu[0, :ff] = np.linspace(-100.0, 100.0, ff, dtype=np.float32)   # expf from underflow to overflow
    gu[1, :] = 0.0
    h_want = np.stack([orc.swiglu(gu[r, :ff], gu[r, ff:]) for r in range(rows)])
    gs = 2 * ff + 64
    gp = np.zeros((rows, gs), np.float32)
    gp[:, :2 * ff] = gu
    dgu = hip.upload(gp)
    dh = hip.alloc(h_want.nbytes)
    d80 = hip.alloc(rows * (ff // 32) * 36)
    k = ff % 256 == 0
    d8k = hip.alloc(rows * (ff // 256) * 292) if k else None
    hip.swiglu_prepare_dev(dgu, gs, rows, ff, dh, 0, d80, 0, d8k, 0)
    assert np.array_equal(bits(hip.download(dh, np.zeros_like(h_want))), bits(h_want))
    assert np.array_equal(hip.download(d80, np.zeros((rows, (ff // 32) * 36), np.uint8)), blocks(orc, h_want, "q80"))
    if k:
        assert np.array_equal(hip.download(d8k, np.zeros((rows, (ff // 256) * 292), np.uint8)), blocks(orc, h_want, "q8k"))


def test_act_prepare_rejects_bad_arguments(hip):
    dx, d = hip.alloc(4096 * 4), hip.alloc(1 << 16)
    with pytest.raises(E.EsHipError):
        hip.act_prepare_dev(dx, 0, 2, 100, d, 0, None, 0)          # Q8_0 needs cols % 32 == 0
    with pytest.raises(E.EsHipError):
        hip.act_prepare_dev(dx, 0, 2, 96, None, 0, d, 0)           # Q8_K needs cols % 256 == 0
    with pytest.raises(E.EsHipError):
        hip.act_prepare_dev(dx, 0, 2, 256, None, 0, None, 0)       # nothing asked for
    with pytest.raises(E.EsHipError):
        hip.rmsnorm_prepare_dev(dx, 0, None, 1e-5, 1, 16640, None, 0, d, 0, None, 0)   # above the LDS-staged row length
    with pytest.raises(E.EsHipError):
        hip.rmsnorm_prepare_dev(dx, 0, None, 1e-5, 1, 100, d, 0, None, 0, None, 0)      # not a multiple of 32


def test_rmsnorm_matches_reference_engine_goldens(hip, engine_golden):
    """device rmsnorm on the rows the reference engine's own rmsnorm() was run on (tests/golden/engine_vectors.npz):
    bit-identical floats, weighted and unweighted, n = 896, 2048, 8192, tiny / huge / zero rows"""
    from conftest import golden_cases
    for c in golden_cases(engine_golden, "rms"):
        x = engine_golden[f"rms/{c}/x"]
        w = engine_golden.get(f"rms/{c}/w")
        rows, cols = x.shape
        dx, dxn = hip.upload(x), hip.alloc(x.nbytes)
        dw = hip.upload(w) if w is not None else None
        d80 = hip.alloc(rows * (cols // 32) * 36)
        hip.rmsnorm_prepare_dev(dx, 0, dw, float(engine_golden[f"rms/{c}/eps"][0]), rows, cols, dxn, 0, d80, 0, None, 0)
        assert np.array_equal(bits(hip.download(dxn, np.zeros_like(x))), bits(engine_golden[f"rms/{c}/o"])), c
