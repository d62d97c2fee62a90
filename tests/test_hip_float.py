"""GPU parity of the float path (es_hip_dequant.hip, fdot_kernel): activations prepared without Q8 blocks (es_act_prepare
with no Q8_K buffer, an exhausted Q8_0 arena, or ES_FLOAT_ACT; reference src/es_quant.c:499-512) are multiplied as
es_matvec does for them (src/es_quant.c:1941-1944): each weight row dequantized, then dot_f32 against the fp32 activation
(src/es_quant.c:514-526). Checked bit for bit against the reference's own outputs (the golden fixture, every format)
and against the oracle on larger shapes: decode (one activation) and batches, ragged row counts, chunk tails (32-element
formats whose rows are not a multiple of 256), row sub-ranges with padded strides, and the host drop-ins with
activations of both kinds in one call."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

FMTS = ["Q5_0", "Q4_0", "Q4_K", "Q6_K", "Q2_K", "Q8_0", "Q5_K", "Q3_K"]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def float_dev(hip, t, W, cols, r0, r1, x, ystride=None, xpad=0):
    """es_hip_matvec_float_dev on uploaded copies; rows outside [r0, r1) keep the sentinel -777"""
    na = x.shape[0]
    ystride = r1 if ystride is None else ystride
    xs = cols + xpad
    xp = np.zeros((na, xs), np.float32)
    xp[:, :cols] = x
    dW, dX = hip.upload(W), hip.upload(xp)
    dY = hip.upload(np.full(na * ystride, -777.0, np.float32))
    hip.matvec_float_dev(t, dW, cols, r0, r1, dX, xs, na, dY, ystride)
    y = hip.download(dY, np.zeros((na, ystride), np.float32))
    for b in (dW, dX, dY):
        b.close()
    return y


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", ["mtest", "gauss"])
def test_float_path_vs_reference(hip, golden, F, case):
    """the reference's float-path outputs (rows [3, rows), every activation), one call per activation and one call for all"""
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/{case}_shape"])
    W, x, want = golden[f"{F}/{case}_W"], golden[f"{F}/{case}_x"], golden[f"{F}/{case}_yfloat"]
    y = float_dev(hip, t, W, cols, 3, rows, x)
    assert np.array_equal(bits(y[:, 3:]), bits(want[:, 3:])) and np.all(y[:, :3] == -777.0)
    for q in (0, x.shape[0] - 1):
        y1 = float_dev(hip, t, W, cols, 3, rows, x[q:q + 1])
        assert np.array_equal(bits(y1[0, 3:]), bits(want[q, 3:]))


@pytest.mark.parametrize("F,rows,cols,na", [("Q4_K", 300, 8192, 1), ("Q4_K", 77, 2048, 13), ("Q6_K", 129, 768, 9),
                                            ("Q4_0", 70, 896, 1), ("Q4_0", 33, 896, 20), ("Q5_0", 45, 2080, 3),
                                            ("Q8_0", 17, 4128, 2), ("Q2_K", 40, 2048, 1), ("Q3_K", 50, 1024, 17),
                                            ("Q5_K", 23, 512, 8)])
def test_float_path_shapes_vs_oracle(hip, orc, F, rows, cols, na):
    """ragged row counts (not multiples of the 16- or 8-row tiles), activation counts around the 8-wide tile, rows whose
    length leaves a partial 256-column chunk (896, 2080, 4128), a row sub-range with padded x and y strides"""
    t = O.TYPES[F]
    st = np.array([1000 + t + rows], np.uint64)
    W = orc.mtest_blocks(t, st, rows, cols)
    x = orc.gauss(rows + na, 1.0, na * cols).reshape(na, cols)
    ref = orc.matvec_float(t, W, cols, rows, x)
    y = float_dev(hip, t, W, cols, 0, rows, x)
    assert np.array_equal(bits(y), bits(ref))
    r0, r1 = 5, rows - 2
    y = float_dev(hip, t, W, cols, r0, r1, x, ystride=rows + 3, xpad=64)
    assert np.array_equal(bits(y[:, r0:r1]), bits(ref[:, r0:r1]))
    assert np.all(y[:, :r0] == -777.0) and np.all(y[:, r1:] == -777.0)


def test_float_path_large_values(hip, orc):
    """activations spanning many binades (products that cancel): each running sum's rounding order shows"""
    t, rows, cols, na = O.Q8_0, 64, 4096, 4
    W = orc.quantize_rows(t, orc.gauss(3, 0.02, rows * cols).reshape(rows, cols))
    x = orc.gauss(4, 1.0, na * cols).reshape(na, cols) * np.float32(2.0) ** np.random.default_rng(9).integers(-20, 21, (na, cols))
    x = x.astype(np.float32)
    assert np.array_equal(bits(float_dev(hip, t, W, cols, 0, rows, x)), bits(orc.matvec_float(t, W, cols, rows, x)))


@pytest.mark.parametrize("F", ["Q4_K", "Q4_0", "Q6_K"])
def test_host_drop_ins_mixed_activations(hip, orc, F):
    """es_hip_matvec / es_hip_matvec_multi with host activations of both kinds in one call: those with blocks give the
    integer path's outputs, those without (q8 = q80 = NULL) the float path's, as es_matvec_multi falls back to es_matvec
    per activation in the reference (src/es_quant.c:1850)"""
    t = O.TYPES[F]
    rows, cols, na = 96, 2048, 5
    W = orc.quantize_rows(t, orc.gauss(t + 50, 0.02, rows * cols).reshape(rows, cols))
    x = orc.gauss(t + 51, 1.0, na * cols).reshape(na, cols)
    acts = orc.quantize_act(t, x)
    yi = orc.matvec_multi(t, W, cols, rows, acts)
    yf = orc.matvec_float(t, W, cols, rows, x)
    floats = (1, 4)
    y = np.zeros((na, rows + 7), np.float32)
    hip.host_matvec_multi(t, W, cols, 2, rows, acts, y, x=x, floats=floats)
    for q in range(na):
        want = yf[q] if q in floats else yi[q]
        assert np.array_equal(bits(y[q, 2:rows]), bits(want[2:])), q
        assert np.all(y[q, :2] == 0) and np.all(y[q, rows:] == 0)
    y1 = np.zeros((1, rows), np.float32)   # es_hip_matvec, one float activation
    hip.host_matvec_multi(t, W, cols, 0, rows, None, y1, x=x[2:3])
    assert np.array_equal(bits(y1[0]), bits(yf[2]))


def test_run_jobs_host_float_activations(hip, orc):
    """the engine's queue on host memory with a job whose activations carry no blocks and one with both kinds"""
    n, ff, na = 1024, 512, 3
    Wg = orc.quantize_rows(O.Q4_K, orc.gauss(61, 0.02, ff * n).reshape(ff, n))
    Wd = orc.quantize_rows(O.Q6_K, orc.gauss(62, 0.02, n * ff).reshape(n, ff))
    x = orc.gauss(63, 1.0, na * n).reshape(na, n)
    h = orc.gauss(64, 1.0, na * ff).reshape(na, ff)
    hacts = orc.quantize_act(O.Q6_K, h)
    yg = np.zeros((na, ff), np.float32)
    yd = np.zeros((na, n), np.float32)
    hip.run_jobs_host([(O.Q4_K, Wg, ff, n, None, yg, x, ()), (O.Q6_K, Wd, n, ff, hacts, yd, h, (0,))])
    assert np.array_equal(bits(yg), bits(orc.matvec_float(O.Q4_K, Wg, n, ff, x)))
    assert np.array_equal(bits(yd[0]), bits(orc.matvec_float(O.Q6_K, Wd, ff, n, h[:1])[0]))
    assert np.array_equal(bits(yd[1:]), bits(orc.matvec_multi(O.Q6_K, Wd, ff, n, hacts[1:])))


def test_float_path_refusals(hip):
    """bad calls fail with an error and launch nothing: an activation with neither blocks nor floats, a misaligned W, x
    stride below cols, overlapping outputs"""
    W = np.zeros(144 * 4, np.uint8)
    y = np.zeros((1, 4), np.float32)
    recs = E.act_records(O.Q4_K, None, 256, np.zeros((1, 256), np.float32))
    recs[0].x = None
    hip._L.es_hip_matvec(O.Q4_K, W.ctypes.data, 256, 0, 4, recs, y.ctypes.data, None)
    assert "neither" in hip.last_error()
    buf = hip.alloc(1 << 16)
    with pytest.raises(E.EsHipError):
        hip.matvec_float_dev(O.Q4_K, buf.offset(1), 256, 0, 4, buf, 0, 1, buf, 0)
    with pytest.raises(E.EsHipError):
        hip.matvec_float_dev(O.Q4_K, buf, 256, 0, 4, buf, 128, 2, buf, 8)
    with pytest.raises(E.EsHipError):
        hip.matvec_float_dev(O.Q4_K, buf, 256, 0, 4, buf, 256, 2, buf, 2)
    with pytest.raises(E.EsHipError):
        hip.matvec_float_dev(O.Q4_K, buf, 300, 0, 4, buf, 0, 1, buf, 0)
    hip.matvec_float_dev(O.Q4_K, buf, 256, 4, 4, buf, 0, 1, buf, 0)   # empty range: nothing to do
    buf.close()
