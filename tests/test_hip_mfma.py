"""GPU parity of the batched (matrix-core) Q4_K path: bit-identical to the oracle, and to the vector kernels, in every
reference order, at config 2's prefill shapes and at ragged edges (rows not a multiple of the 64-row tile, activation
counts not a multiple of the 128-activation tile, row sub-ranges, padded strides)."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

MODES = [(E.ORDER_X86_CONTRACT, O.CONTRACT, O.PATH_X86), (E.ORDER_X86_STRICT, O.STRICT, O.PATH_X86),
         (E.ORDER_SCALAR, O.STRICT, O.PATH_SCALAR)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def inputs(orc, rows, cols, na, seed, gauss=False):
    st = np.array([seed], np.uint64)
    if gauss:
        W = orc.quantize_rows(O.Q4_K, orc.gauss(seed, 0.02, rows * cols).reshape(rows, cols))
        x = orc.gauss(seed + 1, 1.0, na * cols).reshape(na, cols)
    else:
        W = orc.mtest_blocks(O.Q4_K, st, rows, cols)
        x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(O.Q4_K, x)


@pytest.fixture(params=[8, 32], ids=["lds", "regs"])
def hipm(hip, request):
    """Q4_K batches of 8..31 on the LDS-staged kernel (threshold 8) or on the register-streaming one (threshold 32); the
    direct-activation kernel (tests/test_hip_direct.py) switched off"""
    prev = hip.set_mfma_min_batch(request.param)
    prev_s = hip.set_small_batch_min(8)
    prev_d = hip.set_direct_mfma_min_batch(0)
    yield hip
    hip.set_mfma_min_batch(prev)
    hip.set_small_batch_min(prev_s)
    hip.set_direct_mfma_min_batch(prev_d)
    hip.set_order(E.ORDER_X86_CONTRACT)


def vector_path(hip, fn):
    """fn() with every Q4_K matrix-core kernel switched off"""
    a, b, c = hip.set_mfma_min_batch(0), hip.set_small_batch_min(0), hip.set_direct_mfma_min_batch(0)
    try:
        return fn()
    finally:
        hip.set_mfma_min_batch(a)
        hip.set_small_batch_min(b)
        hip.set_direct_mfma_min_batch(c)


@pytest.mark.parametrize("rows,cols,na,gauss", [(8192, 2048, 40, True), (2048, 8192, 33, False), (768, 2048, 130, False),
                                                (100, 512, 37, False), (64, 256, 128, True)])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_mfma_vs_oracle(hipm, orc, rows, cols, na, gauss, mode):
    hipm.set_order(mode[0])
    W, acts = inputs(orc, rows, cols, na, rows + na, gauss)
    y = hipm.matvec_multi(O.Q4_K, W, cols, rows, acts)
    pick = np.unique(np.array([0, 1, na // 2, na - 1]))
    ref = orc.matvec_multi(O.Q4_K, W, cols, rows, acts[pick], mode[1], mode[2])
    assert np.array_equal(bits(y[pick]), bits(ref))


@pytest.mark.parametrize("rows,cols,na", [(8192, 2048, 512), (2048, 8192, 512), (1000, 1024, 200)])
def test_mfma_equals_vector_path(hipm, orc, rows, cols, na):
    """config 2's full prefill shape (T=512): matrix-core result == vector-kernel result, bit for bit"""
    W, acts = inputs(orc, rows, cols, na, 7 * rows + na)
    y_mm = hipm.matvec_multi(O.Q4_K, W, cols, rows, acts)
    y_mv = vector_path(hipm, lambda: hipm.matvec_multi(O.Q4_K, W, cols, rows, acts))
    assert np.array_equal(bits(y_mm), bits(y_mv))
    ref = orc.matvec_multi(O.Q4_K, W, cols, rows, acts[:2])
    assert np.array_equal(bits(y_mm[:2]), bits(ref))


TILES = [(128, 128, 8), (128, 64, 8), (64, 64, 8), (64, 64, 4), (32, 128, 4)]


@pytest.mark.parametrize("tile", TILES, ids=["x".join(map(str, t)) for t in TILES])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_mfma_every_tile(hip, orc, tile, mode):
    """each workgroup tile of the prefill kernel (forced), on ragged rows and activations: bit-identical to the oracle"""
    rows, cols, na = 200, 1024, 150
    W, acts = inputs(orc, rows, cols, na, 4242)
    hip.set_order(mode[0])
    hip.set_mfma_tile(*tile)
    prev_d = hip.set_direct_mfma_min_batch(0)
    try:
        y = hip.matvec_multi(O.Q4_K, W, cols, rows, acts)
    finally:
        hip.set_mfma_tile(0, 0, 0)
        hip.set_order(E.ORDER_X86_CONTRACT)
        hip.set_direct_mfma_min_batch(prev_d)
    pick = np.array([0, 1, 63, 64, 127, 128, 149])
    ref = orc.matvec_multi(O.Q4_K, W, cols, rows, acts[pick], mode[1], mode[2])
    assert np.array_equal(bits(y[pick]), bits(ref))


def test_mfma_tile_knob_rejects_unknown_shapes(hip):
    for bad in [(128, 128, 4), (64, 128, 8), (96, 64, 8), (128, 16, 8)]:
        with pytest.raises(E.EsHipError):
            hip.set_mfma_tile(*bad)


def test_mfma_row_range_and_strides(hipm, orc):
    rows, cols, na, r0, r1 = 300, 1024, 70, 37, 251
    W, acts = inputs(orc, rows, cols, na, 99)
    ab = cols // 256 * 292
    astride = ab + 52
    araw = np.zeros(na * astride, np.uint8)
    for q in range(na):
        araw[q * astride:q * astride + ab] = acts[q].view(np.uint8)
    ystride = rows + 13
    sentinel = np.float32(-777.0)
    dW, dA = hipm.upload(W), hipm.upload(araw)
    dY = hipm.upload(np.full(na * ystride, sentinel, np.float32))
    hipm.matvec_multi_dev(O.Q4_K, dW, cols, r0, r1, dA, astride, na, dY, ystride)
    y = hipm.download(dY, np.zeros((na, ystride), np.float32))
    ref = orc.matvec_multi(O.Q4_K, W, cols, rows, acts[[0, 69]])
    assert np.array_equal(bits(y[[0, 69], r0:r1]), bits(ref[:, r0:r1]))
    assert np.all(y[:, :r0] == sentinel) and np.all(y[:, r1:rows] == sentinel) and np.all(y[:, rows:] == sentinel)


def test_mfma_in_job_batches_and_plans(hipm, orc):
    """gate and up sharing one activation set (one pre-pass) plus down, in one run_jobs call and in a plan"""
    n, ff, T = 1024, 768, 64
    Wg, xa = inputs(orc, ff, n, T, 11)
    Wu, _ = inputs(orc, ff, n, T, 12)
    Wd, ha = inputs(orc, n, ff, T, 13)
    dWg, dWu, dWd, dxa, dha = (hipm.upload(a) for a in (Wg, Wu, Wd, xa, ha))
    dgu, dy = hipm.alloc(T * 2 * ff * 4), hipm.alloc(T * n * 4)
    specs = [dict(type=O.Q4_K, rows=ff, cols=n, W=dWg, act=dxa, astride=xa.strides[0], nb=T, y=dgu, ystride=2 * ff),
             dict(type=O.Q4_K, rows=ff, cols=n, W=dWu, act=dxa, astride=xa.strides[0], nb=T, y=dgu.offset(ff * 4), ystride=2 * ff),
             dict(type=O.Q4_K, rows=n, cols=ff, W=dWd, act=dha, astride=ha.strides[0], nb=T, y=dy, ystride=n)]
    refs = [orc.matvec_multi(O.Q4_K, Wg, n, ff, xa[:3]), orc.matvec_multi(O.Q4_K, Wu, n, ff, xa[:3]),
            orc.matvec_multi(O.Q4_K, Wd, ff, n, ha[:3])]
    for runner in ("run_jobs", "plan"):
        hipm.memset(dgu, 0, T * 2 * ff * 4)
        hipm.memset(dy, 0, T * n * 4)
        if runner == "run_jobs":
            hipm.run_jobs(specs)
        else:
            p = hipm.plan(specs)
            p.run()
            hipm.synchronize()
            p.close()
        gu = hipm.download(dgu, np.zeros((T, 2 * ff), np.float32))
        y = hipm.download(dy, np.zeros((T, n), np.float32))
        assert np.array_equal(bits(gu[:3, :ff]), bits(refs[0])), runner
        assert np.array_equal(bits(gu[:3, ff:]), bits(refs[1])), runner
        assert np.array_equal(bits(y[:3]), bits(refs[2])), runner


# ---- the small-batch kernel (Q2_K and Q4_K with 8 .. 31 activations, and Q2_K with more) ---------------------------------
def sb_inputs(orc, t, rows, cols, na, seed):
    st = np.array([seed], np.uint64)
    W = orc.mtest_blocks(t, st, rows, cols)
    x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(t, x)


@pytest.mark.parametrize("t,rows,cols,na", [(O.Q2_K, 1024, 2048, 16), (O.Q2_K, 2048, 1024, 17), (O.Q2_K, 300, 512, 64),
                                            (O.Q2_K, 100, 256, 100), (O.Q4_K, 768, 2048, 8), (O.Q4_K, 2048, 768, 31),
                                            (O.Q4_K, 77, 512, 20)])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_small_batch_vs_oracle(hipm, orc, t, rows, cols, na, mode):
    hipm.set_order(mode[0])
    W, acts = sb_inputs(orc, t, rows, cols, na, rows * 3 + na)
    y = hipm.matvec_multi(t, W, cols, rows, acts)
    ref = orc.matvec_multi(t, W, cols, rows, acts, mode[1], mode[2])
    assert np.array_equal(bits(y), bits(ref))


@pytest.mark.parametrize("t", [O.Q2_K, O.Q4_K])
def test_small_batch_equals_vector_path_with_ranges(hipm, orc, t):
    rows, cols, na, r0, r1 = 260, 1024, 24, 13, 251
    W, acts = sb_inputs(orc, t, rows, cols, na, 5)
    ab = acts.strides[0]
    araw = np.zeros((na, ab + 36), np.uint8)
    araw[:, :ab] = acts.view(np.uint8).reshape(na, ab)
    ystride = rows + 7
    out = []
    for fn in (lambda f: f(), lambda f: vector_path(hipm, f)):
        dW, dA = hipm.upload(W), hipm.upload(araw)
        dY = hipm.upload(np.full(na * ystride, -555.0, np.float32))
        fn(lambda: hipm.matvec_multi_dev(t, dW, cols, r0, r1, dA, araw.strides[0], na, dY, ystride))
        out.append(hipm.download(dY, np.zeros((na, ystride), np.float32)))
    assert np.array_equal(bits(out[0]), bits(out[1]))
    assert np.all(out[0][:, :r0] == -555.0) and np.all(out[0][:, r1:] == -555.0)
