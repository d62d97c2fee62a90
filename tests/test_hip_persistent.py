"""GPU parity of the persistent direct-activation kernels (es_hip_mk.hip): Q4_K and Q3_K products of an even number of
superblocks share one launch whose workgroups each compute a host-scheduled list of tiles, their loads running ahead
across tile boundaries. Both forms: pk_kernel (two workgroups per CU, tiles of 64 rows x 128 or 64 activations) and, for
Q4_K, ws_kernel (one workgroup of 8 waves per CU, 128-activation tiles, four waves staging activations and unpacked
weights in LDS for the four that run the matrix cores). Checked bit for bit against the oracle (in every reference
order) and against the same batches with the persistent launch switched off (the per-tile kernels): config 2's three
prefill products in one launch, mixed row lengths and activation counts in one launch, ragged rows and activation counts
(tiles of fewer than 128 activations), row sub-ranges with padded strides, batches of at most 64 activations, many tiles
per workgroup, plans rerun with new inputs, Q3_K."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

MODES = [(E.ORDER_X86_CONTRACT, O.CONTRACT, O.PATH_X86), (E.ORDER_X86_STRICT, O.STRICT, O.PATH_X86),
         (E.ORDER_SCALAR, O.STRICT, O.PATH_SCALAR)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def inputs(orc, t, rows, cols, na, seed, gauss=False):
    st = np.array([seed], np.uint64)
    if gauss:
        W = orc.quantize_rows(t, orc.gauss(seed, 0.02, rows * cols).reshape(rows, cols))
        x = orc.gauss(seed + 1, 1.0, na * cols).reshape(na, cols)
    else:
        W = orc.mtest_blocks(t, st, rows, cols)
        x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(t, x)


@pytest.fixture(params=[3, 2], ids=["pk", "ws"])
def hipp(hip, request):
    """the persistent launch on in one form (3: two workgroups per CU, 2: wave-specialised for Q4_K), every batch of >= 8
    activations eligible"""
    hip.pk_form = request.param
    prev = (hip.set_direct_persistent(request.param), hip.set_direct_mfma_min_batch(8), hip.set_q3k_mfma_min_batch(8))
    yield hip
    hip.set_direct_persistent(prev[0])
    hip.set_direct_mfma_min_batch(prev[1])
    hip.set_q3k_mfma_min_batch(prev[2])
    hip.set_order(E.ORDER_X86_CONTRACT)


def run_batch(hip, prods, persistent):
    """one run_jobs call over prods = [(type, W, cols, rows, acts, r0, r1, ystride)] with the fixture's persistent form
    (or none); outputs [na][ystride]"""
    prev = hip.set_direct_persistent(hip.pk_form if persistent else 0)
    try:
        specs, outs, keep = [], [], []
        for (t, W, cols, rows, acts, r0, r1, ystride) in prods:
            dW, dA = hip.upload(W), hip.upload(acts)
            dY = hip.upload(np.full(len(acts) * ystride, -777.0, np.float32))
            # a job covers rows [0, rows) from its W and y: a sub-range starts both at row r0
            specs.append(dict(type=t, rows=r1 - r0, cols=cols, W=dW.offset(r0 * E.row_bytes(t, cols)), act=dA,
                              astride=acts.strides[0], nb=len(acts), y=dY.offset(4 * r0), ystride=ystride))
            outs.append((dY, len(acts), ystride))
            keep += [dW, dA]
        hip.run_jobs(specs)
        return [hip.download(d, np.zeros((na, ys), np.float32)) for (d, na, ys) in outs]
    finally:
        hip.set_direct_persistent(prev)


def test_config2_prefill_one_launch(hipp, orc):
    """config 2 at T = 512: gate and up (8192 x 2048) and down (2048 x 8192) in one persistent launch; every output equal
    to the per-tile kernels' and oracle picks (tiles of both widths) in the clang order"""
    T = 512
    Wg, xg = inputs(orc, O.Q4_K, 8192, 2048, T, 21, gauss=True)
    Wu, xu = inputs(orc, O.Q4_K, 8192, 2048, T, 22, gauss=True)
    Wd, xd = inputs(orc, O.Q4_K, 2048, 8192, T, 23, gauss=True)
    prods = [(O.Q4_K, Wg, 2048, 8192, xg, 0, 8192, 8192), (O.Q4_K, Wu, 2048, 8192, xu, 0, 8192, 8192),
             (O.Q4_K, Wd, 8192, 2048, xd, 0, 2048, 2048)]
    yp = run_batch(hipp, prods, True)
    yk = run_batch(hipp, prods, False)
    for a, b in zip(yp, yk):
        assert np.array_equal(bits(a), bits(b))
    pick = [0, 63, 64, 127, 128, 300, 511]
    for (t, W, cols, rows, acts, r0, r1, ys), y in zip(prods, yp):
        ref = orc.matvec_multi(t, W, cols, rows, acts[pick])
        assert np.array_equal(bits(y[pick]), bits(ref))


@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_mixed_launch_vs_oracle(hipp, orc, mode):
    """one launch of products with 2, 4, 8 and 32 superblocks per row, ragged rows (not multiples of 64) and activation
    counts (8, 64, 65, 130, 200), row sub-ranges with padded output strides; every output against the oracle"""
    hipp.set_order(mode[0])
    shapes = [(300, 512, 130, 0, 300, 300), (129, 1024, 65, 5, 129, 140), (700, 2048, 200, 64, 650, 701),
              (96, 8192, 64, 0, 96, 100), (64, 2048, 8, 0, 64, 64), (1, 512, 9, 0, 1, 1)]
    prods = []
    for i, (rows, cols, na, r0, r1, ys) in enumerate(shapes):
        W, acts = inputs(orc, O.Q4_K, rows, cols, na, 100 + i, gauss=bool(i & 1))
        prods.append((O.Q4_K, W, cols, rows, acts, r0, r1, ys))
    ys_out = run_batch(hipp, prods, True)
    for (t, W, cols, rows, acts, r0, r1, ys), y in zip(prods, ys_out):
        ref = orc.matvec_multi(t, W, cols, rows, acts, mode[1], mode[2])
        assert np.array_equal(bits(y[:, r0:r1]), bits(ref[:, r0:r1]))
        assert np.all(y[:, :r0] == -777.0) and np.all(y[:, r1:] == -777.0)


def test_many_tiles_per_workgroup(hipp, orc):
    """a batch of 1024 activations on two 8192 x 2048 products (2048 tiles, four or more a workgroup): equal to the
    per-tile kernels everywhere"""
    T = 1024
    Wa, xa = inputs(orc, O.Q4_K, 8192, 2048, T, 31)
    Wb, xb = inputs(orc, O.Q4_K, 8192, 2048, T, 32)
    prods = [(O.Q4_K, Wa, 2048, 8192, xa, 0, 8192, 8192), (O.Q4_K, Wb, 2048, 8192, xb, 0, 8192, 8192)]
    yp = run_batch(hipp, prods, True)
    yk = run_batch(hipp, prods, False)
    for a, b in zip(yp, yk):
        assert np.array_equal(bits(a), bits(b))
    ref = orc.matvec_multi(O.Q4_K, Wa, 2048, 8192, xa[[0, 777, 1023]])
    assert np.array_equal(bits(yp[0][[0, 777, 1023]]), bits(ref))


@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_q3k_persistent(hipp, orc, mode):
    """Q3_K products (110-byte superblocks at 2-byte alignment) in one persistent launch: 64-wide and 128-wide tiles"""
    hipp.set_order(mode[0])
    prods = []
    for i, (rows, cols, na) in enumerate([(2048, 8192, 96), (300, 2048, 130), (64, 512, 20)]):
        W, acts = inputs(orc, O.Q3_K, rows, cols, na, 200 + i, gauss=bool(i & 1))
        prods.append((O.Q3_K, W, cols, rows, acts, 0, rows, rows))
    ys_out = run_batch(hipp, prods, True)
    for (t, W, cols, rows, acts, r0, r1, ys), y in zip(prods, ys_out):
        pick = np.unique(np.array([0, 1, 63, 64, len(acts) - 1]) % len(acts))
        ref = orc.matvec_multi(t, W, cols, rows, acts[pick], mode[1], mode[2])
        assert np.array_equal(bits(y[pick]), bits(ref))


def test_plan_reruns(hipp, orc):
    """a prepared plan of two products run twice, the activations overwritten in between: each run equals the oracle"""
    n, ff, T = 2048, 4096, 96
    Wu, x1 = inputs(orc, O.Q4_K, ff, n, T, 41)
    Wd, h1 = inputs(orc, O.Q4_K, n, ff, T, 42)
    _, x2 = inputs(orc, O.Q4_K, ff, n, T, 43)
    _, h2 = inputs(orc, O.Q4_K, n, ff, T, 44)
    dWu, dWd, dx, dh = hipp.upload(Wu), hipp.upload(Wd), hipp.upload(x1), hipp.upload(h1)
    dyu, dyd = hipp.alloc(T * ff * 4), hipp.alloc(T * n * 4)
    specs = [dict(type=O.Q4_K, rows=ff, cols=n, W=dWu, act=dx, astride=x1.strides[0], nb=T, y=dyu, ystride=ff),
             dict(type=O.Q4_K, rows=n, cols=ff, W=dWd, act=dh, astride=h1.strides[0], nb=T, y=dyd, ystride=n)]
    p = hipp.plan(specs)
    try:
        for (x, h) in ((x1, h1), (x2, h2)):
            for d, a in ((dx, x), (dh, h)):
                assert hipp._L.es_hip_memcpy_h2d(int(d), np.ascontiguousarray(a).ctypes.data, a.nbytes) == 0
            p.run()
            hipp.synchronize()
            yu = hipp.download(dyu, np.zeros((T, ff), np.float32))
            yd = hipp.download(dyd, np.zeros((T, n), np.float32))
            pick = [0, 50, 95]
            assert np.array_equal(bits(yu[pick]), bits(orc.matvec_multi(O.Q4_K, Wu, n, ff, x[pick])))
            assert np.array_equal(bits(yd[pick]), bits(orc.matvec_multi(O.Q4_K, Wd, ff, n, h[pick])))
    finally:
        p.close()
