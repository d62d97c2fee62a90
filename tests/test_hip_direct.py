"""GPU parity of the direct-activation Q4_K matrix-core kernel (es_hip_mk.hip: reads the Q8_K rows itself, no pre-pass):
bit-identical to the oracle in every reference order and to the vector kernels, at config 2's full prefill shapes
(T = 512: gate/up 8192x2048, down 2048x8192) and at ragged edges: rows not a multiple of the 128-row tile, activation
counts not a multiple of the 64-activation tile (1, 3, 63, 65, 130), one superblock per row, row sub-ranges with padded
activation and output strides, extreme blocks, gathered activation rows (MoE experts), job batches and plans."""
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


@pytest.fixture
def hipd(hip):
    """every Q4_K product with at least one activation on the direct-activation kernel"""
    prev, prev_t = hip.set_direct_mfma_min_batch(1), hip.set_direct_mfma_min_tiles(1)
    yield hip
    hip.set_direct_mfma_min_batch(prev)
    hip.set_direct_mfma_min_tiles(prev_t)
    hip.set_order(E.ORDER_X86_CONTRACT)


def vector_path(hip, fn):
    a, b, c = hip.set_mfma_min_batch(0), hip.set_small_batch_min(0), hip.set_direct_mfma_min_batch(0)
    try:
        return fn()
    finally:
        hip.set_mfma_min_batch(a)
        hip.set_small_batch_min(b)
        hip.set_direct_mfma_min_batch(c)


@pytest.mark.parametrize("rows,cols,na,gauss", [(8192, 2048, 512, True), (2048, 8192, 130, False), (300, 512, 65, False),
                                                (129, 2048, 64, True), (100, 256, 1, False), (1, 256, 3, False),
                                                (257, 1024, 63, True), (200, 768, 70, False), (96, 1280, 129, True)])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_direct_vs_oracle(hipd, orc, rows, cols, na, gauss, mode):
    hipd.set_order(mode[0])
    W, acts = inputs(orc, rows, cols, na, rows + na + cols, gauss)
    y = hipd.matvec_multi(O.Q4_K, W, cols, rows, acts)
    pick = np.unique(np.array([0, 1, na // 2, 63, 64, na - 1]) % na)
    ref = orc.matvec_multi(O.Q4_K, W, cols, rows, acts[pick], mode[1], mode[2])
    assert np.array_equal(bits(y[pick]), bits(ref))


@pytest.mark.parametrize("rows,cols,na", [(8192, 2048, 512), (2048, 8192, 512)])
def test_direct_equals_vector_path_config2(hipd, orc, rows, cols, na):
    """config 2's full prefill shapes at T = 512: every output equal to the vector kernel's, bit for bit"""
    W, acts = inputs(orc, rows, cols, na, 3 * rows + na)
    y = hipd.matvec_multi(O.Q4_K, W, cols, rows, acts)
    y_mv = vector_path(hipd, lambda: hipd.matvec_multi(O.Q4_K, W, cols, rows, acts))
    assert np.array_equal(bits(y), bits(y_mv))


def test_direct_extreme_blocks(hipd, orc):
    """all-0xFF and all-zero weight codes, maximal 6-bit scales and mins, +-127 activations"""
    rows, cols, na = 160, 1024, 70
    W, _ = inputs(orc, rows, cols, na, 5)
    Wb = W.reshape(rows, cols // 256, 144)
    Wb[0::3, :, 4:] = 0xFF                       # every scale and min 63, every nibble 15
    Wb[1::3, :, 16:] = 0x00                      # zero codes
    x = np.where(np.arange(na * cols).reshape(na, cols) % 3 == 0, 127.0, -127.0).astype(np.float32)
    x[1::2] *= np.float32(0.5)
    acts = orc.quantize_act(O.Q4_K, x)
    for mode in MODES:
        hipd.set_order(mode[0])
        y = hipd.matvec_multi(O.Q4_K, W, cols, rows, acts)
        ref = orc.matvec_multi(O.Q4_K, W, cols, rows, acts, mode[1], mode[2])
        assert np.array_equal(bits(y), bits(ref)), mode


def test_direct_row_range_and_strides(hipd, orc):
    rows, cols, na, r0, r1 = 300, 1024, 70, 37, 251
    W, acts = inputs(orc, rows, cols, na, 99)
    ab = cols // 256 * 292
    astride = ab + 52
    araw = np.zeros(na * astride, np.uint8)
    for q in range(na):
        araw[q * astride:q * astride + ab] = acts[q].view(np.uint8)
    ystride = rows + 13
    sentinel = np.float32(-777.0)
    dW, dA = hipd.upload(W), hipd.upload(araw)
    dY = hipd.upload(np.full(na * ystride, sentinel, np.float32))
    hipd.matvec_multi_dev(O.Q4_K, dW, cols, r0, r1, dA, astride, na, dY, ystride)
    y = hipd.download(dY, np.zeros((na, ystride), np.float32))
    ref = orc.matvec_multi(O.Q4_K, W, cols, rows, acts[[0, 64, 69]])
    assert np.array_equal(bits(y[[0, 64, 69], r0:r1]), bits(ref[:, r0:r1]))
    assert np.all(y[:, :r0] == sentinel) and np.all(y[:, r1:rows] == sentinel) and np.all(y[:, rows:] == sentinel)


def test_direct_in_job_batches_and_plans(hipd, orc):
    """gate and up sharing one activation set plus down, in one run_jobs call and in a plan (config 2 at T = 64)"""
    n, ff, T = 2048, 8192, 64
    Wg, xa = inputs(orc, ff, n, T, 11)
    Wu, _ = inputs(orc, ff, n, T, 12)
    Wd, ha = inputs(orc, n, ff, T, 13)
    dWg, dWu, dWd, dxa, dha = (hipd.upload(a) for a in (Wg, Wu, Wd, xa, ha))
    dgu, dy = hipd.alloc(T * 2 * ff * 4), hipd.alloc(T * n * 4)
    specs = [dict(type=O.Q4_K, rows=ff, cols=n, W=dWg, act=dxa, astride=xa.strides[0], nb=T, y=dgu, ystride=2 * ff),
             dict(type=O.Q4_K, rows=ff, cols=n, W=dWu, act=dxa, astride=xa.strides[0], nb=T, y=dgu.offset(ff * 4), ystride=2 * ff),
             dict(type=O.Q4_K, rows=n, cols=ff, W=dWd, act=dha, astride=ha.strides[0], nb=T, y=dy, ystride=n)]
    pick = [0, 31, 63]
    refs = [orc.matvec_multi(O.Q4_K, Wg, n, ff, xa[pick]), orc.matvec_multi(O.Q4_K, Wu, n, ff, xa[pick]),
            orc.matvec_multi(O.Q4_K, Wd, ff, n, ha[pick])]
    for runner in ("run_jobs", "plan"):
        hipd.memset(dgu, 0, T * 2 * ff * 4)
        hipd.memset(dy, 0, T * n * 4)
        if runner == "run_jobs":
            hipd.run_jobs(specs)
        else:
            p = hipd.plan(specs)
            p.run()
            hipd.synchronize()
            p.close()
        gu = hipd.download(dgu, np.zeros((T, 2 * ff), np.float32))
        y = hipd.download(dy, np.zeros((T, n), np.float32))
        assert np.array_equal(bits(gu[pick, :ff]), bits(refs[0])), runner
        assert np.array_equal(bits(gu[pick, ff:]), bits(refs[1])), runner
        assert np.array_equal(bits(y[pick]), bits(refs[2])), runner


@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_direct_moe_gathers(hipd, orc, mode):
    """MoE experts with Q4_K gate/up on the direct kernel: activation rows gathered through the expert's token table (one
    expert takes 70 tokens, others a few), a padded token stride; bit-identical to the oracle's moe_n restatement"""
    from test_hip_moe import Experts
    hipd.set_order(mode[0])
    n, ff, n_exp, kmax, N = 1024, 512, 5, 2, 80
    types = (E.Q4_K, E.Q4_K, E.Q4_K)
    ex = Experts(hipd, orc, types, n_exp, n, ff, 77)
    rng = np.random.default_rng(8)
    k = np.full(N, kmax, np.int32)
    k[::9] = 1
    sel = np.zeros((N, kmax), np.int32)
    for t in range(N):
        sel[t] = rng.permutation(n_exp)[:kmax]
        if t < 70:
            sel[t, 0] = 3
            if sel[t, 1] == 3:
                sel[t, 1] = 4
    w = rng.random((N, kmax)).astype(np.float32)
    x = orc.quantize_act(E.Q4_K, orc.gauss(15, 1.0, N * n).reshape(N, n))
    xb = x.view(np.uint8).reshape(N, -1)
    pad = np.zeros((N, xb.shape[1] + 44), np.uint8)
    pad[:, :xb.shape[1]] = xb
    dx = hipd.upload(pad)
    dout = hipd.upload(np.full((N, n), -777.0, np.float32))
    hipd.moe_ffn(ex.args(k, sel, w), dx, pad.strides[0], dout, n)
    out = hipd.download(dout, np.zeros((N, n), np.float32))
    ref = orc.moe_ffn(types, ex.host, n, ff, x, sel, w, k=k, order=mode[1], path=mode[2])
    assert np.array_equal(bits(out), bits(ref))
