"""GPU parity of the Q6_K matrix-core path (es_hip_mm6.hip), each test with its persistent form for single short-row
products on ("persistent": one workgroup per CU, activations copied into LDS once, row tiles streamed back to back) and
off ("tiled"): bit-identical to the oracle in every reference order and to the vector kernel, at the config 3 head shape
and at ragged edges (rows not a multiple of the 128-row tile, activation counts between the 16/32/64-wide tiles and
above 64, row sub-ranges, padded strides, rows at and past the persistent form's superblock limits), and rows of an odd
number of superblocks (2-byte aligned rows)."""
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
        W = orc.quantize_rows(O.Q6_K, orc.gauss(seed, 0.02, rows * cols).reshape(rows, cols))
        x = orc.gauss(seed + 1, 1.0, na * cols).reshape(na, cols)
    else:
        W = orc.mtest_blocks(O.Q6_K, st, rows, cols)
        x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(O.Q6_K, x)


@pytest.fixture(params=["persistent", "tiled"])
def hip6(hip, request):
    prev = hip.set_q6k_mfma_min_batch(16)
    prevp = hip.set_q6k_persistent(request.param == "persistent")
    yield hip
    hip.set_q6k_mfma_min_batch(prev)
    hip.set_q6k_persistent(prevp)
    hip.set_order(E.ORDER_X86_CONTRACT)


def vector_path(hip, fn):
    """fn() with the Q6_K matrix-core kernel switched off"""
    a = hip.set_q6k_mfma_min_batch(0)
    try:
        return fn()
    finally:
        hip.set_q6k_mfma_min_batch(a)


@pytest.mark.parametrize("rows,cols,na,gauss", [(4096, 1024, 64, True), (300, 1024, 64, False), (200, 2048, 40, False),
                                                (128, 512, 16, True), (77, 512, 23, False), (150, 1024, 130, False),
                                                (64, 4096, 33, True), (40000, 1280, 64, False), (40000, 1536, 64, False),
                                                (33000, 2816, 32, False), (20000, 3072, 32, False), (9000, 5888, 16, False),
                                                (9000, 6144, 16, False)])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_q6k_mfma_vs_oracle(hip6, orc, rows, cols, na, gauss, mode):
    hip6.set_order(mode[0])
    W, acts = inputs(orc, rows, cols, na, rows + 3 * na, gauss)
    y = hip6.matvec_multi(O.Q6_K, W, cols, rows, acts)
    pick = np.unique(np.array([t for t in (0, 1, 15, 16, na // 2, na - 1) if t < na]))
    ref = orc.matvec_multi(O.Q6_K, W, cols, rows, acts[pick], mode[1], mode[2])
    assert np.array_equal(bits(y[pick]), bits(ref))


@pytest.mark.parametrize("rows,cols,na", [(151936, 1024, 64), (1000, 2048, 100), (512, 512, 17)])
def test_q6k_mfma_equals_vector_path(hip6, orc, rows, cols, na):
    """the full config 3 head (151,936 rows, K padded to 1024) at batch 64: matrix-core result == vector-kernel result,
    bit for bit, and three of the activations (first, middle, last) against the oracle"""
    W, acts = inputs(orc, rows, cols, na, 5 * rows + na)
    y_mm = hip6.matvec_multi(O.Q6_K, W, cols, rows, acts)
    y_mv = vector_path(hip6, lambda: hip6.matvec_multi(O.Q6_K, W, cols, rows, acts))
    assert np.array_equal(bits(y_mm), bits(y_mv))
    pick = [0, na // 2, na - 1]
    ref = orc.matvec_multi(O.Q6_K, W, cols, rows, acts[pick])
    assert np.array_equal(bits(y_mm[pick]), bits(ref))


def test_q6k_mfma_row_range_and_strides(hip6, orc):
    rows, cols, na, r0, r1 = 300, 1024, 70, 37, 251
    W, acts = inputs(orc, rows, cols, na, 98)
    ab = cols // 256 * 292
    astride = ab + 52
    araw = np.zeros(na * astride, np.uint8)
    for q in range(na):
        araw[q * astride:q * astride + ab] = acts[q].view(np.uint8)
    ystride = rows + 13
    sentinel = np.float32(-777.0)
    dW, dA = hip6.upload(W), hip6.upload(araw)
    dY = hip6.upload(np.full(na * ystride, sentinel, np.float32))
    hip6.matvec_multi_dev(O.Q6_K, dW, cols, r0, r1, dA, astride, na, dY, ystride)
    y = hip6.download(dY, np.zeros((na, ystride), np.float32))
    ref = orc.matvec_multi(O.Q6_K, W, cols, rows, acts[[0, 69]])
    assert np.array_equal(bits(y[[0, 69], r0:r1]), bits(ref[:, r0:r1]))
    assert np.all(y[:, :r0] == sentinel) and np.all(y[:, r1:rows] == sentinel) and np.all(y[:, rows:] == sentinel)


@pytest.mark.parametrize("cols,na", [(768, 40), (256, 17), (1280, 64), (768, 130)])
def test_q6k_odd_superblock_rows_on_the_matrix_cores(hip6, orc, cols, na):
    """an odd number of superblocks: 210-byte blocks make every other row start 2 bytes past a dword (config 5's
    2048 x 768 down experts); the matrix-core kernel reads them at that alignment and stays exact against the oracle
    and the vector kernel"""
    rows = 200
    W, acts = inputs(orc, rows, cols, na, 77 + cols)
    y = hip6.matvec_multi(O.Q6_K, W, cols, rows, acts)
    ref = orc.matvec_multi(O.Q6_K, W, cols, rows, acts[[0, na // 2, na - 1]])
    assert np.array_equal(bits(y[[0, na // 2, na - 1]]), bits(ref))
    assert np.array_equal(bits(y), bits(vector_path(hip6, lambda: hip6.matvec_multi(O.Q6_K, W, cols, rows, acts))))


def test_q6k_mfma_extreme_codes(hip6, orc):
    """every 6-bit code and scale at its extremes (q = -32 and 31, sc = -128 and 127) against +-127 activations"""
    rows, cols, na = 128, 512, 16
    rng = np.random.default_rng(8)
    W, acts = inputs(orc, rows, cols, na, 5)
    Wb = W.view(np.uint8).reshape(rows, -1).copy()
    for r in range(rows):
        for b in range(cols // 256):
            blk = Wb[r, 210 * b:210 * (b + 1)]
            pat = rng.integers(0, 4)
            if pat == 0:
                blk[:192] = 0xff                                   # q = 63 - 32 = 31 everywhere
            elif pat == 1:
                blk[:192] = 0x00                                   # q = -32 everywhere
            blk[192:208] = rng.choice(np.array([0x80, 0x7f, 0x81, 0x01], np.uint8), 16)   # -128, 127, -127, 1
    W = Wb.reshape(W.shape)
    A = acts.view(np.uint8).reshape(na, -1).copy()
    for t in range(na):
        for b in range(cols // 256):
            blk = A[t, 292 * b:292 * (b + 1)]
            qs = np.where(rng.random(256) < 0.5, 127, -127).astype(np.int8)
            blk[4:260] = qs.view(np.uint8)
            blk[260:292] = qs.reshape(16, 16).sum(axis=1).astype(np.int16).view(np.uint8)
    acts = A.view(acts.dtype).reshape(acts.shape)
    for mode in MODES:
        hip6.set_order(mode[0])
        y = hip6.matvec_multi(O.Q6_K, W, cols, rows, acts)
        ref = orc.matvec_multi(O.Q6_K, W, cols, rows, acts, mode[1], mode[2])
        assert np.array_equal(bits(y), bits(ref)), mode


@pytest.mark.parametrize("na", [64, 20])
def test_q6k_persistent_batch_equals_tiled(hip, orc, na):
    """a batch of three large short-row products (each at least two row tiles per CU, one with a row range) through
    es_hip_run_jobs: the persistent form launched per product equals the tiled form bit for bit, and the oracle on
    sampled rows"""
    rows, cols = 70000, 1024
    W, acts = inputs(orc, rows, cols, na, 77 + na)
    dW, dA = hip.upload(W), hip.upload(acts)
    outs = {}
    for pers in (1, 0):
        prev = hip.set_q6k_persistent(pers)
        prevm = hip.set_q6k_mfma_min_batch(16)
        try:
            dY = [hip.upload(np.full((na, rows), -5.0, np.float32)) for _ in range(3)]
            specs = [dict(type=O.Q6_K, rows=rows, cols=cols, W=dW, act=dA, astride=acts.strides[0], nb=na, y=dY[i],
                          ystride=rows) for i in range(3)]
            hip.run_jobs(specs)
            hip.synchronize()
            outs[pers] = [hip.download(d, np.zeros((na, rows), np.float32)) for d in dY]
        finally:
            hip.set_q6k_persistent(prev)
            hip.set_q6k_mfma_min_batch(prevm)
    for a, b in zip(outs[1], outs[0]):
        assert np.array_equal(bits(a), bits(b))
    sel = np.array([0, 1, 777, 65535, rows - 1])
    ref = orc.matvec_multi(O.Q6_K, W.reshape(rows, -1)[sel].reshape(-1), cols, len(sel), acts[[0, na - 1]])
    assert np.array_equal(bits(outs[1][0][[0, na - 1]][:, sel]), bits(ref))
