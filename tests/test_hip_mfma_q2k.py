"""GPU parity of the Q2_K matrix-core kernels, each test run on both: the LDS-staged kernel (es_hip_mm2.hip, "lds") and the
expert-sized kernel that copies the activations' Q8_K rows into LDS once and streams the weights (es_hip_mx.hip, "expert",
for 2 to 64 activations; larger batches stay on the LDS-staged kernel). Bit-identical to the oracle in every reference
order and to the vector kernel, at the config 4 expert shapes and at ragged edges (rows not a multiple of the row tiles,
activation counts between the 16/32/64-wide tiles and above 64, rows of 1 to 16 superblocks, row sub-ranges, padded
strides, matrices at any 4-byte offset), with codes and scales at their extremes."""
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
        W = orc.quantize_rows(O.Q2_K, orc.gauss(seed, 0.02, rows * cols).reshape(rows, cols))
        x = orc.gauss(seed + 1, 1.0, na * cols).reshape(na, cols)
    else:
        W = orc.mtest_blocks(O.Q2_K, st, rows, cols)
        x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(O.Q2_K, x)


@pytest.fixture(params=["lds", "expert"])
def hip2(hip, request):
    prev = hip.set_q2k_mfma_min_batch(2)
    prev_x = hip.set_q2k_expert_max_batch(64 if request.param == "expert" else 1)
    yield hip
    hip.set_q2k_mfma_min_batch(prev)
    hip.set_q2k_expert_max_batch(prev_x)
    hip.set_order(E.ORDER_X86_CONTRACT)


def vector_path(hip, fn):
    """fn() with the Q2_K matrix-core kernels switched off"""
    a, b, c = hip.set_q2k_mfma_min_batch(0), hip.set_small_batch_min(0), hip.set_q2k_expert_max_batch(1)
    try:
        return fn()
    finally:
        hip.set_q2k_mfma_min_batch(a)
        hip.set_small_batch_min(b)
        hip.set_q2k_expert_max_batch(c)


@pytest.mark.parametrize("rows,cols,na,gauss", [(1024, 2048, 2, True), (300, 1024, 5, False), (1024, 2048, 16, True),
                                                (2048, 1024, 24, True), (300, 1024, 64, False),
                                                (200, 2048, 40, False), (77, 768, 9, False), (150, 1024, 130, False),
                                                (64, 4096, 33, True), (1, 256, 17, False), (257, 1280, 31, False),
                                                (130, 3328, 48, True)])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_q2k_mfma_vs_oracle(hip2, orc, rows, cols, na, gauss, mode):
    hip2.set_order(mode[0])
    W, acts = inputs(orc, rows, cols, na, rows + 3 * na, gauss)
    y = hip2.matvec_multi(O.Q2_K, W, cols, rows, acts)
    pick = np.unique(np.array([t for t in (0, 1, 15, 16, na // 2, na - 1) if t < na]))
    ref = orc.matvec_multi(O.Q2_K, W, cols, rows, acts[pick], mode[1], mode[2])
    assert np.array_equal(bits(y[pick]), bits(ref))


@pytest.mark.parametrize("rows,cols,na", [(1024, 2048, 16), (2048, 1024, 32), (1000, 2048, 100), (512, 768, 9)])
def test_q2k_mfma_equals_vector_path(hip2, orc, rows, cols, na):
    """the config 4 expert shapes: matrix-core result == vector-kernel result, bit for bit"""
    W, acts = inputs(orc, rows, cols, na, 5 * rows + na)
    y_mm = hip2.matvec_multi(O.Q2_K, W, cols, rows, acts)
    y_mv = vector_path(hip2, lambda: hip2.matvec_multi(O.Q2_K, W, cols, rows, acts))
    assert np.array_equal(bits(y_mm), bits(y_mv))
    ref = orc.matvec_multi(O.Q2_K, W, cols, rows, acts[:2])
    assert np.array_equal(bits(y_mm[:2]), bits(ref))


@pytest.mark.parametrize("na", [70, 40, 7])
def test_q2k_mfma_row_range_and_strides(hip2, orc, na):
    rows, cols, r0, r1 = 300, 1024, 37, 251
    W, acts = inputs(orc, rows, cols, na, 98)
    ab = cols // 256 * 292
    astride = ab + 52
    araw = np.zeros(na * astride, np.uint8)
    for q in range(na):
        araw[q * astride:q * astride + ab] = acts[q].view(np.uint8)
    ystride = rows + 13
    sentinel = np.float32(-777.0)
    dW, dA = hip2.upload(W), hip2.upload(araw)
    dY = hip2.upload(np.full(na * ystride, sentinel, np.float32))
    hip2.matvec_multi_dev(O.Q2_K, dW, cols, r0, r1, dA, astride, na, dY, ystride)
    y = hip2.download(dY, np.zeros((na, ystride), np.float32))
    ref = orc.matvec_multi(O.Q2_K, W, cols, rows, acts[[0, na - 1]])
    assert np.array_equal(bits(y[[0, na - 1], r0:r1]), bits(ref[:, r0:r1]))
    assert np.all(y[:, :r0] == sentinel) and np.all(y[:, r1:rows] == sentinel) and np.all(y[:, rows:] == sentinel)


@pytest.mark.parametrize("shift", [4, 8, 12])
def test_q2k_mfma_matrix_at_any_4_byte_offset(hip2, orc, shift):
    """the weight matrix starting 4, 8 or 12 bytes past a 16-byte boundary (its superblocks staged through aligned chunks)"""
    rows, cols, na = 200, 768, 20
    W, acts = inputs(orc, rows, cols, na, 60 + shift)
    buf = np.zeros(W.nbytes + 16, np.uint8)
    buf[shift:shift + W.nbytes] = W.view(np.uint8)
    dbuf, dA = hip2.upload(buf), hip2.upload(acts)
    dY = hip2.alloc(na * rows * 4)
    hip2.matvec_multi_dev(O.Q2_K, dbuf.offset(shift), cols, 0, rows, dA, acts.strides[0], na, dY, rows)
    y = hip2.download(dY, np.zeros((na, rows), np.float32))
    ref = orc.matvec_multi(O.Q2_K, W, cols, rows, acts[[0, 19]])
    assert np.array_equal(bits(y[[0, 19]]), bits(ref))


def test_q2k_mfma_extreme_codes(hip2, orc):
    """codes, scales and mins at their extremes (q = 0 and 3, sc and m = 0 and 15) against +-127 activations"""
    rows, cols, na = 128, 512, 16
    rng = np.random.default_rng(9)
    W, acts = inputs(orc, rows, cols, na, 6)
    Wb = W.view(np.uint8).reshape(rows, -1).copy()
    for r in range(rows):
        for b in range(cols // 256):
            blk = Wb[r, 84 * b:84 * (b + 1)]
            pat = rng.integers(0, 3)
            if pat == 0:
                blk[16:80] = 0xff                                  # q = 3 everywhere
            elif pat == 1:
                blk[16:80] = 0x00
            blk[0:16] = rng.choice(np.array([0xff, 0x0f, 0xf0, 0x00, 0x5a], np.uint8), 16)
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
        hip2.set_order(mode[0])
        y = hip2.matvec_multi(O.Q2_K, W, cols, rows, acts)
        ref = orc.matvec_multi(O.Q2_K, W, cols, rows, acts, mode[1], mode[2])
        assert np.array_equal(bits(y), bits(ref)), mode
