"""GPU parity of the Q5_K form of the direct-activation matrix-core kernel (es_hip_mk.hip: Q4_K's two int8 planes plus a
third for the fifth bit, dot = D_lo + 8 D_hi + 16 D_q5, the scalar mv_q5_K epilogue): bit-identical to the oracle in every
reference order and to the vector kernel, at prompt-sized batches (config 2's shapes at T = 512 and a 70B-sized row),
ragged edges (rows not a multiple of the 64-row tile, activation counts not a multiple of the 128-activation tile, one
superblock per row), row sub-ranges with padded strides, extreme blocks (every fifth bit set, maximal scales and mins),
and gathered activation rows (MoE experts)."""
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
        W = orc.quantize_rows(O.Q5_K, orc.gauss(seed, 0.02, rows * cols).reshape(rows, cols))
        x = orc.gauss(seed + 1, 1.0, na * cols).reshape(na, cols)
    else:
        W = orc.mtest_blocks(O.Q5_K, st, rows, cols)
        x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(O.Q5_K, x)


@pytest.fixture(params=["tok64", "tok128"])
def hip5(hip, request):
    """every Q5_K product with at least one activation on the matrix-core kernel; products short of row tiles in tiles of
    64 activations ("tok64") or always 128 ("tok128")"""
    prev = hip.set_q5k_mfma_min_batch(1)
    prev_64 = hip.set_direct_mfma_tok64(request.param == "tok64")
    yield hip
    hip.set_q5k_mfma_min_batch(prev)
    hip.set_direct_mfma_tok64(prev_64)
    hip.set_order(E.ORDER_X86_CONTRACT)


def vector_path(hip, fn):
    prev = hip.set_q5k_mfma_min_batch(0)
    try:
        return fn()
    finally:
        hip.set_q5k_mfma_min_batch(prev)


@pytest.mark.parametrize("rows,cols,na,gauss", [(300, 512, 65, False), (129, 2048, 64, True), (100, 256, 1, False),
                                                (1, 256, 3, False), (257, 1024, 130, True), (200, 768, 8, False),
                                                (96, 28672, 20, True)])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_q5k_mfma_vs_oracle(hip5, orc, rows, cols, na, gauss, mode):
    hip5.set_order(mode[0])
    W, acts = inputs(orc, rows, cols, na, rows + na + cols, gauss)
    y = hip5.matvec_multi(O.Q5_K, W, cols, rows, acts)
    pick = np.unique(np.array([0, 1, na // 2, 63, 64, na - 1]) % na)
    ref = orc.matvec_multi(O.Q5_K, W, cols, rows, acts[pick], mode[1], mode[2])
    assert np.array_equal(bits(y[pick]), bits(ref))


@pytest.mark.parametrize("rows,cols,na", [(8192, 2048, 512), (2048, 8192, 512)])
def test_q5k_mfma_equals_vector_path_config2(hip5, orc, rows, cols, na):
    """config 2's prefill shapes in Q5_K at T = 512: every output equal to the vector kernel's, bit for bit"""
    W, acts = inputs(orc, rows, cols, na, 3 * rows + na)
    y = hip5.matvec_multi(O.Q5_K, W, cols, rows, acts)
    y_mv = vector_path(hip5, lambda: hip5.matvec_multi(O.Q5_K, W, cols, rows, acts))
    assert np.array_equal(bits(y), bits(y_mv))


def test_q5k_mfma_extreme_blocks(hip5, orc):
    """all-0xFF (every fifth bit set, nibbles 15, scales and mins 63) and all-zero codes, +-127 activations"""
    rows, cols, na = 160, 1024, 70
    W, _ = inputs(orc, rows, cols, na, 5)
    Wb = W.reshape(rows, cols // 256, 176)
    Wb[0::3, :, 4:] = 0xFF
    Wb[1::3, :, 16:] = 0x00
    Wb[2::3, :, 16:48] = 0xFF                    # every fifth bit, codes as they were
    x = np.where(np.arange(na * cols).reshape(na, cols) % 3 == 0, 127.0, -127.0).astype(np.float32)
    x[1::2] *= np.float32(0.5)
    acts = orc.quantize_act(O.Q5_K, x)
    for mode in MODES:
        hip5.set_order(mode[0])
        y = hip5.matvec_multi(O.Q5_K, W, cols, rows, acts)
        ref = orc.matvec_multi(O.Q5_K, W, cols, rows, acts, mode[1], mode[2])
        assert np.array_equal(bits(y), bits(ref)), mode


def test_q5k_mfma_row_range_and_strides(hip5, orc):
    rows, cols, na, r0, r1 = 300, 1024, 70, 37, 251
    W, acts = inputs(orc, rows, cols, na, 99)
    ab = cols // 256 * 292
    astride = ab + 52
    araw = np.zeros(na * astride, np.uint8)
    for q in range(na):
        araw[q * astride:q * astride + ab] = acts[q].view(np.uint8)
    ystride = rows + 13
    sentinel = np.float32(-777.0)
    dW, dA = hip5.upload(W), hip5.upload(araw)
    dY = hip5.upload(np.full(na * ystride, sentinel, np.float32))
    hip5.matvec_multi_dev(O.Q5_K, dW, cols, r0, r1, dA, astride, na, dY, ystride)
    y = hip5.download(dY, np.zeros((na, ystride), np.float32))
    ref = orc.matvec_multi(O.Q5_K, W, cols, rows, acts[[0, 64, 69]])
    assert np.array_equal(bits(y[[0, 64, 69], r0:r1]), bits(ref[:, r0:r1]))
    assert np.all(y[:, :r0] == sentinel) and np.all(y[:, r1:rows] == sentinel) and np.all(y[:, rows:] == sentinel)


@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_q5k_mfma_moe_gathers(hip5, orc, mode):
    """MoE experts with Q5_K gate/up/down: the experts' products gather their activation rows through the token table
    (one expert takes 70 tokens, others a few); bit-identical to the oracle's moe_n restatement"""
    from test_hip_moe import Experts
    hip5.set_order(mode[0])
    n, ff, n_exp, kmax, N = 1024, 512, 5, 2, 80
    types = (E.Q5_K, E.Q5_K, E.Q5_K)
    ex = Experts(hip5, orc, types, n_exp, n, ff, 79)
    rng = np.random.default_rng(10)
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
    x = orc.quantize_act(E.Q5_K, orc.gauss(17, 1.0, N * n).reshape(N, n))
    xb = x.view(np.uint8).reshape(N, -1)
    pad = np.zeros((N, xb.shape[1] + 44), np.uint8)
    pad[:, :xb.shape[1]] = xb
    dx = hip5.upload(pad)
    dout = hip5.upload(np.full((N, n), -777.0, np.float32))
    hip5.moe_ffn(ex.args(k, sel, w), dx, pad.strides[0], dout, n)
    out = hip5.download(dout, np.zeros((N, n), np.float32))
    ref = orc.moe_ffn(types, ex.host, n, ff, x, sel, w, k=k, order=mode[1], path=mode[2])
    assert np.array_equal(bits(out), bits(ref))
