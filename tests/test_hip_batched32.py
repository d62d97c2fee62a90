"""GPU parity of the batched Q4_0 / Q5_0 kernel (one lane per row and activation, chains in registers): bit-identical to the
oracle in every reference order and to the vector kernel, over activation counts that exercise every lane split (2 .. 64
per group, several groups), ragged row counts and padded strides."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

MODES = [(E.ORDER_X86_CONTRACT, O.CONTRACT, O.PATH_X86), (E.ORDER_X86_STRICT, O.STRICT, O.PATH_X86),
         (E.ORDER_SCALAR, O.STRICT, O.PATH_SCALAR)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture
def hipb(hip):
    prev = hip.set_batched32_min(2)
    yield hip
    hip.set_batched32_min(prev)
    hip.set_order(E.ORDER_X86_CONTRACT)


def inputs(orc, t, rows, cols, na, seed):
    st = np.array([seed], np.uint64)
    W = orc.mtest_blocks(t, st, rows, cols)
    x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(t, x)


@pytest.mark.parametrize("t", [O.Q4_0, O.Q5_0], ids=["q4_0", "q5_0"])
@pytest.mark.parametrize("rows,cols,na", [(4096, 2048, 32), (512, 2048, 32), (37, 896, 2), (100, 320, 3), (65, 1024, 64),
                                          (33, 512, 70), (20, 256, 130)])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_batched32_vs_oracle(hipb, orc, t, rows, cols, na, mode):
    hipb.set_order(mode[0])
    W, acts = inputs(orc, t, rows, cols, na, rows + 7 * na + t)
    y = hipb.matvec_multi(t, W, cols, rows, acts)
    ref = orc.matvec_multi(t, W, cols, rows, acts, mode[1], mode[2])
    assert np.array_equal(bits(y), bits(ref))


@pytest.mark.parametrize("t", [O.Q4_0, O.Q5_0], ids=["q4_0", "q5_0"])
def test_batched32_equals_vector_kernel_with_ranges(hipb, orc, t):
    rows, cols, na, r0, r1 = 150, 1024, 19, 9, 141
    W, acts = inputs(orc, t, rows, cols, na, 3)
    ab = acts.strides[0]
    araw = np.zeros((na, ab + 12), np.uint8)
    araw[:, :ab] = acts.view(np.uint8).reshape(na, ab)
    ystride = rows + 3
    out = []
    for off in (False, True):
        prev = hipb.set_batched32_min(0) if off else None
        try:
            dW, dA = hipb.upload(W), hipb.upload(araw)
            dY = hipb.upload(np.full(na * ystride, -555.0, np.float32))
            hipb.matvec_multi_dev(t, dW, cols, r0, r1, dA, araw.strides[0], na, dY, ystride)
            out.append(hipb.download(dY, np.zeros((na, ystride), np.float32)))
        finally:
            if off:
                hipb.set_batched32_min(prev)
    assert np.array_equal(bits(out[0]), bits(out[1]))
    assert np.all(out[0][:, :r0] == -555.0) and np.all(out[0][:, r1:] == -555.0)
