"""GPU parity of the batched Q4_0 / Q5_0 / Q8_0 kernels, each test run on all three: the matrix-core one reading the
activations' Q8_0 rows from LDS ("direct", es_hip_mbx.hip: one int8 MFMA per block for 4 rows x 32 activations), the
matrix-core one reading a pre-pass layout ("mfma", es_hip_mb.hip) and the one-lane-per-output one ("lanes",
es_hip_mv.hip): bit-identical to the oracle in every reference order and to the vector kernel, over activation counts that
exercise every lane split and token tile (2 .. 64 per group, several groups, 130), ragged row counts, rows of every block
count around the load pipeline's depth and across the direct kernel's LDS size classes (up to 128 blocks, and past them,
where the pre-pass kernel takes over), 2-byte aligned rows, extreme codes and padded strides."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

MODES = [(E.ORDER_X86_CONTRACT, O.CONTRACT, O.PATH_X86), (E.ORDER_X86_STRICT, O.STRICT, O.PATH_X86),
         (E.ORDER_SCALAR, O.STRICT, O.PATH_SCALAR)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


KERNELS = {"direct": (2, 1), "mfma": (2, 0), "lanes": (0, 0)}   # (es_hip_set_batched32_mfma_min, _direct) per kernel


@pytest.fixture(params=list(KERNELS))
def hipb(hip, request):
    prev = hip.set_batched32_min(2)
    prevm = hip.set_batched32_mfma_min(KERNELS[request.param][0])
    prevd = hip.set_batched32_direct(KERNELS[request.param][1])
    yield hip
    hip.set_batched32_min(prev)
    hip.set_batched32_mfma_min(prevm)
    hip.set_batched32_direct(prevd)
    hip.set_order(E.ORDER_X86_CONTRACT)


def inputs(orc, t, rows, cols, na, seed):
    st = np.array([seed], np.uint64)
    W = orc.mtest_blocks(t, st, rows, cols)
    x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(t, x)


@pytest.mark.parametrize("t", [O.Q4_0, O.Q5_0, O.Q8_0], ids=["q4_0", "q5_0", "q8_0"])
@pytest.mark.parametrize("rows,cols,na", [(4096, 2048, 32), (512, 2048, 32), (37, 896, 2), (100, 320, 3), (65, 1024, 64),
                                          (33, 512, 70), (20, 256, 130)])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_batched32_vs_oracle(hipb, orc, t, rows, cols, na, mode):
    hipb.set_order(mode[0])
    W, acts = inputs(orc, t, rows, cols, na, rows + 7 * na + t)
    y = hipb.matvec_multi(t, W, cols, rows, acts)
    ref = orc.matvec_multi(t, W, cols, rows, acts, mode[1], mode[2])
    assert np.array_equal(bits(y), bits(ref))


@pytest.mark.parametrize("t", [O.Q4_0, O.Q5_0, O.Q8_0], ids=["q4_0", "q5_0", "q8_0"])
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


@pytest.mark.parametrize("t", [O.Q4_0, O.Q5_0, O.Q8_0], ids=["q4_0", "q5_0", "q8_0"])
@pytest.mark.parametrize("cols", [32, 96, 224, 256, 288, 544, 2080, 3104, 4096, 4128])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_batched32_block_counts(hipb, orc, t, cols, mode):
    """1 .. 129 blocks per row: fewer than, exactly and just past the 8 blocks the matrix-core kernels keep in flight, the
    direct kernel's LDS size classes (32, 64, 128 blocks) and one block past the last; odd block counts give rows that
    start only 2-byte aligned"""
    hipb.set_order(mode[0])
    rows, na = 45, 33
    W, acts = inputs(orc, t, rows, cols, na, cols + t)
    y = hipb.matvec_multi(t, W, cols, rows, acts)
    ref = orc.matvec_multi(t, W, cols, rows, acts, mode[1], mode[2])
    assert np.array_equal(bits(y), bits(ref))


@pytest.mark.parametrize("t", [O.Q4_0, O.Q5_0, O.Q8_0], ids=["q4_0", "q5_0", "q8_0"])
def test_batched32_extreme_codes(hipb, orc, t):
    """codes at both ends (0 and 15 / 31, every high bit set or clear; Q8_0: -128 and 127) against activations of +-127"""
    rows, cols, na = 40, 512, 32
    rng = np.random.default_rng(11)
    W, acts = inputs(orc, t, rows, cols, na, 4)
    bb = O.BLOCK_BYTES[t]
    Wb = W.view(np.uint8).reshape(rows, -1).copy()
    for r in range(rows):
        for b in range(cols // 32):
            blk = Wb[r, bb * b:bb * (b + 1)]
            pat = rng.integers(0, 3)
            if pat < 2 and t == O.Q8_0:
                blk[2:] = 0x80 if pat == 0 else 0x7f          # int8 codes -128 / 127
            elif pat < 2:
                blk[bb - 16:] = 0xff if pat == 0 else 0x00
                if t == O.Q5_0:
                    blk[2:6] = 0xff if pat == 0 else 0x00
    W = Wb.reshape(W.shape)
    A = acts.view(np.uint8).reshape(na, -1).copy()
    for q in range(na):
        for b in range(cols // 32):
            A[q, 36 * b + 4:36 * (b + 1)] = np.where(rng.random(32) < 0.5, 127, 0x81).astype(np.uint8)   # +127 / -127
    acts = A.view(acts.dtype).reshape(acts.shape)
    for mode in MODES:
        hipb.set_order(mode[0])
        y = hipb.matvec_multi(t, W, cols, rows, acts)
        ref = orc.matvec_multi(t, W, cols, rows, acts, mode[1], mode[2])
        assert np.array_equal(bits(y), bits(ref)), mode
