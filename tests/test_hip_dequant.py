"""GPU parity of es_hip_dequant_row_dev (es_dequant_row, src/es_quant.c:425-476, src/es_q2k.c:88-100): the reference's own
dequantized rows (golden vectors) and the oracle's dequantization of es_mtest's random blocks, bit for bit, in all eight
formats, from sources at any byte alignment."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

FMTS = ["Q4_0", "Q5_0", "Q8_0", "Q2_K", "Q3_K", "Q4_K", "Q5_K", "Q6_K"]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def dequant(hip, t, W, n, offset=0):
    raw = np.zeros(W.size + offset, np.uint8)
    raw[offset:] = W.view(np.uint8).reshape(-1)
    dsrc = hip.upload(raw)
    ddst = hip.alloc(4 * n)
    hip.dequant_row_dev(t, int(dsrc) + offset, ddst, n)
    return hip.download(ddst, np.zeros(n, np.float32))


@pytest.mark.parametrize("F", FMTS)
def test_dequant_matches_reference_rows(hip, golden, F):
    t = O.TYPES[F]
    cols = int(golden[f"{F}/gauss_shape"][0])
    W = golden[f"{F}/gauss_W"][: O.row_bytes(t, cols)]
    assert np.array_equal(bits(dequant(hip, t, W, cols)), bits(golden[f"{F}/dequant"]))


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("offset", [0, 1, 2, 3])
def test_dequant_random_blocks(hip, orc, F, offset):
    t = O.TYPES[F]
    rows, cols = 9, 1024
    W = orc.mtest_blocks(t, np.array([77 + t], np.uint64), rows, cols)
    n = rows * cols
    assert np.array_equal(bits(dequant(hip, t, W, n, offset)), bits(orc.dequant(t, W, n)))


def test_dequant_rejects_bad_arguments(hip):
    d = hip.alloc(1 << 12)
    with pytest.raises(E.EsHipError):
        hip.dequant_row_dev(E.Q4_K, d, d, 100)          # not a whole superblock
    with pytest.raises(E.EsHipError):
        hip.dequant_row_dev(7, d, d, 256)               # Q5_1 is not computed here
    with pytest.raises(E.EsHipError):
        hip.dequant_row_dev(E.Q4_0, d, int(d) + 2, 32)  # misaligned output
