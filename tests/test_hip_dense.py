"""GPU parity of dense_n on the device (es_hip_dense_ffn_dev; src/es_engine.c:957-972): gate and up into the engine's
[token][2 ff] rows, SwiGLU fused with the down type's activation preparation, down. Checked at config 2's full prefill shape
(Q4_K, n = 2048, ff = 8192, T = 512) against the oracle's composition (matvec, swiglu, quantize, matvec) for three tokens
bit for bit, and for every token against the same composition of the separately tested device pieces (run_jobs with
ystride 2 ff, es_hip_swiglu_prepare_dev, run_jobs); at config 1's Q4_0 shape (n = 896, ff = 4864: Q8_0 activations on both
sides) and in every reference order on a smaller Q4_K layer."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

MODES = [(E.ORDER_X86_CONTRACT, O.CONTRACT, O.PATH_X86), (E.ORDER_X86_STRICT, O.STRICT, O.PATH_X86),
         (E.ORDER_SCALAR, O.STRICT, O.PATH_SCALAR)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def layer(orc, t_gu, t_d, n, ff, N, seed):
    Wg = orc.quantize_rows(t_gu, orc.gauss(seed, 0.02, ff * n).reshape(ff, n))
    Wu = orc.quantize_rows(t_gu, orc.gauss(seed + 1, 0.02, ff * n).reshape(ff, n))
    Wd = orc.quantize_rows(t_d, orc.gauss(seed + 2, 0.02, n * ff).reshape(n, ff))
    x = orc.gauss(seed + 3, 1.0, N * n).reshape(N, n)
    return Wg, Wu, Wd, np.ascontiguousarray(orc.quantize_act(t_gu, x))


def device_dense(hip, t_gu, t_d, Wg, Wu, Wd, acts, n, ff):
    N = acts.shape[0]
    hs = (ff // E.BLOCK_ELEMS[t_d]) * E.ACT_BYTES[t_d]
    d = [hip.upload(a) for a in (Wg, Wu, Wd, acts)]
    gu, hq, out = hip.alloc(N * 2 * ff * 4), hip.alloc(N * hs), hip.alloc(N * n * 4)
    hip.dense_ffn_dev(t_gu, d[0], t_gu, d[1], t_d, d[2], n, ff, N, d[3], acts.strides[0], gu, hq, out, n)
    hip.synchronize()
    y = hip.download(out, np.zeros((N, n), np.float32))
    g = hip.download(gu, np.zeros((N, 2 * ff), np.float32))
    for b in d + [gu, hq, out]:
        b.close()
    return y, g


def device_pieces(hip, t_gu, t_d, Wg, Wu, Wd, acts, n, ff):
    """the same layer from the separately tested pieces"""
    N = acts.shape[0]
    hs = (ff // E.BLOCK_ELEMS[t_d]) * E.ACT_BYTES[t_d]
    d = [hip.upload(a) for a in (Wg, Wu, Wd, acts)]
    gu, hq, out = hip.alloc(N * 2 * ff * 4), hip.alloc(N * hs), hip.alloc(N * n * 4)
    a0 = acts.strides[0]
    hip.run_jobs([dict(type=t_gu, rows=ff, cols=n, W=d[0], act=d[3], astride=a0, nb=N, y=gu, ystride=2 * ff),
                  dict(type=t_gu, rows=ff, cols=n, W=d[1], act=d[3], astride=a0, nb=N, y=int(gu) + 4 * ff, ystride=2 * ff)])
    q8k = E.ACT_BYTES[t_d] == 292
    hip.swiglu_prepare_dev(gu, 2 * ff, N, ff, None, 0, None if q8k else hq, hs, hq if q8k else None, hs)
    hip.run_jobs([dict(type=t_d, rows=n, cols=ff, W=d[2], act=hq, astride=hs, nb=N, y=out, ystride=n)])
    hip.synchronize()
    y = hip.download(out, np.zeros((N, n), np.float32))
    for b in d + [gu, hq, out]:
        b.close()
    return y


def oracle_dense(orc, t_gu, t_d, Wg, Wu, Wd, act, n, ff, order=O.CONTRACT, path=O.PATH_X86):
    g = orc.matvec(t_gu, Wg, n, 0, ff, act, order, path)
    u = orc.matvec(t_gu, Wu, n, 0, ff, act, order, path)
    h = orc.swiglu(g, u)
    hq = orc.quantize_act(t_d, h[None, :])[0]
    return orc.matvec(t_d, Wd, ff, 0, n, hq, order, path), g, u


def test_dense_config2_prefill_t512(hip, orc):
    n, ff, N = 2048, 8192, 512
    Wg, Wu, Wd, acts = layer(orc, O.Q4_K, O.Q4_K, n, ff, N, 11)
    y, gu = device_dense(hip, O.Q4_K, O.Q4_K, Wg, Wu, Wd, acts, n, ff)
    assert np.isfinite(y).all() and np.abs(y).max() > 0
    for t in (0, 257, 511):
        ref, g, u = oracle_dense(orc, O.Q4_K, O.Q4_K, Wg, Wu, Wd, acts[t], n, ff)
        assert np.array_equal(bits(gu[t, :ff]), bits(g)) and np.array_equal(bits(gu[t, ff:]), bits(u)), t
        assert np.array_equal(bits(y[t]), bits(ref)), t
    assert np.array_equal(bits(y), bits(device_pieces(hip, O.Q4_K, O.Q4_K, Wg, Wu, Wd, acts, n, ff)))


def test_dense_config1_q4_0(hip, orc):
    n, ff, N = 896, 4864, 32
    Wg, Wu, Wd, acts = layer(orc, O.Q4_0, O.Q4_0, n, ff, N, 21)
    y, _ = device_dense(hip, O.Q4_0, O.Q4_0, Wg, Wu, Wd, acts, n, ff)
    for t in (0, 13, 31):
        ref, _, _ = oracle_dense(orc, O.Q4_0, O.Q4_0, Wg, Wu, Wd, acts[t], n, ff)
        assert np.array_equal(bits(y[t]), bits(ref)), t
    assert np.array_equal(bits(y), bits(device_pieces(hip, O.Q4_0, O.Q4_0, Wg, Wu, Wd, acts, n, ff)))


@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
@pytest.mark.parametrize("N", [1, 7, 64, 130])
def test_dense_orders_and_token_counts(hip, orc, mode, N):
    n, ff = 512, 1024
    Wg, Wu, Wd, acts = layer(orc, O.Q4_K, O.Q6_K, n, ff, N, 31 + N)
    prev = hip.set_order(mode[0])
    try:
        y, _ = device_dense(hip, O.Q4_K, O.Q6_K, Wg, Wu, Wd, acts, n, ff)
    finally:
        hip.set_order(prev)
    for t in sorted({0, N // 2, N - 1}):
        ref, _, _ = oracle_dense(orc, O.Q4_K, O.Q6_K, Wg, Wu, Wd, acts[t], n, ff, mode[1], mode[2])
        assert np.array_equal(bits(y[t]), bits(ref)), t


def test_dense_rejects_bad_shapes(hip):
    d = hip.alloc(1 << 16)
    with pytest.raises(E.EsHipError):   # ff not a whole number of Q8_K blocks for a K-quant down
        hip.dense_ffn_dev(O.Q4_K, d, O.Q4_K, d, O.Q4_K, d, 256, 288, 2, d, 0, d, d, d, 256)
    with pytest.raises(E.EsHipError):   # gate and up take different activation kinds
        hip.dense_ffn_dev(O.Q4_K, d, O.Q4_0, d, O.Q4_K, d, 256, 256, 2, d, 0, d, d, d, 256)
    with pytest.raises(E.EsHipError):   # ostride below n
        hip.dense_ffn_dev(O.Q4_K, d, O.Q4_K, d, O.Q4_K, d, 256, 256, 2, d, 0, d, d, d, 128)
