"""The product entry point that allocates nothing (es_hip_matvec_multi_dev_noalloc): its job tables and pre-pass workspace
live in the library's static device scratch. Its outputs must equal es_hip_matvec_multi_dev's bit for bit on every kernel
path that uses tables or a workspace (pre-pass matrix-core kernels for Q4_K, Q6_K, Q2_K, the direct-activation kernel, the
small-batch kernel, the batched Q4_0 kernel, decode), on two calls in a row through the shared scratch, the second with a
smaller input; a product whose tables and workspace exceed the scratch is refused and leaves the outputs untouched."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def make(orc, t, rows, cols, na, seed):
    st = np.array([seed], np.uint64)
    W = orc.mtest_blocks(t, st, rows, cols)
    x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, np.ascontiguousarray(orc.quantize_act(t, x))


def run(hip, fn, t, W, cols, rows, acts):
    na = acts.shape[0]
    dW, dA = hip.upload(W), hip.upload(acts)
    dY = hip.alloc(na * rows * 4)
    hip.memset(dY, 0, na * rows * 4)
    fn(t, dW, cols, 0, rows, dA, acts.strides[0] if na > 1 else 0, na, dY, rows)
    hip.synchronize()
    y = hip.download(dY, np.zeros((na, rows), np.float32))
    for b in (dW, dA, dY):
        b.close()
    return y


# (name, type, (rows, cols, na) of the first call, of the second, smaller one)
CASES = [
    ("q4k_prepass_mm", O.Q4_K, (2048, 8192, 96), (1024, 4096, 40)),
    ("q4k_direct", O.Q4_K, (8192, 2048, 64), (8192, 2048, 33)),
    ("q4k_small_batch", O.Q4_K, (2048, 2048, 16), (512, 1024, 9)),
    ("q6k_mm", O.Q6_K, (1024, 1024, 32), (512, 1024, 17)),
    ("q2k_mm", O.Q2_K, (512, 2048, 8), (256, 1024, 3)),
    ("q4_0_batched", O.Q4_0, (4864, 896, 32), (4864, 896, 5)),
    ("q4k_decode", O.Q4_K, (4096, 2048, 1), (100, 2048, 1)),
]


@pytest.mark.parametrize("name,t,big,small", CASES, ids=[c[0] for c in CASES])
def test_noalloc_equals_allocating_entry(hip, orc, name, t, big, small):
    outs = []
    for k, (rows, cols, na) in enumerate((big, small)):   # two calls in a row through the shared scratch
        W, acts = make(orc, t, rows, cols, na, 1000 * k + rows + na)
        y = run(hip, hip.matvec_multi_dev_noalloc, t, W, cols, rows, acts)
        ref = run(hip, hip.matvec_multi_dev, t, W, cols, rows, acts)
        assert np.array_equal(bits(y), bits(ref)), (name, k)
        assert np.isfinite(y).all() and np.any(y != 0), (name, k)
        outs.append(y)


def test_noalloc_back_to_back_on_one_stream(hip, orc):
    """two pre-pass products queued back to back without a sync between them: the second's tables and planes overwrite
    the first's in the scratch only after the first's kernels, in stream order"""
    (r1, c1, n1), (r2, c2, n2) = (2048, 8192, 96), (1024, 4096, 40)
    W1, A1 = make(orc, O.Q4_K, r1, c1, n1, 7)
    W2, A2 = make(orc, O.Q4_K, r2, c2, n2, 8)
    d = [hip.upload(a) for a in (W1, A1, W2, A2)]
    y1, y2 = hip.alloc(n1 * r1 * 4), hip.alloc(n2 * r2 * 4)
    hip.matvec_multi_dev_noalloc(O.Q4_K, d[0], c1, 0, r1, d[1], A1.strides[0], n1, y1, r1)
    hip.matvec_multi_dev_noalloc(O.Q4_K, d[2], c2, 0, r2, d[3], A2.strides[0], n2, y2, r2)
    hip.synchronize()
    got1 = hip.download(y1, np.zeros((n1, r1), np.float32))
    got2 = hip.download(y2, np.zeros((n2, r2), np.float32))
    for b in d + [y1, y2]:
        b.close()
    assert np.array_equal(bits(got1), bits(run(hip, hip.matvec_multi_dev, O.Q4_K, W1, c1, r1, A1)))
    assert np.array_equal(bits(got2), bits(run(hip, hip.matvec_multi_dev, O.Q4_K, W2, c2, r2, A2)))


def test_noalloc_refuses_more_than_the_scratch(hip):
    """Q6_K, 64 rows x 8192 columns against 8192 activations (the pre-pass matrix-core kernel): the pre-pass planes alone
    (8192 x 32 superblocks x ~292 bytes) exceed the scratch; the call fails with EINVAL before launching anything. (A Q4_K
    product of that shape runs on the direct kernel, whose tile tables fit.)"""
    rows, cols, na = 64, 8192, 8192
    nbk = cols // 256
    assert na * nbk * 292 > E.NOALLOC_SCRATCH_BYTES
    dW = hip.alloc(rows * nbk * 210)
    dA = hip.alloc(na * nbk * 292)
    hip.memset(dW, 0, rows * nbk * 210)
    hip.memset(dA, 0, na * nbk * 292)
    dY = hip.alloc(na * rows * 4)
    hip.memset(dY, 0x7f, na * rows * 4)
    with pytest.raises(E.EsHipError) as ei:
        hip.matvec_multi_dev_noalloc(O.Q6_K, dW, cols, 0, rows, dA, nbk * 292, na, dY, rows)
    assert "no-allocation scratch" in str(ei.value) or "no-allocation scratch" in hip.last_error()
    hip.synchronize()
    y = hip.download(dY, np.zeros(na * rows, np.uint32))
    assert (y == 0x7f7f7f7f).all()
    for b in (dW, dA, dY):
        b.close()


def test_noalloc_refuses_graph_capture(hip, orc):
    """on a stream under HIP graph capture the call is refused with EINVAL (its job tables are copied from host memory at
    the call, which a captured graph could not replay); the capture ends cleanly and the entry point works after it"""
    import ctypes as C
    import glob
    hiprt = C.CDLL(sorted(glob.glob("/opt/rocm/lib/libamdhip64.so*"))[0])
    rows, cols, na = 1024, 2048, 40
    W, acts = make(orc, O.Q4_K, rows, cols, na, 77)
    dW, dA, dY = hip.upload(W), hip.upload(acts), hip.alloc(na * rows * 4)
    s, g = C.c_void_p(), C.c_void_p()
    assert hiprt.hipStreamCreate(C.byref(s)) == 0
    assert hiprt.hipStreamBeginCapture(s, 2) == 0   # hipStreamCaptureModeRelaxed
    try:
        with pytest.raises(E.EsHipError):
            hip.matvec_multi_dev_noalloc(O.Q4_K, dW, cols, 0, rows, dA, acts.strides[0], na, dY, rows, stream=s.value)
    finally:
        rc = hiprt.hipStreamEndCapture(s, C.byref(g))
        if g.value:
            hiprt.hipGraphDestroy(g)
        hiprt.hipStreamDestroy(s)
    assert rc == 0
    assert "capturing stream" in hip.last_error()
    for b in (dW, dA, dY):
        b.close()
    y = run(hip, hip.matvec_multi_dev_noalloc, O.Q4_K, W, cols, rows, acts)
    assert np.array_equal(bits(y), bits(run(hip, hip.matvec_multi_dev, O.Q4_K, W, cols, rows, acts)))
