"""GPU parity of route() on the device (softmax gating, top-k, norm_topk; es_hip_moe.hip) against the oracle's restatement:
selected experts equal and weights bit-identical, over the configs' router shapes, exact ties (equal logits, repeated values),
logits far enough apart to underflow expf, k from 1 to 64, with and without renormalisation."""
import numpy as np
import pytest

import es_hip_quant as E

pytestmark = pytest.mark.gpu


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def device_route(hip, logits, k, norm, kmax=None):
    ntok, ne = logits.shape
    kmax = kmax or k
    dl = hip.upload(np.ascontiguousarray(logits, np.float32))
    ds, dw = hip.alloc(ntok * kmax * 4), hip.alloc(ntok * kmax * 4)
    hip.route_softmax_dev(dl, 0, ntok, ne, k, norm, ds, dw, kmax)
    sel = hip.download(ds, np.zeros((ntok, kmax), np.int32))
    w = hip.download(dw, np.zeros((ntok, kmax), np.float32))
    return sel[:, :k], w[:, :k]


@pytest.mark.parametrize("ntok,ne,k,norm", [(32, 128, 8, True), (128, 64, 8, False), (7, 1000, 16, True), (5, 64, 64, True),
                                            (9, 256, 1, False), (3, 60, 5, True)])
def test_route_matches_oracle(hip, orc, ntok, ne, k, norm):
    rng = np.random.default_rng(ntok * ne + k)
    lg = rng.standard_normal((ntok, ne)).astype(np.float32)
    lg[0] = 0.0                                            # all equal: ties everywhere
    if ntok > 1:
        lg[1] = np.round(lg[1] * 2) / 2                    # repeated values
    if ntok > 2:
        lg[2] = (rng.standard_normal(ne) * 60).astype(np.float32)   # expf underflows for most experts
    sel, w = device_route(hip, lg, k, norm)
    osel, ow, _ = orc.route_softmax(lg, k, norm)
    assert np.array_equal(sel, osel)
    assert np.array_equal(bits(w), bits(ow))


def test_route_rows_of_kmax(hip, orc):
    lg = np.random.default_rng(4).standard_normal((6, 128)).astype(np.float32)
    sel, w = device_route(hip, lg, 8, True, kmax=10)
    osel, ow, _ = orc.route_softmax(lg, 8, True)
    assert np.array_equal(sel, osel) and np.array_equal(bits(w), bits(ow))


def test_route_rejects_bad_shapes(hip):
    d = hip.alloc(1 << 16)
    with pytest.raises(E.EsHipError):
        hip.route_softmax_dev(d, 0, 2, 2048, 8, True, d, d, 8)   # more experts than the kernel stages
    with pytest.raises(E.EsHipError):
        hip.route_softmax_dev(d, 0, 2, 64, 8, True, d, d, 4)     # kmax < k


def test_route_matches_reference_engine_goldens(hip, engine_golden):
    """device route() on the logits the reference engine's own route() was run on (tests/golden/engine_vectors.npz):
    the same experts and bit-identical weights, without the oracle in between"""
    from conftest import golden_cases
    for c in golden_cases(engine_golden, "route"):
        g = lambda n: engine_golden[f"route/{c}/{n}"]
        k, norm = (int(v) for v in g("params"))
        sel, w = device_route(hip, g("logits"), k, bool(norm))
        assert np.array_equal(sel, g("sel")), c
        assert np.array_equal(bits(w), bits(g("w"))), c
