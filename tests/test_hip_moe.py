"""GPU parity of the MoE expert FFN (es_hip_moe_ffn, the expert part of moe_n, src/es_engine.c:848-942) against the oracle's
restatement: routing from seeded logits (route(), :744-835), grouping, grouped gate/up products, SwiGLU with glibc's expf,
requantization, grouped down products and the weighted combine. Outputs must be bit-identical."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

MODES = [(E.ORDER_X86_CONTRACT, O.CONTRACT, O.PATH_X86), (E.ORDER_X86_STRICT, O.STRICT, O.PATH_X86),
         (E.ORDER_SCALAR, O.STRICT, O.PATH_SCALAR)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


class Experts:
    """n_exp experts of (gate, up, down) random blocks (the es_mtest recipe), on the host and on the device"""

    def __init__(self, hip, orc, types, n_exp, n, ff, seed):
        st = np.array([seed], np.uint64)
        self.types, self.n, self.ff = types, n, ff
        gt, ut, dt = types
        self.host = [(orc.mtest_blocks(gt, st, ff, n), orc.mtest_blocks(ut, st, ff, n), orc.mtest_blocks(dt, st, n, ff))
                     for _ in range(n_exp)]
        self.dev = [dict(gate=hip.upload(g), up=hip.upload(u), down=hip.upload(d)) for (g, u, d) in self.host]

    def args(self, k, sel, w):
        return E.MoeArgs(*self.types, self.n, self.ff, self.dev, k, sel, w)


def routed(orc, n_tok, n_exp, kmax, norm_topk, seed):
    logits = orc.gauss(seed, 1.0, n_tok * n_exp).reshape(n_tok, n_exp)
    sel, w, _ = orc.route_softmax(logits, kmax, norm_topk)
    return sel, w


def run_gpu(hip, ex, x_acts, k, sel, w):
    N = x_acts.shape[0]
    dx = hip.upload(x_acts)
    dout = hip.upload(np.full((N, ex.n), -777.0, np.float32))
    hip.moe_ffn(ex.args(k, sel, w), dx, x_acts.strides[0], dout, ex.n)
    return hip.download(dout, np.zeros((N, ex.n), np.float32))


@pytest.fixture
def hipo(hip):
    yield hip
    hip.set_order(E.ORDER_X86_CONTRACT)


def test_swiglu_bit_exact(hip, orc):
    """h = g / (1 + expf(-g)) * u over a dense sweep of g (every regime of expf: overflow, underflow, subnormal results)"""
    rng = np.random.default_rng(3)
    g = np.concatenate([np.linspace(-120.0, 120.0, 1 << 20, dtype=np.float32),
                        rng.standard_normal(1 << 20).astype(np.float32) * 4,
                        np.array([0.0, -0.0, 88.72, -88.72, 103.9, -103.9, 1e-30, -1e-30, np.inf, -np.inf], np.float32)])
    u = rng.standard_normal(g.size).astype(np.float32)
    dg, du, dh = hip.upload(g), hip.upload(u), hip.alloc(g.nbytes)
    hip.swiglu_dev(dg, du, dh, g.size)
    h = hip.download(dh, np.zeros_like(g))
    ref = orc.swiglu(g, u)
    same = (bits(h) == bits(ref)) | (np.isnan(h) & np.isnan(ref))
    assert same.all(), np.flatnonzero(~same)[:10]


@pytest.mark.parametrize("gated", [1, 0], ids=["gated", "two-job"])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_moe_config4_olmoe_q2k(hipo, orc, mode, gated):
    """config 4: 64 experts of Q2_K (gate/up 1024x2048, down 2048x1024), 128 tokens, top-8 softmax, no renormalisation;
    gate and up in one workgroup writing SwiGLU's Q8_K blocks (gated), or as two jobs and a SwiGLU pass"""
    hipo.set_order(mode[0])
    prev = hipo.set_moe_gated(gated)
    try:
        n, ff, n_exp, kmax, N = 2048, 1024, 64, 8, 128
        types = (E.Q2_K, E.Q2_K, E.Q2_K)
        ex = Experts(hipo, orc, types, n_exp, n, ff, 46)
        sel, w = routed(orc, N, n_exp, kmax, False, 1238)
        x = orc.quantize_act(E.Q2_K, orc.gauss(11, 1.0, N * n).reshape(N, n))
        out = run_gpu(hipo, ex, x, np.full(N, kmax), sel, w)
        ref = orc.moe_ffn(types, ex.host, n, ff, x, sel, w, order=mode[1], path=mode[2])
        assert np.array_equal(bits(out), bits(ref))
    finally:
        hipo.set_moe_gated(prev)


def test_moe_config5_qwen3_mixed(hipo, orc):
    """config 5: 128 experts, gate/up Q4_K 768x2048, down Q6_K 2048x768, 32 tokens, top-8 with renormalisation"""
    n, ff, n_exp, kmax, N = 2048, 768, 128, 8, 32
    types = (E.Q4_K, E.Q4_K, E.Q6_K)
    ex = Experts(hipo, orc, types, n_exp, n, ff, 47)
    sel, w = routed(orc, N, n_exp, kmax, True, 1239)
    x = orc.quantize_act(E.Q4_K, orc.gauss(12, 1.0, N * n).reshape(N, n))
    out = run_gpu(hipo, ex, x, np.full(N, kmax), sel, w)
    ref = orc.moe_ffn(types, ex.host, n, ff, x, sel, w)
    assert np.array_equal(bits(out), bits(ref))


@pytest.mark.parametrize("types,gated", [((E.Q4_K, E.Q4_K, E.Q5_0), 1), ((E.Q5_0, E.Q5_0, E.Q4_0), 1),
                                         ((E.Q6_K, E.Q6_K, E.Q2_K), 1), ((E.Q2_K, E.Q2_K, E.Q2_K), 1),
                                         ((E.Q2_K, E.Q2_K, E.Q2_K), 0)],
                         ids=["q4k-q50", "q50-q40", "q6k-q2k", "q2k-gated", "q2k-two-job"])
def test_moe_variable_k_and_gathers(hipo, orc, types, gated):
    """tokens with 0..kmax experts, experts chosen by several tokens, one expert taking 40 tokens (the matrix-core path
    with its activation gather for Q4_K; for Q2_K two activation tiles of the expert-sized kernel, gated or not), a token
    stride with padding, Q8_0 requantization for a 32-wide down type"""
    prev = hipo.set_moe_gated(gated)
    try:
        run_variable_k(hipo, orc, types)
    finally:
        hipo.set_moe_gated(prev)


def run_variable_k(hipo, orc, types):
    n, ff, n_exp, kmax, N = 512, 256, 6, 3, 45
    ex = Experts(hipo, orc, types, n_exp, n, ff, 48)
    rng = np.random.default_rng(4)
    k = rng.integers(0, kmax + 1, N).astype(np.int32)
    k[:40] = np.maximum(k[:40], 1)
    sel = np.zeros((N, kmax), np.int32)
    for t in range(N):
        sel[t] = rng.permutation(n_exp)[:kmax]
        if t < 40:
            sel[t, 0] = 2
    w = rng.random((N, kmax)).astype(np.float32)
    x = orc.quantize_act(types[0], orc.gauss(13, 1.0, N * n).reshape(N, n))
    xb = x.view(np.uint8).reshape(N, -1)
    pad = np.zeros((N, xb.shape[1] + 20), np.uint8)
    pad[:, :xb.shape[1]] = xb
    dx = hipo.upload(pad)
    dout = hipo.upload(np.full((N, n + 5), -777.0, np.float32))
    hipo.moe_ffn(ex.args(k, sel, w), dx, pad.strides[0], dout, n + 5)
    out = hipo.download(dout, np.zeros((N, n + 5), np.float32))
    ref = orc.moe_ffn(types, ex.host, n, ff, x, sel, w, k=k)
    assert np.array_equal(bits(out[:, :n]), bits(ref))
    assert np.all(out[:, n:] == -777.0)


def test_moe_plan_reruns_with_new_inputs(hipo, orc):
    """a plan captures the routing; the activations may change between runs"""
    n, ff, n_exp, kmax, N = 512, 256, 8, 2, 16
    types = (E.Q4_K, E.Q4_K, E.Q6_K)
    ex = Experts(hipo, orc, types, n_exp, n, ff, 49)
    sel, w = routed(orc, N, n_exp, kmax, True, 77)
    x1 = orc.quantize_act(E.Q4_K, orc.gauss(21, 1.0, N * n).reshape(N, n))
    x2 = orc.quantize_act(E.Q4_K, orc.gauss(22, 1.0, N * n).reshape(N, n))
    dx, dout = hipo.upload(x1), hipo.alloc(N * n * 4)
    plan = hipo.moe_plan(ex.args(np.full(N, kmax), sel, w), dx, x1.strides[0], dout, n)
    for x in (x1, x2, x1):
        hipo.copy_d2d(dx, hipo.upload(x), x.nbytes)
        plan.run()
        hipo.synchronize()
        out = hipo.download(dout, np.zeros((N, n), np.float32))
        assert np.array_equal(bits(out), bits(orc.moe_ffn(types, ex.host, n, ff, x, sel, w)))
    plan.close()


def test_moe_rejects_bad_routing(hip, orc):
    n, ff = 512, 256
    ex = Experts(hip, orc, (E.Q4_K, E.Q4_K, E.Q4_K), 2, n, ff, 50)
    x = orc.quantize_act(E.Q4_K, orc.gauss(1, 1.0, n).reshape(1, n))
    dx, dout = hip.upload(x), hip.alloc(n * 4)
    for k, sel in [([1], [[5]]), ([3], [[0, 1]]), ([-1], [[0, 1]])]:
        sel = np.array(sel, np.int32)
        with pytest.raises(E.EsHipError):
            hip.moe_ffn(ex.args(np.array(k), sel, np.ones(sel.shape, np.float32)), dx, 0, dout, n)


@pytest.mark.parametrize("types,n_exp,N,k,norm", [((E.Q2_K, E.Q2_K, E.Q2_K), 64, 40, 8, False),
                                                  ((E.Q4_K, E.Q4_K, E.Q6_K), 128, 32, 8, True)])
def test_moe_from_device_logits(hipo, orc, types, n_exp, N, k, norm):
    """es_hip_moe_ffn_logits: routing on the device from the router's logits, then the expert FFN; the routing equals the
    oracle's route() and the outputs its moe_n restatement, bit for bit"""
    n, ff = 2048, 768 if types[0] == E.Q4_K else 1024
    ex = Experts(hipo, orc, types, n_exp, n, ff, 60 + n_exp)
    logits = orc.gauss(1300 + N, 1.0, N * n_exp).reshape(N, n_exp)
    want_sel, want_w = routed(orc, N, n_exp, k, norm, 1300 + N)
    x = orc.quantize_act(types[0], orc.gauss(17, 1.0, N * n).reshape(N, n))
    dl, dx = hipo.upload(logits), hipo.upload(x)
    dout = hipo.upload(np.full((N, n), -777.0, np.float32))
    args = ex.args(np.zeros(1, np.int32), np.zeros((1, k), np.int32), np.zeros((1, k), np.float32))
    sel, w = hipo.moe_ffn_logits(args, N, dl, 0, k, norm, dx, x.strides[0], dout, n)
    assert np.array_equal(sel, want_sel) and np.array_equal(bits(w), bits(want_w))
    out = hipo.download(dout, np.zeros((N, n), np.float32))
    ref = orc.moe_ffn(types, ex.host, n, ff, x, want_sel, want_w)
    assert np.array_equal(bits(out), bits(ref))
