"""GPU parity of the device-routed MoE layer (es_hip_moe_ctx_*): moe_n's grouping (src/es_engine.c:871-888) and the job
tables built on the device from a routing in device memory, then the expert FFN, with no allocation and no host round
trip per call. Outputs must equal the oracle's moe_n restatement bit for bit: configs 4 and 5 from device logits (the
routing equal to the oracle's route()), every reference order, every kernel family (decode kernel, pre-pass +
matrix-core kernel, expert-sized Q2_K kernel), skewed routings where one expert takes every token, fresh routings and token counts call after call
on one context without a wait between them, routing shapes up to 300 experts and k = 16, NaN logits, and the rejected
shapes."""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O
from test_hip_moe import MODES, Experts, bits, routed

pytestmark = pytest.mark.gpu


@pytest.fixture
def hipo(hip):
    yield hip
    hip.set_order(E.ORDER_X86_CONTRACT)


def run_logits(hip, ctx, orc, ex, N, n_exp, k, norm, seed, xseed):
    n = ex.n
    logits = orc.gauss(seed, 1.0, N * n_exp).reshape(N, n_exp)
    x = orc.quantize_act(ex.types[0], orc.gauss(xseed, 1.0, N * n).reshape(N, n))
    dl, dx = hip.upload(logits), hip.upload(x)
    dout = hip.upload(np.full((N, n), -777.0, np.float32))
    dsel, dw = hip.alloc(N * k * 4), hip.alloc(N * k * 4)
    ctx.run_logits(N, dl, 0, norm, dx, x.strides[0], dout, n, dsel, dw)
    hip.synchronize()
    out = hip.download(dout, np.zeros((N, n), np.float32))
    sel = hip.download(dsel, np.zeros((N, k), np.int32))
    w = hip.download(dw, np.zeros((N, k), np.float32))
    return x, out, sel, w


@pytest.mark.parametrize("family", ["expert", "expert-two-job", "prepass"])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_ctx_config4_olmoe_q2k_from_logits(hipo, orc, mode, family):
    """config 4: 64 Q2_K experts (gate/up 1024x2048, down 2048x1024), 128 tokens top-8: the expert-sized kernel family
    (default) with gate and up in one workgroup writing SwiGLU's Q8_K blocks, the same family with gate and up as two jobs
    and a SwiGLU pass, and the pre-pass + matrix-core family (the expert kernel switched off)"""
    hipo.set_order(mode[0])
    prev = hipo.set_q2k_expert_max_batch(1 if family == "prepass" else 64)
    prev_g = hipo.set_moe_gated(0 if family == "expert-two-job" else 1)
    try:
        n, ff, n_exp, k, N = 2048, 1024, 64, 8, 128
        types = (E.Q2_K, E.Q2_K, E.Q2_K)
        ex = Experts(hipo, orc, types, n_exp, n, ff, 46)
        ctx = hipo.moe_ctx(ex.args(np.zeros(1, np.int32), np.zeros((1, k), np.int32), np.zeros((1, k), np.float32)), N, k)
        x, out, sel, w = run_logits(hipo, ctx, orc, ex, N, n_exp, k, False, 1238, 11)
        want_sel, want_w = routed(orc, N, n_exp, k, False, 1238)
        assert np.array_equal(sel, want_sel) and np.array_equal(bits(w), bits(want_w))
        ref = orc.moe_ffn(types, ex.host, n, ff, x, want_sel, want_w, order=mode[1], path=mode[2])
        assert np.array_equal(bits(out), bits(ref))
        ctx.close()
    finally:
        hipo.set_q2k_expert_max_batch(prev)
        hipo.set_moe_gated(prev_g)


def test_ctx_config5_qwen3_mixed_from_logits(hipo, orc):
    """config 5: 128 experts, gate/up Q4_K 768x2048, down Q6_K 2048x768, 32 tokens top-8 renormalised: the decode family"""
    n, ff, n_exp, k, N = 2048, 768, 128, 8, 32
    types = (E.Q4_K, E.Q4_K, E.Q6_K)
    ex = Experts(hipo, orc, types, n_exp, n, ff, 47)
    ctx = hipo.moe_ctx(ex.args(np.zeros(1, np.int32), np.zeros((1, k), np.int32), np.zeros((1, k), np.float32)), N, k)
    x, out, sel, w = run_logits(hipo, ctx, orc, ex, N, n_exp, k, True, 1239, 12)
    want_sel, want_w = routed(orc, N, n_exp, k, True, 1239)
    assert np.array_equal(sel, want_sel) and np.array_equal(bits(w), bits(want_w))
    assert np.array_equal(bits(out), bits(orc.moe_ffn(types, ex.host, n, ff, x, want_sel, want_w)))
    ctx.close()


def run_logits_given(hip, ctx, ex, logits, k, norm, x):
    N, n = logits.shape[0], ex.n
    dl, dx = hip.upload(np.ascontiguousarray(logits, np.float32)), hip.upload(x)
    dout = hip.upload(np.full((N, n), -777.0, np.float32))
    dsel, dw = hip.alloc(N * k * 4), hip.alloc(N * k * 4)
    ctx.run_logits(N, dl, 0, norm, dx, x.strides[0], dout, n, dsel, dw)
    hip.synchronize()
    return (hip.download(dout, np.zeros((N, n), np.float32)), hip.download(dsel, np.zeros((N, k), np.int32)),
            hip.download(dw, np.zeros((N, k), np.float32)))


@pytest.mark.parametrize("n_exp,k,N,norm", [(256, 16, 70, True), (256, 1, 65, False), (300, 8, 20, True), (40, 12, 129, False)],
                         ids=["e256-k16", "e256-k1", "e300-k8", "e40-k12-n129"])
def test_ctx_routing_shapes(hipo, orc, n_exp, k, N, norm):
    """device routing of layers with many experts, k from 1 to 16 and token counts that are not multiples of anything:
    sel and w equal the oracle's route() (ties, underflowing experts), and the layer's outputs equal the oracle's moe_n"""
    n, ff = 256, 256
    types = (E.Q4_K, E.Q4_K, E.Q6_K)
    ex = Experts(hipo, orc, types, n_exp, n, ff, 300 + n_exp)
    rng = np.random.default_rng(n_exp * N + k)
    lg = rng.standard_normal((N, n_exp)).astype(np.float32)
    lg[0] = 0.0                                                  # all equal: ties everywhere
    lg[1] = np.round(lg[1] * 2) / 2                              # repeated values
    lg[2] = (rng.standard_normal(n_exp) * 60).astype(np.float32)  # expf underflows for most experts
    x = orc.quantize_act(types[0], orc.gauss(17 + N, 1.0, N * n).reshape(N, n))
    ctx = hipo.moe_ctx(ex.args(np.zeros(1, np.int32), np.zeros((1, k), np.int32), np.zeros((1, k), np.float32)), N, k)
    out, sel, w = run_logits_given(hipo, ctx, ex, lg, k, norm, x)
    osel, ow, _ = orc.route_softmax(lg, k, norm)
    assert np.array_equal(sel, osel) and np.array_equal(bits(w), bits(ow))
    assert np.array_equal(bits(out), bits(orc.moe_ffn(types, ex.host, n, ff, x, osel, ow)))
    ctx.close()


def test_ctx_routing_nan_logits(hipo, orc):
    """a token whose logits hold a NaN takes route()'s plain scan (every probability NaN: experts 0, 1, 2, ... in order);
    the other tokens of the same call route normally"""
    n, ff, n_exp, k, N = 256, 256, 64, 4, 9
    types = (E.Q4_K, E.Q4_K, E.Q4_K)
    ex = Experts(hipo, orc, types, n_exp, n, ff, 333)
    lg = np.random.default_rng(3).standard_normal((N, n_exp)).astype(np.float32)
    lg[4, 10] = np.nan
    x = orc.quantize_act(types[0], orc.gauss(19, 1.0, N * n).reshape(N, n))
    ctx = hipo.moe_ctx(ex.args(np.zeros(1, np.int32), np.zeros((1, k), np.int32), np.zeros((1, k), np.float32)), N, k)
    _, sel, w = run_logits_given(hipo, ctx, ex, lg, k, True, x)
    osel, ow, _ = orc.route_softmax(lg, k, True)
    assert np.array_equal(sel, osel)
    assert np.array_equal(sel[4], np.arange(k)) and np.all(np.isnan(w[4]))
    ok = np.arange(N) != 4
    assert np.array_equal(bits(w[ok]), bits(ow[ok]))
    ctx.close()


def skewed(N, n_exp, k, rng, hot=2):
    """every token's first choice is expert `hot`, the others distinct random experts"""
    sel = np.zeros((N, k), np.int32)
    for t in range(N):
        rest = [e for e in rng.permutation(n_exp) if e != hot][:k - 1]
        sel[t] = [hot] + rest
    return sel, rng.random((N, k)).astype(np.float32)


@pytest.mark.parametrize("types,n_exp,N,k", [((E.Q4_K, E.Q4_K, E.Q6_K), 16, 48, 4), ((E.Q2_K, E.Q2_K, E.Q2_K), 8, 70, 3),
                                             ((E.Q5_0, E.Q5_0, E.Q4_0), 12, 40, 2), ((E.Q6_K, E.Q6_K, E.Q4_K), 6, 33, 2)],
                         ids=["q4k-q6k", "q2k", "q50-q40", "q6k-q4k"])
def test_ctx_skewed_device_routing(hipo, orc, types, n_exp, N, k):
    """one expert chosen by every token (counts far from the mean), routing given in device memory"""
    n, ff = 512, 512
    ex = Experts(hipo, orc, types, n_exp, n, ff, 70 + n_exp)
    sel, w = skewed(N, n_exp, k, np.random.default_rng(N))
    x = orc.quantize_act(types[0], orc.gauss(5 + N, 1.0, N * n).reshape(N, n))
    ctx = hipo.moe_ctx(ex.args(np.zeros(1, np.int32), np.zeros((1, k), np.int32), np.zeros((1, k), np.float32)), N, k)
    dsel, dw, dx = hipo.upload(sel), hipo.upload(w), hipo.upload(x)
    dout = hipo.upload(np.full((N, n), -777.0, np.float32))
    ctx.run(N, dsel, dw, dx, x.strides[0], dout, n)
    hipo.synchronize()
    out = hipo.download(dout, np.zeros((N, n), np.float32))
    assert np.array_equal(bits(out), bits(orc.moe_ffn(types, ex.host, n, ff, x, sel, w)))
    ctx.close()


def test_ctx_fresh_routing_every_call(hipo, orc):
    """one context, five layers queued back to back on one stream with different routings and token counts (the largest
    first, then smaller, then the maximum again), no wait between them: each equals its own oracle result"""
    n, ff, n_exp, k, Nmax = 512, 256, 32, 4, 64
    types = (E.Q4_K, E.Q4_K, E.Q6_K)
    ex = Experts(hipo, orc, types, n_exp, n, ff, 91)
    ctx = hipo.moe_ctx(ex.args(np.zeros(1, np.int32), np.zeros((1, k), np.int32), np.zeros((1, k), np.float32)), Nmax, k)
    calls = []
    for i, N in enumerate((64, 17, 1, 40, 64)):
        logits = orc.gauss(400 + i, 1.0, N * n_exp).reshape(N, n_exp)
        x = orc.quantize_act(E.Q4_K, orc.gauss(500 + i, 1.0, N * n).reshape(N, n))
        dl, dx, dout = hipo.upload(logits), hipo.upload(x), hipo.alloc(N * n * 4)
        ctx.run_logits(N, dl, 0, True, dx, x.strides[0], dout, n)
        calls.append((N, x, dl, dx, dout, 400 + i))
    hipo.synchronize()
    for N, x, dl, dx, dout, seed in calls:
        sel, w = routed(orc, N, n_exp, k, True, seed)
        out = hipo.download(dout, np.zeros((N, n), np.float32))
        assert np.array_equal(bits(out), bits(orc.moe_ffn(types, ex.host, n, ff, x, sel, w))), N
    ctx.close()


def test_ctx_rejects_bad_shapes(hip, orc):
    n, ff, k = 512, 256, 2
    ex = Experts(hip, orc, (E.Q4_K, E.Q4_K, E.Q4_K), 4, n, ff, 95)
    args = ex.args(np.zeros(1, np.int32), np.zeros((1, k), np.int32), np.zeros((1, k), np.float32))
    with pytest.raises(E.EsHipError):
        hip.moe_ctx(args, 20000, 1)          # more choices than one grouping workgroup takes
    with pytest.raises(E.EsHipError):
        hip.moe_ctx(args, 8, 5)              # k above the expert count
    ctx = hip.moe_ctx(args, 8, k)
    d = hip.alloc(1 << 16)
    with pytest.raises(E.EsHipError):
        ctx.run(9, d, d, d, 0, d, n)         # more tokens than the context holds
    with pytest.raises(E.EsHipError):
        ctx.run(2, d, d, d.offset(2), 0, d, n)   # token rows not 4-byte aligned
    with pytest.raises(E.EsHipError):
        ctx.run(2, d, d, d, 580, d, n)       # token stride below one token's Q8_K blocks (2 x 292 bytes)
    with pytest.raises(E.EsHipError):
        ctx.run(2, d, d, d, 586, d, n)       # token stride not a multiple of 4
    ctx.run(0, d, d, d, 0, d, n)             # nothing to do
    ctx.close()
    bad = E.MoeArgs(E.Q4_K, E.Q4_0, E.Q4_K, n, ff, ex.dev, np.zeros(1, np.int32), np.zeros((1, k), np.int32),
                    np.zeros((1, k), np.float32))
    with pytest.raises(E.EsHipError):
        hip.moe_ctx(bad, 8, k)               # gate and up of different types
