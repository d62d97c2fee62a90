"""CPU tests: pin the oracle to the reference's own outputs (golden vectors, and the live reference build where present),
and to brute force / closed forms where no reference output exists."""
import numpy as np
import pytest

import oracle as O
import _layouts as L

FMTS = ["Q5_0", "Q4_0", "Q4_K", "Q6_K", "Q2_K", "Q8_0", "Q5_K", "Q3_K"]
CASES = ["mtest", "gauss"]


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _acts(golden, F, case):
    t = O.TYPES[F]
    raw = golden[f"{F}/{case}_q8"]
    return np.ascontiguousarray(raw).view(O.act_dtype(t)).reshape(raw.shape[0], -1)


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", CASES)
def test_activation_quantizer_matches_reference(orc, golden, F, case):
    t = O.TYPES[F]
    x = golden[f"{F}/{case}_x"]
    mine = orc.quantize_act(t, x)
    assert mine.tobytes() == _acts(golden, F, case).tobytes()


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", CASES)
@pytest.mark.parametrize("build,order,path", [("gcc", O.STRICT, O.PATH_X86), ("clang", O.CONTRACT, O.PATH_X86),
                                              ("scalar", O.STRICT, O.PATH_SCALAR)])
def test_matvec_bit_exact_vs_reference(orc, golden, F, case, build, order, path):
    t = O.TYPES[F]
    cols, rows = golden[f"{F}/{case}_shape"]
    W = golden[f"{F}/{case}_W"]
    acts = _acts(golden, F, case)
    y = orc.matvec_multi(t, W, int(cols), int(rows), acts, order, path)
    y[:, :3] = 0   # the reference call covered rows [3, rows) (tools/es_mtest.c:40)
    ref = golden[f"{F}/{case}_y_{build}"]
    assert np.array_equal(_bits(y), _bits(ref))


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", CASES)
def test_reference_multi_equals_single(golden, F, case):
    # es_mtest's invariant, as the reference's own build satisfies it
    assert np.array_equal(_bits(golden[f"{F}/{case}_ymulti_clang"]), _bits(golden[f"{F}/{case}_y_clang"]))


@pytest.mark.parametrize("F", FMTS)
def test_dequant_vs_reference(orc, golden, F):
    t = O.TYPES[F]
    cols = int(golden[f"{F}/gauss_shape"][0])
    W = golden[f"{F}/gauss_W"][: O.row_bytes(t, cols)]
    assert np.array_equal(_bits(orc.dequant(t, W, cols)), _bits(golden[f"{F}/dequant"]))


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", CASES)
def test_layout_decoder_pinned_by_reference_dequant(orc, golden, F, case):
    """the independent numpy decoder rebuilds the reference's dequantized floats exactly (gauss: golden row;
    mtest: every row, against the oracle's dequant, itself pinned by the golden row above)"""
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/{case}_shape"])
    W = golden[f"{F}/{case}_W"]
    dec = L.decode(t, W, cols)
    w = L.dequant_like_reference(t, dec)
    if case == "gauss":
        assert np.array_equal(_bits(w[0]), _bits(golden[f"{F}/dequant"]))
    ref = np.stack([orc.dequant(t, W[r * O.row_bytes(t, cols):(r + 1) * O.row_bytes(t, cols)], cols) for r in range(rows)])
    assert np.array_equal(_bits(w), _bits(ref))


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", CASES)
def test_block_integer_dots_brute_force(orc, golden, F, case):
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/{case}_shape"])
    W = golden[f"{F}/{case}_W"]
    acts = _acts(golden, F, case)
    dec = L.decode(t, W, cols)
    for q in range(acts.shape[0]):
        dots, aux = orc.block_ints(t, W, cols, rows, acts[q])
        bd, bm = L.int_dots(dec, acts[q]["qs"].reshape(-1))
        assert np.array_equal(dots.astype(np.int64), bd)
        if t in (O.Q4_K, O.Q2_K):
            assert np.array_equal(aux.astype(np.int64), bm)


@pytest.mark.parametrize("F", FMTS)
def test_integer_path_close_to_float_dot(orc, golden, F):
    """es_qtest --mv's bound: integer kernel vs float dequant dot, relative error < 0.03 (scripts/test_quants.py:65-71)"""
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/gauss_shape"])
    W = golden[f"{F}/gauss_W"]
    x = golden[f"{F}/gauss_x"]
    acts = _acts(golden, F, "gauss")
    y = orc.matvec_multi(t, W, cols, rows, acts)
    w = L.dequant_like_reference(t, L.decode(t, W, cols)).astype(np.float64)
    exact = x.astype(np.float64) @ w.T
    assert np.max(np.abs(y - exact)) / np.max(np.abs(exact)) < 0.03


def test_planted_mistake_is_caught(orc, golden):
    """flip one weight nibble in the oracle's input: the bit-exact comparison must fail"""
    F = "Q4_K"
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/mtest_shape"])
    W = golden[f"{F}/mtest_W"].copy()
    W[5 * O.row_bytes(t, cols) + 40] ^= 0x01
    y = orc.matvec_multi(t, W, cols, rows, _acts(golden, F, "mtest"), O.CONTRACT, O.PATH_X86)
    y[:, :3] = 0
    assert not np.array_equal(_bits(y), _bits(golden[f"{F}/mtest_y_clang"]))


def test_q2k_quantizer_and_reference_dot(orc, golden):
    w = golden["q2k/w"]
    W = np.concatenate([orc.quantize_q2_K_ref(w[r]) for r in range(w.shape[0])])
    assert W.tobytes() == golden["q2k/W"].tobytes()
    xq = orc.quantize_q8_K(golden["q2k/x"])
    assert xq.view(np.uint8).tobytes() == golden["q2k/xq"].tobytes()
    Wb = W.reshape(w.shape[0], -1)
    y = orc.matvec(O.Q2_K, Wb, 4096, 0, w.shape[0], xq, O.STRICT, O.PATH_SCALAR)
    # es_dot_q2_K_q8_K_ref: same integers, float epilogue sumf += dall*isum - dmin*summs
    assert np.array_equal(_bits(y), _bits(golden["q2k/dot_ref"]))
    # es_kbench's quantizer check: 2-bit weight relative error < 0.6 (tools/es_kbench.c:184)
    wd = np.concatenate([orc.dequant(O.Q2_K, Wb[r], 4096) for r in range(w.shape[0])]).reshape(w.shape)
    assert np.sqrt(np.sum((w - wd) ** 2) / np.sum(w ** 2)) < 0.6


def test_q8_quantizer_edge_cases(orc, golden):
    x = golden["q8k_edge/x"]
    assert orc.quantize_q8_K(x).view(np.uint8).tobytes() == golden["q8k_edge/q"].tobytes()
    assert orc.quantize_q8_0(x).view(np.uint8).tobytes() == golden["q80_edge/q"].tobytes()
    q = orc.quantize_q8_K(x)
    assert q[0]["d"] == 0 and not q[0]["qs"].any() and not q[0]["bsums"].any()   # all-zero block
    assert np.all(np.abs(q["qs"].astype(int)) <= 127)
    assert np.array_equal(q["bsums"], q["qs"].reshape(-1, 16, 16).astype(np.int64).sum(axis=2))


def test_fp16_conversions(orc, golden):
    for f, h in zip(golden["fp16/f"], golden["fp16/h"]):
        assert orc.float_to_half(float(f)) == int(h)
    # half -> float is exact for every finite half (closed form: numpy's IEEE conversion)
    hs = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = hs.view(np.float16).astype(np.float32)
    fin = np.isfinite(ref)
    mine = np.array([orc.half_to_float(int(h)) for h in hs[fin][::7]], np.float32)
    assert np.array_equal(mine.view(np.uint32), ref[fin][::7].view(np.uint32))


def test_weight_quantizers_round_trip(orc):
    rows, cols = 8, 1024
    w = orc.gauss(5, 0.02, rows * cols).reshape(rows, cols)
    for F, bound in (("Q4_0", 0.2), ("Q5_0", 0.1), ("Q8_0", 0.01), ("Q4_K", 0.15), ("Q5_K", 0.08), ("Q6_K", 0.05),
                     ("Q3_K", 0.3), ("Q2_K", 0.6)):
        t = O.TYPES[F]
        W = orc.quantize_rows(t, w)
        rb = O.row_bytes(t, cols)
        wd = np.stack([orc.dequant(t, W[r * rb:(r + 1) * rb], cols) for r in range(rows)])
        assert np.sqrt(np.sum((w - wd) ** 2) / np.sum(w ** 2)) < bound, F


def test_route_softmax_properties(orc):
    # equal logits: ties go to the lowest index, weights equal
    sel, w, p = orc.route_softmax(np.zeros((1, 64), np.float32), 8, norm_topk=False)
    assert sel[0].tolist() == list(range(8))
    assert np.allclose(w, 1 / 64)
    rng = np.random.default_rng(3)
    lg = rng.standard_normal((32, 128)).astype(np.float32)
    sel, w, p = orc.route_softmax(lg, 8, norm_topk=True)
    for t in range(32):
        assert len(set(sel[t].tolist())) == 8
        order = np.argsort(-lg[t], kind="stable")[:8]   # softmax is monotone: top-8 probabilities = top-8 logits
        assert sel[t].tolist() == order.tolist()
        assert abs(float(w[t].sum()) - 1.0) < 1e-6
    ex = np.exp(lg.astype(np.float64) - lg.max(axis=1, keepdims=True))
    assert np.allclose(p, ex / ex.sum(axis=1, keepdims=True), rtol=1e-5, atol=1e-7)


def test_moe_grouping_is_stable_partition(orc):
    rng = np.random.default_rng(4)
    sel = np.stack([rng.choice(64, 8, replace=False) for _ in range(128)]).astype(np.int32)
    uex, cnt, start, rowof, tok_of = orc.moe_group(sel)
    first = []
    for e in sel.reshape(-1):
        if e not in first:
            first.append(int(e))
    assert uex.tolist() == first                                       # order of first use
    assert cnt.sum() == sel.size and np.all(start == np.concatenate([[0], np.cumsum(cnt)[:-1]]))
    assert sorted(rowof.reshape(-1).tolist()) == list(range(sel.size))  # a bijection onto rows
    for t in range(sel.shape[0]):
        for j in range(8):
            r = rowof[t, j]
            u = uex.tolist().index(int(sel[t, j]))
            assert start[u] <= r < start[u] + cnt[u] and tok_of[r] == t
    for u in range(len(uex)):   # inside an expert, rows follow token order
        toks = tok_of[start[u]:start[u] + cnt[u]]
        assert np.all(np.diff(toks) > 0)


def test_swiglu_and_combine(orc):
    g = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 2.5], np.float32)
    u = np.array([3.0, 2.0, 2.0, 1.0, 1.0, -1.0], np.float32)
    h = orc.swiglu(g, u)
    ref = g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u
    assert h[0] == 0.0 and np.allclose(h, ref, rtol=1e-6, atol=1e-12)
    rng = np.random.default_rng(5)
    ye = rng.standard_normal((12, 16)).astype(np.float32)
    rowof = np.arange(12, dtype=np.int32).reshape(3, 4)
    w = rng.random((3, 4)).astype(np.float32)
    out = orc.moe_combine(ye, rowof, w)
    for t in range(3):
        s = np.zeros(16, np.float32)
        for j in range(4):
            s = (s + np.float32(w[t, j]) * ye[rowof[t, j]]).astype(np.float32)
        assert np.array_equal(out[t].view(np.uint32), s.view(np.uint32))


def test_cpu_bench_harness_runs(orc):
    t = O.Q4_K
    rows, cols = 64, 512
    W = orc.quantize_rows(t, orc.gauss(1, 0.02, rows * cols).reshape(rows, cols))
    acts = orc.quantize_act(t, orc.gauss(2, 1.0, 3 * cols).reshape(3, cols))
    sec, passes, y = orc.cpu_bench(orc.multi_fn_ptr(), t, W, W.size, 1, rows, cols, acts, 2, 0.01)
    assert passes >= 1 and sec > 0
    assert np.array_equal(y, orc.matvec_multi(t, W, cols, rows, acts))


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", CASES)
def test_float_path_vs_reference(orc, golden, F, case):
    """activations prepared without blocks: es_dequant_row + dot_f32 per row, as the reference computed it (the fixture
    was checked equal across its gcc, clang and scalar builds and es_matvec_multi when it was written)"""
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/{case}_shape"])
    y = orc.matvec_float(t, golden[f"{F}/{case}_W"], cols, rows, golden[f"{F}/{case}_x"], r0=3)
    assert np.array_equal(_bits(y), _bits(golden[f"{F}/{case}_yfloat"]))


def _chain_variants(w, x):
    """dot products of rows w [rows, n] with x [n] summed three wrong ways: one running sum; four running sums added
    left to right; four running sums with each product fused into its sum (rounded once, through float64)"""
    one = np.zeros(w.shape[0], np.float32)
    four = np.zeros((4, w.shape[0]), np.float32)
    fused = np.zeros((4, w.shape[0]), np.float32)
    for i in range(w.shape[1]):
        p = w[:, i] * x[i]
        one = (one + p).astype(np.float32)
        four[i % 4] = (four[i % 4] + p).astype(np.float32)
        fused[i % 4] = (fused[i % 4].astype(np.float64) + w[:, i].astype(np.float64) * np.float64(x[i])).astype(np.float32)
    left = (((four[0] + four[1]) + four[2]) + four[3]).astype(np.float32)
    return one, left, ((fused[0] + fused[1]) + (fused[2] + fused[3])).astype(np.float32)


@pytest.mark.parametrize("F", ["Q4_K", "Q8_0", "Q6_K"])
def test_float_path_fixture_pins_the_summation_order(orc, golden, F):
    """the fixture rejects the plausible mistakes in dot_f32's order: each wrong summation differs from it somewhere"""
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/gauss_shape"])
    W, x = golden[f"{F}/gauss_W"], golden[f"{F}/gauss_x"]
    w = np.stack([orc.dequant(t, W[r * O.row_bytes(t, cols):(r + 1) * O.row_bytes(t, cols)], cols) for r in range(rows)])
    ref = golden[f"{F}/gauss_yfloat"]
    for q in range(x.shape[0]):
        for wrong in _chain_variants(w, x[q]):
            assert not np.array_equal(_bits(wrong[3:]), _bits(ref[q, 3:]))


@pytest.mark.parametrize("F", ["Q8_0", "Q4_0", "Q4_K"])
def test_float_path_exact_integers(orc, F):
    """weights and activations that are small integers (block scales 1.0, integer mins) make every product and partial sum
    exact, so the float path must equal the int64 dot of the dequantized integers"""
    t = O.TYPES[F]
    rows, cols = 9, 1024
    rng = np.random.default_rng(5)
    bb, be = O.BLOCK_BYTES[t], O.BLOCK_ELEMS[t]
    W = rng.integers(0, 256, rows * cols // be * bb, dtype=np.uint8).reshape(rows, cols // be, bb)
    if F in ("Q8_0", "Q4_0"):
        W[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)   # d = 1.0
    else:   # Q4_K: d = 1.0, dmin = 1.0; 6-bit scales and mins are small integers already
        W[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
        W[:, :, 2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    W = W.reshape(-1)
    x = rng.integers(-6, 7, (2, cols)).astype(np.float32)
    rb = O.row_bytes(t, cols)
    wi = np.stack([orc.dequant(t, W[r * rb:(r + 1) * rb], cols) for r in range(rows)]).astype(np.int64)
    assert np.array_equal(wi.astype(np.float32), np.stack([orc.dequant(t, W[r * rb:(r + 1) * rb], cols) for r in range(rows)]))
    exact = x.astype(np.int64) @ wi.T
    assert np.abs(exact).max() < 1 << 24
    assert np.array_equal(orc.matvec_float(t, W, cols, rows, x), exact.astype(np.float32))


@pytest.mark.skipif(not O.ref_available("clang"), reason="reference not built here (no /root/reference)")
def test_live_reference_wide_shapes(orc):
    """the live reference build on the benchmark configurations' column counts, many rows, contract and strict orders"""
    for F, cols in (("Q4_0", 896), ("Q5_0", 2048), ("Q4_K", 2048), ("Q4_K", 8192), ("Q6_K", 1024), ("Q2_K", 2048),
                    ("Q6_K", 768)):
        t = O.TYPES[F]
        rows = 64
        W = orc.quantize_rows(t, orc.gauss(11, 0.02, rows * cols).reshape(rows, cols))
        x = orc.gauss(12, 1.0, 3 * cols).reshape(3, cols)
        acts = orc.quantize_act(t, x)
        for cc, order in (("clang", O.CONTRACT), ("gcc", O.STRICT)):
            R = O.RefLib(cc)
            ref = R.matvec_f32(t, W, cols, rows, x, multi=True)
            assert np.array_equal(_bits(orc.matvec_multi(t, W, cols, rows, acts, order)), _bits(ref)), (F, cols, cc)
            # the float path (activations prepared without blocks)
            assert np.array_equal(_bits(orc.matvec_float(t, W, cols, rows, x)),
                                  _bits(R.matvec_float(t, W, cols, rows, x, multi=True))), (F, cols, cc)


@pytest.mark.skipif(not O.ref_available("clang"), reason="reference not built here (no /root/reference)")
def test_reference_adapter_for_cpu_baseline(orc):
    """the cpu_baseline leg times the reference's es_matvec_multi through esq_multi_reference: it must compute the same
    numbers as es_act_prepare + es_matvec_multi, and the threaded harness must not change them"""
    R = O.RefLib("clang")
    for F, cols in (("Q4_K", 2048), ("Q4_0", 896), ("Q6_K", 1024), ("Q2_K", 1024), ("Q5_0", 512)):
        t = O.TYPES[F]
        rows = 40
        W = orc.quantize_rows(t, orc.gauss(21, 0.02, rows * cols).reshape(rows, cols))
        x = orc.gauss(22, 1.0, 3 * cols).reshape(3, cols)
        acts = orc.quantize_act(t, x)
        ref = R.matvec_f32(t, W, cols, rows, x, multi=True)
        assert np.array_equal(_bits(orc.matvec_multi_reference(R, t, W, cols, rows, acts)), _bits(ref)), F
        sec, passes, y = orc.cpu_bench(orc.reference_fn_ptr(R), t, W, W.size, 1, rows, cols, acts, 3, 0.01)
        assert passes >= 1 and np.array_equal(_bits(y), _bits(ref)), F


def _rmsnorm_numpy(x, w, eps):
    """src/es_engine.c:189-194 restated with numpy: float64 running sum (cumsum adds in element order), double division,
    sqrt and reciprocal, float32 products"""
    x = np.asarray(x, np.float32)
    sq = x.astype(np.float64) * x.astype(np.float64)   # exact in double
    ss = np.cumsum(sq)[-1]
    s = np.float32(1.0 / np.sqrt(ss / np.float64(x.size) + np.float64(np.float32(eps))))
    o = x * s
    return o * (np.ones_like(x) if w is None else np.asarray(w, np.float32))


@pytest.mark.parametrize("n,eps,scale,weighted", [(2048, 1e-5, 1.0, True), (8192, 1e-6, 0.1, True), (896, 1e-5, 30.0, False),
                                                  (256, 1e-6, 1e-3, True), (33, 1e-5, 1.0, False)])
def test_rmsnorm_matches_numpy_restatement(orc, n, eps, scale, weighted):
    rng = np.random.default_rng(n)
    x = (rng.standard_normal((3, n)) * scale).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32) if weighted else None
    mine = orc.rmsnorm(x, w, eps)
    for r in range(3):
        assert np.array_equal(_bits(mine[r]), _bits(_rmsnorm_numpy(x[r], w, eps)))


def test_rmsnorm_closed_forms(orc):
    n, eps = 512, np.float32(1e-5)
    zero = orc.rmsnorm(np.zeros((1, n), np.float32), None, eps)
    assert np.all(zero == 0.0)
    c = np.float32(0.75)
    const = orc.rmsnorm(np.full((1, n), c, np.float32), None, eps)
    s = np.float32(1.0 / np.sqrt(np.float64(c) * np.float64(c) + np.float64(eps)))   # mean of c^2 is c^2 exactly
    assert np.all(const == c * s)
    x = np.random.default_rng(3).standard_normal((2, n)).astype(np.float32)
    assert np.array_equal(_bits(orc.rmsnorm(x, None, eps)), _bits(orc.rmsnorm(x, np.ones(n, np.float32), eps)))


# ---- engine glue pinned to the reference engine's own route() / rmsnorm() (tests/golden/engine_vectors.npz) ----------
def test_route_matches_reference_engine_goldens(orc, engine_golden):
    from conftest import golden_cases
    cases = golden_cases(engine_golden, "route")
    assert {"olmoe", "qwen3", "ties", "ties_norm", "underflow", "underflow_norm", "k1", "k32", "wide"} <= set(cases)
    for c in cases:
        g = lambda n: engine_golden[f"route/{c}/{n}"]
        k, norm = (int(v) for v in g("params"))
        sel, w, _ = orc.route_softmax(g("logits"), k, bool(norm))
        assert np.array_equal(sel, g("sel")), c
        assert np.array_equal(_bits(w), _bits(g("w"))), c


def test_rmsnorm_matches_reference_engine_goldens(orc, engine_golden):
    from conftest import golden_cases
    cases = golden_cases(engine_golden, "rms")
    assert {"n896", "n896_w", "n2048", "n2048_w", "n8192", "n8192_w", "tiny", "huge", "zero"} <= set(cases)
    for c in cases:
        w = engine_golden.get(f"rms/{c}/w")
        o = orc.rmsnorm(engine_golden[f"rms/{c}/x"], w, float(engine_golden[f"rms/{c}/eps"][0]))
        assert np.array_equal(_bits(o), _bits(engine_golden[f"rms/{c}/o"])), c


def test_engine_goldens_catch_planted_mistakes(engine_golden):
    """the goldens tell apart the plausible slips of a restatement: a float (not double) sum of squares, a dropped eps,
    the weight applied before the scale, top-k by logits with ties to the highest index, renormalising without the clamp"""
    x = engine_golden["rms/n2048_w/x"][0]
    w = engine_golden["rms/n2048_w/w"]
    eps = float(engine_golden["rms/n2048_w/eps"][0])
    want = engine_golden["rms/n2048_w/o"][0]
    ssf = np.float32(0)
    for v in x:
        ssf = np.float32(ssf + v * v)
    s_f = np.float32(1.0 / np.sqrt(np.float64(ssf) / x.size + eps))
    ss = float(np.cumsum(x.astype(np.float64) ** 2)[-1])
    s = np.float32(1.0 / np.sqrt(ss / x.size + np.float64(np.float32(eps))))
    s_noeps = np.float32(1.0 / np.sqrt(ss / x.size))
    right = x * s * w
    assert np.array_equal(_bits(right), _bits(want))
    assert not np.array_equal(_bits(x * s_f * w), _bits(want))
    assert not np.array_equal(_bits(x * s_noeps * w), _bits(want))
    assert not np.array_equal(_bits(x * (s * w)), _bits(want))
    t = engine_golden["route/ties/logits"]
    sel = engine_golden["route/ties/sel"]
    last_max = np.stack([np.argsort(-row[::-1], kind="stable")[:8] for row in t])
    last_max = t.shape[1] - 1 - last_max
    assert not np.array_equal(last_max, sel)


@pytest.mark.skipif(not O.ref_engine_available("clang"), reason="reference engine not built here (no /root/reference)")
def test_route_and_rmsnorm_live_reference_engine(orc):
    """the live reference engine against the oracle on fresh inputs (shapes of configs 4 and 5, both compilers)"""
    rng = np.random.default_rng(77)
    for cc in ("clang", "gcc"):
        R = O.RefEngine(cc)
        for ntok, ne, k, norm in ((64, 64, 8, False), (16, 128, 8, True), (5, 300, 32, True), (8, 64, 1, True)):
            lg = rng.standard_normal((ntok, ne)).astype(np.float32)
            lg[0, ::5] = 2.0
            sel, w = R.route(lg, k, norm)
            osel, ow, _ = orc.route_softmax(lg, k, norm)
            assert np.array_equal(sel, osel) and np.array_equal(_bits(w), _bits(ow)), (cc, ntok, ne, k, norm)
        for n in (256, 1024, 4096):
            x = rng.standard_normal((2, n)).astype(np.float32) * 5
            wv = rng.random(n).astype(np.float32)
            for ww in (None, wv):
                assert np.array_equal(_bits(R.rmsnorm(x, ww, 1e-5)), _bits(orc.rmsnorm(x, ww, 1e-5))), (cc, n)
