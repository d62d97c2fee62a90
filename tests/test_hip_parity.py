"""GPU parity: the HIP kernels against the reference's own outputs (golden vectors made from the reference built from its
sources) and against the oracle (the CPU restatement pinned to those vectors), bit for bit.

Every call goes through the C ABI of libes_hip_quant.so. Order modes map to the reference builds:
X86_CONTRACT = clang (the reference's default CC), X86_STRICT = gcc -std=c11, SCALAR = gcc with ES_NO_AVX2=1.
"""
import numpy as np
import pytest

import es_hip_quant as E
import oracle as O

pytestmark = pytest.mark.gpu

FMTS = ["Q5_0", "Q4_0", "Q4_K", "Q6_K", "Q2_K", "Q8_0", "Q5_K", "Q3_K"]
MODES = [(E.ORDER_X86_CONTRACT, "clang", O.CONTRACT, O.PATH_X86), (E.ORDER_X86_STRICT, "gcc", O.STRICT, O.PATH_X86),
         (E.ORDER_SCALAR, "scalar", O.STRICT, O.PATH_SCALAR)]


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def golden_acts(golden, F, case):
    t = O.TYPES[F]
    raw = golden[f"{F}/{case}_q8"]
    return np.ascontiguousarray(raw).view(O.act_dtype(t)).reshape(raw.shape[0], -1)


@pytest.fixture
def order(hip):
    """restore the default order after a test that changes it"""
    yield hip
    hip.set_order(E.ORDER_X86_CONTRACT)


def mismatch_report(y, ref):
    bad = np.argwhere(bits(y) != bits(ref))
    if not len(bad):
        return ""
    q, r = bad[0]
    return f"{len(bad)} of {y.size} differ; first at act {q} row {r}: {y[q, r]!r} vs {ref[q, r]!r}"


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", ["mtest", "gauss"])
@pytest.mark.parametrize("mode", MODES, ids=[m[1] for m in MODES])
def test_golden_vectors_bit_exact(order, golden, F, case, mode):
    """es_matvec over rows [3, rows) of the reference's own test shapes (tools/es_mtest.c:17, 40)"""
    hip = order
    hip.set_order(mode[0])
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/{case}_shape"])
    y = hip.matvec_multi(t, golden[f"{F}/{case}_W"], cols, rows, golden_acts(golden, F, case), r0=3)
    ref = golden[f"{F}/{case}_y_{mode[1]}"]
    assert np.array_equal(bits(y), bits(ref)), mismatch_report(y, ref)


@pytest.mark.parametrize("F", FMTS)
@pytest.mark.parametrize("case", ["mtest", "gauss"])
def test_block_integer_dots_exact(hip, orc, golden, F, case):
    t = O.TYPES[F]
    cols, rows = (int(v) for v in golden[f"{F}/{case}_shape"])
    W = golden[f"{F}/{case}_W"]
    acts = golden_acts(golden, F, case)
    dW = hip.upload(W)
    for q in range(acts.shape[0]):
        dA = hip.upload(acts[q])
        dots, aux = hip.block_ints_dev(t, dW, cols, rows, dA)
        rd, ra = orc.block_ints(t, W, cols, rows, acts[q])
        assert np.array_equal(dots, rd), (F, case, q)
        assert np.array_equal(aux, ra), (F, case, q)


def mtest_inputs(orc, t, rows, cols, na, seed):
    st = np.array([seed], np.uint64)
    W = orc.mtest_blocks(t, st, rows, cols)
    x = orc.mtest_acts(st, na * cols).reshape(na, cols)
    return W, orc.quantize_act(t, x)


# the benchmark configurations' shapes (rows x cols), at token counts the oracle finishes in seconds
SHAPES = [
    ("Q4_0", 4864, 896, 1),     # config 1
    ("Q4_K", 8192, 2048, 3),    # config 2 gate/up
    ("Q4_K", 2048, 8192, 2),    # config 2 down
    ("Q6_K", 151936, 1024, 1),  # config 3 head (K padded to 1024)
    ("Q2_K", 1024, 2048, 5),    # config 4 expert gate/up
    ("Q2_K", 2048, 1024, 4),    # config 4 expert down
    ("Q4_K", 768, 2048, 3),     # config 5 expert gate/up
    ("Q6_K", 2048, 768, 3),     # config 5 expert down
    ("Q5_0", 4096, 2048, 4),    # config 5 attention q
    ("Q5_0", 512, 2048, 5),     # config 5 attention k/v
    ("Q5_K", 2048, 768, 3),     # Q5_K / Q3_K tensors of the K-quant mixes, odd block count per row
    ("Q5_K", 1024, 4096, 2),
    ("Q3_K", 2048, 768, 3),
    ("Q3_K", 1024, 4096, 2),
]


@pytest.mark.parametrize("F,rows,cols,na", SHAPES, ids=[f"{s[0]}-{s[1]}x{s[2]}-n{s[3]}" for s in SHAPES])
@pytest.mark.parametrize("mode", MODES[:2], ids=["clang", "gcc"])
def test_baseline_shapes_vs_oracle(order, orc, F, rows, cols, na, mode):
    hip = order
    hip.set_order(mode[0])
    t = O.TYPES[F]
    W, acts = mtest_inputs(orc, t, rows, cols, na, 1000 + rows + cols)
    y = hip.matvec_multi(t, W, cols, rows, acts)
    ref = orc.matvec_multi(t, W, cols, rows, acts, mode[2], mode[3])
    assert np.array_equal(bits(y), bits(ref)), mismatch_report(y, ref)


@pytest.mark.parametrize("F,rows,cols", [("Q4_K", 512, 2048), ("Q6_K", 300, 1024), ("Q2_K", 256, 2048),
                                          ("Q4_0", 200, 896), ("Q5_0", 128, 2048), ("Q4_K", 64, 14336),
                                          ("Q8_0", 300, 2048), ("Q5_K", 300, 2048), ("Q3_K", 257, 768)])
def test_multi_equals_single(hip, orc, F, rows, cols):
    """es_mtest's invariant on the device: one launch over na activations == na single-activation launches"""
    t = O.TYPES[F]
    na = 11
    W, acts = mtest_inputs(orc, t, rows, cols, na, 7 + rows)
    ym = hip.matvec_multi(t, W, cols, rows, acts)
    for q in range(na):
        y1 = hip.matvec_multi(t, W, cols, rows, acts[q:q + 1])
        assert np.array_equal(bits(ym[q]), bits(y1[0])), (F, q)
    # and the oracle on a few of them
    ref = orc.matvec_multi(t, W, cols, rows, acts[:3])
    assert np.array_equal(bits(ym[:3]), bits(ref))


@pytest.mark.parametrize("F", FMTS)
def test_row_ranges_and_strides(hip, orc, F):
    """rows [r0, r1) only, absolute indices, padded activation and output strides; nothing else is written"""
    t = O.TYPES[F]
    cols = 512 if O.BLOCK_ELEMS[t] == 256 else 256
    rows, na, r0, r1 = 97, 3, 13, 90
    W, acts = mtest_inputs(orc, t, rows, cols, na, 31)
    ab = O.row_bytes(t, cols) // O.BLOCK_BYTES[t] * O.act_dtype(t).itemsize
    astride = ab + 40                      # padded activation records
    araw = np.zeros(na * astride, np.uint8)
    for q in range(na):
        araw[q * astride:q * astride + ab] = acts[q].view(np.uint8)
    ystride = rows + 29
    sentinel = np.float32(-12345.0)
    dW, dA = hip.upload(W), hip.upload(araw)
    dY = hip.upload(np.full(na * ystride, sentinel, np.float32))
    hip.matvec_multi_dev(t, dW, cols, r0, r1, dA, astride, na, dY, ystride)
    y = hip.download(dY, np.zeros((na, ystride), np.float32))
    ref = orc.matvec_multi(t, W, cols, rows, acts)
    assert np.array_equal(bits(y[:, r0:r1]), bits(ref[:, r0:r1]))
    assert np.all(y[:, :r0] == sentinel) and np.all(y[:, r1:] == sentinel)


@pytest.mark.parametrize("F", FMTS)
def test_edge_blocks(hip, orc, F):
    """all-0xff and all-zero weight bytes, zero activations (d = 0 blocks), subnormal fp16 scales, +-127 activations"""
    t = O.TYPES[F]
    be, bb = O.BLOCK_ELEMS[t], O.BLOCK_BYTES[t]
    cols = 4 * be
    rows = 6
    W = np.zeros((rows, cols // be, bb), np.uint8)
    W[0] = 0xFF
    W[2] = 0xFF
    rng = np.random.default_rng(9)
    W[3] = rng.integers(0, 256, W[3].shape, dtype=np.uint8)
    W[4] = rng.integers(0, 256, W[4].shape, dtype=np.uint8)
    dpos = {O.Q4_0: [0], O.Q5_0: [0], O.Q8_0: [0], O.Q4_K: [0, 2], O.Q6_K: [208], O.Q2_K: [80, 82],
            O.Q5_K: [0, 2], O.Q3_K: [108]}[t]
    for p in dpos:
        W[2, :, p:p + 2] = np.frombuffer(np.uint16(0x3C00).tobytes(), np.uint8)   # 1.0: extreme integers, sane scale
        W[3, :, p:p + 2] = np.frombuffer(np.uint16(0x0007).tobytes(), np.uint8)   # subnormal half
        W[4, :, p:p + 2] = np.frombuffer(np.uint16(0x8201).tobytes(), np.uint8)   # negative subnormal
    W = W.reshape(-1)
    x = np.zeros((4, cols), np.float32)
    x[1] = np.where(np.arange(cols) % 2, 3.0, -3.0)
    x[2] = 3.0
    x[3] = rng.standard_normal(cols).astype(np.float32)
    acts = orc.quantize_act(t, x)
    for mode in MODES:
        hip.set_order(mode[0])
        y = hip.matvec_multi(t, W, cols, rows, acts)
        ref = orc.matvec_multi(t, W, cols, rows, acts, mode[2], mode[3])
        assert np.array_equal(bits(y), bits(ref)), (mode[1], mismatch_report(y, ref))
    hip.set_order(E.ORDER_X86_CONTRACT)


def test_host_drop_in_matches_device_path(hip, orc):
    """es_hip_matvec / es_hip_matvec_multi on host memory, with and without a registered weight copy"""
    t = O.Q4_K
    rows, cols, na = 300, 2048, 4
    W, acts = mtest_inputs(orc, t, rows, cols, na, 77)
    ref = orc.matvec_multi(t, W, cols, rows, acts)
    for registered in (False, True):
        if registered:
            hip.register(W)
        y = np.full((na, rows), -1.0, np.float32)
        hip.host_matvec_multi(t, W, cols, 10, 290, acts, y)
        assert np.array_equal(bits(y[:, 10:290]), bits(ref[:, 10:290]))
        assert np.all(y[:, :10] == -1.0) and np.all(y[:, 290:] == -1.0)
        y1 = np.zeros((1, rows), np.float32)
        hip.host_matvec_multi(t, W, cols, 0, rows, acts[2:3], y1)
        assert np.array_equal(bits(y1[0]), bits(ref[2]))
    # a changed host weight is seen after es_hip_update
    W2 = W.copy()
    W[:] = orc.mtest_blocks(t, np.array([5], np.uint64), rows, cols)
    hip.update(W)
    y = np.zeros((1, rows), np.float32)
    hip.host_matvec_multi(t, W, cols, 0, rows, acts[:1], y)
    assert np.array_equal(bits(y[0]), bits(orc.matvec_multi(t, W, cols, rows, acts[:1])[0]))
    assert hip.unregister(W) == 0
    del W2


def test_run_jobs_and_plan_mixed_formats(hip, orc):
    """one queued batch over all five formats (the engine's run_jobs) == the products one by one"""
    specs, keep, refs = [], [], []
    for k, (F, rows, cols, na) in enumerate([("Q4_K", 256, 2048, 1), ("Q6_K", 130, 768, 3), ("Q2_K", 96, 1024, 2),
                                             ("Q4_0", 77, 896, 1), ("Q5_0", 64, 2048, 5), ("Q4_K", 33, 512, 4),
                                             ("Q8_0", 50, 1024, 3)]):
        t = O.TYPES[F]
        W, acts = mtest_inputs(orc, t, rows, cols, na, 300 + k)
        dW, dA, dY = hip.upload(W), hip.upload(acts), hip.alloc(na * rows * 4)
        keep += [dW, dA, dY]
        specs.append(dict(type=t, rows=rows, cols=cols, W=dW, act=dA, astride=acts.strides[0], nb=na, y=dY,
                          ystride=rows))
        refs.append((dY, na, rows, orc.matvec_multi(t, W, cols, rows, acts)))
    hip.run_jobs(specs)
    for dY, na, rows, ref in refs:
        assert np.array_equal(bits(hip.download(dY, np.zeros((na, rows), np.float32))), bits(ref))
        hip.memset(dY, 0, na * rows * 4)
    plan = hip.plan(specs)
    plan.run()
    hip.synchronize()
    for dY, na, rows, ref in refs:
        assert np.array_equal(bits(hip.download(dY, np.zeros((na, rows), np.float32))), bits(ref))
    assert plan.time_ms(1, 3) > 0
    plan.close()


@pytest.mark.parametrize("mode", [(E.ORDER_X86_CONTRACT, O.CONTRACT, O.PATH_X86), (E.ORDER_SCALAR, O.STRICT, O.PATH_SCALAR)],
                         ids=["clang", "scalar"])
def test_decode_launch_of_mixed_pass_widths(hip, orc, mode):
    """one decode-kernel launch whose jobs take different activations per pass (1, 2 and 4: 1, 2, 3, 5 and 8
    activations, as an MoE layer's experts do), for a K-quant and a 32-element format, repeated calls through a kept
    plan and fresh run_jobs calls with new values: every output equals the oracle's"""
    hip.set_order(mode[0])
    prev = (hip.set_direct_mfma_min_batch(0), hip.set_mfma_min_batch(0), hip.set_small_batch_min(0),
            hip.set_batched32_min(0), hip.set_q6k_mfma_min_batch(0))
    try:
        for F, rows, cols in (("Q4_K", 200, 2048), ("Q6_K", 70, 768), ("Q5_0", 90, 1024)):
            t = O.TYPES[F]
            for rep in range(2):
                specs, keep, refs = [], [], []
                for k, na in enumerate((1, 5, 2, 3, 8, 1, 2)):
                    W, acts = mtest_inputs(orc, t, rows, cols, na, 700 + 10 * k + rep)
                    dW, dA, dY = hip.upload(W), hip.upload(acts), hip.alloc(na * rows * 4)
                    keep += [dW, dA, dY]
                    specs.append(dict(type=t, rows=rows, cols=cols, W=dW, act=dA, astride=acts.strides[0], nb=na, y=dY,
                                      ystride=rows))
                    refs.append((dY, na, orc.matvec_multi(t, W, cols, rows, acts, mode[1], mode[2])))
                hip.run_jobs(specs)
                for dY, na, ref in refs:
                    assert np.array_equal(bits(hip.download(dY, np.zeros((na, rows), np.float32))), bits(ref)), (F, na)
    finally:
        hip.set_direct_mfma_min_batch(prev[0])
        hip.set_mfma_min_batch(prev[1])
        hip.set_small_batch_min(prev[2])
        hip.set_batched32_min(prev[3])
        hip.set_q6k_mfma_min_batch(prev[4])
        hip.set_order(E.ORDER_X86_CONTRACT)


def test_invalid_arguments_are_rejected(hip):
    buf = hip.alloc(1 << 16)
    with pytest.raises(E.EsHipError):   # cols not a multiple of the block
        hip.matvec_multi_dev(E.Q4_K, buf, 300, 0, 4, buf, 0, 1, buf, 0)
    with pytest.raises(E.EsHipError):   # misaligned weights
        hip.matvec_multi_dev(E.Q4_K, buf.offset(2), 256, 0, 4, buf, 0, 1, buf, 0)
    with pytest.raises(E.EsHipError):   # unsupported type
        hip.matvec_multi_dev(7, buf, 256, 0, 4, buf, 0, 1, buf, 0)
    with pytest.raises(E.EsHipError):   # overlapping outputs
        hip.matvec_multi_dev(E.Q4_K, buf, 256, 0, 4, buf, 292, 2, buf, 2)
    hip.matvec_multi_dev(E.Q4_K, buf, 256, 4, 4, buf, 0, 1, buf, 0)   # empty range: nothing to do
    buf.close()


def test_run_jobs_host_is_the_engine_queue(hip, orc):
    """es_hip_run_jobs_host: the engine's run_jobs queue on host memory (registered and unregistered weights, mixed formats,
    gate/up written into one buffer with ystride 2ff as moe_n/dense_n do, src/es_engine.c:899-902, 957-960)"""
    ff, n, na = 768, 2048, 3
    Wg, acts = mtest_inputs(orc, O.Q4_K, ff, n, na, 501)
    Wu, _ = mtest_inputs(orc, O.Q4_K, ff, n, na, 502)
    Wh, hacts = mtest_inputs(orc, O.Q6_K, n, ff, na, 503)
    hip.register(Wu)
    gu = np.zeros((na, 2 * ff), np.float32)
    yd = np.zeros((na, n), np.float32)
    hip.run_jobs_host([(O.Q4_K, Wg, ff, n, acts, gu[:, :ff]), (O.Q4_K, Wu, ff, n, acts, gu[:, ff:]),
                       (O.Q6_K, Wh, n, ff, hacts, yd)])
    assert np.array_equal(bits(gu[:, :ff]), bits(orc.matvec_multi(O.Q4_K, Wg, n, ff, acts)))
    assert np.array_equal(bits(gu[:, ff:]), bits(orc.matvec_multi(O.Q4_K, Wu, n, ff, acts)))
    assert np.array_equal(bits(yd), bits(orc.matvec_multi(O.Q6_K, Wh, ff, n, hacts)))
    hip.unregister(Wu)


def test_matvec_q2_K_drop_in(hip, golden):
    """es_matvec_q2_K's drop-in: the reference's own es_dot_q2_K_q8_K_ref values (kbench's correctness rows) and its scalar
    build's outputs, bit for bit, under every es_hip_set_order setting (es_matvec_q2_K never takes the AVX2 path)"""
    W, xq, want = golden["q2k/W"], golden["q2k/xq"], golden["q2k/dot_ref"]
    cols, rows = golden["q2k/x"].size, want.size
    try:
        for order in (E.ORDER_X86_CONTRACT, E.ORDER_X86_STRICT, E.ORDER_SCALAR):
            hip.set_order(order)
            y = hip.matvec_q2_K(W, cols, 0, rows, xq, rows)
            assert np.array_equal(bits(y), bits(want)), order
            cols2, rows2 = (int(v) for v in golden["Q2_K/mtest_shape"])
            acts = golden_acts(golden, "Q2_K", "mtest")
            y2 = hip.matvec_q2_K(golden["Q2_K/mtest_W"], cols2, 3, rows2, acts[0], rows2)
            assert np.array_equal(bits(y2[3:]), bits(golden["Q2_K/mtest_y_scalar"][0][3:])) and np.all(y2[:3] == 0)
    finally:
        hip.set_order(E.ORDER_X86_CONTRACT)


@pytest.mark.parametrize("F,cols", [("Q8_0", 28672), ("Q4_0", 28672), ("Q5_0", 29568), ("Q4_K", 53248), ("Q6_K", 28672),
                                    ("Q2_K", 53248), ("Q8_0", 131072), ("Q4_0", 131072), ("Q4_K", 1048576), ("Q2_K", 1048576)])
def test_long_rows(hip, orc, F, cols):
    """rows longer than the decode kernel's 8 waves cover in one pass (each wave then takes several groups of blocks in
    turn): Llama-3-70B's 28672-wide and Qwen2.5-72B's 29568-wide down projections, Llama-3.1-405B's 53248, and the longest
    rows the library takes (ES_HIP_MAX_COLS_32 = 131072 columns, ES_HIP_MAX_COLS_256 = 1048576), against the oracle at one
    and several activations"""
    t = O.TYPES[F]
    rows = 48 if cols < 131072 else 8
    W, acts = mtest_inputs(orc, t, rows, cols, 3, 99 + t + cols)
    y = hip.matvec_multi(t, W, cols, rows, acts)
    assert np.array_equal(bits(y), bits(orc.matvec_multi(t, W, cols, rows, acts)))
    y1 = hip.matvec_multi(t, W, cols, rows, acts[:1])
    assert np.array_equal(bits(y1[0]), bits(y[0]))


LONG = [("Q8_0", 3), ("Q4_0", 4096 + 5), ("Q5_0", 2), ("Q4_K", 3), ("Q6_K", 4096 + 1), ("Q2_K", 2)]


@pytest.mark.parametrize("F,extra", LONG, ids=[f"{f}+{x}" for f, x in LONG])
@pytest.mark.parametrize("mode", MODES, ids=["clang", "gcc", "scalar"])
def test_rows_past_the_limit(order, orc, F, extra, mode):
    """rows longer than ES_HIP_MAX_COLS_* (131072 / 1048576 columns) run as column pieces of at most that length, each
    continuing the chains where the one before stopped (the one chain in y; the AVX2 order's eight lane chains per output
    in a stream-ordered buffer): bit-identical to the oracle's whole-row sums in every order, at one and three
    activations, through the device entry point, run_jobs and the host drop-in; two and three pieces"""
    hip = order
    hip.set_order(mode[0])
    t = O.TYPES[F]
    be = O.BLOCK_ELEMS[t]
    cols = (131072 if be == 32 else 1048576) + extra * be
    rows = 5
    W, acts = mtest_inputs(orc, t, rows, cols, 3, 4242 + t + extra)
    ref = orc.matvec_multi(t, W, cols, rows, acts, mode[2], mode[3])
    y = hip.matvec_multi(t, W, cols, rows, acts)
    assert np.array_equal(bits(y), bits(ref)), mismatch_report(y, ref)
    y1 = hip.matvec_multi(t, W, cols, rows, acts[:1], r0=1, r1=4)
    assert np.array_equal(bits(y1[0, 1:4]), bits(ref[0, 1:4])) and np.all(y1[0, [0, 4]] == 0)
    dW, dA = hip.upload(W), hip.upload(np.ascontiguousarray(acts))
    dY = hip.upload(np.full((3, rows), -1.0, np.float32))
    hip.run_jobs([dict(type=t, rows=rows, cols=cols, W=dW, act=dA, astride=acts.strides[0], nb=3, y=dY, ystride=rows)])
    yj = hip.download(dY, np.zeros((3, rows), np.float32))
    assert np.array_equal(bits(yj), bits(ref))
    for b in (dW, dA, dY):
        b.close()
    yh = np.full((3, rows), -1.0, np.float32)
    hip.host_matvec_multi(t, W, cols, 0, rows, acts, yh)
    assert np.array_equal(bits(yh), bits(ref))
    dW, dA = hip.upload(W), hip.upload(np.ascontiguousarray(acts))
    dY = hip.upload(np.full((3, rows), -1.0, np.float32))
    plan = hip.plan([dict(type=t, rows=rows, cols=cols, W=dW, act=dA, astride=acts.strides[0], nb=3, y=dY, ystride=rows)])
    try:
        for _ in range(2):   # the kept phases and lane chains serve every run
            hip.memset(dY, 0, 3 * rows * 4)
            plan.run()
            assert np.array_equal(bits(hip.download(dY, np.zeros((3, rows), np.float32))), bits(ref))
    finally:
        plan.close()
        for b in (dW, dA, dY):
            b.close()


@pytest.mark.parametrize("F", ["Q8_0", "Q4_K"])
def test_row_limit_noalloc(hip, orc, F):
    """the no-allocation product, whose scratch is sized once, still takes rows of at most ES_HIP_MAX_COLS_*: one block
    more is refused with EINVAL and y is untouched"""
    t = O.TYPES[F]
    cmax = 131072 if O.BLOCK_ELEMS[t] == 32 else 1048576
    c = cmax + O.BLOCK_ELEMS[t]
    nbk = c // O.BLOCK_ELEMS[t]
    dW, dA = hip.alloc(4 * E.row_bytes(t, c)), hip.alloc(nbk * E.ACT_BYTES[t])
    dY = hip.upload(np.full(4, -5.0, np.float32))
    with pytest.raises(E.EsHipError) as ei:
        hip.matvec_multi_dev_noalloc(t, dW, c, 0, 4, dA, 0, 1, dY, 0)
    assert "above" in str(ei.value)
    assert np.all(hip.download(dY, np.zeros(4, np.float32)) == -5.0)
    for b in (dW, dA, dY):
        b.close()
