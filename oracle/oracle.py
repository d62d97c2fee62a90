"""ctypes binding of the CPU oracle (liboracle.so) and of the reference kernels built from source (_ref/).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker. The shipped library never loads this. Functions mirror oracle/esq_oracle.h; arrays are numpy.
"""
from __future__ import annotations

import ctypes as C
import os
import shutil
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))

Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 2, 6, 8, 10, 11, 12, 13, 14
TYPES = {"Q4_0": Q4_0, "Q5_0": Q5_0, "Q8_0": Q8_0, "Q2_K": Q2_K, "Q3_K": Q3_K, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}
NAMES = {v: k for k, v in TYPES.items()}
STRICT, CONTRACT = 0, 1
PATH_X86, PATH_SCALAR = 0, 1

# activation blocks: es_blk_q80 (src/es_quant.h:31), es_block_q8_K (src/es_q2k.h:31-38)
Q80 = np.dtype([("d", "<f4"), ("qs", "i1", (32,))])
Q8K = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
assert Q80.itemsize == 36 and Q8K.itemsize == 292

BLOCK_ELEMS = {Q4_0: 32, Q5_0: 32, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q4_0: 18, Q5_0: 22, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}


def uses_q8k(t: int) -> bool:
    return BLOCK_ELEMS[t] == 256


def row_bytes(t: int, cols: int) -> int:
    return cols // BLOCK_ELEMS[t] * BLOCK_BYTES[t]


def act_dtype(t: int):
    return Q8K if uses_q8k(t) else Q80


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


class Oracle:
    """The CPU restatement (esq_oracle.c)."""

    def __init__(self, path: str | None = None):
        # ESQ_ORACLE_LIB: another build of the oracle (the sanitizer build of the CPU sanitizer test)
        path = path or os.environ.get("ESQ_ORACLE_LIB") or os.path.join(HERE, "liboracle.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
        L = self.lib = C.CDLL(path)
        vp, i, u32, sz, f = C.c_void_p, C.c_int, C.c_uint32, C.c_size_t, C.c_float
        sig = {
            "esq_half_to_float": (f, [C.c_uint16]),
            "esq_float_to_half": (C.c_uint16, [f]),
            "esq_quantize_q8_0": (None, [vp, vp, i]),
            "esq_quantize_q8_K": (None, [vp, vp, i]),
            "esq_matvec": (None, [u32, vp, i, i, i, vp, vp, i, i]),
            "esq_matvec_multi": (None, [u32, vp, i, i, i, vp, sz, i, vp, sz, i, i]),
            "esq_block_ints": (None, [u32, vp, i, i, vp, vp, vp]),
            "esq_matvec_float": (None, [u32, vp, i, i, i, vp, vp]),
            "esq_dequant_row": (None, [u32, vp, vp, i]),
            "esq_quantize_q2_K_ref": (None, [vp, vp, i]),
            "esq_quantize_row": (None, [u32, vp, vp, i]),
            "esq_fill_gauss": (None, [C.c_uint64, f, vp, sz]),
            "esq_mtest_blocks": (None, [u32, vp, vp, i, i]),
            "esq_mtest_acts": (None, [vp, vp, sz]),
            "esq_route_softmax": (i, [vp, i, i, i, vp, vp]),
            "esq_moe_group": (i, [vp, i, i, vp, vp, vp, vp, vp]),
            "esq_swiglu": (None, [vp, vp, vp, i]),
            "esq_rmsnorm": (None, [vp, vp, vp, i, f]),
            "esq_moe_combine": (None, [vp, vp, vp, i, i, i, vp]),
            "esq_cache_trace": (i, [i, i, i, C.c_double, vp, i, vp, vp, vp]),
            "esq_cpu_bench": (C.c_double, [vp, u32, vp, sz, i, i, i, vp, sz, i, vp, i, C.c_double, vp]),
            "esq_bind_reference": (None, [vp]),
            "esq_multi_reference": (None, [u32, vp, i, i, i, vp, sz, i, vp, sz]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args

    # ---- fp16 / activations ----
    def half_to_float(self, h: int) -> float:
        return self.lib.esq_half_to_float(h)

    def float_to_half(self, x: float) -> int:
        return self.lib.esq_float_to_half(x)

    def quantize_q8_0(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        y = np.zeros(x.size // 32, Q80)
        self.lib.esq_quantize_q8_0(_p(x), _p(y), x.size)
        return y

    def quantize_q8_K(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        y = np.zeros(x.size // 256, Q8K)
        self.lib.esq_quantize_q8_K(_p(x), _p(y), x.size)
        return y

    def quantize_act(self, t: int, x: np.ndarray) -> np.ndarray:
        """x [na, cols] fp32 -> [na, nblocks] activation blocks of the type's kind"""
        x = np.ascontiguousarray(x, np.float32)
        na, cols = x.reshape(-1, x.shape[-1]).shape
        q = self.quantize_q8_K(x) if uses_q8k(t) else self.quantize_q8_0(x)
        return q.reshape(na, -1)

    # ---- products ----
    def matvec(self, t, W, cols, r0, r1, act, order=CONTRACT, path=PATH_X86, rows=None):
        rows = rows if rows is not None else r1
        y = np.zeros(rows, np.float32)
        act = np.ascontiguousarray(act)
        self.lib.esq_matvec(t, _p(W), cols, r0, r1, _p(act), _p(y), order, path)
        return y

    def matvec_multi(self, t, W, cols, rows, acts, order=CONTRACT, path=PATH_X86):
        """acts [na, nblocks] -> y [na, rows]"""
        acts = np.ascontiguousarray(acts)
        na = acts.shape[0]
        y = np.zeros((na, rows), np.float32)
        self.lib.esq_matvec_multi(t, _p(W), cols, 0, rows, _p(acts), acts.strides[0], na, _p(y), rows, order, path)
        return y

    def matvec_float(self, t, W, cols, rows, x, r0=0):
        """the float path (dequantized rows . fp32 activations): x [na, cols] -> y [na, rows], rows [r0, rows) written"""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, cols)
        y = np.zeros((x.shape[0], rows), np.float32)
        for q in range(x.shape[0]):
            self.lib.esq_matvec_float(t, _p(W), cols, r0, rows, C.c_void_p(x.ctypes.data + q * cols * 4),
                                      C.c_void_p(y.ctypes.data + q * rows * 4))
        return y

    def block_ints(self, t, W, cols, rows, act):
        nb = cols // BLOCK_ELEMS[t]
        dots = np.zeros((rows, nb), np.int32)
        aux = np.zeros((rows, nb), np.int32)
        self.lib.esq_block_ints(t, _p(W), cols, rows, _p(np.ascontiguousarray(act)), _p(dots), _p(aux))
        return dots, aux

    def dequant(self, t, W, n):
        y = np.zeros(n, np.float32)
        self.lib.esq_dequant_row(t, _p(W), _p(y), n)
        return y

    # ---- weights / inputs ----
    def quantize_rows(self, t, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        rows, cols = x.shape
        W = np.zeros(rows * row_bytes(t, cols), np.uint8)
        rb = row_bytes(t, cols)
        for r in range(rows):
            self.lib.esq_quantize_row(t, _p(x[r]), C.c_void_p(W.ctypes.data + r * rb), cols)
        return W

    def quantize_q2_K_ref(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        W = np.zeros(x.size // 256 * 84, np.uint8)
        self.lib.esq_quantize_q2_K_ref(_p(x), _p(W), x.size)
        return W

    def gauss(self, seed: int, sigma: float, n: int) -> np.ndarray:
        x = np.zeros(n, np.float32)
        self.lib.esq_fill_gauss(seed, sigma, _p(x), n)
        return x

    def mtest_blocks(self, t, state: np.ndarray, rows, cols) -> np.ndarray:
        W = np.zeros(rows * row_bytes(t, cols), np.uint8)
        self.lib.esq_mtest_blocks(t, _p(state), _p(W), rows, cols)
        return W

    def mtest_acts(self, state: np.ndarray, n) -> np.ndarray:
        x = np.zeros(n, np.float32)
        self.lib.esq_mtest_acts(_p(state), _p(x), n)
        return x

    # ---- MoE glue ----
    def route_softmax(self, logits: np.ndarray, k: int, norm_topk: bool):
        """logits [n_tok, ne] -> sel [n_tok, k] int32, w [n_tok, k] fp32 (softmax probs left in a copy)"""
        lg = np.ascontiguousarray(logits, np.float32).copy()
        n_tok, ne = lg.shape
        sel = np.zeros((n_tok, k), np.int32)
        w = np.zeros((n_tok, k), np.float32)
        for t in range(n_tok):
            self.lib.esq_route_softmax(C.c_void_p(lg.ctypes.data + t * ne * 4), ne, k, int(norm_topk),
                                       C.c_void_p(sel.ctypes.data + t * k * 4), C.c_void_p(w.ctypes.data + t * k * 4))
        return sel, w, lg

    def moe_group(self, sel: np.ndarray):
        sel = np.ascontiguousarray(sel, np.int32)
        n_tok, k = sel.shape
        n = n_tok * k
        uex, cnt, start = (np.zeros(n, np.int32) for _ in range(3))
        rowof = np.zeros((n_tok, k), np.int32)
        tok_of = np.zeros(n, np.int32)
        nu = self.lib.esq_moe_group(_p(sel), n_tok, k, _p(uex), _p(cnt), _p(start), _p(rowof), _p(tok_of))
        return uex[:nu].copy(), cnt[:nu].copy(), start[:nu].copy(), rowof, tok_of

    def swiglu(self, g: np.ndarray, u: np.ndarray) -> np.ndarray:
        g = np.ascontiguousarray(g, np.float32)
        u = np.ascontiguousarray(u, np.float32)
        h = np.zeros_like(g)
        self.lib.esq_swiglu(_p(g), _p(u), _p(h), g.size)
        return h

    def cache_trace(self, nslots, nlayers, nexperts, freq_weight, ops):
        """the hot-expert cache policy restated (esq_cache.c): -> (res, slots [nslots, 7], stats [7])"""
        return cache_trace_run(self.lib.esq_cache_trace, nslots, nlayers, nexperts, freq_weight, ops)

    def rmsnorm(self, x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
        """rows of x (2-D) normalised one by one"""
        x = np.ascontiguousarray(x, np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        o = np.zeros_like(x2)
        wp = None if w is None else np.ascontiguousarray(w, np.float32)
        for r in range(x2.shape[0]):
            self.lib.esq_rmsnorm(_p(x2[r]), None if wp is None else _p(wp), _p(o[r]), x2.shape[1], eps)
        return o.reshape(x.shape)

    def moe_combine(self, ye: np.ndarray, rowof: np.ndarray, w: np.ndarray) -> np.ndarray:
        n_tok, k = rowof.shape
        n = ye.shape[1]
        out = np.zeros((n_tok, n), np.float32)
        self.lib.esq_moe_combine(_p(np.ascontiguousarray(ye, np.float32)), _p(np.ascontiguousarray(rowof, np.int32)),
                                 _p(np.ascontiguousarray(w, np.float32)), n_tok, k, n, _p(out))
        return out

    def moe_ffn(self, types, experts, n, ff, x_acts, sel, w, k=None, order=CONTRACT, path=PATH_X86):
        """The expert part of moe_n (src/es_engine.c:871-932) for N tokens, composed from the restated pieces:
        types = (gate, up, down); experts[e] = (Wg, Wu, Wd) block bytes; x_acts [N, blocks] Q8 rows of the gate/up type;
        sel, w [N, kmax]; k [N] experts per token (default kmax). Returns out [N, n]."""
        sel = np.asarray(sel, np.int32)
        N, kmax = sel.shape
        k = np.full(N, kmax, np.int32) if k is None else np.asarray(k, np.int32)
        uex, cnt = [], []            # distinct experts in order of first use (:871-879)
        for t in range(N):
            for j in range(k[t]):
                e = int(sel[t, j])
                if e not in uex:
                    uex.append(e)
                    cnt.append(0)
                cnt[uex.index(e)] += 1
        start = np.concatenate([[0], np.cumsum(cnt)[:-1]]).astype(int) if uex else np.zeros(0, int)
        fill = [0] * len(uex)
        rowof = np.zeros((N, kmax), np.int32)
        tok_of = np.zeros(int(sum(cnt)), np.int32)
        for t in range(N):           # (:880-888)
            for j in range(k[t]):
                u = uex.index(int(sel[t, j]))
                r = start[u] + fill[u]
                fill[u] += 1
                rowof[t, j] = r
                tok_of[r] = t
        R = len(tok_of)
        gt, ut, dt = types
        gu = np.zeros((R, 2 * ff), np.float32)
        for u, e in enumerate(uex):  # gate/up multi-jobs (:899-903)
            rows = slice(start[u], start[u] + cnt[u])
            xa = x_acts[tok_of[rows]]
            gu[rows, :ff] = self.matvec_multi(gt, experts[e][0], n, ff, xa, order, path)
            gu[rows, ff:] = self.matvec_multi(ut, experts[e][1], n, ff, xa, order, path)
        h = self.swiglu(gu[:, :ff], gu[:, ff:]) if R else np.zeros((0, ff), np.float32)   # (:913)
        ha = self.quantize_act(dt, h) if R else None                                      # (:914)
        ye = np.zeros((R, n), np.float32)
        for u, e in enumerate(uex):  # down multi-jobs (:916-918)
            rows = slice(start[u], start[u] + cnt[u])
            ye[rows] = self.matvec_multi(dt, experts[e][2], ff, n, ha[rows], order, path)
        out = np.zeros((N, n), np.float32)
        for t in range(N):           # combine (:925-932), one token at a time so k may vary
            if k[t]:
                out[t] = self.moe_combine(ye, rowof[t:t + 1, :k[t]], np.asarray(w, np.float32)[t:t + 1, :k[t]])[0]
        return out

    # ---- CPU baseline ----
    def cpu_bench(self, fn_ptr, t, W, mat_bytes, nmat, rows, cols, acts, nthreads, min_seconds=0.4):
        acts = np.ascontiguousarray(acts)
        na = acts.shape[0]
        y = np.zeros((na, rows), np.float32)
        passes = C.c_int(0)
        sec = self.lib.esq_cpu_bench(fn_ptr, t, _p(W), mat_bytes, nmat, rows, cols, _p(acts), acts.strides[0], na,
                                     _p(y), nthreads, min_seconds, C.byref(passes))
        return sec, passes.value, y

    def multi_fn_ptr(self):
        return C.cast(self.lib.esq_multi_x86_contract, C.c_void_p)

    def reference_fn_ptr(self, ref: "RefLib"):
        """the reference's es_matvec_multi (from a RefLib) behind the esq_multi_fn signature"""
        self.lib.esq_bind_reference(C.cast(ref.lib.es_matvec_multi, C.c_void_p))
        return C.cast(self.lib.esq_multi_reference, C.c_void_p)

    def matvec_multi_reference(self, ref: "RefLib", t, W, cols, rows, acts):
        """acts [na, nblocks] through the reference's es_matvec_multi (es_act records over these blocks)"""
        self.reference_fn_ptr(ref)
        acts = np.ascontiguousarray(acts)
        na = acts.shape[0]
        y = np.zeros((na, rows), np.float32)
        self.lib.esq_multi_reference(t, _p(W), cols, 0, rows, _p(acts), acts.strides[0], na, _p(y), rows)
        return y


# ---------------------------------------------------------------------------------------------------------------------
# the reference's kernels built from its own sources (oracle/_ref, see oracle/Makefile)

class _EsAct(C.Structure):   # es_act, src/es_quant.h:32-37
    _fields_ = [("x", C.c_void_p), ("q8", C.c_void_p), ("q80", C.c_void_p), ("cols", C.c_int)]


# ---- expert cache traces (esq_cache.h) ----
OP_STEP, OP_ACQUIRE, OP_PREFETCH = 1, 2, 3


def cache_trace_run(fn, nslots, nlayers, nexperts, freq_weight, ops):
    """run a trace [n, 3] int32 through fn (esq_cache_trace or esref_cache_trace) -> (res, slots [nslots, 7], stats [7])"""
    ops = np.ascontiguousarray(ops, np.int32).reshape(-1, 3)
    res = np.zeros(len(ops), np.int32)
    slots = np.zeros((nslots, 7), np.int64)
    stats = np.zeros(7, np.uint64)
    rc = fn(nslots, nlayers, nexperts, float(freq_weight), _p(ops), len(ops), _p(res), _p(slots), _p(stats))
    if rc:
        raise ValueError("bad cache trace arguments")
    return res, slots, stats


def make_cache_trace(seed, nlayers, nexperts, k, tokens, passes, prefetch="top"):
    """an engine-like trace: for each pass over the layers, each layer one load_experts call of k distinct experts drawn
    with a skewed popularity (so some experts stay hot), followed by a prefetch of k/2 experts of the next layer: its
    most popular ones (prefetch="top"), random ones (prefetch="random", many of them wasted) or none (None)"""
    rng = np.random.default_rng(seed)
    pop = rng.zipf(1.3, size=(nlayers, nexperts)).astype(np.float64)
    pop /= pop.sum(axis=1, keepdims=True)
    ops = []
    for _ in range(passes):
        for l in range(nlayers):
            for _ in range(tokens):
                sel = rng.choice(nexperts, size=k, replace=False, p=pop[l])
                ops.append((OP_STEP, l, 0))
                ops += [(OP_ACQUIRE, l, int(e)) for e in sel]
                if prefetch and l + 1 < nlayers:
                    guess = (np.argsort(-pop[l + 1], kind="stable")[: max(1, k // 2)] if prefetch == "top" else
                             rng.choice(nexperts, size=max(1, k // 2), replace=False))
                    ops += [(OP_PREFETCH, l + 1, int(e)) for e in guess]
    return np.array(ops, np.int32)


class RefEngine:
    """the reference engine's own route() and rmsnorm() (src/es_engine.c:744-835, 189-194), compiled from its source by
    oracle/Makefile into oracle/_ref/libesref_engine_{clang,gcc}.so through esq_engine_ref.c"""

    def __init__(self, cc: str = "clang"):
        path = os.path.join(HERE, "_ref", f"libesref_engine_{cc}.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` where /root/reference exists")
        self.lib = C.CDLL(path)
        self.lib.esref_route.restype = C.c_int
        self.lib.esref_route.argtypes = [C.c_int, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p, C.c_void_p]
        self.lib.esref_rmsnorm.restype = None
        self.lib.esref_rmsnorm.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_float]

    def route(self, logits: np.ndarray, k: int, norm_topk: bool):
        """softmax gating over rows of logits -> (sel [n_tok, k] int32, w [n_tok, k] fp32)"""
        lg = np.ascontiguousarray(logits, np.float32)
        n_tok, ne = lg.shape
        sel = np.zeros((n_tok, k), np.int32)
        w = np.zeros((n_tok, k), np.float32)
        got = self.lib.esref_route(n_tok, ne, k, int(norm_topk), _p(lg), _p(sel), _p(w))
        if got != k:
            raise RuntimeError(f"reference route() returned k={got}, expected {k}")
        return sel, w

    def rmsnorm(self, x: np.ndarray, w: np.ndarray | None, eps: float) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        x2 = x.reshape(-1, x.shape[-1])
        o = np.zeros_like(x2)
        wp = None if w is None else np.ascontiguousarray(w, np.float32)
        self.lib.esref_rmsnorm(_p(o), _p(x2), None if wp is None else _p(wp), x2.shape[0], x2.shape[1], eps)
        return o.reshape(x.shape)


def ref_engine_available(cc: str = "clang") -> bool:
    return os.path.exists(os.path.join(HERE, "_ref", f"libesref_engine_{cc}.so"))


class RefCache:
    """the reference's es_cache.c driven by esq_cache_ref.c (oracle/_ref/libesref_cache.so)"""

    def __init__(self):
        path = os.path.join(HERE, "_ref", "libesref_cache.so")
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` where /root/reference exists")
        self.lib = C.CDLL(path)
        self.lib.esref_cache_trace.restype = C.c_int
        self.lib.esref_cache_trace.argtypes = [C.c_int, C.c_int, C.c_int, C.c_double] + [C.c_void_p, C.c_int] + [C.c_void_p] * 3

    def trace(self, nslots, nlayers, nexperts, freq_weight, ops):
        return cache_trace_run(self.lib.esref_cache_trace, nslots, nlayers, nexperts, freq_weight, ops)


def ref_path(cc: str) -> str:
    return os.path.join(HERE, "_ref", f"libesref_{cc}.so")


def ref_available(cc: str = "gcc") -> bool:
    return os.path.exists(ref_path(cc))


class RefLib:
    """The reference's es_quant.c/es_q2k.c, compiled from /root/reference by oracle/Makefile.

    scalar=True loads a private copy of the library with ES_NO_AVX2 set before its first call, which selects the
    scalar mv_* kernels (src/es_quant.c:1833, 1857); the variable is read once per library instance.
    """

    def __init__(self, cc: str = "gcc", scalar: bool = False):
        path = ref_path(cc)
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run `make -C oracle ref` where /root/reference exists")
        self._tmp = None
        if scalar:
            self._tmp = tempfile.mkdtemp(prefix="esref_")
            dst = os.path.join(self._tmp, f"libesref_{cc}_scalar.so")
            shutil.copy(path, dst)
            path = dst
        old = os.environ.get("ES_NO_AVX2")
        if scalar:
            os.environ["ES_NO_AVX2"] = "1"
        elif "ES_NO_AVX2" in os.environ:
            del os.environ["ES_NO_AVX2"]
        L = self.lib = C.CDLL(path)
        vp, i, u32, sz = C.c_void_p, C.c_int, C.c_uint32, C.c_size_t
        for name, res, args in [
            ("es_act_arena_init", None, [sz]),
            ("es_act_arena_reset", None, []),
            ("es_act_prepare", None, [vp, vp, i, vp]),
            ("es_matvec", None, [u32, vp, i, i, i, vp, vp, vp]),
            ("es_matvec_multi", None, [u32, vp, i, i, i, vp, i, vp, sz, vp]),
            ("es_row_bytes", sz, [u32, i]),
            ("es_dequant_row", None, [u32, vp, vp, i]),
            ("es_quantize_q8_K", None, [vp, vp, i]),
            ("es_quantize_q2_K_ref", None, [vp, vp, i]),
            ("es_fp32_to_fp16", C.c_uint16, [C.c_float]),
            ("es_dot_q2_K_q8_K_ref", C.c_float, [i, vp, vp]),
            ("es_dot_q2_K_q8_K", C.c_float, [i, vp, vp]),
        ]:
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args
        L.es_act_arena_init(1 << 26)
        # force the one-time dispatch decision now, while the environment is as requested
        self._warm()
        if old is None:
            os.environ.pop("ES_NO_AVX2", None)
        else:
            os.environ["ES_NO_AVX2"] = old

    def _warm(self):
        x = np.ones(256, np.float32)
        W = np.zeros(144, np.uint8)
        self.matvec_f32(Q4_K, W, 256, 1, x[None, :])

    def prepare(self, x: np.ndarray):
        """fp32 rows -> (es_act array, keep-alive list, q80 view, q8K view) exactly as es_act_prepare makes them"""
        x = np.ascontiguousarray(x, np.float32)
        na, cols = x.shape
        self.lib.es_act_arena_reset()
        nk = cols // 256
        q8 = np.zeros((na, max(nk, 1)), Q8K)
        acts = (_EsAct * na)()
        for q in range(na):
            self.lib.es_act_prepare(C.byref(acts[q]), C.c_void_p(x.ctypes.data + q * cols * 4), cols,
                                    C.c_void_p(q8.ctypes.data + q * q8.strides[0]) if nk else None)
        q80 = np.zeros((na, cols // 32), Q80)
        for q in range(na):
            if acts[q].q80:
                C.memmove(q80.ctypes.data + q * q80.strides[0], acts[q].q80, (cols // 32) * 36)
        return acts, [x, q8], q80, q8[:, :nk]

    def matvec_f32(self, t, W, cols, rows, x: np.ndarray, r0=0, multi=False):
        """x [na, cols] fp32 through es_act_prepare + es_matvec (one per activation) or es_matvec_multi"""
        acts, keep, _, _ = self.prepare(x)
        na = x.shape[0]
        y = np.zeros((na, rows), np.float32)
        scratch = np.zeros(cols, np.float32)
        if multi:
            self.lib.es_matvec_multi(t, _p(W), cols, r0, rows, acts, na, _p(y), rows, _p(scratch))
        else:
            for q in range(na):
                self.lib.es_matvec(t, _p(W), cols, r0, rows, C.byref(acts[q]), C.c_void_p(y.ctypes.data + q * rows * 4),
                                   _p(scratch))
        del keep
        return y

    def matvec_float(self, t, W, cols, rows, x: np.ndarray, r0=0, multi=False):
        """x [na, cols] fp32 as activations prepared without blocks (es_act.q8 = q80 = NULL, what es_act_prepare leaves
        under ES_FLOAT_ACT or an exhausted arena): es_matvec's float path, one call per activation or es_matvec_multi"""
        x = np.ascontiguousarray(x, np.float32)
        na = x.shape[0]
        acts = (_EsAct * na)()
        for q in range(na):
            acts[q].x, acts[q].q8, acts[q].q80, acts[q].cols = x.ctypes.data + q * cols * 4, None, None, cols
        y = np.zeros((na, rows), np.float32)
        scratch = np.zeros(cols, np.float32)
        if multi:
            self.lib.es_matvec_multi(t, _p(W), cols, r0, rows, acts, na, _p(y), rows, _p(scratch))
        else:
            for q in range(na):
                self.lib.es_matvec(t, _p(W), cols, r0, rows, C.byref(acts[q]), C.c_void_p(y.ctypes.data + q * rows * 4),
                                   _p(scratch))
        return y

    def quantize_q8_K(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        y = np.zeros(x.size // 256, Q8K)
        self.lib.es_quantize_q8_K(_p(x), _p(y), x.size)
        return y

    def quantize_q2_K_ref(self, x):
        x = np.ascontiguousarray(x, np.float32).reshape(-1)
        W = np.zeros(x.size // 256 * 84, np.uint8)
        self.lib.es_quantize_q2_K_ref(_p(x), _p(W), x.size)
        return W

    def dequant(self, t, W, n):
        y = np.zeros(n, np.float32)
        self.lib.es_dequant_row(t, _p(W), _p(y), n)
        return y

    def fp32_to_fp16(self, f):
        return self.lib.es_fp32_to_fp16(f)

    def multi_fn_ptr(self):
        return None   # the reference's es_matvec_multi takes es_act*, not strided blocks; timed via bench_ref below
