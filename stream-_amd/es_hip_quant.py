"""ctypes binding of libes_hip_quant.so (the C ABI of include/es_hip_quant.h).

Plumbing for the tests and bench.py: device buffers, job tables and the drop-in entry points, with numpy arrays on the host
side. Every compute call goes through the HIP library; a failing call raises EsHipError with the library's message, and a
missing library or device raises too: there is no CPU path here.
"""
from __future__ import annotations

import ctypes as C
import os

import weakref

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# ES_HIP_LIB: another build of the same library (the host-sanitizer build of the CPU sanitizer test)
LIB_PATH = os.environ.get("ES_HIP_LIB") or os.path.join(HERE, "libes_hip_quant.so")

Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 2, 6, 8, 10, 11, 12, 13, 14
TYPES = {"Q4_0": Q4_0, "Q5_0": Q5_0, "Q8_0": Q8_0, "Q2_K": Q2_K, "Q3_K": Q3_K, "Q4_K": Q4_K, "Q5_K": Q5_K, "Q6_K": Q6_K}
ORDER_X86_CONTRACT, ORDER_X86_STRICT, ORDER_SCALAR = 0, 1, 2
NOALLOC_SCRATCH_BYTES = 32 << 20   # ES_HIP_NOALLOC_SCRATCH_BYTES
BLOCK_ELEMS = {Q4_0: 32, Q5_0: 32, Q8_0: 32, Q2_K: 256, Q3_K: 256, Q4_K: 256, Q5_K: 256, Q6_K: 256}
BLOCK_BYTES = {Q4_0: 18, Q5_0: 22, Q8_0: 34, Q2_K: 84, Q3_K: 110, Q4_K: 144, Q5_K: 176, Q6_K: 210}
ACT_BYTES = {Q4_0: 36, Q5_0: 36, Q8_0: 36, Q2_K: 292, Q3_K: 292, Q4_K: 292, Q5_K: 292, Q6_K: 292}


class EsHipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"es_hip error {code}: {msg}")
        self.code = code


class Job(C.Structure):   # es_hip_job
    _fields_ = [("type", C.c_uint32), ("rows", C.c_int), ("cols", C.c_int), ("W", C.c_void_p), ("act", C.c_void_p),
                ("astride", C.c_size_t), ("nb", C.c_int), ("y", C.c_void_p), ("ystride", C.c_size_t)]


class Moe(C.Structure):   # es_hip_moe
    _fields_ = [("gate_type", C.c_uint32), ("up_type", C.c_uint32), ("down_type", C.c_uint32), ("n", C.c_int),
                ("ff", C.c_int), ("n_exp", C.c_int), ("gate", C.c_void_p), ("up", C.c_void_p), ("down", C.c_void_p)]


class Act(C.Structure):   # es_hip_act (= the reference's es_act)
    _fields_ = [("x", C.c_void_p), ("q8", C.c_void_p), ("q80", C.c_void_p), ("cols", C.c_int)]


class HostJob(C.Structure):   # es_hip_host_job (= the reference engine's mv_job)
    _fields_ = [("type", C.c_uint32), ("w", C.c_void_p), ("rows", C.c_int), ("cols", C.c_int), ("a", C.c_void_p),
                ("y", C.c_void_p), ("nb", C.c_int), ("ys", C.c_size_t)]


def act_records(t: int, acts, cols: int, x=None, floats=()):
    """es_act records pointing at the rows of `acts` [na, nblocks] (q8 for K-quants, q80 for Q4_0/Q5_0/Q8_0) and of x
    [na, cols] fp32 when given; the activations listed in `floats` (all of them when acts is None) carry no blocks, as
    es_act_prepare leaves them without a Q8_K buffer or Q8_0 arena room, and take the float path"""
    na = acts.shape[0] if acts is not None else x.shape[0]
    recs = (Act * max(na, 1))()
    for q in range(na):
        px = x.ctypes.data + q * x.strides[0] if x is not None else None
        if acts is None or q in floats:
            recs[q] = Act(px, None, None, cols)
            continue
        p = acts.ctypes.data + q * acts.strides[0]
        recs[q] = Act(px, p if BLOCK_ELEMS[t] == 256 else None, p if BLOCK_ELEMS[t] == 32 else None, cols)
    return recs


def row_bytes(t: int, cols: int) -> int:
    return cols // BLOCK_ELEMS[t] * BLOCK_BYTES[t]


def act_bytes(t: int, cols: int) -> int:
    return cols // BLOCK_ELEMS[t] * ACT_BYTES[t]


class DevBuf:
    """A device allocation owned by Python; freed on close() or garbage collection."""

    def __init__(self, lib: "Lib", nbytes: int):
        self.lib, self.nbytes = lib, int(nbytes)
        self.ptr = lib._L.es_hip_malloc(max(self.nbytes, 1))
        if not self.ptr:
            raise EsHipError(-4, lib.last_error())

    def close(self):
        if self.ptr:
            self.lib._L.es_hip_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __int__(self):
        return int(self.ptr)

    def offset(self, nbytes: int) -> int:
        return int(self.ptr) + int(nbytes)


class SlotInfo(C.Structure):
    _fields_ = [("layer", C.c_int), ("expert", C.c_int), ("state", C.c_int), ("prefetched", C.c_int),
                ("last_use", C.c_uint64), ("uses", C.c_uint32), ("protect_until", C.c_uint64)]


class CacheStats(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in ("hits", "misses", "prefetch_issued", "prefetch_used", "prefetch_wasted",
                                          "evictions", "step")]


class ExpertSrc(C.Structure):
    """es_hip_expert_src: part r of expert e is bytes[r] bytes at base[r] + e * stride[r], placed at offset[r] in the slot"""
    _fields_ = [("base", C.c_void_p * 3), ("stride", C.c_uint64 * 3), ("bytes", C.c_uint64 * 3), ("offset", C.c_uint64 * 3)]


EBUSY = -5
ES_HIP_SLOT_EMPTY, ES_HIP_SLOT_LOADING, ES_HIP_SLOT_READY = 0, 1, 2


class ExpertCache:
    """es_hip_cache_*: the reference's hot-expert cache with its slots in HBM (slot_bytes = 0: bookkeeping only)"""

    def __init__(self, lib, nslots, slot_bytes, nlayers, nexperts, freq_weight):
        self.lib, self.nslots, self.h = lib, nslots, None
        h = C.c_void_p()
        lib._check(lib._L.es_hip_cache_create(C.byref(h), nslots, slot_bytes, nlayers, nexperts, float(freq_weight)))
        self.h = h.value

    def close(self):
        if self.h:
            self.lib._L.es_hip_cache_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def find(self, layer, expert):
        return self.lib._L.es_hip_cache_find(self.h, layer, expert)

    def claim(self, layer, expert):
        return self.lib._check(self.lib._L.es_hip_cache_claim(self.h, layer, expert))

    def slot_ptr(self, slot):
        return self.lib._L.es_hip_cache_slot_ptr(self.h, slot)

    def load(self, slot, offset, host: np.ndarray, stream=None):
        self.lib._check(self.lib._L.es_hip_cache_load(self.h, slot, offset, host.ctypes.data, host.nbytes, stream))

    def wait(self, slot):
        self.lib._check(self.lib._L.es_hip_cache_wait(self.h, slot))

    def step(self):
        self.lib._check(self.lib._L.es_hip_cache_step(self.h))

    def acquire(self, layer, sel, src=None, stream=None, allow_busy=False):
        sel = np.ascontiguousarray(sel, np.int32)
        slots = np.zeros(len(sel), np.int32)
        rc = self.lib._L.es_hip_cache_acquire(self.h, layer, sel.ctypes.data, len(sel), C.byref(src) if src else None,
                                              slots.ctypes.data, stream)
        if not (allow_busy and rc == EBUSY):
            self.lib._check(rc)
        return slots

    def prefetch(self, layer, expert, src=None, stream=None):
        """the claimed slot; -2 if the expert was cached already, -1 if no slot was free (the oracle's trace codes)"""
        slot = C.c_int(-1)
        rc = self.lib._L.es_hip_cache_prefetch(self.h, layer, expert, C.byref(src) if src else None, stream, C.byref(slot))
        if rc == EBUSY:
            return -1
        self.lib._check(rc)
        return slot.value if slot.value >= 0 else -2

    def slot_info(self, slot):
        o = SlotInfo()
        self.lib._check(self.lib._L.es_hip_cache_slot_info(self.h, slot, C.byref(o)))
        return o

    def stats(self):
        o = CacheStats()
        self.lib._check(self.lib._L.es_hip_cache_get_stats(self.h, C.byref(o)))
        return o

    def run_trace(self, ops):
        """replay an oracle cache trace (ops [n, 3]: 1 = step, 2 = acquire, 3 = prefetch; a step and the acquires after it
        are one es_hip_cache_acquire call) -> (res, slots [nslots, 7], stats [7]) in the oracle's format"""
        ops = np.asarray(ops, np.int32).reshape(-1, 3)
        res = np.zeros(len(ops), np.int32)
        i = 0
        while i < len(ops):
            op, l, e = (int(v) for v in ops[i])
            if op == 1:
                j = i + 1
                while j < len(ops) and ops[j, 0] == 2 and ops[j, 1] == l:
                    j += 1
                res[i + 1:j] = self.acquire(l, ops[i + 1:j, 2], allow_busy=True)
                i = j
                continue
            if op == 3:
                res[i] = self.prefetch(l, e)
            else:
                raise ValueError(f"operation {op} outside a step")
            i += 1
        slots = np.array([[x.layer, x.expert, x.state, x.prefetched, x.last_use, x.uses, x.protect_until]
                          for x in (self.slot_info(k) for k in range(self.nslots))], np.int64)
        st = self.stats()
        stats = np.array([st.hits, st.misses, st.prefetch_issued, st.prefetch_used, st.prefetch_wasted, st.evictions, st.step],
                         np.uint64)
        return res, slots, stats


class Lib:
    def __init__(self, path: str | None = None):
        path = path or LIB_PATH
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is missing: build it with `make -C stream-_amd` (or __graft_entry__.build())")
        L = self._L = C.CDLL(path)
        vp, i, u32, sz = C.c_void_p, C.c_int, C.c_uint32, C.c_size_t
        for name, res, args in [
            ("es_hip_available", i, []), ("es_hip_last_error", C.c_char_p, []), ("es_hip_device_name", C.c_char_p, []),
            ("es_hip_set_order", i, [i]), ("es_hip_get_order", i, []),
            ("es_hip_quant_supported", i, [u32]), ("es_hip_row_bytes", sz, [u32, i]),
            ("es_hip_malloc", vp, [sz]), ("es_hip_free", i, [vp]),
            ("es_hip_host_alloc", vp, [sz]), ("es_hip_host_free", i, [vp]),
            ("es_hip_matvec_q2_K", None, [vp, i, i, i, vp, vp]), ("es_hip_q2k_kernel_name", C.c_char_p, []),
            ("es_hip_q2k_force_scalar", None, [i]),
            ("es_hip_memcpy_h2d", i, [vp, vp, sz]), ("es_hip_memcpy_d2h", i, [vp, vp, sz]),
            ("es_hip_memcpy_d2d", i, [vp, vp, sz]), ("es_hip_memset", i, [vp, i, sz]), ("es_hip_synchronize", i, []),
            ("es_hip_matvec_dev", i, [u32, vp, i, i, i, vp, vp, vp]),
            ("es_hip_matvec_multi_dev", i, [u32, vp, i, i, i, vp, sz, i, vp, sz, vp]),
            ("es_hip_matvec_multi_dev_noalloc", i, [u32, vp, i, i, i, vp, sz, i, vp, sz, vp]),
            ("es_hip_dense_ffn_dev", i, [u32, vp, u32, vp, u32, vp, i, i, i, vp, sz, vp, vp, vp, sz, vp]),
            ("es_hip_moe_ctx_create", vp, [vp, i, i]), ("es_hip_moe_ctx_destroy", None, [vp]),
            ("es_hip_moe_ctx_run", i, [vp, i, vp, vp, vp, sz, vp, sz, vp]),
            ("es_hip_moe_ctx_run_logits", i, [vp, i, vp, sz, i, vp, sz, vp, sz, vp, vp, vp]),
            ("es_hip_run_jobs", i, [vp, i, vp]),
            ("es_hip_plan_create", vp, [vp, i]), ("es_hip_plan_run", i, [vp, vp]), ("es_hip_plan_destroy", None, [vp]),
            ("es_hip_plan_time_ms", C.c_double, [vp, i, i, vp]),
            ("es_hip_register", i, [vp, sz]), ("es_hip_update", i, [vp]), ("es_hip_unregister", i, [vp]),
            ("es_hip_matvec", None, [u32, vp, i, i, i, vp, vp, vp]),
            ("es_hip_matvec_multi", None, [u32, vp, i, i, i, vp, i, vp, sz, vp]),
            ("es_hip_block_ints_dev", i, [u32, vp, i, i, vp, vp, vp, vp]),
            ("es_hip_run_jobs_host", i, [vp, i]),
            ("es_hip_set_mfma_min_batch", i, [i]), ("es_hip_set_small_batch_min", i, [i]),
            ("es_hip_set_mfma_tile", i, [i, i, i]),
            ("es_hip_set_batched32_min", i, [i]), ("es_hip_set_batched32_mfma_min", i, [i]), ("es_hip_set_q6k_mfma_min_batch", i, [i]), ("es_hip_set_q2k_mfma_min_batch", i, [i]), ("es_hip_set_direct_mfma_min_batch", i, [i]), ("es_hip_set_direct_mfma_min_tiles", i, [i]), ("es_hip_set_q5k_mfma_min_batch", i, [i]), ("es_hip_set_q3k_mfma_min_batch", i, [i]), ("es_hip_set_q2k_expert_max_batch", i, [i]), ("es_hip_set_moe_gated", i, [i]), ("es_hip_set_batched32_direct", i, [i]), ("es_hip_set_q6k_persistent", i, [i]), ("es_hip_set_direct_mfma_tok64", i, [i]), ("es_hip_set_direct_persistent", i, [i]),
            ("es_hip_moe_ffn", i, [vp, i, vp, vp, vp, i, vp, sz, vp, sz, vp]),
            ("es_hip_moe_plan_create", vp, [vp, i, vp, vp, vp, i, vp, sz, vp, sz]),
            ("es_hip_moe_plan_run", i, [vp, vp]), ("es_hip_moe_plan_destroy", None, [vp]),
            ("es_hip_moe_ffn_logits", i, [vp, i, vp, sz, i, i, vp, sz, vp, sz, vp, vp, vp]),
            ("es_hip_step_time_ms", C.c_double, [vp, i, vp, i, i, i, vp]),
            ("es_hip_swiglu_dev", i, [vp, vp, vp, C.c_long, vp]),
            ("es_hip_act_prepare_dev", i, [vp, sz, i, i, vp, sz, vp, sz, vp]),
            ("es_hip_route_softmax_dev", i, [vp, sz, i, i, i, i, vp, vp, i, vp]),
            ("es_hip_dequant_row_dev", i, [u32, vp, vp, C.c_long, vp]),
            ("es_hip_matvec_float_dev", i, [u32, vp, i, i, i, vp, sz, i, vp, sz, vp]),
            ("es_hip_rmsnorm_prepare_dev", i, [vp, sz, vp, C.c_float, i, i, vp, sz, vp, sz, vp, sz, vp]),
            ("es_hip_swiglu_prepare_dev", i, [vp, sz, i, i, vp, sz, vp, sz, vp, sz, vp]),
            ("es_hip_cache_create", i, [vp, i, sz, i, i, C.c_double]), ("es_hip_cache_destroy", None, [vp]),
            ("es_hip_cache_find", i, [vp, i, i]), ("es_hip_cache_claim", i, [vp, i, i]),
            ("es_hip_cache_slot_ptr", vp, [vp, i]), ("es_hip_cache_load", i, [vp, i, sz, vp, sz, vp]),
            ("es_hip_cache_wait", i, [vp, i]), ("es_hip_cache_step", i, [vp]),
            ("es_hip_cache_acquire", i, [vp, i, vp, i, vp, vp, vp]), ("es_hip_cache_prefetch", i, [vp, i, i, vp, vp, vp]),
            ("es_hip_cache_slot_info", i, [vp, i, vp]), ("es_hip_cache_get_stats", i, [vp, vp]),
        ]:
            fn = getattr(L, name)
            fn.restype, fn.argtypes = res, args

    # ---- state ----
    def available(self) -> bool:
        return bool(self._L.es_hip_available())

    def last_error(self) -> str:
        return (self._L.es_hip_last_error() or b"").decode()

    def device_name(self) -> str:
        return (self._L.es_hip_device_name() or b"").decode()

    def set_order(self, order: int) -> int:
        return self._check(self._L.es_hip_set_order(order))

    def get_order(self) -> int:
        return self._L.es_hip_get_order()

    def set_mfma_min_batch(self, n: int) -> int:
        return self._L.es_hip_set_mfma_min_batch(n)

    def set_small_batch_min(self, n: int) -> int:
        return self._L.es_hip_set_small_batch_min(n)

    def set_mfma_tile(self, bm: int = 0, bn: int = 0, waves: int = 0) -> int:
        return self._check(self._L.es_hip_set_mfma_tile(bm, bn, waves))

    def set_batched32_min(self, n: int) -> int:
        return self._L.es_hip_set_batched32_min(n)

    def set_batched32_mfma_min(self, n: int) -> int:
        return self._L.es_hip_set_batched32_mfma_min(n)

    def set_q6k_mfma_min_batch(self, n: int) -> int:
        return self._L.es_hip_set_q6k_mfma_min_batch(n)

    def set_q2k_mfma_min_batch(self, n: int) -> int:
        return self._L.es_hip_set_q2k_mfma_min_batch(n)

    def set_direct_mfma_min_batch(self, n: int) -> int:
        return self._L.es_hip_set_direct_mfma_min_batch(n)

    def set_direct_mfma_min_tiles(self, n: int) -> int:
        return self._L.es_hip_set_direct_mfma_min_tiles(n)

    def set_q5k_mfma_min_batch(self, n: int) -> int:
        return self._L.es_hip_set_q5k_mfma_min_batch(n)

    def set_q3k_mfma_min_batch(self, n: int) -> int:
        return self._L.es_hip_set_q3k_mfma_min_batch(n)

    def set_q2k_expert_max_batch(self, n: int) -> int:
        return self._L.es_hip_set_q2k_expert_max_batch(n)

    def set_moe_gated(self, on: int) -> int:
        return self._L.es_hip_set_moe_gated(on)

    def set_batched32_direct(self, on: int) -> int:
        return self._L.es_hip_set_batched32_direct(on)

    def set_q6k_persistent(self, on: int) -> int:
        return self._L.es_hip_set_q6k_persistent(on)

    def set_direct_mfma_tok64(self, on: int) -> int:
        return self._L.es_hip_set_direct_mfma_tok64(on)

    def set_direct_persistent(self, on: int) -> int:
        return self._L.es_hip_set_direct_persistent(on)

    def _check(self, rc):
        if rc is not None and rc < 0:
            raise EsHipError(rc, self.last_error())
        return rc

    # ---- memory ----
    def matvec_q2_K(self, W: np.ndarray, cols: int, r0: int, r1: int, xq: np.ndarray, rows: int) -> np.ndarray:
        """es_matvec_q2_K's drop-in on host arrays: y[rows] with rows [r0, r1) written (the rest stay zero)"""
        y = np.zeros(rows, np.float32)
        self._L.es_hip_matvec_q2_K(np.ascontiguousarray(W).ctypes.data, cols, r0, r1, np.ascontiguousarray(xq).ctypes.data,
                                   y.ctypes.data)
        err = self.last_error()
        if err:
            raise EsHipError(-3, err)
        return y

    def host_array(self, shape, dtype) -> np.ndarray:
        """a numpy array over page-locked host memory (es_hip_host_alloc), freed when the array is collected"""
        dtype = np.dtype(dtype)
        n = int(np.prod(shape)) * dtype.itemsize
        p = self._L.es_hip_host_alloc(n)
        if not p:
            raise EsHipError(-4, self.last_error())
        buf = (C.c_uint8 * max(n, 1)).from_address(p)
        arr = np.frombuffer(buf, np.uint8, count=n).view(dtype).reshape(shape)
        weakref.finalize(arr, self._L.es_hip_host_free, p)
        return arr

    def alloc(self, nbytes: int) -> DevBuf:
        return DevBuf(self, nbytes)

    def upload(self, arr: np.ndarray) -> DevBuf:
        arr = np.ascontiguousarray(arr)
        buf = DevBuf(self, arr.nbytes)
        if arr.nbytes:
            self._check(self._L.es_hip_memcpy_h2d(buf.ptr, arr.ctypes.data, arr.nbytes))
        return buf

    def download(self, dev, out: np.ndarray, offset: int = 0) -> np.ndarray:
        assert out.flags.c_contiguous
        if out.nbytes:
            self._check(self._L.es_hip_memcpy_d2h(out.ctypes.data, int(dev) + offset, out.nbytes))
        return out

    def memset(self, dev, value: int, nbytes: int):
        self._check(self._L.es_hip_memset(int(dev), value, nbytes))

    def copy_d2d(self, dst, src, nbytes: int):
        self._check(self._L.es_hip_memcpy_d2d(int(dst), int(src), nbytes))

    def synchronize(self):
        self._check(self._L.es_hip_synchronize())

    # ---- device-pointer products ----
    def matvec_multi_dev(self, t, W, cols, r0, r1, act, astride, na, y, ystride, stream=None):
        self._check(self._L.es_hip_matvec_multi_dev(t, int(W), cols, r0, r1, int(act), astride, na, int(y), ystride, stream))

    def matvec_multi_dev_noalloc(self, t, W, cols, r0, r1, act, astride, na, y, ystride, stream=None):
        """es_hip_matvec_multi_dev with its tables and workspace in the library's static device scratch (no allocation)"""
        self._check(self._L.es_hip_matvec_multi_dev_noalloc(t, int(W), cols, r0, r1, int(act), astride, na, int(y), ystride,
                                                            stream))

    def dense_ffn_dev(self, tg, wg, tu, wu, td, wd, n, ff, N, x, xstride, gu, hq, out, ostride, stream=None):
        """dense_n on the device (es_hip_dense_ffn_dev); every pointer a device buffer"""
        self._check(self._L.es_hip_dense_ffn_dev(tg, int(wg), tu, int(wu), td, int(wd), n, ff, N, int(x), xstride, int(gu),
                                                 int(hq), int(out), ostride, stream))

    def matvec_dev(self, t, W, cols, r0, r1, act, y, stream=None):
        self._check(self._L.es_hip_matvec_dev(t, int(W), cols, r0, r1, int(act), int(y), stream))

    @staticmethod
    def make_jobs(specs) -> C.Array:
        """specs: iterable of dicts with type, rows, cols, W, act, astride, nb, y, ystride (device pointers as ints)"""
        specs = list(specs)
        arr = (Job * max(len(specs), 1))()
        for k, s in enumerate(specs):
            arr[k] = Job(s["type"], s["rows"], s["cols"], int(s["W"]), int(s["act"]), s.get("astride", 0), s.get("nb", 1),
                         int(s["y"]), s.get("ystride", 0))
        return arr, len(specs)

    def run_jobs(self, specs, stream=None):
        arr, n = self.make_jobs(specs)
        self._check(self._L.es_hip_run_jobs(arr, n, stream))

    def plan(self, specs) -> "Plan":
        arr, n = self.make_jobs(specs)
        p = self._L.es_hip_plan_create(arr, n)
        if not p:
            raise EsHipError(-2, self.last_error())
        return Plan(self, p)

    # ---- MoE expert FFN ----
    def moe_ffn(self, args: "MoeArgs", x, xstride, out, ostride, stream=None):
        self._check(self._L.es_hip_moe_ffn(*args.c_args(), int(x), xstride, int(out), ostride, stream))

    def moe_ffn_logits(self, args: "MoeArgs", N, logits, lstride, k, norm_topk, x, xstride, out, ostride, stream=None):
        """the MoE layer from device logits (es_hip_moe_ffn_logits); args' routing arrays are ignored. -> (sel, w) [N, k]"""
        sel = np.zeros((N, k), np.int32)
        w = np.zeros((N, k), np.float32)
        self._check(self._L.es_hip_moe_ffn_logits(C.byref(args.m), N, int(logits), lstride, k, int(norm_topk), int(x), xstride,
                                                  int(out), ostride, sel.ctypes.data, w.ctypes.data, stream))
        return sel, w

    def moe_plan(self, args: "MoeArgs", x, xstride, out, ostride) -> "Plan":
        h = self._L.es_hip_moe_plan_create(*args.c_args(), int(x), xstride, int(out), ostride)
        if not h:
            raise EsHipError(-2, self.last_error())
        return Plan(self, h, moe=True)

    def moe_ctx(self, args: "MoeArgs", max_tokens: int, k: int) -> "MoeCtx":
        """a device-routed MoE context for args' expert set (es_hip_moe_ctx_create); args' routing arrays are unused"""
        h = self._L.es_hip_moe_ctx_create(C.byref(args.m), max_tokens, k)
        if not h:
            raise EsHipError(-2, self.last_error())
        return MoeCtx(self, h, args)

    def step_time_ms(self, plans, moe_plans, warmup: int, iters: int, stream=None) -> float:
        """ms per iteration of: every plan in `plans`, then every MoE plan in `moe_plans`, timed with HIP events"""
        P = (C.c_void_p * max(len(plans), 1))(*[p.h for p in plans])
        M = (C.c_void_p * max(len(moe_plans), 1))(*[p.h for p in moe_plans])
        ms = self._L.es_hip_step_time_ms(P, len(plans), M, len(moe_plans), warmup, iters, stream)
        if ms < 0:
            raise EsHipError(-3, self.last_error())
        return ms

    def swiglu_dev(self, g, u, h, n, stream=None):
        self._check(self._L.es_hip_swiglu_dev(int(g), int(u), int(h), n, stream))

    def dequant_row_dev(self, t, src, dst, n, stream=None):
        self._check(self._L.es_hip_dequant_row_dev(t, int(src), int(dst), n, stream))

    def matvec_float_dev(self, t, W, cols, r0, r1, x, xstride, na, y, ystride, stream=None):
        self._check(self._L.es_hip_matvec_float_dev(t, int(W), cols, r0, r1, int(x), xstride, na, int(y), ystride, stream))

    def route_softmax_dev(self, logits, lstride, ntok, n_exp, k, norm_topk, sel, w, kmax, stream=None):
        self._check(self._L.es_hip_route_softmax_dev(int(logits), lstride, ntok, n_exp, k, int(norm_topk), int(sel), int(w),
                                                     kmax, stream))

    # ---- activation preparation on the device (device pointers as DevBuf / ints; None for an output not wanted) ----
    @staticmethod
    def _ptr(b):
        return None if b is None else int(b)

    def act_prepare_dev(self, x, xstride, rows, cols, q80, q80_stride, q8k, q8k_stride, stream=None):
        self._check(self._L.es_hip_act_prepare_dev(int(x), xstride, rows, cols, self._ptr(q80), q80_stride, self._ptr(q8k),
                                                   q8k_stride, stream))

    def rmsnorm_prepare_dev(self, x, xstride, w, eps, rows, cols, xn, xn_stride, q80, q80_stride, q8k, q8k_stride,
                            stream=None):
        self._check(self._L.es_hip_rmsnorm_prepare_dev(int(x), xstride, self._ptr(w), eps, rows, cols, self._ptr(xn),
                                                       xn_stride, self._ptr(q80), q80_stride, self._ptr(q8k), q8k_stride,
                                                       stream))

    def swiglu_prepare_dev(self, gu, gu_stride, rows, ff, h, h_stride, q80, q80_stride, q8k, q8k_stride, stream=None):
        self._check(self._L.es_hip_swiglu_prepare_dev(int(gu), gu_stride, rows, ff, self._ptr(h), h_stride, self._ptr(q80),
                                                      q80_stride, self._ptr(q8k), q8k_stride, stream))

    def block_ints_dev(self, t, W, cols, rows, act):
        nb = cols // BLOCK_ELEMS[t]
        d = self.alloc(rows * nb * 4)
        a = self.alloc(rows * nb * 4)
        self._check(self._L.es_hip_block_ints_dev(t, int(W), cols, rows, int(act), d.ptr, a.ptr, None))
        dots = self.download(d, np.zeros((rows, nb), np.int32))
        aux = self.download(a, np.zeros((rows, nb), np.int32))
        return dots, aux

    # ---- host-memory convenience (uploads, computes, downloads) ----
    def matvec_multi(self, t, W: np.ndarray, cols: int, rows: int, acts: np.ndarray, r0: int = 0, r1: int | None = None):
        """acts: [na, nblocks] activation blocks (any structured dtype of the right size) -> y [na, rows] fp32;
        rows outside [r0, r1) stay zero"""
        r1 = rows if r1 is None else r1
        acts = np.ascontiguousarray(acts)
        na = acts.shape[0]
        dW, dA = self.upload(W), self.upload(acts)
        dY = self.alloc(na * rows * 4)
        self.memset(dY, 0, na * rows * 4)
        self.matvec_multi_dev(t, dW, cols, r0, r1, dA, acts.strides[0] if na > 1 else 0, na, dY, rows)
        y = self.download(dY, np.zeros((na, rows), np.float32))
        for b in (dW, dA, dY):
            b.close()
        return y

    # ---- the reference prototypes on host memory ----
    def register(self, W: np.ndarray):
        self._check(self._L.es_hip_register(W.ctypes.data, W.nbytes))

    def update(self, W: np.ndarray):
        self._check(self._L.es_hip_update(W.ctypes.data))

    def unregister(self, W: np.ndarray):
        return self._L.es_hip_unregister(W.ctypes.data)

    def host_matvec_multi(self, t, W: np.ndarray, cols: int, r0: int, r1: int, acts, y: np.ndarray, x=None, floats=()):
        """es_hip_matvec_multi with es_act records pointing at `acts` [na, nblocks] (and at x [na, cols] fp32, if given);
        the activations in `floats` (all when acts is None) carry no blocks; y [na, ystride] updated in place"""
        acts = None if acts is None else np.ascontiguousarray(acts)
        x = None if x is None else np.ascontiguousarray(x, np.float32)
        recs = act_records(t, acts, cols, x, floats)
        na = acts.shape[0] if acts is not None else x.shape[0]
        if na == 1:
            self._L.es_hip_matvec(t, W.ctypes.data, cols, r0, r1, recs, y.ctypes.data, None)
        else:
            self._L.es_hip_matvec_multi(t, W.ctypes.data, cols, r0, r1, recs, na, y.ctypes.data, y.strides[0] // 4, None)
        err = self.last_error()   # the void drop-ins clear it on entry
        if err:
            raise EsHipError(-1, err)
        return y

    @staticmethod
    def host_jobs(jobs):
        """(es_hip_host_job array, keep-alive list) for jobs: list of (type, W host uint8, rows, cols, acts [nb, nblocks],
        y [nb, ys] float32 written in place), each optionally extended by (x [nb, cols] fp32, floats): the activations
        listed in floats carry no blocks (float path)"""
        arr = (HostJob * max(len(jobs), 1))()
        keep = [arr]
        for k, job in enumerate(jobs):
            t, W, rows, cols, acts, y = job[:6]
            x, floats = (job[6], job[7]) if len(job) > 6 else (None, ())
            acts = None if acts is None else np.ascontiguousarray(acts)
            x = None if x is None else np.ascontiguousarray(x, np.float32)
            recs = act_records(t, acts, cols, x, floats)
            keep += [acts, x, recs]
            nb = acts.shape[0] if acts is not None else x.shape[0]
            arr[k] = HostJob(t, W.ctypes.data, rows, cols, C.cast(recs, C.c_void_p), y.ctypes.data, nb, y.strides[0] // 4)
        return arr, keep

    def run_jobs_host(self, jobs):
        """es_hip_run_jobs_host over host_jobs(jobs)"""
        arr, keep = self.host_jobs(jobs)
        self._check(self._L.es_hip_run_jobs_host(arr, len(jobs)))
        del keep


class MoeArgs:
    """es_hip_moe plus the routing arrays, kept alive for the C call. experts: dicts of gate/up/down device pointers
    (None for experts never routed); k: [N] ints; sel, w: [N, kmax]."""

    def __init__(self, gate_type, up_type, down_type, n, ff, experts, k, sel, w):
        ne = len(experts)
        P = C.c_void_p * max(ne, 1)
        self.g = P(*[int(e["gate"]) if e else None for e in experts])
        self.u = P(*[int(e["up"]) if e else None for e in experts])
        self.d = P(*[int(e["down"]) if e else None for e in experts])
        self.m = Moe(gate_type, up_type, down_type, n, ff, ne, C.cast(self.g, C.c_void_p), C.cast(self.u, C.c_void_p),
                     C.cast(self.d, C.c_void_p))
        self.k = np.ascontiguousarray(k, np.int32)
        self.sel = np.ascontiguousarray(sel, np.int32)
        self.w = np.ascontiguousarray(w, np.float32)
        self.N, self.kmax = int(self.k.shape[0]), int(self.sel.shape[1]) if self.sel.ndim == 2 else 1

    def c_args(self):
        return (C.byref(self.m), self.N, self.k.ctypes.data, self.sel.ctypes.data, self.w.ctypes.data, self.kmax)



class MoeCtx:
    """es_hip_moe_ctx: run(N, sel, w, x, xstride, out, ostride) with device routing arrays, or run_logits(...)"""

    def __init__(self, lib: Lib, handle, args):
        self.lib, self.h, self.args = lib, handle, args   # args keeps the expert pointer arrays alive

    def run(self, N, sel, w, x, xstride, out, ostride, stream=None):
        self.lib._check(self.lib._L.es_hip_moe_ctx_run(self.h, N, int(sel), int(w), int(x), xstride, int(out), ostride, stream))

    def run_logits(self, N, logits, lstride, norm_topk, x, xstride, out, ostride, sel_out=None, w_out=None, stream=None):
        L = self.lib
        L._check(L._L.es_hip_moe_ctx_run_logits(self.h, N, int(logits), lstride, int(norm_topk), int(x), xstride, int(out),
                                                ostride, L._ptr(sel_out), L._ptr(w_out), stream))

    def close(self):
        if self.h:
            self.lib._L.es_hip_moe_ctx_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()


class Plan:
    def __init__(self, lib: Lib, handle, moe: bool = False):
        self.lib, self.h = lib, handle
        p = "es_hip_moe_plan_" if moe else "es_hip_plan_"
        self.moe = moe
        self._run, self._destroy = getattr(lib._L, p + "run"), getattr(lib._L, p + "destroy")

    def run(self, stream=None):
        self.lib._check(self._run(self.h, stream))

    def time_ms(self, warmup: int, iters: int, stream=None) -> float:
        return self.lib.step_time_ms([] if self.moe else [self], [self] if self.moe else [], warmup, iters, stream)

    def close(self):
        if self.h:
            self._destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
