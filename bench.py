#!/usr/bin/env python3
"""Benchmark of the quantized matrix-product path on one MI355X.

Headline (decode form): Q4_K matvec at T=1 over the Llama-3.2-1B FFN shapes (gate and up
8192x2048, down 2048x8192), 38 layer copies = 1.08 GB of packed weights in HBM, rotated so every step streams from HBM rather
than the 256 MB Infinity Cache. One step = one launch of a prepared job batch (the engine's run_jobs) over all 114
matrices. value = weight bytes / step time, the reference's "weight GB/s" (tools/es_fmtbench.c:40, tools/es_kbench.c:294).

Also reported: config 2's prefill form (T=512, int8 TOPS = 2*T*rows*cols / time), configs 1 and 3, the MoE layers of
configs 4 and 5 (weight GB/s over the experts actually routed, plus config 5's attention products), the kernel's roofline
(achieved vs 8 TB/s, kernel time from HIP events on the launch stream) and the reference's CPU kernels timed on this host
(cpu_baseline: the reference's es_matvec_multi built from its sources, oracle/_ref, driven es_kbench-style).

Inputs are synthetic: es_mtest-style random weight blocks with sane fp16 scales (tools/es_mtest.c:9-35) and N(0,1)
activations quantized to the reference's Q8 blocks in numpy. Kernel speed does not depend on the values.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only WORKLOAD]
"""
import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "stream-_amd"))
import es_hip_quant as E  # noqa: E402

METRIC = "decode matvec weight GB/s (% HBM peak); prefill int8 TOPS (% MFMA peak)"
HBM_PEAK_GBS = 8000.0
INT8_PEAK_TOPS = 5000.0

Q80 = np.dtype([("d", "<f4"), ("qs", "i1", (32,))])
Q8K = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
SETTLE_S = 0.3   # untimed runs before each workload's warmup steps: the GPU leaves its idle clocks
SCALE_POS = {E.Q4_0: (0, None), E.Q5_0: (0, None), E.Q8_0: (0, None), E.Q4_K: (0, 2), E.Q5_K: (0, 2), E.Q6_K: (208, None),
             E.Q3_K: (108, None), E.Q2_K: (80, 82)}


def random_blocks(t, rows, cols, rng):
    """random block bytes with sane fp16 scales, the es_mtest recipe (tools/es_mtest.c:30-35)"""
    nb, bb = cols // E.BLOCK_ELEMS[t], E.BLOCK_BYTES[t]
    W = rng.integers(0, 256, (rows, nb, bb), dtype=np.uint8)
    dp, mp = SCALE_POS[t]
    W[:, :, dp:dp + 2] = (0.001 + rng.integers(0, 1000, (rows, nb)) / 1e5).astype(np.float16)[..., None].view(np.uint8)
    if mp is not None:
        W[:, :, mp:mp + 2] = (0.0005 + rng.integers(0, 1000, (rows, nb)) / 1e5).astype(np.float16)[..., None].view(np.uint8)
    return W.reshape(-1)


def quantize_acts(t, x):
    """fp32 [n, cols] -> the reference's activation blocks [n, nblocks] (Q8_K for K-quants, Q8_0 otherwise)"""
    n, cols = x.shape
    if E.BLOCK_ELEMS[t] == 256:
        xb = x.reshape(n, cols // 256, 256)
        amax = np.abs(xb).max(axis=2)
        q = np.clip(np.rint(xb * (127.0 / np.maximum(amax, 1e-30))[..., None]), -127, 127).astype(np.int8)
        out = np.zeros((n, cols // 256), Q8K)
        out["d"] = amax / 127.0
        out["qs"] = q
        out["bsums"] = q.reshape(n, cols // 256, 16, 16).astype(np.int32).sum(axis=3)
        return out
    xb = x.reshape(n, cols // 32, 32)
    d = np.abs(xb).max(axis=2) / 127.0
    v = xb * np.where(d > 0, 1.0 / np.maximum(d, 1e-30), 0.0)[..., None]
    out = np.zeros((n, cols // 32), Q80)
    out["d"] = d
    out["qs"] = np.trunc(np.where(v < 0, v - 0.5, v + 0.5)).astype(np.int8)
    return out


class Workload:
    """A rotating set of `copies` copies of some matrices, all against the same activations, as one prepared batch."""

    def __init__(self, lib, rng, mats, na, copies):
        self.lib, self.keep, specs = lib, [], []
        self.weight_bytes = 0
        self.ops = 0
        for (t, rows, cols) in mats:
            W = random_blocks(t, rows, cols, rng)
            acts = quantize_acts(t, rng.standard_normal((na, cols)).astype(np.float32))
            dA = lib.upload(acts)
            dW = lib.alloc(W.nbytes * copies)
            src = lib.upload(W)
            for c in range(copies):
                lib.copy_d2d(dW.offset(c * W.nbytes), src, W.nbytes)
            src.close()
            dY = lib.alloc(4 * na * rows * copies)
            self.keep += [dA, dW, dY]
            for c in range(copies):
                specs.append(dict(type=t, rows=rows, cols=cols, W=dW.offset(c * W.nbytes), act=dA,
                                  astride=acts.strides[0], nb=na, y=dY.offset(4 * na * rows * c), ystride=rows))
                self.weight_bytes += W.nbytes
                self.ops += 2 * na * rows * cols
        self.plan = lib.plan(specs)
        self.launches_per_step = len(self.plan_groups(mats))

    @staticmethod
    def plan_groups(mats):
        return {m[0] for m in mats}   # one launch per format

    def time(self, warmup, steps):
        """(wall ms per step, event ms per step): events on the launch stream around `steps` back-to-back runs, after
        SETTLE_S seconds of untimed runs (so the clocks have left idle) and `warmup` more"""
        t_end = time.perf_counter() + SETTLE_S
        while time.perf_counter() < t_end:
            for _ in range(10):
                self.plan.run()
            self.lib.synchronize()
        for _ in range(warmup):
            self.plan.run()
        self.lib.synchronize()
        t0 = time.perf_counter()
        ev = self.plan.time_ms(0, steps)
        self.lib.synchronize()
        wall = (time.perf_counter() - t0) * 1e3 / steps
        return wall, ev

    def close(self):
        self.plan.close()
        for b in self.keep:
            b.close()


def route_topk(rng, n_tok, n_exp, k, norm_topk, with_logits=False):
    """synthetic routing: softmax over N(0,1) logits, the k largest probabilities (route(), src/es_engine.c:744-835)"""
    logits = rng.standard_normal((n_tok, n_exp)).astype(np.float32)
    p = np.exp(logits - logits.max(axis=1, keepdims=True))
    p /= p.sum(axis=1, keepdims=True)
    sel = np.argsort(-p, axis=1, kind="stable")[:, :k].astype(np.int32)
    w = np.take_along_axis(p, sel, axis=1).astype(np.float32)
    if norm_topk:
        w /= w.sum(axis=1, keepdims=True)
    return (sel, w, logits) if with_logits else (sel, w)


def moe_rng(config):
    """each MoE workload's own generator: the same routing (and so the same experts and counts, which move the layer time
    by over 10%) whether the workload runs alone (--only) or after the others"""
    return np.random.default_rng(20260100 + config)


class MoeWorkload:
    """`copies` copies of one MoE layer (experts in device memory) with one routing of N tokens, one MoE plan per copy, and
    optionally the attention products of the same tokens (one job-batch plan per copy). A step runs every copy once."""

    def __init__(self, lib, rng, types, n, ff, n_exp, k, n_tok, norm_topk, copies, attn=()):
        self.lib, self.keep, self.plans, self.moe, self.ctx_args = lib, [], [], [], []
        self.n_tok, self.n_exp, self.n, self.norm = n_tok, n_exp, n, norm_topk
        gt, ut, dt = types
        sel, w, plan_logits = route_topk(rng, n_tok, n_exp, k, norm_topk, with_logits=True)
        used = sorted(set(sel.reshape(-1).tolist()))
        eb = [E.row_bytes(gt, n) * ff, E.row_bytes(ut, n) * ff, E.row_bytes(dt, ff) * n]
        self.weight_bytes = copies * len(used) * sum(eb)
        one = [random_blocks(gt, ff, n, rng), random_blocks(ut, ff, n, rng), random_blocks(dt, n, ff, rng)]
        x = quantize_acts(gt, rng.standard_normal((n_tok, n)).astype(np.float32))
        dx = lib.upload(x)
        self.keep.append(dx)
        self.dx, self.xstride = dx, x.strides[0]
        # router logits for the device-routed leg: a fresh routing every step (8 sets in rotation), or the logits of the
        # plan's own routing (the same experts and counts as the plan, routed again on the device every step)
        self.logits = [lib.upload(rng.standard_normal((n_tok, n_exp)).astype(np.float32)) for _ in range(8)]
        self.plan_logits = lib.upload(plan_logits)
        self.keep += self.logits + [self.plan_logits]
        xa = quantize_acts(E.Q5_0, rng.standard_normal((n_tok, n)).astype(np.float32)) if attn else None
        dxa = lib.upload(xa) if attn else None
        for c in range(copies):
            dev = lib.alloc(n_exp * sum(eb))
            self.keep.append(dev)
            srcs = [lib.upload(m) for m in one]
            experts = []
            for e in range(n_exp):
                base = e * sum(eb)
                ptrs = {}
                for m, (name, nb) in enumerate(zip(("gate", "up", "down"), eb)):
                    lib.copy_d2d(dev.offset(base), srcs[m], nb)   # every expert its own copy of the bytes
                    ptrs[name] = dev.offset(base)
                    base += nb
                experts.append(ptrs)
            for b in srcs:
                b.close()
            out = lib.alloc(n_tok * n * 4)
            self.keep.append(out)
            args = E.MoeArgs(gt, ut, dt, n, ff, experts, np.full(n_tok, k), sel, w)
            self.moe.append(lib.moe_plan(args, dx, x.strides[0], out, n))
            self.ctx_args.append((lib.moe_ctx(args, n_tok, k), out))
            if attn:
                specs = []
                for (rows, cols) in attn:
                    Wa = lib.upload(random_blocks(E.Q5_0, rows, cols, rng))
                    ya = lib.alloc(n_tok * rows * 4)
                    self.keep += [Wa, ya]
                    specs.append(dict(type=E.Q5_0, rows=rows, cols=cols, W=Wa, act=dxa, astride=xa.strides[0], nb=n_tok,
                                      y=ya, ystride=rows))
                    self.weight_bytes += E.row_bytes(E.Q5_0, cols) * rows
                self.plans.append(lib.plan(specs))
        if attn:
            self.keep.append(dxa)
        self.copies, self.distinct = copies, len(used)

    def time(self, warmup, steps):
        """ms per copy (one layer), after SETTLE_S seconds of untimed steps"""
        t_end = time.perf_counter() + SETTLE_S
        while time.perf_counter() < t_end:
            self.lib.step_time_ms(self.plans, self.moe, 0, 2)
        return self.lib.step_time_ms(self.plans, self.moe, warmup, steps) / self.copies

    def time_device_routed(self, warmup, steps, same_routing=False):
        """ms per copy (one layer) with the routing computed on the device from fresh logits every step (same_routing:
        from the logits of the plan's routing, so the layer reads the same experts as time()) and the layer run through
        its context (es_hip_moe_ctx_run_logits: grouping and job tables on the device, no host round trip), the attention
        plans as in time(); HIP events on the null stream around `steps` steps"""
        it = [0]

        def step():
            for i, (ctx, out) in enumerate(self.ctx_args):
                if self.plans:
                    self.plans[i].run()
                lg = self.plan_logits if same_routing else self.logits[it[0] % len(self.logits)]
                ctx.run_logits(self.n_tok, lg, 0, self.norm, self.dx, self.xstride, out, self.n)
            it[0] += 1

        t_end = time.perf_counter() + SETTLE_S
        while time.perf_counter() < t_end:
            step()
            self.lib.synchronize()
        return HipEvents().time_ms(step, warmup, steps) / self.copies

    def close(self):
        for p in self.plans + self.moe:
            p.close()
        for ctx, _ in self.ctx_args:
            ctx.close()
        for b in self.keep:
            b.close()


class CpuRef:
    """The reference's es_matvec_multi (oracle/_ref/libesref_clang.so, built from its sources) or, where that build is
    absent, the oracle's restatement, timed es_kbench-style on this host: pinned threads taking 16-row chunks of a rotating
    set of matrices, activations in the engine's batches of at most 64 (src/es_engine.c:43, 152-171)."""

    def __init__(self):
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import oracle as O

        self.orc = O.Oracle()
        if O.ref_available("clang"):
            self.ref = O.RefLib("clang")
            self.fn, self.kind = self.orc.reference_fn_ptr(self.ref), "reference"
        else:
            self.fn, self.kind = self.orc.multi_fn_ptr(), "port"
        avail = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
        self.avail, self.allc = avail, max(1, min(16, avail))
        self.threads = sorted({1, min(8, self.allc), self.allc})

    def seconds(self, t, rows, cols, na, rng, seconds, nt, min_bytes=288 << 20):
        """seconds per pass of one matrix against na activations at nt threads (the rotating set at least min_bytes)"""
        W1 = random_blocks(t, rows, cols, rng)
        nmat = max(1, min_bytes // W1.nbytes + (1 if min_bytes else 0))
        W = np.tile(W1, nmat) if nmat > 1 else W1
        acts = quantize_acts(t, rng.standard_normal((na, cols)).astype(np.float32))
        sec, _, _ = self.orc.cpu_bench(self.fn, t, W, W1.nbytes, nmat, rows, cols, acts, nt, seconds)
        return sec / nmat, W1.nbytes

    def point(self, t, rows, cols, na, rng, seconds, min_bytes=288 << 20):
        """{threads: (weight GB/s, TOPS)} for one matrix shape"""
        out = {}
        for nt in self.threads:
            sec, wb = self.seconds(t, rows, cols, na, rng, seconds, nt, min_bytes)
            out[nt] = (wb / sec / 1e9, 2.0 * na * rows * cols / sec / 1e12)
        return out

    def record(self, pts, unit, sample):
        k = 0 if unit == "GB/s" else 1
        return {"value": round(pts[self.allc][k], 3), "unit": unit, "cores": self.allc, "kind": self.kind, "sample": sample,
                "by_threads": {str(n): round(v[k], 3) for n, v in pts.items()}, "host_cpus_visible": self.avail}


def cpu_baseline(rng, seconds):
    """the headline's CPU figure: config 2 decode (Q4_K 8192x2048, T=1) in weight GB/s"""
    c = CpuRef()
    pts = c.point(E.Q4_K, 8192, 2048, 1, rng, seconds)
    return c.record(pts, "GB/s", f"Q4_K 8192x2048 matvec (T=1), rotating set >= 288 MiB, >= {seconds:.1f} s per point, "
                                 "16-row chunks (src/es_engine.c:152-171)")


def cpu_configs(rng, seconds):
    """the other configurations' CPU figures (the reference's kernels on this host), each a bounded sample"""
    c = CpuRef()
    out = {}
    pts = c.point(E.Q4_0, 4864, 896, 1, rng, seconds)
    out["config1_q4_0_decode"] = c.record(pts, "GB/s", "Q4_0 4864x896 matvec (T=1), rotating set >= 288 MiB")
    pts = c.point(E.Q4_K, 8192, 2048, 512, rng, seconds, min_bytes=0)
    out["prefill"] = c.record(pts, "TOPS", "Q4_K 8192x2048 against 512 activations (gate/up shape), batches of 64, 16-row "
                                           "chunks; int8 TOPS = 2 x 512 x rows x cols / time")
    for b in (1, 64):
        pts = c.point(E.Q6_K, 151936, 1024, b, rng, seconds, min_bytes=(288 << 20) if b == 1 else 0)
        out[f"config3_q6_k_head_b{b}"] = c.record(pts, "GB/s", f"Q6_K 151936x1024 head against {b} activation(s)")
    # MoE layers through moe_n's job pattern (src/es_engine.c:871-918): per distinct expert, gate and up against the
    # tokens routed to it, then down; the per-expert products are timed at the mean tokens per expert, over a rotating
    # set of expert matrices
    for name, (cfg, t3, n, ff, n_exp, k, n_tok, norm) in {
            "config4_q2_k_moe": (4, (E.Q2_K, E.Q2_K, E.Q2_K), 2048, 1024, 64, 8, 128, False),
            "config5_mixed_moe_decode": (5, (E.Q4_K, E.Q4_K, E.Q6_K), 2048, 768, 128, 8, 32, True)}.items():
        # the same synthetic routing as the device legs: their generator's first draw (MoeWorkload routes first)
        sel, _ = route_topk(moe_rng(cfg), n_tok, n_exp, k, norm)
        used = len(set(sel.reshape(-1).tolist()))
        per = max(1, round(n_tok * k / used))
        pts, ms = {}, {}
        for nt in c.threads:
            sg, bg = c.seconds(t3[0], ff, n, per, rng, seconds, nt)
            su, bu = c.seconds(t3[1], ff, n, per, rng, seconds, nt)
            sd, bd = c.seconds(t3[2], n, ff, per, rng, seconds, nt)
            layer = used * (sg + su + sd)
            ms[nt] = layer * 1e3
            pts[nt] = (used * (bg + bu + bd) / layer / 1e9, 2.0 * used * per * 3 * n * ff / layer / 1e12)
        rec = c.record(pts, "GB/s", f"{used} experts x (gate, up {ff}x{n}, down {n}x{ff}) at {per} tokens each "
                                    f"({n_tok} tokens top-{k}); expert bytes / layer time")
        rec["ms_per_layer"] = round(ms[c.allc], 4)
        out[name] = rec
    return out


Q4K_FFN = [(E.Q4_K, 8192, 2048), (E.Q4_K, 8192, 2048), (E.Q4_K, 2048, 8192)]


class HipEvents:
    """HIP events on the null stream (the one the activation-preparation calls below launch on), through the HIP runtime
    the library itself loaded"""

    def __init__(self):
        import ctypes
        self.C = ctypes
        self.h = ctypes.CDLL("libamdhip64.so")

    def time_ms(self, fn, warmup, iters):
        C, h = self.C, self.h
        for _ in range(warmup):
            fn()
        a, b = C.c_void_p(), C.c_void_p()
        if h.hipEventCreate(C.byref(a)) or h.hipEventCreate(C.byref(b)):
            raise RuntimeError("hipEventCreate failed")
        h.hipEventRecord(a, None)
        for _ in range(iters):
            fn()
        h.hipEventRecord(b, None)
        h.hipEventSynchronize(b)
        ms = C.c_float()
        h.hipEventElapsedTime(C.byref(ms), a, b)
        h.hipEventDestroy(a)
        h.hipEventDestroy(b)
        return ms.value / iters


def cache_load_rate(lib, rng, K, Wm, pinned=False):
    """Expert loads through the device expert cache (es_hip_cache_acquire) at config 5's expert size: gate/up Q4_K 768x2048
    and down Q6_K 2048x768 (3,059,712 bytes), from pageable host slabs of 64 experts, 16 slots. Every call takes 8 experts
    that are not cached (the cycle through 64 experts with 16 slots always misses), so each call copies 8 experts host ->
    HBM and evicts 8, and waits for its copies as load_experts does. Host-to-device bound (PCIe), not an HBM figure.
    pinned: the slabs in page-locked memory (es_hip_host_alloc), else pageable numpy arrays."""
    ne, nslots, k = 64, 16, 8
    parts = [768 * 8 * 144, 768 * 8 * 144, 2048 * 3 * 210]
    slabs = [rng.integers(0, 256, (ne, b), dtype=np.uint8) for b in parts]
    if pinned:   # the same bytes in page-locked memory (es_hip_host_alloc)
        pinned_slabs = []
        for s in slabs:
            h = lib.host_array(s.shape, np.uint8)
            h[...] = s
            pinned_slabs.append(h)
        slabs = pinned_slabs
    src = E.ExpertSrc()
    off = 0
    for r in range(3):
        src.base[r], src.stride[r], src.bytes[r], src.offset[r] = slabs[r].ctypes.data, parts[r], parts[r], off
        off += parts[r]
    c = E.ExpertCache(lib, nslots, off, 1, ne, 1.0)
    calls = [np.arange(k * i, k * i + k) % ne for i in range(Wm + K)]

    def step(sel):   # load_experts: the experts of the call, then a wait for their copies (gio_wait)
        for s in c.acquire(0, sel, src):
            c.wait(int(s))

    for sel in calls[:Wm]:
        step(sel)
    lib.synchronize()
    t0 = time.perf_counter()
    for sel in calls[Wm:]:
        step(sel)
    lib.synchronize()
    dt = (time.perf_counter() - t0) / K
    st = c.stats()
    c.close()
    return {"expert_bytes": off, "experts_per_call": k, "ms_per_call": round(dt * 1e3, 4),
            "gbs": round(k * off / dt / 1e9, 2), "misses": st.misses, "evictions": st.evictions}


def act_prep_times(lib, rng, K, Wm):
    """Device activation preparation at config 2's prefill shapes (T = 512): rmsnorm + Q8_K/Q8_0 of the 2048-wide layer
    input, SwiGLU + Q8_K of the dense FFN's 8192-wide gate|up rows, and the plain Q8_K/Q8_0 quantizers. us per call
    (HIP events around K back-to-back calls) and GB/s over the fp32 bytes read plus the block bytes written."""
    T, n, ff = 512, 2048, 8192
    ev = HipEvents()
    x = rng.standard_normal((T, n)).astype(np.float32)
    w = (1.0 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    gu = rng.standard_normal((T, 2 * ff)).astype(np.float32)
    dx, dw, dgu = lib.upload(x), lib.upload(w), lib.upload(gu)
    b80, b8k, h8k = lib.alloc(T * (n // 32) * 36), lib.alloc(T * (n // 256) * 292), lib.alloc(T * (ff // 256) * 292)
    out = {}

    def rec(name, fn, nbytes):
        ms = ev.time_ms(fn, Wm, K)
        out[name] = {"us": round(ms * 1e3, 2), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 1), "bytes": nbytes}

    blocks = T * ((n // 32) * 36 + (n // 256) * 292)
    rec("rmsnorm_q8k_q80_512x2048", lambda: lib.rmsnorm_prepare_dev(dx, 0, dw, 1e-5, T, n, None, 0, b80, 0, b8k, 0),
        x.nbytes + w.nbytes + blocks)
    rec("plain_q8k_q80_512x2048", lambda: lib.act_prepare_dev(dx, 0, T, n, b80, 0, b8k, 0), x.nbytes + blocks)
    rec("swiglu_q8k_512x8192", lambda: lib.swiglu_prepare_dev(dgu, 0, T, ff, None, 0, None, 0, h8k, 0),
        gu.nbytes + T * (ff // 256) * 292)
    for buf in (dx, dw, dgu, b80, b8k, h8k):
        buf.close()
    return out


def dense_ffn_time(lib, rng, K, Wm, T=512, n=2048, ff=8192):
    """dense_n on the device (es_hip_dense_ffn_dev) at config 2's prefill shape: gate/up Q4_K ff x n into [T][2 ff], SwiGLU
    + Q8_K of h, down Q4_K n x ff. us per layer (HIP events on the null stream around K calls) and int8 TOPS over the three
    products."""
    t = E.Q4_K
    W = [random_blocks(t, ff, n, rng), random_blocks(t, ff, n, rng), random_blocks(t, n, ff, rng)]
    x = quantize_acts(t, rng.standard_normal((T, n)).astype(np.float32))
    d = [lib.upload(a) for a in W + [x]]
    gu, hq, out = lib.alloc(T * 2 * ff * 4), lib.alloc(T * (ff // 256) * 292), lib.alloc(T * n * 4)
    fn = lambda: lib.dense_ffn_dev(t, d[0], t, d[1], t, d[2], n, ff, T, d[3], x.strides[0], gu, hq, out, n)
    t_end = time.perf_counter() + SETTLE_S
    while time.perf_counter() < t_end:
        fn()
        lib.synchronize()
    ms = HipEvents().time_ms(fn, Wm, K)
    for b in d + [gu, hq, out]:
        b.close()
    ops = 2 * T * 3 * n * ff
    return {"us": round(ms * 1e3, 2), "tops": round(ops / (ms * 1e-3) / 1e12, 2),
            "frac": round(ops / (ms * 1e-3) / 1e12 / INT8_PEAK_TOPS, 4),
            "workload": f"dense_n T={T}: gate/up {ff}x{n} + SwiGLU/Q8_K + down {n}x{ff}, Q4_K, three dependent steps"}


def host_queue_time(lib, rng, K, Wm, T):
    """es_hip_run_jobs_host, the engine-facing binding (run_jobs over host buffers, src/es_engine.c:177-186), at config 2's
    FFN shapes: the engine's two queues per layer around SwiGLU, gate + up (Q4_K 8192x2048) in one call and down (Q4_K
    2048x8192) in a second, weights registered (resident in HBM, as es_hip_register keeps them), activation blocks and
    outputs in host memory. Each call is synchronous: activations up, launches, outputs down. ms per layer by the wall
    clock over K layers, and the PCIe bytes moved per layer (activation blocks up, fp32 outputs down)."""
    t, n, ff = E.Q4_K, 2048, 8192
    W = [random_blocks(t, ff, n, rng), random_blocks(t, ff, n, rng), random_blocks(t, n, ff, rng)]
    for w in W:
        lib.register(w)
    x = quantize_acts(t, rng.standard_normal((T, n)).astype(np.float32))
    h = quantize_acts(t, rng.standard_normal((T, ff)).astype(np.float32))
    gu = np.zeros((T, 2 * ff), np.float32)
    out = np.zeros((T, n), np.float32)
    q1, k1 = lib.host_jobs([(t, W[0], ff, n, x, gu[:, :ff]), (t, W[1], ff, n, x, gu[:, ff:])])
    q2, k2 = lib.host_jobs([(t, W[2], n, ff, h, out)])
    run = lib._L.es_hip_run_jobs_host

    def layer():
        if run(q1, 2) or run(q2, 1):
            raise RuntimeError("es_hip_run_jobs_host: " + lib.last_error())

    for _ in range(Wm):
        layer()
    t0 = time.perf_counter()
    for _ in range(K):
        layer()
    dt = (time.perf_counter() - t0) / K
    for w in W:
        lib.unregister(w)
    del k1, k2
    pcie = x.nbytes + h.nbytes + gu.nbytes + out.nbytes
    wbytes = sum(w.nbytes for w in W)
    return {"ms_per_layer": round(dt * 1e3, 4), "pcie_bytes_per_layer": pcie,
            "pcie_gbs": round(pcie / dt / 1e9, 2), "weight_gbs": round(wbytes / dt / 1e9, 1),
            "workload": f"run_jobs_host T={T}: [gate, up] then [down], Q4_K, registered weights, host activations/outputs"}


def only(lib, rng, name, K, Wm, moe_leg="both"):
    """one workload of the bench, alone: the command profiler summaries are taken from"""
    if name == "copy":   # a plain device copy of known size, the reference for HBM byte counters
        n = 1 << 30
        a, b = lib.alloc(n), lib.alloc(n)
        lib.memset(a, 1, n)
        for _ in range(Wm + K):
            lib.copy_d2d(b, a, n)
        lib.synchronize()
        a.close()
        b.close()
        return {"workload": "copy", "bytes_read_per_copy": n, "bytes_written_per_copy": n, "copies": Wm + K}
    if name == "act":
        return {"workload": "act", **act_prep_times(lib, rng, K, Wm)}
    if name == "dense":
        return {"workload": "dense", **dense_ffn_time(lib, rng, K, Wm)}
    if name == "host_queue":
        return {"workload": "host_queue", "t1": host_queue_time(lib, rng, K, Wm, 1),
                "t512": host_queue_time(lib, rng, max(3, K // 4), Wm, 512)}
    if name == "cache":
        return {"workload": "cache", "pageable": cache_load_rate(lib, rng, K, Wm),
                "pinned": cache_load_rate(lib, rng, K, Wm, pinned=True)}
    if name in ("config4", "config5"):
        w = (MoeWorkload(lib, moe_rng(4), (E.Q2_K, E.Q2_K, E.Q2_K), 2048, 1024, 64, 8, 128, False, 8) if name == "config4" else
             MoeWorkload(lib, moe_rng(5), (E.Q4_K, E.Q4_K, E.Q6_K), 2048, 768, 128, 8, 32, True, 3,
                         attn=((4096, 2048), (512, 2048), (512, 2048))))
        out = {"workload": name, "weight_bytes_per_layer": w.weight_bytes // w.copies}
        if moe_leg in ("both", "plan"):
            out["ms_per_layer"] = round(w.time(Wm, K), 4)
        if moe_leg in ("both", "device"):
            out["device_routed_ms_per_layer"] = round(w.time_device_routed(Wm, K), 4)
            out["device_routed_same_routing_ms_per_layer"] = round(w.time_device_routed(Wm, K, same_routing=True), 4)
        w.close()
        return out
    if name.startswith("decode_"):   # config 2's decode in another weight format (same shapes, same 38 layer copies)
        t = E.TYPES[name[len("decode_"):].upper()]
        mats, na, copies = [(t, r, c) for _, r, c in Q4K_FFN], 1, 38
    elif name in ("prefill_q5k", "prefill_q3k"):   # config 2's prefill with the weights in Q5_K / Q3_K
        t = E.Q5_K if name == "prefill_q5k" else E.Q3_K
        mats, na, copies = [(t, r, c) for _, r, c in Q4K_FFN], 512, 1
    else:
        mats, na, copies = {"decode": (Q4K_FFN, 1, 38), "prefill": (Q4K_FFN, 512, 1), "config1": ([(E.Q4_0, 4864, 896)], 1, 410),
                            "config3b1": ([(E.Q6_K, 151936, 1024)], 1, 8), "config3b64": ([(E.Q6_K, 151936, 1024)], 64, 8)}[name]
    w = Workload(lib, rng, mats, na, copies)
    _, ev = w.time(Wm, K)
    out = {"workload": name, "ms_per_launch": round(ev, 4), "weight_bytes_per_launch": w.weight_bytes,
           "gbs": round(w.weight_bytes / (ev * 1e-3) / 1e9, 1), "tops": round(w.ops / (ev * 1e-3) / 1e12, 2)}
    w.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-seconds", type=float, default=2.0)
    ap.add_argument("--only", choices=["decode", "prefill", "prefill_q5k", "prefill_q3k", "dense", "config1", "config3b1", "config3b64", "config4", "config5", "act",
                                       "cache", "copy", "host_queue"] + [f"decode_{f.lower()}" for f in E.TYPES],
                    help="run one workload alone (for profiler runs) and print its own JSON line")
    ap.add_argument("--moe-leg", choices=["both", "plan", "device"], default="both",
                    help="with --only config4/config5: time the prepared plan, the device-routed context, or both")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); the path shards by output rows or by "
              "experts across GPUs, which is not part of this build", file=sys.stderr)
        sys.exit(2)

    lib = E.Lib()
    if not lib.available():
        raise SystemExit("no usable gfx950 device: " + lib.last_error())
    rng = np.random.default_rng(20260101)
    K, Wm = args.steps, args.warmup
    if args.only:
        print(json.dumps(only(lib, rng, args.only, K, Wm, args.moe_leg)), flush=True)
        return

    # ---- headline: config 2 decode, Q4_K, T=1, 1.08 GB rotating set
    copies = 38
    dec = Workload(lib, rng, Q4K_FFN, 1, copies)
    wall, ev = dec.time(Wm, K)
    gbs = dec.weight_bytes / (ev * 1e-3) / 1e9
    head_bytes = dec.weight_bytes
    dec.close()

    # ---- config 2 prefill, T=512
    pre = Workload(lib, rng, Q4K_FFN, 512, 1)
    pwall, pev = pre.time(Wm, max(3, K // 4))
    tops = pre.ops / (pev * 1e-3) / 1e12
    pre.close()

    extra = {}
    # ---- config 2 prefill with the weights in Q5_K (the matrix-core kernel's third plane) and in Q3_K, T=512
    for key, t in (("prefill_q5k_t512", E.Q5_K), ("prefill_q3k_t512", E.Q3_K)):
        pk = Workload(lib, rng, [(t, r, c) for _, r, c in Q4K_FFN], 512, 1)
        _, pkev = pk.time(Wm, max(3, K // 4))
        pktops = pk.ops / (pkev * 1e-3) / 1e12
        extra[key] = {"tops": round(pktops, 2), "ms": round(pkev, 4), "frac": round(pktops / INT8_PEAK_TOPS, 4)}
        pk.close()
    # ---- config 2 dense_n on the device (gate/up, SwiGLU + Q8_K, down), T=512
    extra["config2_dense_ffn_t512"] = dense_ffn_time(lib, rng, max(3, K // 4), Wm)
    # ---- config 1: Q4_0 4864x896, b=1, 410 copies (1.0 GB)
    c1 = Workload(lib, rng, [(E.Q4_0, 4864, 896)], 1, 410)
    _, e1 = c1.time(Wm, K)
    extra["config1_q4_0_decode"] = {"gbs": round(c1.weight_bytes / (e1 * 1e-3) / 1e9, 1), "ms": round(e1, 4),
                                    "weight_bytes": c1.weight_bytes}
    c1.close()
    # ---- config 3: Q6_K head 151936x1024 (K padded from 896), b=1 and b=64, 8 copies (1.0 GB)
    for b in (1, 64):
        c3 = Workload(lib, rng, [(E.Q6_K, 151936, 1024)], b, 8)
        _, e3 = c3.time(Wm, max(3, K // 2))
        extra[f"config3_q6_k_head_b{b}"] = {"gbs": round(c3.weight_bytes / (e3 * 1e-3) / 1e9, 1), "ms": round(e3, 4),
                                           "weight_bytes": c3.weight_bytes}
        c3.close()

    # ---- config 4: OLMoE Q2_K experts (64 x gate/up 1024x2048, down 2048x1024), 128 tokens top-8; 8 layer copies
    c4 = MoeWorkload(lib, moe_rng(4), (E.Q2_K, E.Q2_K, E.Q2_K), 2048, 1024, 64, 8, 128, False, 8)
    e4 = c4.time(Wm, max(3, K // 2))
    d4 = c4.time_device_routed(Wm, max(3, K // 2))
    s4 = c4.time_device_routed(Wm, max(3, K // 2), same_routing=True)
    extra["config4_q2_k_moe"] = {"gbs": round(c4.weight_bytes / c4.copies / (e4 * 1e-3) / 1e9, 1), "ms": round(e4, 4),
                                 "weight_bytes": c4.weight_bytes // c4.copies, "experts_used": c4.distinct,
                                 "hbm_frac": round(c4.weight_bytes / c4.copies / (e4 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                 "device_routed_ms": round(d4, 4), "device_routed_vs_plan": round(d4 / e4, 3),
                                 "device_routed_same_routing_ms": round(s4, 4),
                                 "device_routed_same_routing_vs_plan": round(s4 / e4, 3)}
    c4.close()
    # ---- config 5: Qwen3-30B-A3B-like decode batch of 32: Q5_0 attention q/k/v + 128 experts (Q4_K gate/up 768x2048,
    # Q6_K down 2048x768) top-8 renormalised; 3 layer copies
    c5 = MoeWorkload(lib, moe_rng(5), (E.Q4_K, E.Q4_K, E.Q6_K), 2048, 768, 128, 8, 32, True, 3,
                     attn=((4096, 2048), (512, 2048), (512, 2048)))
    e5 = c5.time(Wm, max(3, K // 2))
    d5 = c5.time_device_routed(Wm, max(3, K // 2))
    s5 = c5.time_device_routed(Wm, max(3, K // 2), same_routing=True)
    extra["config5_mixed_moe_decode"] = {"gbs": round(c5.weight_bytes / c5.copies / (e5 * 1e-3) / 1e9, 1),
                                         "ms": round(e5, 4), "weight_bytes": c5.weight_bytes // c5.copies,
                                         "experts_used": c5.distinct,
                                         "hbm_frac": round(c5.weight_bytes / c5.copies / (e5 * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                         "device_routed_ms": round(d5, 4), "device_routed_vs_plan": round(d5 / e5, 3),
                                         "device_routed_same_routing_ms": round(s5, 4),
                                         "device_routed_same_routing_vs_plan": round(s5 / e5, 3)}
    c5.close()
    # ---- device activation preparation at config 2's prefill shapes (rmsnorm / SwiGLU fused with the quantizers)
    extra["act_prep_t512"] = act_prep_times(lib, rng, K, Wm)
    extra["expert_cache_load"] = cache_load_rate(lib, rng, K, Wm)
    extra["expert_cache_load_pinned"] = cache_load_rate(lib, rng, K, Wm, pinned=True)
    # ---- the engine-facing host binding (es_hip_run_jobs_host) at config 2 decode and prefill: PCIe-inclusive
    extra["host_queue_t1"] = host_queue_time(lib, rng, K, Wm, 1)
    extra["host_queue_t512"] = host_queue_time(lib, rng, max(3, K // 4), Wm, 512)

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(rng, args.cpu_seconds)
        cfg_cpu = cpu_configs(rng, args.cpu_seconds / 2)
        for key, rec in cfg_cpu.items():
            if key == "prefill":
                continue
            extra.setdefault(key, {})["cpu"] = rec

    # HBM bytes per launch of the same workloads, from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summaries
    traffic = {}
    tj = os.path.join(ROOT, "profiles", "hbm_traffic.json")
    if os.path.exists(tj):
        for k, v in json.load(open(tj))["workloads"].items():
            traffic[k] = v["hbm_read_bytes"] + v["hbm_write_bytes"]
    line = {
        "metric": METRIC, "value": round(gbs, 1), "unit": "GB/s", "n_gpus": 1, "steps": K, "warmup": Wm,
        "ms_per_step": round(wall, 4), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8", "data": "synthetic",
        "config": {"workload": "Q4_K decode matvec, Llama-3.2-1B FFN shapes (gate/up 8192x2048, down 2048x8192), T=1, "
                               f"{copies} layer copies = {head_bytes / 1e9:.2f} GB rotating, one batched launch per step",
                   "global_batch": 1, "hbm_frac": round(gbs / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": traffic.get("decode"),
                     "algorithmic_bytes": head_bytes},
        "cpu_baseline": cpu,
        "prefill": {"workload": "Q4_K prefill T=512: gate/up 8192x2048 and down 2048x8192, one batched launch",
                    "value": round(tops, 2), "unit": "TOPS", "ms": round(pev, 4),
                    "cpu": None if args.no_cpu else cfg_cpu["prefill"],
                    "roofline": {"bound": "mfma", "achieved": round(tops, 2), "peak": INT8_PEAK_TOPS, "unit": "TOPS",
                                 "frac": round(tops / INT8_PEAK_TOPS, 4), "traffic": traffic.get("prefill")}},
        "configs": extra,
        "device": lib.device_name(),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
