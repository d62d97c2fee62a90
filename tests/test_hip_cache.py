"""GPU tests of the device expert cache (es_hip_cache_*): after every load_experts step and prefetch, each cached expert's
bytes sit in its HBM slot exactly as they are in the host slabs (gate | up | down at their offsets), the slot choices and
counters equal the oracle's (itself pinned to the reference's es_cache.c), products read straight from slot memory equal
the oracle's on the host bytes, and loads outside a slot are refused."""
import numpy as np
import pytest

import oracle as O
import es_hip_quant as E

pytestmark = pytest.mark.gpu

N, FF = 512, 256                       # expert FFN: gate/up Q4_K FF x N, down Q6_K N x FF
PARTS = [(E.Q4_K, FF, N), (E.Q4_K, FF, N), (E.Q6_K, N, FF)]


def part_bytes():
    return [rows * O.row_bytes(t, cols) for t, rows, cols in PARTS]


def make_slabs(orc, nl, ne, seed):
    """per layer, the three 3-D slabs [ne, part bytes] of valid blocks (es_mtest's generator)"""
    st = np.array([seed], np.uint64)
    return [[np.stack([orc.mtest_blocks(t, st, rows, cols) for _ in range(ne)]) for t, rows, cols in PARTS]
            for _ in range(nl)]


def src_of(layer_slabs):
    pb = part_bytes()
    s = E.ExpertSrc()
    off = 0
    for r in range(3):
        s.base[r] = layer_slabs[r].ctypes.data
        s.stride[r] = pb[r]
        s.bytes[r] = pb[r]
        s.offset[r] = off
        off += pb[r]
    return s


def check_resident(hip, c, slabs, nslots):
    slot_bytes = sum(part_bytes())
    for k in range(nslots):
        info = c.slot_info(k)
        if info.layer < 0:
            continue
        got = hip.download(c.slot_ptr(k), np.zeros(slot_bytes, np.uint8))
        want = np.concatenate([slabs[info.layer][r][info.expert] for r in range(3)])
        assert np.array_equal(got, want), (k, info.layer, info.expert)


@pytest.mark.parametrize("seed,nslots,fw,prefetch", [(11, 6, 3.0, "top"), (12, 5, 0.0, "random"), (13, 9, 1.5, None)])
def test_cache_loads_experts_byte_for_byte(hip, orc, seed, nslots, fw, prefetch):
    nl, ne, k = 3, 12, 4
    slabs = make_slabs(orc, nl, ne, seed)
    srcs = [src_of(s) for s in slabs]
    ops = O.make_cache_trace(seed, nl, ne, k, 2, 2, prefetch=prefetch)
    want_res, want_slots, want_stats = orc.cache_trace(nslots, nl, ne, fw, ops)
    c = E.ExpertCache(hip, nslots, sum(part_bytes()), nl, ne, fw)
    try:
        i = 0
        while i < len(ops):
            op, l, e = (int(v) for v in ops[i])
            if op == O.OP_STEP:
                j = i + 1
                while j < len(ops) and ops[j, 0] == O.OP_ACQUIRE:
                    j += 1
                got = c.acquire(l, ops[i + 1:j, 2], srcs[l], allow_busy=True)
                assert got.tolist() == want_res[i + 1:j].tolist(), i
                i = j
            else:
                assert c.prefetch(l, e, srcs[l]) == want_res[i], i
                i += 1
            hip.synchronize()   # every copy done before the next claim, as the oracle assumes
            check_resident(hip, c, slabs, nslots)
        st = c.stats()
        got_stats = [st.hits, st.misses, st.prefetch_issued, st.prefetch_used, st.prefetch_wasted, st.evictions, st.step]
        assert got_stats == want_stats.tolist()
        for s in range(nslots):
            info = c.slot_info(s)
            assert [info.layer, info.expert] == want_slots[s, :2].tolist()
    finally:
        c.close()


def test_products_from_slot_memory(hip, orc):
    """gate and down products of a cached expert, read from its slot, equal the oracle's on the host bytes"""
    nl, ne = 2, 6
    slabs = make_slabs(orc, nl, ne, 21)
    c = E.ExpertCache(hip, 3, sum(part_bytes()), nl, ne, 2.0)
    try:
        slots = c.acquire(1, [4, 0], src_of(slabs[1]))
        for s in slots:
            c.wait(int(s))
            assert c.slot_info(int(s)).state == E.ES_HIP_SLOT_READY
        rng = np.random.default_rng(3)
        x = rng.standard_normal((3, N)).astype(np.float32)
        h = rng.standard_normal((3, FF)).astype(np.float32)
        off_down = 2 * part_bytes()[0]
        for e, s in zip([4, 0], slots):
            base = c.slot_ptr(int(s))
            for (t, rows, cols), W, xin, off in [(PARTS[0], slabs[1][0][e], x, 0), (PARTS[2], slabs[1][2][e], h, off_down)]:
                acts = orc.quantize_act(t, xin)
                dA = hip.upload(acts)
                dY = hip.alloc(3 * rows * 4)
                hip.matvec_multi_dev(t, base + off, cols, 0, rows, dA, acts.strides[0], 3, dY, rows)
                y = hip.download(dY, np.zeros((3, rows), np.float32))
                ref = orc.matvec_multi(t, W, cols, rows, acts)
                assert np.array_equal(y.view(np.uint32), ref.view(np.uint32)), (e, t)
                dA.close()
                dY.close()
    finally:
        c.close()


def test_prefetch_then_hit(hip, orc):
    nl, ne = 2, 8
    slabs = make_slabs(orc, nl, ne, 31)
    c = E.ExpertCache(hip, 4, sum(part_bytes()), nl, ne, 1.0)
    try:
        s = c.prefetch(1, 5, src_of(slabs[1]))
        assert s == 0 and c.slot_info(s).prefetched == 1 and c.slot_info(s).protect_until == 3
        assert c.prefetch(1, 5, src_of(slabs[1])) == -2
        c.wait(s)
        check_resident(hip, c, slabs, 4)
        assert c.acquire(1, [5], src_of(slabs[1])).tolist() == [0]
        st = c.stats()
        assert (st.hits, st.misses, st.prefetch_issued, st.prefetch_used) == (1, 0, 1, 1)
    finally:
        c.close()


def test_load_bounds(hip):
    c = E.ExpertCache(hip, 2, 1000, 1, 4, 0.0)
    try:
        s = c.claim(0, 1)
        c.load(s, 0, (np.arange(1000) % 251).astype(np.uint8))
        c.load(s, 996, np.ones(4, np.uint8))
        c.wait(s)
        got = hip.download(c.slot_ptr(s), np.zeros(1000, np.uint8))
        assert np.array_equal(got[:996], (np.arange(996) % 251).astype(np.uint8)) and np.all(got[996:] == 1)
        with pytest.raises(E.EsHipError):
            c.load(s, 997, np.ones(4, np.uint8))      # one byte past the slot
        with pytest.raises(E.EsHipError):
            c.load(1, 0, np.ones(4, np.uint8))        # slot 1 was never claimed
        assert c.slot_ptr(1) - c.slot_ptr(0) == 1024   # slots 256-byte aligned
    finally:
        c.close()


def test_pinned_host_slabs(hip, orc):
    """expert slabs in page-locked memory (es_hip_host_alloc) load like pageable ones"""
    nl, ne = 1, 4
    slabs = make_slabs(orc, nl, ne, 41)
    pinned = []
    for part in slabs[0]:
        h = hip.host_array(part.shape, np.uint8)
        h[...] = part
        pinned.append(h)
    c = E.ExpertCache(hip, 2, sum(part_bytes()), nl, ne, 0.0)
    try:
        slots = c.acquire(0, [3, 1], src_of(pinned))
        hip.synchronize()
        check_resident(hip, c, [pinned], 2)
        assert [c.slot_info(int(s)).expert for s in slots] == [3, 1]
    finally:
        c.close()


def test_failed_part_empties_the_slot_after_its_copies(hip, orc):
    """an expert whose second part cannot be read (no base pointer) leaves its slot EMPTY, and only after the first part's
    copy has landed: the next expert acquired into that slot holds its own bytes, nothing of the failed load"""
    slabs = make_slabs(orc, 1, 3, 31)
    good = src_of(slabs[0])
    bad = src_of(slabs[0])
    bad.base[1] = None
    c = E.ExpertCache(hip, 1, sum(part_bytes()), 1, 3, 0.0)
    try:
        with pytest.raises(E.EsHipError):
            c.acquire(0, np.array([0], np.int32), bad)
        assert c.slot_info(0).layer == -1 and c.find(0, 0) == -1
        c.step()
        for s in c.acquire(0, np.array([1], np.int32), good):
            c.wait(int(s))
        check_resident(hip, c, slabs, 1)
        assert c.slot_info(0).expert == 1
    finally:
        c.close()
