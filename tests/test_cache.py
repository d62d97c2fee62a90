"""CPU tests of the expert cache policy: the oracle's restatement (oracle/esq_cache.c) against golden traces written by the
reference's own es_cache.c (tests/golden/make_golden.py), textbook cases of LRU and frequency-weighted eviction, and the
library's device cache (es_hip_cache_*, bookkeeping-only mode: no device memory) against both."""
import numpy as np
import pytest

import oracle as O
import es_hip_quant as E

TRACES = ["lru", "engine", "olmoe", "wasted", "tiny", "noprefetch"]


def golden_trace(golden, name):
    ns, nl, ne = (int(v) for v in golden[f"cache/{name}/params"])
    fw = float(golden[f"cache/{name}/freq_weight"][0])
    want = tuple(golden[f"cache/{name}/{k}"] for k in ("res", "slots", "stats"))
    return ns, nl, ne, fw, golden[f"cache/{name}/ops"], want


def same(a, b):
    return all(np.array_equal(x, y) for x, y in zip(a, b))


@pytest.mark.parametrize("name", TRACES)
def test_oracle_cache_matches_reference(orc, golden, name):
    ns, nl, ne, fw, ops, want = golden_trace(golden, name)
    assert same(orc.cache_trace(ns, nl, ne, fw, ops), want)


@pytest.mark.parametrize("name", TRACES)
def test_library_cache_policy_matches_reference(hiplib, golden, name):
    ns, nl, ne, fw, ops, want = golden_trace(golden, name)
    c = E.ExpertCache(hiplib, ns, 0, nl, ne, fw)
    try:
        assert same(c.run_trace(ops), want)
    finally:
        c.close()


def test_golden_traces_exercise_every_branch(golden):
    """the fixture covers hits, misses, evictions, used and wasted prefetches, already-cached prefetches and a full cache"""
    st = np.stack([golden[f"cache/{n}/stats"] for n in TRACES])
    res = np.concatenate([golden[f"cache/{n}/res"] for n in TRACES])
    assert (st[:, 0] > 0).any() and (st[:, 1] > 0).all() and (st[:, 5] > 0).all()
    assert (st[:, 3] > 0).any() and (st[:, 4] > 0).any()
    assert (res == -1).any() and (res == -2).any()


@pytest.mark.parametrize("seed", range(6))
def test_library_cache_equals_oracle_on_random_traces(orc, hiplib, seed):
    rng = np.random.default_rng(seed)
    nl, ne, k = int(rng.integers(2, 6)), int(rng.integers(8, 96)), int(rng.integers(1, 9))
    ns = int(rng.integers(max(2, k // 2), 3 * k + 4))
    fw = float(rng.choice([0.0, 0.5, 1.0 * nl, 10.0]))
    ops = O.make_cache_trace(100 + seed, nl, ne, min(k, ne), int(rng.integers(1, 4)), 2,
                             prefetch=[None, "top", "random"][seed % 3])
    c = E.ExpertCache(hiplib, ns, 0, nl, ne, fw)
    try:
        assert same(c.run_trace(ops), orc.cache_trace(ns, nl, ne, fw, ops))
    finally:
        c.close()


def acq(l, *experts):
    return [(O.OP_STEP, l, 0)] + [(O.OP_ACQUIRE, l, e) for e in experts]


def test_plain_lru_closed_form(orc):
    """freq_weight 0 is LRU: with 2 slots, a third expert evicts the least recently used one"""
    ops = acq(0, 0) + acq(0, 1) + acq(0, 2) + acq(0, 0) + acq(0, 2)
    res, slots, stats = orc.cache_trace(2, 1, 4, 0.0, np.array(ops))
    # slots: e0 -> 0, e1 -> 1, e2 evicts e0 (used at step 1) -> 0, e0 evicts e1 (step 2) -> 1, e2 hits in 0
    assert res[[1, 3, 5, 7, 9]].tolist() == [0, 1, 0, 1, 0]
    assert stats.tolist() == [1, 4, 0, 0, 0, 2, 5]
    assert slots[:, :2].tolist() == [[0, 2], [0, 0]]


def test_frequency_weight_keeps_a_hot_expert(orc):
    """with freq_weight 10 an expert used 3 times outlives a newer one used once (score last_use + 10 min(uses, 16))"""
    ops = acq(0, 0) + acq(0, 0) + acq(0, 0) + acq(0, 1) + acq(0, 2)
    res, _, _ = orc.cache_trace(2, 1, 4, 10.0, np.array(ops))
    assert res[-1] == 1        # e1 (score 4 + 10) goes, e0 (3 + 30) stays
    res, _, _ = orc.cache_trace(2, 1, 4, 0.0, np.array(ops))
    assert res[-1] == 0        # plain LRU evicts e0 (last used at step 3)


def test_protected_and_full(orc, hiplib):
    """experts of the current step are protected: a step needing more experts than slots gets -1 (ES_HIP_EBUSY)"""
    ops = np.array(acq(0, 0, 1, 2))
    res, _, stats = orc.cache_trace(2, 1, 4, 0.0, ops)
    assert res[1:].tolist() == [0, 1, -1] and stats[1] == 3
    c = E.ExpertCache(hiplib, 2, 0, 1, 4, 0.0)
    with pytest.raises(E.EsHipError):
        c.acquire(0, [0, 1, 2])
    assert c.find(0, 0) == 0 and c.find(0, 1) == 1 and c.find(0, 2) == -1
    c.close()


def test_cache_rejects_bad_arguments(hiplib):
    with pytest.raises(E.EsHipError):
        E.ExpertCache(hiplib, 0, 0, 1, 4, 0.0)
    with pytest.raises(E.EsHipError):
        E.ExpertCache(hiplib, 2, 0, 1, 4, -1.0)
    with pytest.raises(E.EsHipError) as err:
        E.ExpertCache(hiplib, 1 << 20, 1 << 62, 1, 4, 0.0)   # nslots x slot_bytes overflows: refused before any device use
    assert err.value.code == -2
    c = E.ExpertCache(hiplib, 2, 0, 2, 4, 1.0)
    try:
        with pytest.raises(E.EsHipError):
            c.claim(2, 0)                       # layer out of range
        s = c.claim(1, 3)
        assert s == 0 and c.find(1, 3) == 0
        with pytest.raises(E.EsHipError):
            c.claim(1, 3)                       # already cached
        with pytest.raises(E.EsHipError):
            c.load(s, 0, np.zeros(16, np.uint8))   # no device slots in bookkeeping mode
        with pytest.raises(E.EsHipError):
            c.acquire(0, [5])                   # expert out of range
        assert c.slot_ptr(0) is None
        assert c.find(-1, 0) == -1 and c.find(0, 99) == -1
    finally:
        c.close()
