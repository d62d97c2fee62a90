// Device expert cache: the reference's hot-expert RAM cache (src/es_cache.h:1-56, src/es_cache.c:1-71) with its slots in
// HBM, and the engine's use of it (load_experts, src/es_engine.c:665-708; the router's prefetch, :606-611).
//
// The slot policy is the reference's: a fixed number of equal-size slots, one expert each, keyed by (layer, expert).
// A claim scans the slots in index order; a slot still loading is skipped until its load has finished (a HIP event on the
// stream that carried the copy), the first empty slot is taken at once, slots with protect_until >= step are skipped, and
// among the rest the lowest last_use + freq_weight * min(uses, 16) is evicted (the first of equal scores). Expert bytes
// move host -> device with hipMemcpyAsync on the caller's stream, so products launched later on that stream see them
// without a host wait. All slots live in one device allocation (slot stride rounded up to 256 bytes). slot_bytes = 0
// makes a cache with bookkeeping only (no device memory, usable without a GPU).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <vector>

#include "es_hip_common.h"
#include "es_hip_host.h"

struct es_hip_cache {
    struct Slot {
        int layer = -1, expert = -1, state = ES_HIP_SLOT_EMPTY, prefetched = 0;
        uint64_t last_use = 0, protect_until = 0;
        uint32_t uses = 0;
        hipEvent_t ev = nullptr;   // the slot's last load, while `pending`
        bool pending = false;
    };
    int nslots = 0, nlayers = 0, nexperts = 0;
    size_t slot_bytes = 0, stride = 0;
    double freq_weight = 0.0;
    uint64_t step = 0;
    uint8_t *base = nullptr;
    std::vector<Slot> slots;
    std::vector<int> where;   // layer * nexperts + expert -> slot, or -1
    es_hip_cache_stats st{};
};

namespace {

using esq::host_fail;

bool key_ok(const es_hip_cache *c, int layer, int expert) {
    return layer >= 0 && layer < c->nlayers && expert >= 0 && expert < c->nexperts;
}

// a loading slot whose copy has finished becomes READY; returns whether the slot is still loading
bool reap(es_hip_cache::Slot &s) {
    if (s.state != ES_HIP_SLOT_LOADING) return false;
    if (s.pending) {
        if (hipEventQuery(s.ev) != hipSuccess) return true;   // not done yet (or failed: never evicted)
        s.pending = false;
    }
    s.state = ES_HIP_SLOT_READY;
    return false;
}

int claim(es_hip_cache *c, int layer, int expert) {
    int best = -1;
    double best_score = 0.0;
    for (int i = 0; i < c->nslots; i++) {
        es_hip_cache::Slot &s = c->slots[i];
        if (reap(s)) continue;
        if (s.state == ES_HIP_SLOT_EMPTY) { best = i; break; }
        if (s.protect_until >= c->step) continue;
        const uint32_t u = s.uses < 16 ? s.uses : 16;
        const double score = static_cast<double>(s.last_use) + c->freq_weight * static_cast<double>(u);
        if (best < 0 || score < best_score) { best = i; best_score = score; }
    }
    if (best < 0) return -1;
    es_hip_cache::Slot &s = c->slots[best];
    if (s.layer >= 0) {
        c->where[(size_t)s.layer * c->nexperts + s.expert] = -1;
        c->st.evictions++;
        if (s.prefetched) c->st.prefetch_wasted++;
    }
    s.layer = layer;
    s.expert = expert;
    s.state = ES_HIP_SLOT_LOADING;
    s.prefetched = 0;
    s.uses = 0;
    s.last_use = c->step;
    s.protect_until = c->step + 1;
    c->where[(size_t)layer * c->nexperts + expert] = best;
    return best;
}

int load(es_hip_cache *c, int slot, size_t offset, const void *host, size_t bytes, hipStream_t stream) {
    es_hip_cache::Slot &s = c->slots[slot];
    if (!c->base) return host_fail(ES_HIP_EINVAL, "this cache has no device slots (slot_bytes 0)");
    if (s.layer < 0) return host_fail(ES_HIP_EINVAL, "slot is empty: claim it first");
    if (!host || bytes == 0 || offset > c->slot_bytes || bytes > c->slot_bytes - offset)
        return host_fail(ES_HIP_EINVAL, "load outside the slot (or null source)");
    if (int rc = esq::host_need_device()) return rc;
    hipError_t e;
    if (!s.ev && (e = hipEventCreateWithFlags(&s.ev, hipEventDisableTiming)) != hipSuccess)
        return esq::host_hip_fail(e, "hipEventCreateWithFlags");
    if ((e = hipMemcpyAsync(c->base + (size_t)slot * c->stride + offset, host, bytes, hipMemcpyHostToDevice, stream)) !=
        hipSuccess)
        return esq::host_hip_fail(e, "hipMemcpyAsync (expert load)");
    if ((e = hipEventRecord(s.ev, stream)) != hipSuccess) return esq::host_hip_fail(e, "hipEventRecord");
    s.pending = true;
    s.state = ES_HIP_SLOT_LOADING;
    return ES_HIP_OK;
}

// a slot whose expert could not be loaded is emptied, so it can never be found holding partial bytes; copies of its
// earlier parts still in flight are waited for first (a reload into the slot, perhaps on another stream, must not be
// overwritten by them)
void unmap(es_hip_cache *c, int slot) {
    es_hip_cache::Slot &s = c->slots[slot];
    if (s.pending) {
        (void)hipEventSynchronize(s.ev);
        s.pending = false;
    }
    if (s.layer >= 0) c->where[(size_t)s.layer * c->nexperts + s.expert] = -1;
    s.layer = s.expert = -1;
    s.state = ES_HIP_SLOT_EMPTY;
    s.prefetched = 0;
    s.uses = 0;
}

// the expert's parts from their host slabs into the slot (read_expert_part / the expert file, src/es_engine.c:686-699)
int load_parts(es_hip_cache *c, int slot, int expert, const es_hip_expert_src *src, hipStream_t stream) {
    for (int r = 0; r < 3; r++) {
        if (!src->bytes[r]) continue;
        const uint8_t *h = static_cast<const uint8_t *>(src->base[r]);
        int rc = h ? load(c, slot, src->offset[r], h + (size_t)expert * src->stride[r], src->bytes[r], stream)
                   : host_fail(ES_HIP_EINVAL, "expert source part without a base pointer");
        if (rc) {
            unmap(c, slot);
            return rc;
        }
    }
    return ES_HIP_OK;
}

}  // namespace

extern "C" {

int es_hip_cache_create(es_hip_cache **out, int nslots, size_t slot_bytes, int nlayers, int nexperts, double freq_weight) {
    if (!out) return host_fail(ES_HIP_EINVAL, "null output pointer");
    *out = nullptr;
    if (nslots <= 0 || nlayers <= 0 || nexperts <= 0 || (long long)nlayers * nexperts > (1LL << 30))
        return host_fail(ES_HIP_EINVAL, "nslots, nlayers and nexperts must be positive (nlayers * nexperts <= 2^30)");
    if (!std::isfinite(freq_weight) || freq_weight < 0.0) return host_fail(ES_HIP_EINVAL, "freq_weight must be finite and >= 0");
    if (slot_bytes > (SIZE_MAX - 255) / 2 || (slot_bytes + 255) / 256 * 256 > SIZE_MAX / (size_t)nslots)
        return host_fail(ES_HIP_EINVAL, "nslots x slot_bytes overflows");
    es_hip_cache *c = new es_hip_cache;
    c->nslots = nslots;
    c->nlayers = nlayers;
    c->nexperts = nexperts;
    c->slot_bytes = slot_bytes;
    c->stride = (slot_bytes + 255) / 256 * 256;
    c->freq_weight = freq_weight;
    c->slots.resize(nslots);
    c->where.assign((size_t)nlayers * nexperts, -1);
    if (slot_bytes) {
        if (int rc = esq::host_need_device()) { delete c; return rc; }
        hipError_t e = hipMalloc(reinterpret_cast<void **>(&c->base), c->stride * (size_t)nslots);
        if (e != hipSuccess) { delete c; return esq::host_hip_fail(e, "hipMalloc (expert cache slots)"); }
    }
    *out = c;
    return ES_HIP_OK;
}

void es_hip_cache_destroy(es_hip_cache *c) {
    if (!c) return;
    for (auto &s : c->slots)
        if (s.ev) {
            if (s.pending) (void)hipEventSynchronize(s.ev);
            (void)hipEventDestroy(s.ev);
        }
    if (c->base) (void)hipFree(c->base);
    delete c;
}

int es_hip_cache_find(const es_hip_cache *c, int layer, int expert) {
    if (!c || !key_ok(c, layer, expert)) return -1;
    return c->where[(size_t)layer * c->nexperts + expert];
}

int es_hip_cache_claim(es_hip_cache *c, int layer, int expert) {
    if (!c || !key_ok(c, layer, expert)) return host_fail(ES_HIP_EINVAL, "null cache or (layer, expert) out of range");
    if (c->where[(size_t)layer * c->nexperts + expert] >= 0)
        return host_fail(ES_HIP_EINVAL, "(layer, expert) is already in the cache");
    const int s = claim(c, layer, expert);
    return s >= 0 ? s : host_fail(ES_HIP_EBUSY, "every slot is loading or protected");
}

void *es_hip_cache_slot_ptr(const es_hip_cache *c, int slot) {
    if (!c || !c->base || slot < 0 || slot >= c->nslots) return nullptr;
    return c->base + (size_t)slot * c->stride;
}

int es_hip_cache_load(es_hip_cache *c, int slot, size_t offset, const void *host, size_t bytes, void *stream) {
    if (!c || slot < 0 || slot >= c->nslots) return host_fail(ES_HIP_EINVAL, "null cache or slot out of range");
    return load(c, slot, offset, host, bytes, static_cast<hipStream_t>(stream));
}

int es_hip_cache_wait(es_hip_cache *c, int slot) {
    if (!c || slot < 0 || slot >= c->nslots) return host_fail(ES_HIP_EINVAL, "null cache or slot out of range");
    es_hip_cache::Slot &s = c->slots[slot];
    if (s.pending) {
        hipError_t e = hipEventSynchronize(s.ev);
        if (e != hipSuccess) return esq::host_hip_fail(e, "hipEventSynchronize (expert load)");
        s.pending = false;
    }
    if (s.state == ES_HIP_SLOT_LOADING) s.state = ES_HIP_SLOT_READY;
    return ES_HIP_OK;
}

int es_hip_cache_step(es_hip_cache *c) {
    if (!c) return host_fail(ES_HIP_EINVAL, "null cache");
    c->step++;
    return ES_HIP_OK;
}

int es_hip_cache_acquire(es_hip_cache *c, int layer, const int *sel, int k, const es_hip_expert_src *src, int *slots,
                         void *stream) {
    if (!c || k < 0 || (k > 0 && (!sel || !slots))) return host_fail(ES_HIP_EINVAL, "null cache, selection or slot array");
    if (layer < 0 || layer >= c->nlayers) return host_fail(ES_HIP_EINVAL, "layer out of range");
    for (int j = 0; j < k; j++)
        if (sel[j] < 0 || sel[j] >= c->nexperts) return host_fail(ES_HIP_EINVAL, "expert out of range");
    if (src && !c->base) return host_fail(ES_HIP_EINVAL, "expert sources given to a cache without device slots");
    const hipStream_t st = static_cast<hipStream_t>(stream);
    c->step++;
    int busy = 0;
    for (int j = 0; j < k; j++) {
        int s = c->where[(size_t)layer * c->nexperts + sel[j]];
        if (s >= 0) {
            c->st.hits++;
            if (c->slots[s].prefetched) { c->st.prefetch_used++; c->slots[s].prefetched = 0; }
        } else {
            c->st.misses++;
            s = claim(c, layer, sel[j]);
            if (s >= 0) {
                if (src) {
                    if (int rc = load_parts(c, s, sel[j], src, st)) return rc;
                } else {
                    c->slots[s].state = ES_HIP_SLOT_READY;   // bookkeeping only: nothing to load
                }
            }
        }
        slots[j] = s;
        if (s < 0) { busy = 1; continue; }
        es_hip_cache::Slot &q = c->slots[s];
        q.uses++;
        q.last_use = c->step;
        q.protect_until = c->step;
    }
    return busy ? host_fail(ES_HIP_EBUSY, "expert cache too small: every slot is loading or protected") : ES_HIP_OK;
}

int es_hip_cache_prefetch(es_hip_cache *c, int layer, int expert, const es_hip_expert_src *src, void *stream, int *slot) {
    if (!c || !slot || !key_ok(c, layer, expert)) return host_fail(ES_HIP_EINVAL, "null cache/slot or (layer, expert) out of range");
    if (src && !c->base) return host_fail(ES_HIP_EINVAL, "expert sources given to a cache without device slots");
    *slot = -1;
    if (c->where[(size_t)layer * c->nexperts + expert] >= 0) return ES_HIP_OK;   // cached already: nothing to do
    const int s = claim(c, layer, expert);
    if (s < 0) return host_fail(ES_HIP_EBUSY, "no slot free for the prefetch");
    c->slots[s].prefetched = 1;
    c->slots[s].protect_until = c->step + 3;
    c->st.prefetch_issued++;
    *slot = s;
    if (src) return load_parts(c, s, expert, src, static_cast<hipStream_t>(stream));
    return ES_HIP_OK;
}

int es_hip_cache_slot_info(const es_hip_cache *c, int slot, es_hip_slot_info *out) {
    if (!c || !out || slot < 0 || slot >= c->nslots) return host_fail(ES_HIP_EINVAL, "null cache/output or slot out of range");
    const es_hip_cache::Slot &s = c->slots[slot];
    *out = es_hip_slot_info{s.layer, s.expert, s.state, s.prefetched, s.last_use, s.uses, s.protect_until};
    return ES_HIP_OK;
}

int es_hip_cache_get_stats(const es_hip_cache *c, es_hip_cache_stats *out) {
    if (!c || !out) return host_fail(ES_HIP_EINVAL, "null cache or output");
    *out = c->st;
    out->step = c->step;
    return ES_HIP_OK;
}

}  // extern "C"
