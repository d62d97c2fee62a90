/*
 * esref_cache_trace — runs a cache trace (oracle/esq_cache.h) through the reference's own es_cache_init / es_cache_find /
 * es_cache_claim (src/es_cache.c), with the bookkeeping load_experts and the router's prefetch do around them
 * (src/es_engine.c:606-611, 671-707). TEST INFRASTRUCTURE ONLY: built by oracle/Makefile together with the reference's
 * src/es_cache.c and src/es_io.c, where they lie, into oracle/_ref/libesref_cache.so; used to write golden traces.
 * The hit/miss/prefetch counters are kept in the reference's es_cache fields of those names (the engine keeps its own
 * copies; es_cache_claim itself counts evictions and wasted prefetches).
 */
#include "esq_cache.h"

#include <string.h>

#include "es_cache.h"

int esref_cache_trace(int nslots, int nlayers, int nexperts, double freq_weight, const int32_t *ops, int nops,
                      int32_t *res, int64_t *slots_out, uint64_t *stats_out) {
    es_cache c;
    if (es_cache_init(&c, nslots, 64, nlayers, nexperts, freq_weight)) { es_cache_free(&c); return -1; }
    for (int i = 0; i < nops; i++) {
        const int op = ops[3 * i], l = ops[3 * i + 1], e = ops[3 * i + 2];
        int r = 0;
        if (op == ESQ_OP_STEP) {
            c.step++;
        } else if (op == ESQ_OP_ACQUIRE) {
            int s = es_cache_find(&c, l, e);
            if (s >= 0) {
                c.hits++;
                if (c.slots[s].prefetched) { c.prefetch_used++; c.slots[s].prefetched = 0; }
            } else {
                c.misses++;
                s = es_cache_claim(&c, NULL, l, e);
                if (s >= 0) c.slots[s].state = ES_SLOT_READY;
            }
            if (s >= 0) {
                c.slots[s].uses++;
                c.slots[s].last_use = c.step;
                c.slots[s].protect_until = c.step;
            }
            r = s;
        } else if (op == ESQ_OP_PREFETCH) {
            if (es_cache_find(&c, l, e) >= 0) {
                r = -2;
            } else {
                const int s = es_cache_claim(&c, NULL, l, e);
                if (s >= 0) {
                    c.slots[s].prefetched = 1;
                    c.slots[s].protect_until = c.step + 3;
                    c.prefetch_issued++;
                }
                r = s;
            }
        }
        res[i] = r;
    }
    for (int i = 0; i < nslots; i++) {
        const es_slot *s = &c.slots[i];
        int64_t *o = slots_out + 7 * (size_t)i;
        o[0] = s->layer; o[1] = s->expert; o[2] = s->state; o[3] = s->prefetched;
        o[4] = (int64_t)s->last_use; o[5] = s->uses; o[6] = (int64_t)s->protect_until;
    }
    const uint64_t st[7] = {c.hits, c.misses, c.prefetch_issued, c.prefetch_used, c.prefetch_wasted, c.evictions, c.step};
    memcpy(stats_out, st, sizeof st);
    es_cache_free(&c);
    return 0;
}
