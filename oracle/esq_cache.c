/*
 * esq_cache — CPU restatement of the hot-expert cache policy. TEST INFRASTRUCTURE ONLY (see esq_cache.h).
 *
 * Eviction (es_cache_claim, src/es_cache.c:39-71): scanning slots in index order, a LOADING slot whose load has finished
 * becomes READY (here every load has finished); the first EMPTY slot is taken at once; a slot with protect_until >= step
 * is skipped; otherwise the slot with the lowest score last_use + freq_weight * min(uses, 16) wins, the first of equal
 * scores. The victim's old key is unmapped (an eviction, and a wasted prefetch if it was never used), the new key mapped,
 * and the slot reset: LOADING, prefetched 0, uses 0, last_use = step, protect_until = step + 1.
 */
#include "esq_cache.h"

#include <stdlib.h>
#include <string.h>

enum { SLOT_EMPTY = 0, SLOT_LOADING = 1, SLOT_READY = 2 };

typedef struct {
    int layer, expert, state, prefetched;
    uint64_t last_use, protect_until;
    uint32_t uses;
} slot_t;

typedef struct {
    int nslots, nexperts;
    double freq_weight;
    uint64_t step;
    slot_t *s;
    int *where;   /* layer * nexperts + expert -> slot or -1 */
    uint64_t hits, misses, pf_issued, pf_used, pf_wasted, evictions;
} cache_t;

static int pick_victim(cache_t *c) {
    int best = -1;
    double best_score = 0.0;
    for (int i = 0; i < c->nslots; i++) {
        slot_t *s = &c->s[i];
        if (s->state == SLOT_LOADING) s->state = SLOT_READY;   /* its load is done */
        if (s->state == SLOT_EMPTY) return i;
        if (s->protect_until >= c->step) continue;
        const uint32_t u = s->uses < 16 ? s->uses : 16;
        const double score = (double)s->last_use + c->freq_weight * (double)u;
        if (best < 0 || score < best_score) {
            best = i;
            best_score = score;
        }
    }
    return best;
}

static int claim(cache_t *c, int layer, int expert) {
    const int v = pick_victim(c);
    if (v < 0) return -1;
    slot_t *s = &c->s[v];
    if (s->layer >= 0) {
        c->where[s->layer * c->nexperts + s->expert] = -1;
        c->evictions++;
        if (s->prefetched) c->pf_wasted++;
    }
    s->layer = layer;
    s->expert = expert;
    s->state = SLOT_LOADING;
    s->prefetched = 0;
    s->uses = 0;
    s->last_use = c->step;
    s->protect_until = c->step + 1;
    c->where[layer * c->nexperts + expert] = v;
    return v;
}

int esq_cache_trace(int nslots, int nlayers, int nexperts, double freq_weight, const int32_t *ops, int nops, int32_t *res,
                    int64_t *slots_out, uint64_t *stats_out) {
    if (nslots <= 0 || nlayers <= 0 || nexperts <= 0) return -1;
    cache_t c;
    memset(&c, 0, sizeof c);
    c.nslots = nslots;
    c.nexperts = nexperts;
    c.freq_weight = freq_weight;
    c.s = calloc((size_t)nslots, sizeof(slot_t));
    c.where = malloc(sizeof(int) * (size_t)nlayers * (size_t)nexperts);
    if (!c.s || !c.where) { free(c.s); free(c.where); return -1; }
    for (int i = 0; i < nlayers * nexperts; i++) c.where[i] = -1;
    for (int i = 0; i < nslots; i++) c.s[i].layer = c.s[i].expert = -1;
    for (int i = 0; i < nops; i++) {
        const int op = ops[3 * i], l = ops[3 * i + 1], e = ops[3 * i + 2];
        int r = 0;
        if (op == ESQ_OP_STEP) {
            c.step++;
        } else if (op == ESQ_OP_ACQUIRE) {   /* load_experts, one expert (src/es_engine.c:673-707) */
            int s = c.where[l * nexperts + e];
            if (s >= 0) {
                c.hits++;
                if (c.s[s].prefetched) { c.pf_used++; c.s[s].prefetched = 0; }
            } else {
                c.misses++;
                s = claim(&c, l, e);
                if (s >= 0) c.s[s].state = SLOT_READY;   /* read at once */
            }
            if (s >= 0) {
                c.s[s].uses++;
                c.s[s].last_use = c.step;
                c.s[s].protect_until = c.step;
            }
            r = s;
        } else if (op == ESQ_OP_PREFETCH) {   /* the router's prefetch (src/es_engine.c:606-611) */
            if (c.where[l * nexperts + e] >= 0) {
                r = -2;
            } else {
                const int s = claim(&c, l, e);
                if (s >= 0) {
                    c.s[s].prefetched = 1;
                    c.s[s].protect_until = c.step + 3;
                    c.pf_issued++;
                }
                r = s;
            }
        }
        res[i] = r;
    }
    for (int i = 0; i < nslots; i++) {
        const slot_t *s = &c.s[i];
        int64_t *o = slots_out + 7 * (size_t)i;
        o[0] = s->layer; o[1] = s->expert; o[2] = s->state; o[3] = s->prefetched;
        o[4] = (int64_t)s->last_use; o[5] = s->uses; o[6] = (int64_t)s->protect_until;
    }
    const uint64_t st[7] = {c.hits, c.misses, c.pf_issued, c.pf_used, c.pf_wasted, c.evictions, c.step};
    memcpy(stats_out, st, sizeof st);
    free(c.s);
    free(c.where);
    return 0;
}
