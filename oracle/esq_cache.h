/*
 * esq_cache — CPU restatement of ExpertStream's hot-expert cache policy (src/es_cache.h:1-56, src/es_cache.c:1-71) and of
 * the way the engine drives it (load_experts, src/es_engine.c:665-708; the router's prefetch, :606-613).
 *
 * TEST INFRASTRUCTURE ONLY: the checker for the device expert cache's slot policy (es_hip_cache_*), never linked into the
 * shipped library.
 *
 * A trace is a list of operations, three int32 each (op, layer, expert):
 *   ESQ_OP_STEP      the start of load_experts for one layer: step += 1 (:671)
 *   ESQ_OP_ACQUIRE   one expert of that call (:673-707): a hit counts (and clears `prefetched`, counting a used
 *                    prefetch); a miss claims a slot (-1: every slot busy or protected) and loads it; then uses += 1,
 *                    last_use = step, protect_until = step. Result: the slot.
 *   ESQ_OP_PREFETCH  the router's prefetch of one expert (:606-611): -2 if already cached, else claim (-1 on failure),
 *                    prefetched = 1, protect_until = step + 3. Result: the slot.
 * Loads complete at once here (the reference's claim with no I/O pool finds every request done), so a LOADING slot is
 * reaped to READY by the next claim that scans it.
 * Outputs: res[i] per operation; per slot 7 int64 (layer, expert, state, prefetched, last_use, uses, protect_until);
 * 7 uint64 counters (hits, misses, prefetch_issued, prefetch_used, prefetch_wasted, evictions, step).
 */
#ifndef ESQ_CACHE_H
#define ESQ_CACHE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { ESQ_OP_STEP = 1, ESQ_OP_ACQUIRE = 2, ESQ_OP_PREFETCH = 3 };

/* the oracle's restatement; returns 0, or -1 on bad arguments */
int esq_cache_trace(int nslots, int nlayers, int nexperts, double freq_weight, const int32_t *ops, int nops, int32_t *res,
                    int64_t *slots_out, uint64_t *stats_out);

/* the same trace driven through the reference's own es_cache_init / find / claim (oracle/esq_cache_ref.c, built with the
 * reference's src/es_cache.c and src/es_io.c into oracle/_ref/libesref_cache.so) */
int esref_cache_trace(int nslots, int nlayers, int nexperts, double freq_weight, const int32_t *ops, int nops,
                      int32_t *res, int64_t *slots_out, uint64_t *stats_out);

#ifdef __cplusplus
}
#endif
#endif
