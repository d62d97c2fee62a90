/*
 * esref_route / esref_rmsnorm — the reference engine's own route() and rmsnorm() (src/es_engine.c:744-835, 189-194),
 * reached by compiling src/es_engine.c into this translation unit where it lies under the reference tree (its functions
 * are static). TEST INFRASTRUCTURE ONLY: built by oracle/Makefile (`make ref`) with the rest of the reference's engine
 * sources (src/es_graft.c, es_gguf.c, es_quant.c, es_tok.c, es_regex.c, es_fetch.c and its CORE set, the same list its own
 * Makefile links into es_chat / es_mtest) into oracle/_ref/libesref_engine.so; used by tests/golden/make_golden.py to
 * write the routing and rmsnorm golden vectors. Nothing of the reference is copied here.
 *
 * Only the model fields route() reads are set: one layer with no router bias and no selection bias, softmax gating,
 * n_exp, n_used, norm_topk; no expert groups, no weight scale. The engine's run-time options that change the choice
 * (TOPK, CACHE_ROUTE, SKIP_THR, REMOTE) keep their defaults (off), as in a plain local run.
 */
#include "es_engine.c"

static layer esref_layer0;

/* route() over `ntok` tokens of `ne` logits each (rows `ne` floats apart): choices and weights into rows of `k`.
 * Returns the k route() returned for the last token (the same for every token here), or -1 on bad sizes. */
int esref_route(int ntok, int ne, int k, int norm_topk, const float *logits, int *sel, float *w) {
    if (ne < 1 || ne > 1024 || k < 1 || k > ne || k > MAXK) return -1;
    memset(&esref_layer0, 0, sizeof esref_layer0);
    M.L = &esref_layer0;
    M.n_exp = ne;
    M.n_used = k;
    M.gating = GATE_SOFTMAX;
    M.norm_topk = norm_topk;
    M.n_group = 0;
    M.n_group_used = 0;
    M.w_scale = 0.0f;
    float r[1024];
    int got = -1;
    for (int t = 0; t < ntok; t++) {
        memcpy(r, logits + (size_t)t * ne, sizeof(float) * (size_t)ne);   /* route() overwrites its logits */
        got = route(0, r, sel + (size_t)t * k, w + (size_t)t * k);
    }
    return got;
}

/* rmsnorm() of `rows` rows of n floats (w may be null: unweighted) */
void esref_rmsnorm(float *o, const float *x, const float *w, int rows, int n, float eps) {
    for (int i = 0; i < rows; i++) rmsnorm(o + (size_t)i * n, x + (size_t)i * n, w, n, eps);
}
