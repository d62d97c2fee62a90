/*
 * es_hip_quant.h — C ABI of the MI355X (gfx950) quantized matrix-product library (libes_hip_quant.so).
 *
 * What it replaces. The reference engine (Tharunmaks/Stream-, "ExpertStream") computes every weight x activation product on
 * the CPU through three headers:
 *   src/es_quant.h:25-49    es_act_prepare / es_matvec / es_matvec_multi / es_row_bytes / es_quant_supported
 *   src/es_q2k.h:24-86      the Q2_K / Q8_K block structs, es_quantize_q8_K, es_matvec_q2_K
 *   src/es_compute.h:10-25  the thread pool that fans a queue of row jobs out to cores (driven by src/es_engine.c:144-186)
 * This library computes the same products on one MI355X for the GGUF formats Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K and Q6_K against
 * the reference's Q8 activations, with the packed weight blocks kept byte-for-byte in device memory.
 *
 * Results. The integer block dots are exact. The fp32 epilogue is evaluated in the reference's own order, so outputs are
 * bit-identical to the reference's CPU kernels in the selected build flavour (es_hip_set_order):
 *   ES_HIP_ORDER_X86_CONTRACT  the reference's default x86 build (clang, -ffp-contract=on; Makefile:1-4) — the default here
 *   ES_HIP_ORDER_X86_STRICT    the same AVX2 kernels built by gcc -std=c11 (no contraction)
 *   ES_HIP_ORDER_SCALAR        the scalar mv_* kernels (ES_NO_AVX2=1, src/es_quant.c:1013-1175)
 * Q5_K has no AVX2 kernel in the reference (its x86 build runs the scalar mv_q5_K, without FMA), so all three orders give
 * the same Q5_K results.
 *
 * Conventions (same as the reference): every buffer belongs to the caller; W points at row 0 of a row-major matrix whose row
 * stride is es_hip_row_bytes(type, cols); outputs are written only for rows [r0, r1), at absolute row indices, activation q's
 * result at y + q * ystride. Activation blocks are the reference's: Q8_0 (36 bytes: float d, int8 qs[32]) for Q4_0/Q5_0/Q8_0 and
 * Q8_K (292 bytes: float d, int8 qs[256], int16 bsums[16]) for Q2_K/Q3_K/Q4_K/Q5_K/Q6_K.
 *
 * Errors. The reference's entry points return void and cannot fail. Here the device-pointer entry points return 0 on success
 * and a negative ES_HIP_E* code otherwise; es_hip_last_error() describes the most recent failure. There is no CPU fallback:
 * without a usable gfx950 device every compute call fails with ES_HIP_ENODEV.
 *
 * Streams are passed as void* (a hipStream_t; NULL means the null stream) so this header needs no HIP include.
 */
#ifndef ES_HIP_QUANT_H
#define ES_HIP_QUANT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids of the formats computed here (reference src/es_quant.h:15-22) */
enum {
    ES_HIP_Q4_0 = 2, ES_HIP_Q5_0 = 6, ES_HIP_Q8_0 = 8, ES_HIP_Q2_K = 10, ES_HIP_Q3_K = 11, ES_HIP_Q4_K = 12, ES_HIP_Q5_K = 13,
    ES_HIP_Q6_K = 14
};

/* fp32 epilogue order, see the header comment */
enum { ES_HIP_ORDER_X86_CONTRACT = 0, ES_HIP_ORDER_X86_STRICT = 1, ES_HIP_ORDER_SCALAR = 2 };

/* status codes */
enum {
    ES_HIP_OK = 0,
    ES_HIP_ENODEV = -1,   /* no usable gfx950 device */
    ES_HIP_EINVAL = -2,   /* bad type, shape, stride, alignment or pointer */
    ES_HIP_ERUNTIME = -3, /* a HIP runtime call failed */
    ES_HIP_ENOMEM = -4,
    ES_HIP_EBUSY = -5     /* expert cache: every slot is loading or protected (the reference exits "expert cache too small") */
};

/* Activation blocks and the prepared-activation record: the same byte layouts as the reference's es_blk_q80
 * (src/es_quant.h:31), es_block_q8_K (src/es_q2k.h:31-38) and es_act (src/es_quant.h:32-37). */
typedef struct { float d; int8_t qs[32]; } es_hip_blk_q80;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } es_hip_block_q8_K;
typedef struct {
    const float *x;
    es_hip_block_q8_K *q8;   /* NULL unless cols % 256 == 0 */
    es_hip_blk_q80 *q80;     /* NULL unless cols % 32 == 0 */
    int cols;
} es_hip_act;

/* ---- library state ------------------------------------------------------------------------------------------------ */
int         es_hip_available(void);          /* 1 if a gfx950 device is usable (initialises the library once) */
const char *es_hip_last_error(void);         /* text of the most recent failure ("" if none); per thread */
const char *es_hip_device_name(void);        /* gcnArchName of the device in use, or "" */
int         es_hip_set_order(int order);     /* select the epilogue order; returns the previous one, or ES_HIP_EINVAL */
int         es_hip_get_order(void);

/* ---- format facts (reference src/es_quant.h:24-26, 48-49; src/es_quant.c:39-73) ------------------------------------- */
int    es_hip_quant_supported(uint32_t type);   /* 1 for the eight formats above */
size_t es_hip_row_bytes(uint32_t type, int cols);

/* ---- device memory helpers (plumbing for callers without their own HIP allocator) ---------------------------------- */
void *es_hip_malloc(size_t bytes);                            /* NULL on failure */
int   es_hip_free(void *dev);
/* page-locked host memory (hipHostMalloc): expert slabs staged here load into the expert cache asynchronously at the
 * link's full rate; pageable sources are staged by the runtime */
void *es_hip_host_alloc(size_t bytes);                        /* NULL on failure */
int   es_hip_host_free(void *host);
int   es_hip_memcpy_h2d(void *dev, const void *host, size_t bytes);
int   es_hip_memcpy_d2h(void *host, const void *dev, size_t bytes);
int   es_hip_memcpy_d2d(void *dst, const void *src, size_t bytes);
int   es_hip_memset(void *dev, int value, size_t bytes);
int   es_hip_synchronize(void);

/* ---- products on device memory --------------------------------------------------------------------------------------- */
/* es_matvec (src/es_quant.h:44-45) on device memory: y[r] for r in [r0, r1). act: the activation blocks of one input. */
int es_hip_matvec_dev(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, float *y, void *stream);
/* es_matvec_multi (src/es_quant.h:46-47) on device memory: na activations, activation q's blocks at act + q * astride bytes,
 * outputs at y + q * ystride. Bit-identical to na calls of es_hip_matvec_dev (the reference's es_mtest invariant). */
int es_hip_matvec_multi_dev(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, size_t astride, int na,
                            float *y, size_t ystride, void *stream);
/* es_hip_matvec_multi_dev without any device allocation. No counterpart in the reference: it is for callers that cannot
 * allocate (tight serving loops, harnesses that forbid hipMalloc). The job tables and the activation pre-pass workspace
 * live in a static device array of ES_HIP_NOALLOC_SCRATCH_BYTES per device, held until the process ends; a product that
 * needs more fails with ES_HIP_EINVAL (es_hip_matvec_multi_dev serves it). Every call on a device shares that array: calls
 * that overlap on one device (different streams, or threads) race; calls ordered on one stream do not. Not for HIP graph
 * capture: the tables are copied from host memory at the call, so a capturing stream is refused with ES_HIP_EINVAL.
 * Same outputs as es_hip_matvec_multi_dev, bit for bit. */
#define ES_HIP_NOALLOC_SCRATCH_BYTES (32u << 20)
int es_hip_matvec_multi_dev_noalloc(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, size_t astride,
                                    int na, float *y, size_t ystride, void *stream);

/* The float path of es_matvec (src/es_quant.c:1941-1944) on device memory: an activation prepared without blocks
 * (es_act_prepare without a Q8_K buffer, with its Q8_0 arena exhausted, or under ES_FLOAT_ACT; src/es_quant.c:499-512) is
 * multiplied by dequantizing each weight row (es_dequant_row) and taking dot_f32 against its floats (src/es_quant.c:514-526:
 * four running sums over i mod 4, products and sums rounded separately, then (s0 + s1) + (s2 + s3)). x: na activations of
 * cols floats, activation q at x + q * xstride floats (0: cols); y as es_hip_matvec_multi_dev. W at 2-byte alignment, x and
 * y at 4. The same floats as the reference's in every build (dot_f32 has no FMA target on x86). No row length limit. */
int es_hip_matvec_float_dev(uint32_t type, const void *W, int cols, int r0, int r1, const float *x, size_t xstride, int na,
                            float *y, size_t ystride, void *stream);

/* One queued product: the reference engine's mv_job (src/es_engine.c:144) with device pointers. rows are [0, rows). */
typedef struct {
    uint32_t type;
    int rows, cols;
    const void *W;      /* device, row 0 */
    const void *act;    /* device activation blocks, activation q at act + q * astride bytes */
    size_t astride;     /* bytes; 0 means packed (cols / block elements * block bytes) */
    int nb;             /* number of activations (the reference's nb) */
    float *y;           /* device, activation q's outputs at y + q * ystride */
    size_t ystride;     /* floats */
} es_hip_job;

/* run_jobs (src/es_engine.c:177-186): every queued product in as few launches as possible (one per format). */
int es_hip_run_jobs(const es_hip_job *jobs, int njobs, void *stream);

/* A prepared job batch: the job table is uploaded once, so a launch costs only the kernel dispatches. The jobs' pointers
 * are captured when the plan is made; the memory they point to may change between runs. A plan with rows past
 * ES_HIP_MAX_COLS_* keeps one batch per phase of column pieces (run in order) and the lane chains between them, so two
 * runs of one such plan must not overlap (runs on one stream never do). */
typedef struct es_hip_plan es_hip_plan;
es_hip_plan *es_hip_plan_create(const es_hip_job *jobs, int njobs);   /* NULL on failure */
int          es_hip_plan_run(es_hip_plan *plan, void *stream);
void         es_hip_plan_destroy(es_hip_plan *plan);

/* ---- drop-ins on host memory (same prototypes and meaning as the reference) ------------------------------------------ */
/* Weights registered here stay resident on the device, byte-for-byte; es_hip_matvec / es_hip_matvec_multi find a W inside a
 * registered range and use the device copy. Unregistered weights are uploaded for the one call. Re-register (or
 * es_hip_update) after the host bytes change (e.g. an expert cache slot that received another expert). */
int es_hip_register(const void *host, size_t bytes);
int es_hip_update(const void *host);
int es_hip_unregister(const void *host);
/* es_matvec / es_matvec_multi (src/es_quant.h:44-47): host W, host activations (a->q80 for Q4_0/Q5_0/Q8_0, a->q8 for the
 * K-quants; an activation without them takes the float path from a->x, as in the reference), host y. Synchronous. The
 * scratch argument is unused (kept for the prototype). They clear es_hip_last_error() on entry; on failure y is left
 * untouched and es_hip_last_error() says why (the reference's void prototype has no other error channel). Row length:
 * any multiple of the block size, as in the reference. Rows past ES_HIP_MAX_COLS_32 columns for the 32-element formats
 * (Q4_0, Q5_0, Q8_0) or ES_HIP_MAX_COLS_256 for the K-quants (where one row's float terms stop fitting a workgroup's LDS
 * in the decode kernel) run as column pieces of at most that length, one launch each in stream order, every piece
 * continuing the sums where the previous one stopped (the same outputs; the AVX2 order's lane sums between pieces take a
 * stream-ordered allocation). This holds for es_hip_matvec[_multi], es_hip_matvec[_multi]_dev, es_hip_run_jobs[_host]
 * and es_hip_plan_*; es_hip_matvec_multi_dev_noalloc (whose scratch is sized once) and the dense and MoE layers refuse
 * longer rows with ES_HIP_EINVAL. */
#define ES_HIP_MAX_COLS_32 131072
#define ES_HIP_MAX_COLS_256 1048576
void es_hip_matvec(uint32_t type, const void *W, int cols, int r0, int r1, const es_hip_act *a, float *y, float *scratch);
void es_hip_matvec_multi(uint32_t type, const void *W, int cols, int r0, int r1, const es_hip_act *a, int na, float *y,
                         size_t ystride, float *scratch);
/* es_q2k.h's Q2_K drop-ins (src/es_q2k.h:78-86): es_matvec_q2_K over host rows of es_block_q2_K and one activation's
 * Q8_K blocks (xq, cols / 256 of them), y[r] for r in [r0, r1), in the reference's portable order (sumf += dall * isum -
 * dmin * summs per block, no fusion) whatever es_hip_set_order says, as es_matvec_q2_K computes on every build; the
 * kernel name, and a scalar switch kept for A/B scripts (the reference's scalar and portable dots give the same floats). */
void        es_hip_matvec_q2_K(const void *W, int cols, int r0, int r1, const void *xq, float *y);
const char *es_hip_q2k_kernel_name(void);
void        es_hip_q2k_force_scalar(int on);
/* The engine's queued job on host memory: mv_job (src/es_engine.c:144) field for field. */
typedef struct {
    uint32_t type;
    const void *w;          /* host weights, row 0 (registered ranges are used in place) */
    int rows, cols;
    const es_hip_act *a;    /* nb prepared activations */
    float *y;               /* host outputs, activation q's row r at y[q * ys + r] */
    int nb;
    size_t ys;
} es_hip_host_job;
/* run_jobs (src/es_engine.c:177-186) for a queue on host memory: activations go up in one copy, every job runs in one
 * launch per format (activations without blocks in the float path's launch, from a->x), outputs come back in one copy.
 * Synchronous, like the reference's. Returns 0 or ES_HIP_E*. */
int es_hip_run_jobs_host(const es_hip_host_job *jobs, int njobs);

/* ---- dense FFN: dense_n (src/es_engine.c:957-972) ------------------------------------------------------------------- */
/* The SwiGLU FFN of N tokens on the device, as dense_n computes it for a layer without LoRA or the situ activation:
 *   gate and up products into gu, token t's gate at gu[t * 2 ff + i], up at gu[t * 2 ff + ff + i] (the engine's BGU);
 *   h = g / (1 + expf(-g)) * u, prepared as es_act_prepare does for the down type (Q8_K for K-quants, Q8_0 otherwise) into
 *   hq, token t's ff / 256 Q8_K (or ff / 32 Q8_0) blocks packed at hq + t * (that many blocks' bytes);
 *   down products into out, token t's n outputs at out + t * ostride floats.
 * Weights: device pointers to row 0 (gate, up: ff rows of n; down: n rows of ff). x: the N tokens' activation blocks
 * (Q8_K for K-quant gate/up, Q8_0 otherwise), token t at x + t * xstride bytes (0: packed). gu (N * 2 ff floats) and hq
 * are the caller's device workspaces. Stream-ordered; bit-identical to dense_n's outputs (and to its BGU rows). */
int es_hip_dense_ffn_dev(uint32_t gate_type, const void *wg, uint32_t up_type, const void *wu, uint32_t down_type,
                         const void *wd, int n, int ff, int N, const void *x, size_t xstride, float *gu, void *hq,
                         float *out, size_t ostride, void *stream);

/* ---- MoE expert FFN: the expert part of moe_n (src/es_engine.c:848-942) --------------------------------------------- */
/* The routed experts of one layer, resident on the device. Experts whose pointers are NULL must not be routed. */
typedef struct {
    uint32_t gate_type, up_type, down_type;   /* GGML types; gate and up take the same kind of activation blocks */
    int n;                                    /* model width: gate/up cols, down rows */
    int ff;                                   /* expert width: gate/up rows, down cols */
    int n_exp;
    const void *const *gate;                  /* host arrays of n_exp device pointers, row 0 of expert e's matrix */
    const void *const *up;
    const void *const *down;
} es_hip_moe;
/* The expert FFN of N tokens routed by route() (src/es_engine.c:744-835): token t's k[t] <= kmax experts are
 * sel[t * kmax + j] with weights w[t * kmax + j] (host arrays). x: device activation blocks of the N tokens (Q8_K for a
 * K-quant gate/up, Q8_0 for Q4_0/Q5_0/Q8_0), token t at x + t * xstride bytes (0: packed). out: device, token t's n outputs at
 * out + t * ostride floats. In stream order on the device:
 *   the pairs (t, j) are grouped by expert in order of first use (:871-888);
 *   gate and up products of every pair into [pair][2 ff] (:899-903), one launch per format;
 *   h = g / (1 + expf(-g)) * u, requantized as es_act_prepare does for the down type (:913-914);
 *   down products into [pair][n] (:916-918);
 *   out[t] = sum over j of w[t][j] * y[pair (t, j)], in j order from 0 (:925-932).
 * Results are bit-identical to moe_n's expert part for a model without expert biases, latent projection or the gpt-oss /
 * situ activations. es_hip_moe_ffn is synchronous. */
int es_hip_moe_ffn(const es_hip_moe *m, int N, const int *k, const int *sel, const float *w, int kmax, const void *x,
                   size_t xstride, float *out, size_t ostride, void *stream);
/* The MoE layer from the router's logits (device, token t's n_exp logits at logits + t * lstride floats, 0: packed):
 * route() for softmax gating on the device (es_hip_route_softmax_dev: top k, norm_topk), the k choices and weights of every
 * token copied to the host for the grouping, then es_hip_moe_ffn with them. sel_out / w_out (host, N * k each, optional)
 * receive the routing. Synchronous. */
int es_hip_moe_ffn_logits(const es_hip_moe *m, int N, const float *logits, size_t lstride, int k, int norm_topk,
                          const void *x, size_t xstride, float *out, size_t ostride, int *sel_out, float *w_out,
                          void *stream);
/* The same as a prepared plan: grouping, job tables and workspace are made once; runs are asynchronous on `stream`. The
 * routing (k, sel, w) is captured at creation; x, out and the expert bytes may change between runs. */
typedef struct es_hip_moe_plan es_hip_moe_plan;
es_hip_moe_plan *es_hip_moe_plan_create(const es_hip_moe *m, int N, const int *k, const int *sel, const float *w, int kmax,
                                        const void *x, size_t xstride, float *out, size_t ostride);   /* NULL on failure */
int    es_hip_moe_plan_run(es_hip_moe_plan *plan, void *stream);
void   es_hip_moe_plan_destroy(es_hip_moe_plan *plan);

/* ---- device-routed MoE layer: no allocation, no host round trip per call -------------------------------------------- */
typedef struct es_hip_moe_ctx es_hip_moe_ctx;
/* A context for one layer's expert set (the es_hip_moe arrays are copied; the expert weights must stay resident and
 * unrouted experts may be NULL) and up to max_tokens tokens of k choices each (max_tokens * k <= 16384, k <= 64):
 * every buffer and job table of a layer is allocated here, once. NULL on failure (es_hip_last_error). */
es_hip_moe_ctx *es_hip_moe_ctx_create(const es_hip_moe *m, int max_tokens, int k);
/* moe_n's expert part (src/es_engine.c:848-942) for N <= max_tokens tokens whose k choices and weights are in device
 * memory (sel: int [N][k], valid expert ids; w: float [N][k]): the grouping of :871-888 (distinct experts in order of
 * first use, each expert's rows in choice order) and the job tables are computed on the device, then gate/up, SwiGLU +
 * requantization, down and the combine run as in es_hip_moe_ffn, with the same outputs bit for bit. x / out as for
 * es_hip_moe_ffn (device). Stream-ordered and asynchronous: no allocation, no copy to or from the host, no wait. Calls on
 * one context share its buffers: order them on one stream (or synchronise between streams). */
int es_hip_moe_ctx_run(es_hip_moe_ctx *c, int N, const int *sel, const float *w, const void *x, size_t xstride, float *out,
                       size_t ostride, void *stream);
/* The layer from the router's logits (device, token t's n_exp logits at logits + t * lstride floats, 0: packed): route()
 * for softmax gating on the device (as es_hip_route_softmax_dev), then es_hip_moe_ctx_run's work. sel_out / w_out
 * (device, N * k each, optional) receive the routing. Asynchronous as es_hip_moe_ctx_run. */
int es_hip_moe_ctx_run_logits(es_hip_moe_ctx *c, int N, const float *logits, size_t lstride, int norm_topk, const void *x,
                              size_t xstride, float *out, size_t ostride, int *sel_out, float *w_out, void *stream);
void es_hip_moe_ctx_destroy(es_hip_moe_ctx *c);

/* ---- diagnostics ----------------------------------------------------------------------------------------------------- */
/* The integer part of every (row, block) of rows [0, rows) against one activation, as the reference's kernels form it:
 * dots[r * nb + b] = the block's integer dot (Q4_0/Q5_0/Q8_0: the sum of the eight AVX2 lane sums; Q4_K: dot; Q6_K: tot;
 * Q2_K: isum) and aux[r * nb + b] = Q4_K mins or Q2_K summs (0 for the others). nb = cols / block elements. Device memory. */
int es_hip_block_ints_dev(uint32_t type, const void *W, int cols, int rows, const void *act, int32_t *dots, int32_t *aux,
                          void *stream);
/* Kernel choice by batch size (results are identical either way; each returns the previous value):
 *   es_hip_set_mfma_min_batch: Q4_K products with at least n activations run on the matrix-core kernel that stages weights
 *     and activations through LDS (default 8; batches up to 64 use 16-, 32- or 64-wide activation tiles);
 *   es_hip_set_small_batch_min: other Q2_K / Q4_K products with at least n activations run on the small-batch matrix-core
 *     kernel that streams weights through registers (default 8);
 * the rest go to the vector kernels. n <= 0 switches the kernel off (here and below). */
int es_hip_set_mfma_min_batch(int n);
int es_hip_set_small_batch_min(int n);
/* Workgroup tile of the matrix-core kernel for products of at least 128 activations: bm rows x bn activations on `waves`
 * waves, one of 128 x 128 x 8, 128 x 64 x 8, 64 x 64 x 8, 64 x 64 x 4, 32 x 128 x 4; (0, 0, 0) restores the automatic
 * choice (128 x 128 when that gives every CU a workgroup, else 64 x 64 x 8). Returns ES_HIP_OK or ES_HIP_EINVAL. */
int es_hip_set_mfma_tile(int bm, int bn, int waves);
/* Q4_0 / Q5_0 / Q8_0 products with at least n activations run on the batched kernel (one lane per row and activation) instead of
 * the vector kernel (default 2). */
int es_hip_set_batched32_min(int n);
/* Of those, products with at least n activations run on the batched matrix-core kernel (one int8 MFMA per block forms the
 * eight AVX2 lane sums of 4 rows x 32 activations; default 2); the others on the one-lane-per-output kernel. */
int es_hip_set_batched32_mfma_min(int n);
/* Q6_K products with at least n activations (and an even number of superblocks per row) run on the Q6_K matrix-core
 * kernel (default 16). */
int es_hip_set_q6k_mfma_min_batch(int n);
/* Q2_K products with at least n activations run on the Q2_K LDS-staged matrix-core kernel (default 2); below that, or
 * with it off, the small-batch kernel (es_hip_set_small_batch_min) or the vector kernel. */
int es_hip_set_q2k_mfma_min_batch(int n);
/* Q4_K products with at least n activations (default 32) and at least es_hip_set_direct_mfma_min_tiles tiles run on the
 * direct-activation matrix-core kernel: it reads the activations' Q8_K rows itself (no pre-pass) in tiles of 64 rows x 128
 * activations. Otherwise, or with it off (n <= 0), the pre-pass kernels of es_hip_set_mfma_min_batch /
 * es_hip_set_small_batch_min or the vector kernel. Results are identical on every kernel. Returns the previous value. */
int es_hip_set_direct_mfma_min_batch(int n);
/* The direct-activation kernel's minimum tile count per product (default 128; twice that for rows longer than 4096):
 * below it a product has too few workgroups to fill the device. Returns the previous value. */
int es_hip_set_direct_mfma_min_tiles(int n);
/* Q5_K products with at least n activations (default 8) run on the direct-activation matrix-core kernel (a third int8
 * plane for the fifth bit); below it, or with it off (n <= 0), on the vector kernel. Results are identical on both. Returns
 * the previous value. */
int es_hip_set_q5k_mfma_min_batch(int n);
/* Q3_K products with at least n activations (default 8) run on the direct-activation matrix-core kernel (two int8 planes of
 * the signed codes against the split scales); below it, or with it off (n <= 0), on the vector kernel. Results are
 * identical on both. Returns the previous value. */
int es_hip_set_q3k_mfma_min_batch(int n);
/* Q2_K products with 2 to n activations (default 64) and rows of at most 4096 columns run on the expert-sized matrix-core
 * kernel: it copies the activations' Q8_K rows into LDS once per tile of 256 rows x 32 activations and streams the weights
 * (no pre-pass). Larger batches, or all with n < 2, run on the LDS-staged Q2_K kernel of es_hip_set_q2k_mfma_min_batch.
 * Results are identical on every kernel. Returns the previous value. */
int es_hip_set_q2k_expert_max_batch(int n);
/* A MoE layer whose gate and up projections are Q2_K, whose down projection takes Q8_K activations and whose batches run
 * on the expert-sized kernel computes, with on != 0 (the default), the gate and up rows of each block of 256 in one
 * workgroup and writes SwiGLU(gate, up) as that block's Q8_K activation directly (no float gate/up buffer, no SwiGLU
 * launch); with 0, gate and up run as two jobs and a separate SwiGLU + Q8_K pass follows. Results are identical on both.
 * Applies to plans and contexts created after the call. Returns the previous setting. */
int es_hip_set_moe_gated(int on);
/* Q4_0 / Q5_0 / Q8_0 batches that run on the matrix cores (es_hip_set_batched32_mfma_min) and have rows of at most 4096
 * columns use, with on != 0 (the default), the kernel that copies the activations' Q8_0 rows into LDS once per tile of
 * 16 rows x 32 activations (no pre-pass); with 0, the one that reads them from a pre-pass layout. Results are identical
 * on both. Returns the previous setting. */
int es_hip_set_batched32_direct(int on);
/* A Q6_K product on the matrix cores that is alone in its launch, has one tile of activations (at most 64) and short
 * rows (at most 5 superblocks at 64 activations, 11 at 32, 22 at 16) runs, with on != 0 (the default), as a persistent
 * launch: one workgroup per CU copies the activations into LDS once and streams its row tiles back to back. Results
 * are identical either way. Returns the previous setting. */
int es_hip_set_q6k_persistent(int on);
/* Q4_K and Q3_K products that take the direct-activation kernel and have an even number (at least 2) of superblocks per
 * row, with no gathered activations, run, with on != 0, in one persistent launch per format, each workgroup computing a
 * host-scheduled list of tiles with its loads running ahead across tile boundaries, in one of two forms: two workgroups
 * per CU (tiles of 64 rows x 128 or 64 activations), or, for Q4_K, one workgroup of 8 waves per CU (tiles of 64 rows x
 * 128 activations; four waves stage the activations and the unpacked weights in LDS for the four that run the matrix
 * cores). on = 1 (the default) picks the second form for Q4_K launches of at least 4 tiles of 128 activations per CU
 * (config 2's three prefill products in one launch), the first otherwise; on = 2 takes the second for every Q4_K
 * launch, on = 3 the first for every launch. Q4_K products of this kind take the persistent launch at any tile count
 * (config 2's 2048 x 8192 down product shares the launch with gate and up). Results are identical in every form.
 * Returns the previous setting. */
int es_hip_set_direct_persistent(int on);
/* Q5_K and Q3_K products on the direct-activation kernel that would have fewer than 256 tiles of 64 rows x 128
 * activations run, with on != 0 (the default) and at least 64 activations, in tiles of 64 activations (twice the
 * workgroups: config 2's down product at T = 512 in those formats). Results are identical either way. Returns the
 * previous setting. */
int es_hip_set_direct_mfma_tok64(int on);
/* ---- activation preparation on the device ---------------------------------------------------------------------------
 * es_act_prepare (src/es_quant.c:499-512) for `rows` rows of `cols` fp32 values in device memory: q80 (when non-NULL;
 * cols % 32 == 0) receives cols/32 Q8_0 blocks per row exactly as quantize_q80 (src/es_quant.c:489-497) writes them, q8k
 * (when non-NULL; cols % 256 == 0) cols/256 Q8_K blocks per row as es_quantize_q8_K (src/es_q2k.c:102-125), bsums
 * included. Float strides are in floats, block strides in bytes; 0 means packed. Stream-ordered; nothing is allocated. */
int es_hip_act_prepare_dev(const float *x, size_t xstride, int rows, int cols, void *q80, size_t q80_stride, void *q8k,
                           size_t q8k_stride, void *stream);
/* rmsnorm (src/es_engine.c:189-194: the sum of squares in double in element order, s = (float)(1 / sqrt(ss / cols + eps)),
 * xn = x * s * w) fused with the same preparation of xn (the engine's `prep` after its rmsnorm, src/es_engine.c:1284-1292).
 * w may be NULL (weights 1); xn (optional) receives the normalised rows. cols: a multiple of 32, at most 16384. */
int es_hip_rmsnorm_prepare_dev(const float *x, size_t xstride, const float *w, float eps, int rows, int cols, float *xn,
                               size_t xn_stride, void *q80, size_t q80_stride, void *q8k, size_t q8k_stride, void *stream);
/* SwiGLU of gate|up rows as dense_n / moe_n lay them out (gate at [r][0, ff), up at [r][ff, 2 ff); src/es_engine.c:957-972,
 * 913-914), h = g / (1 + expf(-g)) * u, fused with the preparation of h; h (optional) receives the values. */
int es_hip_swiglu_prepare_dev(const float *gu, size_t gu_stride, int rows, int ff, float *h, size_t h_stride, void *q80,
                              size_t q80_stride, void *q8k, size_t q8k_stride, void *stream);
/* es_dequant_row (src/es_quant.h:28, src/es_quant.c:425-476) on the device: n weights (a whole number of blocks, any byte
 * alignment) of src to fp32 at dst, each by its format's formula in the reference's operation order (bit-identical). */
int es_hip_dequant_row_dev(uint32_t type, const void *src, float *dst, long n, void *stream);
/* route() for softmax gating on the device (src/es_engine.c:744-835, its GATE_SOFTMAX path: no gate bias, selection bias,
 * expert groups, cache bonus or top-k override): for each of ntok tokens, the softmax of its n_exp logits (expf(l - max),
 * summed in expert order, divided), the k largest probabilities by repeated argmax with ties to the lowest expert into
 * sel[t * kmax + j] / w[t * kmax + j], and with norm_topk the weights divided by max(their sum, 2^-14). The results are the
 * reference's bit for bit, so es_hip_moe_ffn / es_hip_moe_plan_create can take them as they are. Device pointers;
 * n_exp <= 1024, k <= 64, k <= n_exp, k <= kmax; lstride in floats (0: n_exp). */
int es_hip_route_softmax_dev(const float *logits, size_t lstride, int ntok, int n_exp, int k, int norm_topk, int *sel, float *w,
                             int kmax, void *stream);
/* The MoE SwiGLU alone on n device floats: h[i] = g[i] / (1 + expf(-g[i])) * u[i] as src/es_engine.c:913 computes it. */
int es_hip_swiglu_dev(const float *g, const float *u, float *h, long n, void *stream);
/* Average kernel time in milliseconds of `iters` back-to-back runs of a plan, measured with HIP events on `stream`
 * (after `warmup` untimed runs). */
double es_hip_plan_time_ms(es_hip_plan *plan, int warmup, int iters, void *stream);
/* The same for a step made of several prepared batches: each iteration runs the np plans, then the nm MoE plans, in order.
 * Returns milliseconds per iteration, or a negative value on failure. */
double es_hip_step_time_ms(es_hip_plan *const *plans, int np, es_hip_moe_plan *const *moe, int nm, int warmup, int iters,
                           void *stream);

/* ---- Device expert cache: the reference's hot-expert RAM cache (src/es_cache.h:1-56, src/es_cache.c:1-71) with its slots
 * in HBM, so expert products read their weights from device memory. Same slot policy: nslots equal slots of slot_bytes,
 * keyed by (layer, expert); a claim takes the first empty slot, else evicts the lowest last_use + freq_weight * min(uses,
 * 16) among slots not loading and not protected (protect_until >= step), the first of equal scores. Loads are
 * hipMemcpyAsync copies on the caller's stream; a slot stays LOADING until its copy has finished (a HIP event), and a
 * loading slot is never evicted: like load_experts, which waits for its reads before it returns, wait for a call's slots
 * (es_hip_cache_wait, or a stream synchronisation) before claims that may need them, or a cache of in-flight copies
 * answers ES_HIP_EBUSY. slot_bytes = 0 creates a bookkeeping-only cache (no device memory, no GPU needed). One
 * cache is used from one host thread. */
typedef struct es_hip_cache es_hip_cache;
enum { ES_HIP_SLOT_EMPTY = 0, ES_HIP_SLOT_LOADING = 1, ES_HIP_SLOT_READY = 2 };   /* ES_SLOT_*, src/es_cache.h:19 */
typedef struct {   /* the policy fields of es_slot (src/es_cache.h:21-30) */
    int layer, expert, state, prefetched;
    uint64_t last_use;
    uint32_t uses;
    uint64_t protect_until;
} es_hip_slot_info;
typedef struct {   /* es_cache's counters (src/es_cache.h:40-41) and its step */
    uint64_t hits, misses, prefetch_issued, prefetch_used, prefetch_wasted, evictions, step;
} es_hip_cache_stats;
/* Where an expert's bytes are on the host: part r (gate, up, down) of expert e is bytes[r] bytes at base[r] + e * stride[r]
 * (a 3-D GGUF slab: stride = the per-expert size, src/es_engine.c:663-664), placed at offset[r] inside the slot (the
 * reference's XOFF). Parts with bytes[r] = 0 are skipped. */
typedef struct {
    const void *base[3];
    uint64_t stride[3], bytes[3], offset[3];
} es_hip_expert_src;

/* es_cache_init / es_cache_free (src/es_cache.h:44-46) */
int  es_hip_cache_create(es_hip_cache **out, int nslots, size_t slot_bytes, int nlayers, int nexperts, double freq_weight);
void es_hip_cache_destroy(es_hip_cache *c);
/* es_cache_find (src/es_cache.h:48-49): the slot holding (layer, expert), or -1 */
int  es_hip_cache_find(const es_hip_cache *c, int layer, int expert);
/* es_cache_claim (src/es_cache.h:51-54): pick a victim, map it to (layer, expert) in state LOADING; the slot, or
 * ES_HIP_EBUSY when every slot is loading or protected. (layer, expert) must not be cached already. */
int  es_hip_cache_claim(es_hip_cache *c, int layer, int expert);
/* device address of a slot (NULL for a bookkeeping-only cache) */
void *es_hip_cache_slot_ptr(const es_hip_cache *c, int slot);
/* copy bytes from host memory into the slot at offset, asynchronously on stream (es_submit / read_expert_part) */
int  es_hip_cache_load(es_hip_cache *c, int slot, size_t offset, const void *host, size_t bytes, void *stream);
/* wait for the slot's copies, then mark it READY (es_wait / gio_wait) */
int  es_hip_cache_wait(es_hip_cache *c, int slot);
/* advance the layer-step counter (C.step++) */
int  es_hip_cache_step(es_hip_cache *c);
/* load_experts for layer (src/es_engine.c:665-708): step += 1; for each selected expert a hit (clearing `prefetched`,
 * counted as a used prefetch) or a miss that claims a slot and loads the expert's parts from src (NULL: bookkeeping only);
 * then uses += 1, last_use = step, protect_until = step. slots[j] receives expert sel[j]'s slot (-1 where no slot was
 * free: the call then returns ES_HIP_EBUSY after handling the others). */
int  es_hip_cache_acquire(es_hip_cache *c, int layer, const int *sel, int k, const es_hip_expert_src *src, int *slots,
                          void *stream);
/* the router's prefetch of one expert (src/es_engine.c:606-611): *slot = the claimed slot, marked prefetched and protected
 * for 3 more steps, its parts loading from src (NULL: bookkeeping only); *slot = -1 and ES_HIP_OK when the expert is cached
 * already; ES_HIP_EBUSY (*slot = -1) when no slot is free (the reference then stops prefetching) */
int  es_hip_cache_prefetch(es_hip_cache *c, int layer, int expert, const es_hip_expert_src *src, void *stream, int *slot);
int  es_hip_cache_slot_info(const es_hip_cache *c, int slot, es_hip_slot_info *out);
int  es_hip_cache_get_stats(const es_hip_cache *c, es_hip_cache_stats *out);

#ifdef __cplusplus
}
#endif
#endif
