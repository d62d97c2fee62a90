/*
 * esq_oracle — CPU restatement of ExpertStream's quantized matrix-product path.
 *
 * TEST INFRASTRUCTURE ONLY. Nothing in the shipped library links, loads or calls this code: it is the checker that
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use. Every function restates the arithmetic of the
 * reference (Tharunmaks/Stream-, "ExpertStream") in plain C and cites the reference lines it follows.
 *
 * Formats covered: Q4_0, Q5_0, Q8_0, Q2_K, Q3_K, Q4_K, Q5_K, Q6_K weights against Q8_0 (float scale, 36 B) and Q8_K (292 B) activations.
 *
 * Float order. The reference's fp32 epilogues are compiler dependent (its Makefile defaults to clang, which contracts
 * a*b+c into an FMA inside the AVX2 functions; gcc in -std=c11 mode does not). Every matvec here takes
 *   order = ESQ_STRICT    : no contraction (gcc -std=c11 build of the reference),
 *   order = ESQ_CONTRACT  : clang -ffp-contract=on build of the reference,
 *   path  = ESQ_PATH_X86  : the x86 AVX2 dispatch (es_quant.c:1852-1884),
 *   path  = ESQ_PATH_SCALAR: the scalar mv_* kernels (ES_NO_AVX2=1, es_quant.c:1013-1175); order has no effect there.
 * Q5_K has no AVX2 kernel: the x86 dispatch falls through to the scalar mv_q5_K (es_quant.c:1935), built without FMA, so
 * its order is strict in every build and path. Q3_K's AVX2 epilogue has Q6_K's shape (s += y.d * d * tot).
 * Integer block dots are exact and order independent.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   fp16<->fp32, quantize_q8_0/q8_K, quantize_q2_K_ref, dequant, matvec (both orders, both paths), matvec_multi:
 *       bit-exact against the reference built from its own sources (oracle/_ref) and against the committed golden
 *       vectors made from that build (tests/golden/);
 *   block integer dots: brute force over dequantized integers (int64), plus the fp32 matvec identities above;
 *   route / grouping / SwiGLU / combine (moe_n restatement): golden vectors are not possible (the reference's engine
 *       needs a whole model), so these are pinned by invariants and textbook special cases in the tests
 *       (softmax of equal logits, ties to lowest index, norm_topk sums to one, grouping is a stable partition).
 *   rmsnorm (es_engine.c is not buildable on its own): against an independent numpy restatement (float64 running sum
 *       via cumsum, float32 products) on random rows, and the closed forms of a zero row (s = 1/sqrt(eps)), a constant
 *       row (s = 1/sqrt(c^2 + eps)) and w = NULL equal to w = ones.
 *   Weight quantizers for Q4_0/Q5_0/Q8_0/Q3_K/Q4_K/Q5_K/Q6_K are this project's own (the reference has none); they are test-input
 *       generators, checked only for round-trip error bounds.
 */
#ifndef ESQ_ORACLE_H
#define ESQ_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGML type ids used by the path (reference src/es_quant.h:15-22) */
enum { ESQ_Q4_0 = 2, ESQ_Q5_0 = 6, ESQ_Q8_0 = 8, ESQ_Q2_K = 10, ESQ_Q3_K = 11, ESQ_Q4_K = 12, ESQ_Q5_K = 13, ESQ_Q6_K = 14 };
enum { ESQ_STRICT = 0, ESQ_CONTRACT = 1 };
enum { ESQ_PATH_X86 = 0, ESQ_PATH_SCALAR = 1 };

/* activation blocks, byte layouts of es_blk_q80 (src/es_quant.h:31) and es_block_q8_K (src/es_q2k.h:31-38) */
typedef struct { float d; int8_t qs[32]; } esq_q80;
typedef struct { float d; int8_t qs[256]; int16_t bsums[16]; } esq_q8K;

/* ---- format facts ---- */
int    esq_block_elems(uint32_t type);          /* 32 or 256; 0 if unknown */
int    esq_block_bytes(uint32_t type);          /* 18, 22, 34, 84, 110, 144, 176, 210 */
size_t esq_row_bytes(uint32_t type, int cols); /* src/es_quant.c:39-73 */
int    esq_uses_q8K(uint32_t type);            /* 1: Q8_K activations, 0: Q8_0 */

/* ---- fp16 ---- */
float    esq_half_to_float(uint16_t h);  /* exact for every finite half, src/es_q2k.h:40-64 */
uint16_t esq_float_to_half(float f);     /* the reference's rounding, src/es_q2k.c:12-37 */

/* ---- activation quantizers ---- */
void esq_quantize_q8_0(const float *x, esq_q80 *y, int n); /* src/es_quant.c:489-497 */
void esq_quantize_q8_K(const float *x, esq_q8K *y, int n); /* src/es_q2k.c:102-125 */

/* ---- block integer dots (one weight block against its activation block) ---- */
/* 32-wide: the eight AVX2 lane sums (4 weights each, offset already removed); their sum is the scalar integer dot */
void    esq_blkdot_q4_0(const uint8_t *blk, const esq_q80 *y, int32_t lane[8]);
void    esq_blkdot_q5_0(const uint8_t *blk, const esq_q80 *y, int32_t lane[8]);
void    esq_blkdot_q8_0(const uint8_t *blk, const esq_q80 *y, int32_t lane[8]);
int32_t esq_blkdot_q4_K(const uint8_t *blk, const esq_q8K *y, int32_t *mins);
int32_t esq_blkdot_q6_K(const uint8_t *blk, const esq_q8K *y);
int32_t esq_blkdot_q5_K(const uint8_t *blk, const esq_q8K *y, int32_t *mins);
int32_t esq_blkdot_q3_K(const uint8_t *blk, const esq_q8K *y);
/* Q3_K's sixteen 6-bit scales, minus 32 (src/es_quant.c:1125-1129) */
void    esq_q3k_scales(const uint8_t *s12, int8_t sc[16]);
int32_t esq_blkdot_q2_K(const uint8_t *blk, const esq_q8K *y, int32_t *summs);
/* Q4_K 6-bit scale/min unpack for sub-block j (src/es_quant.c:75-83) */
void    esq_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn);

/* ---- products ---- */
/* y[r] for r in [r0, r1). act: Q8_0 blocks (cols/32) or Q8_K blocks (cols/256) depending on type. */
void esq_matvec(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, float *y, int order, int path);
/* na activations, activation q at act + q*astride bytes, output y[q*ystride + r] (src/es_quant.c:1818-1850) */
void esq_matvec_multi(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, size_t astride, int na,
                      float *y, size_t ystride, int order, int path);
/* the float path for activations without blocks: es_dequant_row + dot_f32 per row (src/es_quant.c:514-526, 1941-1944),
 * y[r] for r in [r0, r1); x holds cols floats. The same in every build and path. */
void esq_matvec_float(uint32_t type, const void *W, int cols, int r0, int r1, const float *x, float *y);
/* integer parts of every (row, block): dots[r*nb + b] (Q4_0/Q5_0: sum of lanes), aux = mins/summs (0 otherwise) */
void esq_block_ints(uint32_t type, const void *W, int cols, int rows, const void *act, int32_t *dots, int32_t *aux);

/* ---- dequantizers (src/es_quant.c:117-181, 425-472; src/es_q2k.c:88-100) ---- */
void esq_dequant_row(uint32_t type, const void *src, float *dst, int n);

/* ---- weight quantizers ---- */
void esq_quantize_q2_K_ref(const float *x, void *dst, int n); /* src/es_q2k.c:47-86 */
/* this project's own min/max quantizers for Q4_0/Q5_0/Q8_0/Q3_K/Q4_K/Q5_K/Q6_K; Q2_K goes to the reference's method */
void esq_quantize_row(uint32_t type, const float *x, void *dst, int n);

/* ---- deterministic inputs ---- */
uint64_t esq_rng_next(uint64_t *s);                     /* xorshift64*, tools/es_common.h:13-18 */
float    esq_frand(uint64_t *s);                        /* Irwin-Hall(4) ~N(0,1), tools/es_kbench.c:30-34 */
void     esq_fill_gauss(uint64_t seed, float sigma, float *x, size_t n);
/* es_mtest's random blocks: random bytes, then sane fp16 scales (tools/es_mtest.c:9-13, 30-35). The xorshift
 * state is the caller's, so a sequence of calls reproduces es_mtest's stream. */
void     esq_mtest_blocks(uint32_t type, uint64_t *state, uint8_t *W, int rows, int cols);
void     esq_mtest_acts(uint64_t *state, float *x, size_t n);   /* ((rnd%2001)-1000)/250, tools/es_mtest.c:37 */

/* ---- MoE glue: restatement of moe_n (src/es_engine.c:744-942) for softmax gating, no biases ---- */
/* route(): softmax, top-k by repeated argmax (ties to the lowest index), optional renormalisation. Returns k. */
int  esq_route_softmax(float *logits, int ne, int k, int norm_topk, int *sel, float *w);
/* distinct experts in order of first use; start/cnt per expert; rowof[t*k + j] = grouped row of (t, j) */
int  esq_moe_group(const int *sel, int n_tok, int k, int *uex, int *cnt, int *start, int *rowof, int *tok_of);
void esq_swiglu(const float *g, const float *u, float *h, int n);  /* g/(1+expf(-g))*u, src/es_engine.c:913 */
/* rmsnorm (src/es_engine.c:189-194): o = x * (float)(1/sqrt(sum of x^2 / n + eps)) * w; w may be NULL (weights 1) */
void esq_rmsnorm(const float *x, const float *w, float *o, int n, float eps);
/* out[t][i] = sum_j w[t][j] * ye[rowof[t][j]][i], sequential over j (src/es_engine.c:925-932) */
void esq_moe_combine(const float *ye, const int *rowof, const float *w, int n_tok, int k, int n, float *out);

/* ---- CPU baseline timing harness (es_kbench style, tools/es_kbench.c:136-149, 260-320) ---- */
typedef void (*esq_multi_fn)(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, size_t astride,
                             int na, float *y, size_t ystride);
/* Runs nmat matrices (W + m*mat_bytes) against na activations with nthreads pinned threads taking 16-row chunks
 * from a shared counter, activations in batches of at most 64 (src/es_engine.c:43, 152-171). Repeats the whole set
 * until at least min_seconds have passed. Returns seconds per pass over the set; *passes receives the count. */
double esq_cpu_bench(esq_multi_fn fn, uint32_t type, const void *W, size_t mat_bytes, int nmat, int rows, int cols,
                     const void *act, size_t astride, int na, float *y, int nthreads, double min_seconds, int *passes);
/* the oracle itself as an esq_multi_fn (x86 path, contract order) */
void esq_multi_x86_contract(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, size_t astride,
                            int na, float *y, size_t ystride);
/* The reference's own es_matvec_multi (oracle/_ref, loaded by the caller) as an esq_multi_fn: esq_bind_reference takes its
 * address; esq_multi_reference builds the reference's es_act records (src/es_quant.h:32-37) over the strided activation
 * blocks (q8 for the K-quants, q80 for Q4_0/Q5_0) and calls it with a per-thread scratch of cols floats. */
void esq_bind_reference(void *es_matvec_multi_fn);
void esq_multi_reference(uint32_t type, const void *W, int cols, int r0, int r1, const void *act, size_t astride, int na,
                         float *y, size_t ystride);

#ifdef __cplusplus
}
#endif
#endif
