/*
 * esq_oracle.c — CPU restatement of the reference's quantized products. TEST INFRASTRUCTURE ONLY (see esq_oracle.h).
 * Built with -ffp-contract=off so every float operation rounds where the C source says; the contracted order of the
 * reference's clang build is spelled out with fmaf().
 */
#define _GNU_SOURCE
#include "esq_oracle.h"

#include <math.h>
#include <pthread.h>
#include <sched.h>
#include <stdatomic.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

/* ------------------------------------------------------------------------------------------------------------------ */
/* format facts                                                                                                        */

int esq_block_elems(uint32_t t) {
    switch (t) {
    case ESQ_Q4_0: case ESQ_Q5_0: case ESQ_Q8_0: return 32;
    case ESQ_Q2_K: case ESQ_Q3_K: case ESQ_Q4_K: case ESQ_Q5_K: case ESQ_Q6_K: return 256;
    }
    return 0;
}

int esq_block_bytes(uint32_t t) {
    switch (t) {
    case ESQ_Q4_0: return 18;   /* d f16, qs[16]                              src/es_quant.c:12 */
    case ESQ_Q5_0: return 22;   /* d f16, qh[4], qs[16]                       src/es_quant.c:14 */
    case ESQ_Q8_0: return 34;   /* d f16, int8 qs[32]                         src/es_quant.c:11 */
    case ESQ_Q2_K: return 84;   /* scales[16], qs[64], d, dmin                src/es_q2k.h:24-29 */
    case ESQ_Q3_K: return 110;  /* hmask[32], qs[64], scales[12], d          src/es_quant.c:16 */
    case ESQ_Q4_K: return 144;  /* d, dmin, scales[12], qs[128]               src/es_quant.c:17 */
    case ESQ_Q5_K: return 176;  /* d, dmin, scales[12], qh[32], qs[128]      src/es_quant.c:18 */
    case ESQ_Q6_K: return 210;  /* ql[128], qh[64], int8 scales[16], d        src/es_quant.c:19 */
    }
    return 0;
}

size_t esq_row_bytes(uint32_t t, int cols) {
    const int e = esq_block_elems(t);
    return e ? (size_t)cols / (size_t)e * (size_t)esq_block_bytes(t) : 0;
}

int esq_uses_q8K(uint32_t t) { return esq_block_elems(t) == 256; }

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }
static uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
static void wr16(uint8_t *p, uint16_t v) { p[0] = (uint8_t)v; p[1] = (uint8_t)(v >> 8); }

/* ------------------------------------------------------------------------------------------------------------------ */
/* fp16                                                                                                                */

float esq_half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h >> 15) << 31;
    const int e = (h >> 10) & 31;
    const uint32_t m = h & 1023u;
    uint32_t bits;
    if (e == 31) {
        bits = sign | 0x7f800000u | (m << 13);
    } else if (e != 0) {
        bits = sign | ((uint32_t)(e + 112) << 23) | (m << 13);
    } else {
        const float f = (float)m * 5.9604644775390625e-08f;   /* m * 2^-24, exact */
        memcpy(&bits, &f, 4);
        bits |= sign;
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

/* round half up in magnitude, overflow to inf, like the reference's converter */
uint16_t esq_float_to_half(float f) {
    uint32_t b;
    memcpy(&b, &f, 4);
    const uint32_t s = (b >> 16) & 0x8000u;
    const int e = (int)((b >> 23) & 0xff) - 112;
    uint32_t m = b & 0x7fffffu;
    if (e >= 31) return (uint16_t)(s | 0x7c00u);
    if (e <= 0) {
        if (e < -10) return (uint16_t)s;
        m |= 0x800000u;
        const int sh = 14 - e;
        return (uint16_t)(s | ((m >> sh) + ((m >> (sh - 1)) & 1u)));
    }
    return (uint16_t)((s | ((uint32_t)e << 10) | (m >> 13)) + ((m >> 12) & 1u));
}

/* ------------------------------------------------------------------------------------------------------------------ */
/* activation quantizers                                                                                               */

void esq_quantize_q8_0(const float *x, esq_q80 *y, int n) {
    for (int b = 0; b < n / 32; b++) {
        const float *v = x + 32 * b;
        float amax = 0.0f;
        for (int i = 0; i < 32; i++) {
            const float a = v[i] < 0 ? -v[i] : v[i];
            if (a > amax) amax = a;
        }
        const float d = amax / 127.0f;
        const float id = d != 0.0f ? 1.0f / d : 0.0f;
        y[b].d = d;
        for (int i = 0; i < 32; i++) {
            const float s = v[i] * id;
            const float r = s < 0 ? s - 0.5f : s + 0.5f;   /* round half away, then truncate */
            y[b].qs[i] = (int8_t)(int)r;
        }
    }
}

void esq_quantize_q8_K(const float *x, esq_q8K *y, int n) {
    for (int b = 0; b < n / 256; b++) {
        const float *v = x + 256 * b;
        float amax = 0.0f;
        for (int i = 0; i < 256; i++)
            if (fabsf(v[i]) > amax) amax = fabsf(v[i]);
        memset(&y[b], 0, sizeof y[b]);
        if (amax == 0.0f) continue;
        const float id = 127.0f / amax;
        y[b].d = amax / 127.0f;
        for (int i = 0; i < 256; i++) {
            long q = lrintf(v[i] * id);   /* round half to even */
            if (q > 127) q = 127;
            if (q < -127) q = -127;
            y[b].qs[i] = (int8_t)q;
        }
        for (int g = 0; g < 16; g++) {
            int s = 0;
            for (int l = 0; l < 16; l++) s += y[b].qs[16 * g + l];
            y[b].bsums[g] = (int16_t)s;
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------------ */
/* block integer dots                                                                                                  */

/* element e (0..31) of a 32-wide 4-bit block: low nibbles are elements 0..15, high nibbles 16..31 */
static int nib32(const uint8_t *qs, int e) { return e < 16 ? (qs[e] & 15) : (qs[e - 16] >> 4); }

void esq_blkdot_q4_0(const uint8_t *blk, const esq_q80 *y, int32_t lane[8]) {
    const uint8_t *qs = blk + 2;
    for (int i = 0; i < 8; i++) {   /* AVX2 lane i sums elements 4i..4i+3 (src/es_quant.c:1252-1262) */
        int32_t a = 0;
        for (int m = 0; m < 4; m++) a += (nib32(qs, 4 * i + m) - 8) * y->qs[4 * i + m];
        lane[i] = a;
    }
}

void esq_blkdot_q5_0(const uint8_t *blk, const esq_q80 *y, int32_t lane[8]) {
    const uint32_t qh = rd32(blk + 2);
    const uint8_t *qs = blk + 6;
    for (int i = 0; i < 8; i++) {   /* fifth bit of element e is bit e of qh (src/es_quant.c:1031-1055, 1286-1296) */
        int32_t a = 0;
        for (int m = 0; m < 4; m++) {
            const int e = 4 * i + m;
            const int u = nib32(qs, e) | (int)(((qh >> e) & 1u) << 4);
            a += (u - 16) * y->qs[e];
        }
        lane[i] = a;
    }
}

void esq_blkdot_q8_0(const uint8_t *blk, const esq_q80 *y, int32_t lane[8]) {
    const int8_t *qs = (const int8_t *)(blk + 2);
    for (int i = 0; i < 8; i++) {   /* AVX2 lane i sums elements 4i..4i+3 (dot32_ss, src/es_quant.c:1198-1221) */
        int32_t a = 0;
        for (int m = 0; m < 4; m++) a += qs[4 * i + m] * y->qs[4 * i + m];
        lane[i] = a;
    }
}

static void blkdot_32(uint32_t t, const uint8_t *blk, const esq_q80 *y, int32_t lane[8]) {
    if (t == ESQ_Q4_0) esq_blkdot_q4_0(blk, y, lane);
    else if (t == ESQ_Q5_0) esq_blkdot_q5_0(blk, y, lane);
    else esq_blkdot_q8_0(blk, y, lane);
}

void esq_scale_min_k4(int j, const uint8_t *q, uint8_t *sc, uint8_t *mn) {
    if (j < 4) {
        *sc = q[j] & 63;
        *mn = q[j + 4] & 63;
    } else {
        *sc = (uint8_t)((q[j + 4] & 15) | ((q[j - 4] >> 6) << 4));
        *mn = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

int32_t esq_blkdot_q4_K(const uint8_t *blk, const esq_q8K *y, int32_t *mins) {
    const uint8_t *scales = blk + 4, *q = blk + 16;
    int32_t dot = 0, mm = 0;
    for (int c = 0; c < 4; c++) {   /* chunk c: low nibbles -> sub-block 2c, high -> 2c+1 (src/es_quant.c:1056-1080) */
        uint8_t s0, m0, s1, m1;
        esq_scale_min_k4(2 * c, scales, &s0, &m0);
        esq_scale_min_k4(2 * c + 1, scales, &s1, &m1);
        int32_t lo = 0, hi = 0;
        for (int l = 0; l < 32; l++) {
            lo += (q[32 * c + l] & 15) * y->qs[64 * c + l];
            hi += (q[32 * c + l] >> 4) * y->qs[64 * c + 32 + l];
        }
        dot += s0 * lo + s1 * hi;
        mm += m0 * (y->bsums[4 * c] + y->bsums[4 * c + 1]) + m1 * (y->bsums[4 * c + 2] + y->bsums[4 * c + 3]);
    }
    *mins = mm;
    return dot;
}

int32_t esq_blkdot_q5_K(const uint8_t *blk, const esq_q8K *y, int32_t *mins) {
    const uint8_t *scales = blk + 4, *qh = blk + 16, *q = blk + 48;
    int32_t dot = 0, mm = 0;
    for (int c = 0; c < 4; c++) {   /* Q4_K's chunks plus a fifth bit: qh bit 2c (low), 2c+1 (high) (src/es_quant.c:1153-1175) */
        uint8_t s0, m0, s1, m1;
        esq_scale_min_k4(2 * c, scales, &s0, &m0);
        esq_scale_min_k4(2 * c + 1, scales, &s1, &m1);
        int32_t lo = 0, hi = 0;
        for (int l = 0; l < 32; l++) {
            lo += ((q[32 * c + l] & 15) | (((qh[l] >> (2 * c)) & 1) << 4)) * y->qs[64 * c + l];
            hi += ((q[32 * c + l] >> 4) | (((qh[l] >> (2 * c + 1)) & 1) << 4)) * y->qs[64 * c + 32 + l];
        }
        dot += s0 * lo + s1 * hi;
        mm += m0 * (y->bsums[4 * c] + y->bsums[4 * c + 1]) + m1 * (y->bsums[4 * c + 2] + y->bsums[4 * c + 3]);
    }
    *mins = mm;
    return dot;
}

void esq_q3k_scales(const uint8_t *s12, int8_t sc[16]) {
    /* sixteen 6-bit scales: low nibbles from bytes 0-7, high pairs from bytes 8-11 (src/es_quant.c:1125-1128) */
    for (int g = 0; g < 16; g++) {
        const int lo = g < 8 ? s12[g] & 15 : s12[g - 8] >> 4;
        const int hi = (s12[8 + (g & 3)] >> (2 * (g >> 2))) & 3;
        sc[g] = (int8_t)((lo | (hi << 4)) - 32);
    }
}

int32_t esq_blkdot_q3_K(const uint8_t *blk, const esq_q8K *y) {
    const uint8_t *hm = blk, *q = blk + 32;
    int8_t sc[16];
    esq_q3k_scales(blk + 96, sc);
    int32_t tot = 0;
    for (int g = 0; g < 16; g++) {   /* group g = 8n + 2j + half: bits 2j of qs[32n + 16half + l], hmask bit 4n+j (src/es_quant.c:1131-1146) */
        const int n = g >> 3, j = (g >> 1) & 3, half = g & 1;
        int32_t s16 = 0;
        for (int l = 0; l < 16; l++) {
            const int v = ((q[32 * n + 16 * half + l] >> (2 * j)) & 3) - (((hm[16 * half + l] >> (4 * n + j)) & 1) ? 0 : 4);
            s16 += v * y->qs[16 * g + l];
        }
        tot += sc[g] * s16;
    }
    return tot;
}

int32_t esq_blkdot_q6_K(const uint8_t *blk, const esq_q8K *y) {
    const uint8_t *ql = blk, *qh = blk + 128;
    const int8_t *sc = (const int8_t *)(blk + 192);
    int32_t tot = 0;
    for (int h = 0; h < 2; h++) {   /* src/es_quant.c:1081-1117 */
        int32_t p[8] = {0, 0, 0, 0, 0, 0, 0, 0};
        for (int l = 0; l < 32; l++) {
            const int is = l >> 4;
            const uint8_t a = ql[64 * h + l], b = ql[64 * h + 32 + l], hb = qh[32 * h + l];
            const int v1 = ((a & 15) | ((hb & 3) << 4)) - 32;
            const int v2 = ((b & 15) | (((hb >> 2) & 3) << 4)) - 32;
            const int v3 = ((a >> 4) | (((hb >> 4) & 3) << 4)) - 32;
            const int v4 = ((b >> 4) | ((hb >> 6) << 4)) - 32;
            const int8_t *yy = y->qs + 128 * h + l;
            p[is] += v1 * yy[0];
            p[is + 2] += v2 * yy[32];
            p[is + 4] += v3 * yy[64];
            p[is + 6] += v4 * yy[96];
        }
        for (int k = 0; k < 8; k++) tot += sc[8 * h + k] * p[k];
    }
    return tot;
}

int32_t esq_blkdot_q2_K(const uint8_t *blk, const esq_q8K *y, int32_t *summs) {
    const uint8_t *sc = blk, *qs = blk + 16;
    int32_t sm = 0, isum = 0;
    for (int g = 0; g < 16; g++) {   /* group g: half g/8, shift 2*((g%8)/2), bytes 16*(g%2).. (src/es_q2k.h:1-15) */
        sm += y->bsums[g] * (sc[g] >> 4);
        const int w = g & 7, shift = (w >> 1) * 2, base = 32 * (g >> 3) + 16 * (w & 1);
        int32_t s = 0;
        for (int l = 0; l < 16; l++) s += y->qs[16 * g + l] * ((qs[base + l] >> shift) & 3);
        isum += (sc[g] & 15) * s;
    }
    *summs = sm;
    return isum;
}

/* ------------------------------------------------------------------------------------------------------------------ */
/* rows                                                                                                                */

/* x86 AVX2 32-wide path: 8 fused lane accumulators per row, then the hsum_ps tree (src/es_quant.c:1185-1187,
 * 1198-1221, 1262-1285, 1297-1323). _mm256_fmadd_ps is fused under either compiler, so order does not matter here. */
static float row_32_x86(uint32_t t, const uint8_t *w, int nb, const esq_q80 *y) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = w + (size_t)b * esq_block_bytes(t);
        int32_t lane[8];
        blkdot_32(t, blk, &y[b], lane);
        const float dyd = esq_half_to_float(rd16(blk)) * y[b].d;
        for (int i = 0; i < 8; i++) acc[i] = fmaf((float)lane[i], dyd, acc[i]);
    }
    return ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
}

/* scalar 32-wide path: one integer per block, s += (d*yd)*a (src/es_quant.c:1005-1055) */
static float row_32_scalar(uint32_t t, const uint8_t *w, int nb, const esq_q80 *y) {
    float s = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = w + (size_t)b * esq_block_bytes(t);
        int32_t lane[8], a = 0;
        blkdot_32(t, blk, &y[b], lane);
        for (int i = 0; i < 8; i++) a += lane[i];
        const float dd = esq_half_to_float(rd16(blk)) * y[b].d;
        s = s + dd * (float)a;
    }
    return s;
}

static float row_k(uint32_t t, const uint8_t *w, int nb, const esq_q8K *y, int contract) {
    float s = 0.0f;
    for (int b = 0; b < nb; b++) {
        const uint8_t *blk = w + (size_t)b * esq_block_bytes(t);
        const float yd = y[b].d;
        if (t == ESQ_Q4_K) {   /* s += y.d * (d*dot - dmin*mins)   (src/es_quant.c:1077, 1339) */
            int32_t mins;
            const int32_t dot = esq_blkdot_q4_K(blk, &y[b], &mins);
            const float d = esq_half_to_float(rd16(blk)), dm = esq_half_to_float(rd16(blk + 2));
            const float q = dm * (float)mins;
            if (contract) s = fmaf(yd, fmaf(d, (float)dot, -q), s);
            else s = s + yd * (d * (float)dot - q);
        } else if (t == ESQ_Q5_K) {   /* s += y.d * (d*dot - dmin*mins), the scalar kernel only: never fused (src/es_quant.c:1173) */
            int32_t mins;
            const int32_t dot = esq_blkdot_q5_K(blk, &y[b], &mins);
            const float d = esq_half_to_float(rd16(blk)), dm = esq_half_to_float(rd16(blk + 2));
            s = s + yd * (d * (float)dot - dm * (float)mins);
        } else if (t == ESQ_Q6_K || t == ESQ_Q3_K) {   /* s += y.d * d * tot   (src/es_quant.c:1114, 1466; Q3_K 1147, 1391) */
            const int32_t tot = t == ESQ_Q6_K ? esq_blkdot_q6_K(blk, &y[b]) : esq_blkdot_q3_K(blk, &y[b]);
            const float yd_d = yd * esq_half_to_float(rd16(blk + (t == ESQ_Q6_K ? 208 : 108)));
            if (contract) s = fmaf(yd_d, (float)tot, s);
            else s = s + yd_d * (float)tot;
        } else {   /* Q2_K: s += dall*isum - dmin*summs   (src/es_q2k.c:142-146, src/es_quant.c:1364-1365) */
            int32_t summs;
            const int32_t isum = esq_blkdot_q2_K(blk, &y[b], &summs);
            const float dall = yd * esq_half_to_float(rd16(blk + 80));
            const float dmin = yd * esq_half_to_float(rd16(blk + 82));
            const float q = dmin * (float)summs;
            if (contract) s = s + fmaf(dall, (float)isum, -q);
            else s = s + (dall * (float)isum - q);
        }
    }
    return s;
}

void esq_matvec(uint32_t t, const void *W, int cols, int r0, int r1, const void *act, float *y, int order, int path) {
    const int nb = cols / esq_block_elems(t);
    const size_t rb = esq_row_bytes(t, cols);
    const uint8_t *w = (const uint8_t *)W;
    for (int r = r0; r < r1; r++) {
        const uint8_t *row = w + rb * (size_t)r;
        if (esq_uses_q8K(t))
            y[r] = row_k(t, row, nb, (const esq_q8K *)act, path == ESQ_PATH_X86 && order == ESQ_CONTRACT);
        else
            y[r] = path == ESQ_PATH_X86 ? row_32_x86(t, row, nb, (const esq_q80 *)act)
                                        : row_32_scalar(t, row, nb, (const esq_q80 *)act);
    }
}

void esq_matvec_multi(uint32_t t, const void *W, int cols, int r0, int r1, const void *act, size_t astride, int na,
                      float *y, size_t ystride, int order, int path) {
    /* the reference's multi kernels replay the single-activation arithmetic exactly (tools/es_mtest.c) */
    for (int q = 0; q < na; q++)
        esq_matvec(t, W, cols, r0, r1, (const uint8_t *)act + (size_t)q * astride, y + (size_t)q * ystride, order, path);
}

/* The float path (src/es_quant.c:1941-1944): an activation prepared without its blocks (es_act_prepare with no Q8_K
 * buffer, an exhausted Q8_0 arena, or ES_FLOAT_ACT; src/es_quant.c:499-512) is multiplied by dequantizing each row and
 * taking dot_f32 (src/es_quant.c:514-526): four running sums over the elements i = 0, 1, 2, 3 (mod 4), each product and
 * sum rounded on its own (the function has no FMA target on x86, so no build contracts it), then (s0 + s1) + (s2 + s3). */
static float dot_f32_4(const float *a, const float *b, int n) {
    float s[4] = {0, 0, 0, 0};
    int i = 0;
    for (; i + 4 <= n; i += 4)
        for (int j = 0; j < 4; j++) s[j] += a[i + j] * b[i + j];
    for (; i < n; i++) s[0] += a[i] * b[i];
    return (s[0] + s[1]) + (s[2] + s[3]);
}

void esq_matvec_float(uint32_t t, const void *W, int cols, int r0, int r1, const float *x, float *y) {
    const size_t rb = esq_row_bytes(t, cols);
    float *row = (float *)malloc(sizeof(float) * (size_t)cols);
    if (!row) return;
    for (int r = r0; r < r1; r++) {
        esq_dequant_row(t, (const uint8_t *)W + rb * (size_t)r, row, cols);
        y[r] = dot_f32_4(row, x, cols);
    }
    free(row);
}

void esq_block_ints(uint32_t t, const void *W, int cols, int rows, const void *act, int32_t *dots, int32_t *aux) {
    const int nb = cols / esq_block_elems(t);
    const size_t rb = esq_row_bytes(t, cols);
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < nb; b++) {
            const uint8_t *blk = (const uint8_t *)W + rb * (size_t)r + (size_t)b * esq_block_bytes(t);
            int32_t v = 0, x = 0, lane[8];
            switch (t) {
            case ESQ_Q4_0: esq_blkdot_q4_0(blk, (const esq_q80 *)act + b, lane); for (int i = 0; i < 8; i++) v += lane[i]; break;
            case ESQ_Q5_0: esq_blkdot_q5_0(blk, (const esq_q80 *)act + b, lane); for (int i = 0; i < 8; i++) v += lane[i]; break;
            case ESQ_Q8_0: esq_blkdot_q8_0(blk, (const esq_q80 *)act + b, lane); for (int i = 0; i < 8; i++) v += lane[i]; break;
            case ESQ_Q4_K: v = esq_blkdot_q4_K(blk, (const esq_q8K *)act + b, &x); break;
            case ESQ_Q6_K: v = esq_blkdot_q6_K(blk, (const esq_q8K *)act + b); break;
            case ESQ_Q5_K: v = esq_blkdot_q5_K(blk, (const esq_q8K *)act + b, &x); break;
            case ESQ_Q3_K: v = esq_blkdot_q3_K(blk, (const esq_q8K *)act + b); break;
            case ESQ_Q2_K: v = esq_blkdot_q2_K(blk, (const esq_q8K *)act + b, &x); break;
            }
            dots[(size_t)r * nb + b] = v;
            if (aux) aux[(size_t)r * nb + b] = x;
        }
}

/* ------------------------------------------------------------------------------------------------------------------ */
/* dequantizers                                                                                                        */

void esq_dequant_row(uint32_t t, const void *src, float *y, int n) {
    const uint8_t *p = (const uint8_t *)src;
    const int bb = esq_block_bytes(t);
    for (int b = 0; b < n / esq_block_elems(t); b++, p += bb) {
        switch (t) {
        case ESQ_Q4_0: {   /* (x-8)*d, src/es_quant.c:433-449 */
            const float d = esq_half_to_float(rd16(p));
            for (int e = 0; e < 32; e++) *y++ = (float)(nib32(p + 2, e) - 8) * d;
            break;
        }
        case ESQ_Q8_0: {   /* d*q, src/es_quant.c:425-431 */
            const float d = esq_half_to_float(rd16(p));
            for (int e = 0; e < 32; e++) *y++ = d * (float)(int8_t)p[2 + e];
            break;
        }
        case ESQ_Q5_0: {   /* (x-16)*d, src/es_quant.c:451-468 */
            const float d = esq_half_to_float(rd16(p));
            const uint32_t qh = rd32(p + 2);
            for (int e = 0; e < 32; e++) *y++ = (float)((nib32(p + 6, e) | (int)(((qh >> e) & 1u) << 4)) - 16) * d;
            break;
        }
        case ESQ_Q4_K: {   /* d*sc*q - dmin*m, src/es_quant.c:117-133 */
            const float d = esq_half_to_float(rd16(p)), dm = esq_half_to_float(rd16(p + 2));
            for (int c = 0; c < 4; c++) {
                uint8_t s0, m0, s1, m1;
                esq_scale_min_k4(2 * c, p + 4, &s0, &m0);
                esq_scale_min_k4(2 * c + 1, p + 4, &s1, &m1);
                const float d1 = d * (float)s0, n1 = dm * (float)m0, d2 = d * (float)s1, n2 = dm * (float)m1;
                for (int l = 0; l < 32; l++) *y++ = d1 * (float)(p[16 + 32 * c + l] & 15) - n1;
                for (int l = 0; l < 32; l++) *y++ = d2 * (float)(p[16 + 32 * c + l] >> 4) - n2;
            }
            break;
        }
        case ESQ_Q5_K: {   /* d*sc*q - dmin*m, q with its fifth bit, src/es_quant.c:136-154 */
            const float d = esq_half_to_float(rd16(p)), dm = esq_half_to_float(rd16(p + 2));
            for (int c = 0; c < 4; c++) {
                uint8_t s0, m0, s1, m1;
                esq_scale_min_k4(2 * c, p + 4, &s0, &m0);
                esq_scale_min_k4(2 * c + 1, p + 4, &s1, &m1);
                const float d1 = d * (float)s0, n1 = dm * (float)m0, d2 = d * (float)s1, n2 = dm * (float)m1;
                for (int l = 0; l < 32; l++)
                    *y++ = d1 * (float)((p[48 + 32 * c + l] & 15) + ((p[16 + l] >> (2 * c)) & 1) * 16) - n1;
                for (int l = 0; l < 32; l++)
                    *y++ = d2 * (float)((p[48 + 32 * c + l] >> 4) + ((p[16 + l] >> (2 * c + 1)) & 1) * 16) - n2;
            }
            break;
        }
        case ESQ_Q3_K: {   /* d*(sc-32)*(q - (hbit ? 0 : 4)), src/es_quant.c:85-115 */
            const float d = esq_half_to_float(rd16(p + 108));
            int8_t sc[16];
            esq_q3k_scales(p + 96, sc);
            for (int g = 0; g < 16; g++) {
                const int n = g >> 3, j = (g >> 1) & 3, half = g & 1;
                const float dl = d * (float)sc[g];
                for (int l = 0; l < 16; l++)
                    *y++ = dl * (float)(((p[32 + 32 * n + 16 * half + l] >> (2 * j)) & 3) -
                                        (((p[16 * half + l] >> (4 * n + j)) & 1) ? 0 : 4));
            }
            break;
        }
        case ESQ_Q6_K: {   /* d*sc*(q-32), src/es_quant.c:156-181 */
            const float d = esq_half_to_float(rd16(p + 208));
            const int8_t *sc = (const int8_t *)(p + 192);
            for (int h = 0; h < 2; h++) {
                for (int l = 0; l < 32; l++) {
                    const uint8_t a = p[64 * h + l], c2 = p[64 * h + 32 + l], hb = p[128 + 32 * h + l];
                    const int is = 8 * h + l / 16;
                    y[l] = d * (float)sc[is] * (float)(((a & 15) | ((hb & 3) << 4)) - 32);
                    y[l + 32] = d * (float)sc[is + 2] * (float)(((c2 & 15) | (((hb >> 2) & 3) << 4)) - 32);
                    y[l + 64] = d * (float)sc[is + 4] * (float)(((a >> 4) | (((hb >> 4) & 3) << 4)) - 32);
                    y[l + 96] = d * (float)sc[is + 6] * (float)(((c2 >> 4) | ((hb >> 6) << 4)) - 32);
                }
                y += 128;
            }
            break;
        }
        case ESQ_Q2_K: {   /* d*(sc&15)*q - dmin*(sc>>4), src/es_q2k.c:88-100 */
            const float d = esq_half_to_float(rd16(p + 80)), dm = esq_half_to_float(rd16(p + 82));
            for (int g = 0; g < 16; g++) {
                const float dl = d * (float)(p[g] & 15), ml = dm * (float)(p[g] >> 4);
                const int w = g & 7, shift = (w >> 1) * 2, base = 16 + 32 * (g >> 3) + 16 * (w & 1);
                for (int l = 0; l < 16; l++) *y++ = dl * (float)((p[base + l] >> shift) & 3) - ml;
            }
            break;
        }
        default: return;
        }
    }
}

/* ------------------------------------------------------------------------------------------------------------------ */
/* weight quantizers                                                                                                   */

static int clampi(long v, int lo, int hi) { return v < lo ? lo : v > hi ? hi : (int)v; }

/* the reference's test quantizer: per group of 16, min (<= 0) / max -> 2-bit codes (src/es_q2k.c:47-86) */
void esq_quantize_q2_K_ref(const float *x, void *dst, int n) {
    uint8_t *blk = (uint8_t *)dst;
    for (int b = 0; b < n / 256; b++, x += 256, blk += 84) {
        float scale[16], mn[16], smax = 0.0f, mmax = 0.0f;
        for (int g = 0; g < 16; g++) {
            float lo = x[16 * g], hi = x[16 * g];
            for (int l = 1; l < 16; l++) {
                if (x[16 * g + l] < lo) lo = x[16 * g + l];
                if (x[16 * g + l] > hi) hi = x[16 * g + l];
            }
            if (lo > 0) lo = 0;
            scale[g] = (hi - lo) / 3;
            mn[g] = -lo;
            if (scale[g] > smax) smax = scale[g];
            if (mn[g] > mmax) mmax = mn[g];
        }
        memset(blk, 0, 84);
        const uint16_t dh = esq_float_to_half(smax / 15), mh = esq_float_to_half(mmax / 15);
        wr16(blk + 80, dh);
        wr16(blk + 82, mh);
        const float d = esq_half_to_float(dh), dmin = esq_half_to_float(mh);
        for (int g = 0; g < 16; g++) {
            const int ls = clampi(d > 0 ? lrintf(scale[g] / d) : 0, 0, 15);
            const int lm = clampi(dmin > 0 ? lrintf(mn[g] / dmin) : 0, 0, 15);
            blk[g] = (uint8_t)(ls | (lm << 4));
            const float dl = d * (float)ls, ml = dmin * (float)lm;
            const int w = g & 7, shift = (w >> 1) * 2, base = 16 + 32 * (g >> 3) + 16 * (w & 1);
            for (int l = 0; l < 16; l++) {
                const int q = clampi(dl > 0 ? lrintf((x[16 * g + l] + ml) / dl) : 0, 0, 3);
                blk[base + l] |= (uint8_t)(q << shift);
            }
        }
    }
}

static float absmax(const float *x, int n) {
    float a = 0.0f;
    for (int i = 0; i < n; i++) if (fabsf(x[i]) > a) a = fabsf(x[i]);
    return a;
}

void esq_quantize_row(uint32_t t, const float *x, void *dst, int n) {
    uint8_t *p = (uint8_t *)dst;
    switch (t) {
    case ESQ_Q2_K: esq_quantize_q2_K_ref(x, dst, n); return;
    case ESQ_Q8_0:   /* symmetric: d = amax/127, code = round(x/d) */
        for (int b = 0; b < n / 32; b++, x += 32, p += 34) {
            const uint16_t dh = esq_float_to_half(absmax(x, 32) / 127.0f);
            wr16(p, dh);
            const float d = esq_half_to_float(dh);
            for (int e = 0; e < 32; e++) p[2 + e] = (uint8_t)(int8_t)(d > 0 ? clampi(lrintf(x[e] / d), -127, 127) : 0);
        }
        return;
    case ESQ_Q4_0: case ESQ_Q5_0: {   /* symmetric: d = amax/(2^(bits-1)-1), code = round(x/d) + offset */
        const int five = t == ESQ_Q5_0, off = five ? 16 : 8, top = five ? 31 : 15, bb = five ? 22 : 18;
        for (int b = 0; b < n / 32; b++, x += 32, p += bb) {
            memset(p, 0, (size_t)bb);
            const uint16_t dh = esq_float_to_half(absmax(x, 32) / (float)(off - 1));
            wr16(p, dh);
            const float d = esq_half_to_float(dh);
            uint32_t qh = 0;
            uint8_t *qs = p + (five ? 6 : 2);
            for (int e = 0; e < 32; e++) {
                const int q = d > 0 ? clampi(lrintf(x[e] / d) + off, 0, top) : off;
                qs[e & 15] |= (uint8_t)((q & 15) << (e < 16 ? 0 : 4));
                qh |= (uint32_t)((q >> 4) & 1) << e;
            }
            if (five) { p[2] = (uint8_t)qh; p[3] = (uint8_t)(qh >> 8); p[4] = (uint8_t)(qh >> 16); p[5] = (uint8_t)(qh >> 24); }
        }
        return;
    }
    case ESQ_Q4_K: case ESQ_Q5_K: {   /* per 32: min (<= 0)/max -> 15 (31) steps; 6-bit scale and min against fp16 d and dmin */
        const int five = t == ESQ_Q5_K, top = five ? 31 : 15, bb = five ? 176 : 144, qo = five ? 48 : 16;
        for (int b = 0; b < n / 256; b++, x += 256, p += bb) {
            float sc[8], mn[8], smax = 0.0f, mmax = 0.0f;
            for (int j = 0; j < 8; j++) {
                float lo = 0.0f, hi = x[32 * j];
                for (int l = 0; l < 32; l++) {
                    if (x[32 * j + l] < lo) lo = x[32 * j + l];
                    if (x[32 * j + l] > hi) hi = x[32 * j + l];
                }
                if (hi < 0) hi = 0;
                sc[j] = (hi - lo) / (float)top;
                mn[j] = -lo;
                if (sc[j] > smax) smax = sc[j];
                if (mn[j] > mmax) mmax = mn[j];
            }
            memset(p, 0, (size_t)bb);
            const uint16_t dh = esq_float_to_half(smax / 63), mh = esq_float_to_half(mmax / 63);
            wr16(p, dh);
            wr16(p + 2, mh);
            const float d = esq_half_to_float(dh), dmin = esq_half_to_float(mh);
            uint8_t is[8], im[8];
            for (int j = 0; j < 8; j++) {
                is[j] = (uint8_t)clampi(d > 0 ? lrintf(sc[j] / d) : 0, 0, 63);
                im[j] = (uint8_t)clampi(dmin > 0 ? lrintf(mn[j] / dmin) : 0, 0, 63);
            }
            uint8_t *s12 = p + 4;   /* inverse of scale_min_k4 */
            for (int j = 0; j < 4; j++) {
                s12[j] = (uint8_t)(is[j] | ((is[j + 4] >> 4) << 6));
                s12[j + 4] = (uint8_t)(im[j] | ((im[j + 4] >> 4) << 6));
                s12[j + 8] = (uint8_t)((is[j + 4] & 15) | ((im[j + 4] & 15) << 4));
            }
            for (int j = 0; j < 8; j++) {
                const float dl = d * (float)is[j], ml = dmin * (float)im[j];
                for (int l = 0; l < 32; l++) {
                    const int q = dl > 0 ? clampi(lrintf((x[32 * j + l] + ml) / dl), 0, top) : 0;
                    p[qo + 32 * (j >> 1) + l] |= (uint8_t)((q & 15) << ((j & 1) * 4));
                    if (five) p[16 + l] |= (uint8_t)(((q >> 4) & 1) << j);
                }
            }
        }
        return;
    }
    case ESQ_Q3_K: {   /* per 16: codes -4..3, 6-bit scale (stored + 32) against fp16 d */
        for (int b = 0; b < n / 256; b++, x += 256, p += 110) {
            float sc[16], smax = 0.0f;
            for (int g = 0; g < 16; g++) {
                sc[g] = absmax(x + 16 * g, 16) / 4;
                if (sc[g] > smax) smax = sc[g];
            }
            memset(p, 0, 110);
            const uint16_t dh = esq_float_to_half(smax / 31);
            wr16(p + 108, dh);
            const float d = esq_half_to_float(dh);
            for (int g = 0; g < 16; g++) {   /* group g = 8n + 2j + half, as esq_q3k_scales reads it */
                const int isc = clampi(d > 0 ? lrintf(sc[g] / d) : 0, 0, 31), u = isc + 32;
                if (g < 8) p[96 + g] |= (uint8_t)(u & 15); else p[96 + g - 8] |= (uint8_t)((u & 15) << 4);
                p[104 + (g & 3)] |= (uint8_t)((u >> 4) << (2 * (g >> 2)));
                const int nn = g >> 3, j = (g >> 1) & 3, half = g & 1;
                const float dl = d * (float)isc;
                for (int l = 0; l < 16; l++) {
                    const int q = dl > 0 ? clampi(lrintf(x[16 * g + l] / dl), -4, 3) : 0, c = q + 4;   /* c = low2 + 4*hbit */
                    p[32 + 32 * nn + 16 * half + l] |= (uint8_t)((c & 3) << (2 * j));
                    p[16 * half + l] |= (uint8_t)((c >> 2) << (4 * nn + j));
                }
            }
        }
        return;
    }
    case ESQ_Q6_K: {   /* per 16: symmetric 6-bit codes, int8 scale against fp16 d */
        for (int b = 0; b < n / 256; b++, x += 256, p += 210) {
            float sc[16], smax = 0.0f;
            for (int g = 0; g < 16; g++) {
                sc[g] = absmax(x + 16 * g, 16) / 31;
                if (sc[g] > smax) smax = sc[g];
            }
            memset(p, 0, 210);
            const uint16_t dh = esq_float_to_half(smax / 127);
            wr16(p + 208, dh);
            const float d = esq_half_to_float(dh);
            for (int g = 0; g < 16; g++) {
                const int isc = clampi(d > 0 ? lrintf(sc[g] / d) : 0, 0, 127);
                p[192 + g] = (uint8_t)isc;
                const float dl = d * (float)isc;
                for (int l = 0; l < 16; l++) {
                    const int e = 16 * g + l;
                    const int q = dl > 0 ? clampi(lrintf(x[e] / dl) + 32, 0, 63) : 32;
                    const int h = e >> 7, k = (e >> 5) & 3, ll = e & 31;   /* e = 128h + 32k + ll */
                    p[64 * h + 32 * (k & 1) + ll] |= (uint8_t)((q & 15) << ((k >> 1) * 4));
                    p[128 + 32 * h + ll] |= (uint8_t)((q >> 4) << (2 * k));
                }
            }
        }
        return;
    }
    }
}

/* ------------------------------------------------------------------------------------------------------------------ */
/* deterministic inputs                                                                                                */

uint64_t esq_rng_next(uint64_t *s) {
    uint64_t x = *s;
    x ^= x >> 12;
    x ^= x << 25;
    x ^= x >> 27;
    *s = x;
    return x * 0x2545F4914F6CDD1Dull;
}

float esq_frand(uint64_t *s) {
    float a = 0.0f;
    for (int i = 0; i < 4; i++) a += (float)(esq_rng_next(s) >> 40) / (float)(1 << 24);
    return (a - 2.0f) * 1.7f;
}

void esq_fill_gauss(uint64_t seed, float sigma, float *x, size_t n) {
    uint64_t s = seed;
    for (size_t i = 0; i < n; i++) x[i] = esq_frand(&s) * sigma;
}

static uint32_t mt_rnd(uint64_t *r) {   /* xorshift of tools/es_mtest.c:9-10 */
    uint64_t v = *r;
    v ^= v << 13;
    v ^= v >> 7;
    v ^= v << 17;
    *r = v;
    return (uint32_t)v;
}

static uint16_t mt_f16(float f) {   /* truncating, positive normals only (tools/es_mtest.c:11-13) */
    uint32_t u;
    memcpy(&u, &f, 4);
    const int e = (int)((u >> 23) & 255) - 127 + 15;
    return (uint16_t)((e << 10) | ((u >> 13) & 1023));
}

void esq_mtest_blocks(uint32_t t, uint64_t *state, uint8_t *W, int rows, int cols) {
    const int bs = esq_block_elems(t), bb = esq_block_bytes(t);
    const size_t rb = esq_row_bytes(t, cols);
    int dpos = 0, mpos = -1;
    if (t == ESQ_Q6_K) dpos = 208;
    if (t == ESQ_Q3_K) dpos = 108;
    if (t == ESQ_Q4_K || t == ESQ_Q5_K) mpos = 2;   /* es_mtest sets dmin for Q4_K; Q5_K's is placed the same way */
    if (t == ESQ_Q2_K) { dpos = 80; mpos = 82; }
    for (size_t i = 0; i < rb * (size_t)rows; i++) W[i] = (uint8_t)mt_rnd(state);
    for (int r = 0; r < rows; r++)
        for (int b = 0; b < cols / bs; b++) {
            uint8_t *blk = W + (size_t)r * rb + (size_t)b * bb;
            const uint16_t d = mt_f16(0.001f + (float)(mt_rnd(state) % 1000) / 1e5f);
            const uint16_t dm = mt_f16(0.0005f + (float)(mt_rnd(state) % 1000) / 1e5f);
            wr16(blk + dpos, d);
            if (mpos >= 0) wr16(blk + mpos, dm);
        }
}

void esq_mtest_acts(uint64_t *state, float *x, size_t n) {
    for (size_t i = 0; i < n; i++) x[i] = (float)((int)(mt_rnd(state) % 2001) - 1000) / 250.0f;
}

/* ------------------------------------------------------------------------------------------------------------------ */
/* MoE glue                                                                                                            */

int esq_route_softmax(float *r, int ne, int k, int norm_topk, int *sel, float *w) {
    float mx = -INFINITY, sum = 0.0f;   /* src/es_engine.c:752-756 */
    for (int e = 0; e < ne; e++) if (r[e] > mx) mx = r[e];
    for (int e = 0; e < ne; e++) { r[e] = expf(r[e] - mx); sum += r[e]; }
    for (int e = 0; e < ne; e++) r[e] /= sum;
    float wsum = 0.0f;
    for (int j = 0; j < k; j++) {   /* repeated argmax, first maximum wins (src/es_engine.c:794-804) */
        int best = -1;
        for (int e = 0; e < ne; e++) {
            int taken = 0;
            for (int i = 0; i < j; i++) taken |= sel[i] == e;
            if (!taken && (best < 0 || r[e] > r[best])) best = e;
        }
        sel[j] = best;
        w[j] = r[best];
        wsum += w[j];
    }
    if (norm_topk) {   /* src/es_engine.c:832 */
        const float d = wsum > 6.103515625e-5f ? wsum : 6.103515625e-5f;
        for (int j = 0; j < k; j++) w[j] /= d;
    }
    return k;
}

int esq_moe_group(const int *sel, int n_tok, int k, int *uex, int *cnt, int *start, int *rowof, int *tok_of) {
    int nu = 0;   /* src/es_engine.c:871-888 */
    for (int i = 0; i < n_tok * k; i++) {
        int u = 0;
        while (u < nu && uex[u] != sel[i]) u++;
        if (u == nu) { uex[nu] = sel[i]; cnt[nu] = 0; nu++; }
        cnt[u]++;
    }
    int *fill = (int *)calloc((size_t)(nu > 0 ? nu : 1), sizeof(int));
    for (int u = 0, r = 0; u < nu; u++) { start[u] = r; r += cnt[u]; }
    for (int t = 0; t < n_tok; t++)
        for (int j = 0; j < k; j++) {
            int u = 0;
            while (uex[u] != sel[t * k + j]) u++;
            const int r = start[u] + fill[u]++;
            rowof[t * k + j] = r;
            tok_of[r] = t;
        }
    free(fill);
    return nu;
}

void esq_swiglu(const float *g, const float *u, float *h, int n) {
    for (int i = 0; i < n; i++) h[i] = g[i] / (1.0f + expf(-g[i])) * u[i];
}

/* src/es_engine.c:189-194: the sum of squares in double, in element order (each square is exact in double, each sum is
 * rounded); s = (float)(1 / sqrt(ss / n + eps)) in double; o = (x * s) * w in float. The engine is built for baseline
 * x86-64 (no FMA), and this file with -ffp-contract=off, so no operation here is fused. */
void esq_rmsnorm(const float *x, const float *w, float *o, int n, float eps) {
    double ss = 0;
    for (int i = 0; i < n; i++) ss += (double)x[i] * x[i];
    const float s = (float)(1.0 / sqrt(ss / n + eps));
    for (int i = 0; i < n; i++) o[i] = x[i] * s * (w ? w[i] : 1.0f);
}

void esq_moe_combine(const float *ye, const int *rowof, const float *w, int n_tok, int k, int n, float *out) {
    for (int t = 0; t < n_tok; t++)
        for (int i = 0; i < n; i++) {
            float s = 0.0f;
            for (int j = 0; j < k; j++) s = s + w[t * k + j] * ye[(size_t)rowof[t * k + j] * n + i];
            out[(size_t)t * n + i] = s;
        }
}

/* ------------------------------------------------------------------------------------------------------------------ */
/* CPU baseline harness                                                                                                */

void esq_multi_x86_contract(uint32_t t, const void *W, int cols, int r0, int r1, const void *act, size_t astride,
                            int na, float *y, size_t ystride) {
    esq_matvec_multi(t, W, cols, r0, r1, act, astride, na, y, ystride, ESQ_CONTRACT, ESQ_PATH_X86);
}

typedef struct { const float *x; const void *q8; const void *q80; int cols; } ref_act;   /* es_act layout */
typedef void (*ref_multi_t)(uint32_t, const void *, int, int, int, const ref_act *, int, float *, size_t, float *);
static ref_multi_t REF_MULTI;

void esq_bind_reference(void *fn) { REF_MULTI = (ref_multi_t)fn; }

void esq_multi_reference(uint32_t t, const void *W, int cols, int r0, int r1, const void *act, size_t astride, int na,
                         float *y, size_t ystride) {
    static _Thread_local float *scratch;
    static _Thread_local int scratch_n;
    if (scratch_n < cols) {
        free(scratch);
        scratch = (float *)calloc((size_t)cols, sizeof(float));
        scratch_n = scratch ? cols : 0;
    }
    ref_act a[64];
    for (int q0 = 0; q0 < na; q0 += 64) {
        const int n = na - q0 < 64 ? na - q0 : 64;
        for (int q = 0; q < n; q++) {
            const void *blk = (const uint8_t *)act + (size_t)(q0 + q) * astride;
            a[q].x = NULL;
            a[q].q8 = esq_uses_q8K(t) ? blk : NULL;
            a[q].q80 = esq_uses_q8K(t) ? NULL : blk;
            a[q].cols = cols;
        }
        REF_MULTI(t, W, cols, r0, r1, a, n, y + (size_t)q0 * ystride, ystride, scratch);
    }
}

typedef struct {
    esq_multi_fn fn;
    uint32_t type;
    const uint8_t *W;
    size_t mat_bytes;
    int nmat, rows, cols, na, nthreads;
    const uint8_t *act;
    size_t astride;
    float *y;
    double min_seconds;
    pthread_barrier_t bar;
    atomic_long next;
    atomic_int stop;
    int passes;
    double seconds;
} bench_ctx;

typedef struct { bench_ctx *c; int tid; } bench_arg;

static double now_s(void) {
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + (double)ts.tv_nsec * 1e-9;
}

static void *bench_worker(void *p) {
    bench_arg *a = (bench_arg *)p;
    bench_ctx *c = a->c;
    cpu_set_t cs;
    CPU_ZERO(&cs);
    CPU_SET(a->tid, &cs);
    sched_setaffinity(0, sizeof cs, &cs);   /* pin thread i to cpu i; failure leaves it unpinned */
    const long CH = 16;
    double t0 = 0.0;
    for (int pass = 0;; pass++) {
        pthread_barrier_wait(&c->bar);
        if (a->tid == 0 && pass == 0) t0 = now_s();
        if (atomic_load(&c->stop)) break;
        for (int m = 0; m < c->nmat; m++) {
            const uint8_t *W = c->W + (size_t)m * c->mat_bytes;
            for (int q0 = 0; q0 < c->na; q0 += 64) {   /* the engine's batches of at most BMAX = 64 */
                const int nq = c->na - q0 < 64 ? c->na - q0 : 64;
                for (;;) {
                    const long r = atomic_fetch_add(&c->next, CH);
                    if (r >= c->rows) break;
                    const int r1 = (int)(r + CH < c->rows ? r + CH : c->rows);
                    c->fn(c->type, W, c->cols, (int)r, r1, c->act + (size_t)q0 * c->astride, c->astride, nq,
                          c->y + (size_t)q0 * c->rows, (size_t)c->rows);
                }
                if (pthread_barrier_wait(&c->bar) == PTHREAD_BARRIER_SERIAL_THREAD) atomic_store(&c->next, 0);
                pthread_barrier_wait(&c->bar);
            }
        }
        if (a->tid == 0) {
            c->passes = pass + 1;
            c->seconds = now_s() - t0;
            if (c->seconds >= c->min_seconds) atomic_store(&c->stop, 1);
        }
    }
    return NULL;
}

double esq_cpu_bench(esq_multi_fn fn, uint32_t type, const void *W, size_t mat_bytes, int nmat, int rows, int cols,
                     const void *act, size_t astride, int na, float *y, int nthreads, double min_seconds, int *passes) {
    if (nthreads < 1) nthreads = 1;
    bench_ctx c;
    memset(&c, 0, sizeof c);
    c.fn = fn; c.type = type; c.W = (const uint8_t *)W; c.mat_bytes = mat_bytes; c.nmat = nmat; c.rows = rows;
    c.cols = cols; c.na = na; c.nthreads = nthreads; c.act = (const uint8_t *)act; c.astride = astride; c.y = y;
    c.min_seconds = min_seconds;
    atomic_store(&c.next, 0);
    atomic_store(&c.stop, 0);
    pthread_barrier_init(&c.bar, NULL, (unsigned)nthreads);
    pthread_t *th = (pthread_t *)calloc((size_t)nthreads, sizeof(pthread_t));
    bench_arg *args = (bench_arg *)calloc((size_t)nthreads, sizeof(bench_arg));
    for (int i = 0; i < nthreads; i++) {
        args[i].c = &c;
        args[i].tid = i;
        if (i) pthread_create(&th[i], NULL, bench_worker, &args[i]);
    }
    cpu_set_t keep;   /* worker 0 is the calling thread: its own affinity comes back afterwards */
    const int have = sched_getaffinity(0, sizeof keep, &keep) == 0;
    bench_worker(&args[0]);
    for (int i = 1; i < nthreads; i++) pthread_join(th[i], NULL);
    if (have) sched_setaffinity(0, sizeof keep, &keep);
    pthread_barrier_destroy(&c.bar);
    free(th);
    free(args);
    if (passes) *passes = c.passes;
    return c.passes ? c.seconds / c.passes : 0.0;
}
