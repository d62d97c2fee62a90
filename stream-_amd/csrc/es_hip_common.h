// Shared device helpers and the job record of the quantized products. Included by the .hip translation units only.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "es_hip_quant.h"

namespace esq {

constexpr int WAVE = 64;

// Block geometry of the eight formats (reference src/es_quant.c:11-19, src/es_q2k.h:24-38):
//   BE elements per block, BB bytes per block, AB bytes of the matching activation block (Q8_0 36, Q8_K 292),
//   LPB lanes that share one block in the decode kernels.
template <int F> struct Fmt;
template <> struct Fmt<ES_HIP_Q4_0> { static constexpr int BE = 32, BB = 18, AB = 36, LPB = 1; };
template <> struct Fmt<ES_HIP_Q5_0> { static constexpr int BE = 32, BB = 22, AB = 36, LPB = 1; };
template <> struct Fmt<ES_HIP_Q8_0> { static constexpr int BE = 32, BB = 34, AB = 36, LPB = 1; };
template <> struct Fmt<ES_HIP_Q2_K> { static constexpr int BE = 256, BB = 84, AB = 292, LPB = 4; };
template <> struct Fmt<ES_HIP_Q3_K> { static constexpr int BE = 256, BB = 110, AB = 292, LPB = 4; };
template <> struct Fmt<ES_HIP_Q4_K> { static constexpr int BE = 256, BB = 144, AB = 292, LPB = 4; };
template <> struct Fmt<ES_HIP_Q5_K> { static constexpr int BE = 256, BB = 176, AB = 292, LPB = 4; };
template <> struct Fmt<ES_HIP_Q6_K> { static constexpr int BE = 256, BB = 210, AB = 292, LPB = 4; };

// One product handed to a kernel: rows [r0, r1) of W against na activations. Tiles of `rows_per_wg` rows, one per
// workgroup, numbered from tile0 across the jobs of a launch.
struct MvJob {
    const uint8_t *W;     // row 0
    const uint8_t *act;   // activation 0's first block
    float *y;             // activation q's row r at y[q * ystride + r]
    int32_t *ints;        // optional: per (row, block) integer dots of activation 0 (diagnostics), else null
    int32_t *ints_aux;
    const int *arow;      // optional: activation q is row arow[q] of act (a gather), else row q
    uint64_t astride;     // bytes between activations
    uint64_t ystride;     // floats between activations' outputs
    uint64_t row_bytes;
    int r0, r1, cols, na;
    int tile0, rows_per_wg, chain_rows;
    int nt;               // activations per pass (1, 2 or 4): the launch's, or this job's in a launch of mixed widths
    // A row longer than one workgroup's LDS holds is run as consecutive column pieces, one launch each, every piece
    // continuing the chains where the previous one stopped (MV_CHAIN_* flags; 0 for a whole row). The AVX2 order of
    // the 32-element formats carries eight lane chains per output between pieces, in lanes[((q * (r1 - r0) + r - r0) * 8 + i].
    int chain;
    float *lanes;
};
constexpr int MV_CHAIN_IN = 1;          // the chains start from the previous piece's values (y, or lanes)
constexpr int MV_CHAIN_LANES_OUT = 2;   // (AVX2 order, not the last piece) the eight lane chains go to lanes, y untouched

// Floats per row of the decode kernel's LDS terms (nbk blocks, nt activations): the K-quants' 2 per (block, activation)
// plus one, so the pitch is odd; the 32-element formats' 9 per (block, activation).
__host__ __device__ constexpr int mv_row_pitch(bool w32, int nbk, int nt) { return w32 ? nbk * nt * 9 : nbk * nt * 2 + 1; }

// One launch of the decode kernel: format, activations per pass (0: each job's own), waves per workgroup, workgroups,
// LDS bytes.
struct MvLaunch {
    int type, nt, waves;
    int grid;
    size_t lds;
    bool seg_loop = false;   // some row of the launch needs more than `waves` block groups (each wave takes several)
};
hipError_t mv_launch(const MvLaunch &L, const MvJob *jobs, int njobs, const MvJob &single, int order, hipStream_t s);

// Batched 32-wide form (Q4_0 / Q5_0, es_hip_mv.hip): rows [r0, r1) against activations [t0, t0 + ta) of na, one lane per
// (row, activation); ta is a power of two <= 64 and a workgroup of 4 waves covers 4 * 64 / ta rows.
struct MbJob {
    const uint8_t *W;     // row 0
    const uint8_t *act;   // activation 0's first block
    const int *arow;      // optional gather: activation q is row arow[q] of act
    const uint8_t *xq;    // matrix-core form: the activations as a kind 3 pre-pass laid them out (act / arow unused)
    const uint8_t *xm;
    float *y;
    uint64_t astride, ystride, row_bytes;
    int r0, r1, cols, na, t0, ta;
    int tile0, pad_;
};
hipError_t mb32_launch(int type, const MbJob *jobs, int njobs, const MbJob &single, int grid, int order, hipStream_t s);
// The same products on the matrix cores (es_hip_mb.hip): workgroups of 16 rows x activations [t0, t0 + 32), the
// activations read from a kind 3 pre-pass.
constexpr int MB32M_ROWS = 16, MB32M_TOKENS = 32, PREP_KIND_Q80 = 3;
__host__ __device__ constexpr uint32_t prep_words(int kind) { return kind == PREP_KIND_Q80 ? 9u : 19u; }   // items per block
hipError_t mb32m_launch(int type, const MbJob *jobs, int njobs, const MbJob &single, int grid, int order, hipStream_t s);

// The batched (matrix-core) form: rows [r0, r1) against na activations that a pre-pass has re-laid out as
// xq[nbk][na_pad][256] int8 values, then (at xm, in the same allocation) xm[nbk][na_pad][16 or 32] meta and
// xd[nbk][na_pad] float scales right after the xm plane.
constexpr int MM_NA_PAD = 128;    // activation count padding of the pre-pass planes for the prefill kernel
struct MmJob {
    const uint8_t *W;     // row 0
    const uint8_t *xq;
    const uint8_t *xm;
    float *y;
    uint64_t ystride, row_bytes;
    int r0, r1, cols, na, na_pad;
    int tile0, ntok_tiles;
};
// The batched form reading the activations' Q8_K rows directly (es_hip_mk.hip, no pre-pass): rows [r0, r1) against na
// activations, activation q at act + (arow ? arow[q] : q) * astride. Workgroup tiles of MK_ROWS rows x MK_TOK
// activations, numbered from tile0; ntok_tiles activation tiles per row tile. The activation rows of a product must lie
// within 4 GiB of act (32-bit offsets; checked by the host).
// rows per workgroup tile: 64 (two workgroups of 4 waves per CU) or, built with ESQ_MK_ROWS=128, 128 (one of 8 waves)
#ifndef ESQ_MK_ROWS
#define ESQ_MK_ROWS 64
#endif
constexpr int MK_TOK = 128, MK_ROWS = ESQ_MK_ROWS;
struct MkJob {
    const uint8_t *W;     // row 0
    const uint8_t *act;   // activation 0's first block
    const int *arow;      // optional gather
    float *y;
    uint64_t astride, ystride, row_bytes;
    int r0, r1, cols, na;
    int tile0, ntok_tiles;
    int rows_per_wg;      // the batched 32-wide kernel's rows per workgroup tile (1 .. MBX_ROWS), set per job by the host
    int pad_;
    const uint8_t *W2;    // the gated expert kernel: the up projection's row 0 (W is the gate's); y then holds the h rows'
                          // Q8_K blocks (bytes, ystride bytes apart)
};
// Expert-sized Q2_K products (es_hip_mx.hip): the same jobs, workgroup tiles of MX_ROWS rows x MX_TOK activations (ntok_tiles
// per row tile; with one, tile ids are the row tiles themselves), rows of at most MX_NBK superblocks (the whole row's
// activations sit in LDS). nbk_max: the longest row of the launch; mx_nbk_max gives the LDS size class it runs in (0: too
// long).
// rows per workgroup tile: 256 (four waves, two workgroups per CU) or, built with ESQ_MX_ROWS=512, 512 (eight waves, one)
#ifndef ESQ_MX_ROWS
#define ESQ_MX_ROWS 256
#endif
constexpr int MX_TOK = 32, MX_ROWS = ESQ_MX_ROWS, MX_NBK = 16;
// the Q6_K matrix-core kernel's persistent form for single products (es_hip_mm6.hip): on (default) or off; returns the
// previous setting
int mm6_set_persistent(int on);
int mx_nbk_max(int nbk);
// The gated form (a Q2_K expert's gate and up products with the SwiGLU and the Q8_K requantization of h fused in): per
// job, W and W2 the gate's and up's rows, y the first h row's Q8_K blocks (bytes), r0 and r1 multiples of 256
hipError_t mxg_launch(bool gather, int nbk_max, const MkJob *jobs, int njobs, const MkJob &single, int grid, int order,
                      hipStream_t s);
hipError_t mx_launch(int type, bool gather, int nbk_max, const MkJob *jobs, int njobs, const MkJob &single,
                     int grid, int order, hipStream_t s);
// Batched 32-wide formats reading the activations' Q8_0 rows directly (es_hip_mbx.hip): the same jobs, workgroup tiles of
// rows_per_wg (<= MBX_ROWS) rows x MBX_TOK activations on MBX_WAVES waves (tile ids as in the expert-sized kernel), rows of
// at most MBX_NBK blocks (the whole row's activations sit in LDS); mbx_nbk_max gives the LDS size class of a launch's
// longest row (0: too long).
constexpr int MBX_TOK = 32, MBX_ROWS = 32, MBX_NBK = 128, MBX_WAVES = 8;
int mbx_nbk_max(int nbk);
hipError_t mbx_launch(int type, bool gather, int nbk_max, const MkJob *jobs, int njobs, const MkJob &single, int grid,
                      int order, hipStream_t s);
// gather: some job of the launch reads its activation rows through arow (a separate kernel build; the others need not);
// tok: activations per workgroup tile, MK_TOK or 64 (ntok_tiles and the tile numbering then count tiles of 64)
hipError_t mk_launch(int type, bool gather, int tok, const MkJob *jobs, int njobs, const MkJob &single, int grid, int order,
                     hipStream_t s);

// The persistent form of the direct kernel (es_hip_mk.hip): a launch of `grid` workgroups (two per CU) in which workgroup
// g computes the tiles tiles[wgptr[g] .. wgptr[g + 1]) one after another, its loads running ahead across tile
// boundaries. A tile is MK_ROWS rows x 128 (or 64) activations of one product, every address it needs written by the
// host. Products of any row length of at least 2 superblocks (no gathered activations) share one launch.
struct PkTile {
    const uint8_t *w;       // the tile's first weight row
    const uint8_t *act;     // the product's activation 0 (every activation row within 4 GiB of it)
    float *y;               // output of the tile's first activation and first row
    uint32_t astride;       // bytes between activations
    uint32_t ystride4;      // bytes between the outputs of consecutive activations
    uint32_t row_bytes;
    int32_t nbk;            // superblocks per row (>= 2)
    int32_t t64;            // 1: a tile of 64 activations, else 128
    int32_t tok0;           // the tile's first activation
    int32_t na;             // activations of the product (sources past the last repeat it)
    int32_t rows;           // rows of the tile (<= MK_ROWS; rows past them repeat the last and are not stored)
    int32_t ntok;           // activations of the tile (those past it are not stored)
    int32_t pad_;
};
static_assert(sizeof(PkTile) == 64, "tile records are copied into LDS as 16-byte pieces");
constexpr int PK_MAX_TILES = 48;   // tiles per workgroup (their records sit in LDS beside the ring: 80 KB a workgroup)
// workgroups [0, g64) take the tiles of 64 activations, the rest those of 128
hipError_t pk_launch(int type, const PkTile *tiles, const int *wgptr, int grid, int g64, int order, hipStream_t s);
// The wave-specialised form (Q4_K): one workgroup of 8 waves per CU, tiles of 128 activations only.
hipError_t ws_launch(int type, const PkTile *tiles, const int *wgptr, int grid, int order, hipStream_t s);

// One activation pre-pass: kind 0 writes 16 bytes of meta per activation and superblock (pair sums of the Q4_K
// sub-blocks, low | high bytes), kind 1 32 bytes (the 16 bsums, low | high bytes), kind 2 32 bytes (the 16 bsums as
// halves); xd follows the xm plane. Kind 3 takes Q8_0 rows (nbk blocks of 9 dwords: d, 32 int8) and writes, per tile of
// 32 activations and block, the 32 x 32 values as halves, xq[tile][block][q][h][activation n][8 halves] (values
// 16 q + 8 h .. + 7 of activation n: lane 32 h + n of the batched matrix-core kernel reads 16 bytes at 1024 q + 16 * lane
// for its instruction q) and the scales as xm[tile][block][n] floats. All the
// pre-passes of a batch run in one launch over `total` items (one dword of an activation row each), pre-pass i taking
// items [start, start + na_pad*nbk*W) (W = 19 16-byte items per Q8_K block, 9 dwords per Q8_0 block); every start is a multiple of PREP_SPAN, the items of one workgroup.
constexpr int PREP_BLOCK = 256, PREP_UNROLL = 4, PREP_SPAN = PREP_BLOCK * PREP_UNROLL;
struct PrepJob {
    const uint8_t *act;
    const int *arow;
    uint8_t *xq, *xm;
    uint64_t astride;
    long start;
    int na, na_pad, nbk, kind;
};
hipError_t prep_launch(const PrepJob *jobs, int njobs, const PrepJob &single, long total, hipStream_t s);
// hjobs: the same jobs in host memory when the caller has them (the Q6_K form may then launch per job)
hipError_t mm_launch(int type, int bm, int bn, int nw, const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                     hipStream_t s, const MmJob *hjobs = nullptr);
bool mm_tile_ok(int bm, int bn, int nw);   // a workgroup tile (rows x activations, waves) mm_launch has
// The Q6_K form (es_hip_mm6.hip): tiles of 128 rows x 16, 32 or 64 activations on 8 waves
hipError_t mm6_launch(int bm, int bn, int nw, const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                      hipStream_t s, const MmJob *hjobs = nullptr);
// The Q2_K form (es_hip_mm2.hip): tiles of 128 rows x 16, 32 or 64 activations on 8 waves
hipError_t mm2_launch(int bm, int bn, int nw, const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                      hipStream_t s);

// The small-batch matrix-core form (es_hip_mq.hip): rows [r0, r1) against activations [t0, t0 + 16*wn) of na (at most
// 64 per job), from pre-pass planes padded to na_pad activations. One workgroup per 64 rows.
struct MqJob {
    const uint8_t *W;     // row 0
    const uint8_t *xq;    // pre-pass planes (xq, then xm and xd)
    const uint8_t *xm;
    float *y;
    uint64_t ystride, row_bytes;
    int r0, r1, cols, na, na_pad, t0;
    int tile0, pad_;
};
hipError_t mq_launch(int type, int wn, const MqJob *jobs, int njobs, const MqJob &single, int grid, int order, hipStream_t s);

// MoE glue (es_hip_moe.hip): SwiGLU + requantization of rows x ff gate|up pairs ([row][2 ff] floats) into Q8_K (q8k) or
// Q8_0 blocks at ha + row * hstride; the weighted combine of the expert outputs ye[pair][n] into out[t][n].
hipError_t moe_swiglu_launch(const float *gu, int rows, int ff, bool q8k, uint8_t *ha, uint64_t hstride, hipStream_t s);
hipError_t moe_combine_launch(const float *ye, const int *rowof, const float *w, const int *k, int kmax, int ntok, int n,
                              float *out, uint64_t ostride, hipStream_t s);
hipError_t swiglu_plain_launch(const float *g, const float *u, float *h, long n, hipStream_t s);
// route() with softmax gating for ntok tokens of ne <= ROUTE_MAX_EXPERTS logits (rows ls floats apart): sel / w rows of
// kmax, the first k filled (k <= 64).
constexpr int ROUTE_MAX_EXPERTS = 1024;
hipError_t dequant_launch(uint32_t type, const void *src, float *dst, long n, hipStream_t s);
// the float path: rows [r0, r1) of W (row stride rb bytes) against na fp32 activations (x + q * xstride floats), into
// y + q * ystride; es_dequant_row + dot_f32 per output (src/es_quant.c:514-526, 1941-1944)
hipError_t fdot_launch(uint32_t type, const void *W, size_t rb, int r0, int r1, int cols, const float *x, size_t xstride,
                       int na, float *y, size_t ystride, hipStream_t s);
hipError_t route_softmax_launch(const float *logits, uint64_t ls, int ntok, int ne, int k, int norm_topk, int *sel, float *w,
                                int kmax, hipStream_t s);

// Device-routed MoE (es_hip_moe.hip): moe_n's grouping (src/es_engine.c:871-888) and the job tables of one layer's
// gate/up and down launches built on the device from a routing in device memory, so a layer needs no host round trip.
// Every expert product of a launch runs on one kernel family, chosen by the host from the expected tokens per expert:
//   MOE_FAM_MV: the decode kernel (one job per expert slot and product, a fixed number of row tiles each);
//   MOE_FAM_MM: a pre-pass of the expert's gathered activations into its planes (packed one expert after another), then
//               the matrix-core kernel (tiles of 128 rows x bn activations, as many activation tiles as the expert's
//               count needs);
//   MOE_FAM_MX: the expert-sized Q2_K kernel on the gathered Q8_K rows themselves (tiles of MX_ROWS rows x MX_TOK
//               activations: mx_tiles row tiles for an expert of one activation tile, row_tiles8 per activation tile for
//               an expert of several).
// Slots u >= the number of experts used, and one sentinel job at the end of every table, are empty jobs placed after the
// last real tile (the host launches upper-bound grids; their workgroups find an empty job and exit).
constexpr int MOE_FAM_MV = 0, MOE_FAM_MM = 1, MOE_FAM_MX = 2, MOE_GROUP_THREADS = 1024, MOE_MAX_PAIRS = 16384;
struct MoeFamily {
    int kind;
    MvJob mv;              // MV: template job (rows, cols, strides, rows_per_wg, chain_rows); mv_tiles row tiles per job
    int mv_tiles;
    MmJob mm;              // MM: template job; bn activations per tile; row tiles (rounded up to 8, the XCD map)
    PrepJob pj;            // MM: template pre-pass (nbk, kind)
    int bn, row_tiles8;
    MkJob mk;              // MX: template job
    int mx_tiles;
    int gated;             // MX gate/up: the gated kernel (one job per expert slot, h written as Q8_K blocks)
};
struct MoeDevArgs {
    const int *sel;         // [ntok][k] routing (experts)
    const float *w;         // [ntok][k] routing weights
    int ntok, k, n_exp, umax, ff, n;
    const uint8_t *const *gate, *const *up, *const *down;   // device arrays of n_exp expert pointers
    const uint8_t *x;       // gate/up activation blocks, token t at x + t * xstride
    uint64_t xstride, hstride;
    float *bgu;             // [pair row][2 ff]
    uint8_t *ha;            // [pair row] requantized h, hstride bytes apart
    float *bye;             // [pair row][n]
    int *tok_of;            // [pair row] token of the row (the gate/up gather table)
    int *rowof;             // [ntok][k] pair row of each choice
    float *wv;              // [ntok][k] weights as the combine reads them
    void *gu_jobs, *dn_jobs;         // MvJob or MmJob tables: gate/up 2 umax + 1 entries, down umax + 1
    PrepJob *gu_prep, *dn_prep;      // MM: umax + 1 entries each
    uint8_t *gu_ws, *dn_ws;          // MM: the experts' planes, packed in slot order (256-byte aligned)
};
hipError_t moe_group_build_launch(const MoeDevArgs &a, const MoeFamily &gu, const MoeFamily &dn, hipStream_t s);

constexpr int ACT_RMS_MAX_COLS = 16384;   // rmsnorm rows' squares are staged whole in LDS (128 KB of doubles)
// Activation preparation (es_hip_act.hip): rows of fp32 values (plain, rmsnorm-ed, or the SwiGLU of gate|up rows) into
// Q8_0 and / or Q8_K blocks (either output may be null). Float strides in floats, block strides in bytes.
hipError_t act_prep_launch(const float *x, uint64_t xs, int rows, int cols, uint8_t *q80, uint64_t q80s, uint8_t *q8k,
                           uint64_t q8ks, hipStream_t s);
hipError_t act_prep_swiglu_launch(const float *gu, uint64_t gs, int rows, int ff, float *h, uint64_t hs, uint8_t *q80,
                                  uint64_t q80s, uint8_t *q8k, uint64_t q8ks, hipStream_t s);
hipError_t act_prep_rms_launch(const float *x, uint64_t xs, const float *w, float eps, int rows, int cols, float *xn,
                               uint64_t xns, uint8_t *q80, uint64_t q80s, uint8_t *q8k, uint64_t q8ks, hipStream_t s);

__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    // exact for every finite half, subnormals included (v_cvt_f32_f16)
    return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(h & 0xffffu)));
}

__device__ __forceinline__ int sdot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4(static_cast<int>(a), static_cast<int>(b), c, false);
}

// ({hi, lo} >> 8 * sel)[31:0]
__device__ __forceinline__ uint32_t alignbyte(uint32_t hi, uint32_t lo, uint32_t sel) {
    return __builtin_amdgcn_alignbyte(hi, lo, sel);
}

// Device memory accesses through pointers that were loaded from job tables: the pointers are generic (flat) to the
// compiler, which would emit flat loads (slower, and counted against the LDS counter too, so every wait drains both).
// These helpers name the global address space explicitly.
#define ESQ_GLOBAL __attribute__((address_space(1)))
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
template <typename T> __device__ __forceinline__ T ldg(const void *p) {   // 8- and 16-byte types go through native vectors
    if constexpr (sizeof(T) == 16) return __builtin_bit_cast(T, *(const ESQ_GLOBAL u32x4 *)p);
    else if constexpr (sizeof(T) == 8) return __builtin_bit_cast(T, *(const ESQ_GLOBAL u32x2 *)p);
    else return *(const ESQ_GLOBAL T *)p;
}
// 16 bytes of global memory at a 2-byte aligned address (Q3_K and Q6_K superblocks: the hardware's unaligned access)
typedef uint32_t u32x4_a2 __attribute__((ext_vector_type(4), aligned(2)));
__device__ __forceinline__ uint4 ldg_u128_a2(const uint8_t *p) {
    const u32x4_a2 v = *(const ESQ_GLOBAL u32x4_a2 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <typename T> __device__ __forceinline__ void stg(void *p, const T &v) {
    if constexpr (sizeof(T) == 16) *(ESQ_GLOBAL u32x4 *)p = __builtin_bit_cast(u32x4, v);
    else if constexpr (sizeof(T) == 8) *(ESQ_GLOBAL u32x2 *)p = __builtin_bit_cast(u32x2, v);
    else *(ESQ_GLOBAL T *)p = v;
}

// Weight loads. Every weight byte is read once per pass, so ESQ_NT_WEIGHTS=1 marks them non-temporal (streamed past the
// caches); 0 uses ordinary loads. Build-time choice, same results either way.
#ifndef ESQ_NT_WEIGHTS
#define ESQ_NT_WEIGHTS 0
#endif
__device__ __forceinline__ uint4 ldw4(const void *p) {
#if ESQ_NT_WEIGHTS
    const u32x4 v = __builtin_nontemporal_load((const ESQ_GLOBAL u32x4 *)p);
    return make_uint4(v.x, v.y, v.z, v.w);
#else
    return ldg<uint4>(p);
#endif
}
__device__ __forceinline__ uint2 ldw2(const void *p) {
#if ESQ_NT_WEIGHTS
    const u32x2 v = __builtin_nontemporal_load((const ESQ_GLOBAL u32x2 *)p);
    return make_uint2(v.x, v.y);
#else
    return ldg<uint2>(p);
#endif
}

// Sum over groups of G consecutive lanes (G = 1, 2, 4, 8, 16); every lane of a group ends with the group's sum.
// DPP lane moves, no LDS round trip: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror (lane i of each 8 reads
// lane 7 - i), row_mirror (lane i of each 16 reads lane 15 - i). After the two quad steps every lane holds its quad's
// sum; the half mirror pairs each quad with the other quad of its 8 lanes, the mirror each 8 with the other 8 of its 16.
// Integer sums, so the pairing order does not matter.
template <int G> __device__ __forceinline__ int group_sum(int v) {
    if constexpr (G >= 2) v += __builtin_amdgcn_update_dpp(0, v, 0xB1, 0xF, 0xF, false);
    if constexpr (G >= 4) v += __builtin_amdgcn_update_dpp(0, v, 0x4E, 0xF, 0xF, false);
    if constexpr (G >= 8) v += __builtin_amdgcn_update_dpp(0, v, 0x141, 0xF, 0xF, false);
    if constexpr (G >= 16) v += __builtin_amdgcn_update_dpp(0, v, 0x140, 0xF, 0xF, false);
    return v;
}
// The maximum over groups of G consecutive lanes, the same moves (exact in any order)
template <int CTRL> __device__ __forceinline__ float dpp_movf(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}
template <int G> __device__ __forceinline__ float group_max(float v) {
    if constexpr (G >= 2) v = __builtin_fmaxf(v, dpp_movf<0xB1>(v));
    if constexpr (G >= 4) v = __builtin_fmaxf(v, dpp_movf<0x4E>(v));
    if constexpr (G >= 8) v = __builtin_fmaxf(v, dpp_movf<0x141>(v));
    if constexpr (G >= 16) v = __builtin_fmaxf(v, dpp_movf<0x140>(v));
    return v;
}


// ---- matrix-core kernel helpers (es_hip_mm.hip, es_hip_mm6.hip) --------------------------------------------------------
typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float v4f __attribute__((ext_vector_type(4)));

// two 16-bit lanes multiplied (v_pk_mul_lo_u16): four bytes times a small scale at once when no byte product exceeds 255
__device__ __forceinline__ uint32_t pk_mul_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, b));
}

// The job of workgroup bid in a launch whose jobs hold consecutive tile ranges from tile0 (the last job with
// tile0 <= bid). When the jobs are of equal size (an MoE layer's experts, copies of one matrix) the proportional guess
// is that job: the guessed job itself and the next job's tile0 are independent loads, so the job arrives in the same
// round trip that checks it; otherwise a binary search and a second load follow.
template <typename JobT> __device__ __forceinline__ JobT load_tile_job(const JobT *jobs, int njobs, int bid) {
    static_assert(sizeof(JobT) % 8 == 0, "jobs are read as 8-byte pieces");
    constexpr int N = sizeof(JobT) / 8;
    const int g = min(njobs - 1, static_cast<int>((static_cast<long>(bid) * njobs) / static_cast<long>(gridDim.x)));
    const int b = g + 1 < njobs ? jobs[g + 1].tile0 : 0x7fffffff;
    uint64_t v[N];
    const uint64_t *src = reinterpret_cast<const uint64_t *>(jobs + g);
#pragma unroll
    for (int i = 0; i < N; i++) v[i] = src[i];
    // every piece is needed here, before the check: otherwise the compiler loads the guessed job's tile0 alone, checks
    // it, and only then the rest of the job (a second round trip)
#pragma unroll
    for (int i = 0; i < N; i++) asm volatile("" ::"s"(v[i]));
    const JobT J = __builtin_bit_cast(JobT, v);
    if (J.tile0 <= bid && bid < b) return J;
    int lo = 0, hi = njobs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (jobs[mid].tile0 <= bid) lo = mid; else hi = mid - 1;
    }
    return jobs[lo];
}

// One wave's 64 x 16 bytes from global memory straight into LDS: lane l's 16 bytes at base + off land at lds + 16*l
// (lds is wave-uniform). Written as inline assembly so that the compiler does not track these LDS writes: it would
// otherwise wait for every one of them to finish before any LDS read. The kernel orders them itself (s_waitcnt vmcnt +
// s_barrier before a stage is read). M0 is set inside the statement; nothing else in these kernels uses M0.
__device__ __forceinline__ void load_lds16(const uint8_t *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory");
}
// The same for 4 bytes per lane (global_load_lds_dword): lane l's dword at base + off lands at lds + 4*l.
__device__ __forceinline__ void load_lds4(const uint8_t *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

// A workgroup barrier that orders LDS only: every wave's LDS accesses before it are complete, and nothing waits for the
// wave's global loads and stores (for kernels where no wave reads global memory another wave of it wrote; copies into LDS
// by global_load_lds are waited for separately, with s_waitcnt vmcnt).
__device__ __forceinline__ void lds_sync() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

template <int N> __device__ __forceinline__ void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
// s_waitcnt vmcnt(n * L) for a wave-uniform n in 0 .. NMAX
template <int L, int NMAX> __device__ __forceinline__ void wait_stages(int n) {
    if constexpr (NMAX > 0) {
        if (n >= NMAX) { wait_vmcnt<L * NMAX>(); return; }
        wait_stages<L, NMAX - 1>(n);
    } else {
        wait_vmcnt<0>();
    }
}

}  // namespace esq
