// Batched Q6_K products on the int8 matrix cores: the prompt-reading form of es_matvec_multi (src/es_quant.c:1818-1850)
// for Q6_K rows against 16 or more activations (e.g. an output head over a prompt tail). The reference forms, per row,
// activation and superblock, tot = sum sc * q_u * x - 32 * sum_g sc_g * bsums_g with q_u the unsigned 6-bit code, then
// s += (y.d * d) * tot (src/es_quant.c:1602-1640).
//
// The products q_u * sc (up to 63 * 128 in size) do not fit int8. With sc_u = sc + 128 = 16h + l and q_u = 8a + b (h, l
// in 0..15, a, b in 0..7):  q_u * sc = q_u * sc_u - 128 q_u = 128 (a h - q_u) + 16 b h + 8 a l + b l,
// four int8 planes (a h - q_u in -63..105, the others in 0..105) through the matrix cores, recombined exactly in int32:
//   sum q_u * sc * x = 128 D(ah - q_u) + 16 D(bh) + 8 D(al) + D(bl).
// corr = sum_g sc_g * bsums_g goes through one f16 MFMA (scales and bsums are exact halves and every partial sum stays
// below 2^24: exact).
//
// Weights: a 210-byte superblock starts 2-byte aligned. Each row's superblock is read with 16-byte loads at 2-byte aligned
// addresses (the hardware's unaligned global access) and a 2-byte load of d, and written to LDS as an aligned 208-byte
// row (ql | qh | scales) plus d in a separate array. Activations come through the same registers-to-LDS path, from the
// pre-pass planes. Rows must be 4-byte aligned (an even number of superblocks).
// K order: MFMA slice ks (0..3) and lane group lg (0..3) take scale group g = 4 ks + lg: with n = ks >> 1, qn = ks & 1,
// qo = lg >> 1, lh = lg & 1, the 16 elements 128 n + 32 (2 qn + qo) + 16 lh + [0, 16), whose low 4 bits are nibble qn of
// ql[64 n + 32 qo + 16 lh + i] and high 2 bits field 2 qn + qo of qh[32 n + 16 lh + i] (src/es_quant.c:158-176). The
// activation operand is the natural 16-element chunk g of the activation row, as in the pre-pass planes.
#include "es_hip_common.h"

#include <algorithm>
#include <atomic>

namespace esq {

template <int RW, int TW, int WN> struct Mm6Geom {
    static constexpr int NW = RW * TW, NT = 64 * NW, BM = 16 * RW, BN = 16 * WN * TW;
    // stage: weight rows BM x 208 (ql | qh | scales) | d BM x 2 | activations BN x 256 | bsums BN x 32 | scales BN x 4
    static constexpr int CW = BM * 13, CX = BN * 18 + BN / 4;          // 16-byte chunks
    static constexpr int D_W = BM * 208, X_OFF = D_W + (BM * 2 + 15) / 16 * 16;
    static constexpr int M_OFF = X_OFF + BN * 256, D_OFF = M_OFF + BN * 32, STAGE = D_OFF + (BN * 4 + 15) / 16 * 16;
    static constexpr int SW = (CW + NT - 1) / NT, SX = (CX + NT - 1) / NT;   // chunks per thread
    static constexpr int LDS = 2 * STAGE;
    // persistent form: two stages of weights (and d) only, then the activations of every superblock (NBKP at most)
    static constexpr int WST = X_OFF, XSB = STAGE - X_OFF, ACT0 = 2 * WST, NBKP = (160 * 1024 - ACT0) / XSB;
    static constexpr int LDSP = ACT0 + NBKP * XSB;
    static_assert(NW == 8, "8 waves");
    static_assert(LDS <= 160 * 1024 && LDSP <= 160 * 1024, "two stages fit the LDS");
    static_assert(BM <= NT, "one d per thread");
};

// RW x TW waves: RW along the rows, TW along the activations; WN: 16 x 16 MFMA tiles per wave along the activations.
// CONTRACT: the clang order (fused multiply-adds), else the gcc / scalar order.
// PERS: the persistent form for one product of one activation tile with at most NBKP superblocks per row (config 3's
// head at 64 activations): a workgroup per CU takes row tiles blockIdx.x, + gridDim.x, ...; the activations of every
// superblock are copied into LDS once, and the weights of (row tile, superblock) items stream through the two stages
// back to back, so no row tile pays the pipeline's start (job lookup, first loads, first stage write) again.
template <int RW, int TW, int WN, bool CONTRACT, bool PERS>
__global__ __launch_bounds__(64 * RW * TW) void mm_q6k_kernel(const MmJob *__restrict__ jobs, int njobs, MmJob single) {
    using G = Mm6Geom<RW, TW, WN>;
    __shared__ __align__(16) uint8_t smem[PERS ? G::LDSP : G::LDS];

    MmJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    int rt, tt, ntile;
    if constexpr (PERS) {   // row tiles blockIdx.x + i * gridDim.x, i < ntile; one activation tile
        const int rtiles = (J.r1 - J.r0 + G::BM - 1) / G::BM;
        rt = blockIdx.x;
        tt = 0;
        ntile = rt < rtiles ? (rtiles - 1 - rt) / (int)gridDim.x + 1 : 0;
        if (ntile == 0) return;
    } else {
        // XCD-aware tile order, as in the Q4_K kernel: all activation tiles of row tile rt on one XCD
        const int tile = blockIdx.x - J.tile0;
        const int x = tile & 7, kq = tile >> 3;
        rt = x + 8 * (kq / J.ntok_tiles);
        tt = kq % J.ntok_tiles;
        ntile = 1;
        if (rt * G::BM >= J.r1 - J.r0) return;
    }
    const int tok0 = tt * G::BN;
    const int nbk = J.cols / 256;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int wr = (wave % RW) * 16, wt = (wave / RW) * 16 * WN;   // this wave's rows / activations in the tile
    const int lr = lane & 15, lg = lane >> 4;

    // ---- this thread's share of a stage: weight chunk c = tid + NT*k (row c / 13, 16-byte piece c % 13 of its first 208
    // bytes; rows past the end repeat the last one, their results are not stored), d of row tid, activation chunk
    // tid + NT*k (values, swizzled: chunk q of activation t at slot q ^ (t & 15); bsums; scales, four activations a chunk)
    // (PERS: the chunk's row and piece, clamped per row tile at each load; else the chunk's offset in the one row tile)
    const int row00 = J.r0 + rt * G::BM;
    uint32_t wsrc[G::SW], wdst[G::SW], xsrc[G::SX], xstep[G::SX], xdst[G::SX];
    bool wok[G::SW], xok[G::SX];
#pragma unroll
    for (int k = 0; k < G::SW; k++) {
        const int c = tid + G::NT * k;
        wok[k] = c < G::CW;
        wsrc[k] = PERS ? (uint32_t)(c / 13) << 8 | (uint32_t)(16 * (c % 13))
                       : (uint32_t)min(c / 13, J.r1 - 1 - row00) * (uint32_t)J.row_bytes + 16 * (c % 13);
        wdst[k] = 16 * c;
    }
    const bool dok = tid < G::BM;
    const uint32_t xm_rel = (uint32_t)(J.xm - J.xq), xd_rel = xm_rel + (uint32_t)nbk * J.na_pad * 32;
#pragma unroll
    for (int k = 0; k < G::SX; k++) {
        const int c = tid + G::NT * k;
        xok[k] = c < G::CX;
        if (c < G::BN * 16) {
            const int t = c >> 4, q = c & 15;
            xsrc[k] = (uint32_t)(tok0 + t) * 256 + 16 * q;
            xstep[k] = (uint32_t)J.na_pad * 256;
            xdst[k] = G::X_OFF + t * 256 + 16 * (q ^ (t & 15));
        } else if (c < G::BN * 18) {
            const int cm = c - G::BN * 16;
            xsrc[k] = xm_rel + (uint32_t)(tok0 + (cm >> 1)) * 32 + 16 * (cm & 1);
            xstep[k] = (uint32_t)J.na_pad * 32;
            xdst[k] = G::M_OFF + 16 * cm;
        } else {
            const int t4 = min(c - G::BN * 18, G::BN / 4 - 1);
            xsrc[k] = xd_rel + (uint32_t)(tok0 + 4 * t4) * 4;
            xstep[k] = (uint32_t)J.na_pad * 4;
            xdst[k] = G::D_OFF + 16 * t4;
        }
    }
    // item it = (row tile rt + (it / nbk) * gridDim.x, superblock it % nbk): the global loads of its weights (and, unless
    // PERS, of its activations) into registers, and their LDS writes into stage st
    constexpr int STG = PERS ? G::WST : G::STAGE;
    uint4 rw[G::SW], rx[G::SX];
    uint32_t rd = 0;
    auto gload = [&](int it) {
        const int ti = PERS ? it / nbk : 0, bi = it - ti * nbk;
        const int row0 = row00 + ti * (int)gridDim.x * G::BM, last_row = J.r1 - 1 - row0;
        const uint8_t *wbase = J.W + (size_t)row0 * J.row_bytes + 210u * bi;
#pragma unroll
        for (int k = 0; k < G::SW; k++) {
            if (!wok[k]) continue;
            if constexpr (PERS)
                rw[k] = ldg_u128_a2(wbase + (uint32_t)min((int)(wsrc[k] >> 8), last_row) * (uint32_t)J.row_bytes + (wsrc[k] & 255u));
            else
                rw[k] = ldg_u128_a2(wbase + wsrc[k]);
        }
        if (dok) rd = ldg<uint16_t>(wbase + (uint32_t)min(tid, last_row) * (uint32_t)J.row_bytes + 208);
        if constexpr (!PERS) {
#pragma unroll
            for (int k = 0; k < G::SX; k++)
                if (xok[k]) rx[k] = ldg<uint4>(J.xq + xsrc[k] + (uint32_t)bi * xstep[k]);
        }
    };
    auto lstore = [&](int st) {
        uint8_t *sb = smem + st * STG;
#pragma unroll
        for (int k = 0; k < G::SW; k++)
            if (wok[k]) *reinterpret_cast<uint4 *>(sb + wdst[k]) = rw[k];
        if (dok) *reinterpret_cast<uint16_t *>(sb + G::D_W + 2 * tid) = (uint16_t)rd;
        if constexpr (!PERS) {
#pragma unroll
            for (int k = 0; k < G::SX; k++)
                if (xok[k]) *reinterpret_cast<uint4 *>(sb + xdst[k]) = rx[k];
        }
    };
    if constexpr (PERS) {   // every superblock's activations into their own LDS region, once
        for (int bi = 0; bi < nbk; bi++) {
#pragma unroll
            for (int k = 0; k < G::SX; k++)
                if (xok[k]) rx[k] = ldg<uint4>(J.xq + xsrc[k] + (uint32_t)bi * xstep[k]);
#pragma unroll
            for (int k = 0; k < G::SX; k++)
                if (xok[k]) *reinterpret_cast<uint4 *>(smem + G::ACT0 + bi * G::XSB + (xdst[k] - G::X_OFF)) = rx[k];
        }
    }

    uint32_t xo[4];   // activation chunk offsets of this lane in a stage (tile c adds 4096*c): chunk 4ks + lg
#pragma unroll
    for (int ks = 0; ks < 4; ks++) xo[ks] = G::X_OFF + (wt + lr) * 256 + 16 * ((4 * ks + lg) ^ lr);
    const uint32_t mo = G::M_OFF + (wt + lr) * 32 + 16 * (lg & 1), dof = G::D_OFF + (wt + lr) * 4;
    const int qo = lg >> 1, lh = lg & 1;
    const uint32_t rowoff = (wr + lr) * 208, ddoff = G::D_W + (wr + 4 * lg) * 2;
    const uint32_t sel = 0x0c000c00u + (uint32_t)lg * 0x00010001u;   // byte lg of a word into both 16-bit halves

    float s[WN][4];
#pragma unroll
    for (int c = 0; c < WN; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) s[c][i] = 0.0f;

    // Two stages. Item it+1's loads went out during item it-1 (into registers); at the top of it they are written to
    // stage (it+1) & 1, whose last readers finished it-1 (barrier), and item it+2's loads go out.
    const int nitem = ntile * nbk;
    gload(0);
    lstore(0);
    if (nitem > 1) gload(1);
    for (int it = 0; it < nitem; it++) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's LDS writes of stage it and reads of it-1 are done
        __builtin_amdgcn_s_barrier();                         // ... and every wave's
        asm volatile("" ::: "memory");
        const int ti = PERS ? it / nbk : 0, b = it - ti * nbk;
        const uint8_t *wb = smem + (it & 1) * STG;
        // the activation operands: in the stage, or (PERS) in superblock b's region, addressed as if it were a stage
        const uint8_t *xb = PERS ? smem + G::ACT0 + b * G::XSB - G::X_OFF : wb;
        if (it + 1 < nitem) {
            lstore((it + 1) & 1);
            if (it + 2 < nitem) gload(it + 2);
        }
        __builtin_amdgcn_sched_barrier(0);   // the loads stay here, a whole item ahead of their LDS writes

        // LDS reads in the order they are needed: the weight fields, the row scales, then activation tile 0
        const uint8_t *rowp = wb + rowoff;
        auto ld16 = [&](int off) { return *reinterpret_cast<const uint4 *>(rowp + off); };
        const uint4 ql0 = ld16(32 * qo + 16 * lh), ql1 = ld16(64 + 32 * qo + 16 * lh);
        const uint4 qh0 = ld16(128 + 16 * lh), qh1 = ld16(160 + 16 * lh), scw = ld16(192);
        float dv[4];   // d of this lane's four output rows
#pragma unroll
        for (int i = 0; i < 4; i++) dv[i] = half_bits_to_float(*reinterpret_cast<const uint16_t *>(wb + ddoff + 2 * i));
        struct Bt { v4i x[4]; v8h m; float td; };
        auto load_b = [&](int c, Bt &B) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) B.x[ks] = *reinterpret_cast<const v4i *>(xb + xo[ks] + 4096 * c);
            B.m = *reinterpret_cast<const v8h *>(xb + mo + 512 * c);
            B.td = *reinterpret_cast<const float *>(xb + dof + 64 * c);
        };
        Bt B[2];
        load_b(0, B[0]);

        // ---- A operands: per slice ks the four planes, and the scales as halves for corr
        const uint32_t u[4] = {scw.x ^ 0x80808080u, scw.y ^ 0x80808080u, scw.z ^ 0x80808080u, scw.w ^ 0x80808080u};   // sc + 128
        v4i p1[4], p2[4], p3[4], p4[4];
        // the qh dwords shifted by this lane's field pair once (2 qo bits): field 2 qn + qo of each byte then sits at bits
        // 4 qn .. 4 qn + 1, so slice ks takes it with one shift (qn = 0) or none (qn = 1)
        const uint32_t qs0[4] = {qh0.x >> (2 * qo), qh0.y >> (2 * qo), qh0.z >> (2 * qo), qh0.w >> (2 * qo)};
        const uint32_t qs1[4] = {qh1.x >> (2 * qo), qh1.y >> (2 * qo), qh1.z >> (2 * qo), qh1.w >> (2 * qo)};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int n = ks >> 1, qn = ks & 1;
            const uint32_t lsc = __builtin_amdgcn_perm(0, u[ks] & 0x0f0f0f0fu, sel);          // l, in both halves
            const uint32_t hsc = __builtin_amdgcn_perm(0, (u[ks] >> 4) & 0x0f0f0f0fu, sel);   // h
            const uint4 qlv = n ? ql1 : ql0;
            const uint32_t qlw[4] = {qlv.x, qlv.y, qlv.z, qlv.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t nib = qn ? (qlw[i] >> 4) & 0x0f0f0f0fu : qlw[i] & 0x0f0f0f0fu;
                const uint32_t qsw = n ? qs1[i] : qs0[i];
                const uint32_t qu = nib | ((qn ? qsw : qsw << 4) & 0x30303030u);   // 6-bit codes, one per byte
                const uint32_t a = (qu >> 3) & 0x07070707u, bb = qu & 0x07070707u;
                // a h - q_u per byte: (a h + 128 - q_u) stays in 65..233, so no borrow crosses a byte
                p1[ks][i] = (int)(((pk_mul_u16(a, hsc) | 0x80808080u) - qu) ^ 0x80808080u);
                p2[ks][i] = (int)pk_mul_u16(a, lsc);
                p3[ks][i] = (int)pk_mul_u16(bb, hsc);
                p4[ks][i] = (int)pk_mul_u16(bb, lsc);
            }
        }
        // corr operand (halves): lanes 0..15 carry sc_0..7, lanes 16..31 sc_8..15 (k positions meet bsums 0..7 / 8..15);
        // lanes 32..63 zero. Each half is built as 1024 + sc_u (byte under the exponent of 1024), then 1152 subtracted.
        v8h acorr;
        {
            const uint32_t w0 = lg == 0 ? u[0] : u[2], w1 = lg == 0 ? u[1] : u[3];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t k0 = (2 * e) & 3;
                const uint32_t pr = __builtin_amdgcn_perm(0x64646464u, e < 2 ? w0 : w1,
                                                          k0 | 0x0400u | (k0 + 1) << 16 | 0x04000000u);
                const h2 v = __builtin_bit_cast(h2, pr) + __builtin_bit_cast(h2, 0xe480e480u);   // - 1152
                acorr[2 * e] = v[0];
                acorr[2 * e + 1] = v[1];
            }
            if (lg >= 2) acorr = v8h{0, 0, 0, 0, 0, 0, 0, 0};
        }

        v4i d1[2], d2[2], d3[2], d4[2];
        v4f dc[2];
        float tdv[2];
        auto mma = [&](int c, const Bt &Bc) {
            const int w = c & 1;
            tdv[w] = Bc.td;
            dc[w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(acorr, Bc.m, v4f{0, 0, 0, 0}, 0, 0, 0);
            d1[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(p1[0], Bc.x[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            d2[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(p2[0], Bc.x[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            d3[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(p3[0], Bc.x[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            d4[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(p4[0], Bc.x[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int ks = 1; ks < 4; ks++) {
                d1[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(p1[ks], Bc.x[ks], d1[w], 0, 0, 0);
                d2[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(p2[ks], Bc.x[ks], d2[w], 0, 0, 0);
                d3[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(p3[ks], Bc.x[ks], d3[w], 0, 0, 0);
                d4[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(p4[ks], Bc.x[ks], d4[w], 0, 0, 0);
            }
        };
        // fp32 epilogue of superblock b for tile c, per (row, activation), in the reference's order
        auto epi = [&](int c) {
            const int w = c & 1;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int tot = d4[w][i] + 8 * d2[w][i] + 16 * d3[w][i] + 128 * d1[w][i] - 32 * (int)dc[w][i];
                const float f = tdv[w] * dv[i];
                if constexpr (CONTRACT) s[c][i] = __builtin_fmaf(f, static_cast<float>(tot), s[c][i]);
                else s[c][i] = s[c][i] + f * static_cast<float>(tot);
            }
        };
        // one scheduling group per tile: tile c+1's LDS reads, tile c's matrix work and tile c-1's epilogue, interleaved as
        // 1 MFMA : 2 VALU (: 1 LDS read)
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < WN; c++) {
            if (c + 1 < WN) load_b(c + 1, B[(c + 1) & 1]);
            mma(c, B[c & 1]);
            if (c) epi(c - 1);
#pragma unroll
            for (int k = 0; k < 17; k++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // VALU
                if (k < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        epi(WN - 1);
        asm volatile("" ::: "memory");   // stage it's LDS reads stay before the next item's barrier

        if (b == nbk - 1) {   // ---- the row tile's outputs
            const int row0 = row00 + ti * (int)gridDim.x * G::BM;
#pragma unroll
            for (int c = 0; c < WN; c++) {
                const int t = tok0 + wt + 16 * c + lr;
                if (t < J.na) {
                    const int r = row0 + wr + 4 * lg;   // this lane holds rows r .. r+3 of activation t
                    float *yp = J.y + (size_t)t * J.ystride + r;
                    if (r + 3 < J.r1 && (reinterpret_cast<uintptr_t>(yp) & 15) == 0) {
                        stg<float4>(yp, make_float4(s[c][0], s[c][1], s[c][2], s[c][3]));
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; i++)
                            if (r + i < J.r1) stg<float>(yp + i, s[c][i]);
                    }
                }
#pragma unroll
                for (int i = 0; i < 4; i++) s[c][i] = 0.0f;
            }
        }
    }
}

std::atomic<int> g_mm6_persistent{1};

template <int RW, int TW, int WN>
static hipError_t mm6_launch_cfg(const MmJob *jobs, int njobs, const MmJob &single, int grid, int order, hipStream_t s,
                                 const MmJob *hjobs) {
    using G = Mm6Geom<RW, TW, WN>;
    const bool contract = order == ES_HIP_ORDER_X86_CONTRACT;
    static const int ncu = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            n = 256;
        return n > 0 ? n : 256;
    }();
    // The persistent form, one launch per product with a workgroup per CU: for a lone product of one activation tile with
    // short rows, or for a few such products each of at least two row tiles per CU (a head or projection per call, or
    // their copies in one batch). Otherwise the tiled form.
    auto rtiles = [](const MmJob &j) { return (j.r1 - j.r0 + G::BM - 1) / G::BM; };
    auto fits = [&](const MmJob &j) { return j.ntok_tiles == 1 && j.cols / 256 <= G::NBKP; };
    bool pers = g_mm6_persistent.load() && (njobs == 1 ? fits(single) : hjobs != nullptr && njobs <= 16);
    for (int i = 0; pers && njobs > 1 && i < njobs; i++) pers = fits(hjobs[i]) && rtiles(hjobs[i]) >= 2 * ncu;
    if (pers) {
        const dim3 b(64 * RW * TW);
        for (int i = 0; i < njobs; i++) {
            const MmJob &j = njobs == 1 ? single : hjobs[i];
            const dim3 g(std::min(rtiles(j), ncu));
            if (contract) hipLaunchKernelGGL((mm_q6k_kernel<RW, TW, WN, true, true>), g, b, 0, s, nullptr, 1, j);
            else hipLaunchKernelGGL((mm_q6k_kernel<RW, TW, WN, false, true>), g, b, 0, s, nullptr, 1, j);
        }
        return hipGetLastError();
    }
    if (contract)
        hipLaunchKernelGGL((mm_q6k_kernel<RW, TW, WN, true, false>), dim3(grid), dim3(64 * RW * TW), 0, s, jobs, njobs, single);
    else
        hipLaunchKernelGGL((mm_q6k_kernel<RW, TW, WN, false, false>), dim3(grid), dim3(64 * RW * TW), 0, s, jobs, njobs, single);
    return hipGetLastError();
}

int mm6_set_persistent(int on) { return g_mm6_persistent.exchange(on ? 1 : 0); }

// Q6_K workgroup tiles: 128 rows x 16, 32 or 64 activations on 8 waves (16 rows x all the activations each)
bool mm6_tile_ok(int bm, int bn, int nw) { return nw == 8 && bm == 128 && (bn == 16 || bn == 32 || bn == 64); }

hipError_t mm6_launch(int bm, int bn, int nw, const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                      hipStream_t s, const MmJob *hjobs) {
    if (nw == 8 && bm == 128) {
        if (bn == 64) return mm6_launch_cfg<8, 1, 4>(jobs, njobs, single, grid, order, s, hjobs);
        if (bn == 32) return mm6_launch_cfg<8, 1, 2>(jobs, njobs, single, grid, order, s, hjobs);
        if (bn == 16) return mm6_launch_cfg<8, 1, 1>(jobs, njobs, single, grid, order, s, hjobs);
    }
    return hipErrorInvalidValue;
}

}  // namespace esq
