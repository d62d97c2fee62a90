// Batched Q2_K products on the int8 matrix cores: es_matvec_multi (src/es_quant.c:1818-1850) for Q2_K rows against 8 or
// more activations (MoE experts, prompt tails). Per row, activation and superblock the reference forms
// isum = sum_g (sc_g & 15) * sum q2 * x and summs = sum_g (sc_g >> 4) * bsums_g, then
// s += y.d * d * isum - y.d * dmin * summs (src/es_q2k.c:127-148, src/es_quant.c:1344-1368).
//
// q2 * (sc & 15) <= 45 is one int8 plane through the matrix cores; summs goes through one f16 MFMA (the 4-bit mins and the
// bsums are exact halves, every partial sum below 2^24: exact).
//
// Weights: an 84-byte superblock starts 4-byte aligned. Each row's superblock is staged as the six 16-byte aligned chunks
// that cover it (from its start rounded down to 16). Every chunk holds bytes of the superblock, so it lies within their
// memory page; the extra bytes are never used. The superblock then starts at offset o = start mod 16 of its row's 96-byte
// LDS stretch. The activation operands come from the pre-pass planes (values, bsums as halves, scales) through the same
// global-to-LDS loads. Small stages, so that two workgroups share a CU and one's loads overlap the other's work.
//
// K order (as in the vector kernels): MFMA slice ks (0..3), lane group lg (0..3) take group g = 4 ks + lg, the elements
// 16 g + [0, 16): bits 2 (2 (ks & 1) + (lg >> 1)) of qs[32 (ks >> 1) + 16 (lg & 1) + i].
#include "es_hip_common.h"

namespace esq {

template <int RW, int TW, int WN, int NST> struct Mm2Geom {
    static constexpr int NW = RW * TW, BM = 16 * RW, BN = 16 * WN * TW;
    static constexpr int RB = 96;                                        // staged bytes per row: 6 aligned chunks
    static constexpr int NWLW = (BM * 6 + 63) / 64;                      // wave-loads of weights (1 KB each)
    static constexpr int CX = BN * 18 + BN / 4, NWLX = (CX + 63) / 64;   // 16-byte activation chunks, their wave-loads
    static constexpr int X_OFF = NWLW * 1024, M_OFF = X_OFF + BN * 256, D_OFF = M_OFF + BN * 32;
    static constexpr int STAGE = X_OFF + NWLX * 1024;
    static constexpr int LW = (NWLW + NW - 1) / NW, LX = (NWLX + NW - 1) / NW, LOADS = LW + LX;   // per wave per stage
    static constexpr int SINK = NST * STAGE, LDS = SINK + 1024;          // the stages and a sink for the spare loads
    static constexpr int PER_TILE = (LOADS + WN - 1) / WN;               // loads issued with each activation tile
    static_assert(NW == 8, "8 waves");
    static_assert(NST >= 2 && LDS <= 160 * 1024, "stages fit the LDS");
    static_assert(LOADS * (NST - 2) <= 63, "vmcnt range");
};


// RW x TW waves: RW along the rows, TW along the activations; WN: 16 x 16 MFMA tiles per wave along the activations;
// NST: LDS stages. CONTRACT: the clang order (fused multiply-adds), else the gcc / scalar order.
template <int RW, int TW, int WN, int NST, int OCC, bool CONTRACT>
__global__ __launch_bounds__(64 * RW * TW, OCC) void mm_q2k_kernel(const MmJob *__restrict__ jobs, int njobs, MmJob single) {
    using G = Mm2Geom<RW, TW, WN, NST>;
    static_assert(OCC == 1 || G::LDS <= 80 * 1024, "two workgroups per CU");
    __shared__ __align__(16) uint8_t smem[G::LDS];

    MmJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    // XCD-aware tile order, as in the Q4_K kernel: all activation tiles of row tile rt on one XCD
    const int tile = blockIdx.x - J.tile0;
    const int x = tile & 7, kq = tile >> 3;
    const int rt = x + 8 * (kq / J.ntok_tiles), tt = kq % J.ntok_tiles;
    if (rt * G::BM >= J.r1 - J.r0) return;
    const int row0 = J.r0 + rt * G::BM, tok0 = tt * G::BN;
    const int nbk = J.cols / 256;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wr = (wave % RW) * 16, wt = (wave / RW) * 16 * WN;   // this wave's rows / activations in the tile
    const int lr = lane & 15, lg = lane >> 4;
    const uint32_t lds0 = lds_addr(smem);

    // ---- per-lane sources of this wave's stage loads. Weight wave-load L (16-byte chunks 64L .. 64L+63 of a stage): chunk
    // c is chunk c % 6 of row c / 6's stretch, at ((mis + row * row_bytes + 84b) & ~15) + 16(c % 6) from the aligned
    // base wal = J.W - mis (rows past the end repeat the last one; their results are not stored). Activation wave-load L:
    // the three planes of one workspace allocation, base J.xq, + the plane stride per superblock.
    const uint32_t mis = (uint32_t)(reinterpret_cast<uintptr_t>(J.W) & 15);
    const uint8_t *wal = J.W - mis;
    const uint32_t mrow0 = mis + (uint32_t)row0 * (uint32_t)J.row_bytes;   // byte of row row0 from wal
    const uint32_t xm_rel = (uint32_t)(J.xm - J.xq), xd_rel = xm_rel + (uint32_t)nbk * J.na_pad * 32;
    const int last_row = J.r1 - 1 - row0;
    uint32_t offw[G::LW], cw[G::LW], offx[G::LX], stepx[G::LX];
    bool livew[G::LW], livex[G::LX];
#pragma unroll
    for (int kk = 0; kk < G::LW; kk++) {
        const int L = wave + G::NW * kk, c = 64 * L + lane;
        livew[kk] = c < G::BM * 6;
        offw[kk] = mrow0 + (uint32_t)min(c / 6, last_row) * (uint32_t)J.row_bytes;   // + 84b, rounded down, + 16 (c % 6)
        cw[kk] = 16 * (c % 6);
    }
#pragma unroll
    for (int kk = 0; kk < G::LX; kk++) {
        const int L = wave + G::NW * kk, c = 64 * L + lane;
        livex[kk] = c < G::CX;
        if (c < G::BN * 16) {
            const int t = c >> 4, q = (c & 15) ^ (t & 15);   // chunk q of activation t at slot q ^ (t & 15)
            offx[kk] = (uint32_t)(tok0 + t) * 256 + 16 * q;
            stepx[kk] = (uint32_t)J.na_pad * 256;
        } else if (c < G::BN * 18) {
            const int cm = c - G::BN * 16;
            offx[kk] = xm_rel + (uint32_t)(tok0 + (cm >> 1)) * 32 + 16 * (cm & 1);
            stepx[kk] = (uint32_t)J.na_pad * 32;
        } else {
            const int t4 = min(c - G::BN * 18, G::BN / 4 - 1);
            offx[kk] = xd_rel + (uint32_t)(tok0 + 4 * t4) * 4;
            stepx[kk] = (uint32_t)J.na_pad * 4;
        }
    }
    const uint32_t offw0 = (offw[0] & ~15u) + cw[0];   // an aligned chunk of superblock 0: the source of the spare loads
    // load u (of LOADS) of superblock bi into stage st; every wave issues LOADS per stage (the spares go to the sink)
    auto issue_unit = [&](int u, int st, int bi) {
        const uint32_t base = lds0 + st * G::STAGE;
        if (u < G::LW) {
            const int L = wave + G::NW * u;
            if (L < G::NWLW) {
                if (livew[u]) load_lds16(wal, ((offw[u] + 84u * bi) & ~15u) + cw[u], base + 1024 * L);
            } else {
                load_lds16(wal, offw0, lds0 + G::SINK);
            }
        } else {
            const int k = u - G::LW, L = wave + G::NW * k;
            if (L < G::NWLX) {
                if (livex[k]) load_lds16(J.xq, offx[k] + (uint32_t)bi * stepx[k], base + G::X_OFF + 1024 * L);
            } else {
                load_lds16(J.xq, 0, lds0 + G::SINK);
            }
        }
    };

    uint32_t xo[4];   // activation chunk offsets of this lane in a stage (tile c adds 4096*c): chunk 4ks + lg
#pragma unroll
    for (int ks = 0; ks < 4; ks++) xo[ks] = G::X_OFF + (wt + lr) * 256 + 16 * ((4 * ks + lg) ^ lr);
    const uint32_t mo = G::M_OFF + (wt + lr) * 32 + 16 * (lg & 1), dof = G::D_OFF + (wt + lr) * 4;
    const uint32_t rowoff = (wr + lr) * G::RB, ddoff = (wr + 4 * lg) * G::RB + 80;
    // offsets of this lane's row and of its four output rows from wal (the superblock's start mod 16 places it in LDS)
    const uint32_t myrow_b = mrow0 + (uint32_t)min(wr + lr, last_row) * (uint32_t)J.row_bytes;
    uint32_t orow_b[4];
#pragma unroll
    for (int i = 0; i < 4; i++) orow_b[i] = mrow0 + (uint32_t)min(wr + 4 * lg + i, last_row) * (uint32_t)J.row_bytes;
    const uint32_t sel = 0x0c000c00u + (uint32_t)lg * 0x00010001u;   // byte lg of a word into both 16-bit halves

    float s[WN][4];
#pragma unroll
    for (int c = 0; c < WN; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) s[c][i] = 0.0f;

#pragma unroll
    for (int k = 0; k < NST - 1; k++)
        if (k < nbk)
#pragma unroll
            for (int u = 0; u < G::LOADS; u++) issue_unit(u, k, k);
    int st = 0;   // stage of superblock b
    for (int b = 0; b < nbk; b++) {
        wait_stages<G::LOADS, NST - 2>(min(NST - 2, nbk - 1 - b));   // this wave's loads of stage b are in LDS
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");           // this wave's reads of stage b-1 are done
        __builtin_amdgcn_s_barrier();                                 // ... and every wave's loads and reads
        asm volatile("" ::: "memory");
        const uint8_t *wb = smem + st * G::STAGE;
        const int sti = st == 0 ? NST - 1 : st - 1;   // stage of superblock b + NST - 1 (its loads go out with the tiles)
        const bool more = b + NST - 1 < nbk;
        st = st == NST - 1 ? 0 : st + 1;

        // LDS reads in the order they are needed: the weight fields, the row scales, then activation tile 0
        const uint8_t *rowp = wb + rowoff + ((myrow_b + 84u * b) & 15u);   // 4-byte aligned
        const uint4 scw = *reinterpret_cast<const uint4 *>(__builtin_assume_aligned(rowp, 4));
        const uint4 q0 = *reinterpret_cast<const uint4 *>(__builtin_assume_aligned(rowp + 16 + 16 * (lg & 1), 4));
        const uint4 q1 = *reinterpret_cast<const uint4 *>(__builtin_assume_aligned(rowp + 48 + 16 * (lg & 1), 4));
        uint32_t dd[4];   // d | dmin of this lane's four output rows
#pragma unroll
        for (int i = 0; i < 4; i++)
            dd[i] = *reinterpret_cast<const uint32_t *>(wb + ddoff + ((orow_b[i] + 84u * b) & 15u) + G::RB * i);
        struct Bt { v4i x[4]; v8h m; float td; };
        auto load_b = [&](int c, Bt &B) {
#pragma unroll
            for (int ks = 0; ks < 4; ks++) B.x[ks] = *reinterpret_cast<const v4i *>(wb + xo[ks] + 4096 * c);
            B.m = *reinterpret_cast<const v8h *>(wb + mo + 512 * c);
            B.td = *reinterpret_cast<const float *>(wb + dof + 64 * c);
        };
        Bt B[2];
        load_b(0, B[0]);

        // ---- A operands: per slice the 2-bit codes times their 4-bit scale (<= 45), and the mins as halves
        const uint32_t scv[4] = {scw.x, scw.y, scw.z, scw.w};
        v4i ap[4];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const uint32_t sc16 = __builtin_amdgcn_perm(0, scv[ks] & 0x0f0f0f0fu, sel);   // sc_g & 15 in both halves
            const uint32_t shift = 2 * (2 * (ks & 1) + (lg >> 1));
            const uint4 q = (ks >> 1) ? q1 : q0;
            const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; i++) ap[ks][i] = (int)pk_mul_u16((qq[i] >> shift) & 0x03030303u, sc16);
        }
        // mins operand: lanes 0..15 carry m_0..7 (scales 0..7 >> 4), lanes 16..31 m_8..15 (k positions meet bsums 0..7 /
        // 8..15); lanes 32..63 zero. Each half is built as 1024 + m (byte under the exponent of 1024), 1024 subtracted.
        v8h am;
        {
            const uint32_t w0 = ((lg == 0 ? scw.x : scw.z) >> 4) & 0x0f0f0f0fu, w1 = ((lg == 0 ? scw.y : scw.w) >> 4) & 0x0f0f0f0fu;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t k0 = (2 * e) & 3;
                const uint32_t pr = __builtin_amdgcn_perm(0x64646464u, e < 2 ? w0 : w1,
                                                          k0 | 0x0400u | (k0 + 1) << 16 | 0x04000000u);
                const h2 v = __builtin_bit_cast(h2, pr) + __builtin_bit_cast(h2, 0xe400e400u);   // - 1024
                am[2 * e] = v[0];
                am[2 * e + 1] = v[1];
            }
            if (lg >= 2) am = v8h{0, 0, 0, 0, 0, 0, 0, 0};
        }

        v4i di[2];
        v4f dm[2];
        float tdv[2];
        auto mma = [&](int c, const Bt &Bc) {
            const int w = c & 1;
            tdv[w] = Bc.td;
            dm[w] = __builtin_amdgcn_mfma_f32_16x16x32_f16(am, Bc.m, v4f{0, 0, 0, 0}, 0, 0, 0);
            di[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ap[0], Bc.x[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int ks = 1; ks < 4; ks++) di[w] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ap[ks], Bc.x[ks], di[w], 0, 0, 0);
        };
        // fp32 epilogue of superblock b for tile c, per (row, activation), in the reference's order
        auto epi = [&](int c) {
            const int w = c & 1;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float dall = tdv[w] * half_bits_to_float(dd[i]), dmn = tdv[w] * half_bits_to_float(dd[i] >> 16);
                const float q = dmn * dm[w][i];   // summs: an exact integer in the f32 accumulator
                if constexpr (CONTRACT) s[c][i] = s[c][i] + __builtin_fmaf(dall, static_cast<float>(di[w][i]), -q);
                else s[c][i] = s[c][i] + (dall * static_cast<float>(di[w][i]) - q);
            }
        };
        // one scheduling group per tile: the next superblock's loads, tile c+1's LDS reads, tile c's matrix work and tile
        // c-1's epilogue
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < WN; c++) {
            if (more) {
#pragma unroll
                for (int uu = c * G::PER_TILE; uu < (c + 1) * G::PER_TILE; uu++)
                    if (uu < G::LOADS) issue_unit(uu, sti, b + NST - 1);
            }
            if (c + 1 < WN) load_b(c + 1, B[(c + 1) & 1]);
            mma(c, B[c & 1]);
            if (c) epi(c - 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        epi(WN - 1);
        asm volatile("" ::: "memory");   // stage b's LDS reads stay before the next superblock's barrier
    }

    // ---- outputs
#pragma unroll
    for (int c = 0; c < WN; c++) {
        const int t = tok0 + wt + 16 * c + lr;
        if (t >= J.na) continue;
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
}

template <int RW, int TW, int WN, int NST, int OCC>
static hipError_t mm2_launch_cfg(const MmJob *jobs, int njobs, const MmJob &single, int grid, int order, hipStream_t s) {
    if (order == ES_HIP_ORDER_X86_CONTRACT)
        hipLaunchKernelGGL((mm_q2k_kernel<RW, TW, WN, NST, OCC, true>), dim3(grid), dim3(64 * RW * TW), 0, s, jobs, njobs, single);
    else
        hipLaunchKernelGGL((mm_q2k_kernel<RW, TW, WN, NST, OCC, false>), dim3(grid), dim3(64 * RW * TW), 0, s, jobs, njobs, single);
    return hipGetLastError();
}

// Q2_K workgroup tiles: 128 rows x 16, 32 or 64 activations on 8 waves (16 rows x all the activations each), each small
// enough for two workgroups per CU
hipError_t mm2_launch(int bm, int bn, int nw, const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                      hipStream_t s) {
    if (nw == 8 && bm == 128) {
        if (bn == 64) return mm2_launch_cfg<8, 1, 4, 2, 2>(jobs, njobs, single, grid, order, s);
        if (bn == 32) return mm2_launch_cfg<8, 1, 2, 3, 2>(jobs, njobs, single, grid, order, s);
        if (bn == 16) return mm2_launch_cfg<8, 1, 1, 4, 2>(jobs, njobs, single, grid, order, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace esq
