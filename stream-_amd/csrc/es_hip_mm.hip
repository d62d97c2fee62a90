// Batched products on the int8 matrix cores (v_mfma_i32_16x16x64_i8): the prompt-reading form of es_matvec_multi
// (src/es_quant.c:1818-1850) for Q4_K, where every weight row meets many activations.
//
// Pre-pass. The activations' Q8_K blocks (292 bytes, token-major) are copied into planes per superblock b:
// xq[b][t][256] (the int8 values), xm[b][t][16] (the pair sums p_j = bsums[2j] + bsums[2j+1] of the eight 32-element
// sub-blocks, split as p = 128*hi + lo with lo in 0..127 and hi in -32..31: eight low bytes, then eight high bytes) and
// xd[b][t] (the float scale). A token tile of one superblock is then one contiguous stretch of each plane.
//
// Main kernel. A workgroup of 8 waves (two per SIMD, so one wave's vector work overlaps the other's matrix work) computes a
// tile of BM = 16*WM*RW rows x BN = 16*WN*(8/RW) activations; wave w takes 16*WM rows and 16*WN activations of it, i.e.
// WM x WN MFMA tiles of 16 x 16. Superblocks stream through a ring of three LDS stages filled by direct global-to-LDS
// loads (global_load_lds_dwordx4: lane l's 16 bytes land at the wave-uniform LDS address + 16*l, checked on the device),
// two superblocks ahead of the one being computed. A stage is one array of 16-byte chunks (weights, activations, pair
// sums, scales); wave-load L fills chunks 64L .. 64L+63, and every wave issues the same number of wave-loads per stage
// (the spare ones go to a sink), so "s_waitcnt vmcnt(loads per stage)" proves the wave's part of the current stage has
// landed and a raw s_barrier publishes it. Activation chunks are stored XOR-swizzled (chunk q of activation t at slot
// q ^ (t & 15)) so the 16 lanes reading one k-slice of 16 activations hit 16 different banks.
// Per superblock and wave:
//   mins = sum_j mn_j * p_j on the matrix cores: k positions 0..7 of one slice carry the eight (mn_j, p_j) pairs;
//     mins = D(mn, lo) + 128 * D(mn, hi), folded at once into the float dmin*mins (exact: |mins| < 2^24).
//   dot, for each of the four 64-wide k slices:
//     B operand (activations): lane l takes activation l%16 of the MFMA tile, values 16*(l/16) .. +16 of the slice;
//     A operand (weights): lane l takes row l%16, the same 16 positions: 16 nibbles of one sub-block j. The sub-block
//     scale sc (0..63) times the nibble does not fit int8, so it is split as sc = 8*sh + sl and two int8 planes go
//     through the matrix cores: A_lo = q*sl and A_hi = q*sh (both <= 105). dot = D_lo + 8*D_hi, exact in int32.
//   The fp32 epilogue s += y.d * (d*dot - dmin*mins) then runs per (row, activation) in superblock order, in the selected
//   reference order, so the results are bit-identical to the CPU kernels (src/es_quant.c:1056-1080, 1324-1343,
//   1564-1602).
// MFMA output layout (checked on the device): lane l, register i holds D[4*(l/16) + i][l % 16].
#include "es_hip_common.h"

namespace esq {




// ---- pre-pass --------------------------------------------------------------------------------------------------------
// Items of an activation's row, consecutive items on consecutive threads so the reads are coalesced, PREP_UNROLL items
// per thread with every load issued before the first store; padding activations t >= na get zeros. Activation t is row
// arow[t] of act when arow is given. A Q8_K block (292 bytes: d, qs[256], bsums[16]) is 19 items of 16 bytes: item 0 at
// byte 0 (d and the first qs, of which only d is used), item w = 1 .. 18 at byte 16w - 12 (qs for w <= 16, then bsums
// 0..7 and 8..15); the rows are only dword-aligned, so the loads are dword-aligned 16-byte loads. A Q8_0 block is 9 dword
// items (d, 8 words of qs).
// kind 0 writes the pair sums (Q4_K sub-blocks) and kind 1 the 16 bsums, both split as 128*hi + lo, one byte each; kind 2
// writes the 16 bsums as halves (exact: a Q8_K block's bsums are sums of 16 int8 values, |bsums| <= 2048). Kind 3 reads
// Q8_0 rows and writes the batched 32-wide matrix-core layout (tiles of 32 activations).
// Index arithmetic is 32-bit within a pre-pass (the host keeps every pre-pass below 2^31 threads).
typedef uint32_t u32x4_a4 __attribute__((ext_vector_type(4), aligned(4)));

// the loads of one thread's items: row indices (for a gather), then the activation items (WIDE: 16 bytes, else a dword)
template <bool GATHER, bool WIDE>
__device__ __forceinline__ void prep_loads(const PrepJob &P, uint32_t base, uint32_t per, const bool (&ok)[PREP_UNROLL],
                                           uint32_t (&row)[PREP_UNROLL], uint4 (&v)[PREP_UNROLL]) {
    if constexpr (GATHER) {
#pragma unroll
        for (int u = 0; u < PREP_UNROLL; u++) row[u] = (uint32_t)ldg<int>(P.arow + row[u]);
    }
#pragma unroll
    for (int u = 0; u < PREP_UNROLL; u++) {
        const uint32_t lid = base + u * PREP_BLOCK + threadIdx.x, t = lid / per, k = ok[u] ? lid - t * per : 0u;
        const uint8_t *src = P.act + (size_t)row[u] * P.astride;
        if constexpr (WIDE) {
            const uint32_t b = k / 19u, w = k - 19u * b, off = 292u * b + (w ? 16u * w - 12u : 0u);
            const u32x4_a4 x = *(const ESQ_GLOBAL u32x4_a4 *)(src + off);
            v[u] = make_uint4(x.x, x.y, x.z, x.w);
        } else {
            v[u].x = ldg<uint32_t>(src + 4 * (size_t)k);
        }
    }
}

// the stores of one Q8_K item (d, 16 bytes of qs, or 8 bsums)
__device__ __forceinline__ void prep_store_q8k(const PrepJob &P, uint32_t t, uint32_t k, const uint4 &v) {
    const uint32_t b = k / 19u, w = k - 19u * b;
    const size_t bt = (size_t)b * P.na_pad + t;
    uint8_t *xm = P.xm;
    const int mb = P.kind == 0 ? 16 : 32;   // meta bytes per (activation, superblock)
    if (w == 0) {
        stg<uint32_t>(xm + (size_t)P.nbk * P.na_pad * mb + bt * 4, v.x);   // d
        return;
    }
    if (w <= 16) {
        stg<uint4>(P.xq + bt * 256 + 16 * (w - 1), v);   // qs
        return;
    }
    const int h = (int)w - 17;   // bsums 8h .. 8h+7
    const uint32_t wd[4] = {v.x, v.y, v.z, v.w};
    int bs[8];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        bs[2 * i] = (int16_t)(wd[i] & 0xffff);
        bs[2 * i + 1] = (int16_t)(wd[i] >> 16);
    }
    if (P.kind == 0) {   // pair sums p_jj = bsums[2jj] + bsums[2jj+1], jj = 4h .. 4h+3
        uint32_t lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = bs[2 * i] + bs[2 * i + 1];
            lo |= (uint32_t)(p & 127) << (8 * i);
            hi |= (uint32_t)((p >> 7) & 0xff) << (8 * i);
        }
        stg<uint32_t>(xm + bt * 16 + 4 * h, lo);
        stg<uint32_t>(xm + bt * 16 + 8 + 4 * h, hi);
    } else if (P.kind == 1) {   // bsums g = 8h .. 8h+7: low bytes, then high bytes
        uint32_t lo[2] = {0, 0}, hi[2] = {0, 0};
#pragma unroll
        for (int i = 0; i < 8; i++) {
            lo[i >> 2] |= (uint32_t)(bs[i] & 127) << (8 * (i & 3));
            hi[i >> 2] |= (uint32_t)((bs[i] >> 7) & 0xff) << (8 * (i & 3));
        }
        stg<uint2>(xm + bt * 32 + 8 * h, make_uint2(lo[0], lo[1]));
        stg<uint2>(xm + bt * 32 + 16 + 8 * h, make_uint2(hi[0], hi[1]));
    } else {   // kind 2: halves
        uint32_t hv[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            hv[i] = (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)bs[2 * i]) |
                    (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)bs[2 * i + 1]) << 16;
        stg<uint4>(xm + bt * 32 + 16 * h, make_uint4(hv[0], hv[1], hv[2], hv[3]));
    }
}

// the stores of one Q8_0 dword item (kind 3)
__device__ __forceinline__ void prep_store_q80(const PrepJob &P, uint32_t t, uint32_t k, uint32_t v) {
    const uint32_t b = k / 9u, w = k - 9u * b;
    const uint32_t tb = (t >> 5) * (uint32_t)P.nbk + b, nn = t & 31u;   // (tile, block), activation in the tile
    if (w == 0) {
        stg<uint32_t>(P.xm + ((size_t)tb * 32 + nn) * 4, v);
    } else {   // values e0 .. e0 + 3 as halves: instruction q = e0 / 16, lane half h = e0 % 16 / 8, halves e0 % 8 ..
        const uint32_t e0 = 4 * (w - 1), q = e0 >> 4, hh = (e0 >> 3) & 1;
        h2 lo, hi;
        lo[0] = (_Float16)(int8_t)(v & 0xff);
        lo[1] = (_Float16)(int8_t)((v >> 8) & 0xff);
        hi[0] = (_Float16)(int8_t)((v >> 16) & 0xff);
        hi[1] = (_Float16)(int8_t)(v >> 24);
        const uint2 pr = make_uint2(__builtin_bit_cast(uint32_t, lo), __builtin_bit_cast(uint32_t, hi));
        stg<uint2>(P.xq + ((((size_t)tb * 2 + q) * 2 + hh) * 32 + nn) * 16 + 2 * (e0 & 7), pr);
    }
}

template <bool WIDE>
__device__ __forceinline__ void prep_items(const PrepJob &P, uint32_t base, uint32_t per, uint32_t n) {
    // every load of the span first, unconditionally (items past the end read the first item and keep 0), so they are all
    // in flight together; then the stores
    uint4 v[PREP_UNROLL];
    uint32_t row[PREP_UNROLL];
    bool ok[PREP_UNROLL];
#pragma unroll
    for (int u = 0; u < PREP_UNROLL; u++) {
        const uint32_t lid = base + u * PREP_BLOCK + threadIdx.x, t = lid / per;
        ok[u] = lid < n && (int)t < P.na;
        row[u] = ok[u] ? t : 0u;
    }
    if (P.arow) prep_loads<true, WIDE>(P, base, per, ok, row, v);   // two copies of the loads, so no branch splits them
    else prep_loads<false, WIDE>(P, base, per, ok, row, v);
#pragma unroll
    for (int u = 0; u < PREP_UNROLL; u++) v[u] = ok[u] ? v[u] : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int u = 0; u < PREP_UNROLL; u++) {
        const uint32_t lid = base + u * PREP_BLOCK + threadIdx.x;
        if (lid >= n) break;
        const uint32_t t = lid / per, k = lid - t * per;
        if constexpr (WIDE) prep_store_q8k(P, t, k, v[u]);
        else prep_store_q80(P, t, k, v[u].x);
    }
}

__global__ __launch_bounds__(PREP_BLOCK) void act_prep_q8k(const PrepJob *__restrict__ jobs, int njobs, PrepJob single,
                                                            long total) {
    const long id0 = (long)blockIdx.x * PREP_SPAN;
    int j = 0;
    if (jobs) {   // last pre-pass with start <= id0 (starts are multiples of the span: one search per block)
        int lo = 0, hi = njobs - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (jobs[mid].start <= id0) lo = mid; else hi = mid - 1;
        }
        j = lo;
    }
    PrepJob P;
    if (jobs) P = jobs[j];
    else P = single;
    const uint32_t per = (uint32_t)P.nbk * prep_words(P.kind), n = (uint32_t)P.na_pad * per, base = (uint32_t)(id0 - P.start);
    if (P.kind == PREP_KIND_Q80) prep_items<false>(P, base, per, n);
    else prep_items<true>(P, base, per, n);
}

// ---- main kernel ---------------------------------------------------------------------------------------------------



template <int RW, int TW, int WN, int NST> struct MmGeom {
    static constexpr int NW = RW * TW;   // waves
    static constexpr int BM = 16 * RW, BN = 16 * WN * TW;
    // 16-byte chunks of a stage: weights BM x 9 (the region padded to whole wave-loads) | activations BN x 16 | bsums
    // BN x 2 | scales BN / 4
    static constexpr int CW = BM * 9, CWP = (CW + 63) / 64 * 64, CX = BN * 16, CM = BN * 2, CD = BN / 4;
    static constexpr int NCH = CWP + CX + CM + CD;
    static constexpr int X_OFF = CWP * 16, M_OFF = X_OFF + BN * 256, D_OFF = M_OFF + BN * 32, STAGE = D_OFF + BN * 4;
    static constexpr int NWL = (NCH + 63) / 64;   // wave-loads per stage
    static constexpr int LOADS = (NWL + NW - 1) / NW;   // per wave per stage
    static constexpr int LDS = NST * STAGE + 1024;   // the stages and a sink for the spare loads
    static_assert(NW == 4 || NW == 8, "4 or 8 waves");
    static_assert(NST >= 2 && LDS <= 160 * 1024, "stages fit the LDS");
    static_assert(LOADS * (NST - 2) <= 63, "vmcnt range");
};


// RW x TW waves: RW along the rows, TW along the activations; WN: 16 x 16 MFMA tiles per wave along the activations;
// NST: LDS stages. CONTRACT: the clang order (fused multiply-adds), else the gcc / scalar order.
template <int RW, int TW, int WN, int NST, bool CONTRACT>
__global__ __launch_bounds__(64 * RW * TW) void mm_q4k_kernel(const MmJob *__restrict__ jobs, int njobs, MmJob single) {
    using G = MmGeom<RW, TW, WN, NST>;
    __shared__ __align__(16) uint8_t smem[G::LDS];

    MmJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    // XCD-aware tile order: workgroup ids go round-robin over the 8 XCDs (id % 8), so all activation tiles of row tile rt
    // are given to ids with id % 8 == rt % 8 and the rows' weight blocks are read into a single XCD's L2. Each job's
    // tiles start at a multiple of 8; ids past the last row tile exit at once.
    const int tile = blockIdx.x - J.tile0;
    const int x = tile & 7, kq = tile >> 3;
    const int rt = x + 8 * (kq / J.ntok_tiles), tt = kq % J.ntok_tiles;
    if (rt * G::BM >= J.r1 - J.r0) return;
    const int row0 = J.r0 + rt * G::BM, tok0 = tt * G::BN;
    const int nbk = J.cols / 256;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int wr = (wave % RW) * 16, wt = (wave / RW) * 16 * WN;   // this wave's rows / activations in the tile
    const int lr = lane & 15, lg = lane >> 4;

    // ---- per-lane sources of this wave's stage loads: wave-load L = wave + 8*kk covers chunks 64L .. 64L+63.
    // Weight chunks: base J.W + row0*row_bytes, offset + 144 per superblock. Activation-side chunks (the three planes of
    // one workspace allocation): base J.xq, offset + (plane stride per superblock).
    const uint8_t *wbase = J.W + (size_t)row0 * J.row_bytes;
    const uint32_t xm_rel = (uint32_t)(J.xm - J.xq), xd_rel = xm_rel + (uint32_t)nbk * J.na_pad * 32;
    const int last_row = J.r1 - 1 - row0;
    uint32_t off[G::LOADS], step_off[G::LOADS];
    bool live[G::LOADS];
#pragma unroll
    for (int kk = 0; kk < G::LOADS; kk++) {
        const int L = wave + G::NW * kk, c = 64 * L + lane;
        live[kk] = c < G::NCH && (c < G::CW || c >= G::CWP);
        if (c < G::CWP) {
            const int r = min(c / 9, last_row);   // rows past the end repeat the last one; their results are not stored
            off[kk] = (uint32_t)r * (uint32_t)J.row_bytes + 16 * (c % 9);
            step_off[kk] = 144;
        } else if (c < G::CWP + G::CX) {
            const int cx = c - G::CWP, t = cx >> 4, q = (cx & 15) ^ (t & 15);
            off[kk] = (uint32_t)(tok0 + t) * 256 + 16 * q;
            step_off[kk] = (uint32_t)J.na_pad * 256;
        } else if (c < G::CWP + G::CX + G::CM) {
            const int cm = c - G::CWP - G::CX;
            off[kk] = xm_rel + (uint32_t)(tok0 + (cm >> 1)) * 32 + 16 * (cm & 1);
            step_off[kk] = (uint32_t)J.na_pad * 32;
        } else {
            const int t4 = min(c - G::CWP - G::CX - G::CM, G::CD - 1);
            off[kk] = xd_rel + (uint32_t)(tok0 + 4 * t4) * 4;
            step_off[kk] = (uint32_t)J.na_pad * 4;
        }
    }

    // the loads of the next superblock into stage st (the offsets already point at it)
    auto issue = [&](int st) {
        const uint32_t base = lds_addr(smem) + st * G::STAGE, snk = lds_addr(smem) + NST * G::STAGE, off0 = off[0];
#pragma unroll
        for (int kk = 0; kk < G::LOADS; kk++) {
            const int L = wave + G::NW * kk;
            const bool wl = 64 * L < G::CWP;   // wave-uniform: weight or activation-side wave-load
            if (L < G::NWL) {
                if (live[kk]) load_lds16(wl ? wbase : J.xq, off[kk], base + 1024 * L);
            } else {
                load_lds16(wbase, off0, snk);   // spare (a weight chunk of this superblock): the same count of loads in every wave
            }
            off[kk] += step_off[kk];
        }
    };

    // Permuted k order. MFMA slice s (0..3), lane group lg: the 16 nibbles of qs chunk lg + 4*(s >> 1) (low nibbles for
    // even s, high for odd s), i.e. sub-block j = 2*((lg >> 1) + 2*(s >> 1)) + (s & 1), elements 32j + 16*(lg & 1) + [0, 16).
    // The activation side reads the same elements: natural 16-element chunk nat(s) of the activation row.
    uint32_t xo[4];   // activation chunk offsets of this lane in a stage (tile c adds 4096*c)
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int nat = 4 * (lg >> 1) + 8 * (s >> 1) + 2 * (s & 1) + (lg & 1);
        xo[s] = G::X_OFF + (wt + lr) * 256 + 16 * (nat ^ lr);
    }
    const uint32_t mo = G::M_OFF + (wt + lr) * 32 + 16 * (lg & 1), dof = G::D_OFF + (wt + lr) * 4;
    // byte selectors (v_perm_b32) that put byte (lg >> 1)*2 + e of a word into both 16-bit halves, the other bytes zero
    const uint32_t sel0 = 0x0c000c00u + (uint32_t)(2 * (lg >> 1)) * 0x00010001u, sel1 = sel0 + 0x00010001u;
    const int myrow = wr + lr;

    float s[WN][4];
#pragma unroll
    for (int c = 0; c < WN; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) s[c][i] = 0.0f;

#pragma unroll
    for (int k = 0; k < NST - 1; k++)
        if (k < nbk) issue(k);
    int st = 0;   // stage of superblock b
    for (int b = 0; b < nbk; b++) {
        wait_stages<G::LOADS, NST - 2>(min(NST - 2, nbk - 1 - b));   // this wave's loads of stage b are in LDS
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");           // this wave's reads of stage b-1 are done
        __builtin_amdgcn_s_barrier();                                 // ... and every wave's loads and reads
        asm volatile("" ::: "memory");
        if (b + NST - 1 < nbk) issue(st == 0 ? NST - 1 : st - 1);      // stage (st + NST - 1) % NST
        const uint8_t *wb = smem + st * G::STAGE;
        st = st == NST - 1 ? 0 : st + 1;

        // LDS reads in the order they are needed (they complete in order): the weight rows for the A operands and the row
        // scales, the activation scales of every tile, then the activation tiles 0 and 1; afterwards tile c+2 is read
        // while tile c goes through the matrix cores and tile c-1 through the vector epilogue.
        const uint8_t *row = wb + myrow * 144;
        const uint4 h = *reinterpret_cast<const uint4 *>(row);
        const uint4 q0 = *reinterpret_cast<const uint4 *>(row + 16 + 16 * lg);
        const uint4 q1 = *reinterpret_cast<const uint4 *>(row + 80 + 16 * lg);
        uint32_t ddw[4];
#pragma unroll
        for (int i = 0; i < 4; i++) ddw[i] = *reinterpret_cast<const uint32_t *>(wb + (wr + 4 * lg + i) * 144);
        float tdv[WN];
#pragma unroll
        for (int c = 0; c < WN; c++) tdv[c] = *reinterpret_cast<const float *>(wb + dof + 64 * c);
        struct Bt { v4i x[4]; v8h m; };
        auto load_b = [&](int c, Bt &B) {
#pragma unroll
            for (int sl = 0; sl < 4; sl++) B.x[sl] = *reinterpret_cast<const v4i *>(wb + xo[sl] + 4096 * c);
            B.m = *reinterpret_cast<const v8h *>(wb + mo + 512 * c);
        };
        constexpr int PD = WN < 2 ? WN : 2;   // tiles read ahead
        Bt B[PD + 1];
#pragma unroll
        for (int c = 0; c < PD; c++) load_b(c, B[c]);

        // ---- A operands of this wave's 16 rows: scales byte-parallel (scale_min_k4, src/es_quant.c:75-83)
        const uint32_t sc0 = h.y & 0x3f3f3f3fu, sc1 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
        const uint32_t mn0 = h.z & 0x3f3f3f3fu, mn1 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
        // sc = 8*sh + sl; (sl, sh) of sub-blocks 2*(lg>>1) + {0, 1} (from sc0) and + {4, 5} (from sc1), each byte
        // broadcast into both 16-bit halves
        const uint32_t l0 = sc0 & 0x07070707u, h0 = (sc0 >> 3) & 0x07070707u;
        const uint32_t l1 = sc1 & 0x07070707u, h1 = (sc1 >> 3) & 0x07070707u;
        const uint32_t slw[4] = {__builtin_amdgcn_perm(0, l0, sel0), __builtin_amdgcn_perm(0, l0, sel1),
                                 __builtin_amdgcn_perm(0, l1, sel0), __builtin_amdgcn_perm(0, l1, sel1)};
        const uint32_t shw[4] = {__builtin_amdgcn_perm(0, h0, sel0), __builtin_amdgcn_perm(0, h0, sel1),
                                 __builtin_amdgcn_perm(0, h1, sel0), __builtin_amdgcn_perm(0, h1, sel1)};
        v4i alo[4], ahi[4];
        {
            const uint32_t qa[2][4] = {{q0.x, q0.y, q0.z, q0.w}, {q1.x, q1.y, q1.z, q1.w}};
#pragma unroll
            for (int sl = 0; sl < 4; sl++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t w = qa[sl >> 1][i];
                    const uint32_t nib = (sl & 1) ? (w >> 4) & 0x0f0f0f0fu : w & 0x0f0f0f0fu;
                    alo[sl][i] = (int)pk_mul_u16(nib, slw[sl]);   // byte * scale <= 105: no carry between bytes
                    ahi[sl][i] = (int)pk_mul_u16(nib, shw[sl]);
                }
        }
        // mins operand (halves): lanes 0..15 carry mn_0..3, lanes 16..31 mn_4..7, each twice (k positions 2j, 2j+1 meet
        // bsums[2j], bsums[2j+1]); lanes 32..63 zero. Each half is built as 1024 + m (byte m under the exponent of 1024)
        // and 1024 subtracted exactly.
        v8h amin;
        {
            const uint32_t mw = lg == 0 ? mn0 : lg == 1 ? mn1 : 0u;
            const uint32_t m1024 = 0xe400e400u;   // -1024, -1024
#pragma unroll
            for (int e = 0; e < 4; e++) {
                const uint32_t pr = __builtin_amdgcn_perm(0x64646464u, mw, 0x04000400u + (uint32_t)e * 0x00010001u);
                const h2 v = __builtin_bit_cast(h2, pr) + __builtin_bit_cast(h2, m1024);
                amin[2 * e] = v[0];
                amin[2 * e + 1] = v[1];
            }
            if (lg >= 2) amin = v8h{0, 0, 0, 0, 0, 0, 0, 0};
        }
        // d, dmin of the output rows of this lane: rows wr + 4lg + i
        float dv[4], dm[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            dv[i] = half_bits_to_float(ddw[i]);
            dm[i] = half_bits_to_float(ddw[i] >> 16);
        }

        v4i acc_lo[2], acc_hi[2];
        v4f acc_mn[2];
        auto mma = [&](int c, const Bt &B) {
            const int u = c & 1;
            acc_mn[u] = __builtin_amdgcn_mfma_f32_16x16x32_f16(amin, B.m, v4f{0, 0, 0, 0}, 0, 0, 0);
            acc_lo[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[0], B.x[0], v4i{0, 0, 0, 0}, 0, 0, 0);
            acc_hi[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[0], B.x[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
            for (int sl = 1; sl < 4; sl++) {
                acc_lo[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[sl], B.x[sl], acc_lo[u], 0, 0, 0);
                acc_hi[u] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[sl], B.x[sl], acc_hi[u], 0, 0, 0);
            }
        };
        // fp32 epilogue of superblock b for tile c, per (row, activation), in the reference's order
        auto epi = [&](int c) {
            const int u = c & 1;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int dot = acc_lo[u][i] + 8 * acc_hi[u][i];
                const float q = dm[i] * acc_mn[u][i];   // the mins are exact integers in the f32 accumulator
                if constexpr (CONTRACT)
                    s[c][i] = __builtin_fmaf(tdv[c], __builtin_fmaf(dv[i], static_cast<float>(dot), -q), s[c][i]);
                else
                    s[c][i] = s[c][i] + tdv[c] * (dv[i] * static_cast<float>(dot) - q);
            }
        };
        // One scheduling group per tile, its instructions interleaved as 1 MFMA : 2 VALU (: 1 LDS read): a SIMD issues
        // about two vector instructions in the shadow of each 16-cycle MFMA, the rest would cost their full time.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 0; c < WN; c++) {
            if (c + PD < WN) load_b(c + PD, B[(c + PD) % (PD + 1)]);
            mma(c, B[c % (PD + 1)]);
            if (c) epi(c - 1);
#pragma unroll
            for (int k = 0; k < 9; k++) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);   // VALU
                if (k < 5) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
            }
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

// ---- launch glue -------------------------------------------------------------------------------------------------
hipError_t prep_launch(const PrepJob *jobs, int njobs, const PrepJob &single, long total, hipStream_t s) {
    if (total <= 0) return hipSuccess;
    hipLaunchKernelGGL(act_prep_q8k, dim3((unsigned)((total + PREP_SPAN - 1) / PREP_SPAN)), dim3(PREP_BLOCK), 0, s, jobs, njobs,
                       single, total);
    return hipGetLastError();
}

template <int RW, int TW, int WN, int NST>
static hipError_t mm_launch_cfg(const MmJob *jobs, int njobs, const MmJob &single, int grid, int order, hipStream_t s) {
    if (order == ES_HIP_ORDER_X86_CONTRACT)
        hipLaunchKernelGGL((mm_q4k_kernel<RW, TW, WN, NST, true>), dim3(grid), dim3(64 * RW * TW), 0, s, jobs, njobs, single);
    else
        hipLaunchKernelGGL((mm_q4k_kernel<RW, TW, WN, NST, false>), dim3(grid), dim3(64 * RW * TW), 0, s, jobs, njobs, single);
    return hipGetLastError();
}

// Workgroup tiles (rows x activations, waves): 128 x 128 (8 waves of 16 rows x 128 activations), 64 x 64 (4 x 2 waves of
// 16 x 32, or 4 waves of 16 x 64), 32 x 128 (2 x 2 waves of 16 x 64), and for small batches 128 rows x 16, 32 or 64
// activations; as many LDS stages as fit (at least two).
bool mm_tile_ok(int bm, int bn, int nw) {
    return (nw == 8 && bm == 128 && (bn == 128 || bn == 64 || bn == 32 || bn == 16)) || (nw == 8 && bm == 64 && bn == 64) ||
           (nw == 4 && bm == 64 && bn == 64) || (nw == 4 && bm == 32 && bn == 128);
}

hipError_t mm_launch(int type, int bm, int bn, int nw, const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                     hipStream_t s, const MmJob *hjobs) {
    if (type == ES_HIP_Q6_K) return mm6_launch(bm, bn, nw, jobs, njobs, single, grid, order, s, hjobs);
    if (type == ES_HIP_Q2_K) return mm2_launch(bm, bn, nw, jobs, njobs, single, grid, order, s);
    if (type != ES_HIP_Q4_K) return hipErrorInvalidValue;
    if (nw == 8) {
        if (bm == 128 && bn == 128) return mm_launch_cfg<8, 1, 8, 2>(jobs, njobs, single, grid, order, s);
        if (bm == 128 && bn == 64) return mm_launch_cfg<8, 1, 4, 4>(jobs, njobs, single, grid, order, s);
        if (bm == 128 && bn == 32) return mm_launch_cfg<8, 1, 2, 5>(jobs, njobs, single, grid, order, s);
        if (bm == 128 && bn == 16) return mm_launch_cfg<8, 1, 1, 6>(jobs, njobs, single, grid, order, s);
        if (bm == 64 && bn == 64) return mm_launch_cfg<4, 2, 2, 5>(jobs, njobs, single, grid, order, s);
    } else if (nw == 4) {
        if (bm == 64 && bn == 64) return mm_launch_cfg<4, 1, 4, 5>(jobs, njobs, single, grid, order, s);
        if (bm == 32 && bn == 128) return mm_launch_cfg<2, 2, 4, 3>(jobs, njobs, single, grid, order, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace esq
