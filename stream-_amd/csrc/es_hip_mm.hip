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

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

// two 16-bit lanes multiplied (v_pk_mul_lo_u16): four bytes times a small scale at once when no byte product exceeds 255
__device__ __forceinline__ uint32_t pk_mul_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, b));
}

// ---- pre-pass --------------------------------------------------------------------------------------------------------
// One thread per dword of an activation's Q8_K row (nbk blocks of 73 dwords: d, 64 of qs, 8 of bsums pairs), so the
// reads are coalesced; padding activations t >= na get zeros. Activation t is row arow[t] of act when arow is given.
// kind 0 writes the pair sums (Q4_K sub-blocks), kind 1 the 16 bsums, both split as 128*hi + lo, one byte each.
__global__ void act_prep_q8k(const PrepJob *__restrict__ jobs, int njobs, PrepJob single, long total) {
    const long id0 = (long)blockIdx.x * blockDim.x, id = id0 + threadIdx.x;
    if (id >= total) return;
    int j = 0;
    if (jobs) {   // last pre-pass with start <= id0 (starts are multiples of the block size: one search per block)
        int lo = 0, hi = njobs - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (jobs[mid].start <= id0) lo = mid; else hi = mid - 1;
        }
        j = lo;
    }
    const PrepJob P = jobs ? jobs[j] : single;
    const long per = (long)P.nbk * 73, lid = id - P.start;
    if (lid < 0 || lid >= (long)P.na_pad * per) return;
    const int t = (int)(lid / per), k = (int)(lid % per), b = k / 73, w = k % 73;
    const uint32_t v = t < P.na ? ldg<uint32_t>(P.act + (size_t)(P.arow ? ldg<int>(P.arow + t) : t) * P.astride + 4 * (size_t)k) : 0u;
    const size_t bt = (size_t)b * P.na_pad + t;
    uint8_t *xm = P.xm;
    if (w == 0) {
        stg<uint32_t>(xm + (size_t)P.nbk * P.na_pad * (P.kind ? 32 : 16) + bt * 4, v);   // d
    } else if (w <= 64) {
        stg<uint32_t>(P.xq + bt * 256 + 4 * (w - 1), v);                                  // qs
    } else if (P.kind == 0) {
        const int jj = w - 65, p = (int16_t)(v & 0xffff) + (int16_t)(v >> 16);   // bsums[2jj] + bsums[2jj+1]
        stg<uint8_t>(xm + bt * 16 + jj, (uint8_t)(p & 127));
        stg<uint8_t>(xm + bt * 16 + 8 + jj, (uint8_t)((p >> 7) & 0xff));
    } else {
        const int g = 2 * (w - 65), p0 = (int16_t)(v & 0xffff), p1 = (int16_t)(v >> 16);   // bsums[g], bsums[g+1]
        stg<uint8_t>(xm + bt * 32 + g, (uint8_t)(p0 & 127));
        stg<uint8_t>(xm + bt * 32 + g + 1, (uint8_t)(p1 & 127));
        stg<uint8_t>(xm + bt * 32 + 16 + g, (uint8_t)((p0 >> 7) & 0xff));
        stg<uint8_t>(xm + bt * 32 + 16 + g + 1, (uint8_t)((p1 >> 7) & 0xff));
    }
}

// ---- main kernel ---------------------------------------------------------------------------------------------------
__device__ __forceinline__ int find_mm_job(const MmJob *jobs, int njobs, int bid) {
    int lo = 0, hi = njobs - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (jobs[mid].tile0 <= bid) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// One wave's 64 x 16 bytes from global memory straight into LDS: lane l's 16 bytes at base + off land at lds + 16*l
// (lds is wave-uniform). Written as inline assembly so that the compiler does not track these LDS writes: it would
// otherwise wait for every one of them to finish before any LDS read. The kernel orders them itself (s_waitcnt vmcnt +
// s_barrier before a stage is read). M0 is set inside the statement; nothing else in these kernels uses M0.
__device__ __forceinline__ void load_lds16(const uint8_t *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds)
                 : "memory");
}
__device__ __forceinline__ uint32_t lds_addr(const void *p) {
    return (uint32_t)(size_t)(const __attribute__((address_space(3))) uint8_t *)p;
}

template <int N> __device__ __forceinline__ void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }

template <int RW, int WM, int WN> struct MmGeom {
    static constexpr int TW = 8 / RW;
    static constexpr int BM = 16 * WM * RW, BN = 16 * WN * TW;
    // stage regions in bytes: weights BM x 144 | activations BN x 256 | pair sums BN x 16 | scales BN x 4
    static constexpr int X_OFF = BM * 144, M_OFF = X_OFF + BN * 256, D_OFF = M_OFF + BN * 16, STAGE = D_OFF + BN * 4;
    static constexpr int CW = BM * 9, CX = BN * 16, CM = BN, CD = BN / 4, NCH = CW + CX + CM + CD;   // 16-byte chunks
    static constexpr int NWL = (NCH + 63) / 64;   // wave-loads per stage
    static constexpr int LOADS = (NWL + 7) / 8;   // per wave per stage
    static_assert(CW % 64 == 0, "weight chunks end on a wave-load boundary");
    static_assert(RW * TW == 8, "8 waves");
};

// RW: waves along the rows (the others split the activations); WM, WN: 16 x 16 MFMA tiles per wave along rows and
// activations. CONTRACT: the clang order (fused multiply-adds), else the gcc / scalar order.
template <int RW, int WM, int WN, bool CONTRACT>
__global__ __launch_bounds__(512) void mm_q4k_kernel(const MmJob *__restrict__ jobs, int njobs, MmJob single) {
    using G = MmGeom<RW, WM, WN>;
    __shared__ __align__(16) uint8_t smem[3 * G::STAGE + 1024];   // three stages and a sink for the spare loads

    MmJob J;
    if (jobs) J = jobs[find_mm_job(jobs, njobs, blockIdx.x)];
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
    const int wr = (wave % RW) * 16 * WM, wt = (wave / RW) * 16 * WN;   // this wave's rows / activations in the tile
    const int lr = lane & 15, lg = lane >> 4;

    // ---- per-lane sources of this wave's stage loads: wave-load L = wave + 8*kk covers chunks 64L .. 64L+63.
    // Weight chunks: base J.W + row0*row_bytes, offset + 144 per superblock. Activation-side chunks (the three planes of
    // one workspace allocation): base J.xq, offset + (plane stride per superblock).
    const uint8_t *wbase = J.W + (size_t)row0 * J.row_bytes;
    const uint32_t xm_rel = (uint32_t)(J.xm - J.xq), xd_rel = xm_rel + (uint32_t)nbk * J.na_pad * 16;
    const int last_row = J.r1 - 1 - row0;
    uint32_t off[G::LOADS], step_off[G::LOADS];
    bool live[G::LOADS];
#pragma unroll
    for (int kk = 0; kk < G::LOADS; kk++) {
        const int L = wave + 8 * kk, c = 64 * L + lane;
        live[kk] = c < G::NCH;
        if (c < G::CW) {
            const int r = min(c / 9, last_row);   // rows past the end repeat the last one; their results are not stored
            off[kk] = (uint32_t)r * (uint32_t)J.row_bytes + 16 * (c % 9);
            step_off[kk] = 144;
        } else if (c < G::CW + G::CX) {
            const int cx = c - G::CW, t = cx >> 4, q = (cx & 15) ^ (t & 15);
            off[kk] = (uint32_t)(tok0 + t) * 256 + 16 * q;
            step_off[kk] = (uint32_t)J.na_pad * 256;
        } else if (c < G::CW + G::CX + G::CM) {
            const int t = c - G::CW - G::CX;
            off[kk] = xm_rel + (uint32_t)(tok0 + t) * 16;
            step_off[kk] = (uint32_t)J.na_pad * 16;
        } else {
            const int t4 = min(c - G::CW - G::CX - G::CM, G::CD - 1);
            off[kk] = xd_rel + (uint32_t)(tok0 + 4 * t4) * 4;
            step_off[kk] = (uint32_t)J.na_pad * 4;
        }
    }

    // the loads of superblock b into stage st (the offsets already point at superblock b)
    auto issue = [&](int st) {
        const uint32_t base = lds_addr(smem) + st * G::STAGE, snk = lds_addr(smem) + 3 * G::STAGE, off0 = off[0];
#pragma unroll
        for (int kk = 0; kk < G::LOADS; kk++) {
            const int L = wave + 8 * kk;
            const bool wl = 64 * L < G::CW;   // wave-uniform: weight or activation-side wave-load
            if (L < G::NWL) {
                if (live[kk]) load_lds16(wl ? wbase : J.xq, off[kk], base + 1024 * L);
            } else {
                load_lds16(wbase, off0, snk);   // spare (a weight chunk of this superblock): the same count of loads in every wave
            }
            off[kk] += step_off[kk];
        }
    };

    float s[WM][WN][4];
#pragma unroll
    for (int a = 0; a < WM; a++)
#pragma unroll
        for (int c = 0; c < WN; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) s[a][c][i] = 0.0f;

    const uint32_t nsh = lg >= 2 ? 4 : 0;   // high nibbles for lanes 32..63

    issue(0);
    if (nbk > 1) issue(1);
    int st = 0;   // stage of superblock b
    for (int b = 0; b < nbk; b++) {
        if (b + 1 < nbk) wait_vmcnt<G::LOADS>();   // this wave's loads of stage b are in LDS (stage b+1 may still fly)
        else wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's reads of stage b-1 are done
        __builtin_amdgcn_s_barrier();                         // ... and every wave's loads and reads
        asm volatile("" ::: "memory");
        if (b + 2 < nbk) issue(st == 0 ? 2 : st - 1);         // stage (st + 2) % 3
        const uint8_t *wb = smem + st * G::STAGE, *xb = wb + G::X_OFF, *mb = wb + G::M_OFF, *db = wb + G::D_OFF;
        st = st == 2 ? 0 : st + 1;

        // rows' 6-bit scales and mins, byte-parallel (scale_min_k4, src/es_quant.c:75-83), and the A operands of all four
        // k slices
        v4i amin[WM], alo[WM][4], ahi[WM][4];
#pragma unroll
        for (int a = 0; a < WM; a++) {
            const uint8_t *row = wb + (wr + 16 * a + lr) * 144;
            const uint4 h = *reinterpret_cast<const uint4 *>(row);
            const uint32_t sc0 = h.y & 0x3f3f3f3fu, sc1 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
            const uint32_t mn0 = h.z & 0x3f3f3f3fu, mn1 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
            amin[a] = lg == 0 ? v4i{(int)mn0, (int)mn1, 0, 0} : v4i{0, 0, 0, 0};
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {   // this lane's sub-block in slice ks: j = 2ks + (lg >> 1)
                const uint32_t scw = ks < 2 ? sc0 : sc1;
                const uint32_t sc = (scw >> (16 * (ks & 1) + 8 * (lg >> 1))) & 0xff;
                const uint32_t sl16 = (sc & 7) * 0x00010001u, sh16 = (sc >> 3) * 0x00010001u;
                const uint4 w4 = *reinterpret_cast<const uint4 *>(row + 16 + 32 * ks + 16 * (lg & 1));
                const uint32_t qq[4] = {w4.x, w4.y, w4.z, w4.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t nib = (qq[i] >> nsh) & 0x0f0f0f0fu;
                    alo[a][ks][i] = (int)pk_mul_u16(nib, sl16);   // byte * scale <= 105: no carry between bytes
                    ahi[a][ks][i] = (int)pk_mul_u16(nib, sh16);
                }
            }
        }
        // d, dmin of the output rows of this lane: rows wr + 16a + 4lg + i
        float dv[WM][4], dm[WM][4];
#pragma unroll
        for (int a = 0; a < WM; a++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t dd = *reinterpret_cast<const uint32_t *>(wb + (wr + 16 * a + 4 * lg + i) * 144);
                dv[a][i] = half_bits_to_float(dd);
                dm[a][i] = half_bits_to_float(dd >> 16);
            }

        // Activation tiles one after another, software-pipelined: the LDS reads of tile c+1 are issued before the matrix
        // work of tile c, and that before the vector epilogue of tile c-1.
        struct Bt { v4i x[4]; uint4 m; float td; };
        auto load_b = [&](int c, Bt &B) {
            const int t = wt + 16 * c + lr;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) B.x[ks] = *reinterpret_cast<const v4i *>(xb + t * 256 + 16 * ((4 * ks + lg) ^ lr));
            B.m = *reinterpret_cast<const uint4 *>(mb + t * 16);
            B.td = *reinterpret_cast<const float *>(db + t * 4);
        };
        v4i acc_lo[2][WM], acc_hi[2][WM], mn_lo[2][WM], mn_hi[2][WM];
        float tdv[2];
        auto mma = [&](int c, const Bt &B) {
            const int u = c & 1;
            tdv[u] = B.td;
            // mins on the matrix cores: k positions 0..7 (the first 8 bytes of lanes 0..15) carry the pairs; the other
            // positions of amin are zero, so whatever B holds there does not count
            const v4i blo = v4i{(int)B.m.x, (int)B.m.y, (int)B.m.z, (int)B.m.w};
            const v4i bhi = v4i{(int)B.m.z, (int)B.m.w, (int)B.m.x, (int)B.m.y};
#pragma unroll
            for (int a = 0; a < WM; a++) {
                mn_lo[u][a] = __builtin_amdgcn_mfma_i32_16x16x64_i8(amin[a], blo, v4i{0, 0, 0, 0}, 0, 0, 0);
                mn_hi[u][a] = __builtin_amdgcn_mfma_i32_16x16x64_i8(amin[a], bhi, v4i{0, 0, 0, 0}, 0, 0, 0);
            }
#pragma unroll
            for (int ks = 0; ks < 4; ks++)
#pragma unroll
                for (int a = 0; a < WM; a++) {
                    const v4i zlo = ks ? acc_lo[u][a] : v4i{0, 0, 0, 0}, zhi = ks ? acc_hi[u][a] : v4i{0, 0, 0, 0};
                    acc_lo[u][a] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[a][ks], B.x[ks], zlo, 0, 0, 0);
                    acc_hi[u][a] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[a][ks], B.x[ks], zhi, 0, 0, 0);
                }
        };
        // fp32 epilogue of superblock b for tile c, per (row, activation), in the reference's order
        auto epi = [&](int c) {
            const int u = c & 1;
#pragma unroll
            for (int a = 0; a < WM; a++)
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int dot = acc_lo[u][a][i] + 8 * acc_hi[u][a][i];
                    const float q = dm[a][i] * static_cast<float>(mn_lo[u][a][i] + 128 * mn_hi[u][a][i]);
                    if constexpr (CONTRACT)
                        s[a][c][i] = __builtin_fmaf(tdv[u], __builtin_fmaf(dv[a][i], static_cast<float>(dot), -q), s[a][c][i]);
                    else
                        s[a][c][i] = s[a][c][i] + tdv[u] * (dv[a][i] * static_cast<float>(dot) - q);
                }
        };
        Bt B[2];
        load_b(0, B[0]);
#pragma unroll
        for (int c = 0; c < WN; c++) {
            if (c + 1 < WN) load_b(c + 1, B[(c + 1) & 1]);
            mma(c, B[c & 1]);
            if (c) epi(c - 1);
        }
        epi(WN - 1);
        asm volatile("" ::: "memory");   // stage b's LDS reads stay before the next superblock's barrier
    }

    // ---- outputs
#pragma unroll
    for (int a = 0; a < WM; a++)
#pragma unroll
        for (int c = 0; c < WN; c++) {
            const int t = tok0 + wt + 16 * c + lr;
            if (t >= J.na) continue;
            const int r = row0 + wr + 16 * a + 4 * lg;   // this lane holds rows r .. r+3 of activation t
            float *yp = J.y + (size_t)t * J.ystride + r;
            if (r + 3 < J.r1 && (reinterpret_cast<uintptr_t>(yp) & 15) == 0) {
                stg<float4>(yp, make_float4(s[a][c][0], s[a][c][1], s[a][c][2], s[a][c][3]));
            } else {
#pragma unroll
                for (int i = 0; i < 4; i++)
                    if (r + i < J.r1) stg<float>(yp + i, s[a][c][i]);
            }
        }
}

// ---- launch glue -------------------------------------------------------------------------------------------------
hipError_t prep_launch(const PrepJob *jobs, int njobs, const PrepJob &single, long total, hipStream_t s) {
    if (total <= 0) return hipSuccess;
    const int threads = PREP_BLOCK;
    hipLaunchKernelGGL(act_prep_q8k, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0, s, jobs, njobs, single,
                       total);
    return hipGetLastError();
}

template <int RW, int WM, int WN>
static hipError_t mm_launch_cfg(const MmJob *jobs, int njobs, const MmJob &single, int grid, int order, hipStream_t s) {
    if (order == ES_HIP_ORDER_X86_CONTRACT)
        hipLaunchKernelGGL((mm_q4k_kernel<RW, WM, WN, true>), dim3(grid), dim3(512), 0, s, jobs, njobs, single);
    else
        hipLaunchKernelGGL((mm_q4k_kernel<RW, WM, WN, false>), dim3(grid), dim3(512), 0, s, jobs, njobs, single);
    return hipGetLastError();
}

// workgroup tiles: 128 x 128 (8 waves of 16 rows x 128 activations), 64 x 64 (4 x 2 waves of 16 rows x 32), and for small
// batches 128 rows x 16, 32 or 64 activations
hipError_t mm_launch(int type, int bm, int bn, const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                     hipStream_t s) {
    if (type != ES_HIP_Q4_K) return hipErrorInvalidValue;
    if (bm == 128 && bn == 128) return mm_launch_cfg<8, 1, 8>(jobs, njobs, single, grid, order, s);
    if (bm == 128 && bn == 64) return mm_launch_cfg<8, 1, 4>(jobs, njobs, single, grid, order, s);
    if (bm == 128 && bn == 32) return mm_launch_cfg<8, 1, 2>(jobs, njobs, single, grid, order, s);
    if (bm == 128 && bn == 16) return mm_launch_cfg<8, 1, 1>(jobs, njobs, single, grid, order, s);
    if (bm == 64 && bn == 64) return mm_launch_cfg<4, 1, 2>(jobs, njobs, single, grid, order, s);
    return hipErrorInvalidValue;
}

}  // namespace esq
