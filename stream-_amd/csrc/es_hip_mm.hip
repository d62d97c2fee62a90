// Batched products on the int8 matrix cores (v_mfma_i32_16x16x64_i8): the prompt-reading form of es_matvec_multi
// (src/es_quant.c:1818-1850) for Q4_K, where every weight row meets many activations.
//
// Pre-pass. The activations' Q8_K blocks (292 bytes, token-major) are copied into two planes per superblock b:
// xq[b][t][256] (the int8 values) and xm[b][t] (32 bytes: the pair sums p_j = bsums[2j] + bsums[2j+1] of the eight
// 32-element sub-blocks split as p = 128*hi + lo, lo in 0..127 and hi in -32..31, one byte each, then d). A token tile of
// one superblock is then one contiguous stretch of memory.
//
// Main kernel. A workgroup of 4 waves computes a tile of 64 rows x 32*WN activations; wave w takes rows 32*(w&1) .. +32
// and activations 16*WN*(w>>1) .. +16*WN, i.e. 2 x WN MFMA tiles of 16 x 16. Superblocks stream through a ring of three
// LDS stages filled by direct global-to-LDS loads (global_load_lds_dwordx4: lane l's 16 bytes land at the stage address
// + 16*l, checked on the device), two superblocks ahead of the one being computed; each wave waits only for its own loads
// of the current stage (s_waitcnt vmcnt) and a raw s_barrier publishes the stage. Activation chunks are stored XOR-
// swizzled (chunk q of activation t at slot q ^ (t & 15)) so the 16 lanes reading one k-slice of 16 activations hit 16
// different banks.
// For each of the four 64-wide k slices of a superblock:
//   B operand (activations): lane l takes activation l%16 of the tile, values 16*(l/16) .. +16 of the slice;
//   A operand (weights): lane l takes row l%16, the same 16 positions: 16 nibbles of one sub-block j. The sub-block scale
//     sc (0..63) times the nibble does not fit int8, so it is split as sc = 8*sh + sl and two int8 planes go through the
//     matrix cores: A_lo = q*sl and A_hi = q*sh (both <= 105). dot = D_lo + 8*D_hi, exact in int32.
// mins = sum_j mn_j * p_j goes through the matrix cores too: k positions 0..7 of one slice carry the eight (mn_j, p_j)
// pairs; mins = D(mn, lo) + 128 * D(mn, hi). The fp32 epilogue s += y.d * (d*dot - dmin*mins) then runs per
// (row, activation) in superblock order, in the selected reference order, so the results are bit-identical to the CPU
// kernels (src/es_quant.c:1056-1080, 1324-1343, 1564-1602).
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
// one thread per (superblock, activation, 16-byte piece); piece 16 writes the meta
__global__ void act_prep_q8k(const uint8_t *__restrict__ act, uint64_t astride, int na, int na_pad, int nbk,
                             uint8_t *__restrict__ xq, uint8_t *__restrict__ xm) {
    const long id = (long)blockIdx.x * blockDim.x + threadIdx.x;
    const long total = (long)nbk * na_pad * 17;
    if (id >= total) return;
    const int piece = (int)(id % 17);
    const long bt = id / 17;
    const int t = (int)(bt % na_pad), b = (int)(bt / na_pad);
    const uint8_t *src = act + (size_t)t * astride + (size_t)b * 292;
    if (piece < 16) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (t < na) v = make_uint4(ldg<uint32_t>(src + 4 + 16 * piece), ldg<uint32_t>(src + 8 + 16 * piece),
                                   ldg<uint32_t>(src + 12 + 16 * piece), ldg<uint32_t>(src + 16 + 16 * piece));
        *reinterpret_cast<uint4 *>(xq + ((size_t)b * na_pad + t) * 256 + 16 * piece) = v;
        return;
    }
    uint32_t lo[2] = {0, 0}, hi[2] = {0, 0}, d = 0;
    if (t < na) {
        d = ldg<uint32_t>(src);
        for (int j = 0; j < 8; j++) {
            const uint32_t w = ldg<uint32_t>(src + 260 + 4 * j);   // bsums[2j], bsums[2j+1]
            const int p = (int16_t)(w & 0xffff) + (int16_t)(w >> 16);
            lo[j >> 2] |= (uint32_t)(p & 127) << (8 * (j & 3));
            hi[j >> 2] |= (uint32_t)((p >> 7) & 0xff) << (8 * (j & 3));
        }
    }
    uint8_t *m = xm + ((size_t)b * na_pad + t) * MM_XM_BYTES;
    *reinterpret_cast<uint4 *>(m) = make_uint4(lo[0], lo[1], hi[0], hi[1]);
    *reinterpret_cast<uint4 *>(m + 16) = make_uint4(d, 0, 0, 0);
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

// one wave's 64 x 16 bytes from global memory straight into LDS: lane l's 16 bytes at base + off land at dst + 16*l
// (dst is wave-uniform). Written as inline assembly so that the compiler does not track these LDS writes: it would
// otherwise wait for every one of them to finish before any LDS read. The kernel orders them itself (s_waitcnt vmcnt +
// s_barrier before a stage is read). M0 is set inside the statement; nothing else in these kernels uses M0.
__device__ __forceinline__ void load_lds16(const uint8_t *base, uint32_t off, uint8_t *dst) {
    const uint32_t l = __builtin_amdgcn_readfirstlane((uint32_t)(size_t)(__attribute__((address_space(3))) uint8_t *)dst);
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(l)
                 : "memory");
}

template <int WN> struct MmGeom {
    static constexpr int BM = 64, BN = 32 * WN;
    static constexpr int W_BYTES = BM * 144, X_BYTES = BN * 256, M_BYTES = BN * MM_XM_BYTES;
    static constexpr int STAGE = W_BYTES + X_BYTES + M_BYTES, NS = 3;
    static constexpr int NWL = 3;                 // weight wave-loads per wave per stage (9 per stage, the rest dummies)
    static constexpr int NXL = BN / 16;           // activation wave-loads per wave (BN * 16 chunks / 64 lanes / 4 waves)
    static constexpr int LOADS = NWL + NXL + 1;   // + one meta wave-load
};

template <int N> __device__ __forceinline__ void wait_vmcnt() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
template <int N> struct IC { static constexpr int value = N; };

// WN: 16-wide activation tiles per wave; the workgroup tile is 64 rows x 32*WN activations. CONTRACT: the clang order
// (fused multiply-adds), else the gcc / scalar order. The three stages are separate LDS arrays and the superblock loop is
// unrolled by three, so every stage address is a constant.
template <int WN, bool CONTRACT>
__global__ __launch_bounds__(256) void mm_q4k_kernel(const MmJob *__restrict__ jobs, int njobs, MmJob single) {
    using G = MmGeom<WN>;
    constexpr int BN = G::BN, WM = 2;
    __shared__ __align__(16) uint8_t stage0[G::STAGE], stage1[G::STAGE], stage2[G::STAGE], sink[1024];

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
    const int row0 = J.r0 + rt * G::BM, tok0 = tt * BN;
    const int nbk = J.cols / 256;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int wr = (wave & 1) * 32, wt = (wave >> 1) * (16 * WN);   // this wave's rows / activations inside the tile
    const int lr = lane & 15, lg = lane >> 4;

    // ---- per-lane source offsets of the stage loads (the superblock adds a uniform stride)
    uint32_t woff[G::NWL];
#pragma unroll
    for (int kk = 0; kk < G::NWL; kk++) {
        const int c = 64 * (wave + 4 * kk) + lane, r = c / 9, q = c % 9;
        const int row = min(row0 + r, J.r1 - 1);   // rows past the end repeat the last one; their results are not stored
        woff[kk] = (uint32_t)((size_t)row * J.row_bytes) + 16 * q;
    }
    const int xt = 4 * wave + (lane >> 4);   // activation of this lane's first chunk; +16 per further wave-load
    const uint32_t xoff = (uint32_t)xt * 256 + 16 * ((lane & 15) ^ (xt & 15));
    const uint32_t moff = (uint32_t)(64 * wave + lane) * 16;
    const bool m_real = 64 * wave < G::M_BYTES / 16;

    auto stage = [&](auto S) -> uint8_t * {
        if constexpr (decltype(S)::value == 0) return stage0;
        else if constexpr (decltype(S)::value == 1) return stage1;
        else return stage2;
    };
    auto issue = [&](int b, auto S) {
        uint8_t *wb = stage(S), *xb = wb + G::W_BYTES, *mb = xb + G::X_BYTES;
        const uint8_t *wsrc = J.W + (size_t)b * 144;
        const uint8_t *xsrc = J.xq + ((size_t)b * J.na_pad + tok0) * 256;
        const uint8_t *msrc = J.xm + ((size_t)b * J.na_pad + tok0) * MM_XM_BYTES;
#pragma unroll
        for (int kk = 0; kk < G::NWL; kk++) {
            const int i = wave + 4 * kk;
            if (i < 9) load_lds16(wsrc, woff[kk], wb + 1024 * i);
            else load_lds16(wsrc, woff[0], sink);
        }
#pragma unroll
        for (int kk = 0; kk < G::NXL; kk++) load_lds16(xsrc, xoff + 4096 * kk, xb + 1024 * (wave + 4 * kk));
        if (m_real) load_lds16(msrc, moff, mb + 1024 * wave);
        else load_lds16(msrc, 0, sink);
    };

    float s[WM][WN][4];
#pragma unroll
    for (int a = 0; a < WM; a++)
#pragma unroll
        for (int c = 0; c < WN; c++)
#pragma unroll
            for (int i = 0; i < 4; i++) s[a][c][i] = 0.0f;

    const uint32_t nsh = lg >= 2 ? 4 : 0;   // high nibbles for lanes 32..63

    // one superblock b held in stage S; the loads of superblock b + 2 go to stage (S + 2) % 3
    auto step = [&](int b, auto S) {
        constexpr int SN = (decltype(S)::value + 2) % 3;
        if (b + 1 < nbk) wait_vmcnt<G::LOADS>();   // this wave's loads of stage b are in LDS (stage b+1 may still fly)
        else wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this wave's reads of stage b-1 are done
        __builtin_amdgcn_s_barrier();              // ... and every wave's loads; every wave is also done with stage b-1
        asm volatile("" ::: "memory");
        if (b + 2 < nbk) issue(b + 2, IC<SN>{});
        const uint8_t *wb = stage(S), *xb = wb + G::W_BYTES, *mb = xb + G::X_BYTES;

        // rows' 6-bit scales and mins, byte-parallel (scale_min_k4, src/es_quant.c:75-83)
        uint32_t sl16[WM][4], sh16[WM][4], mnb[WM][2];
#pragma unroll
        for (int a = 0; a < WM; a++) {
            const uint4 h = *reinterpret_cast<const uint4 *>(wb + (wr + 16 * a + lr) * 144);
            const uint32_t sc0 = h.y & 0x3f3f3f3fu, sc1 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
            mnb[a][0] = h.z & 0x3f3f3f3fu;
            mnb[a][1] = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {   // this lane's sub-block in slice ks: j = 2ks + (lg >> 1)
                const uint32_t scw = ks < 2 ? sc0 : sc1;
                const uint32_t sc = (scw >> (16 * (ks & 1) + 8 * (lg >> 1))) & 0xff;
                sl16[a][ks] = (sc & 7) * 0x00010001u;
                sh16[a][ks] = (sc >> 3) * 0x00010001u;
            }
        }

        v4i acc_lo[WM][WN], acc_hi[WM][WN];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            v4i bop[WN];
#pragma unroll
            for (int c = 0; c < WN; c++)
                bop[c] = *reinterpret_cast<const v4i *>(xb + (wt + 16 * c + lr) * 256 + 16 * ((4 * ks + lg) ^ lr));
            v4i alo[WM], ahi[WM];
#pragma unroll
            for (int a = 0; a < WM; a++) {
                const uint4 q = *reinterpret_cast<const uint4 *>(wb + (wr + 16 * a + lr) * 144 + 16 + 32 * ks + 16 * (lg & 1));
                const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const uint32_t nib = (qq[i] >> nsh) & 0x0f0f0f0fu;
                    alo[a][i] = (int)pk_mul_u16(nib, sl16[a][ks]);   // byte * scale <= 105: no carry between bytes
                    ahi[a][i] = (int)pk_mul_u16(nib, sh16[a][ks]);
                }
            }
#pragma unroll
            for (int a = 0; a < WM; a++)
#pragma unroll
                for (int c = 0; c < WN; c++) {
                    const v4i zlo = ks ? acc_lo[a][c] : v4i{0, 0, 0, 0}, zhi = ks ? acc_hi[a][c] : v4i{0, 0, 0, 0};
                    acc_lo[a][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(alo[a], bop[c], zlo, 0, 0, 0);
                    acc_hi[a][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ahi[a], bop[c], zhi, 0, 0, 0);
                }
        }

        // mins on the matrix cores: only k positions 0..7 (lanes 0..15, first 8 bytes) are non-zero
        v4i mn_lo[WM][WN], mn_hi[WM][WN];
        float td[WN];
        {
            v4i amin[WM], blo[WN], bhi[WN];
#pragma unroll
            for (int a = 0; a < WM; a++) amin[a] = lg == 0 ? v4i{(int)mnb[a][0], (int)mnb[a][1], 0, 0} : v4i{0, 0, 0, 0};
#pragma unroll
            for (int c = 0; c < WN; c++) {
                const uint8_t *m = mb + (wt + 16 * c + lr) * MM_XM_BYTES;
                const uint4 v = *reinterpret_cast<const uint4 *>(m);
                td[c] = *reinterpret_cast<const float *>(m + 16);
                blo[c] = lg == 0 ? v4i{(int)v.x, (int)v.y, 0, 0} : v4i{0, 0, 0, 0};
                bhi[c] = lg == 0 ? v4i{(int)v.z, (int)v.w, 0, 0} : v4i{0, 0, 0, 0};
            }
#pragma unroll
            for (int a = 0; a < WM; a++)
#pragma unroll
                for (int c = 0; c < WN; c++) {
                    mn_lo[a][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(amin[a], blo[c], v4i{0, 0, 0, 0}, 0, 0, 0);
                    mn_hi[a][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(amin[a], bhi[c], v4i{0, 0, 0, 0}, 0, 0, 0);
                }
        }

        // ---- fp32 epilogue of superblock b, per (row, activation), in the reference's order
#pragma unroll
        for (int a = 0; a < WM; a++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t dd = *reinterpret_cast<const uint32_t *>(wb + (wr + 16 * a + 4 * lg + i) * 144);
                const float d = half_bits_to_float(dd), dmin = half_bits_to_float(dd >> 16);
#pragma unroll
                for (int c = 0; c < WN; c++) {
                    const int dot = acc_lo[a][c][i] + 8 * acc_hi[a][c][i];
                    const int mins = mn_lo[a][c][i] + 128 * mn_hi[a][c][i];
                    const float q = dmin * static_cast<float>(mins);
                    if constexpr (CONTRACT) s[a][c][i] = __builtin_fmaf(td[c], __builtin_fmaf(d, static_cast<float>(dot), -q), s[a][c][i]);
                    else s[a][c][i] = s[a][c][i] + td[c] * (d * static_cast<float>(dot) - q);
                }
            }
        asm volatile("" ::: "memory");   // stage b's LDS reads stay before the next iteration's barrier
    };

    issue(0, IC<0>{});
    if (nbk > 1) issue(1, IC<1>{});
    for (int b = 0; b < nbk; b += 3) {
        step(b, IC<0>{});
        if (b + 1 < nbk) step(b + 1, IC<1>{});
        if (b + 2 < nbk) step(b + 2, IC<2>{});
    }

    // ---- outputs
#pragma unroll
    for (int a = 0; a < WM; a++)
#pragma unroll
        for (int c = 0; c < WN; c++) {
            const int t = tok0 + wt + 16 * c + lr;
            if (t >= J.na) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int r = row0 + wr + 16 * a + 4 * lg + i;
                if (r < J.r1) J.y[(size_t)t * J.ystride + r] = s[a][c][i];
            }
        }
}

// ---- launch glue -------------------------------------------------------------------------------------------------
hipError_t mm_prep_launch(const uint8_t *act, uint64_t astride, int na, int na_pad, int nbk, uint8_t *xq, uint8_t *xm,
                          hipStream_t s) {
    const long total = (long)nbk * na_pad * 17;
    const int threads = 256;
    hipLaunchKernelGGL(act_prep_q8k, dim3((unsigned)((total + threads - 1) / threads)), dim3(threads), 0, s, act, astride, na,
                       na_pad, nbk, xq, xm);
    return hipGetLastError();
}

template <int WN> static hipError_t mm_launch_wn(const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                                                 hipStream_t s) {
    if (order == ES_HIP_ORDER_X86_CONTRACT)
        hipLaunchKernelGGL((mm_q4k_kernel<WN, true>), dim3(grid), dim3(256), 0, s, jobs, njobs, single);
    else
        hipLaunchKernelGGL((mm_q4k_kernel<WN, false>), dim3(grid), dim3(256), 0, s, jobs, njobs, single);
    return hipGetLastError();
}

hipError_t mm_launch(int type, int bm, int bn, const MmJob *jobs, int njobs, const MmJob &single, int grid, int order,
                     hipStream_t s) {
    if (type != ES_HIP_Q4_K || bm != 64) return hipErrorInvalidValue;
    if (bn == 128) return mm_launch_wn<4>(jobs, njobs, single, grid, order, s);
    if (bn == 64) return mm_launch_wn<2>(jobs, njobs, single, grid, order, s);
    return hipErrorInvalidValue;
}

}  // namespace esq
