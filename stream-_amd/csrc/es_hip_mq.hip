// Small batches on the int8 matrix cores: es_matvec_multi (src/es_quant.c:1818-1850) for K-quant rows against 8..64
// activations (MoE experts, prompt tails, small decode batches), where the vector kernels spend most of their time on
// per-activation integer work.
//
// Every wave owns 16 rows and all of the job's activations (up to four 16-wide tiles), and streams its rows' superblocks
// straight from memory into registers: weights are read once, there is no LDS and no barrier. The activations come from the
// same pre-pass planes as the prefill kernel (xq[b][t][256] int8, per-superblock meta, xd[b][t] float), read as MFMA B
// operands from L2.
// MFMA v_mfma_i32_16x16x64_i8, per 64-wide k slice ks of a superblock: lane l supplies row l%16 (A) / activation l%16 (B),
// k positions 16*(l/16) .. +16, i.e. elements 64ks + 16*(l/16) + [0, 16). Output: lane l, register i holds
// D[4*(l/16) + i][l % 16] (checked on the device).
// Per format (the integers are exact, the float epilogue follows the reference's order per superblock):
//   Q4_K (src/es_quant.c:1056-1080, 1324-1343): the 4-bit code times its 6-bit sub-block scale is split into two int8 planes
//     (q*sl, q*sh with sc = 8*sh + sl); mins = sum_j mn_j * (bsums[2j] + bsums[2j+1]) through one more pair of MFMAs
//     with the pair sums split as 128*hi + lo.
//   Q2_K (src/es_q2k.c:127-148, src/es_quant.c:1344-1368): the 2-bit code times its 4-bit scale (<= 45) is one int8
//     plane; summs = sum_g bsums[g] * (sc[g] >> 4) through a pair of MFMAs with bsums split as 128*hi + lo.
#include "es_hip_common.h"

namespace esq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef uint16_t u16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pk_mul16(uint32_t a, uint32_t b) {   // v_pk_mul_lo_u16
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) * __builtin_bit_cast(u16x2, b));
}
// 16 bytes at a 4-byte aligned address
__device__ __forceinline__ uint4 ld16a4(const uint8_t *p) {
    return make_uint4(ldg<uint32_t>(p), ldg<uint32_t>(p + 4), ldg<uint32_t>(p + 8), ldg<uint32_t>(p + 12));
}
template <int N> struct IC { static constexpr int value = N; };
__device__ __forceinline__ v4i mfma(v4i a, v4i b, v4i c) { return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0); }

// ---- per-format superblock work ---------------------------------------------------------------------------------------
// Raw: the bytes a lane loads for its row; A: the lane's A operands; then per activation tile the integers and the chain.
template <int F> struct Mq;

template <> struct Mq<ES_HIP_Q4_K> {
    static constexpr int BB = 144;
    struct Raw { uint4 h, q[4]; };
    struct A { v4i lo[4], hi[4], mn; };
    static __device__ __forceinline__ void load(const uint8_t *blk, int lg, Raw &r) {
        r.h = ldw4(blk);
#pragma unroll
        for (int ks = 0; ks < 4; ks++) r.q[ks] = ldw4(blk + 16 + 32 * ks + 16 * (lg & 1));
    }
    static __device__ __forceinline__ uint32_t dd(const Raw &r) { return r.h.x; }   // d | dmin << 16
    static __device__ __forceinline__ void build(const Raw &r, int lg, A &a) {
        // 6-bit scales and mins, byte-parallel (scale_min_k4, src/es_quant.c:75-83)
        const uint32_t sc0 = r.h.y & 0x3f3f3f3fu, sc1 = (r.h.w & 0x0f0f0f0fu) | ((r.h.y >> 2) & 0x30303030u);
        const uint32_t mn0 = r.h.z & 0x3f3f3f3fu, mn1 = ((r.h.w >> 4) & 0x0f0f0f0fu) | ((r.h.z >> 2) & 0x30303030u);
        a.mn = lg == 0 ? v4i{(int)mn0, (int)mn1, 0, 0} : v4i{0, 0, 0, 0};
        const uint32_t nsh = lg >= 2 ? 4 : 0;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {   // sub-block j = 2ks + (lg >> 1)
            const uint32_t sc = ((ks < 2 ? sc0 : sc1) >> (16 * (ks & 1) + 8 * (lg >> 1))) & 0xff;
            const uint32_t sl = (sc & 7) * 0x00010001u, sh = (sc >> 3) * 0x00010001u;
            const uint32_t q[4] = {r.q[ks].x, r.q[ks].y, r.q[ks].z, r.q[ks].w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t nib = (q[i] >> nsh) & 0x0f0f0f0fu;
                a.lo[ks][i] = (int)pk_mul16(nib, sl);
                a.hi[ks][i] = (int)pk_mul16(nib, sh);
            }
        }
    }
    struct Acc { v4i lo, hi, mlo, mhi; };
    // meta: 16 bytes per activation (pair sums low bytes | high bytes)
    static __device__ __forceinline__ void mma(const A &a, const v4i *xb, uint4 m, Acc &c) {
        const v4i blo = v4i{(int)m.x, (int)m.y, (int)m.z, (int)m.w}, bhi = v4i{(int)m.z, (int)m.w, (int)m.x, (int)m.y};
        c.mlo = mfma(a.mn, blo, v4i{0, 0, 0, 0});
        c.mhi = mfma(a.mn, bhi, v4i{0, 0, 0, 0});
        c.lo = mfma(a.lo[0], xb[0], v4i{0, 0, 0, 0});
        c.hi = mfma(a.hi[0], xb[0], v4i{0, 0, 0, 0});
#pragma unroll
        for (int ks = 1; ks < 4; ks++) {
            c.lo = mfma(a.lo[ks], xb[ks], c.lo);
            c.hi = mfma(a.hi[ks], xb[ks], c.hi);
        }
    }
    template <bool CONTRACT>
    static __device__ __forceinline__ float chain(float s, const Acc &c, int i, uint32_t dd, float td) {
        const float d = half_bits_to_float(dd), dmin = half_bits_to_float(dd >> 16);
        const int dot = c.lo[i] + 8 * c.hi[i], mins = c.mlo[i] + 128 * c.mhi[i];
        const float q = dmin * static_cast<float>(mins);
        if constexpr (CONTRACT) return __builtin_fmaf(td, __builtin_fmaf(d, static_cast<float>(dot), -q), s);
        else return s + td * (d * static_cast<float>(dot) - q);
    }
};

template <> struct Mq<ES_HIP_Q2_K> {
    static constexpr int BB = 84;
    struct Raw { uint4 sc, q[2]; uint32_t dd; };
    struct A { v4i v[4], mn; };
    static __device__ __forceinline__ void load(const uint8_t *blk, int lg, Raw &r) {
        r.sc = ld16a4(blk);
#pragma unroll
        for (int n = 0; n < 2; n++) r.q[n] = ld16a4(blk + 16 + 32 * n + 16 * (lg & 1));
        r.dd = ldg<uint32_t>(blk + 80);
    }
    static __device__ __forceinline__ uint32_t dd(const Raw &r) { return r.dd; }   // d | dmin << 16
    static __device__ __forceinline__ void build(const Raw &r, int lg, A &a) {
        const uint32_t scw[4] = {r.sc.x, r.sc.y, r.sc.z, r.sc.w};
        a.mn = lg == 0 ? v4i{(int)((scw[0] >> 4) & 0x0f0f0f0fu), (int)((scw[1] >> 4) & 0x0f0f0f0fu),
                             (int)((scw[2] >> 4) & 0x0f0f0f0fu), (int)((scw[3] >> 4) & 0x0f0f0f0fu)}
                       : v4i{0, 0, 0, 0};
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            // elements 64ks + 16lg + i: byte qs[32(ks/2) + 16(lg&1) + i], shift 2(2(ks&1) + (lg>>1)); group g = 4ks + lg
            const int shift = 2 * (2 * (ks & 1) + (lg >> 1));
            const uint32_t sc = ((scw[ks] >> (8 * lg)) & 0x0f) * 0x00010001u;
            const uint4 q = r.q[ks >> 1];
            const uint32_t qq[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; i++) a.v[ks][i] = (int)pk_mul16((qq[i] >> shift) & 0x03030303u, sc);   // <= 45
        }
    }
    struct Acc { v4i v, mlo, mhi; };
    // meta: 32 bytes per activation (bsums low bytes | high bytes); the lane reads its 16-byte half for each operand
    static __device__ __forceinline__ void mma(const A &a, const v4i *xb, uint4 mlo, uint4 mhi, Acc &c) {
        c.mlo = mfma(a.mn, v4i{(int)mlo.x, (int)mlo.y, (int)mlo.z, (int)mlo.w}, v4i{0, 0, 0, 0});
        c.mhi = mfma(a.mn, v4i{(int)mhi.x, (int)mhi.y, (int)mhi.z, (int)mhi.w}, v4i{0, 0, 0, 0});
        c.v = mfma(a.v[0], xb[0], v4i{0, 0, 0, 0});
#pragma unroll
        for (int ks = 1; ks < 4; ks++) c.v = mfma(a.v[ks], xb[ks], c.v);
    }
    template <bool CONTRACT>
    static __device__ __forceinline__ float chain(float s, const Acc &c, int i, uint32_t dd, float td) {
        const float d = half_bits_to_float(dd), dmin = half_bits_to_float(dd >> 16);
        const float dall = td * d, dmn = td * dmin;
        const float q = dmn * static_cast<float>(c.mlo[i] + 128 * c.mhi[i]);
        const int isum = c.v[i];
        if constexpr (CONTRACT) return s + __builtin_fmaf(dall, static_cast<float>(isum), -q);
        else return s + (dall * static_cast<float>(isum) - q);
    }
};

// ---- the kernel -------------------------------------------------------------------------------------------------------
// WN: 16-wide activation tiles per wave (the job's activations rounded up to 16, at most 64 per launch group).
template <int F, int WN, bool CONTRACT>
__global__ __launch_bounds__(256, 2) void mq_kernel(const MqJob *__restrict__ jobs, int njobs, MqJob single) {
    using M = Mq<F>;
    MqJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int tile = blockIdx.x - J.tile0;
    const int row0 = J.r0 + (tile * 4 + wave) * 16;
    if (row0 >= J.r1) return;   // whole waves only: this wave has no rows (the others of the workgroup may)
    const int nbk = J.cols / 256;
    const int myrow = min(row0 + lr, J.r1 - 1);   // rows past the end repeat the last one; their results are not stored
    const uint8_t *wrow = J.W + (size_t)myrow * J.row_bytes;
    constexpr int MB = F == ES_HIP_Q4_K ? 16 : 32;   // meta bytes per activation and superblock
    const uint8_t *xd_plane = J.xm + (size_t)nbk * J.na_pad * MB;

    float s[WN][4];
#pragma unroll
    for (int c = 0; c < WN; c++)
#pragma unroll
        for (int i = 0; i < 4; i++) s[c][i] = 0.0f;

    // the activation side of one superblock: B operands, meta, scales of this lane's activations
    constexpr int MQ = MB / 16;
    struct Bset { v4i xb[WN][4]; uint4 m[WN][MQ]; float td[WN]; };
    auto load_b = [&](int b, Bset &B) {
        const size_t tb = (size_t)b * J.na_pad + J.t0;
#pragma unroll
        for (int c = 0; c < WN; c++) {
            const size_t t = tb + 16 * c + lr;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) B.xb[c][ks] = ldg<v4i>(J.xq + t * 256 + 16 * (4 * ks + lg));
#pragma unroll
            for (int q = 0; q < MQ; q++) B.m[c][q] = ldg<uint4>(J.xm + t * MB + 16 * q);
            B.td[c] = ldg<float>(xd_plane + t * 4);
        }
    };
    // Weights run DEPTH superblocks ahead in a register ring that shifts by one each step; for up to two activation tiles
    // the activation side of superblock b + 1 is loaded while b is computed. Every load is unconditional (past the last
    // superblock the last one is read again), so the compiler's memory-counter waits count exactly and the loads in
    // flight are never drained early.
    constexpr int DEPTH = (F == ES_HIP_Q4_K ? 2 : 3) - (WN > 2 ? 1 : 0);
    constexpr bool PF = WN <= (F == ES_HIP_Q4_K ? 1 : 2);
    typename M::Raw ring[DEPTH];
#pragma unroll
    for (int d = 0; d < DEPTH; d++) M::load(wrow + (size_t)min(d, nbk - 1) * M::BB, lg, ring[d]);
    Bset cur, nxt;
    load_b(0, cur);
    for (int b = 0; b < nbk; b++) {
        typename M::A a;
        M::build(ring[0], lg, a);
        const uint32_t hdd = M::dd(ring[0]);
        if constexpr (PF) load_b(min(b + 1, nbk - 1), nxt);   // issued in the order they are needed
#pragma unroll
        for (int d = 0; d + 1 < DEPTH; d++) ring[d] = ring[d + 1];
        M::load(wrow + (size_t)min(b + DEPTH, nbk - 1) * M::BB, lg, ring[DEPTH - 1]);
        uint32_t dd[4];   // d | dmin of output rows 4lg + i, held by lanes 4lg + i (the A layout puts row r in lane r)
#pragma unroll
        for (int i = 0; i < 4; i++) dd[i] = __shfl(hdd, 4 * lg + i);
#pragma unroll
        for (int c = 0; c < WN; c++) {
            typename M::Acc acc;
            if constexpr (F == ES_HIP_Q4_K) M::mma(a, cur.xb[c], cur.m[c][0], acc);
            else M::mma(a, cur.xb[c], cur.m[c][0], cur.m[c][MQ - 1], acc);
#pragma unroll
            for (int i = 0; i < 4; i++) s[c][i] = M::template chain<CONTRACT>(s[c][i], acc, i, dd[i], cur.td[c]);
        }
        if constexpr (PF) cur = nxt;
        else load_b(min(b + 1, nbk - 1), cur);
    }

    // outputs: lane holds rows row0 + 4lg + i of activation t0 + 16c + lr
#pragma unroll
    for (int c = 0; c < WN; c++) {
        const int t = J.t0 + 16 * c + lr;
        if (t >= J.na) continue;
        const int r = row0 + 4 * lg;
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

template <int F, int WN>
static hipError_t mq_launch_wn(const MqJob *jobs, int njobs, const MqJob &single, int grid, int order, hipStream_t s) {
    if (order == ES_HIP_ORDER_X86_CONTRACT)
        hipLaunchKernelGGL((mq_kernel<F, WN, true>), dim3(grid), dim3(256), 0, s, jobs, njobs, single);
    else
        hipLaunchKernelGGL((mq_kernel<F, WN, false>), dim3(grid), dim3(256), 0, s, jobs, njobs, single);
    return hipGetLastError();
}

template <int F>
static hipError_t mq_launch_f(int wn, const MqJob *jobs, int njobs, const MqJob &single, int grid, int order, hipStream_t s) {
    switch (wn) {
    case 1: return mq_launch_wn<F, 1>(jobs, njobs, single, grid, order, s);
    case 2: return mq_launch_wn<F, 2>(jobs, njobs, single, grid, order, s);
    case 3: return mq_launch_wn<F, 3>(jobs, njobs, single, grid, order, s);
    case 4: return mq_launch_wn<F, 4>(jobs, njobs, single, grid, order, s);
    }
    return hipErrorInvalidValue;
}

hipError_t mq_launch(int type, int wn, const MqJob *jobs, int njobs, const MqJob &single, int grid, int order, hipStream_t s) {
    if (type == ES_HIP_Q4_K) return mq_launch_f<ES_HIP_Q4_K>(wn, jobs, njobs, single, grid, order, s);
    if (type == ES_HIP_Q2_K) return mq_launch_f<ES_HIP_Q2_K>(wn, jobs, njobs, single, grid, order, s);
    return hipErrorInvalidValue;
}

}  // namespace esq
