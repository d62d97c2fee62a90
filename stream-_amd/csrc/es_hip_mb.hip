// Batched 32-wide formats (Q4_0 / Q5_0 against many activations) on the matrix cores.
//
// The reference's AVX2 path forms, per 32-element block, eight integer lane sums lane_i = sum over elements 4i..4i+3 of
// (code - offset) * y and folds them into eight fused chains acc_i = fma((float)lane_i, d * yd, acc_i) in block order,
// summed at the end as ((0+4)+(2+6))+((1+5)+(3+7)) (src/es_quant.c:1185-1187, 1252-1323); its scalar path adds
// (d * yd) * (float)sum-of-all-32 to one chain (src/es_quant.c:1013-1055).
//
// Here one v_mfma_i32_32x32x32_i8 per block and wave produces every lane sum of 4 rows x 32 activations at once: output
// row m = 8 r + i is (weight row r, group i), and A row m holds only group i's four signed codes (code - offset), at the
// four k positions where B (the activation's 32 int8 values, natural order) holds that group's y; every other A byte is
// zero. So D[8 r + i][n] = lane_i of row r against activation n, exactly. Each lane then owns the chains of one activation
// and four groups of all four rows (the MFMA's output layout), run in block order as the reference does.
//
// Operand layouts of v_mfma_i32_32x32x32_i8 (wave64): lane l supplies A row l % 32 and B column l % 32, both for the same
// 16 k positions (half l / 32 of the 32); D register j of lane l is element [8 (j / 4) + 4 (l / 32) + j % 4][l % 32].
// Which 16 k positions a half covers only has to agree between A and B, and it does by construction: the lane that
// supplies group i's codes in register i % 4 of half i / 4 is matched by the activation bytes 16 (i / 4) + 4 (i % 4)..+3
// in the same register of the same half.
//
// Loads: per block a lane reads its group's code dword (+ the Q5_0 high-bit dword) and its row's d, and 16 bytes of its
// activation's block plus that block's d; P blocks are in flight while one is computed. No LDS, no barriers.
#include "es_hip_common.h"

namespace esq {
namespace {

typedef int v16i __attribute__((ext_vector_type(16)));
typedef uint32_t u32_a2 __attribute__((aligned(2)));   // a dword at a 2-byte aligned address (blocks are 18 / 22 bytes)

template <int F> struct Mb32Fmt;
// Q4_0: d f16 @0, qs[16] @2; codes 0..15, offset 8. Q5_0: d f16 @0, qh u32 @2, qs[16] @6; codes 0..31, offset 16.
// (code - offset) as int8 per byte: (code + 0x80 - offset) ^ 0x80, no carry between bytes since code + 0x80 - offset < 256.
template <> struct Mb32Fmt<ES_HIP_Q4_0> { static constexpr int QS = 2, QH = -1; static constexpr uint32_t BIAS = 0x78787878u; };
template <> struct Mb32Fmt<ES_HIP_Q5_0> { static constexpr int QS = 6, QH = 2; static constexpr uint32_t BIAS = 0x70707070u; };

struct Stage {
    uint32_t qs, qh, d16;   // this lane's group codes (packed nibbles), high bits, its row's d
    u32x4 y;                // 16 activation bytes (this lane's half of the block)
    float yd;               // the activation block's d
};

template <int F>
__device__ __forceinline__ void load_stage(Stage &s, const uint8_t *wblk, const uint8_t *xblk, int gq, int h) {
    s.d16 = ldg<uint16_t>(wblk);
    s.qs = ldg<u32_a2>(wblk + Mb32Fmt<F>::QS + 4 * gq);
    if constexpr (Mb32Fmt<F>::QH >= 0) s.qh = ldg<u32_a2>(wblk + Mb32Fmt<F>::QH);
    else s.qh = 0;
    s.y = ldg<u32x4>(xblk + 4 + 16 * h);
    s.yd = ldg<float>(xblk);
}

// Tiles of 4 waves x 4 rows against 32 activations [t0, t0 + 32) of the job (those past na are computed on a copy of
// activation na - 1 and not stored). P: blocks in flight per wave. X86: the AVX2 order (else the scalar one).
template <int F, int P, bool X86>
__global__ __launch_bounds__(256) void mb32m_kernel(const MbJob *__restrict__ jobs, int njobs, MbJob single) {
    constexpr int BB = Fmt<F>::BB, AB = Fmt<F>::AB;
    MbJob J;
    if (jobs) J = jobs[find_tile_job(jobs, njobs, blockIdx.x)];
    else J = single;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = lane & 31, h = lane >> 5;
    const int row0 = J.r0 + ((blockIdx.x - J.tile0) * 4 + wave) * 4;
    if (row0 >= J.r1) return;   // wave-uniform; nothing here synchronises waves

    // A side: this lane supplies group gi of row row0 + n / 8 (non-zero only in the half that holds the group)
    const int gi = n & 7, gq = gi & 3;
    const uint32_t keep = (gi >> 2) == h ? 0xffffffffu : 0u;
    uint32_t sel[4];
#pragma unroll
    for (int j = 0; j < 4; j++) sel[j] = j == gq ? keep : 0u;
    const int nshift = 4 * (gi >> 2), hshift = 4 * gi;
    const uint8_t *const wrow = J.W + (size_t)min(row0 + (n >> 3), J.r1 - 1) * J.row_bytes;
    // B side: activation t
    const int t = J.t0 + n;
    const int tq = min(t, J.na - 1);
    const uint8_t *const xrow = J.act + (size_t)(J.arow ? ldg<int>(J.arow + tq) : tq) * J.astride;
    const int nbk = J.cols / 32;

    float acc[16];   // x86: acc[4 r + jj] = chain of group 4 h + jj of row r; scalar: acc[r] = the row's chain
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = 0.0f;

    auto step = [&](const Stage &c) {
        uint32_t q = (c.qs >> nshift) & 0x0f0f0f0fu;
        if constexpr (F == ES_HIP_Q5_0) q |= ((((c.qh >> hshift) & 15u) * 0x00204081u) & 0x01010101u) << 4;   // bit e of qh -> bit 4 of byte e
        q = (q + Mb32Fmt<F>::BIAS) ^ 0x80808080u;
        v4i a;
#pragma unroll
        for (int j = 0; j < 4; j++) a[j] = static_cast<int>(q & sel[j]);
        const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, __builtin_bit_cast(v4i, c.y), v16i{}, 0, 0, 0);
        // d of rows 0..3 (float), read from lanes 0, 8, 16, 24, which loaded them
        const float wd = half_bits_to_float(c.d16);
        float dy[4];
#pragma unroll
        for (int r = 0; r < 4; r++)
            dy[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wd), 8 * r)) * c.yd;
        if constexpr (X86) {
#pragma unroll
            for (int j = 0; j < 16; j++) acc[j] = __builtin_fmaf(static_cast<float>(d[j]), dy[j >> 2], acc[j]);
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                int s4 = (d[4 * r] + d[4 * r + 1]) + (d[4 * r + 2] + d[4 * r + 3]);
                s4 += __shfl_xor(s4, 32);   // the other four groups
                acc[r] = acc[r] + dy[r] * static_cast<float>(s4);
            }
        }
    };

    Stage st[P];
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int b = min(p, nbk - 1);
        load_stage<F>(st[p], wrow + (size_t)b * BB, xrow + (size_t)b * AB, gq, h);
    }
    int b0 = 0;
    for (; b0 + P <= nbk; b0 += P) {
#pragma unroll
        for (int p = 0; p < P; p++) {
            step(st[p]);
            const int b = min(b0 + p + P, nbk - 1);   // past the end: a harmless reload of the last block
            load_stage<F>(st[p], wrow + (size_t)b * BB, xrow + (size_t)b * AB, gq, h);
        }
    }
#pragma unroll
    for (int p = 0; p < P; p++)
        if (b0 + p < nbk) step(st[p]);

    const bool tok_ok = t < J.na;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        float s;
        if constexpr (X86) {
            float u[4];
#pragma unroll
            for (int jj = 0; jj < 4; jj++) u[jj] = acc[4 * r + jj] + __shfl_xor(acc[4 * r + jj], 32);   // acc_jj + acc_(jj+4)
            s = (u[0] + u[2]) + (u[1] + u[3]);
        } else {
            s = acc[r];
        }
        const int row = row0 + r;
        if (h == 0 && tok_ok && row < J.r1) stg<float>(J.y + (size_t)t * J.ystride + row, s);
    }
}

}  // namespace

template <int F> static void launch(bool x86, const MbJob *jobs, int njobs, const MbJob &single, int grid, hipStream_t s) {
    constexpr int P = 8;
    if (x86) hipLaunchKernelGGL((mb32m_kernel<F, P, true>), dim3(grid), dim3(256), 0, s, jobs, njobs, single);
    else hipLaunchKernelGGL((mb32m_kernel<F, P, false>), dim3(grid), dim3(256), 0, s, jobs, njobs, single);
}

hipError_t mb32m_launch(int type, const MbJob *jobs, int njobs, const MbJob &single, int grid, int order, hipStream_t s) {
    const bool x86 = order != ES_HIP_ORDER_SCALAR;
    if (type == ES_HIP_Q4_0) launch<ES_HIP_Q4_0>(x86, jobs, njobs, single, grid, s);
    else if (type == ES_HIP_Q5_0) launch<ES_HIP_Q5_0>(x86, jobs, njobs, single, grid, s);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace esq
