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
// Loads: per block a lane reads the aligned dwords around its row's d (and Q5_0 high bits) and its group's code dword
// (blocks are 18 or 22 bytes, so fields sit at 2-byte alignment; unaligned dword loads cost more than two aligned ones),
// and from the kind 3 pre-pass layout 16 bytes of activation values (one contiguous 1 KB wave load per block) and the
// activation's block scale. P blocks are in flight while one is computed. No LDS, no barriers.
#include "es_hip_common.h"

namespace esq {
namespace {

typedef int v16i __attribute__((ext_vector_type(16)));

template <int F> struct Mb32Fmt;
// Q4_0: d f16 @0, qs[16] @2; codes 0..15, offset 8. Q5_0: d f16 @0, qh u32 @2, qs[16] @6; codes 0..31, offset 16.
// (code - offset) as int8 per byte: (code + 0x80 - offset) ^ 0x80, no carry between bytes since code + 0x80 - offset < 256.
template <> struct Mb32Fmt<ES_HIP_Q4_0> { static constexpr int QS = 2, QH = -1; static constexpr uint32_t BIAS = 0x78787878u; };
template <> struct Mb32Fmt<ES_HIP_Q5_0> { static constexpr int QS = 6, QH = 2; static constexpr uint32_t BIAS = 0x70707070u; };

struct Stage {
    uint32_t w0, w1;   // the aligned dwords at and after the block's start: d (and Q5_0 qh)
    uint32_t qa, qb;   // the aligned dwords at and after this lane's code dword
    u32x4 y;           // 16 activation values (this lane's half of the block)
    float yd;          // the activation block's scale
};

// wblk: the block (2-byte aligned); every dword read lies inside it: the block's first two aligned dwords (it is at least
// 18 bytes long), the aligned dword holding the code field's first byte, and the next one unless that would pass the
// block's last aligned dword (then the field is 4-byte aligned and the second dword is not used).
template <int F>
__device__ __forceinline__ void load_stage(Stage &s, const uint8_t *wblk, const uint8_t *xq, const uint8_t *xm, int lane, int gq) {
    constexpr int BB = Fmt<F>::BB;
    const uintptr_t a = reinterpret_cast<uintptr_t>(wblk);
    const uint8_t *const al = wblk - (a & 2);
    s.w0 = ldg<uint32_t>(al);
    s.w1 = Mb32Fmt<F>::QH >= 0 ? ldg<uint32_t>(al + 4) : 0u;
    const uintptr_t f = a + Mb32Fmt<F>::QS + 4 * gq, fa = f & ~uintptr_t(3), last = (a + BB - 1) & ~uintptr_t(3);
    s.qa = ldg<uint32_t>(reinterpret_cast<const void *>(fa));
    s.qb = ldg<uint32_t>(reinterpret_cast<const void *>(fa + 4 <= last ? fa + 4 : fa));
    s.y = ldg<u32x4>(xq + 16 * lane);
    s.yd = ldg<float>(xm + 4 * (lane & 31));
}

// Tiles of 4 waves x 4 rows against 32 activations [t0, t0 + 32) of the job (the pre-pass wrote zeros for those past na;
// they are not stored). P: blocks in flight per wave (even). X86: the AVX2 order (else the scalar one).
template <int F, int P, bool X86>
__global__ __launch_bounds__(256) void mb32m_kernel(const MbJob *__restrict__ jobs, int njobs, MbJob single) {
    constexpr int BB = Fmt<F>::BB;
    static_assert(P % 2 == 0, "block parity is the stage's");
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
    const int nshift = 4 * (gi >> 2);
    const uint8_t *const wrow = J.W + (size_t)min(row0 + (n >> 3), J.r1 - 1) * J.row_bytes;
    // Blocks are 2 mod 4 bytes long, so their 2-byte misalignment alternates: block b of this row starts misaligned by
    // wmis ^ (2 * (b & 1)) bytes. The Q5_0 high bits of group gi sit at bit 16 + 4 gi of {w1, w0} (32 + 4 gi when
    // misaligned); the code dword is misaligned exactly when the block is not (QS is 2 mod 4).
    const uint32_t wmis = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(wrow)) & 2u;
    const int t = J.t0 + n;   // B side: activation t (the job's planes start at this tile)
    const int nbk = J.cols / 32;

    float acc[16];   // x86: acc[4 r + jj] = chain of group 4 h + jj of row r; scalar: acc[r] = the row's chain
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = 0.0f;

    auto step = [&](const Stage &c, int parity) {
        const uint32_t mis = wmis ^ (2u * parity);
        const uint32_t qs = alignbyte(c.qb, c.qa, mis ^ 2u);
        uint32_t q = (qs >> nshift) & 0x0f0f0f0fu;
        if constexpr (F == ES_HIP_Q5_0) {   // bit e of qh -> bit 4 of byte e
            const uint64_t hw = (static_cast<uint64_t>(c.w1) << 32 | c.w0) >> (16 + 8 * mis + 4 * gi);
            q |= (((static_cast<uint32_t>(hw) & 15u) * 0x00204081u) & 0x01010101u) << 4;
        }
        q = (q + Mb32Fmt<F>::BIAS) ^ 0x80808080u;
        v4i a;
#pragma unroll
        for (int j = 0; j < 4; j++) a[j] = static_cast<int>(q & sel[j]);
        const v16i d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, __builtin_bit_cast(v4i, c.y), v16i{}, 0, 0, 0);
        // d of rows 0..3 (float), read from lanes 0, 8, 16, 24, which loaded them
        const float wd = half_bits_to_float(alignbyte(c.w0, c.w0, mis));
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

    auto load = [&](Stage &s, int b) {
        load_stage<F>(s, wrow + (size_t)b * BB, J.xq + (size_t)b * 1024, J.xm + (size_t)b * 128, lane, gq);
    };
    Stage st[P];
#pragma unroll
    for (int p = 0; p < P; p++) load(st[p], min(p, nbk - 1));
    int b0 = 0;
    for (; b0 + P <= nbk; b0 += P) {   // block b0 + p is in st[p]; b0 is a multiple of P, so its parity is p's
#pragma unroll
        for (int p = 0; p < P; p++) {
            step(st[p], p & 1);
            load(st[p], min(b0 + p + P, nbk - 1));   // past the end: a harmless reload of the last block
        }
    }
#pragma unroll
    for (int p = 0; p < P; p++)
        if (b0 + p < nbk) step(st[p], p & 1);

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
