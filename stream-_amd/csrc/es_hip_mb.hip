// Batched 32-wide formats (Q4_0 / Q5_0 / Q8_0 against many activations) on the matrix cores.
//
// The reference's AVX2 path forms, per 32-element block, eight integer lane sums lane_i = sum over elements 4i..4i+3 of
// (code - offset) * y and folds them into eight fused chains acc_i = fma((float)lane_i, d * yd, acc_i) in block order,
// summed at the end as ((0+4)+(2+6))+((1+5)+(3+7)) (src/es_quant.c:1185-1187, 1252-1323); its scalar path adds
// (d * yd) * (float)sum-of-all-32 to one chain (src/es_quant.c:1013-1055).
//
// Here two v_mfma_f32_32x32x16_f16 per block and wave produce every lane sum of 4 rows x 32 activations: output row
// m = 8 r + i is (weight row r, group i), and A row m holds only group i's four codes (code - offset, as halves) at the
// four k positions where B (the activation's 32 int8 values as halves) holds that group's values; every other A element is
// zero. The first instruction covers block elements 0..15 (groups 0..3), the second 16..31 (groups 4..7), accumulating
// into the same D. Every product and partial sum is an integer below 2^24 (|lane_i| <= 4 * 16 * 128), so D[8 r + i][n] is
// lane_i of row r against activation n exactly, already a float: the chains consume it directly. Each lane owns the
// chains of one activation and four groups of all four rows (the MFMA's output layout), run in block order as the
// reference does.
//
// Operand layouts of v_mfma_f32_32x32x16_f16 (wave64): lane l supplies A row l % 32 and B column l % 32, both for the same
// 8 k positions (half l / 32 of the 16); D register j of lane l is element [8 (j / 4) + 4 (l / 32) + j % 4][l % 32].
// Which 8 k positions a half covers only has to agree between A and B, and it does by construction: block element
// 16 q + 8 h + e (q: instruction, h: half, e < 8) sits in half e of A / B register e / 2 of lanes 32 h .. 32 h + 31, for A
// in the lanes of the group that holds it, for B in every lane (the pre-pass lays the activations out that way).
//
// Loads: per block a lane reads the aligned dwords around its row's d (and Q5_0 high bits) and its group's code dword
// (blocks are 18 or 22 bytes, so fields sit at 2-byte alignment; unaligned dword loads cost more than two aligned ones),
// and from the kind 3 pre-pass layout 32 bytes of activation values as halves (two contiguous 1 KB wave loads per block)
// and the activation's block scale. P blocks are in flight while one is computed, and each block's MFMAs are issued
// before the previous block's chains run. No LDS, no barriers.
#include "es_hip_common.h"

namespace esq {
namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

template <int F> struct Mb32Fmt;
// Q4_0: d f16 @0, qs[16] @2; codes 0..15, offset 8. Q5_0: d f16 @0, qh u32 @2, qs[16] @6; codes 0..31, offset 16.
// Q8_0: d f16 @0, int8 qs[32] @2 (BYTES: group i's four codes are dword i, taken as c + 128 in 0..255, offset 128).
// NEG: the half pair -(1024 + offset): a code c under the exponent of 1024 (bits 0x6400 | c) is 1024 + c, so adding NEG
// gives c - offset exactly.
template <> struct Mb32Fmt<ES_HIP_Q4_0> {
    static constexpr int QS = 2, QH = -1;
    static constexpr bool BYTES = false;
    static constexpr uint32_t NEG = 0xe408e408u;
};
template <> struct Mb32Fmt<ES_HIP_Q5_0> {
    static constexpr int QS = 6, QH = 2;
    static constexpr bool BYTES = false;
    static constexpr uint32_t NEG = 0xe410e410u;
};
template <> struct Mb32Fmt<ES_HIP_Q8_0> {
    static constexpr int QS = 2, QH = -1;
    static constexpr bool BYTES = true;
    static constexpr uint32_t NEG = 0xe480e480u;
};

struct Stage {
    uint32_t w0, w1;   // the aligned dwords at and after the block's start: d (and Q5_0 qh)
    uint32_t qa, qb;   // the aligned dwords at and after this lane's code dword
    v8h y0, y1;        // activation values 8 h .. 8 h + 7 and 16 + 8 h .. of this lane's activation, as halves
    float yd;          // the activation block's scale
};

// Tiles of 4 waves x 4 rows against 32 activations [t0, t0 + 32) of the job (the pre-pass wrote zeros for those past na;
// they are not stored). P: blocks in flight per wave (even). X86: the AVX2 order (else the scalar one).
template <int F, int P, bool X86>
__global__ __launch_bounds__(256) void mb32m_kernel(const MbJob *__restrict__ jobs, int njobs, MbJob single) {
    constexpr int BB = Fmt<F>::BB;
    static_assert(P % 2 == 0, "block parity is the stage's");
    MbJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int n = lane & 31, h = lane >> 5;
    const int row0 = J.r0 + ((blockIdx.x - J.tile0) * 4 + wave) * 4;
    if (row0 >= J.r1) return;   // wave-uniform; nothing here synchronises waves
    const int t = J.t0 + n;     // B side: activation t (the job's planes start at this tile)
    const int nbk = J.cols / 32;

    // A side: this lane supplies group gi of row row0 + n / 8: its four codes go to halves 4 (gi & 1) .. +3 of
    // instruction gi / 4, in the half h == (gi & 3) / 2 of the lanes; registers elsewhere are zero.
    const int gi = n & 7, gq = gi & 3;
    const bool mine = ((gi & 3) >> 1) == h;
    uint32_t sel[2][4];
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int j = 0; j < 4; j++) sel[q][j] = mine && q == (gi >> 2) && (j >> 1) == (gi & 1) ? 0xffffffffu : 0u;
    const int nshift = 4 * (gi >> 2);

    // Weight offsets from J.W, 32-bit (the host keeps every matrix of this kernel below 2 GiB). Blocks are 2 mod 4 bytes
    // long, so a row's blocks alternate between two 2-byte misalignments: block b (of parity e = b & 1) starts mis[e]
    // bytes past the aligned dword at woff[e] + (b - e) * BB, and the dwords this lane reads sit at fixed distances from
    // it. Each holds at least one of the block's bytes, so none can fault (an aligned dword never crosses a page): the
    // block's first two aligned dwords (a block is at least 18 bytes), the aligned dword holding the code field's first
    // byte, and the next one unless that would pass the block's last aligned dword (then the field is 4-byte aligned and
    // the second dword is not used).
    const uint32_t rowoff = static_cast<uint32_t>(min(row0 + (n >> 3), J.r1 - 1)) * static_cast<uint32_t>(J.row_bytes);
    uint32_t mis[2], woff[2], qaoff[2], qboff[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const uint32_t start = rowoff + e * BB;   // block e of the row
        mis[e] = start & 2u;
        woff[e] = start - mis[e];
        const uint32_t f = mis[e] + Mb32Fmt<F>::QS + 4 * (Mb32Fmt<F>::BYTES ? gi : gq), fa = f & ~3u,
                       last = (mis[e] + BB - 1) & ~3u;
        qaoff[e] = woff[e] + fa;
        qboff[e] = woff[e] + (fa + 4 <= last ? fa + 4 : fa);
    }

    float acc[16];   // x86: acc[4 r + jj] = chain of group 4 h + jj of row r; scalar: acc[r] = the row's chain
#pragma unroll
    for (int j = 0; j < 16; j++) acc[j] = 0.0f;

    auto load = [&](Stage &s, int b, int e) {   // block b, of parity e
        const uint8_t *const wb = J.W + (size_t)(b - e) * BB;
        s.w0 = ldg<uint32_t>(wb + woff[e]);
        s.w1 = Mb32Fmt<F>::QH >= 0 ? ldg<uint32_t>(wb + woff[e] + 4) : 0u;
        s.qa = ldg<uint32_t>(wb + qaoff[e]);
        s.qb = ldg<uint32_t>(wb + qboff[e]);
        const uint8_t *const xb = J.xq + (size_t)b * 2048;
        s.y0 = ldg<v8h>(xb + 16 * lane);
        s.y1 = ldg<v8h>(xb + 1024 + 16 * lane);
        s.yd = ldg<float>(J.xm + (size_t)b * 128 + 4 * n);
    };
    // the block's two MFMAs and its d * yd for rows 0..3
    struct Issued { v16f d; float dy[4]; };
    auto issue = [&](const Stage &c, int e, Issued &o) {
        const uint32_t m = mis[e];
        const uint32_t qs = alignbyte(c.qb, c.qa, m ^ 2u);   // the code dword is misaligned exactly when the block is not
        uint32_t q;
        if constexpr (Mb32Fmt<F>::BYTES) q = qs ^ 0x80808080u;   // signed code + 128, per byte
        else q = (qs >> nshift) & 0x0f0f0f0fu;
        if constexpr (F == ES_HIP_Q5_0) {   // bit e of qh -> bit 4 of byte e; qh starts 2 bytes into the block
            const uint64_t hw = (static_cast<uint64_t>(c.w1) << 32 | c.w0) >> (16 + 8 * m + 4 * gi);
            q |= (((static_cast<uint32_t>(hw) & 15u) * 0x00204081u) & 0x01010101u) << 4;
        }
        // codes 0, 1 and 2, 3 as half pairs c - offset
        const h2 neg = __builtin_bit_cast(h2, Mb32Fmt<F>::NEG);
        const uint32_t v0 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, q, 0x04010400u)) + neg);
        const uint32_t v1 = __builtin_bit_cast(uint32_t, __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, q, 0x04030402u)) + neg);
        u32x4 a0, a1;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint32_t v = (j & 1) ? v1 : v0;
            a0[j] = v & sel[0][j];
            a1[j] = v & sel[1][j];
        }
        o.d = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a0), c.y0, v16f{}, 0, 0, 0);
        o.d = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, a1), c.y1, o.d, 0, 0, 0);
        // d of rows 0..3 (float), read from lanes 0, 8, 16, 24, which loaded them
        const float wd = half_bits_to_float(alignbyte(c.w0, c.w0, m));
#pragma unroll
        for (int r = 0; r < 4; r++)
            o.dy[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wd), 8 * r)) * c.yd;
    };
    auto chain = [&](const Issued &o) {
        if constexpr (X86) {
#pragma unroll
            for (int j = 0; j < 16; j++) acc[j] = __builtin_fmaf(o.d[j], o.dy[j >> 2], acc[j]);
        } else {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                // the block's integer sum, exact in float: this lane's four groups, then the other four
                float s4 = (o.d[4 * r] + o.d[4 * r + 1]) + (o.d[4 * r + 2] + o.d[4 * r + 3]);
                s4 += __shfl_xor(s4, 32);
                acc[r] = acc[r] + o.dy[r] * s4;
            }
        }
    };

    // Chunks of P blocks: block b0 + p is in st[p] (b0 is a multiple of P, so its parity is p's). Within a chunk block
    // p's MFMAs are issued before block p - 1's chains; the stage is refilled with block b0 + p + P right after its issue.
    Stage st[P];
    Issued io[2];
    // The first P loads are unconditional (stages past the last block load the last block again, unused): with a branch
    // around them the compiler's waits at the top of the main loop drained every load in flight (vmcnt(0)), exposing the
    // full memory latency once per chunk.
#pragma unroll
    for (int p = 0; p < P; p++) {
        const int b = min(p, nbk - 1);
        load(st[p], b, b & 1);
    }
    int b0 = 0;
    for (; b0 + 2 * P <= nbk; b0 += P) {   // every refill in range: no conditions
#pragma unroll
        for (int p = 0; p < P; p++) {
            issue(st[p], p & 1, io[p & 1]);
            load(st[p], b0 + p + P, p & 1);
            if (p > 0) chain(io[(p - 1) & 1]);
        }
        chain(io[(P - 1) & 1]);
    }
    for (; b0 < nbk; b0 += P) {   // the last one or two chunks
#pragma unroll
        for (int p = 0; p < P; p++) {
            if (b0 + p < nbk) {
                issue(st[p], p & 1, io[p & 1]);
                if (b0 + p + P < nbk) load(st[p], b0 + p + P, p & 1);
            }
            if (p > 0 && b0 + p - 1 < nbk) chain(io[(p - 1) & 1]);
        }
        if (b0 + P - 1 < nbk) chain(io[(P - 1) & 1]);
    }

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
    else if (type == ES_HIP_Q8_0) launch<ES_HIP_Q8_0>(x86, jobs, njobs, single, grid, s);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace esq
