// Batched 32-wide formats (Q4_0 / Q5_0 / Q8_0 against 2 or more activations) on the int8 matrix cores, reading the
// activations' Q8_0 rows directly (no pre-pass): config 5's attention projections at 32 tokens.
//
// The reference's AVX2 path forms, per 32-element block, eight integer lane sums lane_i = sum over elements 4i..4i+3 of
// (code - offset) * y and folds them into eight fused chains acc_i = fma((float)lane_i, d * yd, acc_i) in block order,
// summed at the end as ((0+4)+(2+6))+((1+5)+(3+7)) (src/es_quant.c:1185-1187, 1252-1323); its scalar path adds
// (d * yd) * (float)sum-of-all-32 to one chain (src/es_quant.c:1013-1055).
//
// Work split. A workgroup of 8 waves (two per SIMD) takes RW <= 32 rows x 32 activations, RW set per job by the host so
// that a launch's workgroups about fill the CUs once (config 5's q/k/v: 5120 rows in 246 workgroups of 21, instead of
// 320 of 16 on 256 CUs, which left 64 CUs with twice the work). The RW rows are cut into 8 contiguous runs of 1..4 rows,
// the longer runs to waves 0, 1, 2, ... so the two waves of a SIMD (w and w + 4) carry about RW / 4 rows between them.
// Every activation value and scale of the tile's whole row (at most NBKM blocks) is copied into LDS once, at the start;
// after one barrier each wave streams its rows' blocks from HBM into registers, P blocks ahead, with no further barrier.
// (The matrix-core kernel of es_hip_mb.hip read each block's activations from L2 in every wave: 2 KB of activation
// halves per block and wave against 88 bytes of weights.)
//
// One v_mfma_i32_32x32x32_i8 per block and wave produces every lane sum of its (up to) 4 rows x 32 activations: output
// row m = 8r + i is (weight row r, group i), and A row m holds only group i's four codes (code - offset, int8) at the
// four k positions where B (the activation's 32 int8 values) holds that group's values; every other A element is zero.
// So D[8r + i][n] is lane_i of row r against activation n, exactly, as an int32. Rows past the wave's run repeat its last
// row; their chains are not run and their outputs not stored.
//
// Operand layouts of v_mfma_i32_32x32x32_i8 (wave64): lane l supplies A row l % 32 and B column l % 32, both for the 16 k
// positions 16 (l / 32) .. + 15; D register j of lane l is element [8 (j / 4) + 4 (l / 32) + j % 4][l % 32]. So a lane
// owns the chains of one activation (l % 32) and four groups (4 (l / 32) .. + 3) of all four rows; lane (n, h) supplies
// group i = n % 8 of row n / 8 only when i / 4 == h (its codes in dword i % 4), and activation n's values 16h .. 16h + 15.
//
// LDS: values [b][32][32] (activation n's 16-byte chunk c at position c ^ ((n >> 3) & 1): the 16 lanes of each quarter
// wave read 16 different bank groups), scales [b][32]. Both go from the Q8_0 rows straight into LDS with
// global_load_lds_dwordx4 / _dword (one instruction per block for the values of all 32 activations).
//
// Weights: per block a lane reads the aligned dwords around its row's d (and Q5_0 high bits) and its group's code dword
// (blocks are 18, 22 or 34 bytes, so fields sit at 2-byte alignment; every dword read holds at least one of the block's
// bytes, so none crosses past the matrix).
#include <type_traits>

#include "es_hip_common.h"

namespace esq {
namespace {

typedef int v16i __attribute__((ext_vector_type(16)));

template <typename T> __device__ __forceinline__ T lds_ld(uint32_t a) {
    return *reinterpret_cast<const __attribute__((address_space(3))) T *>(a);
}

template <int F> struct BxFmt;
// Q4_0: d f16 @0, qs[16] @2, codes 0..15 - 8. Q5_0: d f16 @0, qh u32 @2, qs[16] @6, codes 0..31 - 16.
// Q8_0: d f16 @0, int8 qs[32] @2 (group i's codes are dword i). ADD (Q4_0, Q5_0): the per-byte bias that makes
// (c + ADD) ^ 0x80 the signed byte c - offset (no carry between bytes: c + ADD <= 255).
template <> struct BxFmt<ES_HIP_Q4_0> {
    static constexpr int QS = 2, QH = -1;
    static constexpr bool BYTES = false;
    static constexpr uint32_t ADD = 0x78787878u;
};
template <> struct BxFmt<ES_HIP_Q5_0> {
    static constexpr int QS = 6, QH = 2;
    static constexpr bool BYTES = false;
    static constexpr uint32_t ADD = 0x70707070u;
};
template <> struct BxFmt<ES_HIP_Q8_0> {
    static constexpr int QS = 2, QH = -1;
    static constexpr bool BYTES = true;
};

struct Stage {
    uint32_t w0, w1;   // the aligned dwords at and after the block's start: d (and Q5_0 qh)
    uint32_t qa, qb;   // the aligned dwords at and after this lane's code dword
};

// Tiles of 8 waves x J.rows_per_wg (<= MBX_ROWS) rows against MBX_TOK activations. P: blocks in flight per wave (even).
// X86: the AVX2 order (else the scalar one).
template <int F, int NBKM, int P, bool X86, bool GATHER>
__global__ __launch_bounds__(64 * MBX_WAVES, 1) void mbx_kernel(const MkJob *__restrict__ jobs, int njobs, MkJob single) {
    using BF = BxFmt<F>;
    constexpr int BB = Fmt<F>::BB;
    constexpr uint32_t V0 = 0, D0 = NBKM * 1024;
    static_assert(P % 2 == 0 && NBKM % 2 == 0, "block parity is the stage's; scale copies cover two blocks");
    __shared__ __align__(16) uint8_t smem[NBKM * (1024 + 128)];

    MkJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    // tiles as in the expert-sized kernel: with several activation tiles, all of a row tile's go to one XCD (id % 8)
    const int tile = blockIdx.x - J.tile0;
    int rt = tile, tt = 0;
    if (J.ntok_tiles > 1) {
        const int xcd = tile & 7, kq = tile >> 3;
        rt = xcd + 8 * (kq / J.ntok_tiles);
        tt = kq % J.ntok_tiles;
    }
    const int RW = J.rows_per_wg;
    if (rt * RW >= J.r1 - J.r0) return;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int n = lane & 31, h = lane >> 5;
    // this wave's run of rows: R (0..4) rows from row0, the longer runs to the first waves (waves w and w + 4 share a SIMD)
    const int rbase = RW / MBX_WAVES, rext = RW % MBX_WAVES;
    const int R = rbase + (wave < rext ? 1 : 0);
    const int row0 = J.r0 + rt * RW + wave * rbase + min(wave, rext), tok0 = tt * MBX_TOK;
    const int rlast = max(min(row0 + R, J.r1) - 1, J.r0);   // the run's last row (rows past it repeat it)
    const int nbk = J.cols / 32;
    const uint32_t smem0 = lds_addr(smem);

    // ---- staging: 32-bit offsets from J.act (the host keeps every activation row within 4 GiB of it)
    auto act_off = [&](int t) -> uint32_t {   // activation t of the tile (clamped to the last one)
        const int q = min(tok0 + t, J.na - 1);
        const int r = (GATHER && J.arow) ? ldg<int>(J.arow + q) : q;
        return (uint32_t)r * (uint32_t)J.astride;
    };
    auto blk_base = [&](int b) {   // block b's base, kept opaque in scalar registers
        uint32_t o = 36u * (uint32_t)b;
        asm volatile("" : "+s"(o));
        return J.act + o;
    };
    {
        // values: block b is one instruction of wave b % MBX_WAVES; lane l writes LDS slot l: activation l / 2, position
        // l % 2, source chunk (l % 2) ^ ((n >> 3) & 1)
        const int tv = lane >> 1;
        const uint32_t ov = act_off(tv) + 4 + 16 * ((lane & 1) ^ ((tv >> 3) & 1));
        for (int b = wave; b < nbk; b += MBX_WAVES) load_lds16(blk_base(b), ov, smem0 + V0 + (uint32_t)b * 1024);
        // scales: instruction q covers blocks 2q and 2q + 1 (lane l: block 2q + l / 32, activation l % 32; a block past
        // the last reads the last one again into a slot nobody reads)
        const uint32_t od0 = act_off(n);
        for (int q = wave; 2 * q < nbk; q += MBX_WAVES) {
            const int b = min(2 * q + h, nbk - 1);
            load_lds4(blk_base(2 * q), od0 + 36u * (uint32_t)(b - 2 * q), smem0 + D0 + (uint32_t)q * 256);
        }
    }

    // ---- this lane's weights: group gi = n % 8 of row row0 + n / 8 (rows past the run repeat its last; not stored)
    const int gi = n & 7, gq = gi & 3;
    const bool mine = (gi >> 2) == h;
    const int nshift = 4 * (gi >> 2);
    // 32-bit offsets from J.W (the host keeps every matrix of this kernel below 2 GiB). Blocks are 2 mod 4 bytes long, so
    // block b (of parity e = b & 1) starts mis[e] bytes past the aligned dword at woff[e] + (b - e) * BB; the dwords read
    // sit at fixed distances from it: the block's first two aligned dwords (a block is at least 18 bytes), the aligned
    // dword holding the code field's first byte, and the next one unless that would pass the block's last aligned dword
    // (then the field is 4-byte aligned and the second dword is not used).
    const uint32_t rowoff = static_cast<uint32_t>(min(row0 + (n >> 3), rlast)) * static_cast<uint32_t>(J.row_bytes);
    uint32_t mis[2], woff[2], qaoff[2], qboff[2];
#pragma unroll
    for (int e = 0; e < 2; e++) {
        const uint32_t start = rowoff + e * BB;
        mis[e] = start & 2u;
        woff[e] = start - mis[e];
        const uint32_t f = mis[e] + BF::QS + 4 * (BF::BYTES ? gi : gq), fa = f & ~3u, last = (mis[e] + BB - 1) & ~3u;
        qaoff[e] = woff[e] + fa;
        qboff[e] = woff[e] + (fa + 4 <= last ? fa + 4 : fa);
    }
    auto load = [&](Stage &s, int b) {   // block b (its parity from b itself)
        const int e = b & 1;
        const uint8_t *const wb = J.W + (size_t)(b - e) * BB;
        s.w0 = ldg<uint32_t>(wb + woff[e]);
        s.w1 = BF::QH >= 0 ? ldg<uint32_t>(wb + woff[e] + 4) : 0u;
        s.qa = ldg<uint32_t>(wb + qaoff[e]);
        s.qb = ldg<uint32_t>(wb + qboff[e]);
    };
    Stage st[P];
    // unconditional loads (a stage past the last block loads the last block again, unused): with no branch around a load
    // the compiler's waits count exactly which loads a use needs
#pragma unroll
    for (int p = 0; p < P; p++) load(st[p], min(p, nbk - 1));
    // Every staging copy must have landed before the barrier publishes the LDS. The wait drains the weight prefetch too:
    // counting only the weight loads would depend on how the compiler merges them (Q5_0's d|qh dwords become one
    // 8-byte load), and the first block needs its loads now anyway.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    lds_sync();
    if (R == 0) return;   // (a tile of fewer than 8 rows; no barrier follows)
    // the rest for a run of NR rows (a compile-time count: uniform branches per row inside the block loop kept the
    // compiler from overlapping one block's chains with the next block's matrix work)
    auto run = [&](auto nrc) {
        constexpr int NR = decltype(nrc)::value;

        const uint32_t xo = smem0 + V0 + (uint32_t)n * 32 + 16u * (uint32_t)(h ^ ((n >> 3) & 1)), yo = smem0 + D0 + 4u * n;
        float acc[16];   // x86: acc[4 r + jj] = chain of group 4 h + jj of row r; scalar: acc[r] = the row's chain
    #pragma unroll
        for (int j = 0; j < 16; j++) acc[j] = 0.0f;

        struct Issued { v16i d; float dy[4]; };
        auto issue = [&](const Stage &c, int b, Issued &o) {   // block b's MFMA and its d * yd for the run's rows
            const uint32_t m = mis[b & 1];
            const uint32_t qs = alignbyte(c.qb, c.qa, m ^ 2u);   // the code dword is misaligned exactly when the block is not
            uint32_t q;
            if constexpr (BF::BYTES) {
                q = qs;
            } else {
                q = (qs >> nshift) & 0x0f0f0f0fu;
                if constexpr (F == ES_HIP_Q5_0) {   // bit e of qh -> bit 4 of byte e; qh starts 2 bytes into the block
                    const uint64_t hw = (static_cast<uint64_t>(c.w1) << 32 | c.w0) >> (16 + 8 * m + 4 * gi);
                    q |= (((static_cast<uint32_t>(hw) & 15u) * 0x00204081u) & 0x01010101u) << 4;
                }
                q = (q + BF::ADD) ^ 0x80808080u;   // c - offset as signed bytes
            }
            q = mine ? q : 0u;
            const v4i a = v4i{gq == 0 ? (int)q : 0, gq == 1 ? (int)q : 0, gq == 2 ? (int)q : 0, gq == 3 ? (int)q : 0};
            const v4i x = lds_ld<v4i>(xo + (uint32_t)b * 1024);
            o.d = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, x, v16i{}, 0, 0, 0);
            const float yd = lds_ld<float>(yo + (uint32_t)b * 128);
            // d of rows 0..NR-1 (float), read from lanes 0, 8, 16, 24, which loaded them
            const float wd = half_bits_to_float(alignbyte(c.w0, c.w0, m));
    #pragma unroll
            for (int r = 0; r < 4; r++)
                if (r < NR) o.dy[r] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wd), 8 * r)) * yd;
        };
        auto chain = [&](const Issued &o) {   // the chains of the run's rows (R is wave-uniform)
            if constexpr (X86) {
    #pragma unroll
                for (int r = 0; r < 4; r++)
                    if (r < NR) {
    #pragma unroll
                        for (int jj = 0; jj < 4; jj++)
                            acc[4 * r + jj] = __builtin_fmaf(static_cast<float>(o.d[4 * r + jj]), o.dy[r], acc[4 * r + jj]);
                    }
            } else {
    #pragma unroll
                for (int r = 0; r < 4; r++)
                    if (r < NR) {
                        // the block's integer sum: this lane's four groups, then the other four
                        int s4 = (o.d[4 * r] + o.d[4 * r + 1]) + (o.d[4 * r + 2] + o.d[4 * r + 3]);
                        s4 += __shfl_xor(s4, 32);
                        acc[r] = acc[r] + o.dy[r] * static_cast<float>(s4);
                    }
            }
        };

        // Chunks of P blocks: block b0 + p is in st[p] (b0 is a multiple of P) and its results in io[p & 1]. Block b's MFMA is
        // issued before block b - 1's chains, and the last block's chains follow its own issue; the stage is refilled with
        // block b + P (or the last block again) right after. Every index is a compile-time constant (a runtime index would put
        // io in scratch memory).
        Issued io[2];
        for (int b0 = 0; b0 < nbk; b0 += P) {
    #pragma unroll
            for (int p = 0; p < P; p++) {
                const int b = b0 + p;
                if (b < nbk) {
                    issue(st[p], b, io[p & 1]);
                    if (b > 0) chain(io[(p + 1) & 1]);
                    if (b == nbk - 1) chain(io[p & 1]);
                }
                load(st[p], min(b + P, nbk - 1));
            }
        }

        const int t = tok0 + n;
        const bool tok_ok = t < J.na;
    #pragma unroll
        for (int r = 0; r < 4; r++) {
            if (r >= NR) break;
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
    };
    switch (R) {
    case 1: run(std::integral_constant<int, 1>{}); break;
    case 2: run(std::integral_constant<int, 2>{}); break;
    case 3: run(std::integral_constant<int, 3>{}); break;
    default: run(std::integral_constant<int, 4>{}); break;
    }
}

template <int F, int NBKM>
void launch_nbk(bool x86, bool gather, const MkJob *jobs, int njobs, const MkJob &single, int grid, hipStream_t s) {
    constexpr int P = 8;
    const dim3 g(grid), b(64 * MBX_WAVES);
    if (x86) {
        if (gather) hipLaunchKernelGGL((mbx_kernel<F, NBKM, P, true, true>), g, b, 0, s, jobs, njobs, single);
        else hipLaunchKernelGGL((mbx_kernel<F, NBKM, P, true, false>), g, b, 0, s, jobs, njobs, single);
    } else {
        if (gather) hipLaunchKernelGGL((mbx_kernel<F, NBKM, P, false, true>), g, b, 0, s, jobs, njobs, single);
        else hipLaunchKernelGGL((mbx_kernel<F, NBKM, P, false, false>), g, b, 0, s, jobs, njobs, single);
    }
}

template <int F>
hipError_t launch_fmt(int nbkm, bool x86, bool gather, const MkJob *jobs, int njobs, const MkJob &single, int grid,
                      hipStream_t s) {
    switch (nbkm) {
    case 32: launch_nbk<F, 32>(x86, gather, jobs, njobs, single, grid, s); break;
    case 64: launch_nbk<F, 64>(x86, gather, jobs, njobs, single, grid, s); break;
    case MBX_NBK: launch_nbk<F, MBX_NBK>(x86, gather, jobs, njobs, single, grid, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipSuccess;
}

}  // namespace

int mbx_nbk_max(int nbk) { return nbk <= 32 ? 32 : nbk <= 64 ? 64 : nbk <= MBX_NBK ? MBX_NBK : 0; }

hipError_t mbx_launch(int type, bool gather, int nbk_max, const MkJob *jobs, int njobs, const MkJob &single, int grid,
                      int order, hipStream_t s) {
    const bool x86 = order != ES_HIP_ORDER_SCALAR;
    const int nbkm = mbx_nbk_max(nbk_max);
    hipError_t e;
    if (type == ES_HIP_Q4_0) e = launch_fmt<ES_HIP_Q4_0>(nbkm, x86, gather, jobs, njobs, single, grid, s);
    else if (type == ES_HIP_Q5_0) e = launch_fmt<ES_HIP_Q5_0>(nbkm, x86, gather, jobs, njobs, single, grid, s);
    else if (type == ES_HIP_Q8_0) e = launch_fmt<ES_HIP_Q8_0>(nbkm, x86, gather, jobs, njobs, single, grid, s);
    else return hipErrorInvalidValue;
    return e != hipSuccess ? e : hipGetLastError();
}

}  // namespace esq
