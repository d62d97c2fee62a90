// Batched Q4_K products (and Q5_K, Q3_K: below) on the int8 matrix cores that read the activations' Q8_K rows directly
// (no pre-pass): the prompt-reading form of es_matvec_multi (src/es_quant.c:1818-1850, 1564-1602) for Q4_K.
//
// Work split. A workgroup of 4 waves computes MK_ROWS = 64 rows x MK_TOK = 128 activations; wave w takes the 16 rows
// 16w .. 16w+15 and all 128 activations (eight 16-activation tiles), so a row tile's unpacked weights serve eight MFMA
// tiles. Two workgroups share a CU (one wave of each per SIMD), each with its own LDS ring and barriers, so one
// workgroup's vector work (unpacking weights, the float epilogue) overlaps the other's matrix work. The code is written
// for MK_WAVES = MK_ROWS / 16 waves: a build with MK_ROWS = 128 runs one workgroup of 8 waves per CU (the same results;
// measured no faster for Q4_K and slower for Q5_K and Q3_K, whose short products then get half the tiles).
//
// Activations. Superblock b of the 128 activations passes through a two-slot LDS ring: the Q8_K values (each activation's
// 256 bytes in one LDS row, its 16-byte chunk c at position c ^ (t & 15), so the 16 lanes that read chunk c of 16
// activations hit 16 different bank groups), the 16 bsums as halves (exact: |bsums| <= 16 * 127) grouped by MFMA k-group,
// and the scales d. Values and scales go from the Q8_K rows straight into LDS: global_load_lds_dwordx4 writes lane l's 16
// bytes to LDS position 16*l of the instruction's 1 KB, from any source address, so the swizzle is in the per-lane source
// offsets (4-byte aligned chunks: the device honours any dword alignment of the source), four activations per instruction.
// The bsums pass through registers for their conversion to halves.
//
// Pipeline. One group of loads per superblock, issued early in superblock b's matrix work: superblock b + 1's values and
// scales into the free LDS slot, its weights and bsums into registers (unpacked after the next barrier, written at the end
// of the iteration). Their waits come most of an iteration later and find them arrived (a wait on loads issued just
// before it cost more than half the kernel's time in earlier forms of this loop).
//
// Weights. Each wave unpacks its rows' superblock into the B operands: the nibble q of sub-block j times its 6-bit scale
// sc_j does not fit int8, so sc = 8*sh + sl and two int8 planes go through the matrix cores, q*sl and q*sh (both <= 105):
// dot = D_lo + 8*D_hi, exact in int32. The mins term sum_j mn_j * (bsums[2j] + bsums[2j+1]) goes through one
// v_mfma_f32_16x16x16_f16 over the 16 bsums: mn <= 63 and the bsums are exact halves, every product and partial sum is an
// integer below 2^24, so the f32 result is the exact integer.
//
// MFMA operands: A = activations (16 activations x 64 k), B = weights (64 k x 16 rows), so D[activation][row] sits in
// lane l, register i as activation 4*(l/16)+i of the tile and row l%16 — the row whose weights the lane unpacked: d and
// dmin need no cross-lane moves. K order inside a superblock: slice s (0..3), lane group lg takes the 16 nibbles of qs
// chunk lg + 4*(s>>1) (low nibbles for even s, high for odd s), i.e. sub-block j = 2*(lg>>1) + 4*(s>>1) + (s&1),
// elements 32j + 16*(lg&1) + [0, 16); the activation side reads the same elements, natural 16-element chunk
// 4*(lg>>1) + 8*(s>>1) + 2*(s&1) + (lg&1).
//
// Epilogue per (row, activation) and superblock, in superblock order: s += y.d * (d*dot - dmin*mins) in the selected
// reference order (src/es_quant.c:1056-1080, 1324-1343, 1564-1602), so the outputs are bit-identical to the CPU kernels.
// MFMA lane layouts (A: lane l holds row l%16, k 16*(l/16)..+15 for the i8 form and k 4*(l/16)..+3 for the f16 form;
// D: lane l, register i holds D[4*(l/16)+i][l%16]) are those of the device, checked by the parity tests.
//
// Q5_K (src/es_quant.c:1153-1175): Q4_K's layout plus qh[32] after the scales, bit 2c (2c + 1) of qh[l] the fifth bit of
// element l of sub-block 2c (2c + 1), so q = q4 + 16 q5. A third int8 plane q5 * sc (<= 63) goes through the matrix cores
// and dot = D_lo + 8 D_hi + 16 D_q5, exact. Its epilogue is the reference's scalar mv_q5_K (the x86 build has no AVX2
// Q5_K kernel and no FMA in it): s += y.d * (d * dot - dmin * mins) with every product and sum rounded, in every order.
//
// Q3_K (src/es_quant.c:1120-1150, 1369-1395): 110-byte superblocks hmask[32] | qs[64] | scales[12] | d, 2-byte aligned,
// read with unaligned 16-byte loads (the header as bytes 94..109: qs[62..63], the scales and d, so no load passes the
// superblock's end). Group g = 8n + 2j + half holds the 16 elements v = ((qs[32n + 16 half + l] >> 2j) & 3) - 4 (plus 4
// when bit 4n + j of hmask[16 half + l] is set), v in -4..3, with the scale sc_g = code_g - 32 in -32..31. Split
// code = 8 h + l (h, l in 0..7): sc = l + 8 (h - 4), and v * l (-28..21) and v * (h - 4) (-12..16) both fit int8, so
// tot = sum_g sc_g * sum v y = D_lo + 8 D_hi with no bsums term (the reference sums the codes against the values too).
// Slice s and lane group lg take group g = 8 (lg >> 1) + 2 s + (lg & 1); the planes' bytes come from two 8-entry tables
// per slice (v * l and v * (h - 4) for v + 4 = 0..7) through v_perm_b32, indexed by the 3-bit code v + 4. Epilogue: the
// reference's s += y.d * d * tot (fused in the clang order).
#include "es_hip_common.h"

namespace esq {
namespace {

// LDS loads from a 32-bit LDS address (constant offsets fold into the instruction)
template <typename T> __device__ __forceinline__ T lds_ld(uint32_t a) {
    return *reinterpret_cast<const __attribute__((address_space(3))) T *>(a);
}

// LDS DMA (global_load_lds_dwordx4 / _dword): lane l's 16 (4) bytes at base + off land at LDS address lds + 16*l
// (4*l). Issued from inline assembly: given the builtin, the compiler would wait for these loads before every LDS read
// that might alias them (all of them: both ring slots are one array). The kernel orders them itself: s_waitcnt vmcnt(0)
// and a barrier before a slot is read, the slot having been free since the barrier before the copies. M0 is set inside
// the statement; nothing else in this kernel uses M0. The compiler's own vmcnt waits stay correct (conservative): these
// copies only add to the count it expects.
__device__ __forceinline__ void load_lds16(const uint8_t *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory");
}
__device__ __forceinline__ void load_lds4(const uint8_t *base, uint32_t off, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1" ::"v"(off), "s"(base), "s"(lds) : "memory");
}

constexpr int MK_WAVES = MK_ROWS / 16;
static_assert(MK_WAVES == 4 || MK_WAVES == 8, "four or eight waves of 16 rows");
// workgroups per CU: two of four waves (each with its own LDS ring and barriers), or one of eight
constexpr int MK_WG_PER_CU = MK_WAVES == 4 ? 2 : 1;
// one slot of the activation ring for T activations: values (one swizzled 256-byte row per activation) | bsums as halves
// [lg][activation][4] | scales
constexpr int TROW = 256;
template <int T> struct MkSlot {
    static constexpr int QS = 0, BS = T * TROW, D = BS + T * 32, BYTES = D + T * 4, TT = T / 16;
    static_assert(T == 64 || T == 128, "the staging assignment below is written for 64 or 128 activations");
    static_assert(2 * 2 * BYTES <= 160 * 1024, "two workgroups' two slots fit the LDS");
};

typedef _Float16 v4h __attribute__((ext_vector_type(4)));

template <int F> struct MkFmt;
template <> struct MkFmt<ES_HIP_Q4_K> { static constexpr int BB = 144, QS = 16, QH = -1; };
template <> struct MkFmt<ES_HIP_Q5_K> { static constexpr int BB = 176, QS = 48, QH = 16; };
template <> struct MkFmt<ES_HIP_Q3_K> { static constexpr int BB = 110, QS = 32, QH = 0; };

template <int F> struct WRaw {   // this lane's fields of one row tile's superblock: header, qs chunks lg and lg + 4
    uint4 h, q0, q1;
};
template <> struct WRaw<ES_HIP_Q5_K> {   // ... and the qh bytes of its elements, 16 (lg & 1) .. + 15
    uint4 h, q0, q1, qh;
};
template <> struct WRaw<ES_HIP_Q3_K> {   // bytes 94..109 (qs[62..63] | scales | d), qs chunk lg, hmask chunk lg & 1
    uint4 h, q, hm;
};

template <int F> struct BOps {   // one row tile's B operands for one superblock
    v4i lo[4], hi[4];
    v4h mn;
    float d, dm;
};
template <> struct BOps<ES_HIP_Q5_K> {
    v4i lo[4], hi[4], q5[4];
    v4h mn;
    float d, dm;
};
template <> struct BOps<ES_HIP_Q3_K> {   // dm unused (0)
    v4i lo[4], hi[4];
    float d, dm;
};

// scale_min_k4 (src/es_quant.c:75-83) byte-parallel: the two int8 planes of the four slices (three for Q5_K) and the
// mins operand
template <int F> __device__ __forceinline__ void build_b(const WRaw<F> &w, int lg, BOps<F> &B) {
    const uint4 h = w.h;
    const uint32_t sc0 = h.y & 0x3f3f3f3fu, sc1 = (h.w & 0x0f0f0f0fu) | ((h.y >> 2) & 0x30303030u);
    const uint32_t mn0 = h.z & 0x3f3f3f3fu, mn1 = ((h.w >> 4) & 0x0f0f0f0fu) | ((h.z >> 2) & 0x30303030u);
    // v_perm_b32 selectors putting byte 2*(lg >> 1) (sel0) or 2*(lg >> 1) + 1 (sel1) into both 16-bit halves
    const uint32_t sel0 = 0x0c000c00u + (uint32_t)(2 * (lg >> 1)) * 0x00010001u, sel1 = sel0 + 0x00010001u;
    const uint32_t l0 = sc0 & 0x07070707u, h0 = (sc0 >> 3) & 0x07070707u;
    const uint32_t l1 = sc1 & 0x07070707u, h1 = (sc1 >> 3) & 0x07070707u;
    const uint32_t slw[4] = {__builtin_amdgcn_perm(0, l0, sel0), __builtin_amdgcn_perm(0, l0, sel1),
                             __builtin_amdgcn_perm(0, l1, sel0), __builtin_amdgcn_perm(0, l1, sel1)};
    const uint32_t shw[4] = {__builtin_amdgcn_perm(0, h0, sel0), __builtin_amdgcn_perm(0, h0, sel1),
                             __builtin_amdgcn_perm(0, h1, sel0), __builtin_amdgcn_perm(0, h1, sel1)};
    const uint32_t qa[2][4] = {{w.q0.x, w.q0.y, w.q0.z, w.q0.w}, {w.q1.x, w.q1.y, w.q1.z, w.q1.w}};
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t v = qa[s >> 1][i];
            const uint32_t nib = (s & 1) ? (v >> 4) & 0x0f0f0f0fu : v & 0x0f0f0f0fu;
            B.lo[s][i] = (int)pk_mul_u16(nib, slw[s]);   // byte * scale <= 105: no carry between bytes
            B.hi[s][i] = (int)pk_mul_u16(nib, shw[s]);
        }
    if constexpr (F == ES_HIP_Q5_K) {   // slice s takes sub-block j = 2 (lg >> 1) + 4 (s >> 1) + (s & 1): bit j of its qh bytes
        const uint32_t scw[4] = {__builtin_amdgcn_perm(0, sc0, sel0), __builtin_amdgcn_perm(0, sc0, sel1),
                                 __builtin_amdgcn_perm(0, sc1, sel0), __builtin_amdgcn_perm(0, sc1, sel1)};
        const uint32_t hw[4] = {w.qh.x, w.qh.y, w.qh.z, w.qh.w};
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t j = 2 * (lg >> 1) + 4 * (s >> 1) + (s & 1);
#pragma unroll
            for (int i = 0; i < 4; i++) B.q5[s][i] = (int)pk_mul_u16((hw[i] >> j) & 0x01010101u, scw[s]);   // <= 63
        }
    }
    // mins operand: k positions 4lg .. 4lg+3 meet bsums 4lg .. 4lg+3, i.e. sub-blocks 2lg and 2lg+1, each twice. Each half
    // is built as 1024 + m (byte m under the exponent of 1024) and 1024 subtracted exactly.
    const uint32_t mw = lg < 2 ? mn0 : mn1, kb = 2u * (uint32_t)(lg & 1);
    const h2 m1024 = __builtin_bit_cast(h2, 0xe400e400u);
    const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, mw, 0x04000400u + kb * 0x00010001u)) + m1024;
    const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, mw, 0x04000400u + (kb + 1) * 0x00010001u)) + m1024;
    B.mn = v4h{a[0], a[1], b[0], b[1]};
    B.d = half_bits_to_float(h.x);
    B.dm = half_bits_to_float(h.x >> 16);
}

// Q3_K: the two planes of every slice from the 3-bit codes c = v + 4 and per-slice tables (see the file comment)
template <> __device__ __forceinline__ void build_b<ES_HIP_Q3_K>(const WRaw<ES_HIP_Q3_K> &w, int lg, BOps<ES_HIP_Q3_K> &B) {
    const uint4 h = w.h;
    const uint32_t n4 = 4u * (uint32_t)(lg >> 1), half8 = 8u * (uint32_t)(lg & 1);
    // scale bytes 0-3, 4-7, 8-11 (bytes 2.. of the header load)
    const uint32_t S0 = __builtin_amdgcn_alignbyte(h.y, h.x, 2), S1 = __builtin_amdgcn_alignbyte(h.z, h.y, 2),
                   S2 = __builtin_amdgcn_alignbyte(h.w, h.z, 2);
    // 6-bit codes of groups 8n + 4p + i, byte i of C[p]: nibble n of scales[4p + i], bits 4n + 2p of scales[8 + i]
    // (src/es_quant.c:1125-1128); then the lane's two groups of each, bytes lg & 1 and 2 + (lg & 1), shifted down
    const uint32_t hs = S2 >> n4;
    const uint32_t C0 = (((S0 >> n4) & 0x0f0f0f0fu) | ((hs << 4) & 0x30303030u)) >> half8;
    const uint32_t C1 = (((S1 >> n4) & 0x0f0f0f0fu) | ((hs << 2) & 0x30303030u)) >> half8;
    const uint32_t hd[4] = {w.hm.x >> n4, w.hm.y >> n4, w.hm.z >> n4, w.hm.w >> n4};   // bit j of byte l: group 8n + 2j + half
    const uint32_t qd[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int s = 0; s < 4; s++) {
        // slice s: group 8n + 2s + half, code byte 2 (s & 1) of C[s >> 1]: l = bits 0-2, h = bits 3-5
        const uint32_t C = s < 2 ? C0 : C1, sh = 16u * (uint32_t)(s & 1);
        const uint32_t cl = (C >> sh) & 7u, ch = (C >> (sh + 3)) & 7u;
        // tables: byte c of (T1:T0) = (c - 4) * l, of (U1:U0) = (c - 4) * (h - 4); bytes are formed biased by 0x80 (every
        // partial result stays in 0..255, no borrow between bytes) and the bias flipped back
        const uint32_t T1 = cl * 0x03020100u, T0 = (0x80808080u - cl * 0x01020304u) ^ 0x80808080u;
        const uint32_t U1 = (ch * 0x03020100u + 0x74787c80u) ^ 0x80808080u, U0 = (0x84888c90u - ch * 0x01020304u) ^ 0x80808080u;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t hb = s <= 2 ? hd[i] << (2 - s) : hd[i] >> 1;   // the high bit to bit 2 of each byte
            const uint32_t c = ((qd[i] >> (2 * s)) & 0x03030303u) | (hb & 0x04040404u);
            B.lo[s][i] = (int)__builtin_amdgcn_perm(T1, T0, c);
            B.hi[s][i] = (int)__builtin_amdgcn_perm(U1, U0, c);
        }
    }
    B.d = half_bits_to_float(h.w >> 16);
    B.dm = 0.f;
}

struct AOps {   // one activation tile's A operands for one superblock, and the tile's activation scales
    v4i x[4];
    v4h bs;
    v4f yd;     // y.d of activations 4*lg .. 4*lg+3 of the tile
};

template <int F> struct MAcc {   // the matrix-core results of one 16 x 16 tile and superblock
    v4i lo, hi;
    v4f mn;
};
template <> struct MAcc<ES_HIP_Q5_K> {
    v4i lo, hi, q5;
    v4f mn;
};
template <> struct MAcc<ES_HIP_Q3_K> {
    v4i lo, hi;
};

template <int F> struct Pend {   // a tile's results waiting for their epilogue, with the scales of their superblock
    MAcc<F> m;
    v4f yd;
    float d, dm;
};

template <int F> __device__ __forceinline__ void mma(const AOps &a, const BOps<F> &B, MAcc<F> &m) {
    m.lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.x[0], B.lo[0], v4i{0, 0, 0, 0}, 0, 0, 0);
    m.hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.x[0], B.hi[0], v4i{0, 0, 0, 0}, 0, 0, 0);
    if constexpr (F == ES_HIP_Q5_K) m.q5 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.x[0], B.q5[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int s = 1; s < 4; s++) {
        m.lo = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.x[s], B.lo[s], m.lo, 0, 0, 0);
        m.hi = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.x[s], B.hi[s], m.hi, 0, 0, 0);
        if constexpr (F == ES_HIP_Q5_K) m.q5 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.x[s], B.q5[s], m.q5, 0, 0, 0);
    }
    if constexpr (F != ES_HIP_Q3_K) m.mn = __builtin_amdgcn_mfma_f32_16x16x16f16(a.bs, B.mn, v4f{0, 0, 0, 0}, 0, 0, 0);
}

template <int F, bool CONTRACT>
__device__ __forceinline__ void epilogue(const MAcc<F> &m, float d, float dm, const v4f &yd, v4f &s) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        int dot = m.lo[i] + 8 * m.hi[i];
        if constexpr (F == ES_HIP_Q3_K) {   // s += (y.d * d) * tot
            const float a = yd[i] * d;
            if constexpr (CONTRACT) s[i] = __builtin_fmaf(a, static_cast<float>(dot), s[i]);
            else s[i] = s[i] + a * static_cast<float>(dot);
        } else {
            if constexpr (F == ES_HIP_Q5_K) dot += 16 * m.q5[i];
            const float q = dm * m.mn[i];   // the mins are exact integers in the f32 accumulator
            if constexpr (CONTRACT)
                s[i] = __builtin_fmaf(yd[i], __builtin_fmaf(d, static_cast<float>(dot), -q), s[i]);
            else
                s[i] = s[i] + yd[i] * (d * static_cast<float>(dot) - q);
        }
    }
}

// One tile step: 9 MFMAs (13 for Q5_K, 8 for Q3_K) interleaved with the step's vector work (the previous tile's epilogue) and the
// next tile's LDS reads: 1 MFMA : 3 VALU : 1 LDS read.
template <int NMFMA> __device__ __forceinline__ void step_schedule() {
#pragma unroll
    for (int k = 0; k < NMFMA; k++) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);   // VALU
        if (k < 6) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);   // LDS read
    }
}

// T: activations per workgroup tile, 128, or 64 for products with too few row tiles to fill the device at 128.
template <int F, bool CONTRACT, bool GATHER, int T>
__global__ __launch_bounds__(64 * MK_WAVES, MK_WG_PER_CU) void mk_kernel(const MkJob *__restrict__ jobs, int njobs, MkJob single) {
    using FM = MkFmt<F>;
    using SL = MkSlot<T>;
    constexpr int ST_QS = SL::QS, ST_BS = SL::BS, ST_D = SL::D, ST_BYTES = SL::BYTES, MK_TT = SL::TT;
    constexpr bool FUSED = CONTRACT && F != ES_HIP_Q5_K;   // Q5_K's reference epilogue never fuses
    constexpr bool BSUMS = F != ES_HIP_Q3_K;              // the mins term reads the activations' bsums
    __shared__ __align__(16) uint8_t smem[2 * ST_BYTES];

    MkJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    // XCD-aware tile order: workgroup ids go round-robin over the 8 XCDs (id % 8); all activation tiles of row tile rt go to
    // ids with id % 8 == rt % 8, so a row tile's weights are read into one XCD's L2. Each job's tiles start at a multiple
    // of 8; ids past the last row tile exit at once.
    const int tile = blockIdx.x - J.tile0;
    const int xcd = tile & 7, kq = tile >> 3;
    const int rt_ = xcd + 8 * (kq / J.ntok_tiles), tt_ = kq % J.ntok_tiles;
    if (rt_ * MK_ROWS >= J.r1 - J.r0) return;
    const int row0 = J.r0 + rt_ * MK_ROWS, tok0 = tt_ * T;
    const int nbk = J.cols / 256;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;

    // ---- staging sources (32-bit offsets from J.act; the host keeps every activation row within 4 GiB of it)
    auto act_off = [&](int t) -> uint32_t {   // activation t of the tile (clamped to the last one)
        const int q = min(tok0 + t, J.na - 1);
        const int r = (GATHER && J.arow) ? ldg<int>(J.arow + q) : q;
        return (uint32_t)r * (uint32_t)J.astride;
    };
    // values: wave w of NW copies activations TW w .. TW w + TW - 1 (TW = T / NW), four per instruction: instruction k,
    // lane l: activation t = TW w + 4k + l/16, LDS position l%16 of its row, so source chunk (l%16) ^ (t & 15)
    constexpr int TW = T / MK_WAVES, NV = TW / 4;
    uint32_t qoff[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int t = TW * wave + 4 * k + (lane >> 4);
        qoff[k] = act_off(t) + 4 + 16 * ((lane & 15) ^ (t & 15));
    }
    // scales: wave w, lane l copies activation 64 ds + l's d, ds = w & 1 (at 128 activations; 0 at 64)
    const int ds = T == 128 ? (wave & 1) : 0;
    const uint32_t doff = act_off(64 * ds + lane);
    // bsums: every lane, activation bt, bsums 8*bh .. 8*bh+7 (at 64 activations the upper half of the workgroup repeats the
    // lower half's copies: the same bytes to the same place)
    const int bt = (tid >> 1) & (T - 1), bh = tid & 1;
    const uint32_t boff = act_off(bt) + 260 + 16 * bh;
    const uint32_t bdst0 = ST_BS + (2 * bh) * (T * 8) + bt * 8, bdst1 = bdst0 + T * 8;
    const uint32_t smem0 = lds_addr(smem);

    // the superblock's base address, kept opaque in scalar registers (as plain arithmetic the compiler folds it into
    // per-lane 64-bit pointers)
    auto sb_base = [&](int b) {
        uint32_t sb = 292u * (uint32_t)b;
        asm volatile("" : "+s"(sb));
        return J.act + sb;
    };
    auto stage_dma = [&](int b, int st) {   // values and scales of superblock b into slot st
        const uint8_t *ab = sb_base(b);
        const uint32_t base = smem0 + (uint32_t)st * ST_BYTES + ST_QS + (uint32_t)(TW * wave) * TROW;
#pragma unroll
        for (int k = 0; k < NV; k++) load_lds16(ab, qoff[k], base + 4 * TROW * k);
        // the other waves repeat waves 0 and 1's copy (the same bytes to the same place), which keeps the code branch-free
        load_lds4(ab, doff, smem0 + (uint32_t)st * ST_BYTES + ST_D + 256 * ds);
    };
    auto bs_load = [&](int b) { return ldg<uint4>(sb_base(b) + boff); };
    auto bs_write = [&](const uint4 &v, int st) {
        uint8_t *base = smem + st * ST_BYTES;
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t hv[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {   // two int16 bsums -> two halves (exact)
            const _Float16 e0 = (_Float16)(int16_t)(w[k] & 0xffffu), e1 = (_Float16)(int16_t)(w[k] >> 16);
            hv[k] = (uint32_t)__builtin_bit_cast(uint16_t, e0) | (uint32_t)__builtin_bit_cast(uint16_t, e1) << 16;
        }
        *reinterpret_cast<uint2 *>(base + bdst0) = make_uint2(hv[0], hv[1]);
        *reinterpret_cast<uint2 *>(base + bdst1) = make_uint2(hv[2], hv[3]);
    };
    // ---- this wave's weight rows (rows past the end repeat the last one; their results are not stored)
    const uint8_t *wbase = J.W + (size_t)row0 * J.row_bytes;
    const uint32_t woff = (uint32_t)min(16 * wave + lr, J.r1 - 1 - row0) * (uint32_t)J.row_bytes;
    auto wload = [&](int b, WRaw<F> &W) {
        const uint8_t *p = wbase + woff + (uint32_t)FM::BB * (uint32_t)b;
        if constexpr (F == ES_HIP_Q3_K) {
            W.h = ldg_u128_a2(p + 94);
            W.q = ldg_u128_a2(p + FM::QS + 16 * lg);
            W.hm = ldg_u128_a2(p + FM::QH + 16 * (lg & 1));
        } else {
            W.h = ldg<uint4>(p);
            W.q0 = ldg<uint4>(p + FM::QS + 16 * lg);
            W.q1 = ldg<uint4>(p + FM::QS + 64 + 16 * lg);
            if constexpr (F == ES_HIP_Q5_K) W.qh = ldg<uint4>(p + FM::QH + 16 * (lg & 1));
        }
    };

    // ---- A operand offsets in a slot: activation tile tt adds 16 rows (values), 16 * 8 (bsums), 64 (scales)
    uint32_t xo[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int nat = F == ES_HIP_Q3_K ? 8 * (lg >> 1) + 2 * s + (lg & 1) : 4 * (lg >> 1) + 8 * (s >> 1) + 2 * (s & 1) + (lg & 1);
        xo[s] = ST_QS + lr * TROW + 16 * (nat ^ lr);   // rows 16 tt + lr: the swizzle key is lr
    }
    const uint32_t bso = ST_BS + lg * (T * 8) + lr * 8, ydo = ST_D + 16 * lg;
    // read addresses: per superblock, the slot's base is added once to these six, and an activation tile's reads differ
    // only in their immediate offsets
    auto aload = [&](const uint32_t (&xa)[4], uint32_t ba, uint32_t ya, int tt, AOps &A) {
#pragma unroll
        for (int s = 0; s < 4; s++) A.x[s] = lds_ld<v4i>(xa[s] + 16 * TROW * tt);
        if constexpr (BSUMS) A.bs = lds_ld<v4h>(ba + 128 * tt);
        A.yd = lds_ld<v4f>(ya + 64 * tt);
    };

    v4f acc[MK_TT];   // the outputs of activation tile tt
#pragma unroll
    for (int tt = 0; tt < MK_TT; tt++) acc[tt] = v4f{0, 0, 0, 0};

    // Per superblock b: wait for every load of the previous group and the barrier (slot b & 1 complete, the other slot
    // free); the B operands of superblock b from its weights; the matrix work over the 8 activation tiles, with the next
    // load group (values and scales of superblock b + 1 into the free slot, its weights and bsums into registers) issued
    // after the second tile; the bsums of superblock b + 1 into LDS. The last iteration repeats the last superblock's
    // loads into a slot nobody reads.
    //
    // A tile's epilogue runs two tile steps after its MFMAs (a step's vector work then never waits for the matrix cores),
    // across superblock boundaries: steps 0 and 1 of superblock b finish tiles 6 and 7 of superblock b - 1. The two
    // pending slots start as zeros (all scales 0), whose epilogues add +0 to the +0 of acc[6] and acc[7]: the same bits.
    Pend<F> p0, p1;   // the tiles two and one steps back
    p0.m = MAcc<F>{};
    p0.yd = v4f{0, 0, 0, 0};
    p0.d = p0.dm = 0.f;
    p1 = p0;
    WRaw<F> W;
    stage_dma(0, 0);
    wload(0, W);
    if constexpr (BSUMS) bs_write(bs_load(0), 0);
    for (int b = 0; b < nbk; b++) {
        const int sl = b & 1;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // this wave's copies into LDS (not tracked by the compiler)
        __syncthreads();
        BOps<F> B;
        build_b<F>(W, lg, B);
        const int bn = min(b + 1, nbk - 1);
        uint4 bsn;
        const uint32_t so = smem0 + (uint32_t)sl * ST_BYTES;
        const uint32_t xa[4] = {so + xo[0], so + xo[1], so + xo[2], so + xo[3]}, ba = so + bso, ya = so + ydo;
        AOps A[2];
        aload(xa, ba, ya, 0, A[0]);
#pragma unroll
        for (int tt = 0; tt < MK_TT; tt++) {
            if (tt + 1 < MK_TT) aload(xa, ba, ya, tt + 1, A[(tt + 1) & 1]);
            MAcc<F> cur;
            mma<F>(A[tt & 1], B, cur);
            epilogue<F, FUSED>(p0.m, p0.d, p0.dm, p0.yd, acc[(tt + MK_TT - 2) % MK_TT]);
            p0 = p1;
            p1.m = cur;
            p1.yd = A[tt & 1].yd;
            p1.d = B.d;
            p1.dm = B.dm;
            step_schedule<F == ES_HIP_Q5_K ? 13 : F == ES_HIP_Q3_K ? 8 : 9>();
            __builtin_amdgcn_sched_barrier(0);
            if (tt == 1) {
                // the next load group, once this superblock's weights are unpacked (the first MFMAs used them)
                stage_dma(bn, 1 - sl);
                wload(bn, W);
                if constexpr (BSUMS) bsn = bs_load(bn);
                __builtin_amdgcn_sched_barrier(0);
            }
        }
        if constexpr (BSUMS) bs_write(bsn, 1 - sl);
    }
    epilogue<F, FUSED>(p0.m, p0.d, p0.dm, p0.yd, acc[MK_TT - 2]);
    epilogue<F, FUSED>(p1.m, p1.d, p1.dm, p1.yd, acc[MK_TT - 1]);

    // ---- outputs: lane l, register i holds activation tok0 + 16 tt + 4 lg + i, row row0 + 16 wave + lr. Buffer stores
    // over y[0, (na - 1) * ystride + r1): the hardware's range check drops those of activations past na (ystride >= r1),
    // and rows past r1 get an offset above the range. The host keeps (na + MK_TOK) * ystride * 4 below 2^31, so no offset
    // wraps.
    const int r = row0 + 16 * wave + lr;
    const uint32_t ys4 = 4u * (uint32_t)J.ystride;
    const uint32_t yrange = (uint32_t)(J.na - 1) * ys4 + 4u * (uint32_t)J.r1;
    const __amdgpu_buffer_rsrc_t yrsrc = __builtin_amdgcn_make_buffer_rsrc((void *)J.y, (short)0, (int)yrange, 0x00020000);
    uint32_t yoff = r < J.r1 ? (uint32_t)(tok0 + 4 * lg) * ys4 + 4u * (uint32_t)r : 0x80000000u;
#pragma unroll
    for (int tt = 0; tt < MK_TT; tt++)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float v = acc[tt][i];   // (a bit cast of the vector element itself reads element 0 with this compiler)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yrsrc, (int)yoff, 0, 0);
            yoff += i < 3 ? ys4 : 13 * ys4;   // the next activation: + 1, or + 13 to the next tile's first
        }
}

}  // namespace

template <int F, int T>
static void mk_launch_tok(bool gather, bool contract, const MkJob *jobs, int njobs, const MkJob &single, int grid,
                          hipStream_t s) {
    const dim3 g(grid), b(64 * MK_WAVES);
    if (gather) {
        if (contract) hipLaunchKernelGGL((mk_kernel<F, true, true, T>), g, b, 0, s, jobs, njobs, single);
        else hipLaunchKernelGGL((mk_kernel<F, false, true, T>), g, b, 0, s, jobs, njobs, single);
    } else {
        if (contract) hipLaunchKernelGGL((mk_kernel<F, true, false, T>), g, b, 0, s, jobs, njobs, single);
        else hipLaunchKernelGGL((mk_kernel<F, false, false, T>), g, b, 0, s, jobs, njobs, single);
    }
}

template <int F>
static void mk_launch_fmt(int tok, bool gather, bool contract, const MkJob *jobs, int njobs, const MkJob &single, int grid,
                          hipStream_t s) {
    if (tok == 64) mk_launch_tok<F, 64>(gather, contract, jobs, njobs, single, grid, s);
    else mk_launch_tok<F, 128>(gather, contract, jobs, njobs, single, grid, s);
}

hipError_t mk_launch(int type, bool gather, int tok, const MkJob *jobs, int njobs, const MkJob &single, int grid, int order,
                     hipStream_t s) {
    const bool contract = order == ES_HIP_ORDER_X86_CONTRACT;
    if (tok != 64 && tok != MK_TOK) return hipErrorInvalidValue;
    if (type == ES_HIP_Q4_K) mk_launch_fmt<ES_HIP_Q4_K>(tok, gather, contract, jobs, njobs, single, grid, s);
    else if (type == ES_HIP_Q5_K) mk_launch_fmt<ES_HIP_Q5_K>(tok, gather, false, jobs, njobs, single, grid, s);   // never fused
    else if (type == ES_HIP_Q3_K) mk_launch_fmt<ES_HIP_Q3_K>(tok, gather, contract, jobs, njobs, single, grid, s);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace esq
