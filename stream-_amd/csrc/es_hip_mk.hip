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
#include <type_traits>

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
// [lg][activation][4] | scales. After the two slots, one landing area for the next superblock's raw int16 bsums
// [activation][16] (RAW bytes), converted into a slot's halves by the wave that copied them.
constexpr int TROW = 256;
template <int T> struct MkSlot {
    static constexpr int QS = 0, BS = T * TROW, D = BS + T * 32, BYTES = D + T * 4, TT = T / 16, RAW = T * 32;
    static_assert(T == 64 || T == 128, "the staging assignment below is written for 64 or 128 activations");
    static_assert(MK_WG_PER_CU * (2 * BYTES + RAW) <= 160 * 1024, "the workgroups of a CU fit its LDS");
};

typedef _Float16 v4h __attribute__((ext_vector_type(4)));

template <int F> struct MkFmt;
template <> struct MkFmt<ES_HIP_Q4_K> { static constexpr int BB = 144, QS = 16; };
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

// An empty statement that takes every B operand as an input: placed before the next load group's copies (volatile
// statements keep their order), it keeps the unpacking, and the compiler's wait for the weight registers it reads, above
// the copies. The compiler counts only its own loads: its wait placed after the copies would wait for most of them too.
template <int F> __device__ __forceinline__ void b_ready(const BOps<F> &B) {
#pragma unroll
    for (int s = 0; s < 4; s++) {
        asm volatile("" ::"v"(B.lo[s]), "v"(B.hi[s]));
        if constexpr (F == ES_HIP_Q5_K) asm volatile("" ::"v"(B.q5[s]));
    }
    if constexpr (F != ES_HIP_Q3_K) asm volatile("" ::"v"(B.mn));
    asm volatile("" ::"v"(B.d), "v"(B.dm));
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
    // weight loads per superblock and lane (one 16-byte load each, so the count is exact: no load merges into another)
    constexpr int NW = F == ES_HIP_Q5_K ? 4 : 3;
    constexpr uint32_t RAW0 = 2 * ST_BYTES;
    __shared__ __align__(16) uint8_t smem[2 * ST_BYTES + (BSUMS ? SL::RAW : 0)];

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
    // bsums: the raw int16 rows go into the landing area by LDS DMA, one instruction per wave (wave w, lane l: activation
    // 32 (w % RW) + l / 2, bsums 8 (l & 1) .. + 7; at 64 activations waves 2 and 3 repeat waves 0 and 1: the same bytes to
    // the same place); every thread then converts the 8 bsums it copied (activation bt, bsums 8*bh .. 8*bh+7) to halves.
    constexpr int RW = T / 32;
    const int bt = (tid >> 1) & (T - 1), bh = tid & 1;
    const uint32_t rawoff = act_off(32 * (wave % RW) + (lane >> 1)) + 260 + 16 * (lane & 1);
    const uint32_t bdst0 = ST_BS + (2 * bh) * (T * 8) + bt * 8, bdst1 = bdst0 + T * 8;
    const uint32_t smem0 = lds_addr(smem);
    const uint32_t rawdst = smem0 + RAW0 + 1024u * (uint32_t)(wave % RW), rawsrc = smem0 + RAW0 + 16u * (uint32_t)(tid & (2 * T - 1));

    // the superblock's base address, kept opaque in scalar registers (as plain arithmetic the compiler folds it into
    // per-lane 64-bit pointers)
    auto sb_base = [&](int b) {
        uint32_t sb = 292u * (uint32_t)b;
        asm volatile("" : "+s"(sb));
        return J.act + sb;
    };
    // piece k (0 .. NP - 1) of superblock b's copies into slot st: value chunks, then scales, then raw bsums
    constexpr int NP = NV + 1 + (BSUMS ? 1 : 0);
    auto stage_part = [&](int b, int st, int k) {
        const uint8_t *ab = sb_base(b);
        if (k < NV) {
            load_lds16(ab, qoff[k], smem0 + (uint32_t)st * ST_BYTES + ST_QS + (uint32_t)(TW * wave) * TROW + 4 * TROW * k);
        } else if (k == NV) {
            // the other waves repeat waves 0 and 1's copy (the same bytes to the same place): the code stays branch-free
            load_lds4(ab, doff, smem0 + (uint32_t)st * ST_BYTES + ST_D + 256 * ds);
        } else if constexpr (BSUMS) {
            load_lds16(ab, rawoff, rawdst);
        }
    };
    auto stage_dma = [&](int b, int st) {
#pragma unroll
        for (int k = 0; k < NP; k++) stage_part(b, st, k);
    };
    // the bsums this thread copied (landed: its wave waited for its copies) as halves into slot st
    auto bs_convert = [&](int st) {
        const u32x4 v = lds_ld<u32x4>(rawsrc);
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
    // field f (0 .. NW - 1) of superblock b's weights: one 16-byte load
    auto wload_part = [&](int b, WRaw<F> &W, int f) {
        const uint8_t *p = wbase + woff + (uint32_t)FM::BB * (uint32_t)b;
        if constexpr (F == ES_HIP_Q3_K) {
            if (f == 0) W.h = ldg_u128_a2(p + 94);
            else if (f == 1) W.q = ldg_u128_a2(p + FM::QS + 16 * lg);
            else W.hm = ldg_u128_a2(p + FM::QH + 16 * (lg & 1));
        } else {
            if (f == 0) W.h = ldg<uint4>(p);
            else if (f == 1) W.q0 = ldg<uint4>(p + FM::QS + 16 * lg);
            else if (f == 2) W.q1 = ldg<uint4>(p + FM::QS + 64 + 16 * lg);
            else if constexpr (F == ES_HIP_Q5_K) W.qh = ldg<uint4>(p + FM::QH + 16 * (lg & 1));
        }
    };
    auto wload = [&](int b, WRaw<F> &W) {
#pragma unroll
        for (int f = 0; f < NW; f++) wload_part(b, W, f);
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

    // Per superblock b (slot b & 1, weights in one of two register sets): the barrier (slot b & 1 complete and its bsums
    // converted, the other slot free); the B operands of superblock b from its weights; the copies of superblock b + 1
    // into the free slot and the landing area, then the weights of superblock b + 2 into the register set just unpacked;
    // the matrix work over the 8 activation tiles; a wait for this wave's copies (every load but the NW weight loads
    // issued last) and the conversion of the bsums it copied. So the copies have a whole superblock of matrix work to
    // arrive and the weights two, and no wait drains the weight loads in flight. Loads past the last superblock repeat
    // it into a slot or register set nobody reads.
    //
    // The loop is unrolled by two so that the slot and the register set of each half are compile-time choices (a register
    // set picked at run time would move in-flight load destinations, and the compiler would wait for them first); with
    // an odd number of superblocks the last one follows the loop.
    //
    // A tile's epilogue runs two tile steps after its MFMAs (a step's vector work then never waits for the matrix cores),
    // across superblock boundaries: steps 0 and 1 of superblock b finish tiles 6 and 7 of superblock b - 1. The two
    // pending slots start as zeros (all scales 0), whose epilogues add +0 to the +0 of acc[6] and acc[7]: the same bits.
    Pend<F> p0, p1;   // the tiles two and one steps back
    p0.m = MAcc<F>{};
    p0.yd = v4f{0, 0, 0, 0};
    p0.d = p0.dm = 0.f;
    p1 = p0;
    WRaw<F> Wa, Wb;   // superblocks of even / odd index
    stage_dma(0, 0);
    wload(0, Wa);
    wload(min(1, nbk - 1), Wb);
    wait_vmcnt<NW>();   // superblock 0's copies and weights (superblock 1's weights may still be in flight)
    if constexpr (BSUMS) bs_convert(0);
    auto iter = [&](auto slc, int b, WRaw<F> &Wc) {
        constexpr int sl = decltype(slc)::value;
        lds_sync();
        BOps<F> B;
        build_b<F>(Wc, lg, B);
        b_ready<F>(B);
        stage_dma(min(b + 1, nbk - 1), 1 - sl);
        wload(min(b + 2, nbk - 1), Wc);
        __builtin_amdgcn_sched_barrier(0);
        constexpr uint32_t so = (uint32_t)sl * ST_BYTES;
        const uint32_t xa[4] = {smem0 + so + xo[0], smem0 + so + xo[1], smem0 + so + xo[2], smem0 + so + xo[3]};
        const uint32_t ba = smem0 + so + bso, ya = smem0 + so + ydo;
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
        }
        wait_vmcnt<NW>();   // this wave's copies of superblock b + 1 (the weights of b + 2 may still be in flight)
        if constexpr (BSUMS) bs_convert(1 - sl);
    };
    int b = 0;
    for (; b + 1 < nbk; b += 2) {
        iter(std::integral_constant<int, 0>{}, b, Wa);
        iter(std::integral_constant<int, 1>{}, b + 1, Wb);
    }
    if (b < nbk) iter(std::integral_constant<int, 0>{}, b, Wa);
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

// ---- the persistent form ----------------------------------------------------------------------------------------------
// Workgroup g computes tiles tiles[wgptr[g] .. wgptr[g + 1]) (64 rows x 128 or 64 activations each, records written by
// the host and copied into LDS at the start) as one stream of (tile, superblock) items: the mk_kernel loop above, whose
// copies (one item ahead) and weight loads (two items ahead) run across tile boundaries, so a workgroup waits for its
// first loads once. The ring keeps the 128-activation layout for both tile widths (a 64-wide tile uses the first half of
// every region). At a tile's last item the two pending epilogues run at once, the outputs are stored and the accumulators
// cleared; then the next tile's sources become current.
template <int F, bool CONTRACT> struct PkGeom {
    using SL = MkSlot<128>;
    static constexpr uint32_t RAW0 = 2 * SL::BYTES, REC0 = RAW0 + SL::RAW, BYTES = REC0 + PK_MAX_TILES * sizeof(PkTile);
    static_assert(2 * BYTES <= 160 * 1024, "two workgroups fit a CU's LDS");
};

// the tiles of one workgroup, all of one width (T64: 64 activations); smem: PkGeom's LDS
template <int F, bool CONTRACT, bool T64>
__device__ __forceinline__ void pk_body(const PkTile *__restrict__ tiles, int k0, int nt, uint8_t *smem) {
    using FM = MkFmt<F>;
    using SL = MkSlot<128>;
    constexpr int ST_QS = SL::QS, ST_BS = SL::BS, ST_D = SL::D, ST_BYTES = SL::BYTES;
    constexpr bool FUSED = CONTRACT && F != ES_HIP_Q5_K;
    constexpr bool BSUMS = F != ES_HIP_Q3_K;
    constexpr int NW = F == ES_HIP_Q5_K ? 4 : 3;
    constexpr uint32_t RAW0 = PkGeom<F, CONTRACT>::RAW0, REC0 = PkGeom<F, CONTRACT>::REC0;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const uint32_t smem0 = lds_addr(smem);
    for (int i = tid; i < nt * (int)(sizeof(PkTile) / 16); i += 256)
        *reinterpret_cast<uint4 *>(smem + REC0 + 16 * i) = ldg<uint4>(reinterpret_cast<const uint8_t *>(tiles + k0) + 16 * i);
    __syncthreads();

    struct Rec {
        const uint8_t *w, *act;
        float *y;
        uint32_t astride, ystride4, row_bytes;
        int nbk, t64, tok0, na, rows, ntok;
    };
    auto rec = [&](int k) {   // tile k of the workgroup, in scalar registers
        const uint32_t a = smem0 + REC0 + (uint32_t)k * (uint32_t)sizeof(PkTile);
        const u32x4 v0 = lds_ld<u32x4>(a), v1 = lds_ld<u32x4>(a + 16), v2 = lds_ld<u32x4>(a + 32), v3 = lds_ld<u32x4>(a + 48);
        auto u = [](uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); };
        auto p = [&](uint32_t lo, uint32_t hi) { return (uint64_t)u(lo) | (uint64_t)u(hi) << 32; };
        Rec r;
        r.w = reinterpret_cast<const uint8_t *>(p(v0.x, v0.y));
        r.act = reinterpret_cast<const uint8_t *>(p(v0.z, v0.w));
        r.y = reinterpret_cast<float *>(p(v1.x, v1.y));
        r.astride = u(v1.z);
        r.ystride4 = u(v1.w);
        r.row_bytes = u(v2.x);
        r.nbk = (int)u(v2.y);
        r.t64 = (int)u(v2.z);
        r.tok0 = (int)u(v2.w);
        r.na = (int)u(v3.x);
        r.rows = (int)u(v3.y);
        r.ntok = (int)u(v3.z);
        return r;
    };
    // the per-lane sources of a tile (see mk_kernel): value chunks (NVt = 8, or 4 for 64 activations), scale, raw bsums,
    // weight row
    struct Src {
        uint32_t q[8], d, raw, w;
    };
    auto sources = [&](const Rec &r) {
        auto act_off = [&](int t) { return (uint32_t)min(r.tok0 + t, r.na - 1) * r.astride; };
        const int tw = r.t64 ? 16 : 32, rw = r.t64 ? 2 : 4;
        Src c;
#pragma unroll
        for (int k = 0; k < 8; k++) {
            const int t = tw * wave + 4 * (k & (r.t64 ? 3 : 7)) + (lane >> 4);
            c.q[k] = act_off(t) + 4 + 16 * ((lane & 15) ^ (t & 15));
        }
        c.d = act_off(64 * (r.t64 ? 0 : (wave & 1)) + lane);
        c.raw = act_off(32 * (wave % rw) + (lane >> 1)) + 260 + 16 * (lane & 1);
        c.w = (uint32_t)min(16 * wave + lr, r.rows - 1) * r.row_bytes;
        return c;
    };
    auto sb_base = [&](const uint8_t *act, int b) {
        uint32_t sb = 292u * (uint32_t)b;
        asm volatile("" : "+s"(sb));
        return act + sb;
    };
    // the copies of superblock b of a tile into slot st (values, scale, raw bsums) from its sources c
    auto stage = [&](const Rec &r, const Src &c, int b, int st) {
        const uint8_t *ab = sb_base(r.act, b);
        const uint32_t so = smem0 + (uint32_t)st * ST_BYTES;
        if (r.t64) {
#pragma unroll
            for (int k = 0; k < 4; k++) load_lds16(ab, c.q[k], so + ST_QS + (uint32_t)(16 * wave) * TROW + 4 * TROW * k);
            load_lds4(ab, c.d, so + ST_D);
            if constexpr (BSUMS) load_lds16(ab, c.raw, smem0 + RAW0 + 1024u * (uint32_t)(wave & 1));
        } else {
#pragma unroll
            for (int k = 0; k < 8; k++) load_lds16(ab, c.q[k], so + ST_QS + (uint32_t)(32 * wave) * TROW + 4 * TROW * k);
            load_lds4(ab, c.d, so + ST_D + 256 * (wave & 1));
            if constexpr (BSUMS) load_lds16(ab, c.raw, smem0 + RAW0 + 1024u * (uint32_t)wave);
        }
    };
    // the same for a tile's first superblock while the previous tile is current: each source offset formed as it is issued
    auto stage_first = [&](const Rec &r, int st) {
        const uint8_t *ab = r.act;
        const uint32_t so = smem0 + (uint32_t)st * ST_BYTES;
        auto act_off = [&](int t) { return (uint32_t)min(r.tok0 + t, r.na - 1) * r.astride; };
        const int tw = r.t64 ? 16 : 32, nv = r.t64 ? 4 : 8, rw = r.t64 ? 2 : 4, ds = r.t64 ? 0 : (wave & 1);
        for (int k = 0; k < nv; k++) {
            const int t = tw * wave + 4 * k + (lane >> 4);
            load_lds16(ab, act_off(t) + 4 + 16 * ((lane & 15) ^ (t & 15)), so + ST_QS + (uint32_t)(tw * wave) * TROW + 4 * TROW * k);
        }
        load_lds4(ab, act_off(64 * ds + lane), so + ST_D + 256 * ds);
        if constexpr (BSUMS)
            load_lds16(ab, act_off(32 * (wave % rw) + (lane >> 1)) + 260 + 16 * (lane & 1), smem0 + RAW0 + 1024u * (uint32_t)(wave % rw));
    };
    // the raw bsums this thread copied (its wave waited for them) as halves into slot st
    auto bs_convert = [&](int st, int t64) {
        const int T = t64 ? 64 : 128;
        const int bt = (tid >> 1) & (T - 1), bh = tid & 1;
        const u32x4 v = lds_ld<u32x4>(smem0 + RAW0 + 16u * (uint32_t)(tid & (2 * T - 1)));
        const uint32_t w[4] = {v.x, v.y, v.z, v.w};
        uint32_t hv[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const _Float16 e0 = (_Float16)(int16_t)(w[k] & 0xffffu), e1 = (_Float16)(int16_t)(w[k] >> 16);
            hv[k] = (uint32_t)__builtin_bit_cast(uint16_t, e0) | (uint32_t)__builtin_bit_cast(uint16_t, e1) << 16;
        }
        uint8_t *base = smem + st * ST_BYTES + ST_BS + (2 * bh) * (128 * 8) + bt * 8;
        *reinterpret_cast<uint2 *>(base) = make_uint2(hv[0], hv[1]);
        *reinterpret_cast<uint2 *>(base + 128 * 8) = make_uint2(hv[2], hv[3]);
    };
    auto wload = [&](const uint8_t *wrow, uint32_t woff, int b, WRaw<F> &W) {
        const uint8_t *p = wrow + woff + (uint32_t)FM::BB * (uint32_t)b;
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

    // A operand offsets in a slot (the 128-activation layout)
    uint32_t xo[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int nat = F == ES_HIP_Q3_K ? 8 * (lg >> 1) + 2 * s + (lg & 1) : 4 * (lg >> 1) + 8 * (s >> 1) + 2 * (s & 1) + (lg & 1);
        xo[s] = ST_QS + lr * TROW + 16 * (nat ^ lr);
    }
    const uint32_t bso = ST_BS + lg * (128 * 8) + lr * 8, ydo = ST_D + 16 * lg;
    auto aload = [&](const uint32_t (&xa)[4], uint32_t ba, uint32_t ya, int tt, AOps &A) {
#pragma unroll
        for (int s = 0; s < 4; s++) A.x[s] = lds_ld<v4i>(xa[s] + 16 * TROW * tt);
        if constexpr (BSUMS) A.bs = lds_ld<v4h>(ba + 128 * tt);
        A.yd = lds_ld<v4f>(ya + 64 * tt);
    };

    v4f acc[8];
#pragma unroll
    for (int t = 0; t < 8; t++) acc[t] = v4f{0, 0, 0, 0};
    Pend<F> p0, p1;
    p0.m = MAcc<F>{};
    p0.yd = v4f{0, 0, 0, 0};
    p0.d = p0.dm = 0.f;
    p1 = p0;
    const Pend<F> pzero = p0;

    // The matrix work of one item over its activation tiles (slot base so). A 64-activation tile leaves after four
    // steps: its last two epilogues run there and the pending slots are cleared (the next item's first two steps then
    // add +0 to accumulators 6 and 7, which such a tile never stores).
    auto steps = [&](auto t64c, uint32_t so, const BOps<F> &B) {
        constexpr bool t64 = decltype(t64c)::value;
        const uint32_t xa[4] = {smem0 + so + xo[0], smem0 + so + xo[1], smem0 + so + xo[2], smem0 + so + xo[3]};
        const uint32_t ba = smem0 + so + bso, ya = smem0 + so + ydo;
        AOps A[2];
        aload(xa, ba, ya, 0, A[0]);
#pragma unroll
        for (int tt = 0; tt < (t64 ? 4 : 8); tt++) {
            if (tt + 1 < (t64 ? 4 : 8)) aload(xa, ba, ya, tt + 1, A[(tt + 1) & 1]);
            MAcc<F> cur;
            mma<F>(A[tt & 1], B, cur);
            epilogue<F, FUSED>(p0.m, p0.d, p0.dm, p0.yd, acc[(tt + 6) % 8]);
            p0 = p1;
            p1.m = cur;
            p1.yd = A[tt & 1].yd;
            p1.d = B.d;
            p1.dm = B.dm;
            step_schedule<F == ES_HIP_Q5_K ? 13 : F == ES_HIP_Q3_K ? 8 : 9>();
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (t64) {
            epilogue<F, FUSED>(p0.m, p0.d, p0.dm, p0.yd, acc[2]);
            epilogue<F, FUSED>(p1.m, p1.d, p1.dm, p1.yd, acc[3]);
            p0 = pzero;
            p1 = pzero;
        }
    };
    // a finished tile: the two pending epilogues, the outputs of all eight activation tiles (buffer stores checked against
    // the tile's range: activations past ntok, among them every one of a 64-wide tile's upper half, and rows past rows
    // are dropped), the accumulators and pending slots cleared
    auto flush = [&](const Rec &r) {
        epilogue<F, FUSED>(p0.m, p0.d, p0.dm, p0.yd, acc[6]);
        epilogue<F, FUSED>(p1.m, p1.d, p1.dm, p1.yd, acc[7]);
        p0 = pzero;
        p1 = pzero;
        const int row = 16 * wave + lr;
        const uint32_t yrange = (uint32_t)(r.ntok - 1) * r.ystride4 + 4u * (uint32_t)r.rows;
        const __amdgpu_buffer_rsrc_t yrsrc = __builtin_amdgcn_make_buffer_rsrc((void *)r.y, (short)0, (int)yrange, 0x00020000);
        uint32_t yoff = row < r.rows ? (uint32_t)(4 * lg) * r.ystride4 + 4u * (uint32_t)row : 0x80000000u;
#pragma unroll
        for (int tt = 0; tt < 8; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = acc[tt][i];
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yrsrc, (int)yoff, 0, 0);
                yoff += i < 3 ? r.ystride4 : 13 * r.ystride4;
            }
#pragma unroll
        for (int t = 0; t < 8; t++) acc[t] = v4f{0, 0, 0, 0};
    };

    // ---- the item stream. rc: the current tile (k), rn: the next (or rc again past the last); C: rc's sources
    int k = 0;
    Rec rc = rec(0), rn = rec(nt > 1 ? 1 : 0);
    Src C = sources(rc);
    WRaw<F> Wa, Wb;
    stage(rc, C, 0, 0);
    wload(rc.w, C.w, 0, Wa);
    wload(rc.w, C.w, 1, Wb);
    wait_vmcnt<NW>();
    if constexpr (BSUMS) bs_convert(0, rc.t64);

    // One item: superblock j of the current tile in slot j & 1, its weights in register set Wc (tiles have an even number
    // of superblocks, so every tile starts at j = 0 in slot 0 with its weights in Wa, and a pair of items never spans two
    // tiles). At the tile's last item its outputs are stored and the next tile becomes current.
    int j = 0;
    auto item = [&](auto t64c, auto slc, WRaw<F> &Wc) {
        constexpr int sl = decltype(slc)::value;
        lds_sync();
        BOps<F> B;
        build_b<F>(Wc, lg, B);
        b_ready<F>(B);
        // the copies of the next item: superblock j + 1 of this tile, else the next tile's first
        const bool more = k + 1 < nt;
        int t64n = rc.t64;
        if (j + 1 < rc.nbk || !more) {
            stage(rc, C, min(j + 1, rc.nbk - 1), 1 - sl);
        } else {
            stage_first(rn, 1 - sl);
            t64n = rn.t64;
        }
        // the weights of the item after: superblock j + 2 of this tile, else of the next (every tile has >= 2)
        {
            const bool here = j + 2 < rc.nbk || !more;
            const uint8_t *wr = here ? rc.w : rn.w;
            const uint32_t wo = here ? C.w : (uint32_t)min(16 * wave + lr, rn.rows - 1) * rn.row_bytes;
            const int bw = j + 2 < rc.nbk ? j + 2 : more ? j + 2 - rc.nbk : rc.nbk - 1;
            wload(wr, wo, bw, Wc);
        }
        __builtin_amdgcn_sched_barrier(0);
        steps(t64c, (uint32_t)sl * ST_BYTES, B);
        wait_vmcnt<NW>();   // this wave's copies of the next item (the weights after it may still be in flight)
        if constexpr (BSUMS) bs_convert(1 - sl, t64n);
        if (++j == rc.nbk) {
            flush(rc);
            j = 0;
            if (++k < nt) {
                rc = rn;
                rn = rec(k + 1 < nt ? k + 1 : k);
                C = sources(rc);
            }
        }
    };
    while (k < nt) {
        item(std::integral_constant<bool, T64>{}, std::integral_constant<int, 0>{}, Wa);
        item(std::integral_constant<bool, T64>{}, std::integral_constant<int, 1>{}, Wb);
    }
}

// Workgroups [0, g64) take tiles of 64 activations, the others tiles of 128: two separate bodies, chosen once.
template <int F, bool CONTRACT>
__global__ __launch_bounds__(256, 2) void pk_kernel(const PkTile *__restrict__ tiles, const int *__restrict__ wgptr, int g64) {
    __shared__ __align__(16) uint8_t smem[PkGeom<F, CONTRACT>::BYTES];
    const int k0 = wgptr[blockIdx.x], nt = wgptr[blockIdx.x + 1] - k0;
    if (nt <= 0) return;
    if ((int)blockIdx.x < g64) pk_body<F, CONTRACT, true>(tiles, k0, nt, smem);
    else pk_body<F, CONTRACT, false>(tiles, k0, nt, smem);
}

// ---- the wave-specialised persistent form (Q4_K) ------------------------------------------------------------------------
// One workgroup of 8 waves per CU runs a host-scheduled list of tiles (64 rows x 128 activations) as a stream of items
// (tile, superblock), as pk_body does, but splits each item's work by kind over the waves of a SIMD:
//   waves 0-3 (matrix waves): wave m reads the B operands of rows 16m .. 16m+15 from LDS and runs the item's 8 tile steps
//     (72 MFMAs and the float epilogue of the tiles two steps back) and the tile's stores, as pk_body does;
//   waves 4-7 (staging waves): wave 4 + u loads a quarter of the item's activations (values, scales, bsums) and the
//     weights of rows 16u .. 16u+15 into registers three items ahead, and one item ahead writes them into LDS: the values
//     swizzled as in mk_kernel, the bsums converted to halves, the weights unpacked into the B operands (build_b).
// The unpacking and the loads then run beside the matrix work on every SIMD instead of between its tile steps. Every
// load is an ordinary (compiler-counted) buffer load into registers, so no wait drains loads issued after the ones it
// needs. LDS: two activation slots and two B-operand slots (item i in slots i & 1) and the tile records; one barrier per
// item: at barrier i, item i's slots are complete and item i - 1's are free.
struct WsGeom {
    using SL = MkSlot<128>;
    static constexpr uint32_t ACT = SL::BYTES;            // an activation slot (the 128-activation layout of mk_kernel)
    static constexpr uint32_t PLT = 9 * 1024;             // one row tile's B operands: 9 chunks of 16 bytes per lane
    static constexpr uint32_t PLS = 4 * PLT;              // a B-operand slot: 4 row tiles
    static constexpr uint32_t PL0 = 2 * ACT, REC0 = PL0 + 2 * PLS;
    static constexpr uint32_t BYTES = REC0 + PK_MAX_TILES * sizeof(PkTile);
    static_assert(BYTES <= 160 * 1024, "the workgroup fits a CU's LDS");
};

struct WsRec {   // a tile record in scalar registers
    const uint8_t *w, *act;
    float *y;
    uint32_t astride, ystride4, row_bytes;
    int nbk, tok0, na, rows, ntok;
};
__device__ __forceinline__ WsRec ws_rec(uint32_t rec0, int k) {
    const uint32_t a = rec0 + (uint32_t)k * (uint32_t)sizeof(PkTile);
    const u32x4 v0 = lds_ld<u32x4>(a), v1 = lds_ld<u32x4>(a + 16), v2 = lds_ld<u32x4>(a + 32), v3 = lds_ld<u32x4>(a + 48);
    auto u = [](uint32_t x) { return (uint32_t)__builtin_amdgcn_readfirstlane((int)x); };
    auto p = [&](uint32_t lo, uint32_t hi) { return (uint64_t)u(lo) | (uint64_t)u(hi) << 32; };
    WsRec r;
    r.w = reinterpret_cast<const uint8_t *>(p(v0.x, v0.y));
    r.act = reinterpret_cast<const uint8_t *>(p(v0.z, v0.w));
    r.y = reinterpret_cast<float *>(p(v1.x, v1.y));
    r.astride = u(v1.z);
    r.ystride4 = u(v1.w);
    r.row_bytes = u(v2.x);
    r.nbk = (int)u(v2.y);
    r.tok0 = (int)u(v2.w);
    r.na = (int)u(v3.x);
    r.rows = (int)u(v3.y);
    r.ntok = (int)u(v3.z);
    return r;
}

// the matrix waves (m = 0 .. 3)
template <int F, bool CONTRACT>
__device__ __forceinline__ void ws_matrix(uint8_t *smem, int nt, int nitems, int m) {
    using G = WsGeom;
    using SL = MkSlot<128>;
    constexpr bool FUSED = CONTRACT;
    const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
    const uint32_t smem0 = lds_addr(smem);
    uint32_t xo[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int nat = 4 * (lg >> 1) + 8 * (s >> 1) + 2 * (s & 1) + (lg & 1);
        xo[s] = SL::QS + lr * TROW + 16 * (nat ^ lr);
    }
    const uint32_t bso = SL::BS + lg * (128 * 8) + lr * 8, ydo = SL::D + 16 * lg;
    auto aload = [&](const uint32_t (&xa)[4], uint32_t ba, uint32_t ya, int tt, AOps &A) {
#pragma unroll
        for (int s = 0; s < 4; s++) A.x[s] = lds_ld<v4i>(xa[s] + 16 * TROW * tt);
        A.bs = lds_ld<v4h>(ba + 128 * tt);
        A.yd = lds_ld<v4f>(ya + 64 * tt);
    };
    v4f acc[8];
#pragma unroll
    for (int t = 0; t < 8; t++) acc[t] = v4f{0, 0, 0, 0};
    Pend<F> p0, p1;
    p0.m = MAcc<F>{};
    p0.yd = v4f{0, 0, 0, 0};
    p0.d = p0.dm = 0.f;
    p1 = p0;
    const Pend<F> pzero = p0;
    auto flush = [&](const WsRec &r) {   // as pk_body's: the pending epilogues, the stores, the accumulators cleared
        epilogue<F, FUSED>(p0.m, p0.d, p0.dm, p0.yd, acc[6]);
        epilogue<F, FUSED>(p1.m, p1.d, p1.dm, p1.yd, acc[7]);
        p0 = pzero;
        p1 = pzero;
        const int row = 16 * m + lr;
        const uint32_t yrange = (uint32_t)(r.ntok - 1) * r.ystride4 + 4u * (uint32_t)r.rows;
        const __amdgpu_buffer_rsrc_t yrsrc = __builtin_amdgcn_make_buffer_rsrc((void *)r.y, (short)0, (int)yrange, 0x00020000);
        uint32_t yoff = row < r.rows ? (uint32_t)(4 * lg) * r.ystride4 + 4u * (uint32_t)row : 0x80000000u;
#pragma unroll
        for (int tt = 0; tt < 8; tt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = acc[tt][i];
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yrsrc, (int)yoff, 0, 0);
                yoff += i < 3 ? r.ystride4 : 13 * r.ystride4;
            }
#pragma unroll
        for (int t = 0; t < 8; t++) acc[t] = v4f{0, 0, 0, 0};
    };
    int k = 0, j = 0;
    WsRec rc = ws_rec(smem0 + G::REC0, 0);
    for (int i = 0; i < nitems; i++) {
        lds_sync();   // item i's slots are complete
        const uint32_t so = (uint32_t)(i & 1) * G::ACT;
        const uint32_t pb = smem0 + G::PL0 + (uint32_t)(i & 1) * G::PLS + (uint32_t)m * G::PLT + 16u * (uint32_t)lane;
        BOps<F> B;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            B.lo[s] = lds_ld<v4i>(pb + 1024 * s);
            B.hi[s] = lds_ld<v4i>(pb + 1024 * (4 + s));
        }
        {
            const u32x4 x = lds_ld<u32x4>(pb + 8192);
            B.mn = __builtin_bit_cast(v4h, u32x2{x.x, x.y});
            B.d = __uint_as_float(x.z);
            B.dm = __uint_as_float(x.w);
        }
        const uint32_t xa[4] = {smem0 + so + xo[0], smem0 + so + xo[1], smem0 + so + xo[2], smem0 + so + xo[3]};
        const uint32_t ba = smem0 + so + bso, ya = smem0 + so + ydo;
        AOps A[2];
        aload(xa, ba, ya, 0, A[0]);
        __builtin_amdgcn_sched_barrier(0);   // every operand of the item's first step requested before its first MFMA
#pragma unroll
        for (int tt = 0; tt < 8; tt++) {
            if (tt + 1 < 8) aload(xa, ba, ya, tt + 1, A[(tt + 1) & 1]);
            MAcc<F> cur;
            mma<F>(A[tt & 1], B, cur);
            epilogue<F, FUSED>(p0.m, p0.d, p0.dm, p0.yd, acc[(tt + 6) % 8]);
            p0 = p1;
            p1.m = cur;
            p1.yd = A[tt & 1].yd;
            p1.d = B.d;
            p1.dm = B.dm;
            __builtin_amdgcn_sched_barrier(0);   // (the compiler's own interleaving: 2% faster here than step_schedule's)
        }
        if (++j == rc.nbk) {
            flush(rc);
            j = 0;
            if (++k < nt) rc = ws_rec(smem0 + G::REC0, k);
        }
    }
}

// the staging waves (u = 0 .. 3)
template <int F>
__device__ __forceinline__ void ws_stage(uint8_t *smem, int nt, int nitems, int u) {
    using G = WsGeom;
    using SL = MkSlot<128>;
    using FM = MkFmt<F>;
    const int lane = threadIdx.x & 63, lr = lane & 15, lg = lane >> 4;
    const uint32_t smem0 = lds_addr(smem);
    struct Set {   // one item's loads: 8 value chunks (activations 32u + 4c + lane/16), the scale (activation 32u + lane %
                   // 32), 8 bsums (activation 32u + lane/2, half lane & 1), the weights' header and two qs chunks
        u32x4 q[8], bs, h, q0, q1;
        uint32_t d;
    };
    struct LTile {   // the load stream's tile: buffer resources and per-lane offsets
        __amdgpu_buffer_rsrc_t ar, wr;
        uint32_t q[8], bs, d, wo;
        int nbk;
    };
    auto ltile = [&](int k) {
        const WsRec r = ws_rec(smem0 + G::REC0, k);
        LTile t;
        t.ar = __builtin_amdgcn_make_buffer_rsrc((void *)r.act, (short)0, (int)0xffffffffu, 0x00020000);
        t.wr = __builtin_amdgcn_make_buffer_rsrc((void *)r.w, (short)0, (int)0xffffffffu, 0x00020000);
        auto act_off = [&](int a) { return (uint32_t)min(r.tok0 + a, r.na - 1) * r.astride; };
#pragma unroll
        for (int c = 0; c < 8; c++) t.q[c] = act_off(32 * u + 4 * c + (lane >> 4)) + 4 + 16 * (lane & 15);
        t.bs = act_off(32 * u + (lane >> 1)) + 260 + 16 * (lane & 1);
        t.d = act_off(32 * u + (lane & 31));
        t.wo = (uint32_t)min(16 * u + lr, r.rows - 1) * r.row_bytes;
        t.nbk = r.nbk;
        return t;
    };
    auto ld_value = [&](const LTile &t, int j, int c) {
        return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(t.ar, (int)t.q[c], 292 * j, 0));
    };
    auto ld_scales = [&](const LTile &t, int j, Set &S) {
        S.bs = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(t.ar, (int)t.bs, 292 * j, 0));
        S.d = __builtin_amdgcn_raw_buffer_load_b32(t.ar, (int)t.d, 292 * j, 0);
    };
    auto ld_weights = [&](const LTile &t, int j, Set &S) {
        const int sw = FM::BB * j;
        S.h = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(t.wr, (int)t.wo, sw, 0));
        S.q0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(t.wr, (int)(t.wo + FM::QS + 16 * lg), sw, 0));
        S.q1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(t.wr, (int)(t.wo + FM::QS + 64 + 16 * lg), sw, 0));
    };
    // LDS destinations within a slot: value chunk c of activation a = 32u + 4c + lane/16 at row a, position
    // (lane % 16) ^ (a & 15); the scale at D + 4a (lanes 32-63 repeat lanes 0-31); the bsums' halves as mk_kernel lays
    // them out ([lg][activation][4]); this row tile's B operands at chunk c, 16 bytes per lane
    uint32_t qd[8];
#pragma unroll
    for (int c = 0; c < 8; c++) {
        const int a = 32 * u + 4 * c + (lane >> 4);
        qd[c] = SL::QS + (uint32_t)a * TROW + 16u * (uint32_t)((lane & 15) ^ (a & 15));
    }
    const uint32_t dd = SL::D + 4u * (uint32_t)(32 * u + (lane & 31));
    const uint32_t bd = SL::BS + (uint32_t)(2 * (lane & 1)) * (128 * 8) + (uint32_t)(32 * u + (lane >> 1)) * 8;
    const uint32_t pd = G::PL0 + (uint32_t)u * G::PLT + 16u * (uint32_t)lane;
    auto put_value = [&](const Set &S, int slot, int c) {
        *reinterpret_cast<u32x4 *>(smem + (uint32_t)slot * G::ACT + qd[c]) = S.q[c];
    };
    auto put_scales = [&](const Set &S, int slot) {
        uint8_t *ab = smem + (uint32_t)slot * G::ACT;
        *reinterpret_cast<uint32_t *>(ab + dd) = S.d;
        const uint32_t w[4] = {S.bs.x, S.bs.y, S.bs.z, S.bs.w};
        uint32_t hv[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {   // two int16 bsums -> two halves (exact: |bsums| <= 16 * 127)
            const _Float16 e0 = (_Float16)(int16_t)(w[c] & 0xffffu), e1 = (_Float16)(int16_t)(w[c] >> 16);
            hv[c] = (uint32_t)__builtin_bit_cast(uint16_t, e0) | (uint32_t)__builtin_bit_cast(uint16_t, e1) << 16;
        }
        *reinterpret_cast<uint2 *>(ab + bd) = make_uint2(hv[0], hv[1]);
        *reinterpret_cast<uint2 *>(ab + bd + 128 * 8) = make_uint2(hv[2], hv[3]);
    };
    auto put_operands = [&](const Set &S, int slot) {
        WRaw<F> wr;
        wr.h = make_uint4(S.h.x, S.h.y, S.h.z, S.h.w);
        wr.q0 = make_uint4(S.q0.x, S.q0.y, S.q0.z, S.q0.w);
        wr.q1 = make_uint4(S.q1.x, S.q1.y, S.q1.z, S.q1.w);
        BOps<F> B;
        build_b<F>(wr, lg, B);
        uint8_t *pb = smem + pd + (uint32_t)slot * G::PLS;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            *reinterpret_cast<v4i *>(pb + 1024 * s) = B.lo[s];
            *reinterpret_cast<v4i *>(pb + 1024 * (4 + s)) = B.hi[s];
        }
        const u32x2 mn = __builtin_bit_cast(u32x2, B.mn);
        *reinterpret_cast<u32x4 *>(pb + 8192) = u32x4{mn.x, mn.y, __float_as_uint(B.d), __float_as_uint(B.dm)};
    };
    // the load stream: item (lk, lj); past the last item it repeats the last (loads into a set nobody writes out)
    int lk = 0, lj = 0;
    LTile lt = ltile(0);
    auto advance = [&]() {
        if (lj + 1 < lt.nbk) {
            lj++;
        } else if (lk + 1 < nt) {
            lk++;
            lj = 0;
            lt = ltile(lk);
        }
    };
    auto issue = [&](Set &S) {
#pragma unroll
        for (int c = 0; c < 8; c++) S.q[c] = ld_value(lt, lj, c);
        ld_scales(lt, lj, S);
        ld_weights(lt, lj, S);
        advance();
    };
    Set S0, S1, S2;
    issue(S0);
    issue(S1);
    issue(S2);
#pragma unroll
    for (int c = 0; c < 8; c++) put_value(S0, 0, c);
    put_scales(S0, 0);
    put_operands(S0, 0);
    // item i: the loads of item i + 3 into the set item i used, interleaved with the writes of item i + 1 into slots
    // (i + 1) & 1 (one value load, one value write; the scales; the weights; the unpacking), so the loads enter the memory
    // pipeline a few at a time instead of in one burst that stalls the wave
    auto period = [&](Set &Sl, const Set &Sp, int i) {
        lds_sync();
        const int sl = (i + 1) & 1;
#pragma unroll
        for (int c = 0; c < 8; c++) {
            Sl.q[c] = ld_value(lt, lj, c);
            __builtin_amdgcn_sched_barrier(0);
            put_value(Sp, sl, c);
            __builtin_amdgcn_sched_barrier(0);
        }
        ld_scales(lt, lj, Sl);
        __builtin_amdgcn_sched_barrier(0);
        put_scales(Sp, sl);
        __builtin_amdgcn_sched_barrier(0);
        ld_weights(lt, lj, Sl);
        __builtin_amdgcn_sched_barrier(0);
        put_operands(Sp, sl);
        advance();
    };
    int i = 0;
    for (; i + 3 <= nitems; i += 3) {
        period(S0, S1, i);
        period(S1, S2, i + 1);
        period(S2, S0, i + 2);
    }
    if (i < nitems) period(S0, S1, i++);
    if (i < nitems) period(S1, S2, i++);
}

template <int F, bool CONTRACT>
__global__ __launch_bounds__(512, 1) void ws_kernel(const PkTile *__restrict__ tiles, const int *__restrict__ wgptr) {
    using G = WsGeom;
    __shared__ __align__(16) uint8_t smem[G::BYTES];
    const int k0 = wgptr[blockIdx.x], nt = wgptr[blockIdx.x + 1] - k0;
    if (nt <= 0) return;
    const int tid = threadIdx.x;
    for (int i = tid; i < nt * (int)(sizeof(PkTile) / 16); i += 512)
        *reinterpret_cast<uint4 *>(smem + G::REC0 + 16 * i) = ldg<uint4>(reinterpret_cast<const uint8_t *>(tiles + k0) + 16 * i);
    __syncthreads();
    int nitems = 0;   // every wave counts the items (tile records in LDS, read as scalars)
    for (int k = 0; k < nt; k++) nitems += ws_rec(lds_addr(smem) + G::REC0, k).nbk;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    if (wave < 4) ws_matrix<F, CONTRACT>(smem, nt, nitems, wave);
    else ws_stage<F>(smem, nt, nitems, wave - 4);
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

template <int F>
static void pk_launch_fmt(bool contract, const PkTile *tiles, const int *wgptr, int grid, int g64, hipStream_t s) {
    if (contract) hipLaunchKernelGGL((pk_kernel<F, true>), dim3(grid), dim3(256), 0, s, tiles, wgptr, g64);
    else hipLaunchKernelGGL((pk_kernel<F, false>), dim3(grid), dim3(256), 0, s, tiles, wgptr, g64);
}

hipError_t ws_launch(int type, const PkTile *tiles, const int *wgptr, int grid, int order, hipStream_t s) {
    if (type != ES_HIP_Q4_K) return hipErrorInvalidValue;
    if (order == ES_HIP_ORDER_X86_CONTRACT)
        hipLaunchKernelGGL((ws_kernel<ES_HIP_Q4_K, true>), dim3(grid), dim3(512), 0, s, tiles, wgptr);
    else
        hipLaunchKernelGGL((ws_kernel<ES_HIP_Q4_K, false>), dim3(grid), dim3(512), 0, s, tiles, wgptr);
    return hipGetLastError();
}

hipError_t pk_launch(int type, const PkTile *tiles, const int *wgptr, int grid, int g64, int order, hipStream_t s) {
    const bool contract = order == ES_HIP_ORDER_X86_CONTRACT;
    if (type == ES_HIP_Q4_K) pk_launch_fmt<ES_HIP_Q4_K>(contract, tiles, wgptr, grid, g64, s);
    else if (type == ES_HIP_Q3_K) pk_launch_fmt<ES_HIP_Q3_K>(contract, tiles, wgptr, grid, g64, s);
    else return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace esq
