// Decode / small-batch products on the vector ALU (v_dot4_i32_i8), every format of the library.
//
// One workgroup of W waves owns `rows_per_wg` consecutive rows of one job. Two phases per batch of `chain_rows` rows:
//
//  1. Integer phase, block-parallel and coalesced. The wave's 64 lanes are cut into slots of LPB lanes; each slot takes one
//     weight block (consecutive slots take consecutive blocks, so a wave-wide load covers a contiguous byte range) and each
//     lane of the slot takes a fixed share of the block's elements. The lane unpacks its share into int8 lanes, dots it with
//     the activation bytes it holds in registers (v_dot4) and the slot sums the partials (DPP lane moves). Integer
//     arithmetic is exact, so the order of these sums does not matter. The slot leader turns the block's integers into
//     the float terms of the reference epilogue and stores them in LDS. The raw loads of U units (a unit is one block
//     position of one row) are issued together before any of them is used, so every wave keeps U loads in flight.
//  2. Float phase, one lane per (row, activation[, AVX2 lane]). The lane runs the reference's accumulation over the row's
//     blocks in the reference's order (a strict sequential fp32 chain), so outputs are bit-identical to the CPU kernels.
//
// The activation slice a lane needs depends only on its block position inside the row, which stays fixed while the wave
// walks down the rows (long rows are split across the workgroup's waves), so activations are loaded into registers once
// per batch of NT activations.
//
// Reference kernels restated (integer parts and float order): src/es_quant.c:1013-1117 (scalar mv_*), 1252-1343 and
// 1443-1469 (AVX2 Q4_0/Q5_0/Q4_K/Q6_K), 1344-1368 and src/es_q2k.c:127-190 (Q2_K), 1120-1175 and 1370-1394 (Q3_K, Q5_K).
#include "es_hip_common.h"


// units (one block position of one row each) whose raw loads a wave issues before using any of them; a power of two
#ifndef ESQ_UNITS
#define ESQ_UNITS 4
#endif
#ifndef Q6K_UNITS1
#define Q6K_UNITS1 2
#endif
#ifndef Q6K_UNITSN
#define Q6K_UNITSN 1
#endif
#ifndef K_UNITSN
#define K_UNITSN 2
#endif
// the same at two activations per pass in the per-job-width kernel, whose register budget the four-wide body sets
#ifndef K_UNITS2M
#define K_UNITS2M 4
#endif
#ifndef Q6K_UNITS2M
#define Q6K_UNITS2M 1
#endif
#ifndef Q6K_UNITS1M
#define Q6K_UNITS1M 2
#endif
// resident waves per SIMD the register allocation must allow
#ifndef ESQ_MIN_WAVES
#define ESQ_MIN_WAVES 1
#endif

namespace esq {

// float terms of one block for one activation, consumed by the chain:
//   K-quants and the scalar 32-wide path: s = s (+) A (x) B in the selected order
//   AVX2 32-wide path: acc_i = fma((float)lane_i, dyd, acc_i) for the eight AVX2 lanes
struct Term2 { float a, b; };

enum { CH_FMA = 0, CH_MULADD = 1, CH_LANES = 2 };

// ---------------------------------------------------------------------------------------------------------------------
// Per-format lane work: Raw (the bytes one lane loads), Wt (unpacked), Act (activation slice), Ints (integer partials)

template <int F> struct Lane;

// Q4_K: lane k of 4 takes qs chunk k, bytes [32k, 32k+32): its low nibbles are elements 64k + [0,32) (sub-block 2k),
// its high nibbles 64k + 32 + [0,32) (sub-block 2k+1). src/es_quant.c:1056-1080.
template <> struct Lane<ES_HIP_Q4_K> {
    struct Raw { uint4 hdr, q0, q1; };
    struct Act { uint32_t lo[8], hi[8]; int bs0, bs1; float d; };
    struct Wt { uint32_t lo[8], hi[8]; int sc0, sc1, mn0, mn1; float d, dmin; };
    struct Ints { int dot, aux; };

    static __device__ __forceinline__ void load_act(const uint8_t *a, int k, Act &x) {
        x.d = ldg<float>(a);
#pragma unroll
        for (int v = 0; v < 2; v++) {
            const uint4 l = ldg<uint4>(a + 4 + 64 * k + 16 * v), h = ldg<uint4>(a + 4 + 64 * k + 32 + 16 * v);
            x.lo[4 * v] = l.x; x.lo[4 * v + 1] = l.y; x.lo[4 * v + 2] = l.z; x.lo[4 * v + 3] = l.w;
            x.hi[4 * v] = h.x; x.hi[4 * v + 1] = h.y; x.hi[4 * v + 2] = h.z; x.hi[4 * v + 3] = h.w;
        }
        const uint2 b = ldg<uint2>(a + 260 + 8 * k);   // bsums 4k .. 4k+3, the last 8 bytes of the record for k = 3
        x.bs0 = static_cast<int16_t>(b.x) + static_cast<int16_t>(b.x >> 16);
        x.bs1 = static_cast<int16_t>(b.y) + static_cast<int16_t>(b.y >> 16);
    }
    static __device__ __forceinline__ void zero_act(Act &x) {
        for (int i = 0; i < 8; i++) x.lo[i] = x.hi[i] = 0;
        x.bs0 = x.bs1 = 0;
        x.d = 0.0f;
    }
    static __device__ __forceinline__ void load_raw(const uint8_t *blk, int k, Raw &r) {
        r.hdr = ldw4(blk);
        r.q0 = ldw4(blk + 16 + 32 * k);
        r.q1 = ldw4(blk + 32 + 32 * k);
    }
    // 6-bit scale and min of sub-block j from the 12 packed bytes (scale_min_k4, src/es_quant.c:75-83)
    static __device__ __forceinline__ void scale_min(uint32_t s03, uint32_t s47, uint32_t s811, int j, int &sc, int &mn) {
        const int jj = (j & 3) * 8;
        const uint32_t a = (s03 >> jj) & 0xff, b = (s47 >> jj) & 0xff, c = (s811 >> jj) & 0xff;
        if (j < 4) { sc = a & 63; mn = b & 63; }
        else { sc = (c & 15) | ((a >> 6) << 4); mn = (c >> 4) | ((b >> 6) << 4); }
    }
    static __device__ __forceinline__ void unpack(const Raw &r, int k, Wt &w) {
        const uint32_t qq[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        for (int i = 0; i < 8; i++) { w.lo[i] = qq[i] & 0x0f0f0f0fu; w.hi[i] = (qq[i] >> 4) & 0x0f0f0f0fu; }
        scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * k, w.sc0, w.mn0);
        scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * k + 1, w.sc1, w.mn1);
        w.d = half_bits_to_float(r.hdr.x);
        w.dmin = half_bits_to_float(r.hdr.x >> 16);
    }
    static __device__ __forceinline__ Ints ints(const Wt &w, const Act &x) {
        int lo = 0, hi = 0;
        for (int i = 0; i < 8; i++) { lo = sdot4(w.lo[i], x.lo[i], lo); hi = sdot4(w.hi[i], x.hi[i], hi); }
        return {w.sc0 * lo + w.sc1 * hi, w.mn0 * x.bs0 + w.mn1 * x.bs1};
    }
    // s += y.d * (d * dot - dmin * mins)   (src/es_quant.c:1077, 1339)
    static __device__ __forceinline__ Term2 term(const Wt &w, const Act &x, Ints v, bool contract) {
        const float q = w.dmin * static_cast<float>(v.aux);
        const float in = contract ? __builtin_fmaf(w.d, static_cast<float>(v.dot), -q) : w.d * static_cast<float>(v.dot) - q;
        return {x.d, in};
    }
};

// Q5_K: Q4_K's lanes (same qs chunks at offset 48, same activation slice) plus the fifth bit of each element: qh byte l
// holds bit 2c for low-nibble element 64c + l and bit 2c + 1 for high-nibble element 64c + 32 + l, so every lane also
// takes all 32 qh bytes. src/es_quant.c:1153-1175.
template <> struct Lane<ES_HIP_Q5_K> : Lane<ES_HIP_Q4_K> {
    struct Raw { uint4 hdr, h0, h1, q0, q1; };
    static __device__ __forceinline__ void load_raw(const uint8_t *blk, int k, Raw &r) {
        r.hdr = ldw4(blk);
        r.h0 = ldw4(blk + 16);
        r.h1 = ldw4(blk + 32);
        r.q0 = ldw4(blk + 48 + 32 * k);
        r.q1 = ldw4(blk + 64 + 32 * k);
    }
    static __device__ __forceinline__ void unpack(const Raw &r, int k, Wt &w) {
        const uint32_t qq[8] = {r.q0.x, r.q0.y, r.q0.z, r.q0.w, r.q1.x, r.q1.y, r.q1.z, r.q1.w};
        const uint32_t hh[8] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w};
        for (int i = 0; i < 8; i++) {
            w.lo[i] = (qq[i] & 0x0f0f0f0fu) | (((hh[i] >> (2 * k)) & 0x01010101u) << 4);
            w.hi[i] = ((qq[i] >> 4) & 0x0f0f0f0fu) | (((hh[i] >> (2 * k + 1)) & 0x01010101u) << 4);
        }
        scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * k, w.sc0, w.mn0);
        scale_min(r.hdr.y, r.hdr.z, r.hdr.w, 2 * k + 1, w.sc1, w.mn1);
        w.d = half_bits_to_float(r.hdr.x);
        w.dmin = half_bits_to_float(r.hdr.x >> 16);
    }
    // s += y.d * (d * dot - dmin * mins). The reference has no AVX2 kernel for Q5_K: the x86 build runs the scalar mv_q5_K,
    // compiled without FMA, in every configuration. The whole product is rounded here, so the chain's add (fused with a
    // factor 1 or not) adds exactly that value in either order.
    static __device__ __forceinline__ Term2 term(const Wt &w, const Act &x, Ints v, bool) {
        const float in = w.d * static_cast<float>(v.dot) - w.dmin * static_cast<float>(v.aux);
        return {1.0f, x.d * in};
    }
};

// Q6_K: lane k of 4: half h = k/2, p = k%2. It takes ql[64h + 32p, +32) and qh[32h, +32); for j = 0, 1 the low nibbles
// of ql bytes 16j + [0,16) (with qh bits 2p, 2p+1) are group 8h + 2p + j, the high nibbles (qh bits 2p+4, 2p+5) group
// 8h + 2p + j + 4, where a group is 16 consecutive elements with one int8 scale. The 6-bit codes are dotted unsigned and
// corrected by 32 * bsums (the same integer as the signed form). src/es_quant.c:1081-1117, 1443-1469.
template <> struct Lane<ES_HIP_Q6_K> {
    // 32-byte fields at 2-byte aligned addresses are read as nine aligned dwords and realigned with v_alignbyte. All of it
    // lies inside the block: the block starts 4-byte aligned or 2 bytes past (then the dword before is the previous
    // block's), and the last field read here (d, offset 208) ends the block.
    struct Raw { uint4 l0, l1, h0, h1; uint32_t l8, h8, sel, sa, sb, d16; };
    struct Act { uint32_t y[4][4]; int bs[4]; float d; };   // groups g0, g0 + 1, g0 + 4, g0 + 5 with g0 = 8h + 2p
    struct Wt { uint32_t c[4][4]; int sc[4]; float d; };
    struct Ints { int dot, aux; };

    static __device__ __forceinline__ int grp(int k, int m) { return 8 * (k >> 1) + 2 * (k & 1) + (m & 1) + 4 * (m >> 1); }
    static __device__ __forceinline__ void load_act(const uint8_t *a, int k, Act &x) {
        x.d = ldg<float>(a);
#pragma unroll
        for (int m = 0; m < 4; m++) {
            const int g = grp(k, m);
            const uint4 v = ldg<uint4>(a + 4 + 16 * g);
            x.y[m][0] = v.x; x.y[m][1] = v.y; x.y[m][2] = v.z; x.y[m][3] = v.w;
            x.bs[m] = ldg<int16_t>(a + 260 + 2 * g);
        }
    }
    static __device__ __forceinline__ void zero_act(Act &x) {
        for (int m = 0; m < 4; m++) {
            for (int i = 0; i < 4; i++) x.y[m][i] = 0;
            x.bs[m] = 0;
        }
        x.d = 0.0f;
    }
    static __device__ __forceinline__ void load_raw(const uint8_t *blk, int k, Raw &r) {
        const int h = k >> 1, p = k & 1;
        const uintptr_t al = reinterpret_cast<uintptr_t>(blk + 64 * h + 32 * p);
        const uintptr_t ah = reinterpret_cast<uintptr_t>(blk + 128 + 32 * h);
        const uint8_t *bl = reinterpret_cast<const uint8_t *>(al & ~static_cast<uintptr_t>(3));
        const uint8_t *bh = reinterpret_cast<const uint8_t *>(ah & ~static_cast<uintptr_t>(3));
        r.sel = static_cast<uint32_t>(al & 3);   // same for both fields (offsets differ by multiples of 32)
        r.l0 = ldw4(bl);
        r.l1 = ldw4(bl + 16);
        r.l8 = ldg<uint32_t>(bl + 32);
        r.h0 = ldw4(bh);
        r.h1 = ldw4(bh + 16);
        r.h8 = ldg<uint32_t>(bh + 32);
        r.sa = ldg<uint16_t>(blk + 192 + 8 * h + 2 * p);       // scales of groups g0, g0 + 1
        r.sb = ldg<uint16_t>(blk + 192 + 8 * h + 2 * p + 4);   // g0 + 4, g0 + 5
        r.d16 = ldg<uint16_t>(blk + 208);
    }
    static __device__ __forceinline__ void unpack(const Raw &r, int k, Wt &w) {
        const uint32_t lw[9] = {r.l0.x, r.l0.y, r.l0.z, r.l0.w, r.l1.x, r.l1.y, r.l1.z, r.l1.w, r.l8};
        const uint32_t hw[9] = {r.h0.x, r.h0.y, r.h0.z, r.h0.w, r.h1.x, r.h1.y, r.h1.z, r.h1.w, r.h8};
        const int p = k & 1, sl = 2 * p, sh = 2 * p + 4;
#pragma unroll
        for (int j = 0; j < 2; j++) {
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t ql = alignbyte(lw[4 * j + i + 1], lw[4 * j + i], r.sel);
                const uint32_t qh = alignbyte(hw[4 * j + i + 1], hw[4 * j + i], r.sel);
                w.c[j][i] = (ql & 0x0f0f0f0fu) | (((qh >> sl) & 0x03030303u) << 4);
                w.c[2 + j][i] = ((ql >> 4) & 0x0f0f0f0fu) | (((qh >> sh) & 0x03030303u) << 4);
            }
        }
        w.sc[0] = static_cast<int8_t>(r.sa);
        w.sc[1] = static_cast<int8_t>(r.sa >> 8);
        w.sc[2] = static_cast<int8_t>(r.sb);
        w.sc[3] = static_cast<int8_t>(r.sb >> 8);
        w.d = half_bits_to_float(r.d16);
    }
    static __device__ __forceinline__ Ints ints(const Wt &w, const Act &x) {
        int dot = 0;
#pragma unroll
        for (int m = 0; m < 4; m++) {
            int s = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) s = sdot4(w.c[m][i], x.y[m][i], s);
            dot += w.sc[m] * (s - 32 * x.bs[m]);
        }
        return {dot, 0};
    }
    // s += y.d * d * tot   (src/es_quant.c:1114, 1466)
    static __device__ __forceinline__ Term2 term(const Wt &w, const Act &x, Ints v, bool) {
        return {x.d * w.d, static_cast<float>(v.dot)};
    }
};

// Q3_K: group g = 8n + 2j + half holds elements 16g + [0,16): bits 2j of qs[32n + 16half + l] and hmask[16half + l] bit
// 4n + j (absent: minus 4). Lane k of 4: n = k/2, half = k%2 takes qs[32n + 16half, +16) and hmask[16half, +16), and
// with them the four groups 8n + 2j + half, j = 0..3. The codes low2 + 4*hbit (0..7) are dotted unsigned and corrected by
// 4 * bsums; the 6-bit scales minus 32 come from the 12 packed bytes (src/es_quant.c:1120-1151, 1370-1394). Four lanes
// per block keep the loads per block low: each 16-byte field is read as five aligned dwords (the block is 4-byte aligned
// or 2 bytes past, as for Q6_K), the scales as three aligned dwords and a 2-byte load at 106; the last byte read is d's,
// at 109, inside the block.
template <> struct Lane<ES_HIP_Q3_K> {
    struct Raw { uint4 qv, hv; uint32_t q4, h4, s0, s1, s2, s106, d16, sel; };
    struct Act { uint32_t y[4][4]; int bs[4]; float d; };
    struct Wt { uint32_t c[4][4]; int sc[4]; float d; };
    struct Ints { int dot, aux; };

    static __device__ __forceinline__ void load_act(const uint8_t *a, int k, Act &x) {
        const int n = k >> 1, half = k & 1;
        x.d = ldg<float>(a);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int g = 8 * n + 2 * j + half;
            const uint4 v = ldg<uint4>(a + 4 + 16 * g);
            x.y[j][0] = v.x; x.y[j][1] = v.y; x.y[j][2] = v.z; x.y[j][3] = v.w;
            x.bs[j] = ldg<int16_t>(a + 260 + 2 * g);
        }
    }
    static __device__ __forceinline__ void zero_act(Act &x) {
        for (int j = 0; j < 4; j++) {
            for (int i = 0; i < 4; i++) x.y[j][i] = 0;
            x.bs[j] = 0;
        }
        x.d = 0.0f;
    }
    static __device__ __forceinline__ void load_raw(const uint8_t *blk, int k, Raw &r) {
        const int n = k >> 1, half = k & 1;
        const uintptr_t aq = reinterpret_cast<uintptr_t>(blk + 32 + 32 * n + 16 * half);
        const uintptr_t ah = reinterpret_cast<uintptr_t>(blk + 16 * half);
        const uintptr_t as = reinterpret_cast<uintptr_t>(blk + 96);
        const uint8_t *bq = reinterpret_cast<const uint8_t *>(aq & ~static_cast<uintptr_t>(3));
        const uint8_t *bh = reinterpret_cast<const uint8_t *>(ah & ~static_cast<uintptr_t>(3));
        const uint8_t *bs = reinterpret_cast<const uint8_t *>(as & ~static_cast<uintptr_t>(3));
        r.sel = static_cast<uint32_t>(aq & 3);   // the same for every field (their offsets differ by multiples of 16)
        r.qv = ldw4(bq);
        r.q4 = ldg<uint32_t>(bq + 16);
        r.hv = ldw4(bh);
        r.h4 = ldg<uint32_t>(bh + 16);
        r.s0 = ldg<uint32_t>(bs);
        r.s1 = ldg<uint32_t>(bs + 4);
        r.s2 = ldg<uint32_t>(bs + 8);
        r.s106 = ldg<uint16_t>(blk + 106);   // scale bytes 10, 11: the last aligned dword misses them when sel = 2
        r.d16 = ldg<uint16_t>(blk + 108);
    }
    static __device__ __forceinline__ void unpack(const Raw &r, int k, Wt &w) {
        const uint32_t q[4] = {alignbyte(r.qv.y, r.qv.x, r.sel), alignbyte(r.qv.z, r.qv.y, r.sel),
                               alignbyte(r.qv.w, r.qv.z, r.sel), alignbyte(r.q4, r.qv.w, r.sel)};
        const uint32_t h[4] = {alignbyte(r.hv.y, r.hv.x, r.sel), alignbyte(r.hv.z, r.hv.y, r.sel),
                               alignbyte(r.hv.w, r.hv.z, r.sel), alignbyte(r.h4, r.hv.w, r.sel)};
        // scale bytes 0-3, 4-7, 8-11
        const uint32_t S0 = alignbyte(r.s1, r.s0, r.sel), S1 = alignbyte(r.s2, r.s1, r.sel), S2 = alignbyte(r.s106, r.s2, r.sel);
        const int n = k >> 1, half = k & 1;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const uint32_t hs = h[i] >> (4 * n);   // bits j of every byte: the high bits of group j
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t hb = j <= 2 ? (hs << (2 - j)) & 0x04040404u : (hs >> 1) & 0x04040404u;
                w.c[j][i] = ((q[i] >> (2 * j)) & 0x03030303u) | hb;
            }
        }
        // group g = 8n + 2j + half: low nibble of byte g % 8 (bits 4n), high pair of byte 8 + g % 4 (bits 2(g / 4))
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int bl = 8 * (2 * (j & 1) + half);
            const uint32_t lo = ((j < 2 ? S0 : S1) >> (bl + 4 * n)) & 15u;
            const uint32_t hi = (S2 >> (bl + 2 * (2 * n + (j >> 1)))) & 3u;
            w.sc[j] = static_cast<int>(lo | (hi << 4)) - 32;
        }
        w.d = half_bits_to_float(r.d16);
    }
    static __device__ __forceinline__ Ints ints(const Wt &w, const Act &x) {
        int dot = 0;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            int s = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) s = sdot4(w.c[j][i], x.y[j][i], s);
            dot += w.sc[j] * (s - 4 * x.bs[j]);
        }
        return {dot, 0};
    }
    // s += y.d * d * tot   (src/es_quant.c:1147, 1391)
    static __device__ __forceinline__ Term2 term(const Wt &w, const Act &x, Ints v, bool) {
        return {x.d * w.d, static_cast<float>(v.dot)};
    }
};

// Q2_K: lane k of 4: half h = k/2, part = k%2. It takes qs[32h + 16part, +16); shift 2s of those bytes holds the 16
// elements 16g + [0,16) of group g = 8h + 2s + part (weight order of src/es_q2k.h:1-15), s = 0..3.
// isum = sum_g (sc[g] & 15) * sum q*y; summs = sum_g bsums[g] * (sc[g] >> 4). src/es_q2k.c:127-148,
// src/es_quant.c:1344-1368.
template <> struct Lane<ES_HIP_Q2_K> {
    struct Raw { uint4 q; uint2 sc; uint32_t dd; };
    struct Act { uint32_t y[4][4]; int bs[4]; float d; };
    struct Wt { uint32_t q[4]; int scl[4], mn[4]; float d, dmin; };
    struct Ints { int dot, aux; };

    static __device__ __forceinline__ void load_act(const uint8_t *a, int k, Act &x) {
        const int h = k >> 1, part = k & 1;
        x.d = ldg<float>(a);
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int g = 8 * h + 2 * s + part;
            const uint4 v = ldg<uint4>(a + 4 + 16 * g);
            x.y[s][0] = v.x; x.y[s][1] = v.y; x.y[s][2] = v.z; x.y[s][3] = v.w;
            x.bs[s] = ldg<int16_t>(a + 260 + 2 * g);
        }
    }
    static __device__ __forceinline__ void zero_act(Act &x) {
        for (int s = 0; s < 4; s++) {
            for (int i = 0; i < 4; i++) x.y[s][i] = 0;
            x.bs[s] = 0;
        }
        x.d = 0.0f;
    }
    static __device__ __forceinline__ void load_raw(const uint8_t *blk, int k, Raw &r) {
        const int h = k >> 1, part = k & 1;
        r.q = ldw4(blk + 16 + 32 * h + 16 * part);
        r.sc = ldg<uint2>(blk + 8 * h);   // scales[8h .. 8h+8): byte 2s + part is group 8h + 2s + part
        r.dd = ldg<uint32_t>(blk + 80);
    }
    static __device__ __forceinline__ void unpack(const Raw &r, int k, Wt &w) {
        const int part = k & 1;
        w.q[0] = r.q.x; w.q[1] = r.q.y; w.q[2] = r.q.z; w.q[3] = r.q.w;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const int byte = 2 * s + part;
            const uint32_t v = ((byte < 4 ? r.sc.x : r.sc.y) >> (8 * (byte & 3))) & 0xff;
            w.scl[s] = v & 15;
            w.mn[s] = v >> 4;
        }
        w.d = half_bits_to_float(r.dd);
        w.dmin = half_bits_to_float(r.dd >> 16);
    }
    static __device__ __forceinline__ Ints ints(const Wt &w, const Act &x) {
        int isum = 0, summs = 0;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            int p = 0;
#pragma unroll
            for (int i = 0; i < 4; i++) p = sdot4((w.q[i] >> (2 * s)) & 0x03030303u, x.y[s][i], p);
            isum += w.scl[s] * p;
            summs += x.bs[s] * w.mn[s];
        }
        return {isum, summs};
    }
    // s += dall*isum - dmin*summs with dall = y.d*d, dmin = y.d*dmin   (src/es_q2k.c:142-146, src/es_quant.c:1364-1365)
    static __device__ __forceinline__ Term2 term(const Wt &w, const Act &x, Ints v, bool contract) {
        const float dall = x.d * w.d, dmn = x.d * w.dmin;
        const float q = dmn * static_cast<float>(v.aux);
        const float in = contract ? __builtin_fmaf(dall, static_cast<float>(v.dot), -q) : dall * static_cast<float>(v.dot) - q;
        return {1.0f, in};   // chain: s + 1*in == s + in in both orders
    }
};

// Q4_0 / Q5_0 / Q8_0: one lane per 32-element block. AVX2 lane i of the reference sums elements 4i..4i+3 (one v_dot4
// here): lane_i = sum (code - offset) * y over those four elements, formed as dot(code, y) - offset * sum(y) (Q8_0: the
// stored int8 codes, offset 0). src/es_quant.c:1005-1055 (scalar), 1198-1221, 1252-1323 (AVX2).
template <int F> struct Lane32 {
    static constexpr int OFF = F == ES_HIP_Q4_0 ? 8 : F == ES_HIP_Q5_0 ? 16 : 0;   // Q8_0 codes are signed as stored
    // The block starts 2-aligned. A 16-byte load at the 4-aligned one of blk / blk+2 plus 2- and 4-byte loads for the
    // rest reads exactly the block's bytes.
    struct Raw { uint4 v, v2; uint32_t w4, u, par; };
    struct Act { uint32_t y[8]; int ns[8]; float d; };   // ns[i] = -OFF * (sum of the four bytes of y[i])
    struct Wt { uint32_t q[8]; float d; };
    struct Ints { int lane[8]; };

    static __device__ __forceinline__ void load_act(const uint8_t *a, int, Act &x) {
        x.d = ldg<float>(a);
        const uint4 v0 = ldg<uint4>(a + 4), v1 = ldg<uint4>(a + 20);
        x.y[0] = v0.x; x.y[1] = v0.y; x.y[2] = v0.z; x.y[3] = v0.w;
        x.y[4] = v1.x; x.y[5] = v1.y; x.y[6] = v1.z; x.y[7] = v1.w;
        for (int i = 0; i < 8; i++) x.ns[i] = -OFF * sdot4(0x01010101u, x.y[i], 0);
    }
    static __device__ __forceinline__ void zero_act(Act &x) {
        for (int i = 0; i < 8; i++) { x.y[i] = 0; x.ns[i] = 0; }
        x.d = 0.0f;
    }
    static __device__ __forceinline__ void load_raw(const uint8_t *blk, int, Raw &r) {
        r.par = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(blk) & 2);
        r.v = ldw4(blk + r.par);
        if constexpr (F == ES_HIP_Q8_0) {   // d f16 @0, int8 qs[32] @2: 34 bytes as 16 + 16 + 2
            r.v2 = ldw4(blk + r.par + 16);
            r.w4 = 0;
            r.u = ldg<uint16_t>(r.par ? blk : blk + 32);
        } else if constexpr (F == ES_HIP_Q4_0) {   // d f16 @0, qs[16] @2
            r.w4 = 0;
            r.u = ldg<uint16_t>(r.par ? blk : blk + 16);
        } else {                            // d f16 @0, qh u32 @2, qs[16] @6
            r.w4 = ldg<uint32_t>(blk + r.par + 16);
            r.u = ldg<uint16_t>(r.par ? blk : blk + 20);
        }
    }
    static __device__ __forceinline__ void unpack(const Raw &r, int, Wt &w) {
        uint32_t qs[4], d16, qh = 0;
        const uint4 v = r.v;
        if constexpr (F == ES_HIP_Q8_0) {
            const uint32_t s[9] = {v.x, v.y, v.z, v.w, r.v2.x, r.v2.y, r.v2.z, r.v2.w, r.u};
            if (r.par == 0) {
                d16 = v.x;
#pragma unroll
                for (int i = 0; i < 8; i++) w.q[i] = alignbyte(s[i + 1], s[i], 2);
            } else {
                d16 = r.u;
#pragma unroll
                for (int i = 0; i < 8; i++) w.q[i] = s[i];
            }
            w.d = half_bits_to_float(d16);
            return;
        }
        if constexpr (F == ES_HIP_Q4_0) {
            if (r.par == 0) {
                d16 = v.x;
                qs[0] = alignbyte(v.y, v.x, 2); qs[1] = alignbyte(v.z, v.y, 2);
                qs[2] = alignbyte(v.w, v.z, 2); qs[3] = alignbyte(r.u, v.w, 2);
            } else {
                d16 = r.u;
                qs[0] = v.x; qs[1] = v.y; qs[2] = v.z; qs[3] = v.w;
            }
        } else {
            if (r.par == 0) {
                d16 = v.x;
                qh = alignbyte(v.y, v.x, 2);
                qs[0] = alignbyte(v.z, v.y, 2); qs[1] = alignbyte(v.w, v.z, 2);
                qs[2] = alignbyte(r.w4, v.w, 2); qs[3] = alignbyte(r.u, r.w4, 2);
            } else {
                d16 = r.u;
                qh = v.x;
                qs[0] = v.y; qs[1] = v.z; qs[2] = v.w; qs[3] = r.w4;
            }
        }
        for (int i = 0; i < 4; i++) { w.q[i] = qs[i] & 0x0f0f0f0fu; w.q[i + 4] = (qs[i] >> 4) & 0x0f0f0f0fu; }
        if constexpr (F == ES_HIP_Q5_0) {   // fifth bit of element e is bit e of qh
            for (int i = 0; i < 8; i++) {
                const uint32_t nib = (qh >> (4 * i)) & 15u;
                w.q[i] |= ((nib * 0x00204081u) & 0x01010101u) << 4;
            }
        }
        w.d = half_bits_to_float(d16);
    }
    static __device__ __forceinline__ Ints ints(const Wt &w, const Act &x) {
        Ints v;
        for (int i = 0; i < 8; i++) v.lane[i] = sdot4(w.q[i], x.y[i], x.ns[i]);
        return v;
    }
};
template <> struct Lane<ES_HIP_Q4_0> : Lane32<ES_HIP_Q4_0> {};
template <> struct Lane<ES_HIP_Q5_0> : Lane32<ES_HIP_Q5_0> {};
template <> struct Lane<ES_HIP_Q8_0> : Lane32<ES_HIP_Q8_0> {};

template <int F> constexpr bool is32() { return F == ES_HIP_Q4_0 || F == ES_HIP_Q5_0 || F == ES_HIP_Q8_0; }

// units whose raw loads a wave issues together (a power of two): ESQ_UNITS, fewer where a lane's unit (Q6_K, Q3_K: four
// and three realigned fields) or the activation slices held for NT activations are large enough that more would cost
// resident waves
template <int F, int NT> constexpr int units() {
    if constexpr (F == ES_HIP_Q6_K || F == ES_HIP_Q3_K) return NT == 1 ? Q6K_UNITS1 : Q6K_UNITSN;
    else if constexpr (!is32<F>()) return NT == 1 ? ESQ_UNITS : K_UNITSN;
    else return ESQ_UNITS;
}
// units of the one- and two-wide bodies of mv_kernel_mixed (0: as units())
template <int F, int NT> constexpr int units_mixed() {
    if constexpr (F == ES_HIP_Q6_K || F == ES_HIP_Q3_K) return NT == 1 ? Q6K_UNITS1M : Q6K_UNITS2M;
    else if constexpr (F == ES_HIP_Q4_K) return NT == 1 ? 0 : K_UNITS2M;   // (measured for Q4_K; Q5_K's grew past 168 VGPRs)
    else return 0;
}

// ---------------------------------------------------------------------------------------------------------------------
// The kernel

// W waves per workgroup. A row of nbk blocks is cut into seg = ceil(nbk / slots) segments of `slots` blocks, one wave
// each, so every lane keeps one fixed block position and its activation slice stays in registers; when seg < W the
// W / seg wave groups take different rows, and when seg > W each wave takes seg / W segments in turn (reloading its
// activation slices for each). All waves write their blocks' float terms to the workgroup's LDS, then the
// whole workgroup runs the per-row chains. order: ES_HIP_ORDER_*; NT activations per pass. One workgroup per tile
// (rows_per_wg rows of one job).
template <int F, int NT, int W, bool SEGLOOP, int UO = 0>
__device__ __forceinline__ void mv_body(const MvJob &J, int order) {
    using L = Lane<F>;
    constexpr int LPB = Fmt<F>::LPB, BE = Fmt<F>::BE, BB = Fmt<F>::BB, AB = Fmt<F>::AB;
    constexpr int SLOTS = WAVE / LPB;
    constexpr bool W32 = is32<F>();
    constexpr int U = UO ? UO : units<F, NT>();   // row passes whose raw loads a wave issues before using any of them

    const int nbk = J.cols / BE;
    const int tile = blockIdx.x - J.tile0;
    const int ra0 = J.r0 + tile * J.rows_per_wg;
    const int rend = min(ra0 + J.rows_per_wg, J.r1);
    const uint8_t *const dummy = J.W + (size_t)J.r0 * J.row_bytes;   // a valid block for lanes with nothing to load

    const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
    const int slot = lane / LPB, k = lane % LPB;
    int seg = 1;                                      // groups of SLOTS blocks per row, a power of two
    while (seg * SLOTS < nbk) seg <<= 1;
    const int segw = seg < W ? seg : W;               // waves per row
    const int spw = SEGLOOP ? seg / segw : 1;         // groups per wave: rows of more than W groups give each wave
                                                      // groups my_seg, my_seg + W, ... in turn (SEGLOOP launches)
    const int my_seg = wave % segw, rowgrp = wave / segw, nrowgrp = W / segw;
    int rpi, rowoff, b;
    if (nbk <= SLOTS) { rpi = SLOTS / nbk; rowoff = slot / nbk; b = slot % nbk; }
    else { rpi = 1; rowoff = 0; b = my_seg * SLOTS + slot; }
    bool live = rowoff < rpi && b < nbk;
    const int rstep = nrowgrp * rpi;                  // rows advanced by one pass of the whole workgroup
    const int rfirst = rowgrp * rpi + rowoff;

    const bool x86 = order != ES_HIP_ORDER_SCALAR;
    const bool contract = order == ES_HIP_ORDER_X86_CONTRACT;
    const int cmode = W32 ? (x86 ? CH_LANES : CH_MULADD) : (contract ? CH_FMA : CH_MULADD);
    constexpr int CW = W32 ? 9 : 2;   // floats per (row, block, activation) in LDS
    // LDS row pitch of the terms, [row][block][activation][CW]: odd for the K-quants, whose chains take one row per lane,
    // so consecutive rows' terms sit in consecutive banks (an even pitch of 16 or 64 floats put every row of a wave in one
    // or two banks)
    const int P = mv_row_pitch(W32, nbk, NT);
    extern __shared__ float lds[];

    typename L::Raw raw[U];
    bool ok[U];
    // the first unit batch's weight loads go out before the activation loads, so their latencies overlap (Q4_K at one
    // activation per pass; elsewhere keeping these registers live across the activation loads cost more than it saved)
    constexpr bool PRE = NT == 1 && F == ES_HIP_Q4_K;
    bool pre = PRE && ra0 < rend;
    if (pre) {
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int row = ra0 + rfirst + u * rstep;
            ok[u] = live && row < min(ra0 + J.chain_rows, rend);
            L::load_raw(ok[u] ? J.W + (size_t)row * J.row_bytes + (size_t)b * BB : dummy, k, raw[u]);
        }
    }
    for (int t0 = 0; t0 < J.na; t0 += NT) {
        const int nt = min(NT, J.na - t0);
        typename L::Act act[NT];
        auto load_acts = [&]() {   // the activation slices of this lane's block position b
#pragma unroll
            for (int t = 0; t < NT; t++) {
                if (live && t < nt) {
                    const int q = J.arow ? ldg<int>(J.arow + t0 + t) : t0 + t;
                    L::load_act(J.act + (size_t)q * J.astride + (size_t)b * AB, k, act[t]);
                }
                else L::zero_act(act[t]);
            }
        };
        if (spw == 1) load_acts();

        for (int ra = ra0; ra < rend; ra += J.chain_rows) {
            const int rb = min(ra + J.chain_rows, rend);
            for (int si = 0; si < spw; si++) {
                if (spw > 1) {   // the wave's next group of blocks: its block position and activation slices
                    b = (my_seg + si * W) * SLOTS + slot;
                    live = b < nbk;
                    load_acts();
                }
                // ---- phase 1: integers per block, float terms to LDS
                for (int r0 = ra + rfirst; r0 - rowoff < rb; r0 += U * rstep) {
                    if (!pre) {
#pragma unroll
                        for (int u = 0; u < U; u++) {
                            const int row = r0 + u * rstep;
                            ok[u] = live && row < rb;
                            L::load_raw(ok[u] ? J.W + (size_t)row * J.row_bytes + (size_t)b * BB : dummy, k, raw[u]);
                        }
                    }
                    pre = false;
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        const int row = r0 + u * rstep;
                        typename L::Wt w;
                        L::unpack(raw[u], k, w);
                        typename L::Ints v[NT];
#pragma unroll
                        for (int t = 0; t < NT; t++) {   // activations past nt (a uniform bound) are skipped
                            if (t < nt) v[t] = ok[u] ? L::ints(w, act[t]) : typename L::Ints{};
                            else v[t] = typename L::Ints{};
                        }
                        if constexpr (!W32) {
#pragma unroll
                            for (int t = 0; t < NT; t++)
                                if (t < nt) { v[t].dot = group_sum<LPB>(v[t].dot); v[t].aux = group_sum<LPB>(v[t].aux); }
                        }
                        if (ok[u] && k == 0) {
                            float *e = lds + (size_t)(row - ra) * P + (size_t)b * NT * CW;
                            if constexpr (W32) {
#pragma unroll
                                for (int t = 0; t < NT; t++) {
                                    if (t >= nt) continue;
                                    e[t * CW] = w.d * act[t].d;
                                    if (cmode == CH_LANES) {
                                        for (int i = 0; i < 8; i++) e[t * CW + 1 + i] = static_cast<float>(v[t].lane[i]);
                                    } else {
                                        int a = 0;
                                        for (int i = 0; i < 8; i++) a += v[t].lane[i];
                                        e[t * CW + 1] = static_cast<float>(a);
                                    }
                                }
                                if (J.ints && t0 == 0) {
                                    int a = 0;
                                    for (int i = 0; i < 8; i++) a += v[0].lane[i];
                                    stg<int32_t>(J.ints + (size_t)row * nbk + b, a);
                                    stg<int32_t>(J.ints_aux + (size_t)row * nbk + b, 0);
                                }
                            } else {
#pragma unroll
                                for (int t = 0; t < NT; t++) {
                                    if (t >= nt) continue;
                                    const Term2 tm = L::term(w, act[t], v[t], contract);
                                    e[t * CW] = tm.a;
                                    e[t * CW + 1] = tm.b;
                                }
                                if (J.ints && t0 == 0) {
                                    stg<int32_t>(J.ints + (size_t)row * nbk + b, v[0].dot);
                                    stg<int32_t>(J.ints_aux + (size_t)row * nbk + b, v[0].aux);
                                }
                            }
                        }
                    }
                }
            }
            __syncthreads();
            // ---- phase 2: the reference's sequential accumulation over the row's blocks, terms read 8 blocks ahead
            const int nrow = rb - ra;
            const int per = cmode == CH_LANES ? 8 : 1;
            for (int idx = tid; idx < nrow * nt * per; idx += WAVE * W) {
                // K-quants: rows fastest (consecutive lanes read consecutive banks through the odd pitch); 32-element
                // formats: a row's eight AVX2 chains (per = 8) in consecutive lanes, then activations, then rows
                int i, t, rl;
                if constexpr (!W32) {
                    i = 0;
                    t = 0;
#pragma unroll
                    for (int q = 1; q < NT; q++) t += idx >= q * nrow ? 1 : 0;   // idx / nrow for idx < NT * nrow
                    rl = idx - t * nrow;
                } else {
                    i = idx % per;
                    t = (idx / per) % nt;
                    rl = idx / (per * nt);
                }
                const float *e = lds + (size_t)rl * P + t * CW;
                const int oa = cmode == CH_LANES ? 1 + i : 0, ob = cmode == CH_LANES ? 0 : 1;
                float s = 0.0f;
                size_t lane_at = 0;
                if constexpr (SEGLOOP) {   // (column pieces of long rows run on the SEGLOOP launches only)
                    lane_at = ((size_t)(t0 + t) * (J.r1 - J.r0) + (ra + rl - J.r0)) * 8 + i;
                    if (J.chain & MV_CHAIN_IN)   // a later piece of a long row: the chains so far
                        s = cmode == CH_LANES ? ldg<float>(J.lanes + lane_at) : ldg<float>(J.y + (size_t)(t0 + t) * J.ystride + ra + rl);
                }
                int bb = 0;
                for (; bb + 8 <= nbk; bb += 8) {
                    float ta[8], tb[8];
#pragma unroll
                    for (int q = 0; q < 8; q++) { ta[q] = e[(bb + q) * NT * CW + oa]; tb[q] = e[(bb + q) * NT * CW + ob]; }
                    if (cmode == CH_MULADD) {
#pragma unroll
                        for (int q = 0; q < 8; q++) s = s + ta[q] * tb[q];   // -ffp-contract=off: two roundings
                    } else {
#pragma unroll
                        for (int q = 0; q < 8; q++) s = __builtin_fmaf(ta[q], tb[q], s);
                    }
                }
                for (; bb < nbk; bb++) {
                    const float ta = e[bb * NT * CW + oa], tb = e[bb * NT * CW + ob];
                    s = cmode == CH_MULADD ? s + ta * tb : __builtin_fmaf(ta, tb, s);
                }
                if constexpr (SEGLOOP) {
                    if (J.chain & MV_CHAIN_LANES_OUT) {   // the eight chains continue in the next piece
                        stg<float>(J.lanes + lane_at, s);
                        continue;
                    }
                }
                if (cmode == CH_LANES) {   // hsum_ps of the eight lanes: ((0+4)+(2+6))+((1+5)+(3+7))  (src/es_quant.c:1185-1187)
                    s = s + __shfl_xor(s, 4);
                    s = s + __shfl_xor(s, 2);
                    s = s + __shfl_xor(s, 1);
                }
                if (i == 0 && t < nt) stg<float>(J.y + (size_t)(t0 + t) * J.ystride + ra + rl, s);
            }
            __syncthreads();
        }
    }
}

template <int F, int NT, int W, bool SEGLOOP>
__global__ __launch_bounds__(WAVE * W, ESQ_MIN_WAVES) void mv_kernel(const MvJob *__restrict__ jobs, int njobs, MvJob single,
                                                                     int order) {
    MvJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    mv_body<F, NT, W, SEGLOOP>(J, order);
}

// A launch whose jobs take different activations per pass (J.nt: 1, 2 or 4), e.g. an MoE layer's experts at 1 to 8
// tokens each: every job runs the body compiled for its own pass width (a single expert's token no longer runs in a
// four-wide pass with its fewer loads in flight).
template <int F, int W, bool SEGLOOP>
__global__ __launch_bounds__(WAVE * W, ESQ_MIN_WAVES) void mv_kernel_mixed(const MvJob *__restrict__ jobs, int njobs,
                                                                           MvJob single, int order) {
    MvJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    switch (J.nt) {
    case 1: mv_body<F, 1, W, SEGLOOP, units_mixed<F, 1>()>(J, order); break;
    case 2: mv_body<F, 2, W, SEGLOOP, units_mixed<F, 2>()>(J, order); break;
    default: mv_body<F, 4, W, SEGLOOP>(J, order); break;
    }
}

}  // namespace esq

// ---------------------------------------------------------------------------------------------------------------------
// Launch glue (called from es_hip_quant.hip)

namespace esq {

using MvFn = void (*)(const MvJob *, int, MvJob, int);

// Only the (NT, W) pairs the planner uses are instantiated.
template <int F, int NT> static MvFn pick_w(int w, bool seg_loop) {
    switch (w) {
    case 4: return seg_loop ? nullptr : mv_kernel<F, NT, 4, false>;
    case 8: return seg_loop ? mv_kernel<F, NT, 8, true> : mv_kernel<F, NT, 8, false>;
    }
    return nullptr;
}
template <int F> static MvFn pick_nt(int nt, int w, bool seg_loop) {
    switch (nt) {
    case 0:   // per-job pass widths
        if (w == 4) return seg_loop ? nullptr : mv_kernel_mixed<F, 4, false>;
        if (w == 8) return seg_loop ? mv_kernel_mixed<F, 8, true> : mv_kernel_mixed<F, 8, false>;
        return nullptr;
    case 1: return pick_w<F, 1>(w, seg_loop);
    case 2: return pick_w<F, 2>(w, seg_loop);
    case 4: return pick_w<F, 4>(w, seg_loop);
    }
    return nullptr;
}

hipError_t mv_launch(const MvLaunch &L, const MvJob *jobs, int njobs, const MvJob &single, int order, hipStream_t s) {
    MvFn fn = nullptr;
    switch (L.type) {
    case ES_HIP_Q4_0: fn = pick_nt<ES_HIP_Q4_0>(L.nt, L.waves, L.seg_loop); break;
    case ES_HIP_Q5_0: fn = pick_nt<ES_HIP_Q5_0>(L.nt, L.waves, L.seg_loop); break;
    case ES_HIP_Q8_0: fn = pick_nt<ES_HIP_Q8_0>(L.nt, L.waves, L.seg_loop); break;
    case ES_HIP_Q2_K: fn = pick_nt<ES_HIP_Q2_K>(L.nt, L.waves, L.seg_loop); break;
    case ES_HIP_Q3_K: fn = pick_nt<ES_HIP_Q3_K>(L.nt, L.waves, L.seg_loop); break;
    case ES_HIP_Q4_K: fn = pick_nt<ES_HIP_Q4_K>(L.nt, L.waves, L.seg_loop); break;
    case ES_HIP_Q5_K: fn = pick_nt<ES_HIP_Q5_K>(L.nt, L.waves, L.seg_loop); break;
    case ES_HIP_Q6_K: fn = pick_nt<ES_HIP_Q6_K>(L.nt, L.waves, L.seg_loop); break;
    }
    if (!fn) return hipErrorInvalidValue;
    if (L.lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(fn), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(L.lds));
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(fn, dim3(L.grid), dim3(WAVE * L.waves), L.lds, s, jobs, njobs, single, order);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------------------------------------------------
// Batched 32-wide formats (Q4_0 / Q5_0 against 2..64 activations): one lane per (row, activation) runs that output's whole
// chain over the row's blocks in registers, so there are no LDS terms and no second phase. The lanes of a wave take
// ta consecutive activations (a power of two) of 64 / ta consecutive rows; lanes of one row read the same weight block
// (one memory transaction), the activation blocks come from L2. The next block is loaded while one is computed.
// x86 order: the eight AVX2 lane sums of a block go into eight fused chains acc_i = fma(lane_i, d*yd, acc_i), summed at
// the end as ((0+4)+(2+6))+((1+5)+(3+7)) (src/es_quant.c:1185-1187, 1252-1323); scalar order: s = s + (d*yd)*sum
// (src/es_quant.c:1013-1055).
template <int F>
__global__ __launch_bounds__(256) void mb32_kernel(const MbJob *__restrict__ jobs, int njobs, MbJob single, int order) {
    using L = Lane32<F>;
    constexpr int BB = Fmt<F>::BB, AB = Fmt<F>::AB;
    MbJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int rows_per_wave = 64 / J.ta;
    const int row = J.r0 + ((blockIdx.x - J.tile0) * 4 + wave) * rows_per_wave + lane / J.ta;
    const int t = J.t0 + lane % J.ta;
    const bool live = row < J.r1 && t < J.na;
    const int nbk = J.cols / 32;
    const uint8_t *wrow = J.W + (size_t)min(row, J.r1 - 1) * J.row_bytes;
    const int tq = min(t, J.na - 1);
    const uint8_t *arow = J.act + (size_t)(J.arow ? ldg<int>(J.arow + tq) : tq) * J.astride;
    const bool x86 = order != ES_HIP_ORDER_SCALAR;

    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0}, s = 0.0f;
    typename L::Raw raw;
    typename L::Act x;
    L::load_raw(wrow, 0, raw);
    L::load_act(arow, 0, x);
    for (int b = 0; b < nbk; b++) {
        typename L::Wt w;
        L::unpack(raw, 0, w);
        const typename L::Act xc = x;
        if (b + 1 < nbk) {   // the next block's bytes in flight
            L::load_raw(wrow + (size_t)(b + 1) * BB, 0, raw);
            L::load_act(arow + (size_t)(b + 1) * AB, 0, x);
        }
        const typename L::Ints v = L::ints(w, xc);
        const float dy = w.d * xc.d;
        if (x86) {
#pragma unroll
            for (int i = 0; i < 8; i++) acc[i] = __builtin_fmaf(static_cast<float>(v.lane[i]), dy, acc[i]);
        } else {
            int a = 0;
#pragma unroll
            for (int i = 0; i < 8; i++) a += v.lane[i];
            s = s + dy * static_cast<float>(a);
        }
    }
    if (x86) s = ((acc[0] + acc[4]) + (acc[2] + acc[6])) + ((acc[1] + acc[5]) + (acc[3] + acc[7]));
    if (live) stg<float>(J.y + (size_t)t * J.ystride + row, s);
}

hipError_t mb32_launch(int type, const MbJob *jobs, int njobs, const MbJob &single, int grid, int order, hipStream_t s) {
    if (type == ES_HIP_Q4_0)
        hipLaunchKernelGGL(mb32_kernel<ES_HIP_Q4_0>, dim3(grid), dim3(256), 0, s, jobs, njobs, single, order);
    else if (type == ES_HIP_Q5_0)
        hipLaunchKernelGGL(mb32_kernel<ES_HIP_Q5_0>, dim3(grid), dim3(256), 0, s, jobs, njobs, single, order);
    else if (type == ES_HIP_Q8_0)
        hipLaunchKernelGGL(mb32_kernel<ES_HIP_Q8_0>, dim3(grid), dim3(256), 0, s, jobs, njobs, single, order);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace esq
