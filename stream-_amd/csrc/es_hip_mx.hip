// Expert-sized Q2_K products on the int8 matrix cores, reading the activations' Q8_K rows directly (no pre-pass): the
// form of es_matvec_multi (src/es_quant.c:1818-1850, 1344-1368; src/es_q2k.c:127-148) for a MoE expert's few to few tens
// of activations (config 4: 128 tokens over 64 experts, top 8, about 16 per expert).
//
// Work split. A workgroup of 4 waves takes MX_ROWS = 256 rows x MX_TOK = 32 activations: two 16-activation MFMA tiles, the
// second skipped (wave-uniform) when 16 or fewer activations are left. Every activation value, bsum and scale of the
// tile's whole row (at most NBKM superblocks) is copied into LDS once, at the start (the activations the tile has: 16 or
// 32); after that one barrier each wave streams its rows' superblocks from HBM into registers, one superblock ahead per
// row group (the first already in flight while the activations are copied), with no further barrier.
// Wave w owns the four row groups 16 (4j + w) .. + 15 (j = 0..3) and runs superblock-major: superblock b of its four row
// groups in turn, so the A operands of superblock b, read from LDS once, serve four row groups.
//
// LDS (NBKM superblocks): values [b][32][256] (activation t's 16-byte chunk c at position c ^ (t & 15), so the 16 lanes
// that read chunk c of 16 activations hit 16 different bank groups), bsums as halves [b][lg][32][4] (k group lg holds
// bsums 4lg .. 4lg + 3: exact, |bsums| <= 16 * 127), scales [b][32]. Values go from the Q8_K rows straight into LDS with
// global_load_lds_dwordx4 (the swizzle in the per-lane source offsets); bsums and scales pass through registers.
//
// B operands (weights). Q2_K element order (src/es_q2k.h:1-15): group g = 8n + 2j + half holds bits 2j of
// qs[32n + 16 half + l], l = 0..15, with the scale byte scales[g] (low nibble sc, high nibble min). Slice s and lane group
// lg take g = 8 (lg >> 1) + 2s + (lg & 1): the lane's 16 qs bytes 16 lg .. 16 lg + 15 at shift 2s, against the natural
// 16-element chunk g of the activation row. One int8 plane q * sc (<= 45): isum = D exactly. summs = sum_g bsums_g * min_g
// through one v_mfma_f32_16x16x16_f16 (k positions 4lg .. 4lg + 3 meet bsums 4lg .. 4lg + 3; mins <= 15 and the bsums are
// exact halves, every partial sum an integer below 2^24: exact).
//
// MFMA operands: A = activations (16 x 64 k), B = weights (64 k x 16 rows): D[activation][row] sits in lane l, register i
// as activation 4 (l / 16) + i of the tile and row l % 16, the row whose weights the lane unpacked, so d and dmin need no
// cross-lane moves. Each item's epilogue runs one item later (under the next item's matrix work).
//
// Epilogue per (row, activation) and superblock, in superblock order (src/es_q2k.c:142-146, src/es_quant.c:1364-1365):
// dall = y.d * d, dmin = y.d * dmin, s += dall * isum - dmin * summs, with the product and difference fused as the clang
// build fuses them (s + fma(dall, isum, -(dmin * summs))) or every operation rounded (the gcc and portable builds).
#include "es_hip_common.h"
#include "es_hip_expf.h"

namespace esq {
namespace {

constexpr int MX_WAVES = MX_ROWS / 64, MX_RG = 4;
static_assert((MX_WAVES == 4 || MX_WAVES == 8) && MX_TOK == 32, "four row groups per wave, two activation tiles");
// LDS bytes per superblock: values, bsums, scales
constexpr int XV = MX_TOK * 256, XB = 4 * MX_TOK * 8, XD = MX_TOK * 4;

typedef _Float16 v4h __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_a4 __attribute__((ext_vector_type(2), aligned(4)));

template <typename T> __device__ __forceinline__ T lds_ld(uint32_t a) {
    return *reinterpret_cast<const __attribute__((address_space(3))) T *>(a);
}

struct WRaw {      // this lane's bytes of one row's superblock: qs chunk lg, scale dwords 2 (lg >> 1) and + 1, d | dmin
    uint4 q;
    uint32_t s0, s1, dd;
};
struct BOps {
    v4i q[4];
    v4h mn;
    float d, dm;
};
struct AOps {      // one activation tile's operands for one superblock
    v4i x[4];
    v4h bs;
    v4f yd;        // y.d of activations 4 lg .. 4 lg + 3 of the tile
};
struct MRes {
    v4i i;
    v4f m;
};

__device__ __forceinline__ void build_b(const WRaw &w, int lg, BOps &B) {
    // slice s: scale byte g = 8 (lg >> 1) + 2s + (lg & 1), i.e. byte 2 (s & 1) + (lg & 1) of scale dword 2 (lg >> 1) + (s >> 1),
    // put into both 16-bit halves for the byte-pair multiplies
    const uint32_t selA = 0x0c000c00u + (uint32_t)(lg & 1) * 0x00010001u, selB = selA + 0x00020002u;
    const uint32_t scw[4] = {__builtin_amdgcn_perm(0, w.s0, selA) & 0x000f000fu, __builtin_amdgcn_perm(0, w.s0, selB) & 0x000f000fu,
                             __builtin_amdgcn_perm(0, w.s1, selA) & 0x000f000fu, __builtin_amdgcn_perm(0, w.s1, selB) & 0x000f000fu};
    const uint32_t qa[4] = {w.q.x, w.q.y, w.q.z, w.q.w};
#pragma unroll
    for (int s = 0; s < 4; s++)
#pragma unroll
        for (int i = 0; i < 4; i++) B.q[s][i] = (int)pk_mul_u16((qa[i] >> (2 * s)) & 0x03030303u, scw[s]);   // <= 45
    // mins of groups 4lg .. 4lg + 3: the high nibbles of scale dword lg (= 2 (lg >> 1) + (lg & 1)), as halves built as
    // 1024 + m (byte m under the exponent of 1024) with 1024 subtracted exactly
    const uint32_t mw = ((lg & 1) ? w.s1 : w.s0) >> 4 & 0x0f0f0f0fu;
    const h2 m1024 = __builtin_bit_cast(h2, 0xe400e400u);
    const h2 a = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, mw, 0x04010400u)) + m1024;
    const h2 b = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, mw, 0x04030402u)) + m1024;
    B.mn = v4h{a[0], a[1], b[0], b[1]};
    B.d = half_bits_to_float(w.dd);
    B.dm = half_bits_to_float(w.dd >> 16);
}

__device__ __forceinline__ void mma(const AOps &a, const BOps &B, MRes &m) {
    m.i = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.x[0], B.q[0], v4i{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
    for (int s = 1; s < 4; s++) m.i = __builtin_amdgcn_mfma_i32_16x16x64_i8(a.x[s], B.q[s], m.i, 0, 0, 0);
    m.m = __builtin_amdgcn_mfma_f32_16x16x16f16(a.bs, B.mn, v4f{0, 0, 0, 0}, 0, 0, 0);
}

template <bool CONTRACT> __device__ __forceinline__ void epilogue(const MRes &m, float d, float dm, const v4f &yd, v4f &s) {
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float dall = yd[i] * d, dmn = yd[i] * dm;
        const float q = dmn * m.m[i];   // summs: an exact integer in the f32 accumulator
        if constexpr (CONTRACT) s[i] = s[i] + __builtin_fmaf(dall, static_cast<float>(m.i[i]), -q);
        else s[i] = s[i] + (dall * static_cast<float>(m.i[i]) - q);
    }
}

// GATED: the gate and up products of one expert in one workgroup of eight waves (waves 0-3 the gate's 256 rows, waves 4-7
// the up's same rows, each half split over its waves as the four-wave form splits its tile), followed by h = g / (1 +
// expf(-g)) * u (src/es_engine.c:913) and h's requantization to Q8_K blocks (src/es_q2k.c:102-125) for the down product:
// the tile's 256 rows are one block of h, so its absolute maximum, scale, values and bsums are all formed in the
// workgroup. Gate wave w and up wave 4 + w hold the same rows and activations in the same lanes and registers; each
// forms h for half of its row groups, taking the partner's values of that half through LDS. The per-activation maxima
// over the eight waves meet in LDS, the blocks are assembled in LDS and written as dwords. Every float operation and the order of the integer sums are those of the
// separate SwiGLU kernel (es_hip_moe.hip), so the blocks are bit-identical to its.
template <int NBKM, bool CONTRACT, bool GATHER, bool GATED>
__global__ __launch_bounds__(GATED ? 512 : 64 * MX_WAVES, !GATED && NBKM <= 8 && MX_WAVES == 4 ? 2 : 1) void mx_q2k_kernel(
    const MkJob *__restrict__ jobs, int njobs, MkJob single) {
    constexpr int NW = GATED ? 8 : MX_WAVES;       // waves of the workgroup
    constexpr int RW = GATED ? 4 : MX_WAVES;       // waves that split one product's rows
    constexpr int TROWS = 64 * RW;                 // rows of the tile
    constexpr uint32_t V0 = 0, BS0 = NBKM * XV, D0 = BS0 + NBKM * XB;
    constexpr uint32_t LDS_BYTES = NBKM * (XV + XB + XD) > 32 * 1024 + MX_TOK * 292 + 8 * MX_TOK * 4
                                       ? NBKM * (XV + XB + XD) : 32 * 1024 + MX_TOK * 292 + 8 * MX_TOK * 4;
    __shared__ __align__(16) uint8_t smem[GATED ? LDS_BYTES : NBKM * (XV + XB + XD)];
    __shared__ uint64_t xtab[GATED ? 32 : 1];   // expf's table (the gated epilogue)

    MkJob J;
    if (jobs) J = load_tile_job(jobs, njobs, blockIdx.x);
    else J = single;
    // tiles: row tile rt, activation tile tt. With several activation tiles, ids go round-robin over the 8 XCDs (id % 8)
    // with all activation tiles of row tile rt on ids with id % 8 == rt % 8 (one XCD's L2 serves the repeated weight
    // reads); each job's tiles then start at a multiple of 8 and ids past the last row tile exit at once.
    const int tile = blockIdx.x - J.tile0;
    int rt = tile, tt = 0;
    if (J.ntok_tiles > 1) {
        const int xcd = tile & 7, kq = tile >> 3;
        rt = xcd + 8 * (kq / J.ntok_tiles);
        tt = kq % J.ntok_tiles;
    }
    if (rt * TROWS >= J.r1 - J.r0) return;
    const int row0 = J.r0 + rt * TROWS, tok0 = tt * MX_TOK;
    const bool two = J.na - tok0 > 16;   // the second 16-activation tile has activations
    const int nbk = J.cols / 256;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int lr = lane & 15, lg = lane >> 4;
    const int wq = wave % RW;                     // this wave's share of its product's rows
    if constexpr (GATED) {
        static constexpr uint64_t T_[32] = ESQ_EXPF_TABLE;
        if (tid < 32) xtab[tid] = T_[tid];
    }
    const uint32_t smem0 = lds_addr(smem);

    // ---- staging sources: 32-bit offsets from J.act (the host keeps every activation row within 4 GiB of it)
    auto act_off = [&](int t) -> uint32_t {   // activation t of the tile (clamped to the last one)
        const int q = min(tok0 + t, J.na - 1);
        const int r = (GATHER && J.arow) ? ldg<int>(J.arow + q) : q;
        return (uint32_t)r * (uint32_t)J.astride;
    };
    auto sb_base = [&](int b) {   // superblock b's base, kept opaque in scalar registers
        uint32_t sb = 292u * (uint32_t)b;
        asm volatile("" : "+s"(sb));
        return J.act + sb;
    };
    // values: with four waves, wave w copies activations 4w .. 4w + 3 (and 16 + 4w .. + 3 when the second tile is live) of
    // every superblock, one instruction each (lane l: activation t = 4w + l/16 (+ 16), LDS position l % 16 of its row,
    // source chunk (l % 16) ^ (t & 15)); with eight, waves 4-7 copy the second tile's
    if constexpr (NW == 4) {
        const int t0 = 4 * wave + (lane >> 4), t1 = t0 + 16;
        const uint32_t o0 = act_off(t0) + 4 + 16 * ((lane & 15) ^ (t0 & 15));
        const uint32_t o1 = act_off(t1) + 4 + 16 * ((lane & 15) ^ (t1 & 15));
        const uint32_t l0 = smem0 + V0 + (uint32_t)(4 * wave) * 256;
        for (int b = 0; b < nbk; b++) {
            const uint8_t *ab = sb_base(b);
            load_lds16(ab, o0, l0 + (uint32_t)b * XV);
            if (two) load_lds16(ab, o1, l0 + (uint32_t)b * XV + 16 * 256);
        }
    } else if (wave < 4 || two) {
        const int t0 = 4 * (wave & 3) + 16 * (wave >> 2) + (lane >> 4);
        const uint32_t o0 = act_off(t0) + 4 + 16 * ((lane & 15) ^ (t0 & 15));
        const uint32_t l0 = smem0 + V0 + (uint32_t)(4 * (wave & 3) + 16 * (wave >> 2)) * 256;
        for (int b = 0; b < nbk; b++) load_lds16(sb_base(b), o0, l0 + (uint32_t)b * XV);
    }
    // bsums: thread tid, activation tb = (tid >> 1) & 31, bsums 8 hb .. 8 hb + 7 of superblocks wave + MX_WAVES k;
    // scales: activation td = tid & 31 of superblocks (tid >> 5) + 2 MX_WAVES k (activations 16..31 only when the second
    // tile is live)
    constexpr int KB = (NBKM + NW - 1) / NW, KD = (NBKM + 2 * NW - 1) / (2 * NW);
    const int tb = (tid >> 1) & 31, hb = tid & 1, td = tid & 31;
    const bool bs_live = two || tb < 16, d_live = two || td < 16;
    uint4 bsv[KB];
    float dv[KD];
    {
        const uint32_t ob = act_off(tb) + 260 + 16 * hb, od = act_off(td);
#pragma unroll
        for (int k = 0; k < KB; k++)
            if (wave + NW * k < nbk && bs_live) bsv[k] = ldg<uint4>(sb_base(wave + NW * k) + ob);
#pragma unroll
        for (int k = 0; k < KD; k++) {
            const int b = (tid >> 5) + 2 * NW * k;
            if (b < nbk && d_live) dv[k] = ldg<float>(J.act + (size_t)(292u * (uint32_t)b + od));
        }
    }

    // ---- this wave's weight rows (rows past r1 repeat the last one; their results are not stored)
    // Buffer loads from the tile's first row: per-lane offsets per row group (q chunk, scale pair, d | dmin) and the
    // superblock's 84 b in the scalar offset, so a load needs no address arithmetic.
    const uint8_t *wbase = (GATED && wave >= RW ? J.W2 : J.W) + (size_t)row0 * J.row_bytes;
    const uint32_t wrange = (uint32_t)min(TROWS, J.r1 - row0) * (uint32_t)J.row_bytes;
    const __amdgpu_buffer_rsrc_t wrsrc = __builtin_amdgcn_make_buffer_rsrc((void *)wbase, (short)0, (int)wrange, 0x00020000);
    uint32_t vq[MX_RG], vs[MX_RG], vd[MX_RG];
#pragma unroll
    for (int j = 0; j < MX_RG; j++) {
        const uint32_t o = (uint32_t)min(16 * (RW * j + wq) + lr, J.r1 - 1 - row0) * (uint32_t)J.row_bytes;
        vq[j] = o + 16 + 16 * lg;
        vs[j] = o + 8 * (lg >> 1);
        vd[j] = o + 80;
    }
    auto wload = [&](int j, int b, WRaw &w) {
        const int so = 84 * b;
        const u32x4 q = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrsrc, (int)vq[j], so, 0));
        const u32x2 sc = __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(wrsrc, (int)vs[j], so, 0));
        w.q = make_uint4(q.x, q.y, q.z, q.w);
        w.s0 = sc.x;
        w.s1 = sc.y;
        w.dd = __builtin_amdgcn_raw_buffer_load_b32(wrsrc, (int)vd[j], so, 0);
    };
    // one register set per row group, a superblock ahead. Every load is unconditional (the superblock past the last
    // repeats it, unused): with no branch around a load, the compiler's waits count exactly which loads a use needs
    // instead of draining the queue.
    WRaw R[MX_RG];
#pragma unroll
    for (int j = 0; j < MX_RG; j++) wload(j, 0, R[j]);
    // the staged copies are older than the 3 * MX_RG weight loads just issued
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * MX_RG) : "memory");
#pragma unroll
    for (int k = 0; k < KB; k++) {
        const int b = wave + NW * k;
        if (b >= nbk || !bs_live) continue;
        const uint32_t w[4] = {bsv[k].x, bsv[k].y, bsv[k].z, bsv[k].w};
        uint32_t hv[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {   // two int16 bsums -> two halves (exact)
            const _Float16 e0 = (_Float16)(int16_t)(w[i] & 0xffffu), e1 = (_Float16)(int16_t)(w[i] >> 16);
            hv[i] = (uint32_t)__builtin_bit_cast(uint16_t, e0) | (uint32_t)__builtin_bit_cast(uint16_t, e1) << 16;
        }
        uint8_t *base = smem + BS0 + b * XB + tb * 8;
        *reinterpret_cast<uint2 *>(base + (2 * hb) * (MX_TOK * 8)) = make_uint2(hv[0], hv[1]);
        *reinterpret_cast<uint2 *>(base + (2 * hb + 1) * (MX_TOK * 8)) = make_uint2(hv[2], hv[3]);
    }
#pragma unroll
    for (int k = 0; k < KD; k++) {
        const int b = (tid >> 5) + 2 * NW * k;
        if (b < nbk && d_live) *reinterpret_cast<float *>(smem + D0 + b * XD + td * 4) = dv[k];
    }
    lds_sync();

    // ---- A operand addresses: tile u adds 16 rows (values), 16 * 8 bytes (bsums), 64 bytes (scales)
    uint32_t xo[4];
#pragma unroll
    for (int s = 0; s < 4; s++) {
        const int nat = 8 * (lg >> 1) + 2 * s + (lg & 1);
        xo[s] = smem0 + V0 + lr * 256 + 16 * (nat ^ lr);
    }
    const uint32_t bso = smem0 + BS0 + lg * (MX_TOK * 8) + lr * 8, ydo = smem0 + D0 + 16 * lg;
    auto aload = [&](int b, int u, AOps &A) {
#pragma unroll
        for (int s = 0; s < 4; s++) A.x[s] = lds_ld<v4i>(xo[s] + (uint32_t)b * XV + 16 * 256 * u);
        A.bs = lds_ld<v4h>(bso + (uint32_t)b * XB + 128 * u);
        A.yd = lds_ld<v4f>(ydo + (uint32_t)b * XD + 64 * u);
    };

    v4f acc[MX_RG][2];
#pragma unroll
    for (int j = 0; j < MX_RG; j++) acc[j][0] = acc[j][1] = v4f{0, 0, 0, 0};
    // the previous item's results (starting as zeros: their epilogue adds +0 to the +0 of acc[3])
    // Results and row scales by item parity (j & 1): item j's epilogue reads those of item j - 1 in place, no copies.
    // Item (b - 1, 3), whose epilogue runs at (b, 0), keeps its activation scales in ydl. Its slots start as zeros (all
    // scales 0): the first epilogue adds +0 to the +0 of acc[3].
    MRes mr[2][2];
    mr[1][0].i = mr[1][1].i = v4i{0, 0, 0, 0};
    mr[1][0].m = mr[1][1].m = v4f{0, 0, 0, 0};
    float bd[2] = {0.f, 0.f}, bdm[2] = {0.f, 0.f};
    v4f ydl[2] = {v4f{0, 0, 0, 0}, v4f{0, 0, 0, 0}};
    for (int b = 0; b < nbk; b++) {   // superblock b of the four row groups; their superblock b + 1 loaded in turn
        AOps A[2];
        aload(b, 0, A[0]);
        if (two) aload(b, 1, A[1]);
#pragma unroll
        for (int j = 0; j < MX_RG; j++) {
            const int pc = j & 1, pp = pc ^ 1;
            BOps B;
            build_b(R[j], lg, B);
            wload(j, min(b + 1, nbk - 1), R[j]);
            bd[pc] = B.d;
            bdm[pc] = B.dm;
            mma(A[0], B, mr[pc][0]);
            if (two) mma(A[1], B, mr[pc][1]);
            // the previous item: row group j - 1 of this superblock, or row group 3 of the previous one
            v4f &a0 = acc[(j + MX_RG - 1) % MX_RG][0], &a1 = acc[(j + MX_RG - 1) % MX_RG][1];
            epilogue<CONTRACT>(mr[pp][0], bd[pp], bdm[pp], j ? A[0].yd : ydl[0], a0);
            if (two) epilogue<CONTRACT>(mr[pp][1], bd[pp], bdm[pp], j ? A[1].yd : ydl[1], a1);
        }
        ydl[0] = A[0].yd;
        ydl[1] = A[1].yd;
    }
    epilogue<CONTRACT>(mr[1][0], bd[1], bdm[1], ydl[0], acc[MX_RG - 1][0]);
    if (two) epilogue<CONTRACT>(mr[1][1], bd[1], bdm[1], ydl[1], acc[MX_RG - 1][1]);

    if constexpr (GATED) {
        // ---- h and its Q8_K blocks. Lane l, register i of tile u, row group j: activation 16u + 4lg + i of the tile, h
        // column (row) 16 (4j + wq) + lr of the block, in gate wave wq (its gate value) and up wave 4 + wq (its up value)
        // alike. The two waves split the work: the gate wave forms h for row groups 0 and 1, the up wave for 2 and 3, each
        // taking the other product's values of its row groups through LDS. LDS (the activation area, free after a
        // barrier): the exchanged values xv[writer wave][2][2][lane] (four registers each), then the tile's 32 blocks (292
        // bytes each), then the waves' maxima am[32][wave]. Only the activations of the tile are formed (the second 16 when it has them).
        v4f *xv = reinterpret_cast<v4f *>(smem);
        uint8_t *blk = smem + 32 * 1024;
        float *am = reinterpret_cast<float *>(smem + 32 * 1024 + MX_TOK * 292);
        const int jo = wave < RW ? 0 : 2;   // the row groups this wave forms: jo, jo + 1
        const int nu = two ? 2 : 1;
        __syncthreads();   // every wave is past its last read of the activations
#pragma unroll
        for (int jj = 0; jj < 2; jj++)   // the partner's row groups: 2 - jo + jj
#pragma unroll
            for (int u = 0; u < 2; u++) {
                if (u >= nu) continue;
                const v4f hi = acc[2 + jj][u], lo = acc[jj][u];   // values, not a selected reference (kept in registers)
                xv[((wave * 2 + jj) * 2 + u) * 64 + lane] = wave < RW ? hi : lo;
            }
        __syncthreads();
        float h[2][2][4];
        const int pw = wave ^ RW;   // the partner wave
#pragma unroll
        for (int u = 0; u < 2; u++) {
            if (u >= nu) continue;
            const v4f o0 = xv[((pw * 2 + 0) * 2 + u) * 64 + lane], o1 = xv[((pw * 2 + 1) * 2 + u) * 64 + lane];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                float a = 0.0f;
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    const float lo = acc[jj][u][i], hi = acc[2 + jj][u][i];
                    const float mine = wave < RW ? lo : hi;
                    const float other = jj ? o1[i] : o0[i];
                    const float g = wave < RW ? mine : other, v = wave < RW ? other : mine;
                    h[jj][u][i] = g / (1.0f + esq_expf_tab(-g, xtab)) * v;
                    a = __builtin_fmaxf(a, __builtin_fabsf(h[jj][u][i]));   // the maximum is exact in any order
                }
                a = group_max<16>(a);   // over the 16 rows lr (one DPP row)
                if (lr == 0) am[(16 * u + 4 * lg + i) * NW + wave] = a;
            }
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 2; u++) {
            if (u >= nu) continue;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int t = 16 * u + 4 * lg + i;
                const v4f m0 = *reinterpret_cast<const v4f *>(am + t * NW), m1 = *reinterpret_cast<const v4f *>(am + t * NW + 4);
                const float amax = __builtin_fmaxf(__builtin_fmaxf(__builtin_fmaxf(m0[0], m0[1]), __builtin_fmaxf(m0[2], m0[3])),
                                                   __builtin_fmaxf(__builtin_fmaxf(m1[0], m1[1]), __builtin_fmaxf(m1[2], m1[3])));
                uint8_t *b = blk + t * 292;
#pragma unroll
                for (int jj = 0; jj < 2; jj++) {
                    int q = 0;
                    if (amax != 0.0f) {
                        const int v = static_cast<int>(__builtin_rintf(h[jj][u][i] * (127.0f / amax)));   // lrintf
                        q = v > 127 ? 127 : v < -127 ? -127 : v;
                    }
                    const int g16 = RW * (jo + jj) + wq;   // the block's group of 16 elements
                    b[4 + 16 * g16 + lr] = static_cast<uint8_t>(static_cast<int8_t>(q));
                    const int sum = group_sum<16>(q);   // bsums: the 16 elements of the group (one DPP row)
                    if (lr == 0) reinterpret_cast<int16_t *>(b + 260)[g16] = static_cast<int16_t>(sum);
                }
                if (wave == 0 && lr == 0) *reinterpret_cast<float *>(b) = amax != 0.0f ? amax / 127.0f : 0.0f;
            }
        }
        __syncthreads();
        // the blocks of the tile's activations out, a dword per thread: activation t's block (row0 / 256) of its h row
        const int nt = min(MX_TOK, J.na - tok0);
        uint8_t *hy = reinterpret_cast<uint8_t *>(J.y) + (size_t)(row0 / 256) * 292;
        for (int x = tid; x < nt * 73; x += 64 * NW) {
            const int t = x / 73, d = x - t * 73;
            *reinterpret_cast<uint32_t *>(hy + (size_t)(tok0 + t) * J.ystride + 4 * d) =
                *reinterpret_cast<const uint32_t *>(blk + t * 292 + 4 * d);
        }
        return;
    }
    // ---- outputs: lane l, register i of tile u holds activation tok0 + 16u + 4lg + i, row row0 + 16 (4j + wave) + lr.
    // Buffer stores over y[0, (na - 1) * ystride + r1): the hardware's range check drops those of activations past na
    // (ystride >= r1), and rows past r1 get an offset above the range. The host keeps (na + MX_TOK) * ystride * 4 below
    // 2^31, so no offset wraps.
    const uint32_t ys4 = 4u * (uint32_t)J.ystride;
    const uint32_t yrange = (uint32_t)(J.na - 1) * ys4 + 4u * (uint32_t)J.r1;
    const __amdgpu_buffer_rsrc_t yrsrc = __builtin_amdgcn_make_buffer_rsrc((void *)J.y, (short)0, (int)yrange, 0x00020000);
#pragma unroll
    for (int j = 0; j < MX_RG; j++) {
        const int r = row0 + 16 * (RW * j + wq) + lr;
        uint32_t yoff = r < J.r1 ? (uint32_t)(tok0 + 4 * lg) * ys4 + 4u * (uint32_t)r : 0x80000000u;
#pragma unroll
        for (int u = 0; u < 2; u++) {
            if (u == 1 && !two) break;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const float v = acc[j][u][i];
                __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), yrsrc, (int)yoff, 0, 0);
                yoff += i < 3 ? ys4 : 13 * ys4;   // the next activation: + 1, or + 13 to the next tile's first
            }
        }
    }
}

template <int NBKM>
void mx_launch_nbk(bool gather, bool contract, const MkJob *jobs, int njobs, const MkJob &single, int grid, hipStream_t s) {
    const dim3 g(grid), b(64 * MX_WAVES);
    if (gather) {
        if (contract) hipLaunchKernelGGL((mx_q2k_kernel<NBKM, true, true, false>), g, b, 0, s, jobs, njobs, single);
        else hipLaunchKernelGGL((mx_q2k_kernel<NBKM, false, true, false>), g, b, 0, s, jobs, njobs, single);
    } else {
        if (contract) hipLaunchKernelGGL((mx_q2k_kernel<NBKM, true, false, false>), g, b, 0, s, jobs, njobs, single);
        else hipLaunchKernelGGL((mx_q2k_kernel<NBKM, false, false, false>), g, b, 0, s, jobs, njobs, single);
    }
}

template <int NBKM>
void mxg_launch_nbk(bool gather, bool contract, const MkJob *jobs, int njobs, const MkJob &single, int grid, hipStream_t s) {
    const dim3 g(grid), b(512);
    if (gather) {
        if (contract) hipLaunchKernelGGL((mx_q2k_kernel<NBKM, true, true, true>), g, b, 0, s, jobs, njobs, single);
        else hipLaunchKernelGGL((mx_q2k_kernel<NBKM, false, true, true>), g, b, 0, s, jobs, njobs, single);
    } else {
        if (contract) hipLaunchKernelGGL((mx_q2k_kernel<NBKM, true, false, true>), g, b, 0, s, jobs, njobs, single);
        else hipLaunchKernelGGL((mx_q2k_kernel<NBKM, false, false, true>), g, b, 0, s, jobs, njobs, single);
    }
}

}  // namespace

int mx_nbk_max(int nbk) { return nbk <= 4 ? 4 : nbk <= 8 ? 8 : nbk <= MX_NBK ? MX_NBK : 0; }

hipError_t mxg_launch(bool gather, int nbk_max, const MkJob *jobs, int njobs, const MkJob &single, int grid, int order,
                      hipStream_t s) {
    const bool contract = order == ES_HIP_ORDER_X86_CONTRACT;
    switch (mx_nbk_max(nbk_max)) {
    case 4: mxg_launch_nbk<4>(gather, contract, jobs, njobs, single, grid, s); break;
    case 8: mxg_launch_nbk<8>(gather, contract, jobs, njobs, single, grid, s); break;
    case MX_NBK: mxg_launch_nbk<MX_NBK>(gather, contract, jobs, njobs, single, grid, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t mx_launch(int type, bool gather, int nbk_max, const MkJob *jobs, int njobs, const MkJob &single, int grid,
                     int order, hipStream_t s) {
    if (type != ES_HIP_Q2_K) return hipErrorInvalidValue;
    const bool contract = order == ES_HIP_ORDER_X86_CONTRACT;
    switch (mx_nbk_max(nbk_max)) {
    case 4: mx_launch_nbk<4>(gather, contract, jobs, njobs, single, grid, s); break;
    case 8: mx_launch_nbk<8>(gather, contract, jobs, njobs, single, grid, s); break;
    case MX_NBK: mx_launch_nbk<MX_NBK>(gather, contract, jobs, njobs, single, grid, s); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace esq
