// The vector glue of the MoE expert FFN (moe_n, src/es_engine.c:848-942) between the grouped products:
//   SwiGLU of each (token, expert) pair's gate and up rows, h = g / (1 + expf(-g)) * u (:913), requantized exactly as
//   es_act_prepare does (:914 -> src/es_quant.c:499-512): Q8_K blocks (src/es_q2k.c:102-125) for a K-quant down
//   projection, Q8_0 blocks (src/es_quant.c:489-497) for a 32-wide one;
//   the weighted combine out[t][i] = sum_j w[t][j] * y[rowof[t][j]][i] (:925-932).
// The reference compiles these loops for baseline x86-64 (no FMA instructions), so every product and sum is rounded on its
// own; this file is built with -ffp-contract=off and spells no fused operation. Division is IEEE (correctly rounded) and
// expf follows glibc's method bit for bit (es_hip_expf.h).
#include "es_hip_common.h"
#include "es_hip_expf.h"

namespace esq {

__device__ __forceinline__ float swiglu(float g, float u) { return g / (1.0f + esq_expf(-g)) * u; }

// One workgroup of 256 threads per (pair row, 256-wide block): h, amax, the Q8_K block (d, qs, bsums).
__global__ __launch_bounds__(256) void swiglu_q8k(const float *__restrict__ gu, int ff, uint8_t *__restrict__ ha,
                                                   uint64_t hstride) {
    const int r = blockIdx.y, b = blockIdx.x, i = threadIdx.x;
    const float *g = gu + (size_t)r * 2 * ff + (size_t)b * 256;
    const float h = swiglu(g[i], g[ff + i]);
    __shared__ float wmax[4];
    float a = __builtin_fabsf(h);
    for (int o = 32; o > 0; o >>= 1) a = __builtin_fmaxf(a, __shfl_xor(a, o));   // max is exact in any order
    if ((i & 63) == 0) wmax[i >> 6] = a;
    __syncthreads();
    const float amax = __builtin_fmaxf(__builtin_fmaxf(wmax[0], wmax[1]), __builtin_fmaxf(wmax[2], wmax[3]));
    uint8_t *blk = ha + (size_t)r * hstride + (size_t)b * 292;
    int q = 0;
    if (amax != 0.0f) {
        const float id = 127.0f / amax;
        q = static_cast<int>(__builtin_rintf(h * id));   // lrintf: round to nearest even
        q = q > 127 ? 127 : q < -127 ? -127 : q;
    }
    blk[4 + i] = static_cast<uint8_t>(static_cast<int8_t>(q));
    int s = q;   // bsums: sums of 16 consecutive qs
    for (int o = 8; o > 0; o >>= 1) s += __shfl_xor(s, o, 16);
    if ((i & 15) == 0) reinterpret_cast<int16_t *>(blk + 260)[i >> 4] = static_cast<int16_t>(s);
    if (i == 0) *reinterpret_cast<float *>(blk) = amax != 0.0f ? amax / 127.0f : 0.0f;
}

// One workgroup of 256 threads per (pair row, 8 Q8_0 blocks).
__global__ __launch_bounds__(256) void swiglu_q80(const float *__restrict__ gu, int ff, uint8_t *__restrict__ ha,
                                                   uint64_t hstride) {
    const int r = blockIdx.y, i = threadIdx.x, e = blockIdx.x * 256 + i;
    if (e >= ff) return;   // ff is a multiple of 32: whole blocks drop out together
    const float *g = gu + (size_t)r * 2 * ff;
    const float h = swiglu(g[e], g[ff + e]);
    float a = __builtin_fabsf(h);
    for (int o = 16; o > 0; o >>= 1) a = __builtin_fmaxf(a, __shfl_xor(a, o, 32));
    const float d = a / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const float v = h * id;
    const int q = static_cast<int>(v < 0.0f ? v - 0.5f : v + 0.5f);   // round half away, then truncate
    uint8_t *blk = ha + (size_t)r * hstride + (size_t)(e >> 5) * 36;
    blk[4 + (e & 31)] = static_cast<uint8_t>(static_cast<int8_t>(q));
    if ((e & 31) == 0) *reinterpret_cast<float *>(blk) = d;
}

// One thread per (token, output element): the token's expert outputs summed in routing order, from s = 0.
__global__ __launch_bounds__(256) void moe_combine(const float *__restrict__ ye, const int *__restrict__ rowof,
                                                   const float *__restrict__ w, const int *__restrict__ k, int kmax, int n,
                                                   float *__restrict__ out, uint64_t ostride) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = 0.0f;
    const int kt = k[t];
    for (int j = 0; j < kt; j++) s = s + w[t * kmax + j] * ye[(size_t)rowof[t * kmax + j] * n + i];
    out[(size_t)t * ostride + i] = s;
}

// route() for softmax gating (src/es_engine.c:744-835, the GATE_SOFTMAX path: no gate bias, selection bias, expert groups,
// cache bonus or top-k override): one wave per token. The maximum and every argmax are exact in any order (ties go to the
// lowest expert, as the reference's first-maximum scan does); the two sums (softmax denominator over the experts, chosen
// weights over the picks) run on one lane in the reference's order.
__global__ __launch_bounds__(64) void route_softmax(const float *__restrict__ logits, uint64_t ls, int ne, int k, int norm_topk,
                                                    int *__restrict__ sel, float *__restrict__ w, int kmax) {
    __shared__ float p[ROUTE_MAX_EXPERTS];
    __shared__ float total;
    const int t = blockIdx.x, l = threadIdx.x;
    const float *r = logits + (size_t)t * ls;
    float mx = -__builtin_inff();
    for (int e = l; e < ne; e += 64) {
        const float v = r[e];
        p[e] = v;
        mx = v > mx ? v : mx;   // mx = r[e] > mx ? r[e] : mx (:753)
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float m = __shfl_xor(mx, o);
        mx = m > mx ? m : mx;
    }
    for (int e = l; e < ne; e += 64) p[e] = esq_expf(p[e] - mx);
    __syncthreads();
    if (l == 0) {
        float sum = 0.0f;
        for (int e = 0; e < ne; e++) sum += p[e];   // :754, in expert order
        total = sum;
    }
    __syncthreads();
    const float sum = total;
    for (int e = l; e < ne; e += 64) p[e] /= sum;   // :755
    __syncthreads();
    // k rounds of argmax over the experts not yet taken (:794-804); taken experts are marked in a lane's own bit mask
    uint32_t taken = 0;   // bit m: expert l + 64 m (ne <= 1024: 16 per lane)
    float wsum = 0.0f, wj = 0.0f;
    for (int j = 0; j < k; j++) {
        float bv = 0.0f;
        int be = -1;
        for (int m = 0, e = l; e < ne; m++, e += 64) {
            const float v = p[e];
            if (!((taken >> m) & 1u) && (be < 0 || v > bv)) { bv = v; be = e; }
        }
        for (int o = 32; o > 0; o >>= 1) {   // the larger value, the lower expert on a tie; lanes without a candidate lose
            const float ov = __shfl_xor(bv, o);
            const int oe = __shfl_xor(be, o);
            if (oe >= 0 && (be < 0 || ov > bv || (ov == bv && oe < be))) { bv = ov; be = oe; }
        }
        if ((be & 63) == l) taken |= 1u << (be >> 6);
        if (l == 0) {
            sel[(size_t)t * kmax + j] = be;
            wsum += bv;   // w[j] = r[best]; wsum += w[j] (:802-803)
        }
        if (l == j) wj = bv;
    }
    if (l == 0) total = norm_topk ? (wsum > 6.103515625e-5f ? wsum : 6.103515625e-5f) : 1.0f;   // :832
    __syncthreads();
    if (l < k) w[(size_t)t * kmax + l] = norm_topk ? wj / total : wj;
}

hipError_t route_softmax_launch(const float *logits, uint64_t ls, int ntok, int ne, int k, int norm_topk, int *sel, float *w,
                                int kmax, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(route_softmax, dim3(ntok), dim3(64), 0, s, logits, ls, ne, k, norm_topk, sel, w, kmax);
    return hipGetLastError();
}

hipError_t moe_swiglu_launch(const float *gu, int rows, int ff, bool q8k, uint8_t *ha, uint64_t hstride, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    if (q8k) hipLaunchKernelGGL(swiglu_q8k, dim3(ff / 256, rows), dim3(256), 0, s, gu, ff, ha, hstride);
    else hipLaunchKernelGGL(swiglu_q80, dim3((ff + 255) / 256, rows), dim3(256), 0, s, gu, ff, ha, hstride);
    return hipGetLastError();
}

hipError_t moe_combine_launch(const float *ye, const int *rowof, const float *w, const int *k, int kmax, int ntok, int n,
                              float *out, uint64_t ostride, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    hipLaunchKernelGGL(moe_combine, dim3((n + 255) / 256, ntok), dim3(256), 0, s, ye, rowof, w, k, kmax, n, out, ostride);
    return hipGetLastError();
}

// ---- device-routed MoE: grouping and job tables --------------------------------------------------------------------
namespace {

// Exclusive prefix sums of three values per thread of the block (MOE_GROUP_THREADS threads, 16 waves): shuffles within
// each wave, then the 16 wave totals on one wave. tot receives the three sums.
__device__ int3 block_excl_scan3(int3 v, int3 *wsum, int3 *tot) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    int3 x = v;
    for (int off = 1; off < 64; off <<= 1) {
        const int a = __shfl_up(x.x, off), b = __shfl_up(x.y, off), c = __shfl_up(x.z, off);
        if (lane >= off) { x.x += a; x.y += b; x.z += c; }
    }
    if (lane == 63) wsum[w] = x;
    __syncthreads();
    if (w == 0) {
        constexpr int NW = MOE_GROUP_THREADS / 64;
        int3 y = lane < NW ? wsum[lane] : make_int3(0, 0, 0);
        for (int off = 1; off < NW; off <<= 1) {
            const int a = __shfl_up(y.x, off), b = __shfl_up(y.y, off), c = __shfl_up(y.z, off);
            if (lane >= off) { y.x += a; y.y += b; y.z += c; }
        }
        if (lane < NW) wsum[lane] = y;
        if (lane == NW - 1) *tot = y;
    }
    __syncthreads();
    const int3 pre = w > 0 ? wsum[w - 1] : make_int3(0, 0, 0);
    __syncthreads();   // wsum is reused by the next scan
    return make_int3(pre.x + x.x - v.x, pre.y + x.y - v.y, pre.z + x.z - v.z);
}

__device__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// One workgroup: moe_n's grouping (src/es_engine.c:871-888) of the ntok * k choices, then every job of the layer's two
// launches. Experts take slots in order of first use; an expert's rows follow its choices in (token, j) order.
__global__ __launch_bounds__(MOE_GROUP_THREADS) void moe_group_build(MoeDevArgs A, MoeFamily GU, MoeFamily DN) {
    __shared__ int first[ROUTE_MAX_EXPERTS], cnt[ROUTE_MAX_EXPERTS], slot[ROUTE_MAX_EXPERTS], taken[ROUTE_MAX_EXPERTS];
    __shared__ int uex[ROUTE_MAX_EXPERTS], ustart[ROUTE_MAX_EXPERTS];
    __shared__ int wcnt[MOE_GROUP_THREADS / 64][ROUTE_MAX_EXPERTS];   // per wave of a chunk: choices of each expert
    __shared__ int3 wsum[MOE_GROUP_THREADS / 64];
    __shared__ int3 s_tot;
    __shared__ int s_used;
    const int tid = threadIdx.x, T = MOE_GROUP_THREADS, NE = A.n_exp, R = A.ntok * A.k;
    // the first chunk's choices and weights, loaded before anything waits on them
    const int sel0 = tid < R ? A.sel[tid] : -1;
    const float w0_ = tid < R ? A.w[tid] : 0.0f;
    if (tid == 0) s_used = 0;
    for (int e = tid; e < NE; e += T) {
        first[e] = R;
        cnt[e] = 0;
        taken[e] = 0;
        slot[e] = -1;
    }
    __syncthreads();
    for (int p = tid; p < R; p += T) {
        const int e = p < T ? sel0 : A.sel[p];
        if (e >= 0 && e < NE) {
            atomicMin(&first[e], p);
            atomicAdd(&cnt[e], 1);
        }
    }
    __syncthreads();
    // slot of a used expert: the number of used experts first chosen before it (first uses are distinct choices)
    for (int e = tid; e < NE; e += T)
        if (first[e] < R) {
            int r = 0;
            for (int e2 = 0; e2 < NE; e2++) r += first[e2] < first[e];
            slot[e] = r;
            uex[r] = e;
            atomicAdd(&s_used, 1);
        }
    __syncthreads();
    const int U = s_used;
    const int c_me = tid < U ? cnt[uex[tid]] : 0;   // thread u: slot u's expert's count
    const int st = block_excl_scan3(make_int3(c_me, 0, 0), wsum, &s_tot).x;
    if (tid < NE) ustart[tid] = st;
    // pair rows: the slot's first row + the choices of the same expert before this one, counted in chunks of one choice
    // per thread: earlier chunks (taken), earlier waves of the chunk (wcnt), earlier lanes of the wave (a match mask
    // from ballots over the expert id's bits)
    const int lane = tid & 63, wv = tid >> 6;
    const uint64_t lt = (1ull << lane) - 1;
    for (int c0 = 0; c0 < R; c0 += T) {
        for (int i = tid; i < (T / 64) * NE; i += T) wcnt[i / NE][i % NE] = 0;
        const int p = c0 + tid;
        const int e0 = c0 == 0 ? sel0 : p < R ? A.sel[p] : -1;
        const int e = e0 >= 0 && e0 < NE ? e0 : -1;
        uint64_t same = __ballot(e >= 0);
        for (int b = 0; b < 10; b++) {   // expert ids < 1024
            const uint64_t m = __ballot(e >= 0 && ((e >> b) & 1));
            same &= ((e >> b) & 1) ? m : ~m;
        }
        __syncthreads();
        if (e >= 0 && (same & lt) == 0) wcnt[wv][e] = __popcll(same);   // the wave's first lane with e
        __syncthreads();
        if (p < R) {
            int row = 0;
            float wt = 0.0f;
            if (e >= 0) {
                int r = __popcll(same & lt);
                for (int i = 0; i < wv; i++) r += wcnt[i][e];
                row = ustart[slot[e]] + taken[e] + r;
                wt = c0 == 0 ? w0_ : A.w[p];
                A.tok_of[row] = p / A.k;
            }
            A.rowof[p] = row;   // an invalid expert id contributes 0 * row 0
            A.wv[p] = wt;
        }
        __syncthreads();
        if (p < R && e >= 0 && (same & lt) == 0) atomicAdd(&taken[e], __popcll(same));
        __syncthreads();
    }
    // ---- job tables. Thread u writes slot u's jobs; tiles and pre-pass items are prefix sums over the slots.
    const int u = tid;
    const bool real = u < U;
    const int e = real ? uex[u] : 0, c = real ? cnt[e] : 0, s0 = real ? ustart[u] : 0;
    const int ff = A.ff, n = A.n;
    for (int prod = 0; prod < 2; prod++) {   // 0: gate/up, 1: down
        const MoeFamily &F = prod ? DN : GU;
        const int njob = prod ? 1 : 2;
        int ntok = 0, tiles = 0, items = 0, units = 0;
        if (F.kind == MOE_FAM_MM && real) {
            ntok = ceil_div(c, F.bn);
            tiles = njob * F.row_tiles8 * ntok;
            const int per = F.pj.nbk * (int)prep_words(F.pj.kind);
            items = ceil_div(ntok * F.bn * per, PREP_SPAN) * PREP_SPAN;
            // the expert's planes in 256-byte units: values [nbk][na_pad][256], then meta + scales [nbk][na_pad][36]
            units = ceil_div(F.pj.nbk * ntok * F.bn * 256, 256) + ceil_div(F.pj.nbk * ntok * F.bn * 36, 256);
        }
        int tot_tiles = 0, tot_items = 0, w0 = 0;
        if (F.kind == MOE_FAM_MM) {   // uniform across the block: every thread takes part in the scan
            const int3 sc = block_excl_scan3(make_int3(tiles, items, units), wsum, &s_tot);
            tot_tiles = s_tot.x;
            tot_items = s_tot.y;
            tiles = sc.x;
            items = sc.y;
            w0 = sc.z;
        }
        const int t0 = tiles, i0 = items;
        const uint8_t *const *wsrc = prod ? A.down : A.gate;
        if (F.kind == MOE_FAM_MV) {
            MvJob *jobs = static_cast<MvJob *>(prod ? A.dn_jobs : A.gu_jobs);
            const int end = njob * U * F.mv_tiles;
            if (u < A.umax)
                for (int g = 0; g < njob; g++) {
                    MvJob J = F.mv;
                    if (real) {
                        J.W = (g ? A.up : wsrc)[e];
                        if (prod) {
                            J.act = A.ha + (size_t)s0 * A.hstride;
                            J.arow = nullptr;
                            J.y = A.bye + (size_t)s0 * n;
                        } else {
                            J.act = A.x;
                            J.arow = A.tok_of + s0;
                            J.y = A.bgu + (size_t)s0 * 2 * ff + (size_t)g * ff;
                        }
                        J.na = c;
                        J.tile0 = (njob * u + g) * F.mv_tiles;
                    } else {   // empty: the template's valid pointers, no rows, no activations, after the last real tile
                        J.na = 0;
                        J.r0 = J.r1 = 0;
                        J.tile0 = end;
                    }
                    jobs[njob * u + g] = J;
                }
            if (tid == 0) {   // the sentinel
                MvJob J = F.mv;
                J.na = 0;
                J.r0 = J.r1 = 0;
                J.tile0 = end;
                jobs[njob * A.umax] = J;
            }
        } else {
            MmJob *jobs = static_cast<MmJob *>(prod ? A.dn_jobs : A.gu_jobs);
            PrepJob *pj = prod ? A.dn_prep : A.gu_prep;
            uint8_t *ws = prod ? A.dn_ws : A.gu_ws;
            if (u < A.umax) {
                const int na_pad = ntok * F.bn;
                uint8_t *xq = ws + (size_t)w0 * 256;
                uint8_t *xm = xq + ((size_t)F.pj.nbk * na_pad * 256 + 255) / 256 * 256;
                PrepJob P = F.pj;
                if (real) {
                    P.act = prod ? A.ha + (size_t)s0 * A.hstride : A.x;
                    P.arow = prod ? nullptr : A.tok_of + s0;
                    P.xq = xq;
                    P.xm = xm;
                    P.start = i0;
                    P.na = c;
                    P.na_pad = na_pad;
                } else {
                    P.na = P.na_pad = 0;
                    P.start = tot_items;
                }
                pj[u] = P;
                for (int g = 0; g < njob; g++) {
                    MmJob J = F.mm;
                    if (real) {
                        J.W = (g ? A.up : wsrc)[e];
                        J.xq = xq;
                        J.xm = xm;
                        J.y = prod ? A.bye + (size_t)s0 * n : A.bgu + (size_t)s0 * 2 * ff + (size_t)g * ff;
                        J.na = c;
                        J.na_pad = na_pad;
                        J.ntok_tiles = ntok;
                        J.tile0 = t0 + g * F.row_tiles8 * ntok;
                    } else {
                        J.na = 0;
                        J.r0 = J.r1 = 0;
                        J.ntok_tiles = 1;
                        J.tile0 = tot_tiles;
                    }
                    jobs[njob * u + g] = J;
                }
            }
            if (tid == 0) {
                PrepJob P = F.pj;
                P.na = P.na_pad = 0;
                P.start = tot_items;
                pj[A.umax] = P;
                MmJob J = F.mm;
                J.na = 0;
                J.r0 = J.r1 = 0;
                J.ntok_tiles = 1;
                J.tile0 = tot_tiles;
                jobs[njob * A.umax] = J;
            }
        }
        __syncthreads();
    }
}

}  // namespace

hipError_t moe_group_build_launch(const MoeDevArgs &a, const MoeFamily &gu, const MoeFamily &dn, hipStream_t s) {
    hipLaunchKernelGGL(moe_group_build, dim3(1), dim3(MOE_GROUP_THREADS), 0, s, a, gu, dn);
    return hipGetLastError();
}

// h values only (no requantization), for checking the SwiGLU against the reference's on arbitrary inputs
__global__ void swiglu_plain(const float *__restrict__ g, const float *__restrict__ u, float *__restrict__ h, long n) {
    const long i = (long)blockIdx.x * 256 + threadIdx.x;
    if (i < n) h[i] = swiglu(g[i], u[i]);
}

hipError_t swiglu_plain_launch(const float *g, const float *u, float *h, long n, hipStream_t s) {
    if (n <= 0) return hipSuccess;
    hipLaunchKernelGGL(swiglu_plain, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, u, h, n);
    return hipGetLastError();
}

}  // namespace esq
