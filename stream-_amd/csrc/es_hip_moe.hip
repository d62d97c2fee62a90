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
template <typename TAB> __device__ __forceinline__ float swiglu_tab(float g, float u, const TAB &T) {
    return g / (1.0f + esq_expf_tab(-g, T)) * u;
}
// expf's table copied into LDS by the first 32 threads, its load issued beside the kernel's own (the caller synchronises
// before the first expf)
#define ESQ_EXPF_LDS_TABLE(tab, i)                    \
    __shared__ uint64_t tab[32];                      \
    {                                                 \
        static constexpr uint64_t T_[32] = ESQ_EXPF_TABLE; \
        if ((i) < 32) tab[(i)] = T_[(i)];             \
    }

// One wave per (pair row, 256-wide block), four per workgroup: h, amax, the Q8_K block (d, qs, bsums). Lane l takes
// elements 4l .. 4l + 3; the maximum (exact in any order) and the bsums (integer sums) by wave reductions, so the only
// barrier is the one after expf's table.
__global__ __launch_bounds__(256) void swiglu_q8k(const float *__restrict__ gu, int ff, int rows, uint8_t *__restrict__ ha,
                                                   uint64_t hstride) {
    const int tid = threadIdx.x, l = tid & 63, nb = ff / 256;
    ESQ_EXPF_LDS_TABLE(tab, tid)
    const int item = blockIdx.x * 4 + (tid >> 6);
    const bool live = item < rows * nb;
    const int r = live ? item / nb : 0, b = live ? item - r * nb : 0;
    const float *g = gu + (size_t)r * 2 * ff + (size_t)b * 256 + 4 * l;
    const float4 gv = *reinterpret_cast<const float4 *>(g), uv = *reinterpret_cast<const float4 *>(g + ff);
    __syncthreads();
    if (!live) return;
    const float h[4] = {swiglu_tab(gv.x, uv.x, tab), swiglu_tab(gv.y, uv.y, tab), swiglu_tab(gv.z, uv.z, tab),
                        swiglu_tab(gv.w, uv.w, tab)};
    float a = __builtin_fmaxf(__builtin_fmaxf(__builtin_fabsf(h[0]), __builtin_fabsf(h[1])),
                              __builtin_fmaxf(__builtin_fabsf(h[2]), __builtin_fabsf(h[3])));
    a = group_max<16>(a);   // DPP within each 16 lanes, then across the four rows
    a = __builtin_fmaxf(a, __shfl_xor(a, 16));
    const float amax = __builtin_fmaxf(a, __shfl_xor(a, 32));
    uint8_t *blk = ha + (size_t)r * hstride + (size_t)b * 292;
    int q[4] = {0, 0, 0, 0};
    if (amax != 0.0f) {
        const float id = 127.0f / amax;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const int v = static_cast<int>(__builtin_rintf(h[k] * id));   // lrintf: round to nearest even
            q[k] = v > 127 ? 127 : v < -127 ? -127 : v;
        }
    }
    *reinterpret_cast<uint32_t *>(blk + 4 + 4 * l) = (uint32_t)(q[0] & 0xff) | (uint32_t)(q[1] & 0xff) << 8 |
                                                    (uint32_t)(q[2] & 0xff) << 16 | (uint32_t)(q[3] & 0xff) << 24;
    const int s = group_sum<4>(q[0] + q[1] + q[2] + q[3]);   // bsums: sums of 16 consecutive qs, four lanes each
    if ((l & 3) == 0) reinterpret_cast<int16_t *>(blk + 260)[l >> 2] = static_cast<int16_t>(s);
    if (l == 0) *reinterpret_cast<float *>(blk) = amax != 0.0f ? amax / 127.0f : 0.0f;
}

// One workgroup of 256 threads per (pair row, 8 Q8_0 blocks).
__global__ __launch_bounds__(256) void swiglu_q80(const float *__restrict__ gu, int ff, uint8_t *__restrict__ ha,
                                                   uint64_t hstride) {
    const int r = blockIdx.y, i = threadIdx.x, e = blockIdx.x * 256 + i;
    ESQ_EXPF_LDS_TABLE(tab, i)
    __syncthreads();
    if (e >= ff) return;   // ff is a multiple of 32: whole blocks drop out together
    const float *g = gu + (size_t)r * 2 * ff;
    const float h = swiglu_tab(g[e], g[ff + e], tab);
    float a = __builtin_fabsf(h);
    for (int o = 16; o > 0; o >>= 1) a = __builtin_fmaxf(a, __shfl_xor(a, o, 32));
    const float d = a / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
    const float v = h * id;
    const int q = static_cast<int>(v < 0.0f ? v - 0.5f : v + 0.5f);   // round half away, then truncate
    uint8_t *blk = ha + (size_t)r * hstride + (size_t)(e >> 5) * 36;
    blk[4 + (e & 31)] = static_cast<uint8_t>(static_cast<int8_t>(q));
    if ((e & 31) == 0) *reinterpret_cast<float *>(blk) = d;
}

// One thread per (token, output element): the token's expert outputs summed in routing order, from s = 0. The rows are
// read eight at a time (the last one repeated past k) so that eight loads are in flight before the first sum; the sums
// then run one by one in routing order.
constexpr int COMBINE_BATCH = 8;

__global__ __launch_bounds__(256) void moe_combine(const float *__restrict__ ye, const int *__restrict__ rowof,
                                                   const float *__restrict__ w, const int *__restrict__ k, int kmax, int n,
                                                   float *__restrict__ out, uint64_t ostride) {
    const int t = blockIdx.y, i = blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = 0.0f;
    const int kt = k[t];
    for (int j0 = 0; j0 < kt; j0 += COMBINE_BATCH) {
        float wj[COMBINE_BATCH], y[COMBINE_BATCH];
#pragma unroll
        for (int q = 0; q < COMBINE_BATCH; q++) {
            const int j = min(j0 + q, kt - 1);
            wj[q] = w[t * kmax + j];
            y[q] = ye[(size_t)rowof[t * kmax + j] * n + i];
        }
#pragma unroll
        for (int q = 0; q < COMBINE_BATCH; q++)
            if (j0 + q < kt) s = s + wj[q] * y[q];
    }
    out[(size_t)t * ostride + i] = s;
}

// The same, four consecutive elements per thread (16-byte loads and stores) when n, the output stride and both
// pointers allow it.
__global__ __launch_bounds__(256) void moe_combine4(const float *__restrict__ ye, const int *__restrict__ rowof,
                                                    const float *__restrict__ w, const int *__restrict__ k, int kmax, int n,
                                                    float *__restrict__ out, uint64_t ostride) {
    const int t = blockIdx.y, i = 4 * (blockIdx.x * 256 + threadIdx.x);
    if (i >= n) return;
    float4 s = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    const int kt = k[t];
    for (int j0 = 0; j0 < kt; j0 += COMBINE_BATCH) {
        float wj[COMBINE_BATCH];
        float4 y[COMBINE_BATCH];
#pragma unroll
        for (int q = 0; q < COMBINE_BATCH; q++) {
            const int j = min(j0 + q, kt - 1);
            wj[q] = w[t * kmax + j];
            y[q] = *reinterpret_cast<const float4 *>(ye + (size_t)rowof[t * kmax + j] * n + i);
        }
#pragma unroll
        for (int q = 0; q < COMBINE_BATCH; q++)
            if (j0 + q < kt) {
                s.x = s.x + wj[q] * y[q].x;
                s.y = s.y + wj[q] * y[q].y;
                s.z = s.z + wj[q] * y[q].z;
                s.w = s.w + wj[q] * y[q].w;
            }
    }
    *reinterpret_cast<float4 *>(out + (size_t)t * ostride + i) = s;
}

// route() for softmax gating (src/es_engine.c:744-835, the GATE_SOFTMAX path: no gate bias, selection bias, expert groups,
// cache bonus or top-k override): one wave per token. The maximum is exact in any order; the two sums (softmax
// denominator over the experts, chosen weights over the picks) run in the reference's order.
//
// The k picks: each lane keeps the best of its own untaken experts (e = l + 64 m); per pick the wave takes the largest
// value (probabilities are non-negative, so their bits order as the values do), then the lowest expert holding it (the
// reference's first-maximum scan), and only the lane that owned the pick rescans its experts. Both reductions are DPP
// moves within the wave (no LDS). A probability that is NaN (only from a NaN or infinite logit) takes the reference's
// scan order instead, one comparison per expert as it writes it.
constexpr int ROUTE_PER_LANE = ROUTE_MAX_EXPERTS / 64;

// the wave's maximum (MAX) or minimum of v in every lane: quad_perm [1,0,3,2], [2,3,0,1], row_half_mirror, row_mirror
// (each row of 16 holds its own), row_bcast:15 into rows 1 and 3, row_bcast:31 into rows 2 and 3; lane 63 is read out
template <bool MAX, int CTRL, int ROW_MASK> __device__ __forceinline__ uint32_t dpp_step(uint32_t v) {
    const uint32_t o = (uint32_t)__builtin_amdgcn_update_dpp((int)v, (int)v, CTRL, ROW_MASK, 0xF, false);
    return MAX ? (o > v ? o : v) : (o < v ? o : v);
}
template <bool MAX> __device__ __forceinline__ uint32_t wave_reduce(uint32_t v) {
    v = dpp_step<MAX, 0xB1, 0xF>(v);
    v = dpp_step<MAX, 0x4E, 0xF>(v);
    v = dpp_step<MAX, 0x141, 0xF>(v);
    v = dpp_step<MAX, 0x140, 0xF>(v);
    v = dpp_step<MAX, 0x142, 0xA>(v);
    v = dpp_step<MAX, 0x143, 0xC>(v);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
// the same for a float maximum that skips NaN as the reference's mx = r[e] > mx ? r[e] : mx does
template <int CTRL, int ROW_MASK> __device__ __forceinline__ float dpp_fmax(float v) {
    const float o = __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(v), __float_as_int(v), CTRL, ROW_MASK, 0xF, false));
    return o > v ? o : v;
}
__device__ __forceinline__ float wave_fmax(float v) {
    v = dpp_fmax<0xB1, 0xF>(v);
    v = dpp_fmax<0x4E, 0xF>(v);
    v = dpp_fmax<0x141, 0xF>(v);
    v = dpp_fmax<0x140, 0xF>(v);
    v = dpp_fmax<0x142, 0xA>(v);
    v = dpp_fmax<0x143, 0xC>(v);
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}

__global__ __launch_bounds__(64) void route_softmax(const float *__restrict__ logits, uint64_t ls, int ne, int k, int norm_topk,
                                                    int *__restrict__ sel, float *__restrict__ w, int kmax) {
    __shared__ __align__(16) float p[ROUTE_MAX_EXPERTS];
    __shared__ uint64_t tab[32];
    __shared__ float total;
    static constexpr uint64_t T[32] = ESQ_EXPF_TABLE;
    const int t = blockIdx.x, l = threadIdx.x;
    const int mc = (ne + 63) >> 6;   // experts per lane, wave-uniform
    if (l < 32) tab[l] = T[l];      // expf's table in LDS: its load overlaps the logits'
    const float *r = logits + (size_t)t * ls;
    float v[ROUTE_PER_LANE];
    float mx = -__builtin_inff();
#pragma unroll
    for (int m = 0; m < ROUTE_PER_LANE; m++) {
        if (m >= mc) break;
        const int e = l + 64 * m;
        v[m] = e < ne ? r[e] : -__builtin_inff();
        mx = v[m] > mx ? v[m] : mx;   // mx = r[e] > mx ? r[e] : mx (:753)
    }
    mx = wave_fmax(mx);
    lds_sync();   // the table
#pragma unroll
    for (int m = 0; m < ROUTE_PER_LANE; m++) {
        if (m >= mc) break;
        const int e = l + 64 * m;
        if (e < ne) p[e] = esq_expf_tab(v[m] - mx, tab);
    }
    lds_sync();
    if (l == 0) {   // :754, in expert order: 32 values per batch of LDS reads
        float sum = 0.0f;
        int e = 0;
        for (; e + 32 <= ne; e += 32) {
            float4 q[8];
#pragma unroll
            for (int i = 0; i < 8; i++) q[i] = *reinterpret_cast<const float4 *>(&p[e + 4 * i]);
#pragma unroll
            for (int i = 0; i < 8; i++) {
                sum += q[i].x;
                sum += q[i].y;
                sum += q[i].z;
                sum += q[i].w;
            }
        }
        for (; e < ne; e++) sum += p[e];
        total = sum;
    }
    lds_sync();
    const float sum = total;
    bool nan = false;
#pragma unroll
    for (int m = 0; m < ROUTE_PER_LANE; m++) {
        if (m >= mc) break;
        const int e = l + 64 * m;
        if (e < ne) {
            const float q = p[e] / sum;   // :755
            p[e] = q;
            v[m] = q;
            nan = nan || q != q;
        }
    }
    uint32_t taken = 0;   // bit m: expert l + 64 m
    float wsum = 0.0f, wj = 0.0f;
    int sj = 0;
    if (__ballot(nan) == 0) {
        uint32_t bvb = 0;   // this lane's best untaken value: its bits + 1 (0: none left)
        int bve = 0xffff;   // and its expert (the lowest of that value)
        auto rescan = [&]() {
            bvb = 0;
            bve = 0xffff;
#pragma unroll
            for (int m = 0; m < ROUTE_PER_LANE; m++) {
                if (m >= mc) break;
                const int e = l + 64 * m;
                const uint32_t b = __float_as_uint(v[m]) + 1u;
                if (e < ne && !((taken >> m) & 1u) && b > bvb) { bvb = b; bve = e; }
            }
        };
        rescan();
        for (int j = 0; j < k; j++) {
            const uint32_t vmax = wave_reduce<true>(bvb);
            const int be = (int)wave_reduce<false>(bvb == vmax ? (uint32_t)bve : 0xffffu);
            const float bv = __uint_as_float(vmax - 1u);
            if ((be & 63) == l) {   // the owner drops the pick and finds its next best
                taken |= 1u << (be >> 6);
                rescan();
            }
            wsum += bv;   // w[j] = r[best]; wsum += w[j] (:802-803)
            if (l == j) { wj = bv; sj = be; }
        }
        if (l < k) sel[(size_t)t * kmax + l] = sj;
    } else {
        lds_sync();
        for (int j = 0; j < k; j++) {   // the reference's scan (:794-804), on one lane
            if (l == 0) {
                int be = -1;
                for (int e = 0; e < ne; e++) {
                    bool used = false;
                    for (int i = 0; i < j; i++) used = used || sel[(size_t)t * kmax + i] == e;
                    if (!used && (be < 0 || p[e] > p[be])) be = e;
                }
                sel[(size_t)t * kmax + j] = be;
                wsum += p[be];
                total = p[be];
            }
            lds_sync();
            if (l == j) wj = total;
            lds_sync();
        }
    }
    if (l == 0) total = norm_topk ? (wsum > 6.103515625e-5f ? wsum : 6.103515625e-5f) : 1.0f;   // :832
    lds_sync();
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
    if (q8k) hipLaunchKernelGGL(swiglu_q8k, dim3((rows * (ff / 256) + 3) / 4), dim3(256), 0, s, gu, ff, rows, ha, hstride);
    else hipLaunchKernelGGL(swiglu_q80, dim3((ff + 255) / 256, rows), dim3(256), 0, s, gu, ff, ha, hstride);
    return hipGetLastError();
}

hipError_t moe_combine_launch(const float *ye, const int *rowof, const float *w, const int *k, int kmax, int ntok, int n,
                              float *out, uint64_t ostride, hipStream_t s) {
    if (ntok <= 0) return hipSuccess;
    if (n % 4 == 0 && ostride % 4 == 0 && ((uintptr_t)ye & 15) == 0 && ((uintptr_t)out & 15) == 0)
        hipLaunchKernelGGL(moe_combine4, dim3((n / 4 + 255) / 256, ntok), dim3(256), 0, s, ye, rowof, w, k, kmax, n, out, ostride);
    else
        hipLaunchKernelGGL(moe_combine, dim3((n + 255) / 256, ntok), dim3(256), 0, s, ye, rowof, w, k, kmax, n, out, ostride);
    return hipGetLastError();
}

// ---- device-routed MoE: grouping and job tables --------------------------------------------------------------------
namespace {

// Inclusive prefix sum over the wave's 64 lanes by DPP moves: row_shr 1, 2, 4, 8 (lanes shifted in from outside the row
// add 0), then row_bcast:15 into rows 1 and 3 and row_bcast:31 into rows 2 and 3.
__device__ __forceinline__ int wave_incl_scan(int x) {
    x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xF, 0xF, true);
    x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xA, 0xF, false);
    x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xC, 0xF, false);
    return x;
}

// Exclusive prefix sums of three values per thread of the block (MOE_GROUP_THREADS threads, 16 waves): each wave's scan,
// then the 16 wave totals scanned on one wave. tot receives the three sums.
__device__ int3 block_excl_scan3(int3 v, int3 *wsum, int3 *tot) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int3 x = make_int3(wave_incl_scan(v.x), wave_incl_scan(v.y), wave_incl_scan(v.z));
    if (lane == 63) wsum[w] = x;
    lds_sync();
    if (w == 0) {
        constexpr int NW = MOE_GROUP_THREADS / 64;
        const int3 y0 = lane < NW ? wsum[lane] : make_int3(0, 0, 0);
        const int3 y = make_int3(wave_incl_scan(y0.x), wave_incl_scan(y0.y), wave_incl_scan(y0.z));
        if (lane < NW) wsum[lane] = y;
        if (lane == NW - 1) *tot = y;
    }
    lds_sync();
    const int3 pre = w > 0 ? wsum[w - 1] : make_int3(0, 0, 0);
    lds_sync();   // wsum is reused by the next scan
    return make_int3(pre.x + x.x - v.x, pre.y + x.y - v.y, pre.z + x.z - v.z);
}

__device__ int ceil_div(int a, int b) { return (a + b - 1) / b; }

// One workgroup: moe_n's grouping (src/es_engine.c:871-888) of the ntok * k choices, then every job of the layer's two
// launches. Experts take slots in order of first use; an expert's rows follow its choices in (token, j) order.
// The kernel's arguments as one block (its first and only parameter, at offset 0 of the argument segment).
struct MoeBuildArgs {
    MoeDevArgs A;
    MoeFamily GU, DN;
};
static_assert(sizeof(MoeBuildArgs) % 4 == 0 && sizeof(MoeBuildArgs) / 4 <= MOE_GROUP_THREADS, "one dword per thread");
static_assert(MOE_MAX_PAIRS <= (1 << 20) && ROUTE_MAX_EXPERTS <= 1024, "slot order keys fit an int");

__global__ __launch_bounds__(MOE_GROUP_THREADS) void moe_group_build(MoeBuildArgs P) {
    __shared__ __align__(16) int first[ROUTE_MAX_EXPERTS];
    __shared__ int cnt[ROUTE_MAX_EXPERTS], slot[ROUTE_MAX_EXPERTS], taken[ROUTE_MAX_EXPERTS];
    __shared__ int uex[ROUTE_MAX_EXPERTS], ustart[ROUTE_MAX_EXPERTS];
    __shared__ int wcnt[MOE_GROUP_THREADS / 64][ROUTE_MAX_EXPERTS];   // per wave of a chunk: choices of each expert
    __shared__ int3 wsum[MOE_GROUP_THREADS / 64];
    __shared__ int3 s_tot;
    __shared__ int wfl[MOE_GROUP_THREADS / 64];
    __shared__ __align__(16) MoeBuildArgs sa;
    __shared__ const uint8_t *pg[ROUTE_MAX_EXPERTS], *pu[ROUTE_MAX_EXPERTS], *pd[ROUTE_MAX_EXPERTS];
    const int tid = threadIdx.x, T = MOE_GROUP_THREADS, NE = P.A.n_exp, R = P.A.ntok * P.A.k;
    const int lane = tid & 63, wv = tid >> 6;
    constexpr int NW = MOE_GROUP_THREADS / 64;
    const uint64_t lt = (1ull << lane) - 1;
    // the first chunk's choices and weights, loaded before anything waits on them
    const int sel0 = tid < R ? P.A.sel[tid] : -1;
    const float w0_ = tid < R ? P.A.w[tid] : 0.0f;
    // the arguments into LDS, one dword per thread through vector loads (read as plain scalars, the two families'
    // templates would be loaded in several dependent rounds where the job tables use them), and the experts' matrix
    // pointers: all of these loads are in flight together
    const uint32_t arg = tid < (int)(sizeof(MoeBuildArgs) / 4)
                             ? ((const uint32_t *)__builtin_amdgcn_kernarg_segment_ptr())[tid] : 0u;
    const uint8_t *eg = tid < NE ? P.A.gate[tid] : nullptr, *eu = tid < NE ? P.A.up[tid] : nullptr,
                  *ed = tid < NE ? P.A.down[tid] : nullptr;
    for (int e = tid; e < NE; e += T) {
        first[e] = R;
        cnt[e] = 0;
        taken[e] = 0;
        slot[e] = -1;
    }
    if (tid < (int)(sizeof(MoeBuildArgs) / 4)) reinterpret_cast<uint32_t *>(&sa)[tid] = arg;
    if (tid < NE) {
        pg[tid] = eg;
        pu[tid] = eu;
        pd[tid] = ed;
    }
    const MoeDevArgs &A = P.A;   // pointers from the arguments themselves: the compiler knows them as global memory
    lds_sync();
    for (int p = tid; p < R; p += T) {
        const int e = p < T ? sel0 : A.sel[p];
        if (e >= 0 && e < NE) {
            atomicMin(&first[e], p);
            atomicAdd(&cnt[e], 1);
        }
    }
    lds_sync();
    // slot of a used expert: the number of first uses before its own, a running count over the choices in order (one
    // ballot per wave, then the wave totals)
    int U = 0;
    for (int c0 = 0; c0 < R; c0 += T) {
        const int p = c0 + tid;
        const int e0 = c0 == 0 ? sel0 : p < R ? A.sel[p] : -1;
        const bool fu = p < R && e0 >= 0 && e0 < NE && first[e0] == p;
        const uint64_t b = __ballot(fu);
        if (lane == 0) wfl[wv] = __popcll(b);
        lds_sync();
        int before = U, total = U;
#pragma unroll
        for (int i = 0; i < NW; i++) {
            const int x = wfl[i];
            before += i < wv ? x : 0;
            total += x;
        }
        if (fu) {
            const int r = before + __popcll(b & lt);
            slot[e0] = r;
            uex[r] = e0;
        }
        U = total;
        lds_sync();   // wfl is rewritten by the next chunk; slot and uex are complete
    }
    // slot u's expert
    const int ue = tid < U ? uex[tid] : 0;
    const int c_me = tid < U ? cnt[ue] : 0;   // thread u: slot u's expert's count
    const int st = block_excl_scan3(make_int3(c_me, 0, 0), wsum, &s_tot).x;
    if (tid < NE) ustart[tid] = st;
    // pair rows: the slot's first row + the choices of the same expert before this one, counted in chunks of one choice
    // per thread: earlier chunks (taken), earlier waves of the chunk (wcnt), earlier lanes of the wave (a match mask
    // from ballots over the expert id's bits)
    for (int c0 = 0; c0 < R; c0 += T) {
        for (int i = tid; i < NW * NE; i += T) wcnt[i / NE][i % NE] = 0;
        const int p = c0 + tid;
        const int e0 = c0 == 0 ? sel0 : p < R ? A.sel[p] : -1;
        const int e = e0 >= 0 && e0 < NE ? e0 : -1;
        uint64_t same = __ballot(e >= 0);
        for (int b = 0; b < 10; b++) {   // expert ids < 1024
            const uint64_t m = __ballot(e >= 0 && ((e >> b) & 1));
            same &= ((e >> b) & 1) ? m : ~m;
        }
        lds_sync();
        if (e >= 0 && (same & lt) == 0) wcnt[wv][e] = __popcll(same);   // the wave's first lane with e
        lds_sync();
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
        lds_sync();
        if (p < R && e >= 0 && (same & lt) == 0) atomicAdd(&taken[e], __popcll(same));
        lds_sync();
    }
    // ---- job tables. With a decode-kernel family, slots go by token count, most first (ties in slot order), so the
    // launch starts its longest workgroups first (the expert-sized and matrix-core families keep slot order, which
    // measured as fast); the pair rows keep their slot order. Thread r writes the jobs of the slot ranked r; tiles and
    // pre-pass items are prefix sums in that order. (first, slot and taken are free once the rows are placed.)
    const bool by_count = sa.GU.kind == MOE_FAM_MV || sa.DN.kind == MOE_FAM_MV;
    // slot u's order key: its count, then the earlier slot first (counts <= MOE_MAX_PAIRS and slots < 1024, so the key
    // fits 25 bits and no two are equal); keys padded with -1 to a multiple of four
    const int U4 = (U + 3) & ~3;
    if (by_count) {
        if (tid < U4) first[tid] = tid < U ? c_me << 10 | (1023 - tid) : -1;
        if (tid < U) slot[tid] = 0;   // the ranks' partial counts
        lds_sync();
        // rank of slot u = the keys above its own: thread t counts slot t % S's among keys part t / S of PARTS (S the
        // power of two >= U), the parts' counts added in LDS
        const int S = U <= 1 ? 1 : 1 << (32 - __builtin_clz(U - 1)), parts = MOE_GROUP_THREADS / S;
        const int su = tid & (S - 1), part = tid / S;
        const int q4 = U4 >> 2, per = (q4 + parts - 1) / parts, v0 = part * per, v1 = min(q4, v0 + per);
        if (su < U && v0 < v1) {
            const int me = first[su];
            const int4 *f4 = reinterpret_cast<const int4 *>(first);
            int r = 0;
            for (int v = v0; v < v1; v++) {   // four keys per read, the same address for every lane of a part
                const int4 q = f4[v];
                r += (q.x > me ? 1 : 0) + (q.y > me ? 1 : 0) + (q.z > me ? 1 : 0) + (q.w > me ? 1 : 0);
            }
            atomicAdd(&slot[su], r);
        }
        lds_sync();
        if (tid < U) taken[slot[tid]] = tid;
    } else if (tid < U) {
        taken[tid] = tid;
    }
    lds_sync();
    const int u = tid < U ? taken[tid] : tid;   // the slot whose jobs this thread writes, at position tid
    const bool real = u < U;
    const int uexp = real ? uex[u] : 0;
    const int c = real ? cnt[uexp] : 0, s0 = real ? ustart[u] : 0;
    const uint8_t *wg_u = pg[uexp], *wu_u = pu[uexp], *wd_u = pd[uexp];
    const int ff = A.ff, n = A.n;
    for (int prod = 0; prod < 2; prod++) {   // 0: gate/up, 1: down
        const MoeFamily &F = prod ? sa.DN : sa.GU;
        const int njob = prod || (F.kind == MOE_FAM_MX && F.gated) ? 1 : 2;   // gated: gate and up in one job
        int ntok = 0, tiles = 0, items = 0, units = 0;
        if (F.kind == MOE_FAM_MX && real) {
            ntok = ceil_div(c, MX_TOK);
            tiles = njob * (ntok == 1 ? F.mx_tiles : F.row_tiles8 * ntok);
        }
        if (F.kind == MOE_FAM_MM && real) {
            ntok = ceil_div(c, F.bn);
            tiles = njob * F.row_tiles8 * ntok;
            const int per = F.pj.nbk * (int)prep_words(F.pj.kind);
            items = ceil_div(ntok * F.bn * per, PREP_SPAN) * PREP_SPAN;
            // the expert's planes in 256-byte units: values [nbk][na_pad][256], then meta + scales [nbk][na_pad][36]
            units = ceil_div(F.pj.nbk * ntok * F.bn * 256, 256) + ceil_div(F.pj.nbk * ntok * F.bn * 36, 256);
        }
        int tot_tiles = 0, tot_items = 0, w0 = 0;
        if (F.kind != MOE_FAM_MV) {   // uniform across the block: every thread takes part in the scan
            const int3 sc = block_excl_scan3(make_int3(tiles, items, units), wsum, &s_tot);
            tot_tiles = s_tot.x;
            tot_items = s_tot.y;
            tiles = sc.x;
            items = sc.y;
            w0 = sc.z;
        }
        const int t0 = tiles, i0 = items;
        const uint8_t *wsrc = prod ? wd_u : wg_u;
        if (F.kind == MOE_FAM_MV) {
            MvJob *jobs = static_cast<MvJob *>(prod ? A.dn_jobs : A.gu_jobs);
            const int end = njob * U * F.mv_tiles;
            if (tid < A.umax)
                for (int g = 0; g < njob; g++) {
                    MvJob J = F.mv;
                    if (real) {
                        J.W = g ? wu_u : wsrc;
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
                        J.nt = min(J.nt, c >= 3 ? 4 : c);   // the planner's width for c activations, within the LDS sizing
                        J.tile0 = (njob * tid + g) * F.mv_tiles;
                    } else {   // empty: the template's valid pointers, no rows, no activations, after the last real tile
                        J.na = 0;
                        J.r0 = J.r1 = 0;
                        J.tile0 = end;
                    }
                    jobs[njob * tid + g] = J;
                }
            if (tid == 0) {   // the sentinel
                MvJob J = F.mv;
                J.na = 0;
                J.r0 = J.r1 = 0;
                J.tile0 = end;
                jobs[njob * A.umax] = J;
            }
        } else if (F.kind == MOE_FAM_MX) {
            MkJob *jobs = static_cast<MkJob *>(prod ? A.dn_jobs : A.gu_jobs);
            if (tid < A.umax)
                for (int g = 0; g < njob; g++) {
                    MkJob J = F.mk;
                    if (real) {
                        J.W = g ? wu_u : wsrc;
                        J.act = prod ? A.ha + (size_t)s0 * A.hstride : A.x;
                        J.arow = prod ? nullptr : A.tok_of + s0;
                        J.y = prod ? A.bye + (size_t)s0 * n : A.bgu + (size_t)s0 * 2 * ff + (size_t)g * ff;
                        if (!prod && F.gated) {   // h's Q8_K blocks of the expert's first pair row
                            J.W2 = wu_u;
                            J.y = reinterpret_cast<float *>(A.ha + (size_t)s0 * A.hstride);
                        }
                        J.na = c;
                        J.ntok_tiles = ntok;
                        J.tile0 = t0 + g * (ntok == 1 ? F.mx_tiles : F.row_tiles8 * ntok);
                    } else {
                        J.na = 0;
                        J.r0 = J.r1 = 0;
                        J.ntok_tiles = 1;
                        J.tile0 = tot_tiles;
                    }
                    jobs[njob * tid + g] = J;
                }
            if (tid == 0) {
                MkJob J = F.mk;
                J.na = 0;
                J.r0 = J.r1 = 0;
                J.ntok_tiles = 1;
                J.tile0 = tot_tiles;
                jobs[njob * A.umax] = J;
            }
        } else {
            MmJob *jobs = static_cast<MmJob *>(prod ? A.dn_jobs : A.gu_jobs);
            PrepJob *pj = prod ? A.dn_prep : A.gu_prep;
            uint8_t *ws = prod ? A.dn_ws : A.gu_ws;
            if (tid < A.umax) {
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
                pj[tid] = P;
                for (int g = 0; g < njob; g++) {
                    MmJob J = F.mm;
                    if (real) {
                        J.W = g ? wu_u : wsrc;
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
                    jobs[njob * tid + g] = J;
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
        lds_sync();
    }
}

}  // namespace

hipError_t moe_group_build_launch(const MoeDevArgs &a, const MoeFamily &gu, const MoeFamily &dn, hipStream_t s) {
    const MoeBuildArgs P{a, gu, dn};
    hipLaunchKernelGGL(moe_group_build, dim3(1), dim3(MOE_GROUP_THREADS), 0, s, P);
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
