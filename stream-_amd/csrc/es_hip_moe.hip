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
