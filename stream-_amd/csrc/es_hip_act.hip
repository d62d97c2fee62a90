// Activation preparation on the device: es_act_prepare (src/es_quant.c:499-512) for rows of fp32 values, fused with what
// produces them in the engine:
//   plain rows                       -> Q8_0 (quantize_q80, src/es_quant.c:489-497) and / or Q8_K (es_quantize_q8_K,
//                                       src/es_q2k.c:102-125) blocks;
//   rmsnorm (src/es_engine.c:189-194) -> the normalised row (optional) and its blocks;
//   SwiGLU of gate|up rows (dense_n / moe_n, src/es_engine.c:957-972, 913-914) -> h (optional) and its blocks.
// The reference builds these loops for baseline x86-64 (no FMA), so every product and sum rounds on its own; this file is
// built with -ffp-contract=off and spells no fused operation. Division and square root are IEEE (correctly rounded), in
// float and in double; expf follows glibc's method bit for bit (es_hip_expf.h).
#include "es_hip_common.h"
#include "es_hip_expf.h"

namespace esq {
namespace {

struct QuantOut {
    uint8_t *q80;   // this row's Q8_0 blocks, or null
    uint8_t *q8k;   // this row's Q8_K blocks, or null
};

// The workgroup's 256 threads hold elements e0 .. e0 + 255 of a row (thread i: value v of element e0 + i when `have`);
// e0 is a multiple of 256. Q8_0 blocks are formed by half-waves (32 consecutive elements, all present or all absent: the
// row length is a multiple of 32), the Q8_K block by the whole workgroup (only asked for when the row length is a
// multiple of 256). Every thread of the workgroup must call this (it synchronises the workgroup for the Q8_K maximum).
__device__ __forceinline__ void quant_chunk(float v, bool have, int e0, const QuantOut &o, float *wmax) {
    const int i = threadIdx.x, e = e0 + i;
    if (o.q80) {   // quantize_q80: d = amax / 127, id = 1 / d (0 when d is 0), q = (int)(v * id +- 0.5)
        float a = have ? __builtin_fabsf(v) : 0.0f;
        for (int s = 16; s > 0; s >>= 1) a = __builtin_fmaxf(a, __shfl_xor(a, s, 32));   // a maximum is exact in any order
        if (have) {
            const float d = a / 127.0f, id = d != 0.0f ? 1.0f / d : 0.0f;
            const float x = v * id;
            const int q = static_cast<int>(x < 0.0f ? x - 0.5f : x + 0.5f);
            uint8_t *blk = o.q80 + (size_t)(e >> 5) * 36;
            blk[4 + (e & 31)] = static_cast<uint8_t>(static_cast<int8_t>(q));
            if ((e & 31) == 0) *reinterpret_cast<float *>(blk) = d;
        }
    }
    if (o.q8k) {   // es_quantize_q8_K: id = 127 / amax, q = lrintf(v * id) clamped to +-127, d = amax / 127, bsums
        float a = __builtin_fabsf(v);
        for (int s = 32; s > 0; s >>= 1) a = __builtin_fmaxf(a, __shfl_xor(a, s));
        __syncthreads();   // wmax may still be read by the previous chunk
        if ((i & 63) == 0) wmax[i >> 6] = a;
        __syncthreads();
        const float amax = __builtin_fmaxf(__builtin_fmaxf(wmax[0], wmax[1]), __builtin_fmaxf(wmax[2], wmax[3]));
        uint8_t *blk = o.q8k + (size_t)(e0 >> 8) * 292;
        int q = 0;
        if (amax != 0.0f) {   // a zero block is all zeros (d, qs and bsums)
            const float id = 127.0f / amax;
            q = static_cast<int>(__builtin_rintf(v * id));   // lrintf: round to nearest even
            q = q > 127 ? 127 : q < -127 ? -127 : q;
        }
        blk[4 + i] = static_cast<uint8_t>(static_cast<int8_t>(q));
        int s = q;   // sums of 16 consecutive qs
        for (int m = 8; m > 0; m >>= 1) s += __shfl_xor(s, m, 16);
        if ((i & 15) == 0) reinterpret_cast<int16_t *>(blk + 260)[i >> 4] = static_cast<int16_t>(s);
        if (i == 0) *reinterpret_cast<float *>(blk) = amax != 0.0f ? amax / 127.0f : 0.0f;
    }
}

constexpr int CHUNKS = 4;   // 256-wide chunks per workgroup of the SwiGLU form (all loads issued first)

// Rows of fp32 values: grid (groups of CHUNKS chunks of 256, rows).
template <int CHUNKS>
__global__ __launch_bounds__(256) void act_prep_plain(const float *__restrict__ x, uint64_t xs, int cols, uint8_t *q80,
                                                      uint64_t q80s, uint8_t *q8k, uint64_t q8ks) {
    __shared__ float wmax[4];
    const int r = blockIdx.y, c0 = blockIdx.x * CHUNKS;
    const float *xr = x + (size_t)r * xs;
    float v[CHUNKS];
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int e = (c0 + c) * 256 + threadIdx.x;
        v[c] = e < cols ? xr[e] : 0.0f;
    }
    const QuantOut o{q80 ? q80 + (size_t)r * q80s : nullptr, q8k ? q8k + (size_t)r * q8ks : nullptr};
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int e0 = (c0 + c) * 256;
        if (e0 >= cols) break;   // uniform
        quant_chunk(v[c], e0 + (int)threadIdx.x < cols, e0, o, wmax);
    }
}

// SwiGLU of gate|up rows (gate at gu[r][0, ff), up at gu[r][ff, 2 ff)): grid (groups of CHUNKS chunks of 256, rows).
__global__ __launch_bounds__(256) void act_prep_swiglu(const float *__restrict__ gu, uint64_t gs, int ff, float *h, uint64_t hs,
                                                       uint8_t *q80, uint64_t q80s, uint8_t *q8k, uint64_t q8ks) {
    __shared__ float wmax[4];
    __shared__ uint64_t tab[32];   // expf's table in LDS: its load goes out beside the row's
    {
        static constexpr uint64_t T[32] = ESQ_EXPF_TABLE;
        if (threadIdx.x < 32) tab[threadIdx.x] = T[threadIdx.x];
    }
    const int r = blockIdx.y, c0 = blockIdx.x * CHUNKS;
    const float *g = gu + (size_t)r * gs;
    float gv[CHUNKS], uv[CHUNKS];
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int e = (c0 + c) * 256 + threadIdx.x;
        gv[c] = e < ff ? g[e] : 0.0f;
        uv[c] = e < ff ? g[ff + e] : 0.0f;
    }
    __syncthreads();
    const QuantOut o{q80 ? q80 + (size_t)r * q80s : nullptr, q8k ? q8k + (size_t)r * q8ks : nullptr};
#pragma unroll
    for (int c = 0; c < CHUNKS; c++) {
        const int e0 = (c0 + c) * 256, e = e0 + threadIdx.x;
        if (e0 >= ff) break;   // uniform
        const bool have = e < ff;
        float v = 0.0f;
        if (have) {
            v = gv[c] / (1.0f + esq_expf_tab(-gv[c], tab)) * uv[c];
            if (h) h[(size_t)r * hs + e] = v;
        }
        quant_chunk(v, have, e0, o, wmax);
    }
}

// rmsnorm, then the blocks: one workgroup per row. Every thread squares its elements in double (exact) into LDS; one
// thread adds them in element order (the reference's rounding; the dependent adds are the kernel's critical path), then
// every thread takes its elements of each 256-wide chunk.
__global__ __launch_bounds__(256) void act_prep_rms(const float *__restrict__ x, uint64_t xs, const float *__restrict__ w,
                                                    float eps, int cols, float *xn, uint64_t xns, uint8_t *q80, uint64_t q80s,
                                                    uint8_t *q8k, uint64_t q8ks) {
    extern __shared__ __align__(16) double sq[];   // cols squares (the host keeps cols a multiple of 32)
    __shared__ float wmax[4];
    __shared__ float scale;
    const int r = blockIdx.x, i = threadIdx.x;
    const float *xr = x + (size_t)r * xs;
    for (int e = i; e < cols; e += 256) {
        const double d = static_cast<double>(xr[e]);
        sq[e] = d * d;   // exact: a float's square fits a double
    }
    __syncthreads();
    if (i == 0) {   // two alternating batches of 16 squares: one batch's LDS reads are in flight while the other is added
        double ss = 0.0;
        const double2 *s2 = reinterpret_cast<const double2 *>(sq);
        double2 a[8], b[8];
#pragma unroll
        for (int k = 0; k < 8; k++) a[k] = s2[k];
        for (int e = 0; e < cols; e += 32) {   // cols is a multiple of 32
#pragma unroll
            for (int k = 0; k < 8; k++) b[k] = s2[e / 2 + 8 + k];
#pragma unroll
            for (int k = 0; k < 8; k++) {
                ss = ss + a[k].x;
                ss = ss + a[k].y;
            }
            if (e + 32 < cols) {
#pragma unroll
                for (int k = 0; k < 8; k++) a[k] = s2[e / 2 + 16 + k];
            }
#pragma unroll
            for (int k = 0; k < 8; k++) {
                ss = ss + b[k].x;
                ss = ss + b[k].y;
            }
        }
        scale = static_cast<float>(1.0 / __builtin_sqrt(ss / static_cast<double>(cols) + static_cast<double>(eps)));
    }
    __syncthreads();
    const float s = scale;
    const QuantOut o{q80 ? q80 + (size_t)r * q80s : nullptr, q8k ? q8k + (size_t)r * q8ks : nullptr};
    for (int e0 = 0; e0 < cols; e0 += 256) {   // uniform trip count: every thread reaches quant_chunk's barriers
        const int e = e0 + i;
        const bool have = e < cols;
        float v = 0.0f;
        if (have) {
            v = xr[e] * s * (w ? w[e] : 1.0f);
            if (xn) xn[(size_t)r * xns + e] = v;
        }
        quant_chunk(v, have, e0, o, wmax);
    }
}

}  // namespace

hipError_t act_prep_launch(const float *x, uint64_t xs, int rows, int cols, uint8_t *q80, uint64_t q80s, uint8_t *q8k,
                           uint64_t q8ks, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(act_prep_plain<1>, dim3((cols + 255) / 256, rows), dim3(256), 0, s, x, xs, cols, q80, q80s, q8k, q8ks);
    return hipGetLastError();
}

hipError_t act_prep_swiglu_launch(const float *gu, uint64_t gs, int rows, int ff, float *h, uint64_t hs, uint8_t *q80,
                                  uint64_t q80s, uint8_t *q8k, uint64_t q8ks, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    hipLaunchKernelGGL(act_prep_swiglu, dim3((ff + 256 * CHUNKS - 1) / (256 * CHUNKS), rows), dim3(256), 0, s, gu, gs, ff, h, hs,
                       q80, q80s, q8k, q8ks);
    return hipGetLastError();
}

hipError_t act_prep_rms_launch(const float *x, uint64_t xs, const float *w, float eps, int rows, int cols, float *xn,
                               uint64_t xns, uint8_t *q80, uint64_t q80s, uint8_t *q8k, uint64_t q8ks, hipStream_t s) {
    if (rows <= 0) return hipSuccess;
    const size_t lds = (size_t)cols * sizeof(double);
    if (lds > 64 * 1024) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(act_prep_rms), hipFuncAttributeMaxDynamicSharedMemorySize,
                                           static_cast<int>(lds));
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL(act_prep_rms, dim3(rows), dim3(256), lds, s, x, xs, w, eps, cols, xn, xns, q80, q80s, q8k, q8ks);
    return hipGetLastError();
}

}  // namespace esq
