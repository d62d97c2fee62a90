// es_dequant_row on the device (src/es_quant.c:425-476, src/es_q2k.c:88-100): n weights of one format to fp32, each
// element by its format's formula in the reference's operation order (the products and differences round separately:
// this file is built with -ffp-contract=off). One thread per element; a workgroup of 256 threads covers one 256-element
// superblock or eight 32-element blocks. Also the float path of es_matvec for activations that have no Q8 blocks
// (fdot_kernel below), which dequantizes with the same element formula.
#include "es_hip_common.h"

namespace esq {
namespace {

template <typename P> __device__ __forceinline__ float h2f(P p) { return half_bits_to_float(p[0] | (uint32_t)p[1] << 8); }

// scale_min_k4 (src/es_quant.c:75-83)
template <typename P> __device__ __forceinline__ void scale_min(P q, int j, int &sc, int &mn) {
    if (j < 4) { sc = q[j] & 63; mn = q[j + 4] & 63; }
    else { sc = (q[j + 4] & 15) | ((q[j - 4] >> 6) << 4); mn = (q[j + 4] >> 4) | ((q[j] >> 6) << 4); }
}

// Element e of the block at p, in the reference's formula and order for the format. p may point to global memory or
// to a copy of the block in LDS.
template <int F, typename P> __device__ __forceinline__ float deq_elem(P p, int e) {
    float v;
    if constexpr (F == ES_HIP_Q4_0) {   // (x - 8) * d  (:433-449)
        const int q = e < 16 ? p[2 + e] & 15 : p[2 + e - 16] >> 4;
        v = static_cast<float>(q - 8) * h2f(p);
    } else if constexpr (F == ES_HIP_Q5_0) {   // (x - 16) * d, fifth bit e of qh  (:451-468)
        const uint32_t qh = p[2] | (uint32_t)p[3] << 8 | (uint32_t)p[4] << 16 | (uint32_t)p[5] << 24;
        const int q = (e < 16 ? p[6 + e] & 15 : p[6 + e - 16] >> 4) | (int)(((qh >> e) & 1u) << 4);
        v = static_cast<float>(q - 16) * h2f(p);
    } else if constexpr (F == ES_HIP_Q8_0) {   // d * q  (:425-431)
        v = h2f(p) * static_cast<float>(static_cast<int8_t>(p[2 + e]));
    } else if constexpr (F == ES_HIP_Q4_K || F == ES_HIP_Q5_K) {   // d1 * q - m1  (:117-154)
        const int c = e >> 6, hi = (e >> 5) & 1, l = e & 31, j = 2 * c + hi;
        int sc, mn;
        scale_min(p + 4, j, sc, mn);
        const auto qs = p + (F == ES_HIP_Q4_K ? 16 : 48);
        int q = hi ? qs[32 * c + l] >> 4 : qs[32 * c + l] & 15;
        if constexpr (F == ES_HIP_Q5_K) q += ((p[16 + l] >> j) & 1) ? 16 : 0;
        const float d1 = h2f(p) * static_cast<float>(sc), m1 = h2f(p + 2) * static_cast<float>(mn);
        v = d1 * static_cast<float>(q) - m1;
    } else if constexpr (F == ES_HIP_Q6_K) {   // d * sc * (q - 32)  (:156-181)
        const int h = e >> 7, k = (e >> 5) & 3, l = e & 31;
        const uint8_t a = p[64 * h + 32 * (k & 1) + l], hb = p[128 + 32 * h + l];
        const int q = ((k >> 1 ? a >> 4 : a & 15) | (((hb >> (2 * k)) & 3) << 4)) - 32;
        const int is = 8 * h + l / 16 + 2 * k;
        v = h2f(p + 208) * static_cast<float>(static_cast<int8_t>(p[192 + is])) * static_cast<float>(q);
    } else if constexpr (F == ES_HIP_Q3_K) {   // d * (sc - 32) * (q - (hbit ? 0 : 4))  (:85-115)
        const int g = e >> 4, l = e & 15, n = g >> 3, j = (g >> 1) & 3, half = g & 1;
        const int lo = g < 8 ? p[96 + g] & 15 : p[96 + g - 8] >> 4;
        const int sc = (lo | (((p[104 + (g & 3)] >> (2 * (g >> 2))) & 3) << 4)) - 32;
        const int q = ((p[32 + 32 * n + 16 * half + l] >> (2 * j)) & 3) - (((p[16 * half + l] >> (4 * n + j)) & 1) ? 0 : 4);
        v = (h2f(p + 108) * static_cast<float>(sc)) * static_cast<float>(q);
    } else {   // Q2_K: d * (sc & 15) * q - dmin * (sc >> 4)  (src/es_q2k.c:88-100)
        const int g = e >> 4, l = e & 15, w = g & 7;
        const int q = (p[16 + 32 * (g >> 3) + 16 * (w & 1) + l] >> ((w >> 1) * 2)) & 3;
        const float dl = h2f(p + 80) * static_cast<float>(p[g] & 15), ml = h2f(p + 82) * static_cast<float>(p[g] >> 4);
        v = dl * static_cast<float>(q) - ml;
    }
    return v;
}

template <int F>
__global__ __launch_bounds__(256) void dequant_kernel(const uint8_t *__restrict__ src, float *__restrict__ dst, long nblk) {
    constexpr int BE = Fmt<F>::BE, BB = Fmt<F>::BB;
    constexpr int PER = 256 / BE;   // blocks per workgroup
    const long b = (long)blockIdx.x * PER + threadIdx.x / BE;
    const int e = threadIdx.x % BE;
    if (b >= nblk) return;
    stg<float>(dst + (size_t)b * BE + e, deq_elem<F>(src + (size_t)b * BB, e));
}

// The float path (src/es_quant.c:1941-1944, dot_f32 at :514-526): y[q * ystride + r] for r in [r0, r1) and q in [0, na),
// the dequantized row r dotted with activation q's floats through four running sums, s_j over the elements i = j (mod 4)
// in increasing i, each product and each sum rounded on its own, then (s0 + s1) + (s2 + s3). The sums are sequential by
// definition, so the parallelism is over (row, activation, running sum): a workgroup owns RT rows x AT activations, four
// consecutive lanes per pair, one per running sum. For each chunk of 256 columns the rows' raw blocks are copied into LDS
// (2-byte loads: every format's block size is even), dequantized there into an fp32 tile, the activations' floats copied
// beside it, and each lane adds its 64 products in order. The four lanes of a pair combine their sums at the end.
template <int F, int RT, int AT>
__global__ __launch_bounds__(4 * RT * AT) void fdot_kernel(const uint8_t *__restrict__ W, size_t rb, int r0, int r1, int cols,
                                                          const float *__restrict__ x, size_t xstride, int na,
                                                          float *__restrict__ y, size_t ystride) {
    constexpr int NT = 4 * RT * AT, C = 256, WP = C + 4;   // threads; columns per chunk; fp32 tile row pitch
    constexpr int BE = Fmt<F>::BE, BB = Fmt<F>::BB, CH = C / BE * BB / 2;   // half-words of one row's full chunk
    __shared__ __align__(16) uint16_t raw[RT * CH];
    __shared__ __align__(16) float wt[RT * WP];
    __shared__ __align__(16) float xt[AT * C];
    const int tid = threadIdx.x, chain = tid & 3, o = tid >> 2, rl = o % RT, al = o / RT;
    const int rbase = r0 + blockIdx.x * RT, abase = blockIdx.y * AT;
    const int nr = min(RT, r1 - rbase), nx = min(AT, na - abase);
    const uint8_t *wrow = W + rb * rbase;
    float s = 0.f;
    for (int c0 = 0; c0 < cols; c0 += C) {
        const int n = min(C, cols - c0), hw = n / BE * BB / 2;   // columns and half-words of each row in this chunk
        const uint8_t *wc = wrow + (size_t)(c0 / BE) * BB;
        __syncthreads();   // the previous chunk's tiles are no longer read
#pragma unroll 4
        for (int i = tid; i < RT * CH; i += NT) {
            const int r = i / CH, k = i - r * CH;
            if (r < nr && k < hw) raw[i] = ldg<uint16_t>(wc + rb * r + 2 * k);
        }
#pragma unroll 4
        for (int i = tid; i < AT * C; i += NT) {
            const int a = i / C, k = i % C;
            if (a < nx && k < n) xt[i] = ldg<float>(x + (size_t)(abase + a) * xstride + c0 + k);
        }
        __syncthreads();
#pragma unroll 4
        for (int i = tid; i < RT * C; i += NT) {
            const int r = i / C, k = i % C;
            if (r < nr && k < n)
                wt[r * WP + k] = deq_elem<F>(reinterpret_cast<const uint8_t *>(raw) + 2 * CH * r + k / BE * BB, k % BE);
        }
        __syncthreads();
        if (rl < nr && al < nx) {
            const float *wr = wt + rl * WP, *xr = xt + al * C;
#pragma unroll 8
            for (int k = chain; k < n; k += 4) s = s + wr[k] * xr[k];
        }
    }
    float t = s + __shfl_xor(s, 1);   // chain 0: s0 + s1, chain 2: s2 + s3
    t = t + __shfl_xor(t, 2);         // chain 0: (s0 + s1) + (s2 + s3)
    if (chain == 0 && rl < nr && al < nx) stg<float>(y + (size_t)(abase + al) * ystride + rbase + rl, t);
}

template <int F> hipError_t fdot_go(const uint8_t *W, size_t rb, int r0, int r1, int cols, const float *x, size_t xstride,
                                    int na, float *y, size_t ystride, hipStream_t s) {
    const unsigned rows = (unsigned)(r1 - r0);
    if (na == 1)   // decode: 16 rows per one-wave workgroup
        hipLaunchKernelGGL((fdot_kernel<F, 16, 1>), dim3((rows + 15) / 16, 1), dim3(64), 0, s, W, rb, r0, r1, cols, x,
                           xstride, na, y, ystride);
    else
        hipLaunchKernelGGL((fdot_kernel<F, 8, 8>), dim3((rows + 7) / 8, (unsigned)((na + 7) / 8)), dim3(256), 0, s, W, rb,
                           r0, r1, cols, x, xstride, na, y, ystride);
    return hipGetLastError();
}

template <int F> hipError_t launch(const uint8_t *src, float *dst, long n, hipStream_t s) {
    constexpr int BE = Fmt<F>::BE, PER = 256 / BE;
    const long nblk = n / BE;
    hipLaunchKernelGGL(dequant_kernel<F>, dim3((unsigned)((nblk + PER - 1) / PER)), dim3(256), 0, s, src, dst, nblk);
    return hipGetLastError();
}

}  // namespace

hipError_t dequant_launch(uint32_t type, const void *src, float *dst, long n, hipStream_t s) {
    const uint8_t *p = static_cast<const uint8_t *>(src);
    switch (type) {
    case ES_HIP_Q4_0: return launch<ES_HIP_Q4_0>(p, dst, n, s);
    case ES_HIP_Q5_0: return launch<ES_HIP_Q5_0>(p, dst, n, s);
    case ES_HIP_Q8_0: return launch<ES_HIP_Q8_0>(p, dst, n, s);
    case ES_HIP_Q2_K: return launch<ES_HIP_Q2_K>(p, dst, n, s);
    case ES_HIP_Q3_K: return launch<ES_HIP_Q3_K>(p, dst, n, s);
    case ES_HIP_Q4_K: return launch<ES_HIP_Q4_K>(p, dst, n, s);
    case ES_HIP_Q5_K: return launch<ES_HIP_Q5_K>(p, dst, n, s);
    case ES_HIP_Q6_K: return launch<ES_HIP_Q6_K>(p, dst, n, s);
    }
    return hipErrorInvalidValue;
}

hipError_t fdot_launch(uint32_t type, const void *W, size_t rb, int r0, int r1, int cols, const float *x, size_t xstride,
                       int na, float *y, size_t ystride, hipStream_t s) {
    const uint8_t *p = static_cast<const uint8_t *>(W);
    switch (type) {
    case ES_HIP_Q4_0: return fdot_go<ES_HIP_Q4_0>(p, rb, r0, r1, cols, x, xstride, na, y, ystride, s);
    case ES_HIP_Q5_0: return fdot_go<ES_HIP_Q5_0>(p, rb, r0, r1, cols, x, xstride, na, y, ystride, s);
    case ES_HIP_Q8_0: return fdot_go<ES_HIP_Q8_0>(p, rb, r0, r1, cols, x, xstride, na, y, ystride, s);
    case ES_HIP_Q2_K: return fdot_go<ES_HIP_Q2_K>(p, rb, r0, r1, cols, x, xstride, na, y, ystride, s);
    case ES_HIP_Q3_K: return fdot_go<ES_HIP_Q3_K>(p, rb, r0, r1, cols, x, xstride, na, y, ystride, s);
    case ES_HIP_Q4_K: return fdot_go<ES_HIP_Q4_K>(p, rb, r0, r1, cols, x, xstride, na, y, ystride, s);
    case ES_HIP_Q5_K: return fdot_go<ES_HIP_Q5_K>(p, rb, r0, r1, cols, x, xstride, na, y, ystride, s);
    case ES_HIP_Q6_K: return fdot_go<ES_HIP_Q6_K>(p, rb, r0, r1, cols, x, xstride, na, y, ystride, s);
    }
    return hipErrorInvalidValue;
}

}  // namespace esq
