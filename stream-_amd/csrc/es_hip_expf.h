// expf as the reference's host computes it, for the device.
//
// The reference's SwiGLU (src/es_engine.c:913) and router softmax (:755) call the C library's expf. On its x86-64 Linux
// hosts that is glibc's (2.27 and later), which evaluates the method of Szabolcs Nagy's expf from Arm's
// optimized-routines: with N = 32,
//   z = x * N/ln2 (double), k = round-to-nearest-integer(z) (by adding 1.5 * 2^52), r = z - k (fused),
//   2^(k/N) = the double whose bits are T[k mod N] + (k << 47), where T[i] = bits(2^(i/N)) - (i << 47),
//   exp(x) ~= 2^(k/N) * (C0 r^3 + C1 r^2 + C2 r + 1) with the polynomial in Horner form over fused multiply-adds,
//   and one rounding of the double result to float. Inputs above log(2^128) overflow to +inf, inputs below log(2^-150)
//   underflow to +0, NaN passes through.
// glibc selects a build of that routine with fused multiply-adds on CPUs that have them (every x86-64 host of the GPU
// boxes); the fusions above are that build's. The table entries are 2^(i/32) rounded to double (computed from the
// definition); the polynomial coefficients are the published ones. Checked bit-for-bit against the host's expf over all
// 2^32 float inputs by tests/test_expf.py, which compiles this header for the CPU.
//
// ESQ_EXPF_QUAL is the function qualifier: __device__ in the library, plain static inline in the CPU check.
#ifndef ES_HIP_EXPF_H
#define ES_HIP_EXPF_H
#include <stdint.h>

#ifndef ESQ_EXPF_QUAL
#define ESQ_EXPF_QUAL __device__ __forceinline__
#endif

// T[i] = bits(2^(i/32)) - (i << 47)
#define ESQ_EXPF_TABLE                                                                         \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

// the routine with its table passed in (a kernel may keep a copy in LDS): T is indexed as T[i]
template <typename TAB> ESQ_EXPF_QUAL float esq_expf_tab(float x, const TAB &T) {
    if (x != x) return x + x;
    if (x > 0x1.62e42ep6f) return __builtin_inff();   // > log(2^128)
    if (x < -0x1.9fe368p6f) return 0.0f;              // < log(2^-150)
    const double N = 32.0;
    const double C0 = 0x1.c6af84b912394p-5 / (N * N * N), C1 = 0x1.ebfce50fac4f3p-3 / (N * N), C2 = 0x1.62e42ff0c52d6p-1 / N;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * N, shift = 0x1.8p+52;
    const double xd = x;
    double kd = inv_ln2_n * xd + shift;   // two roundings: the product, then the sum (rounds to an integer)
    const uint64_t ki = __builtin_bit_cast(uint64_t, kd);
    kd -= shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double s = __builtin_bit_cast(double, (uint64_t)T[ki % 32] + (ki << 47));
    const double z = __builtin_fma(C0, r, C1), r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    return static_cast<float>(y * s);
}

ESQ_EXPF_QUAL float esq_expf(float x) {
    static constexpr uint64_t T[32] = ESQ_EXPF_TABLE;
    return esq_expf_tab(x, T);
}

#endif
