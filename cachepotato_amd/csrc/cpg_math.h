/* cpg_math.h — arithmetic shared by the host C code and the HIP kernels.
 *
 * Everything here is integer arithmetic or IEEE-754 operations with one defined rounding
 * (f32/f64 add, multiply, divide, fused multiply-add, conversions), so the host (gcc) and
 * the GPU (hipcc, gfx950) produce identical bits.
 *
 *  - fp16 <-> fp32 and fp64 -> fp16 conversions (Q4_0/Q8_0 scales, format/SPEC.md:157-197)
 *  - the counter-based normal generator that makes the synthetic weights and inputs
 *  - the Q4_0 / Q8_0 encoders (the arithmetic of format/q4.py:30-57, format/q8.py:35-58)
 *  - expf with glibc 2.35's results (used by the router softmax, kernels.c:20-26)
 */
#ifndef CPG_MATH_H
#define CPG_MATH_H
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define CPG_HD __host__ __device__ static inline
#else
#include <math.h>
#define CPG_HD static inline
#endif

CPG_HD uint32_t cpg_f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
CPG_HD float cpg_bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
CPG_HD uint64_t cpg_f64_bits(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
CPG_HD double cpg_bits_f64(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

/* fp16 bits -> fp32 (exact: fp16 is a subset of fp32). Same values as the reference's
   f16_to_f32 (engine/kernels/kernels.c:109-130), including subnormals, inf and NaN. */
CPG_HD float cpg_f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1Fu;
    uint32_t m = h & 0x3FFu;
    if (e == 31) return cpg_bits_f32(sign | 0x7F800000u | (m << 13));
    if (e != 0) return cpg_bits_f32(sign | ((e + 112u) << 23) | (m << 13));
    if (m == 0) return cpg_bits_f32(sign);
    /* subnormal: m * 2^-24, exact in fp32 */
    const float v = (float)m * 5.9604644775390625e-08f;
    return (h & 0x8000u) ? -v : v;
}

/* fp64 -> fp16 bits, round to nearest even, subnormal results, overflow to infinity. */
CPG_HD uint16_t cpg_f64_to_f16(double v) {
    const uint64_t b = cpg_f64_bits(v);
    const uint16_t sign = (uint16_t)((b >> 48) & 0x8000u);
    const int ex = (int)((b >> 52) & 0x7FF);
    const uint64_t man = b & 0xFFFFFFFFFFFFFull;
    if (ex == 0x7FF) return (uint16_t)(sign | (man ? 0x7E00u : 0x7C00u));
    if (ex == 0) return sign;
    const int e = ex - 1023;
    if (e > 15) return (uint16_t)(sign | 0x7C00u);
    const uint64_t m = (1ull << 52) | man;
    const int s = 42 + (e < -14 ? -14 - e : 0);
    if (s >= 64) return sign;
    uint64_t q = m >> s;
    const uint64_t rem = m & ((1ull << s) - 1), half = 1ull << (s - 1);
    if (rem > half || (rem == half && (q & 1))) q++;
    if (e < -14) return (uint16_t)(sign | q);
    return (uint16_t)(sign | ((((uint64_t)(e + 15)) << 10) + (q - 1024)));
}

/* ------------------------------------------------------------------ generator
 * Counter-based, so any element of any tensor can be produced independently on any
 * device: element i of stream s under seed S draws six splitmix64 outputs at counters
 * key + (6i+j+1)*gamma (j = 0..5), splits each into two 24-bit uniforms u, and sums the
 * twelve values (2u+1)/2^25 (an Irwin-Hall(12) variable with mean 6 and variance 1). The
 * sum minus 6 is an exact multiple of 2^-25; it is multiplied by sigma in double and
 * rounded once to float. */
#define CPG_GAMMA 0x9E3779B97F4A7C15ull

CPG_HD uint64_t cpg_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

CPG_HD uint64_t cpg_stream_key(uint64_t seed, uint64_t stream) {
    return cpg_mix64(seed ^ cpg_mix64(stream ^ 0xD1B54A32D192ED03ull));
}

CPG_HD float cpg_gen_normal(uint64_t key, uint64_t i, double sigma) {
    int64_t n = 0;
    for (int j = 0; j < 6; j++) {
        const uint64_t r = cpg_mix64(key + (6 * i + (uint64_t)j + 1) * CPG_GAMMA);
        n += (int64_t)(2 * (r >> 40) + 1) + (int64_t)(2 * ((r >> 8) & 0xFFFFFFu) + 1);
    }
    n -= 12ll << 24;                                  /* sum - 6, in units of 2^-25 */
    const double g = (double)n * 2.98023223876953125e-08;     /* exact: |n| < 2^28 */
    return (float)(g * sigma);
}


/* ------------------------------------------------------------------ block encoders */

/* IEEE division with one rounding on both sides (hipcc's default float division is
   already correctly rounded; the intrinsic makes it independent of compiler flags). */
CPG_HD float cpg_fdiv(float a, float b) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __fdiv_rn(a, b);
#else
    return a / b;
#endif
}

CPG_HD float cpg_rint(float x) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_rintf(x);
#else
    return rintf(x);
#endif
}

/* 32 floats -> one 18-byte Q4_0 block (fp16 d, byte k = q[k] | q[k+16] << 4, q two's
   complement nibbles): d = max|x|/8 in double rounded to fp16, q = clip(rint(x/d), -8, 7)
   with the division in float. The arithmetic of format/q4.py:30-57. */
CPG_HD void cpg_encode_q4_block(const float *v, uint8_t *o) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) { const float a = v[i] < 0.0f ? -v[i] : v[i]; if (a > amax) amax = a; }
    const uint16_t dh = cpg_f64_to_f16(amax > 0.0f ? (double)amax / 8.0 : 0.0);
    const float dq = cpg_f16_to_f32(dh);
    uint8_t q[32];
    for (int i = 0; i < 32; i++) {
        int qi = 0;
        if (dq > 0.0f) {
            float r = cpg_rint(cpg_fdiv(v[i], dq));
            r = r < -8.0f ? -8.0f : (r > 7.0f ? 7.0f : r);
            qi = (int)r;
        }
        q[i] = (uint8_t)(qi & 0xF);
    }
    o[0] = (uint8_t)(dh & 0xFF);
    o[1] = (uint8_t)(dh >> 8);
    for (int k = 0; k < 16; k++) o[2 + k] = (uint8_t)(q[k] | (q[k + 16] << 4));
}

/* 32 floats -> one 34-byte Q8_0 block: d = fl32(max|x|/127) rounded to fp16,
   q = clip(rint(x/d), -127, 127). The arithmetic of format/q8.py:35-58. */
CPG_HD void cpg_encode_q8_block(const float *v, uint8_t *o) {
    float amax = 0.0f;
    for (int i = 0; i < 32; i++) { const float a = v[i] < 0.0f ? -v[i] : v[i]; if (a > amax) amax = a; }
    const float d = amax > 0.0f ? cpg_fdiv(amax, 127.0f) : 0.0f;
    const uint16_t dh = cpg_f64_to_f16((double)d);
    const float dq = cpg_f16_to_f32(dh);
    o[0] = (uint8_t)(dh & 0xFF);
    o[1] = (uint8_t)(dh >> 8);
    for (int i = 0; i < 32; i++) {
        int qi = 0;
        if (dq > 0.0f) {
            float r = cpg_rint(cpg_fdiv(v[i], dq));
            r = r < -127.0f ? -127.0f : (r > 127.0f ? 127.0f : r);
            qi = (int)r;
        }
        o[2 + i] = (uint8_t)(int8_t)qi;
    }
}

/* ------------------------------------------------------------------ expf
 * Results identical to glibc 2.35's expf on x86_64 (checked on all 2^32 inputs). The
 * method is the published one of ARM's optimized-routines, which glibc adopted: write
 * x*32/ln2 = k + r with k an integer (rounded by adding 1.5*2^52), look up 2^(k mod 32 / 32)
 * in a 32-entry table whose entries are binary64 2^(i/32) with i<<47 subtracted from their
 * bits (so adding k<<47 also applies the 2^(k div 32) exponent), and multiply by a cubic
 * in r evaluated in double. glibc's x86_64 build runs it with every multiply-add fused. */
#if defined(__HIPCC__)
__constant__ static const uint64_t cpg_exp2f_tab[32] = {
#else
static const uint64_t cpg_exp2f_tab[32] = {
#endif
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

#if defined(__HIPCC__)
/* Correctly rounded square root (glibc's sqrtf is). On gfx950 __fsqrt_rn lowers to the
   approximate v_sqrt_f32 alone; plain sqrtf, compiled without fast-math, gets the IEEE
   expansion (v_sqrt_f32, then the neighbouring floats checked with FMA residuals). */
__device__ static inline float cpg_sqrt_rn(float x) { return sqrtf(x); }

/* expf with the 2^(i/32) table read through `tab` (e.g. a copy in LDS) */
__device__ static inline float cpg_expf_tab(float x, const uint64_t *tab) {
    const uint32_t abstop = (cpg_f32_bits(x) >> 20) & 0x7ff;
    if (abstop >= 0x42b) {
        if (cpg_f32_bits(x) == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0, shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double xd = (double)x;
    double kd = __fma_rn(inv_ln2_n, xd, shift);
    const uint64_t ki = cpg_f64_bits(kd);
    kd = __dsub_rn(kd, shift);
    const double r = __fma_rn(inv_ln2_n, xd, -kd);
    const double s = cpg_bits_f64(tab[ki % 32] + (ki << 47));
    const double z = __fma_rn(c0, r, c1), r2 = __dmul_rn(r, r);
    double y = __fma_rn(c2, r, 1.0);
    y = __fma_rn(z, r2, y);
    return (float)__dmul_rn(y, s);
}

__device__ static inline float cpg_expf(float x) { return cpg_expf_tab(x, cpg_exp2f_tab); }
#endif

#endif
