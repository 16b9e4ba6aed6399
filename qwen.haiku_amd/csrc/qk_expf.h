/*
 * qk_expf.h -- single-precision exp, bit for bit the host libm's expf.
 *
 * The reference's SiLU on x86 is v / (1.0f + expf(-v)) through libm
 * (simd/simd.c:265-269), so the device must reproduce glibc's expf to the
 * last bit. glibc computes expf with the table-driven method of the ARM
 * Optimized Routines (Szabolcs Nagy, 2017-2018): with N = 32,
 *
 *   x * N/ln2 = k + r,  k integer, |r| <= 1/2,
 *   exp(x)    = 2^(k/N) * 2^(r/N),
 *
 * 2^(k/N) = 2^(k div N) * 2^((k mod N)/N) from a 32-entry table, and
 * 2^(r/N) from a degree-3 polynomial, all in double precision with one
 * final rounding to float. glibc ships two builds of that code and x86
 * hosts with FMA (every AVX2 / AVX-VNNI machine) dispatch to the one whose
 * multiply-adds are fused; this header is that form. Checked against the
 * host expf over all 2^32 inputs (tests/test_chain_oracle.py builds it on
 * the CPU); the table entries are pinned there to the correctly rounded
 * 2^(i/32). The two glibc builds differ on exactly two float inputs,
 * 0x4202422f and 0xc27c65d9 (scanned over all 2^32 with the unfused form
 * of this code); libqk's host side evaluates the host expf there and
 * refuses the entry points that need expf when it is not the fused build.
 *
 * Compiled as device code inside the HIP sources, as host code when
 * QK_EXPF_HOST is defined (the check above), and as plain C by the CPU
 * check.
 */
#ifndef QK_EXPF_H
#define QK_EXPF_H

#include <stdint.h>
#include <string.h>

#if defined(__HIP__) && !defined(QK_EXPF_HOST)
#define QK_EXPF_FN __device__ static inline
#define QK_EXPF_DATA __device__ static const
#else
#define QK_EXPF_FN static inline
#define QK_EXPF_DATA static const
#endif

/* Bits of 2^(i/32) rounded to double, less i << 47: adding k << 47 to
 * entry k mod 32 then yields the bits of 2^(k/32) for any integer k in
 * range (the integer part k div 32 lands in the exponent field). */
QK_EXPF_DATA uint64_t qk_exp2_32[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

QK_EXPF_FN uint64_t qk_bits64(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
QK_EXPF_FN double qk_double(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

QK_EXPF_FN float qk_expf(float x) {
    /* Beyond these the result is +inf / +0 (glibc's own cut-offs: the
       largest x whose exp rounds to a finite float, and the point below
       which it rounds to zero). NaN propagates quietened, as x + x. */
    if (!(x <= 0x1.62e42ep6f)) return x != x ? x + x : __builtin_inff();
    if (x < -0x1.9fe368p6f) return 0.0f;
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0; /* N / ln 2 */
    const double round_shift = 0x1.8p52;                  /* 1.5 * 2^52 */
    /* 2^(r/N) ~ 1 + c1 r + c2 r^2 + c3 r^3 (the published minimax fit of
       2^t on |t| <= 1/2, rescaled by powers of N) */
    const double c1 = 0x1.62e42ff0c52d6p-1 / 32.0;
    const double c2 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c3 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double xd = (double)x;
    /* kd = round(x * N/ln2), held in the low mantissa bits of kb */
    double kb = __builtin_fma(inv_ln2_n, xd, round_shift);
    const uint64_t ki = qk_bits64(kb);
    const double kd = kb - round_shift;
    const double r = __builtin_fma(inv_ln2_n, xd, -kd);
    const double scale = qk_double(qk_exp2_32[ki & 31] + (ki << 47));
    const double hi = __builtin_fma(c3, r, c2);
    const double r2 = r * r;
    double p = __builtin_fma(c1, r, 1.0);
    p = __builtin_fma(hi, r2, p);
    return (float)(p * scale);
}

#undef QK_EXPF_FN
#undef QK_EXPF_DATA
#endif
