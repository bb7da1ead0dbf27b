/*
 * expf_glibc.h -- expf with the results of glibc's expf (2.28 and later,
 * x86-64 with FMA), bit for bit on every float input.
 *
 * The reference scores its router logits with glibc's expf
 * (src/model.c:2724, sigmoid; src/model.c:501, SiLU), and glibc's expf is
 * not correctly rounded, so a correctly rounded exp differs from it on some
 * inputs. This restates the published algorithm glibc uses (Szabolcs
 * Nagy's expf from ARM's optimized-routines): in double precision,
 * x * 32/ln2 = k + r with k an integer (by adding and subtracting
 * 1.5 * 2^52) and |r| <= 1/2; 2^(k/32) from a table of the 32 doubles
 * 2^(i/32) with i << 47 subtracted, its exponent field then advanced by
 * k << 47; 2^(r/32) by the cubic 1 + c2 r + c1 r^2 + c0 r^3 whose
 * coefficients are that method's minimax fit of 2^x scaled by 1/32;
 * the product rounded once to float. The range reduction runs as two fused
 * multiply-adds, as the FMA build of glibc contracts it. Outside
 * |x| < 88 the special cases: +inf, 0, NaN, and x + x for infinities.
 *
 * The table entries are the correctly rounded doubles of 2^(i/32),
 * computed independently to 60 digits. An exhaustive comparison against
 * the host's glibc expf over all 2^32 inputs is part of the CPU tests.
 *
 * WARP_EXPF_QUAL sets the function's qualifiers (the kernels define it as
 * a device function; plain C gets static inline).
 */
#ifndef WARP_EXPF_GLIBC_H
#define WARP_EXPF_GLIBC_H

#include <math.h>
#include <stdint.h>
#include <string.h>

#ifndef WARP_EXPF_QUAL
#define WARP_EXPF_QUAL static inline
#endif

/* 2^(i/32) as double bits, minus i << 47 */
#define WARP_EXP2_TAB {                                                          \
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,\
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,\
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,\
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,\
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,\
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,\
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,\
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,\
}

/* tab: the 32 entries of WARP_EXP2_TAB (a copy anywhere, e.g. in LDS) */
WARP_EXPF_QUAL float warp_expf_t(float x, const uint64_t *tab)
{
    const double inv_ln2_32 = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t ux;
    memcpy(&ux, &x, 4);
    const uint32_t top = (ux >> 20) & 0x7ff;
    if (top >= 0x42bu) {                         /* |x| >= 88, inf or nan   */
        if (ux == 0xff800000u) return 0.0f;      /* -inf                    */
        if (top >= 0x7f8u) return x + x;         /* +inf, nan               */
        if (x > 0x1.62e42ep6f) return INFINITY;  /* above log(2^128)        */
        if (x < -0x1.9fe368p6f) return 0.0f;     /* below log(2^-150)       */
    }
    const double xd = (double)x;
    double kd = fma(inv_ln2_32, xd, shift);
    uint64_t ki;
    memcpy(&ki, &kd, 8);
    kd -= shift;
    const double r = fma(inv_ln2_32, xd, -kd);
    const uint64_t t = tab[ki % 32] + (ki << 47);
    double s;
    memcpy(&s, &t, 8);
    const double z = fma(c0, r, c1);
    const double r2 = r * r;
    double y = fma(c2, r, 1.0);
    y = fma(z, r2, y);
    return (float)(y * s);
}

WARP_EXPF_QUAL float warp_expf(float x)
{
    static const uint64_t tab[32] = WARP_EXP2_TAB;
    return warp_expf_t(x, tab);
}

#endif /* WARP_EXPF_GLIBC_H */
