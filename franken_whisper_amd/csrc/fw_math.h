// fw_math.h — scalar numerics shared by host and device code.
//
// fw_expf: single-precision exp restated from the published table method of
// ARM's optimized-routines (the exp2f-table expf that glibc >= 2.27 ships):
// x*N/ln2 = k + r with N = 32, 2^(k/N) from a 32-entry table of 2^(i/32),
// 2^(r/N) from a degree-3 polynomial evaluated in double, one final rounding
// to float.  The reference's softmax calls the platform expf (f32::exp ->
// glibc expf, nn.rs:4930).  Multiply-adds are fused exactly where glibc's FMA
// build (the variant an x86-64-v3 host dispatches to) fuses them: both
// range-reduction steps and the three polynomial steps.  An exhaustive
// comparison over every float in [-110, 90] against the host's expf pins this
// (zero mismatches; the unfused range reduction differs on 2 inputs).
#pragma once
#include <stdint.h>
#include <string.h>

#if defined(__HIPCC__) || defined(__HIP__)
#define FW_HD __host__ __device__
#else
#define FW_HD
#endif

#if defined(__HIP_DEVICE_COMPILE__)
#define FW_FMA(a, b, c) __builtin_fma((a), (b), (c))
#else
#include <math.h>
#define FW_FMA(a, b, c) fma((a), (b), (c))
#endif

// 2^(i/32) as doubles, each minus (i << 47) so that adding (k << 47) scales by 2^(k/32).
#define FW_EXP2F_TAB                                                                          \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull, \
     0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, \
     0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull, \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull, \
     0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull, \
     0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull, \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull, \
     0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

FW_HD static inline uint32_t fw_f2u(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    return u;
}
FW_HD static inline double fw_u2d(uint64_t u) {
    double d;
    memcpy(&d, &u, 8);
    return d;
}
FW_HD static inline uint64_t fw_d2u(double d) {
    uint64_t u;
    memcpy(&u, &d, 8);
    return u;
}

FW_HD static inline float fw_expf_tab(float x, const uint64_t *tab) {
    const double inv_ln2_n = 0x1.71547652b82fep+0 * 32.0;
    const double shift = 0x1.8p+52;
    const double c0 = 0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0);
    const double c1 = 0x1.ebfce50fac4f3p-3 / (32.0 * 32.0);
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
    uint32_t ux = fw_f2u(x);
    uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) { /* |x| >= 88 or not finite (top12(88.0f) = 0x42b) */
        if (ux == 0xff800000u) return 0.0f;    /* -inf */
        if (abstop >= 0x7f8) return x + x;      /* inf or nan */
        if (x > 0x1.62e42ep6f) return (float)(0x1p97 * 0x1p97); /* overflow -> inf */
        if (x < -0x1.9fe368p6f) return 0.0f;    /* underflow */
    }
    double xd = (double)x;
    double kd = FW_FMA(inv_ln2_n, xd, shift);
    uint64_t ki = fw_d2u(kd);
    kd -= shift;
    double r = FW_FMA(inv_ln2_n, xd, -kd);
    uint64_t t = tab[ki % 32] + (ki << 47);
    double s = fw_u2d(t);
    double zp = FW_FMA(c0, r, c1);
    double r2 = r * r;
    double y = FW_FMA(c2, r, 1.0);
    y = FW_FMA(zp, r2, y);
    y = y * s;
    return (float)y;
}

#if !defined(__HIP_DEVICE_COMPILE__)
static const uint64_t fw_exp2f_tab_host[32] = FW_EXP2F_TAB;
static inline float fw_expf_host(float x) { return fw_expf_tab(x, fw_exp2f_tab_host); }
#endif
