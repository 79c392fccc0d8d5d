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
//
// fw_logf: single-precision natural log restated from the same library's
// published table method (the logf glibc >= 2.28 ships): x = 2^k z with z in
// [0x1.66p-1, 0x1.66p0), z split into 16 subintervals each with a table pair
// (1/c, log c), log1p(z/c - 1) from a degree-4 polynomial in double
// (r + A2 r^2 + A1 r^3 + A0 r^4, evaluated as ((A1 r + A2) + A0 r^2) r^2 +
// (k ln2 + log c + r)), one final rounding to float.  The reference's
// log-softmax calls the platform logf (f32::ln -> glibc logf,
// decode.rs:1690).  An exhaustive comparison over every float in [0, +inf]
// against the host's logf pins this (zero mismatches, fused and unfused).
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

// (1/c, log c) of the 16 subintervals, as doubles
#define FW_LOGF_TAB                                                                                      \
    {0x1.661ec79f8f3bep+0, -0x1.57bf7808caadep-2, 0x1.571ed4aaf883dp+0, -0x1.2bef0a7c06ddbp-2,          \
     0x1.49539f0f010bp+0,  -0x1.01eae7f513a67p-2, 0x1.3c995b0b80385p+0, -0x1.b31d8a68224e9p-3,          \
     0x1.30d190c8864a5p+0, -0x1.6574f0ac07758p-3, 0x1.25e227b0b8eap+0,  -0x1.1aa2bc79c81p-3,            \
     0x1.1bb4a4a1a343fp+0, -0x1.a4e76ce8c0e5ep-4, 0x1.12358f08ae5bap+0, -0x1.1973c5a611cccp-4,          \
     0x1.0953f419900a7p+0, -0x1.252f438e10c1ep-5, 0x1p+0,               0x0p+0,                         \
     0x1.e608cfd9a47acp-1, 0x1.aa5aa5df25984p-5,  0x1.ca4b31f026aap-1,  0x1.c5e53aa362eb4p-4,           \
     0x1.b2036576afce6p-1, 0x1.526e57720db08p-3,  0x1.9c2d163a1aa2dp-1, 0x1.bc2860d22477p-3,            \
     0x1.886e6037841edp-1, 0x1.1058bc8a07ee1p-2,  0x1.767dcf5534862p-1, 0x1.4043057b6ee09p-2}

FW_HD static inline float fw_u2f(uint32_t u) {
    float f;
    memcpy(&f, &u, 4);
    return f;
}

FW_HD static inline float fw_logf_tab(float x, const double *tab) {
    const double ln2 = 0x1.62e42fefa39efp-1;
    const double a0 = -0x1.00ea348b88334p-2, a1 = 0x1.5575b0be00b6ap-2, a2 = -0x1.ffffef20a4123p-2;
    uint32_t ix = fw_f2u(x);
    if (ix == 0x3f800000u) return 0.0f;
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
        if (ix * 2 == 0) return -__builtin_inff();                          /* +-0 */
        if (ix == 0x7f800000u) return x;                                    /* +inf */
        if ((ix & 0x80000000u) || ix * 2 >= 0xff000000u) return __builtin_nanf(""); /* x < 0, nan */
        ix = fw_f2u(x * 0x1p23f) - (23u << 23);                             /* subnormal: normalize */
    }
    const uint32_t tmp = ix - 0x3f330000u;
    const int i = (int)((tmp >> 19) % 16);
    const int k = (int32_t)tmp >> 23;
    const uint32_t iz = ix - (tmp & 0xff800000u);
    const double invc = tab[2 * i], logc = tab[2 * i + 1];
    const double z = (double)fw_u2f(iz);
    const double r = FW_FMA(z, invc, -1.0);
    const double y0 = FW_FMA((double)k, ln2, logc);
    const double r2 = r * r;
    double y = FW_FMA(a1, r, a2);
    y = FW_FMA(a0, r2, y);
    y = FW_FMA(y, r2, y0 + r);
    return (float)y;
}

#if !defined(__HIP_DEVICE_COMPILE__)
static const double fw_logf_tab_host[32] = FW_LOGF_TAB;
static inline float fw_logf_host(float x) { return fw_logf_tab(x, fw_logf_tab_host); }
static const uint64_t fw_exp2f_tab_host[32] = FW_EXP2F_TAB;
static inline float fw_expf_host(float x) { return fw_expf_tab(x, fw_exp2f_tab_host); }
#endif
