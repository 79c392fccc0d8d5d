/*
 * refcpu_fast.c — the FAST restatement of the oracle's dense kernels
 * (TEST INFRASTRUCTURE ONLY: the CPU baseline's timed leg).  Register-blocked
 * AVX2 / F16C / FMA kernels that keep every output's arithmetic order of the
 * strict restatement in refcpu.c, so both give the same bits:
 *
 *   rf_matmul       ascending-k f32 mul then add per output, from +0.0f
 *                   (ref_matmul_strict; nn.rs:587-604 strict-parity sgemm).
 *                   6 x 16 register tile, B packed into 16-wide k-panels.
 *   rf_gemm_u8i8    exact i32 sums of u8 x i7 products (the maddubs form the
 *                   reference's i7 GEMM is built for, nn.rs:1537-1771: the
 *                   pair sums stay below 2 * 255 * 63 = 32130, no saturation).
 *   rf_gemm_i8i8    exact i32 sums of i8 x i8 (matmul_bias_i8, encoder.rs:2524-2606).
 *   rf_dot_f16c     dot_f16c's 4 x 8 FMA lanes and its reduction tree
 *                   (nn.rs:1983-2051) with F16C conversions.
 *   rf_dot_i8       exact i32 dot (nn.rs:2635-2686).
 *   rf_dot_i8w_f32  dot_i8w_f32 (nn.rs:3501-3564), dot_f16c's shape.
 *   rf_softmax_row  softmax_row (nn.rs:4900-4950) with the exponentials 8 at a
 *                   time by the published table method of the platform expf
 *                   (ARM optimized-routines / glibc >= 2.27: N = 32 table,
 *                   degree-3 polynomial in double, FMA where glibc's x86-64-v3
 *                   build fuses), the sum still sequential in index order.
 *
 * Integer sums are exact in any order; every float output is formed by the
 * same sequence of IEEE operations as the scalar loop it replaces (vector
 * lanes hold independent outputs, never partial sums of one output, except in
 * the dot products, whose lanes ARE the reference's lanes).  Built with
 * -ffp-contract=off, so a mul followed by an add stays two roundings.
 */
#include <immintrin.h>
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "refcpu_fast.h"
#include "../franken_whisper_amd/csrc/fw_math.h" /* FW_EXP2F_TAB: 2^(i/32) of the table expf */

#define MR 6
#define NR 16
#define MT 96 /* rows per work item of rf_matmul (multiple of MR) */

static void *amalloc(size_t n) {
    void *p = NULL;
    if (posix_memalign(&p, 64, n ? n : 64)) return NULL;
    return p;
}

/* c[6 x 16] = a[6 x k] . bp[k x 16] (bp packed 16 floats per k) */
static inline void k6x16(const float *a, int64_t lda, const float *bp, int k, float *c, int64_t ldc) {
    __m256 c00 = _mm256_setzero_ps(), c01 = c00, c10 = c00, c11 = c00, c20 = c00, c21 = c00;
    __m256 c30 = c00, c31 = c00, c40 = c00, c41 = c00, c50 = c00, c51 = c00;
    const float *a0 = a, *a1 = a + lda, *a2 = a + 2 * lda, *a3 = a + 3 * lda, *a4 = a + 4 * lda,
                *a5 = a + 5 * lda;
    for (int kk = 0; kk < k; kk++) {
        __m256 b0 = _mm256_load_ps(bp + (int64_t)kk * NR), b1 = _mm256_load_ps(bp + (int64_t)kk * NR + 8);
        __m256 av;
        av = _mm256_broadcast_ss(a0 + kk);
        c00 = _mm256_add_ps(c00, _mm256_mul_ps(av, b0));
        c01 = _mm256_add_ps(c01, _mm256_mul_ps(av, b1));
        av = _mm256_broadcast_ss(a1 + kk);
        c10 = _mm256_add_ps(c10, _mm256_mul_ps(av, b0));
        c11 = _mm256_add_ps(c11, _mm256_mul_ps(av, b1));
        av = _mm256_broadcast_ss(a2 + kk);
        c20 = _mm256_add_ps(c20, _mm256_mul_ps(av, b0));
        c21 = _mm256_add_ps(c21, _mm256_mul_ps(av, b1));
        av = _mm256_broadcast_ss(a3 + kk);
        c30 = _mm256_add_ps(c30, _mm256_mul_ps(av, b0));
        c31 = _mm256_add_ps(c31, _mm256_mul_ps(av, b1));
        av = _mm256_broadcast_ss(a4 + kk);
        c40 = _mm256_add_ps(c40, _mm256_mul_ps(av, b0));
        c41 = _mm256_add_ps(c41, _mm256_mul_ps(av, b1));
        av = _mm256_broadcast_ss(a5 + kk);
        c50 = _mm256_add_ps(c50, _mm256_mul_ps(av, b0));
        c51 = _mm256_add_ps(c51, _mm256_mul_ps(av, b1));
    }
    _mm256_storeu_ps(c, c00); _mm256_storeu_ps(c + 8, c01); c += ldc;
    _mm256_storeu_ps(c, c10); _mm256_storeu_ps(c + 8, c11); c += ldc;
    _mm256_storeu_ps(c, c20); _mm256_storeu_ps(c + 8, c21); c += ldc;
    _mm256_storeu_ps(c, c30); _mm256_storeu_ps(c + 8, c31); c += ldc;
    _mm256_storeu_ps(c, c40); _mm256_storeu_ps(c + 8, c41); c += ldc;
    _mm256_storeu_ps(c, c50); _mm256_storeu_ps(c + 8, c51);
}

static inline void k1x16(const float *a, const float *bp, int k, float *c) {
    __m256 c0 = _mm256_setzero_ps(), c1 = c0;
    for (int kk = 0; kk < k; kk++) {
        __m256 av = _mm256_broadcast_ss(a + kk);
        c0 = _mm256_add_ps(c0, _mm256_mul_ps(av, _mm256_load_ps(bp + (int64_t)kk * NR)));
        c1 = _mm256_add_ps(c1, _mm256_mul_ps(av, _mm256_load_ps(bp + (int64_t)kk * NR + 8)));
    }
    _mm256_storeu_ps(c, c0);
    _mm256_storeu_ps(c + 8, c1);
}

void rf_matmul(const float *a, int64_t lda, const float *b, int64_t ldb, float *c, int64_t ldc, int64_t m,
               int k, int n) {
    int64_t np = n / NR, mt = (m + MT - 1) / MT;
    float *bp = (float *)amalloc(sizeof(float) * (size_t)(np * k * NR));
#pragma omp parallel for schedule(static)
    for (int64_t p = 0; p < np; p++)
        for (int kk = 0; kk < k; kk++)
            memcpy(bp + (p * k + kk) * NR, b + (int64_t)kk * ldb + p * NR, sizeof(float) * NR);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t p = 0; p < np; p++)
        for (int64_t t = 0; t < mt; t++) {
            int64_t r = t * MT, r1 = r + MT < m ? r + MT : m;
            const float *pp = bp + p * k * NR;
            for (; r + MR <= r1; r += MR) k6x16(a + r * lda, lda, pp, k, c + r * ldc + p * NR, ldc);
            for (; r < r1; r++) k1x16(a + r * lda, pp, k, c + r * ldc + p * NR);
        }
    free(bp);
    if (np * NR < n) {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < m; r++)
            for (int j = (int)(np * NR); j < n; j++) {
                float acc = 0.0f;
                for (int kk = 0; kk < k; kk++) acc += a[r * lda + kk] * b[(int64_t)kk * ldb + j];
                c[r * ldc + j] = acc;
            }
    }
}

static inline int32_t hsum_i32(__m256i v) {
    __m128i s = _mm_add_epi32(_mm256_castsi256_si128(v), _mm256_extracti128_si256(v, 1));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0x4e));
    s = _mm_add_epi32(s, _mm_shuffle_epi32(s, 0xb1));
    return _mm_cvtsi128_si32(s);
}

#define GR 4  /* activation rows per register tile */
#define GN 2  /* outputs per register tile */
#define GT 32 /* outputs per work item (weights of a work item stay in L2) */
#define GM 64 /* rows per work item */

/* raw[r][o] = sum_i x[r][i] * w[o][i] over u8 activations and i8 weights of
 * magnitude <= 63 (maddubs pair sums cannot saturate). */
/* The epilogue of one output: acc = raw - 128 * wc[o] (when wc), acc_out,
 * y = (f32)acc * xs[r] * ws[o], then + bias[o], or + 0.0f when add_zero. */
static inline void epi_store(const rf_epi *e, int64_t r, int o, int n, int32_t raw) {
    int32_t acc = e->wc ? raw - 128 * e->wc[o] : raw;
    int64_t at = r * n + o;
    if (e->acc_out) e->acc_out[at] = acc;
    float v = (float)acc * e->xs[r] * e->ws[o];
    if (e->bias) v += e->bias[o];
    else if (e->add_zero) v += 0.0f;
    e->y[at] = v;
}

void rf_gemm_u8i8(const uint8_t *x, const int8_t *w, int64_t m, int k, int n, const rf_epi *e) {
    int k32 = k - k % 32;
    int64_t nt = (n + GT - 1) / GT, mt = (m + GM - 1) / GM;
    const __m256i ones = _mm256_set1_epi16(1);
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t ot = 0; ot < nt; ot++)
        for (int64_t rt = 0; rt < mt; rt++) {
            int64_t r0 = rt * GM, r1 = r0 + GM < m ? r0 + GM : m;
            int o0 = (int)(ot * GT), o1 = o0 + GT < n ? o0 + GT : n;
            for (int64_t r = r0; r < r1; r += GR) {
                int nr = r + GR <= r1 ? GR : (int)(r1 - r);
                for (int o = o0; o < o1; o += GN) {
                    int no = o + GN <= o1 ? GN : o1 - o;
                    __m256i acc[GR][GN];
                    for (int i = 0; i < GR; i++)
                        for (int j = 0; j < GN; j++) acc[i][j] = _mm256_setzero_si256();
                    const uint8_t *xr[GR];
                    const int8_t *wr[GN];
                    for (int i = 0; i < GR; i++) xr[i] = x + (r + (i < nr ? i : 0)) * k;
                    for (int j = 0; j < GN; j++) wr[j] = w + (int64_t)(o + (j < no ? j : 0)) * k;
                    for (int kk = 0; kk < k32; kk += 32) {
                        __m256i wv0 = _mm256_loadu_si256((const __m256i *)(wr[0] + kk));
                        __m256i wv1 = _mm256_loadu_si256((const __m256i *)(wr[1] + kk));
                        for (int i = 0; i < GR; i++) {
                            __m256i xv = _mm256_loadu_si256((const __m256i *)(xr[i] + kk));
                            acc[i][0] = _mm256_add_epi32(acc[i][0], _mm256_madd_epi16(_mm256_maddubs_epi16(xv, wv0), ones));
                            acc[i][1] = _mm256_add_epi32(acc[i][1], _mm256_madd_epi16(_mm256_maddubs_epi16(xv, wv1), ones));
                        }
                    }
                    for (int i = 0; i < nr; i++)
                        for (int j = 0; j < no; j++) {
                            int32_t s = hsum_i32(acc[i][j]);
                            for (int kk = k32; kk < k; kk++) s += (int32_t)xr[i][kk] * (int32_t)wr[j][kk];
                            epi_store(e, r + i, o + j, n, s);
                        }
                }
            }
        }
}

/* raw[r][o] = sum_i x[r][i] * w[o][i], i8 x i8 (sign-extended pairs). */
void rf_gemm_i8i8(const int8_t *x, const int8_t *w, int64_t m, int k, int n, const rf_epi *e) {
    int k16 = k - k % 16;
    int64_t nt = (n + GT - 1) / GT, mt = (m + GM - 1) / GM;
#pragma omp parallel for collapse(2) schedule(static)
    for (int64_t ot = 0; ot < nt; ot++)
        for (int64_t rt = 0; rt < mt; rt++) {
            int64_t r0 = rt * GM, r1 = r0 + GM < m ? r0 + GM : m;
            int o0 = (int)(ot * GT), o1 = o0 + GT < n ? o0 + GT : n;
            for (int64_t r = r0; r < r1; r += GR) {
                int nr = r + GR <= r1 ? GR : (int)(r1 - r);
                for (int o = o0; o < o1; o += GN) {
                    int no = o + GN <= o1 ? GN : o1 - o;
                    __m256i acc[GR][GN];
                    for (int i = 0; i < GR; i++)
                        for (int j = 0; j < GN; j++) acc[i][j] = _mm256_setzero_si256();
                    const int8_t *xr[GR];
                    const int8_t *wr[GN];
                    for (int i = 0; i < GR; i++) xr[i] = x + (r + (i < nr ? i : 0)) * k;
                    for (int j = 0; j < GN; j++) wr[j] = w + (int64_t)(o + (j < no ? j : 0)) * k;
                    for (int kk = 0; kk < k16; kk += 16) {
                        __m256i wv0 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(wr[0] + kk)));
                        __m256i wv1 = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(wr[1] + kk)));
                        for (int i = 0; i < GR; i++) {
                            __m256i xv = _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(xr[i] + kk)));
                            acc[i][0] = _mm256_add_epi32(acc[i][0], _mm256_madd_epi16(xv, wv0));
                            acc[i][1] = _mm256_add_epi32(acc[i][1], _mm256_madd_epi16(xv, wv1));
                        }
                    }
                    for (int i = 0; i < nr; i++)
                        for (int j = 0; j < no; j++) {
                            int32_t s = hsum_i32(acc[i][j]);
                            for (int kk = k16; kk < k; kk++) s += (int32_t)xr[i][kk] * (int32_t)wr[j][kk];
                            epi_store(e, r + i, o + j, n, s);
                        }
                }
            }
        }
}

/* ((t0+t1)+(t2+t3))+((t4+t5)+(t6+t7)) of the 8 lanes of v */
static inline float tree8(__m256 v) {
    float t[8];
    _mm256_storeu_ps(t, v);
    return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

static inline __m256 ld_f16(const uint16_t *p) { return _mm256_cvtph_ps(_mm_loadu_si128((const __m128i *)p)); }
static inline float f16s(uint16_t h) { return _cvtsh_ss(h); }

float rf_dot_f16c(const uint16_t *w, const float *x, int n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        a0 = _mm256_fmadd_ps(ld_f16(w + i), _mm256_loadu_ps(x + i), a0);
        a1 = _mm256_fmadd_ps(ld_f16(w + i + 8), _mm256_loadu_ps(x + i + 8), a1);
        a2 = _mm256_fmadd_ps(ld_f16(w + i + 16), _mm256_loadu_ps(x + i + 16), a2);
        a3 = _mm256_fmadd_ps(ld_f16(w + i + 24), _mm256_loadu_ps(x + i + 24), a3);
    }
    float s = tree8(_mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)));
    for (; i + 8 <= n; i += 8) s += tree8(_mm256_mul_ps(ld_f16(w + i), _mm256_loadu_ps(x + i)));
    for (; i < n; i++) s += f16s(w[i]) * x[i];
    return s;
}

static inline __m256 ld_i8f(const int8_t *p) {
    return _mm256_cvtepi32_ps(_mm256_cvtepi8_epi32(_mm_loadl_epi64((const __m128i *)p)));
}

float rf_dot_i8w_f32(const int8_t *w, const float *x, int n) {
    __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
    int i = 0;
    for (; i + 32 <= n; i += 32) {
        a0 = _mm256_fmadd_ps(ld_i8f(w + i), _mm256_loadu_ps(x + i), a0);
        a1 = _mm256_fmadd_ps(ld_i8f(w + i + 8), _mm256_loadu_ps(x + i + 8), a1);
        a2 = _mm256_fmadd_ps(ld_i8f(w + i + 16), _mm256_loadu_ps(x + i + 16), a2);
        a3 = _mm256_fmadd_ps(ld_i8f(w + i + 24), _mm256_loadu_ps(x + i + 24), a3);
    }
    float s = tree8(_mm256_add_ps(_mm256_add_ps(a0, a1), _mm256_add_ps(a2, a3)));
    for (; i + 8 <= n; i += 8) s += tree8(_mm256_mul_ps(ld_i8f(w + i), _mm256_loadu_ps(x + i)));
    for (; i < n; i++) s += (float)w[i] * x[i];
    return s;
}

int32_t rf_dot_i8(const int8_t *w, const int8_t *x, int n) {
    __m256i acc = _mm256_setzero_si256();
    int i = 0;
    for (; i + 16 <= n; i += 16)
        acc = _mm256_add_epi32(acc, _mm256_madd_epi16(_mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(w + i))),
                                                      _mm256_cvtepi8_epi16(_mm_loadu_si128((const __m128i *)(x + i)))));
    int32_t s = hsum_i32(acc);
    for (; i < n; i++) s += (int32_t)w[i] * (int32_t)x[i];
    return s;
}

static const uint64_t g_exp2_tab[32] __attribute__((aligned(64))) = FW_EXP2F_TAB;

/* expf of 4 floats: x*32/ln2 = k + r, 2^(k/32) from the table, 2^(r/32) from
 * the degree-3 polynomial, one rounding to float.  Lanes past the underflow
 * threshold (and -inf) give +0, past the overflow threshold +inf; NaN stays
 * NaN. */
static inline __m128 expf4(__m128 xf) {
    const __m256d inv = _mm256_set1_pd(0x1.71547652b82fep+0 * 32.0), shift = _mm256_set1_pd(0x1.8p+52);
    const __m256d c0 = _mm256_set1_pd(0x1.c6af84b912394p-5 / (32.0 * 32.0 * 32.0));
    const __m256d c1 = _mm256_set1_pd(0x1.ebfce50fac4f3p-3 / (32.0 * 32.0));
    const __m256d c2 = _mm256_set1_pd(0x1.62e42ff0c52d6p-1 / 32.0);
    __m256d xd = _mm256_cvtps_pd(xf);
    __m256d kd = _mm256_fmadd_pd(inv, xd, shift);
    __m256i ki = _mm256_castpd_si256(kd);
    kd = _mm256_sub_pd(kd, shift);
    __m256d r = _mm256_fmsub_pd(inv, xd, kd);
    __m256i idx = _mm256_and_si256(ki, _mm256_set1_epi64x(31));
    __m256i t = _mm256_add_epi64(_mm256_i64gather_epi64((const long long *)g_exp2_tab, idx, 8),
                                 _mm256_slli_epi64(ki, 47));
    __m256d sc = _mm256_castsi256_pd(t);
    __m256d zp = _mm256_fmadd_pd(c0, r, c1);
    __m256d r2 = _mm256_mul_pd(r, r);
    __m256d y = _mm256_fmadd_pd(c2, r, _mm256_set1_pd(1.0));
    y = _mm256_fmadd_pd(zp, r2, y);
    y = _mm256_mul_pd(y, sc);
    __m128 out = _mm256_cvtpd_ps(y);
    __m128 lo = _mm_cmp_ps(xf, _mm_set1_ps(-0x1.9fe368p6f), _CMP_LT_OQ);
    __m128 hi = _mm_cmp_ps(xf, _mm_set1_ps(0x1.62e42ep6f), _CMP_GT_OQ);
    out = _mm_andnot_ps(lo, out);
    out = _mm_blendv_ps(out, _mm_set1_ps(INFINITY), hi);
    return out;
}

static inline __m256 expf8(__m256 x) {
    return _mm256_set_m128(expf4(_mm256_extractf128_ps(x, 1)), expf4(_mm256_castps256_ps128(x)));
}

void rf_expf_n(const float *x, float *y, int64_t n) {
    int64_t i = 0;
    for (; i + 8 <= n; i += 8) _mm256_storeu_ps(y + i, expf8(_mm256_loadu_ps(x + i)));
    if (i < n) {
        float tx[8] = {0}, ty[8];
        memcpy(tx, x + i, sizeof(float) * (size_t)(n - i));
        _mm256_storeu_ps(ty, expf8(_mm256_loadu_ps(tx)));
        memcpy(y + i, ty, sizeof(float) * (size_t)(n - i));
    }
}

/* softmax_row: max ignoring NaN, return when the max is not finite, e =
 * expf(x - max) with non-finite e -> 0, sequential f32 sum, then *= 1/sum
 * when the sum is positive. */
void rf_softmax_row(float *row, int cols) {
    __m256 vm = _mm256_set1_ps(-INFINITY);
    int j = 0;
    for (; j + 8 <= cols; j += 8) vm = _mm256_max_ps(_mm256_loadu_ps(row + j), vm); /* NaN lanes keep vm */
    float t[8];
    _mm256_storeu_ps(t, vm);
    float mx = -INFINITY;
    for (int l = 0; l < 8; l++) mx = fmaxf(mx, t[l]);
    for (; j < cols; j++) mx = fmaxf(mx, row[j]);
    if (!isfinite(mx)) return;
    const __m256 vmx = _mm256_set1_ps(mx), zero = _mm256_setzero_ps();
    float sum = 0.0f;
    j = 0;
    for (; j + 8 <= cols; j += 8) {
        __m256 e = expf8(_mm256_sub_ps(_mm256_loadu_ps(row + j), vmx));
        __m256 fin = _mm256_cmp_ps(_mm256_sub_ps(e, e), zero, _CMP_EQ_OQ);
        e = _mm256_and_ps(e, fin);
        _mm256_storeu_ps(row + j, e);
        _mm256_storeu_ps(t, e);
        for (int l = 0; l < 8; l++) sum += t[l];
    }
    for (; j < cols; j++) {
        float e = expf(row[j] - mx);
        if (!isfinite(e)) e = 0.0f;
        row[j] = e;
        sum += e;
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        const __m256 vi = _mm256_set1_ps(inv);
        j = 0;
        for (; j + 8 <= cols; j += 8) _mm256_storeu_ps(row + j, _mm256_mul_ps(_mm256_loadu_ps(row + j), vi));
        for (; j < cols; j++) row[j] *= inv;
    }
}

/* sc[j] = sequential sum over i of qh[i] * kt[i*ld + j] from +0.0f, keys 8 per
 * vector. */
void rf_scores_t(const float *qh, const float *kt, int ld, int dh, int tk, float *sc) {
    int j = 0;
    for (; j + 8 <= tk; j += 8) {
        __m256 acc = _mm256_setzero_ps();
        for (int i = 0; i < dh; i++)
            acc = _mm256_add_ps(acc, _mm256_mul_ps(_mm256_broadcast_ss(qh + i), _mm256_loadu_ps(kt + (int64_t)i * ld + j)));
        _mm256_storeu_ps(sc + j, acc);
    }
    for (; j < tk; j++) {
        float acc = 0.0f;
        for (int i = 0; i < dh; i++) acc += qh[i] * kt[(int64_t)i * ld + j];
        sc[j] = acc;
    }
}

/* out[i] = sequential sum over j of p[j] * f16(v[j*ldv + i]) from +0.0f. */
void rf_pv_f16(const float *p, const uint16_t *v, int64_t ldv, int tk, int dh, float *out) {
    int i = 0;
    for (; i + 32 <= dh; i += 32) {
        __m256 a0 = _mm256_setzero_ps(), a1 = a0, a2 = a0, a3 = a0;
        for (int j = 0; j < tk; j++) {
            const uint16_t *vr = v + (int64_t)j * ldv + i;
            __m256 pj = _mm256_broadcast_ss(p + j);
            a0 = _mm256_add_ps(a0, _mm256_mul_ps(pj, ld_f16(vr)));
            a1 = _mm256_add_ps(a1, _mm256_mul_ps(pj, ld_f16(vr + 8)));
            a2 = _mm256_add_ps(a2, _mm256_mul_ps(pj, ld_f16(vr + 16)));
            a3 = _mm256_add_ps(a3, _mm256_mul_ps(pj, ld_f16(vr + 24)));
        }
        _mm256_storeu_ps(out + i, a0);
        _mm256_storeu_ps(out + i + 8, a1);
        _mm256_storeu_ps(out + i + 16, a2);
        _mm256_storeu_ps(out + i + 24, a3);
    }
    for (; i + 8 <= dh; i += 8) {
        __m256 a0 = _mm256_setzero_ps();
        for (int j = 0; j < tk; j++)
            a0 = _mm256_add_ps(a0, _mm256_mul_ps(_mm256_broadcast_ss(p + j), ld_f16(v + (int64_t)j * ldv + i)));
        _mm256_storeu_ps(out + i, a0);
    }
    for (; i < dh; i++) {
        float acc = 0.0f;
        for (int j = 0; j < tk; j++) acc += p[j] * f16s(v[(int64_t)j * ldv + i]);
        out[i] = acc;
    }
}

/* out[i] = sequential sum over j of p[j] * v[j*ldv + i] from +0.0f (f32 rows:
 * the reference's default cache, attention_decode_step's j-ascending axpy,
 * nn.rs:6388-6398). */
void rf_pv_f32(const float *p, const float *v, int64_t ldv, int tk, int dh, float *out) {
    int i = 0;
    for (; i + 8 <= dh; i += 8) {
        __m256 a0 = _mm256_setzero_ps();
        for (int j = 0; j < tk; j++)
            a0 = _mm256_add_ps(a0, _mm256_mul_ps(_mm256_broadcast_ss(p + j), _mm256_loadu_ps(v + (int64_t)j * ldv + i)));
        _mm256_storeu_ps(out + i, a0);
    }
    for (; i < dh; i++) {
        float acc = 0.0f;
        for (int j = 0; j < tk; j++) acc += p[j] * v[(int64_t)j * ldv + i];
        out[i] = acc;
    }
}

/* quantize_row_i7_u8 (nn.rs:3075-3111): the 8-wide body clamp(trunc(v +
 * copysign(0.5, v)), -127, 127) + 128 with v = x * inv, the n % 8 tail with
 * round-half-away; optionally each x first through the GELU table
 * (x <= -10 -> 0, x >= 10 -> x, else table[f16(x)]), with NaN lanes taking the
 * scalar conversion.  Returns the activation scale max(max|g|, 1e-9) / 127. */
float rf_quant_row_i7(const float *x, int n, const float *gelu_tab, uint16_t (*f2h)(float), float *g,
                      uint8_t *out) {
    const float *src = x;
    if (gelu_tab) {
        int i = 0;
        for (; i + 8 <= n; i += 8) {
            __m256 v = _mm256_loadu_ps(x + i);
            __m128i h = _mm256_cvtps_ph(v, _MM_FROUND_TO_NEAREST_INT | _MM_FROUND_NO_EXC);
            uint16_t hh[8];
            _mm_storeu_si128((__m128i *)hh, h);
            float t[8], xv[8];
            _mm256_storeu_ps(xv, v);
            for (int l = 0; l < 8; l++) {
                float f = xv[l];
                t[l] = f <= -10.0f ? 0.0f : (f >= 10.0f ? f : gelu_tab[f != f ? f2h(f) : hh[l]]);
            }
            _mm256_storeu_ps(g + i, _mm256_loadu_ps(t));
        }
        for (; i < n; i++) {
            float f = x[i];
            g[i] = f <= -10.0f ? 0.0f : (f >= 10.0f ? f : gelu_tab[f2h(f)]);
        }
        src = g;
    }
    const __m256 absmask = _mm256_castsi256_ps(_mm256_set1_epi32(0x7fffffff));
    __m256 am = _mm256_setzero_ps();
    int i = 0;
    for (; i + 8 <= n; i += 8) am = _mm256_max_ps(_mm256_and_ps(_mm256_loadu_ps(src + i), absmask), am);
    float t[8];
    _mm256_storeu_ps(t, am);
    float amax = 0.0f;
    for (int l = 0; l < 8; l++) amax = fmaxf(amax, t[l]);
    for (; i < n; i++) amax = fmaxf(amax, fabsf(src[i]));
    amax = fmaxf(amax, 1e-9f);
    float s = amax / 127.0f, inv = 1.0f / s;
    const __m256 vinv = _mm256_set1_ps(inv), half = _mm256_set1_ps(0.5f), sgn = _mm256_set1_ps(-0.0f);
    const __m256 lo = _mm256_set1_ps(-127.0f), hi = _mm256_set1_ps(127.0f);
    int n8 = n - n % 8;
    for (i = 0; i < n8; i += 8) {
        __m256 v = _mm256_mul_ps(_mm256_loadu_ps(src + i), vinv);
        __m256 hv = _mm256_or_ps(half, _mm256_and_ps(v, sgn));
        __m256 r = _mm256_round_ps(_mm256_add_ps(v, hv), _MM_FROUND_TO_ZERO | _MM_FROUND_NO_EXC);
        r = _mm256_min_ps(_mm256_max_ps(r, lo), hi);
        __m256i q = _mm256_add_epi32(_mm256_cvttps_epi32(r), _mm256_set1_epi32(128));
        int32_t qq[8];
        _mm256_storeu_si256((__m256i *)qq, q);
        for (int l = 0; l < 8; l++) out[i + l] = (uint8_t)qq[l];
    }
    for (; i < n; i++) {
        float v = src[i] * inv;
        v = roundf(v);
        v = v < -127.f ? -127.f : (v > 127.f ? 127.f : v);
        out[i] = (uint8_t)((int32_t)v + 128);
    }
    return s;
}
