/*
 * refcpu.c — CPU restatement of franken_whisper's native engine hot path
 * (TEST INFRASTRUCTURE ONLY: parity oracle + CPU baseline; see refcpu.h for the
 * restated flag set).  Every function cites the reference file:line it follows
 * (paths relative to the reference tree, src/native_engine/).
 *
 * Parallelism: OpenMP over independent output rows/heads only, so every value is
 * computed in exactly the reference's per-element order whatever the thread
 * count (the reference's own rayon splits are disjoint row bands too).
 */
#include "refcpu.h"
#include "refcpu_fast.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define LN_EPS 1e-5f
#define CONV_K 3
#define CONV_PAD 1
#define SILENCE_FLOOR (-1.5f) /* mel.rs:235 */

int ref_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
void ref_set_num_threads(int n) {
#ifdef _OPENMP
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* FAST restatement switch: the dense loops below hand their work to the
 * register-blocked kernels of refcpu_fast.c, which form every output by the
 * same sequence of operations (the same bits); off, the scalar loops run. */
static int g_fast = 0;
void ref_set_fast(int on) { g_fast = on != 0; }
int ref_get_fast(void) { return g_fast; }

/* ------------------------------------------------------------------------ */
/* IEEE binary16 <-> binary32, round-to-nearest-even: the `half` 2.7.1 crate's */
/* Float16::{to_f32,from_f32} on an F16C target (vcvtph2ps / vcvtps2ph).       */
/* ------------------------------------------------------------------------ */
static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float ref_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    if (ex == 0) {
        if (man == 0) return u2f(sign);
        int e = -1;
        do { e++; man <<= 1; } while (!(man & 0x400u));
        return u2f(sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13));
    }
    if (ex == 31) return u2f(sign | 0x7f800000u | (man << 13) | (man ? 0x400000u : 0u)); /* F16C quiets NaN */
    return u2f(sign | ((ex + 112u) << 23) | (man << 13));
}

uint16_t ref_f32_to_f16(float f) {
    uint32_t x = f2u(f);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu)); /* quiet NaN */
    if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    if (a >= 0x38800000u) { /* normal f16 range (may overflow to inf) */
        uint32_t r = a - (112u << 23);
        r += 0xfffu + ((r >> 13) & 1u);
        r >>= 13;
        if (r >= 0x7c00u) return (uint16_t)(sign | 0x7c00u);
        return (uint16_t)(sign | r);
    }
    uint32_t e = a >> 23;
    if (e < 102) return sign; /* |f| < 2^-25 */
    uint32_t m = (a & 0x7fffffu) | 0x800000u;
    uint32_t s = 126u - e; /* 14..24 */
    uint32_t q = m >> s, rem = m & ((1u << s) - 1u), half = 1u << (s - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

void ref_f16_to_f32_n(const uint16_t *h, float *f, int64_t n) {
    for (int64_t i = 0; i < n; i++) f[i] = ref_f16_to_f32(h[i]);
}
void ref_f32_to_f16_n(const float *f, uint16_t *h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = ref_f32_to_f16(f[i]);
}

/* f32::round (half away from zero) and Rust's clamp-then-cast. */
static inline float round_half_away(float v) { return roundf(v); }
static inline float clampf(float v, float lo, float hi) { return v < lo ? lo : (v > hi ? hi : v); }
/* AVX2 add-trunc rounding trunc(v + copysign(0.5, v)) (nn.rs:3036-3038):
 * the f32 add rounds, so it differs from round() only at |v| = 0x3EFFFFFF. */
static inline float round_add_trunc(float v) {
    float h = copysignf(0.5f, v);
    return truncf(v + h);
}

/* ------------------------------------------------------------------------ */
/* Quantizers                                                               */
/* ------------------------------------------------------------------------ */

/* quantize_act_i8_into, nn.rs:3020-3049 (AVX2 body, add-trunc) + scalar
 * tail nn.rs:3050-3053 (exact round) for the n % 8 remainder. */
void ref_quantize_act_i8(const float *x, int n, float xinv, int8_t *out) {
    int n8 = n - n % 8, i = 0;
    for (; i < n8; i++) out[i] = (int8_t)clampf(round_add_trunc(x[i] * xinv), -127.f, 127.f);
    for (; i < n; i++) out[i] = (int8_t)clampf(round_half_away(x[i] * xinv), -127.f, 127.f);
}

/* quantize_row_i7_u8_into, nn.rs:3075-3111 (+128 offset into the maddubs u8). */
void ref_quantize_row_i7_u8(const float *x, int n, float inv, uint8_t *out) {
    int n8 = n - n % 8, i = 0;
    for (; i < n8; i++)
        out[i] = (uint8_t)((int32_t)clampf(round_add_trunc(x[i] * inv), -127.f, 127.f) + 128);
    for (; i < n; i++)
        out[i] = (uint8_t)((int32_t)clampf(round_half_away(x[i] * inv), -127.f, 127.f) + 128);
}

/* quant_row_i8, encoder.rs:2468-2508: exact round-half-away in both the AVX2
 * body (trunc + |frac|>=0.5 test) and the tail. */
void ref_quant_row_i8_exact(const float *x, int n, float inv, int8_t *out) {
    for (int i = 0; i < n; i++) out[i] = (int8_t)clampf(round_half_away(x[i] * inv), -127.f, 127.f);
}

/* max(fold(0, max|x|), 1e-9) / 127  (gemv_i8 nn.rs:3178-3180, quantize_act_i7
 * nn.rs:1450-1451, matmul_bias_i8 encoder.rs:2544-2545). */
float ref_act_scale(const float *x, int n) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) amax = fmaxf(amax, fabsf(x[i]));
    amax = fmaxf(amax, 1e-9f);
    return amax / 127.0f;
}

/* quantize_f16_row_to_i8_into, nn.rs:2490-2555: amax over the row, scale =
 * max(amax,1e-9)/127, add-trunc rounding in the 8-wide body, round in the tail. */
float ref_quantize_f16_row_to_i8(const uint16_t *w, int n, int8_t *out) {
    float amax = 0.0f;
    for (int i = 0; i < n; i++) amax = fmaxf(amax, fabsf(ref_f16_to_f32(w[i])));
    float scale = fmaxf(amax, 1e-9f) / 127.0f;
    float inv = 1.0f / scale;
    int n8 = n - n % 8, j = 0;
    for (; j < n8; j++)
        out[j] = (int8_t)clampf(round_add_trunc(ref_f16_to_f32(w[j]) * inv), -127.f, 127.f);
    for (; j < n; j++)
        out[j] = (int8_t)clampf(round_half_away(ref_f16_to_f32(w[j]) * inv), -127.f, 127.f);
    return scale;
}

/* quantize_f16_to_i8, nn.rs:2576-2633 (FW_DEC_EF off: the default). */
void ref_quantize_f16_to_i8(const uint16_t *w, int64_t out, int inp, int8_t *q, float *s) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out; o++) s[o] = ref_quantize_f16_row_to_i8(w + o * inp, inp, q + o * inp);
}

/* quantize_f16_row_blocked_to_int_into, nn.rs:3619-3693 (max_level 127): per
 * block the 8-wide add-trunc body then the scalar round tail. */
void ref_quantize_f16_to_i8_blocked(const uint16_t *w, int64_t out, int inp, int block,
                                    int8_t *q, float *s) {
    int nb = (inp + block - 1) / block;
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out; o++) {
        const uint16_t *wr = w + o * inp;
        int8_t *dr = q + o * inp;
        for (int b = 0; b < nb; b++) {
            int st = b * block, e = (b + 1) * block < inp ? (b + 1) * block : inp;
            float amax = 0.0f;
            for (int i = st; i < e; i++) amax = fmaxf(amax, fabsf(ref_f16_to_f32(wr[i])));
            float sc = fmaxf(amax, 1e-9f) / 127.0f;
            s[o * nb + b] = sc;
            float inv = 1.0f / sc;
            int j = st, e8 = st + ((e - st) / 8) * 8;
            for (; j < e8; j++)
                dr[j] = (int8_t)clampf(round_add_trunc(ref_f16_to_f32(wr[j]) * inv), -127.f, 127.f);
            for (; j < e; j++)
                dr[j] = (int8_t)clampf(round_half_away(ref_f16_to_f32(wr[j]) * inv), -127.f, 127.f);
        }
    }
}

/* quantize_rows_to_i7, nn.rs:869-927, via quantize_f16_bytes_to_i7 (nn.rs:947):
 * amax folded from 1e-9, scale amax/63, error-feedback rounding when ef
 * (FW_ENC_EF_QUANT default on, mod.rs:947-957), colsum of the i7 weights. */
void ref_quantize_rows_to_i7(const uint16_t *w, int64_t out, int inp, int ef, int8_t *q,
                             float *s, int32_t *colsum) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out; o++) {
        const uint16_t *wr = w + o * inp;
        int8_t *dr = q + o * inp;
        float amax = 1e-9f;
        for (int i = 0; i < inp; i++) amax = fmaxf(amax, fabsf(ref_f16_to_f32(wr[i])));
        float sc = amax / 63.0f;
        s[o] = sc;
        float inv = 1.0f / sc;
        int32_t acc = 0;
        if (ef) {
            float err = 0.0f;
            for (int i = 0; i < inp; i++) {
                float target = ref_f16_to_f32(wr[i]) * inv + err;
                float qq = clampf(round_half_away(target), -63.f, 63.f);
                err = target - qq;
                dr[i] = (int8_t)(int32_t)qq;
                acc += (int32_t)qq;
            }
        } else {
            for (int i = 0; i < inp; i++) {
                int32_t qq = (int32_t)clampf(round_half_away(ref_f16_to_f32(wr[i]) * inv), -63.f, 63.f);
                dr[i] = (int8_t)qq;
                acc += qq;
            }
        }
        colsum[o] = acc;
    }
}

/* quantize_enc_i8_rows, encoder.rs:2235-2263 (attn.out full i8). */
void ref_quantize_enc_i8_rows(const uint16_t *w, int64_t out, int inp, int8_t *q, float *s) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out; o++) {
        const uint16_t *wr = w + o * inp;
        float amax = 1e-9f;
        for (int i = 0; i < inp; i++) amax = fmaxf(amax, fabsf(ref_f16_to_f32(wr[i])));
        float sc = amax / 127.0f;
        s[o] = sc;
        float inv = 1.0f / sc;
        for (int i = 0; i < inp; i++)
            q[o * inp + i] = (int8_t)clampf(round_half_away(ref_f16_to_f32(wr[i]) * inv), -127.f, 127.f);
    }
}

/* ------------------------------------------------------------------------ */
/* Dots and GEMVs                                                           */
/* ------------------------------------------------------------------------ */

/* dot_i8, nn.rs:2635-2686: exact i32 sum (|sum| < 2^31 for n <= 5120). */
int32_t ref_dot_i8(const int8_t *w, const int8_t *x, int n) {
    if (g_fast) return rf_dot_i8(w, x, n);
    int32_t acc = 0;
    for (int i = 0; i < n; i++) acc += (int32_t)w[i] * (int32_t)x[i];
    return acc;
}

/* dot_f16c, nn.rs:1983-2051: 4 accumulators x 8 lanes with FMA over 32-wide
 * chunks; lane-wise (a0+a1)+(a2+a3); horizontal ((t0+t1)+(t2+t3))+((t4+t5)+(t6+t7));
 * then each 8-wide tail chunk reduced the same way and added; then scalar
 * mul+add. */
float ref_dot_f16c(const uint16_t *w, const float *x, int n) {
    if (g_fast) return rf_dot_f16c(w, x, n);
    float a[4][8];
    memset(a, 0, sizeof a);
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++)
                a[j][l] = fmaf(ref_f16_to_f32(w[i + 8 * j + l]), x[i + 8 * j + l], a[j][l]);
    float t[8];
    for (int l = 0; l < 8; l++) t[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    float s = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
    for (; i + 8 <= n; i += 8) {
        float p[8];
        for (int l = 0; l < 8; l++) p[l] = ref_f16_to_f32(w[i + l]) * x[i + l];
        s += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
    for (; i < n; i++) s += ref_f16_to_f32(w[i]) * x[i];
    return s;
}

/* dot_i8w_f32, nn.rs:3501-3564: dot_f16c's shape with an i8 weight. */
float ref_dot_i8w_f32(const int8_t *w, const float *x, int n) {
    if (g_fast) return rf_dot_i8w_f32(w, x, n);
    float a[4][8];
    memset(a, 0, sizeof a);
    int i = 0;
    for (; i + 32 <= n; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++)
                a[j][l] = fmaf((float)w[i + 8 * j + l], x[i + 8 * j + l], a[j][l]);
    float t[8];
    for (int l = 0; l < 8; l++) t[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
    float s = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
    for (; i + 8 <= n; i += 8) {
        float p[8];
        for (int l = 0; l < 8; l++) p[l] = (float)w[i + l] * x[i + l];
        s += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
    }
    for (; i < n; i++) s += (float)w[i] * x[i];
    return s;
}

/* gemv_i8, nn.rs:3168-3231: per-vector activation quant, then
 * ((f32)acc * s_w[o]) * s_x + (bias or 0.0)  (nn.rs:3187-3188). */
void ref_gemv_i8(const int8_t *W, const float *s_w, int64_t out, int inp, const float *x,
                 const float *bias, float *y) {
    float xs = ref_act_scale(x, inp);
    float xinv = 1.0f / xs;
    int8_t *xq = (int8_t *)malloc((size_t)inp);
    ref_quantize_act_i8(x, inp, xinv, xq);
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out; o++) {
        float acc = (float)ref_dot_i8(W + o * inp, xq, inp) * s_w[o] * xs;
        y[o] = acc + (bias ? bias[o] : 0.0f);
    }
    free(xq);
}

/* gemv_f16, nn.rs:2346-2460: dot_f16c per row (+ bias when present; the
 * two-row blocked form is bit-identical, nn.rs:2053-2225). */
void ref_gemv_f16(const uint16_t *W, int64_t out, int inp, const float *x, const float *bias,
                  float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out; o++) {
        float acc = ref_dot_f16c(W + o * inp, x, inp);
        y[o] = bias ? acc + bias[o] : acc;
    }
}

/* gemv_i8w_f32a_blocked, nn.rs:3756-3824: acc += dot(block)*scale in block
 * order, then + (bias or 0.0). */
void ref_gemv_i8w_f32a_blocked(const int8_t *W, const float *s, int64_t out, int inp, int block,
                               const float *x, const float *bias, float *y) {
    int nb = (inp + block - 1) / block;
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out; o++) {
        float acc = 0.0f;
        for (int b = 0; b < nb; b++) {
            int st = b * block, e = (b + 1) * block < inp ? (b + 1) * block : inp;
            acc += ref_dot_i8w_f32(W + o * inp + st, x + st, e - st) * s[o * nb + b];
        }
        y[o] = acc + (bias ? bias[o] : 0.0f);
    }
}

/* ------------------------------------------------------------------------ */
/* Row ops                                                                  */
/* ------------------------------------------------------------------------ */

/* layer_norm / layer_norm_into, nn.rs:4351-4545: f64 sequential mean and
 * variance, inv = 1/sqrt(var + (f64)eps), ((x-mean)*inv)*w + b, cast to f32. */
void ref_layer_norm(const float *x, float *y, int64_t rows, int cols, const float *w,
                    const float *b, float eps) {
    double e = (double)eps, n = (double)cols;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) {
        const float *xr = x + r * cols;
        float *yr = y + r * cols;
        double sum = 0.0;
        for (int j = 0; j < cols; j++) sum += (double)xr[j];
        double mean = sum / n;
        double var = 0.0;
        for (int j = 0; j < cols; j++) {
            double d = (double)xr[j] - mean;
            var += d * d;
        }
        var /= n;
        double inv = 1.0 / sqrt(var + e);
        for (int j = 0; j < cols; j++) {
            double normed = ((double)xr[j] - mean) * inv;
            yr[j] = (float)(normed * (double)w[j] + (double)b[j]);
        }
    }
}

/* gelu_table, nn.rs:4561-4575 (GELU_SQRT_2_OVER_PI = 0.797_884_6, GELU_COEF_A =
 * 0.044_715, nn.rs:4545-4547): f16-indexed tanh GELU re-rounded through f16. */
float ref_gelu_scalar(float f) {
    return 0.5f * f * (1.0f + tanhf(0.7978846f * f * (1.0f + 0.044715f * f * f)));
}
static float g_gelu_table[1 << 16];
static int g_gelu_ready = 0;
const float *ref_gelu_table(void) {
    if (!__atomic_load_n(&g_gelu_ready, __ATOMIC_ACQUIRE)) {
#pragma omp critical(refcpu_gelu)
        {
            if (!g_gelu_ready) {
                for (int i = 0; i < (1 << 16); i++) {
                    float f = ref_f16_to_f32((uint16_t)i);
                    g_gelu_table[i] = ref_f16_to_f32(ref_f32_to_f16(ref_gelu_scalar(f)));
                }
                __atomic_store_n(&g_gelu_ready, 1, __ATOMIC_RELEASE);
            }
        }
    }
    return g_gelu_table;
}

/* gelu_slice, nn.rs:4603-4673: x<=-10 -> 0, x>=10 -> x, else T[f16(x)]. */
void ref_gelu_inplace(float *x, int64_t n) {
    const float *t = ref_gelu_table();
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        float v = x[i];
        x[i] = v <= -10.0f ? 0.0f : (v >= 10.0f ? v : t[ref_f32_to_f16(v)]);
    }
}

/* softmax_rows, nn.rs:4880-4963 (FW_SIMD_EXP off): max fold from -inf (NaN
 * ignored), glibc expf, non-finite terms -> 0, sequential sum, *= 1/sum. */
static void softmax_row(float *row, int cols) {
    if (g_fast) {
        rf_softmax_row(row, cols);
        return;
    }
    float mx = -INFINITY;
    for (int j = 0; j < cols; j++) mx = fmaxf(mx, row[j]);
    if (!isfinite(mx)) return;
    float sum = 0.0f;
    for (int j = 0; j < cols; j++) {
        float e = expf(row[j] - mx);
        if (!isfinite(e)) e = 0.0f;
        row[j] = e;
        sum += e;
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int j = 0; j < cols; j++) row[j] *= inv;
    }
}
void ref_softmax_rows(float *x, int64_t rows, int cols) {
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++) softmax_row(x + r * cols, cols);
}

/* matmul with FT_SGEMM_STRICT_PARITY (nn.rs:587-604; m == 1 SAXPY nn.rs:565-577
 * is the same order): ascending-k sequential f32 mul+add per output. */
void ref_matmul_strict(const float *a, const float *b, float *c, int64_t m, int k, int n) {
    if (g_fast) {
        rf_matmul(a, k, b, n, c, n, m, k, n);
        return;
    }
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < m; i++) {
        float *orow = c + i * n;
        for (int j = 0; j < n; j++) orow[j] = 0.0f;
        for (int kk = 0; kk < k; kk++) {
            float av = a[i * k + kk];
            const float *brow = b + (int64_t)kk * n;
            for (int j = 0; j < n; j++) orow[j] += av * brow[j];
        }
    }
}

/* argmax_idx, decode.rs:1708-1780: first index of the max, strict '>'. */
int ref_argmax_first(const float *l, int n) {
    int bi = 0;
    float bv = -INFINITY;
    for (int i = 0; i < n; i++)
        if (l[i] > bv) { bv = l[i]; bi = i; }
    return bi;
}

static void add_bias_rows(float *y, int64_t rows, int cols, const float *b) {
    if (!b) return;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < rows; r++)
        for (int j = 0; j < cols; j++) y[r * cols + j] += b[j];
}

/* transpose a natural [out, in] f16 weight to the f32 [in, out] w_t the f32
 * matmul consumes (dequant_transpose_f16_bytes, encoder.rs:626). */
static float *f16_transpose_to_f32(const uint16_t *w, int64_t out, int64_t inp) {
    float *t = (float *)malloc(sizeof(float) * (size_t)(out * inp));
#pragma omp parallel for schedule(static)
    for (int64_t o = 0; o < out; o++)
        for (int64_t i = 0; i < inp; i++) t[i * out + o] = ref_f16_to_f32(w[o * inp + i]);
    return t;
}

/* conv1d_wt, nn.rs:5006-5103: im2col with column ci*K + kk, zero padding, then
 * matmul_bias (matmul, then the bias pass). */
static void conv1d_wt(const float *x, int t_in, int cin, const float *w_t, int cout,
                      const float *bias, int stride, float *out, int *t_out_p) {
    int patch = cin * CONV_K;
    int t_out = (t_in + 2 * CONV_PAD - CONV_K) / stride + 1;
    float *cols = (float *)calloc((size_t)t_out * patch, sizeof(float));
#pragma omp parallel for schedule(static)
    for (int o = 0; o < t_out; o++) {
        float *row = cols + (int64_t)o * patch;
        for (int kk = 0; kk < CONV_K; kk++) {
            int p = o * stride + kk;
            if (p < CONV_PAD) continue;
            int ti = p - CONV_PAD;
            if (ti >= t_in) continue;
            for (int ci = 0; ci < cin; ci++) row[ci * CONV_K + kk] = x[(int64_t)ti * cin + ci];
        }
    }
    ref_matmul_strict(cols, w_t, out, t_out, patch, cout);
    add_bias_rows(out, t_out, cout, bias);
    free(cols);
    *t_out_p = t_out;
}

/* attention_raw per-head path (FW_ATTN_NO_SDPA=1), nn.rs:6035-6131:
 * qh = q*s, kh = k*s (s = d_head^-0.25), scores = qh @ kh^T (strict), causal
 * mask j > cache_len + i when causal, softmax_rows, out = scores @ vh. */
static void attention_per_head(const float *q, int tq, const float *k, const float *v, int tk,
                               int n_state, int n_head, int causal, int cache_len, float *out) {
    int dh = n_state / n_head;
    float scale = powf((float)dh, -0.25f);
    /* Heads in order, rows in parallel inside (the same per-element order as
     * the reference: kh is transposed to kh_t [dh, tk] exactly as
     * attention_raw builds it, so each score accumulates d ascending while the
     * inner loop runs across independent keys). */
    float *qh = (float *)malloc(sizeof(float) * (size_t)tq * dh);
    float *kht = (float *)malloc(sizeof(float) * (size_t)tk * dh);
    /* FAST: the whole score block of a head as one strict-order matmul
     * (score j of row i: d ascending from +0.0f), the mask and softmax per
     * row, then P @ V_h (value d of row i: j ascending from +0.0f) */
    float *sc = g_fast ? (float *)malloc(sizeof(float) * (size_t)tq * tk) : NULL;
    for (int h = 0; h < n_head; h++) {
        int base = h * dh;
        for (int i = 0; i < tq; i++)
            for (int d = 0; d < dh; d++) qh[i * dh + d] = q[(int64_t)i * n_state + base + d] * scale;
        for (int j = 0; j < tk; j++)
            for (int d = 0; d < dh; d++) kht[(int64_t)d * tk + j] = k[(int64_t)j * n_state + base + d] * scale;
        if (sc) {
            rf_matmul(qh, dh, kht, tk, sc, tk, tq, dh, tk);
#pragma omp parallel for schedule(static)
            for (int i = 0; i < tq; i++) {
                float *srow = sc + (int64_t)i * tk;
                if (causal)
                    for (int j = cache_len + i + 1; j < tk; j++) srow[j] = -INFINITY;
                softmax_row(srow, tk);
            }
            rf_matmul(sc, tk, v + base, n_state, out + base, n_state, tq, tk, dh);
            continue;
        }
#pragma omp parallel
        {
            float *srow = (float *)malloc(sizeof(float) * (size_t)tk);
            float acc[256];
#pragma omp for schedule(static)
            for (int i = 0; i < tq; i++) {
                for (int j = 0; j < tk; j++) srow[j] = 0.0f;
                for (int d = 0; d < dh; d++) {
                    float qd = qh[i * dh + d];
                    const float *kr = kht + (int64_t)d * tk;
                    for (int j = 0; j < tk; j++) srow[j] += qd * kr[j];
                }
                if (causal)
                    for (int j = cache_len + i + 1; j < tk; j++) srow[j] = -INFINITY;
                softmax_row(srow, tk);
                for (int d = 0; d < dh; d++) acc[d] = 0.0f;
                for (int j = 0; j < tk; j++) {
                    float p = srow[j];
                    const float *vr = v + (int64_t)j * n_state + base;
                    for (int d = 0; d < dh; d++) acc[d] += p * vr[d];
                }
                for (int d = 0; d < dh; d++) out[(int64_t)i * n_state + base + d] = acc[d];
            }
            free(srow);
        }
    }
    free(sc);
    free(qh);
    free(kht);
}

/* Exported for the attention invariants (nn.rs:8472-8600): the per-head
 * attention of attention_raw (causal: query i sees keys j <= cache_len + i). */
void ref_attention(const float *q, int tq, const float *k, const float *v, int tk, int n_state,
                   int n_head, int causal, int cache_len, float *out) {
    attention_per_head(q, tq, k, v, tk, n_state, n_head, causal, cache_len, out);
}

/* ------------------------------------------------------------------------ */
/* Encoder                                                                  */
/* ------------------------------------------------------------------------ */
typedef struct {
    const fwhip_enc_layer *src;
    float *q_t, *k_t, *v_t, *o_t, *fc1_t, *fc2_t; /* f32 [in,out] (f32 plan) */
    int8_t *q7, *k7, *v7, *fc1_7, *fc2_7;         /* i7 [out,in] (int8 plan) */
    float *q7s, *k7s, *v7s, *fc1_7s, *fc2_7s;
    int32_t *q7c, *k7c, *v7c, *fc1_7c, *fc2_7c;
    int8_t *o8;
    float *o8s;
} enc_layer_t;

struct ref_encoder {
    fwhip_hparams hp;
    int precision, d, H, L, nmel, nctx, dff;
    float *conv1_t, *conv2_t;
    const float *conv1_b, *conv2_b, *pos_emb, *ln_post_w, *ln_post_b;
    enc_layer_t *layers;
};

static void i7_alloc_quant(const uint16_t *w, int out, int inp, int8_t **q, float **s, int32_t **c) {
    *q = (int8_t *)malloc((size_t)out * inp);
    *s = (float *)malloc(sizeof(float) * out);
    *c = (int32_t *)malloc(sizeof(int32_t) * out);
    ref_quantize_rows_to_i7(w, out, inp, 1, *q, *s, *c);
}

/* EncoderWeights::from_ggml_with_quality_safe_int8, encoder.rs:772-1029. */
ref_encoder *ref_encoder_new(const fwhip_encoder_weights *w, int precision) {
    ref_encoder *e = (ref_encoder *)calloc(1, sizeof *e);
    e->hp = w->hp;
    e->precision = precision;
    e->d = w->hp.n_audio_state;
    e->H = w->hp.n_audio_head;
    e->L = w->hp.n_audio_layer;
    e->nmel = w->hp.n_mels;
    e->nctx = w->hp.n_audio_ctx;
    e->dff = 4 * e->d;
    int d = e->d, dff = e->dff;
    e->conv1_t = f16_transpose_to_f32(w->conv1_w, d, (int64_t)e->nmel * CONV_K);
    e->conv2_t = f16_transpose_to_f32(w->conv2_w, d, (int64_t)d * CONV_K);
    e->conv1_b = w->conv1_b;
    e->conv2_b = w->conv2_b;
    e->pos_emb = w->pos_emb;
    e->ln_post_w = w->ln_post_w;
    e->ln_post_b = w->ln_post_b;
    e->layers = (enc_layer_t *)calloc((size_t)e->L, sizeof(enc_layer_t));
    for (int li = 0; li < e->L; li++) {
        const fwhip_enc_layer *s = &w->layers[li];
        enc_layer_t *l = &e->layers[li];
        l->src = s;
        if (precision == FWHIP_ENC_INT8) {
            i7_alloc_quant(s->q_w, d, d, &l->q7, &l->q7s, &l->q7c);
            i7_alloc_quant(s->k_w, d, d, &l->k7, &l->k7s, &l->k7c);
            i7_alloc_quant(s->v_w, d, d, &l->v7, &l->v7s, &l->v7c);
            i7_alloc_quant(s->fc1_w, dff, d, &l->fc1_7, &l->fc1_7s, &l->fc1_7c);
            i7_alloc_quant(s->fc2_w, d, dff, &l->fc2_7, &l->fc2_7s, &l->fc2_7c);
            l->o8 = (int8_t *)malloc((size_t)d * d);
            l->o8s = (float *)malloc(sizeof(float) * d);
            ref_quantize_enc_i8_rows(s->o_w, d, d, l->o8, l->o8s);
        } else {
            l->q_t = f16_transpose_to_f32(s->q_w, d, d);
            l->k_t = f16_transpose_to_f32(s->k_w, d, d);
            l->v_t = f16_transpose_to_f32(s->v_w, d, d);
            l->o_t = f16_transpose_to_f32(s->o_w, d, d);
            l->fc1_t = f16_transpose_to_f32(s->fc1_w, dff, d);
            l->fc2_t = f16_transpose_to_f32(s->fc2_w, d, dff);
        }
    }
    return e;
}

void ref_encoder_free(ref_encoder *e) {
    if (!e) return;
    for (int li = 0; li < e->L; li++) {
        enc_layer_t *l = &e->layers[li];
        free(l->q_t); free(l->k_t); free(l->v_t); free(l->o_t); free(l->fc1_t); free(l->fc2_t);
        free(l->q7); free(l->k7); free(l->v7); free(l->fc1_7); free(l->fc2_7);
        free(l->q7s); free(l->k7s); free(l->v7s); free(l->fc1_7s); free(l->fc2_7s);
        free(l->q7c); free(l->k7c); free(l->v7c); free(l->fc1_7c); free(l->fc2_7c);
        free(l->o8); free(l->o8s);
    }
    free(e->layers);
    free(e->conv1_t);
    free(e->conv2_t);
    free(e);
}

/* matmul_bias_i7_quantized, nn.rs:1537-1771 (quantize_act_i7 nn.rs:1443-1466 or
 * the GELU-fused quantize_act_i7_gelu nn.rs:1791-1823): acc = sum(u8*w) -
 * 128*colsum = sum(q_x*q_w) (exact), y = (f32)acc*s_x*s_w (+ bias). */
static void i7_gemm(const float *x, int64_t m, int inp, const int8_t *w, const float *ws,
                    const int32_t *wc, int out, const float *bias, int gelu_first, float *y,
                    int32_t *acc_out) {
    uint8_t *xq = (uint8_t *)malloc((size_t)m * inp);
    float *xs = (float *)malloc(sizeof(float) * (size_t)m);
    const float *gt = ref_gelu_table();
#pragma omp parallel
    {
        float *g = (float *)malloc(sizeof(float) * (size_t)inp);
#pragma omp for schedule(static)
        for (int64_t r = 0; r < m; r++) {
            const float *xr = x + r * inp;
            if (g_fast) {
                xs[r] = rf_quant_row_i7(xr, inp, gelu_first ? gt : NULL, ref_f32_to_f16, g, xq + r * inp);
                continue;
            }
            for (int i = 0; i < inp; i++) {
                float v = xr[i];
                if (gelu_first) v = v <= -10.0f ? 0.0f : (v >= 10.0f ? v : gt[ref_f32_to_f16(v)]);
                g[i] = v;
            }
            float s = ref_act_scale(g, inp);
            xs[r] = s;
            ref_quantize_row_i7_u8(g, inp, 1.0f / s, xq + r * inp);
        }
        free(g);
    }
    if (g_fast) {
        rf_epi e = {xs, ws, bias, wc, y, acc_out, 0};
        rf_gemm_u8i8(xq, w, m, inp, out, &e);
    } else {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < m; r++) {
            const uint8_t *xr = xq + r * inp;
            for (int o = 0; o < out; o++) {
                const int8_t *wr = w + (int64_t)o * inp;
                int32_t raw = 0;
                for (int i = 0; i < inp; i++) raw += (int32_t)xr[i] * (int32_t)wr[i];
                int32_t acc = raw - 128 * wc[o];
                if (acc_out) acc_out[r * out + o] = acc;
                float v = (float)acc * xs[r] * ws[o];
                if (bias) v += bias[o];
                y[r * out + o] = v;
            }
        }
    }
    free(xq);
    free(xs);
}

/* matmul_bias_i8, encoder.rs:2524-2606: exact per-row activation quant,
 * y = (f32)acc * s_x * s_w + bias. */
static void i8_gemm_enc(const float *x, int64_t m, int inp, const int8_t *w, const float *ws,
                        int out, const float *bias, float *y, int32_t *acc_out) {
    int8_t *xq = (int8_t *)malloc((size_t)m * inp);
    float *xs = (float *)malloc(sizeof(float) * (size_t)m);
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < m; r++) {
        float s = ref_act_scale(x + r * inp, inp);
        xs[r] = s;
        ref_quant_row_i8_exact(x + r * inp, inp, 1.0f / s, xq + r * inp);
    }
    if (g_fast) {
        rf_epi e = {xs, ws, bias, NULL, y, acc_out, 1};
        rf_gemm_i8i8(xq, w, m, inp, out, &e);
    } else {
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < m; r++) {
            for (int o = 0; o < out; o++) {
                int32_t acc = ref_dot_i8(w + (int64_t)o * inp, xq + r * inp, inp);
                if (acc_out) acc_out[r * out + o] = acc;
                y[r * out + o] = (float)acc * xs[r] * ws[o] + (bias ? bias[o] : 0.0f);
            }
        }
    }
    free(xq);
    free(xs);
}

void ref_enc_i7_gemm(const ref_encoder *e, int layer, int which, const float *x, int64_t m,
                     int32_t *acc_out, float *y_out) {
    const enc_layer_t *l = &e->layers[layer];
    int d = e->d, dff = e->dff;
    switch (which) {
    case 0: i7_gemm(x, m, d, l->q7, l->q7s, l->q7c, d, l->src->q_b, 0, y_out, acc_out); break;
    case 1: i7_gemm(x, m, d, l->k7, l->k7s, l->k7c, d, NULL, 0, y_out, acc_out); break;
    case 2: i7_gemm(x, m, d, l->v7, l->v7s, l->v7c, d, l->src->v_b, 0, y_out, acc_out); break;
    case 3: i8_gemm_enc(x, m, d, l->o8, l->o8s, d, l->src->o_b, y_out, acc_out); break;
    case 4: i7_gemm(x, m, d, l->fc1_7, l->fc1_7s, l->fc1_7c, dff, l->src->fc1_b, 0, y_out, acc_out); break;
    case 5: i7_gemm(x, m, dff, l->fc2_7, l->fc2_7s, l->fc2_7c, d, l->src->fc2_b, 1, y_out, acc_out); break;
    default: break;
    }
}

/* time_major_mel_window_from_full_mel, encoder.rs:684-714. */
void ref_mel_window(const float *full_mel, int n_mel, int64_t mel_frames, int64_t frame_offset,
                    int n_frames, float *out) {
    int64_t avail = mel_frames - frame_offset;
    if (avail < 0) avail = 0;
    int64_t copy = avail < n_frames ? avail : n_frames;
    float fill = copy == n_frames ? 0.0f : SILENCE_FLOOR;
    for (int64_t i = 0; i < (int64_t)n_frames * n_mel; i++) out[i] = fill;
    for (int64_t f = 0; f < copy; f++)
        for (int m = 0; m < n_mel; m++)
            out[f * n_mel + m] = full_mel[(int64_t)m * mel_frames + frame_offset + f];
}

/* encoder_block, encoder.rs:2608-2738, for the f32 plan (FW_ATTN_NO_SDPA=1) and
 * the quality-safe int8 plan with FW_ENC_QKV_FUSED=0 (q/k/v via
 * matmul_bias_i7_quantized, then nn::attention). */
static void encoder_block(const ref_encoder *e, const enc_layer_t *l, float *x, int T) {
    int d = e->d, dff = e->dff;
    int64_t Td = (int64_t)T * d;
    const fwhip_enc_layer *s = l->src;
    float *h = (float *)malloc(sizeof(float) * Td);
    float *q = (float *)malloc(sizeof(float) * Td);
    float *k = (float *)malloc(sizeof(float) * Td);
    float *v = (float *)malloc(sizeof(float) * Td);
    float *att = (float *)malloc(sizeof(float) * Td);
    float *f = (float *)malloc(sizeof(float) * (size_t)T * dff);
    ref_layer_norm(x, h, T, d, s->attn_ln_w, s->attn_ln_b, LN_EPS);
    if (e->precision == FWHIP_ENC_INT8) {
        i7_gemm(h, T, d, l->q7, l->q7s, l->q7c, d, s->q_b, 0, q, NULL);
        i7_gemm(h, T, d, l->k7, l->k7s, l->k7c, d, NULL, 0, k, NULL);
        i7_gemm(h, T, d, l->v7, l->v7s, l->v7c, d, s->v_b, 0, v, NULL);
    } else {
        ref_matmul_strict(h, l->q_t, q, T, d, d);
        add_bias_rows(q, T, d, s->q_b);
        ref_matmul_strict(h, l->k_t, k, T, d, d);
        ref_matmul_strict(h, l->v_t, v, T, d, d);
        add_bias_rows(v, T, d, s->v_b);
    }
    attention_per_head(q, T, k, v, T, d, e->H, 0, 0, att);
    if (e->precision == FWHIP_ENC_INT8) {
        i8_gemm_enc(att, T, d, l->o8, l->o8s, d, s->o_b, q, NULL);
    } else {
        ref_matmul_strict(att, l->o_t, q, T, d, d);
        add_bias_rows(q, T, d, s->o_b);
    }
    for (int64_t i = 0; i < Td; i++) x[i] += q[i]; /* add_in_place, encoder.rs:2753 */
    ref_layer_norm(x, h, T, d, s->mlp_ln_w, s->mlp_ln_b, LN_EPS);
    if (e->precision == FWHIP_ENC_INT8) {
        i7_gemm(h, T, d, l->fc1_7, l->fc1_7s, l->fc1_7c, dff, s->fc1_b, 0, f, NULL);
        i7_gemm(f, T, dff, l->fc2_7, l->fc2_7s, l->fc2_7c, d, s->fc2_b, 1, q, NULL);
        for (int64_t i = 0; i < Td; i++) x[i] += q[i];
    } else {
        /* gelu_add_bias (nn.rs:4703) then add_bias_residual (nn.rs:4741) */
        ref_matmul_strict(h, l->fc1_t, f, T, d, dff);
        add_bias_rows(f, T, dff, s->fc1_b);
        ref_gelu_inplace(f, (int64_t)T * dff);
        ref_matmul_strict(f, l->fc2_t, q, T, dff, d);
#pragma omp parallel for schedule(static)
        for (int64_t r = 0; r < T; r++)
            for (int j = 0; j < d; j++) x[r * d + j] += q[r * d + j] + s->fc2_b[j];
    }
    free(h); free(q); free(k); free(v); free(att); free(f);
}

/* tome_merge, encoder.rs:1403-1506 (bipartite soft matching), in the
 * strict-parity arithmetic: A = rows 0, 2, 4, ..., B = rows 1, 3, ...;
 * sim = A @ B^T by the strict matmul; row norms sqrt of the sequential f32 sum
 * of v*v, floored at 1e-9 (f32::max); cos = s / (na * nb); per A row the first
 * strict maximum over B (start -inf); the r = min(r, n_a, seq - 1) A rows with
 * the largest best similarity (a stable descending sort: ties keep the lower
 * A index) are added to their B partner in ascending A order and each B row
 * with count c > 1 is divided by c; merged = the B rows, then the kept A rows
 * in ascending order.  umap[seq]: original row -> merged row.  Returns the
 * merged row count seq - r. */
int ref_tome_merge(const float *x, int seq, int d, int r, float *merged, int32_t *umap) {
    int n_a = (seq + 1) / 2, n_b = seq / 2;
    if (r > n_a) r = n_a;
    if (r > seq - 1) r = seq - 1 > 0 ? seq - 1 : 0;
    float *a = (float *)malloc(sizeof(float) * ((size_t)n_a * d + 1));
    float *bt = (float *)malloc(sizeof(float) * ((size_t)n_b * d + 1));
    float *sim = (float *)malloc(sizeof(float) * ((size_t)n_a * (n_b > 0 ? n_b : 1) + 1));
    float *an = (float *)malloc(sizeof(float) * (n_a + 1));
    float *bn = (float *)malloc(sizeof(float) * (n_b + 1));
    float *best_sim = (float *)malloc(sizeof(float) * (n_a + 1));
    int *best_b = (int *)malloc(sizeof(int) * (n_a + 1));
    int *rank = (int *)malloc(sizeof(int) * (n_a + 1));
    int *counts = (int *)malloc(sizeof(int) * (n_b + 1));
    for (int i = 0; i < n_a; i++) memcpy(a + (size_t)i * d, x + (size_t)(2 * i) * d, sizeof(float) * d);
    /* b_t = transpose(B) [d, n_b] */
    for (int i = 0; i < n_b; i++)
        for (int k = 0; k < d; k++) bt[(size_t)k * n_b + i] = x[(size_t)(2 * i + 1) * d + k];
    if (n_b > 0) ref_matmul_strict(a, bt, sim, n_a, d, n_b);
    else for (int i = 0; i < n_a; i++) sim[i] = 0.0f; /* the reference's [n_a, 1] zero fallback */
    for (int i = 0; i < n_a; i++) {
        float s = 0.0f;
        for (int k = 0; k < d; k++) s += a[(size_t)i * d + k] * a[(size_t)i * d + k];
        s = sqrtf(s);
        an[i] = s > 1e-9f ? s : 1e-9f; /* f32::max (NaN -> 1e-9) */
    }
    for (int i = 0; i < n_b; i++) {
        const float *row = x + (size_t)(2 * i + 1) * d;
        float s = 0.0f;
        for (int k = 0; k < d; k++) s += row[k] * row[k];
        s = sqrtf(s);
        bn[i] = s > 1e-9f ? s : 1e-9f;
    }
    for (int i = 0; i < n_a; i++) {
        int bb = 0;
        float bs = -INFINITY;
        for (int j = 0; j < n_b; j++) {
            float cs = sim[(size_t)i * n_b + j] / (an[i] * bn[j]);
            if (cs > bs) {
                bs = cs;
                bb = j;
            }
        }
        best_b[i] = bb;
        best_sim[i] = bs;
    }
    /* stable descending sort: rank = #greater + #equal at a lower index */
    for (int i = 0; i < n_a; i++) {
        int rk = 0;
        for (int j = 0; j < n_a; j++)
            if (best_sim[j] > best_sim[i] || (j < i && best_sim[j] == best_sim[i])) rk++;
        rank[i] = rk;
    }
    for (int i = 0; i < n_b; i++) {
        memcpy(merged + (size_t)i * d, x + (size_t)(2 * i + 1) * d, sizeof(float) * d);
        counts[i] = 1;
    }
    for (int i = 0; i < n_a; i++)
        if (rank[i] < r) {
            float *m = merged + (size_t)best_b[i] * d;
            for (int k = 0; k < d; k++) m[k] += a[(size_t)i * d + k];
            counts[best_b[i]]++;
        }
    for (int i = 0; i < n_b; i++)
        if (counts[i] > 1) {
            float c = (float)counts[i];
            for (int k = 0; k < d; k++) merged[(size_t)i * d + k] /= c;
        }
    for (int i = 0; i < n_b; i++) umap[2 * i + 1] = i;
    int slot = n_b;
    for (int i = 0; i < n_a; i++) {
        if (rank[i] < r) {
            umap[2 * i] = best_b[i];
        } else {
            memcpy(merged + (size_t)slot * d, a + (size_t)i * d, sizeof(float) * d);
            umap[2 * i] = slot++;
        }
    }
    free(a); free(bt); free(sim); free(an); free(bn); free(best_sim); free(best_b); free(rank); free(counts);
    return seq - r;
}

/* tome_unmerge, encoder.rs:1509-1517: out[pos] = merged[umap[pos]]. */
void ref_tome_unmerge(const float *merged, const int32_t *umap, int seq, int d, float *out) {
    for (int p = 0; p < seq; p++) memcpy(out + (size_t)p * d, merged + (size_t)umap[p] * d, sizeof(float) * d);
}

/* forward_time_major, encoder.rs:1520-1677 (CPU blocks), with the ToMe
 * schedule of encoder.rs:1590-1632: with tome_r > 0 a merge is due after block
 * li when
 *   tome_every == 0 (single shot, FW_TOME_EVERY unset): no merge yet and
 *     li == tome_after;
 *   tome_every > 0 (progressive): li >= tome_after and (li - tome_after) is a
 *     multiple of tome_every;
 * and it runs (ref_tome_merge) when rows > r + 2 and rows - r >= tome_floor
 * (FW_TOME_FLOOR, 128 by default).  The map from every original row to its
 * current row is composed through each merge (cum[p] = umap[cum[p]]), so one
 * unmerge before ln_post restores the full sequence. */
int ref_encoder_forward_tome2(const ref_encoder *e, const float *x, int n_frames, float *out, int n_layers_run,
                              int tome_r, int tome_after, int tome_every, int tome_floor) {
    if (n_frames <= 0 || n_frames % 2 || n_frames > 2 * e->nctx) return FWHIP_ERR_INVALID;
    if (tome_every < 0 || tome_floor < 0) return FWHIP_ERR_INVALID;
    int d = e->d, t1, t2;
    float *a = (float *)malloc(sizeof(float) * (size_t)n_frames * d);
    conv1d_wt(x, n_frames, e->nmel, e->conv1_t, d, e->conv1_b, 1, a, &t1);
    ref_gelu_inplace(a, (int64_t)t1 * d);
    conv1d_wt(a, t1, d, e->conv2_t, d, e->conv2_b, 2, out, &t2);
    ref_gelu_inplace(out, (int64_t)t2 * d);
    free(a);
    for (int64_t r = 0; r < t2; r++)
        for (int j = 0; j < d; j++) out[r * d + j] += e->pos_emb[r * d + j];
    int n_run = n_layers_run < 0 || n_layers_run > e->L ? e->L : n_layers_run;
    /* cur: the current rows (out until the first merge); nxt: the next merge's
     * output; cum: original row -> current row */
    float *cur = out, *xa = NULL, *xb = NULL;
    int32_t *cum = NULL, *step = NULL;
    int rows = t2, n_merges = 0;
    for (int li = 0; li < n_run; li++) {
        encoder_block(e, &e->layers[li], cur, rows);
        int due = tome_every == 0 ? (n_merges == 0 && li == tome_after)
                                  : (li >= tome_after && (li - tome_after) % tome_every == 0);
        if (tome_r > 0 && due && rows > tome_r + 2 && rows - tome_r >= tome_floor) {
            if (!xa) {
                xa = (float *)malloc(sizeof(float) * (size_t)t2 * d);
                xb = (float *)malloc(sizeof(float) * (size_t)t2 * d);
                cum = (int32_t *)malloc(sizeof(int32_t) * t2);
                step = (int32_t *)malloc(sizeof(int32_t) * t2);
            }
            float *nxt = cur == xa ? xb : xa;
            int pre = rows;
            rows = ref_tome_merge(cur, pre, d, tome_r, nxt, step);
            if (n_merges == 0) memcpy(cum, step, sizeof(int32_t) * t2);
            else
                for (int p = 0; p < t2; p++) cum[p] = step[cum[p]];
            cur = nxt;
            n_merges++;
        }
    }
    if (n_merges) ref_tome_unmerge(cur, cum, t2, d, out);
    free(xa);
    free(xb);
    free(cum);
    free(step);
    float *y = (float *)malloc(sizeof(float) * (size_t)t2 * d);
    ref_layer_norm(out, y, t2, d, e->ln_post_w, e->ln_post_b, LN_EPS);
    memcpy(out, y, sizeof(float) * (size_t)t2 * d);
    free(y);
    return FWHIP_OK;
}

/* the single-shot schedule with the default floor (FW_TOME_EVERY and
 * FW_TOME_FLOOR unset) */
int ref_encoder_forward_tome(const ref_encoder *e, const float *x, int n_frames, float *out, int n_layers_run,
                             int tome_r, int tome_after) {
    return ref_encoder_forward_tome2(e, x, n_frames, out, n_layers_run, tome_r, tome_after, 0, 128);
}

int ref_encoder_forward(const ref_encoder *e, const float *x, int n_frames, float *out, int n_layers_run) {
    return ref_encoder_forward_tome(e, x, n_frames, out, n_layers_run, 0, 0);
}

/* ------------------------------------------------------------------------ */
/* Decoder                                                                  */
/* ------------------------------------------------------------------------ */
typedef struct {
    const fwhip_dec_layer *src;
    uint16_t *qkv_f16; /* [3d, d] fuse_qkv, decoder.rs:2245-2289 */
    float *qkv_b;      /* [q_b | 0 | v_b] */
    int8_t *qkv8, *o8, *cq8, *co8, *fc1_8, *fc2_b8;
    float *qkv8s, *o8s, *cq8s, *co8s, *fc1_8s, *fc2_b8s;
    float *ck_t, *cv_t; /* cross K/V weights dequantized + transposed (cross_proj_f32) */
} dec_layer_t;

struct ref_decoder {
    fwhip_hparams hp;
    int arm, d, H, dh, L, V, nctx, dff;
    int kv_f16; /* FW_KV_F16 for the states made next (1: f16 cache, 0: f32) */
    int cross_v_block; /* FW_CROSS_V_BLOCK for the states made next (int8 arm) */
    const uint16_t *tok_emb;
    const float *pos_emb, *ln_w, *ln_b;
    int8_t *emb8;
    float *emb8s;
    dec_layer_t *layers;
};

struct ref_dstate {
    int enc_frames, len;
    uint16_t *kv_k, *kv_v;   /* [L, nctx, d] f16 (FW_KV_F16) */
    float *kvf_k, *kvf_v;    /* [L, nctx, d] f32 (FW_KV_F16 unset: the reference's default) */
    uint16_t *ck16, *cvt16;  /* [L*H][T*dh] natural K, [L*H][dh*T] transposed V */
    int8_t *ck8, *cvt8;
    int8_t *cvb8;            /* FW_CROSS_V_BLOCK: [L*H][dh*T] block-int8 V^T (32-frame blocks) */
    float *cvbs;             /* [L*H][dh][ceil(T/32)] block scales */
    float *ck8s, *cvt8s;     /* [L*H][T], [L*H][dh] */
    /* FAST restatement only: per layer the scaled self-attention keys
     * f16_to_f32(k) * d_head^-0.25 of cached rows [0, kt_len[l]), transposed
     * [H][dh][kt_ld] so a key block is one vector; rows are appended as the
     * cache grows (the f16 cache stays the source of truth). */
    float *kt;
    int *kt_len, kt_ld, kt_nl;
};

static void q8_alloc(const uint16_t *w, int64_t out, int inp, int8_t **q, float **s) {
    *q = (int8_t *)malloc((size_t)(out * inp));
    *s = (float *)malloc(sizeof(float) * (size_t)out);
    ref_quantize_f16_to_i8(w, out, inp, *q, *s);
}

/* DecoderWeights::from_ggml, decoder.rs:752-932, with the default quant gates. */
ref_decoder *ref_decoder_new(const fwhip_decoder_weights *w, int arm) {
    ref_decoder *dd = (ref_decoder *)calloc(1, sizeof *dd);
    dd->hp = w->hp;
    dd->arm = arm;
    dd->d = w->hp.n_text_state;
    dd->H = w->hp.n_text_head;
    dd->dh = dd->d / dd->H;
    dd->L = w->hp.n_text_layer;
    dd->V = w->hp.n_vocab;
    dd->nctx = w->hp.n_text_ctx;
    dd->dff = 4 * dd->d;
    dd->kv_f16 = 1;
    dd->tok_emb = w->tok_emb;
    dd->pos_emb = w->pos_emb;
    dd->ln_w = w->ln_w;
    dd->ln_b = w->ln_b;
    int d = dd->d, dff = dd->dff;
    if (arm == FWHIP_DEC_INT8) q8_alloc(w->tok_emb, dd->V, d, &dd->emb8, &dd->emb8s);
    dd->layers = (dec_layer_t *)calloc((size_t)dd->L, sizeof(dec_layer_t));
    for (int li = 0; li < dd->L; li++) {
        const fwhip_dec_layer *s = &w->layers[li];
        dec_layer_t *l = &dd->layers[li];
        l->src = s;
        l->qkv_f16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)3 * d * d);
        memcpy(l->qkv_f16, s->q_w, sizeof(uint16_t) * (size_t)d * d);
        memcpy(l->qkv_f16 + (size_t)d * d, s->k_w, sizeof(uint16_t) * (size_t)d * d);
        memcpy(l->qkv_f16 + (size_t)2 * d * d, s->v_w, sizeof(uint16_t) * (size_t)d * d);
        l->qkv_b = (float *)calloc((size_t)3 * d, sizeof(float));
        memcpy(l->qkv_b, s->q_b, sizeof(float) * d);
        memcpy(l->qkv_b + 2 * d, s->v_b, sizeof(float) * d);
        if (arm == FWHIP_DEC_INT8) {
            q8_alloc(l->qkv_f16, 3 * d, d, &l->qkv8, &l->qkv8s);
            q8_alloc(s->o_w, d, d, &l->o8, &l->o8s);
            q8_alloc(s->cq_w, d, d, &l->cq8, &l->cq8s);
            q8_alloc(s->co_w, d, d, &l->co8, &l->co8s);
            q8_alloc(s->fc1_w, dff, d, &l->fc1_8, &l->fc1_8s);
            l->fc2_b8 = (int8_t *)malloc((size_t)d * dff);
            l->fc2_b8s = (float *)malloc(sizeof(float) * (size_t)d * (dff / 32));
            ref_quantize_f16_to_i8_blocked(s->fc2_w, d, dff, 32, l->fc2_b8, l->fc2_b8s);
        }
        l->ck_t = f16_transpose_to_f32(s->ck_w, d, d);
        l->cv_t = f16_transpose_to_f32(s->cv_w, d, d);
    }
    return dd;
}

void ref_decoder_free(ref_decoder *dd) {
    if (!dd) return;
    for (int li = 0; li < dd->L; li++) {
        dec_layer_t *l = &dd->layers[li];
        free(l->qkv_f16); free(l->qkv_b);
        free(l->qkv8); free(l->o8); free(l->cq8); free(l->co8); free(l->fc1_8); free(l->fc2_b8);
        free(l->qkv8s); free(l->o8s); free(l->cq8s); free(l->co8s); free(l->fc1_8s); free(l->fc2_b8s);
        free(l->ck_t); free(l->cv_t);
    }
    free(dd->layers);
    free(dd->emb8);
    free(dd->emb8s);
    free(dd);
}

/* DecoderState::new, decoder.rs:1040-1285: K = (enc @ Wk^T) * d_head^-0.25,
 * V = enc @ Wv^T + bv (cross_proj_f32: strict f32 matmul), per (layer, head)
 * natural K and transposed V rounded to f16, then per-row int8 copies. */
ref_dstate *ref_dstate_new(const ref_decoder *dd, const float *enc, int T) {
    int d = dd->d, H = dd->H, dh = dd->dh, L = dd->L;
    ref_dstate *s = (ref_dstate *)calloc(1, sizeof *s);
    s->enc_frames = T;
    if (dd->kv_f16) { /* KvCache::new reads FW_KV_F16, nn.rs:5097-5109 */
        s->kv_k = (uint16_t *)calloc((size_t)L * dd->nctx * d, sizeof(uint16_t));
        s->kv_v = (uint16_t *)calloc((size_t)L * dd->nctx * d, sizeof(uint16_t));
    } else {
        s->kvf_k = (float *)calloc((size_t)L * dd->nctx * d, sizeof(float));
        s->kvf_v = (float *)calloc((size_t)L * dd->nctx * d, sizeof(float));
    }
    s->ck16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)L * H * T * dh);
    s->cvt16 = (uint16_t *)malloc(sizeof(uint16_t) * (size_t)L * H * T * dh);
    float kscale = powf((float)dh, -0.25f);
    float *K = (float *)malloc(sizeof(float) * (size_t)T * d);
    float *Vv = (float *)malloc(sizeof(float) * (size_t)T * d);
    for (int li = 0; li < L; li++) {
        const dec_layer_t *l = &dd->layers[li];
        ref_matmul_strict(enc, l->ck_t, K, T, d, d);
        for (int64_t i = 0; i < (int64_t)T * d; i++) K[i] *= kscale;
        ref_matmul_strict(enc, l->cv_t, Vv, T, d, d);
        add_bias_rows(Vv, T, d, l->src->cv_b);
        for (int h = 0; h < H; h++) {
            uint16_t *kn = s->ck16 + ((size_t)li * H + h) * T * dh;
            uint16_t *vt = s->cvt16 + ((size_t)li * H + h) * T * dh;
            for (int j = 0; j < T; j++)
                for (int dd2 = 0; dd2 < dh; dd2++) {
                    kn[(size_t)j * dh + dd2] = ref_f32_to_f16(K[(size_t)j * d + h * dh + dd2]);
                    vt[(size_t)dd2 * T + j] = ref_f32_to_f16(Vv[(size_t)j * d + h * dh + dd2]);
                }
        }
    }
    free(K);
    free(Vv);
    if (dd->arm == FWHIP_DEC_INT8) {
        s->ck8 = (int8_t *)malloc((size_t)L * H * T * dh);
        s->cvt8 = (int8_t *)malloc((size_t)L * H * T * dh);
        s->ck8s = (float *)malloc(sizeof(float) * (size_t)L * H * T);
        s->cvt8s = (float *)malloc(sizeof(float) * (size_t)L * H * dh);
        for (int lh = 0; lh < L * H; lh++) {
            ref_quantize_f16_to_i8(s->ck16 + (size_t)lh * T * dh, T, dh, s->ck8 + (size_t)lh * T * dh,
                                   s->ck8s + (size_t)lh * T);
            ref_quantize_f16_to_i8(s->cvt16 + (size_t)lh * T * dh, dh, T, s->cvt8 + (size_t)lh * T * dh,
                                   s->cvt8s + (size_t)lh * dh);
        }
        if (dd->cross_v_block) {
            /* FW_CROSS_V_BLOCK (decoder.rs:1249-1263): each head's f16 V^T
             * [dh, T] block-quantized along the frames, 32 per scale */
            int nb = (T + 31) / 32;
            s->cvb8 = (int8_t *)malloc((size_t)L * H * T * dh);
            s->cvbs = (float *)malloc(sizeof(float) * (size_t)L * H * dh * nb);
            for (int lh = 0; lh < L * H; lh++)
                ref_quantize_f16_to_i8_blocked(s->cvt16 + (size_t)lh * T * dh, dh, T, 32,
                                               s->cvb8 + (size_t)lh * T * dh, s->cvbs + (size_t)lh * dh * nb);
        }
    }
    s->len = 0;
    return s;
}

void ref_dstate_free(ref_dstate *s) {
    if (!s) return;
    free(s->kt); free(s->kt_len);
    free(s->kv_k); free(s->kv_v); free(s->kvf_k); free(s->kvf_v); free(s->ck16); free(s->cvt16);
    free(s->ck8); free(s->cvt8); free(s->ck8s); free(s->cvt8s); free(s->cvb8); free(s->cvbs);
    free(s);
}
void ref_dstate_reset(ref_dstate *s) {
    s->len = 0;
    if (s->kt_len) memset(s->kt_len, 0, sizeof(int) * (size_t)s->kt_nl);
}
int ref_dstate_len(const ref_dstate *s) { return s->len; }
const uint16_t *ref_dstate_cross_k_f16(const ref_dstate *s) { return s->ck16; }
const uint16_t *ref_dstate_cross_vt_f16(const ref_dstate *s) { return s->cvt16; }

/* Linear::forward, decoder.rs:260-371, for one token row.  `prefill` selects
 * the tq > 1 arms (gemv_i8_batch == per-row gemv_i8; block-int8 weights fall
 * through to the f16 batch). kind: 0 qkv, 1 o, 2 cq, 3 co, 4 fc1, 5 fc2. */
static void dec_linear(const ref_decoder *dd, const dec_layer_t *l, int kind, const float *x,
                       int prefill, float *y) {
    const fwhip_dec_layer *s = l->src;
    int d = dd->d, dff = dd->dff;
    const uint16_t *wf = NULL;
    const float *b = NULL;
    int out = d, inp = d;
    const int8_t *w8 = NULL;
    const float *w8s = NULL;
    switch (kind) {
    case 0: wf = l->qkv_f16; b = l->qkv_b; out = 3 * d; w8 = l->qkv8; w8s = l->qkv8s; break;
    case 1: wf = s->o_w; b = s->o_b; w8 = l->o8; w8s = l->o8s; break;
    case 2: wf = s->cq_w; b = s->cq_b; w8 = l->cq8; w8s = l->cq8s; break;
    case 3: wf = s->co_w; b = s->co_b; w8 = l->co8; w8s = l->co8s; break;
    case 4: wf = s->fc1_w; b = s->fc1_b; out = dff; w8 = l->fc1_8; w8s = l->fc1_8s; break;
    default: wf = s->fc2_w; b = s->fc2_b; inp = dff; break;
    }
    if (dd->arm == FWHIP_DEC_INT8) {
        if (kind == 5) {
            if (!prefill) {
                ref_gemv_i8w_f32a_blocked(l->fc2_b8, l->fc2_b8s, d, dff, 32, x, b, y);
                return;
            }
        } else {
            ref_gemv_i8(w8, w8s, out, inp, x, b, y);
            return;
        }
    }
    ref_gemv_f16(wf, out, inp, x, b, y);
}

/* attention_decode_step_f16, nn.rs:6466-6540 (row attends to cache [0, tk)). */
static void self_attn_f16(const float *q, const uint16_t *kc, const uint16_t *vc, int tk, int d,
                          int H, float *out) {
    int dh = d / H;
    float scale = powf((float)dh, -0.25f);
    float *sc = (float *)malloc(sizeof(float) * (size_t)tk);
    for (int h = 0; h < H; h++) {
        int base = h * dh;
        float qh[256];
        for (int i = 0; i < dh; i++) qh[i] = q[base + i] * scale;
        for (int j = 0; j < tk; j++) {
            const uint16_t *kr = kc + (size_t)j * d + base;
            float acc = 0.0f;
            for (int i = 0; i < dh; i++) acc += qh[i] * (ref_f16_to_f32(kr[i]) * scale);
            sc[j] = acc;
        }
        softmax_row(sc, tk);
        for (int i = 0; i < dh; i++) out[base + i] = 0.0f;
        for (int j = 0; j < tk; j++) {
            const uint16_t *vr = vc + (size_t)j * d + base;
            for (int i = 0; i < dh; i++) out[base + i] += sc[j] * ref_f16_to_f32(vr[i]);
        }
    }
    free(sc);
}

/* attention_decode_step (nn.rs:6340-6400) over an f32 cache: the same
 * arithmetic as self_attn_f16 on rows stored as computed. */
static void self_attn_f32(const float *q, const float *kc, const float *vc, int tk, int d, int H, float *out) {
    int dh = d / H;
    float scale = powf((float)dh, -0.25f);
    float *sc = (float *)malloc(sizeof(float) * (size_t)tk);
    for (int h = 0; h < H; h++) {
        int base = h * dh;
        float qh[256];
        for (int i = 0; i < dh; i++) qh[i] = q[base + i] * scale;
        for (int j = 0; j < tk; j++) {
            const float *kr = kc + (size_t)j * d + base;
            float acc = 0.0f;
            for (int i = 0; i < dh; i++) acc += qh[i] * (kr[i] * scale);
            sc[j] = acc;
        }
        softmax_row(sc, tk);
        for (int i = 0; i < dh; i++) out[base + i] = 0.0f;
        for (int j = 0; j < tk; j++) {
            const float *vr = vc + (size_t)j * d + base;
            for (int i = 0; i < dh; i++) out[base + i] += sc[j] * vr[i];
        }
    }
    free(sc);
}

/* self_attn_f16 in the FAST restatement: the same per-element arithmetic
 * (score j = sequential sum over i of qh[i] * (f16_to_f32(k[j][i]) * s) from
 * +0.0f; value i = sequential sum over j of p[j] * f16_to_f32(v[j][i]) from
 * +0.0f), with the scaled keys kept transposed per state and the heads in
 * parallel. */
static void self_attn_fast(const ref_decoder *dd, ref_dstate *s, int li, const float *q, int tk, float *out) {
    int d = dd->d, H = dd->H, dh = d / H, nctx = dd->nctx;
    float scale = powf((float)dh, -0.25f);
    if (!s->kt) {
        s->kt_ld = (nctx + 7) & ~7;
        s->kt_nl = dd->L;
        s->kt = (float *)calloc((size_t)dd->L * d * s->kt_ld, sizeof(float));
        s->kt_len = (int *)calloc((size_t)dd->L, sizeof(int));
    }
    int ld = s->kt_ld;
    float *kt = s->kt + (size_t)li * d * ld;
    const size_t lo = (size_t)li * nctx * d;
    int from = s->kt_len[li] < tk - 1 ? s->kt_len[li] : tk - 1;
    for (int p = from; p < tk; p++)
        for (int c = 0; c < d; c++)
            kt[(size_t)c * ld + p] = (s->kvf_k ? s->kvf_k[lo + (size_t)p * d + c]
                                               : ref_f16_to_f32(s->kv_k[lo + (size_t)p * d + c])) * scale;
    s->kt_len[li] = tk;
#pragma omp parallel for schedule(static)
    for (int h = 0; h < H; h++) {
        int base = h * dh;
        float qh[256];
        float *sc = (float *)malloc(sizeof(float) * (size_t)ld);
        for (int i = 0; i < dh; i++) qh[i] = q[base + i] * scale;
        rf_scores_t(qh, kt + (size_t)base * ld, ld, dh, tk, sc);
        rf_softmax_row(sc, tk);
        if (s->kvf_v) rf_pv_f32(sc, s->kvf_v + lo + base, d, tk, dh, out + base);
        else rf_pv_f16(sc, s->kv_v + lo + base, d, tk, dh, out + base);
        free(sc);
    }
}

/* gemv_i8 (nn.rs:3168-3231) of one thread: the arithmetic of ref_gemv_i8. */
static void gemv_i8_serial(const int8_t *W, const float *s_w, int64_t out, int inp, const float *x, float *y,
                           int8_t *xq) {
    float xs = ref_act_scale(x, inp);
    ref_quantize_act_i8(x, inp, 1.0f / xs, xq);
    for (int64_t o = 0; o < out; o++) {
        float acc = (float)ref_dot_i8(W + o * inp, xq, inp) * s_w[o] * xs;
        y[o] = acc + 0.0f;
    }
}

/* Exported for the KV-cache invariant (nn.rs:8559): one decode-step row
 * attending to an f16 cache of tk rows. */
void ref_attention_decode_f16(const float *q, const uint16_t *kc, const uint16_t *vc, int tk, int d,
                              int H, float *out) {
    self_attn_f16(q, kc, vc, tk, d, H, out);
}
/* The same over an f32 cache (attention_decode_step, nn.rs:6340-6400). */
void ref_attention_decode_f32(const float *q, const float *kc, const float *vc, int tk, int d, int H, float *out) {
    self_attn_f32(q, kc, vc, tk, d, H, out);
}
/* FW_KV_F16 for the states ref_dstate_new makes next (1: f16, the initial
 * setting; 0: f32, the reference's default). */
void ref_decoder_set_kv_f16(ref_decoder *dd, int on) { dd->kv_f16 = on != 0; }
/* FW_CROSS_V_BLOCK for the states made next (the int8 arm; default off). */
void ref_decoder_set_cross_v_block(ref_decoder *dd, int on) { dd->cross_v_block = on != 0; }

/* cross_attention, decoder.rs:1524-1716 (FW_CROSS_F16 on; int8 K/V when the
 * int8 copies exist): qh = q*s; scores = gemv(K_h, qh); softmax; out =
 * gemv(Vt_h, p). */
static void cross_attn(const ref_decoder *dd, const ref_dstate *s, int li, const float *q,
                       float *out) {
    int d = dd->d, H = dd->H, dh = dd->dh, T = s->enc_frames;
    float scale = powf((float)dh, -0.25f);
    if (g_fast) { /* the same arithmetic, heads in parallel */
#pragma omp parallel for schedule(static)
        for (int h = 0; h < H; h++) {
            size_t lh = (size_t)li * H + h;
            float qh[256];
            float *sc = (float *)malloc(sizeof(float) * (size_t)T);
            int8_t *xq = (int8_t *)malloc((size_t)(T > dh ? T : dh));
            for (int i = 0; i < dh; i++) qh[i] = q[h * dh + i] * scale;
            if (dd->arm == FWHIP_DEC_INT8) {
                gemv_i8_serial(s->ck8 + lh * T * dh, s->ck8s + lh * T, T, dh, qh, sc, xq);
                rf_softmax_row(sc, T);
                if (s->cvb8) /* block-int8 V x f32 softmax weights (decoder.rs:1605-1608) */
                    ref_gemv_i8w_f32a_blocked(s->cvb8 + lh * T * dh, s->cvbs + lh * dh * ((T + 31) / 32), dh, T,
                                              32, sc, NULL, out + h * dh);
                else
                    gemv_i8_serial(s->cvt8 + lh * T * dh, s->cvt8s + lh * dh, dh, T, sc, out + h * dh, xq);
            } else {
                for (int j = 0; j < T; j++) sc[j] = rf_dot_f16c(s->ck16 + (lh * T + j) * dh, qh, dh);
                rf_softmax_row(sc, T);
                for (int i = 0; i < dh; i++) out[h * dh + i] = rf_dot_f16c(s->cvt16 + (lh * dh + i) * T, sc, T);
            }
            free(sc);
            free(xq);
        }
        return;
    }
    float *sc = (float *)malloc(sizeof(float) * (size_t)T);
    for (int h = 0; h < H; h++) {
        size_t lh = (size_t)li * H + h;
        float qh[256];
        for (int i = 0; i < dh; i++) qh[i] = q[h * dh + i] * scale;
        if (dd->arm == FWHIP_DEC_INT8) {
            ref_gemv_i8(s->ck8 + lh * T * dh, s->ck8s + lh * T, T, dh, qh, NULL, sc);
            softmax_row(sc, T);
            if (s->cvb8)
                ref_gemv_i8w_f32a_blocked(s->cvb8 + lh * T * dh, s->cvbs + lh * dh * ((T + 31) / 32), dh, T, 32,
                                          sc, NULL, out + h * dh);
            else
                ref_gemv_i8(s->cvt8 + lh * T * dh, s->cvt8s + lh * dh, dh, T, sc, NULL, out + h * dh);
        } else {
            ref_gemv_f16(s->ck16 + lh * T * dh, T, dh, qh, NULL, sc);
            softmax_row(sc, T);
            ref_gemv_f16(s->cvt16 + lh * T * dh, dh, T, sc, NULL, out + h * dh);
        }
    }
    free(sc);
    (void)d;
}

/* forward_step_hidden + logits_last, decoder.rs:1754-1906, 2048-2147, run row
 * by row: a tq > 1 prefill equals tq sequential rows because every op is
 * row-local except the causal self-attention, whose row i sees keys
 * [0, len+i] either way (attention_raw with the f16-dequantized cache,
 * nn.rs:6267-6337). */
int ref_decoder_step(const ref_decoder *dd, ref_dstate *s, const int32_t *tokens, int tq,
                     float *logits) {
    int d = dd->d, dff = dd->dff, nctx = dd->nctx;
    if (tq <= 0) return FWHIP_ERR_INVALID;
    for (int t = 0; t < tq; t++) {
        if (tokens[t] < 0 || tokens[t] >= dd->V) return FWHIP_ERR_INVALID;
        if (s->len + t >= nctx) return FWHIP_ERR_INVALID;
    }
    int prefill = tq > 1;
    float *x = (float *)malloc(sizeof(float) * d);
    float *h = (float *)malloc(sizeof(float) * d);
    float *qkv = (float *)malloc(sizeof(float) * 3 * d);
    float *att = (float *)malloc(sizeof(float) * d);
    float *y = (float *)malloc(sizeof(float) * d);
    float *ff = (float *)malloc(sizeof(float) * dff);
    for (int t = 0; t < tq; t++) {
        int pos = s->len + t;
        const uint16_t *er = dd->tok_emb + (size_t)tokens[t] * d;
        const float *pr = dd->pos_emb + (size_t)pos * d;
        for (int i = 0; i < d; i++) x[i] = ref_f16_to_f32(er[i]) + pr[i]; /* embed_tokens 1323 */
        for (int li = 0; li < dd->L; li++) {
            const dec_layer_t *l = &dd->layers[li];
            const fwhip_dec_layer *sw = l->src;
            ref_layer_norm(x, h, 1, d, sw->attn_ln_w, sw->attn_ln_b, LN_EPS);
            dec_linear(dd, l, 0, h, prefill, qkv);
            const size_t lo = (size_t)li * nctx * d;
            if (s->kvf_k) { /* KvCache::append, nn.rs:5352-5416: f32 rows as computed */
                for (int i = 0; i < d; i++) {
                    s->kvf_k[lo + (size_t)pos * d + i] = qkv[d + i];
                    s->kvf_v[lo + (size_t)pos * d + i] = qkv[2 * d + i];
                }
            } else { /* FW_KV_F16: rows rounded to f16 */
                for (int i = 0; i < d; i++) {
                    s->kv_k[lo + (size_t)pos * d + i] = ref_f32_to_f16(qkv[d + i]);
                    s->kv_v[lo + (size_t)pos * d + i] = ref_f32_to_f16(qkv[2 * d + i]);
                }
            }
            if (g_fast) self_attn_fast(dd, s, li, qkv, pos + 1, att);
            else if (s->kvf_k) self_attn_f32(qkv, s->kvf_k + lo, s->kvf_v + lo, pos + 1, d, dd->H, att);
            else self_attn_f16(qkv, s->kv_k + lo, s->kv_v + lo, pos + 1, d, dd->H, att);
            dec_linear(dd, l, 1, att, prefill, y);
            for (int i = 0; i < d; i++) x[i] += y[i];
            ref_layer_norm(x, h, 1, d, sw->cross_ln_w, sw->cross_ln_b, LN_EPS);
            dec_linear(dd, l, 2, h, prefill, y);
            cross_attn(dd, s, li, y, att);
            dec_linear(dd, l, 3, att, prefill, y);
            for (int i = 0; i < d; i++) x[i] += y[i];
            ref_layer_norm(x, h, 1, d, sw->mlp_ln_w, sw->mlp_ln_b, LN_EPS);
            dec_linear(dd, l, 4, h, prefill, ff);
            ref_gelu_inplace(ff, dff);
            dec_linear(dd, l, 5, ff, prefill, y);
            for (int i = 0; i < d; i++) x[i] += y[i];
        }
    }
    s->len += tq;
    ref_layer_norm(x, h, 1, d, dd->ln_w, dd->ln_b, LN_EPS);
    if (logits) {
        if (dd->arm == FWHIP_DEC_INT8) ref_gemv_i8(dd->emb8, dd->emb8s, dd->V, d, h, NULL, logits);
        else ref_gemv_f16(dd->tok_emb, dd->V, d, h, NULL, logits);
    }
    free(x); free(h); free(qkv); free(att); free(y); free(ff);
    return FWHIP_OK;
}

/* process_logits (decode.rs:702-867) in no-timestamps mode followed by
 * argmax (decode.rs:1782-1790).  With every timestamp masked the pairing,
 * initial-timestamp and monotonic rules mask nothing new and the
 * timestamp-forcing rule cannot fire, so the token is the first-index argmax
 * of the filtered logits. */
int ref_process_argmax(const fwhip_filter *f, const float *logits, int n, int initial) {
    float *l = (float *)malloc(sizeof(float) * (size_t)n);
    memcpy(l, logits, sizeof(float) * (size_t)n);
#define SETNEG(id) do { int _i = (id); if (_i >= 0 && _i < n) l[_i] = -INFINITY; } while (0)
    if (initial) {
        SETNEG(f->eot);
        if (f->space_token >= 0) SETNEG(f->space_token);
    }
    SETNEG(f->no_timestamps);
    for (int i = f->timestamp_begin; i < n; i++) SETNEG(i);
    SETNEG(f->sot);
    SETNEG(f->no_speech);
    SETNEG(f->solm);
    SETNEG(f->translate);
    SETNEG(f->transcribe);
    SETNEG(f->sot_prev);
    for (int li = 0; li < f->n_languages; li++) SETNEG(f->sot + 1 + li);
#undef SETNEG
    int tok = ref_argmax_first(l, n);
    free(l);
    return tok;
}

/* compute_logprobs (decode.rs:1666-1701): non-finite logits sanitized to
 * -inf, max, sequential f32 sum of expf(l - max) over the finite lanes (libm
 * expf), logf(sum) + max; masked lanes stay -inf. */
void ref_compute_logprobs(const float *logits, int n, float *lp) {
    float mx = -INFINITY;
    for (int i = 0; i < n; i++) {
        float l = isfinite(logits[i]) ? logits[i] : -INFINITY;
        mx = fmaxf(mx, l);
    }
    float s = 0.0f;
    for (int i = 0; i < n; i++) {
        float l = isfinite(logits[i]) ? logits[i] : -INFINITY;
        if (l > -INFINITY) s += expf(l - mx);
    }
    const float lse = logf(s) + mx;
    for (int i = 0; i < n; i++) {
        float l = isfinite(logits[i]) ? logits[i] : -INFINITY;
        lp[i] = l > -INFINITY ? l - lse : -INFINITY;
    }
}

/* process_logits (decode.rs:702-867) with FilterConfig (decode.rs:671-693):
 * the suppression rules in the reference's order, then compute_logprobs and
 * the timestamp-mass forcing rule.  logits is filtered in place; logprobs
 * receives the log-softmax (text lanes -inf when a timestamp is forced).
 * Returns 1 when a timestamp was forced. */
int ref_process_logits(const fwhip_filter *f, const ref_filter_cfg *cfg, float *l, float *lp, int n,
                       const int32_t *prev, int n_prev, int has_ts, int64_t seek_delta_cs, int tokens_in_window) {
    const int beg = f->timestamp_begin;
    const int initial = n_prev == 0;
#define SETNEG(id) do { int _i = (id); if (_i >= 0 && _i < n) l[_i] = -INFINITY; } while (0)
    if (cfg->suppress_blank && initial) {
        SETNEG(f->eot);
        if (f->space_token >= 0) SETNEG(f->space_token);
    }
    SETNEG(f->no_timestamps);
    if (cfg->no_timestamps)
        for (int i = beg; i < n; i++) SETNEG(i);
    if (!cfg->no_timestamps && cfg->max_tokens > 0 && tokens_in_window >= cfg->max_tokens)
        for (int i = 0; i < f->eot; i++) SETNEG(i);
    SETNEG(f->sot);
    SETNEG(f->no_speech);
    SETNEG(f->solm);
    SETNEG(f->translate);
    SETNEG(f->transcribe);
    SETNEG(f->sot_prev);
    for (int li = 0; li < f->n_languages; li++) SETNEG(f->sot + 1 + li);
    const int last_ts = n_prev > 0 && prev[n_prev - 1] >= beg;
    const int penult_ts = n_prev < 2 || prev[n_prev - 2] >= beg;
    if (last_ts) {
        if (penult_ts)
            for (int i = beg; i < n; i++) SETNEG(i);
        else
            for (int i = 0; i < f->eot; i++) SETNEG(i);
    }
    if (initial && cfg->max_initial_tid >= 0)
        for (int i = beg + cfg->max_initial_tid + 1; i < n; i++) SETNEG(i);
    if (has_ts) {
        const int tid0 = (int)(seek_delta_cs / 2);
        const int end = beg + tid0 < n ? beg + tid0 : n;
        for (int i = beg; i < end; i++) SETNEG(i);
    }
#undef SETNEG
    ref_compute_logprobs(l, n, lp);
    const int b = beg > 0 ? beg : 0;
    float ts_lp = -INFINITY;
    if (b < n) {
        float m = -INFINITY;
        for (int i = b; i < n; i++) m = fmaxf(m, lp[i]);
        if (isfinite(m)) {
            float s = 0.0f;
            for (int i = b; i < n; i++)
                if (lp[i] > -INFINITY) s += expf(lp[i] - m);
            if (s > 0.0f) ts_lp = logf(s) + m;
        }
    }
    float max_text = -INFINITY;
    for (int i = 0; i < b && i < n; i++) max_text = fmaxf(max_text, lp[i]);
    if (ts_lp > max_text) {
        for (int i = 0; i < b && i < n; i++) {
            l[i] = -INFINITY;
            lp[i] = -INFINITY;
        }
        return 1;
    }
    return 0;
}

/* Greedy window loop, decode.rs:3429-3566 (no timestamps, beam 1). */
int ref_decode_greedy(const ref_decoder *dd, ref_dstate *s, const int32_t *prompt, int n_prompt,
                      int n_max, const fwhip_filter *f, int32_t *out_tokens, int32_t *out_len) {
    float *logits = (float *)malloc(sizeof(float) * (size_t)dd->V);
    int rc = ref_decoder_step(dd, s, prompt, n_prompt, logits);
    int n = 0;
    for (int i = 0; rc == FWHIP_OK && i < n_max; i++) {
        int tok = ref_process_argmax(f, logits, dd->V, n == 0);
        out_tokens[n++] = tok;
        if (tok == f->eot) break;
        if (i + 1 == n_max) break; /* the reference's last forward is never sampled */
        rc = ref_decoder_step(dd, s, &tok, 1, logits);
    }
    *out_len = n;
    free(logits);
    return rc;
}


/* ======================================================================
 * log-mel frontend (mel.rs): periodic Hann window, the default two-for-one
 * real FFT of 400 points (one complex FFT of 200 points: radix-2 splits
 * 200 -> 100 -> 50 -> 25, radix-5 x 5 base), power spectrum, sparse f64 mel
 * projection, log10 approximation, global clamp and normalization.
 * ====================================================================== */
#define MEL_NFFT 400
#define MEL_HOP 160
#define MEL_NBINS 201
#define MEL_PAD1 480000 /* N_SAMPLES_30S */
#define MEL_PAD2 200    /* N_FFT / 2 */

static struct {
    int ready;
    float hann[MEL_NFFT];
    float lcos[4][200], lnsin[4][200]; /* widths 400, 200, 100, 50 (half 200 >> l) */
    float c5[25], s5[25], c25[25], s25[25];
} mel_t;

/* FftTwiddles::build / DftTable::build / hann_window (mel.rs:243-391):
 * f64 transcendentals narrowed to f32 */
static void mel_tables_init(void) {
    if (mel_t.ready) return;
    for (int i = 0; i < MEL_NFFT; i++)
        mel_t.hann[i] = (float)(0.5 * (1.0 - cos((2.0 * M_PI * (double)i) / (double)MEL_NFFT)));
    for (int l = 0; l < 4; l++) {
        const int n = MEL_NFFT >> l, half = n / 2;
        for (int k = 0; k < half; k++) {
            const double th = (2.0 * M_PI * (double)k) / (double)n;
            mel_t.lcos[l][k] = (float)cos(th);
            mel_t.lnsin[l][k] = -(float)sin(th);
        }
    }
    for (int k = 0; k < 5; k++)
        for (int j = 0; j < 5; j++) {
            const double th = (2.0 * M_PI * (double)(k * j)) / 5.0;
            mel_t.c5[k * 5 + j] = (float)cos(th);
            mel_t.s5[k * 5 + j] = (float)sin(th);
            const double th2 = (2.0 * M_PI * (double)(k * j)) / 25.0;
            mel_t.c25[k * 5 + j] = (float)cos(th2);
            mel_t.s25[k * 5 + j] = (float)sin(th2);
        }
    mel_t.ready = 1;
}

/* radix5_cdft, mel.rs:533-577: complex 25-point DFT as 5 x 5 */
static void mel_radix5_cdft(const float *in, float *out) {
    float ir[5][5], ii[5][5], tr[5][5], ti[5][5];
    for (int n2 = 0; n2 < 5; n2++)
        for (int k1 = 0; k1 < 5; k1++) {
            float re = 0.0f, im = 0.0f;
            for (int n1 = 0; n1 < 5; n1++) {
                const float xr = in[2 * (5 * n1 + n2)], xi = in[2 * (5 * n1 + n2) + 1];
                const float c = mel_t.c5[k1 * 5 + n1], sn = mel_t.s5[k1 * 5 + n1];
                re += xr * c + xi * sn;
                im += xi * c - xr * sn;
            }
            ir[n2][k1] = re;
            ii[n2][k1] = im;
        }
    for (int n2 = 0; n2 < 5; n2++)
        for (int k1 = 0; k1 < 5; k1++) {
            const float c = mel_t.c25[n2 * 5 + k1], sn = mel_t.s25[n2 * 5 + k1];
            tr[n2][k1] = ir[n2][k1] * c + ii[n2][k1] * sn;
            ti[n2][k1] = ii[n2][k1] * c - ir[n2][k1] * sn;
        }
    for (int k1 = 0; k1 < 5; k1++)
        for (int k2 = 0; k2 < 5; k2++) {
            float re = 0.0f, im = 0.0f;
            for (int n2 = 0; n2 < 5; n2++) {
                const float c = mel_t.c5[k2 * 5 + n2], sn = mel_t.s5[k2 * 5 + n2];
                re += tr[n2][k1] * c + ti[n2][k1] * sn;
                im += ti[n2][k1] * c - tr[n2][k1] * sn;
            }
            out[2 * (k1 + 5 * k2)] = re;
            out[2 * (k1 + 5 * k2) + 1] = im;
        }
}

/* cfft, mel.rs:604-646: recursive complex radix-2 DIT; level l has width 400 >> l */
static void mel_cfft(const float *in, float *out, int n, int l) {
    if (n == 1) {
        out[0] = in[0];
        out[1] = in[1];
        return;
    }
    if (n % 2 == 1) { /* n == 25 */
        mel_radix5_cdft(in, out);
        return;
    }
    const int half = n / 2;
    float even[400], odd[400], ef[400], of[400];
    for (int i = 0; i < half; i++) {
        even[2 * i] = in[2 * (2 * i)];
        even[2 * i + 1] = in[2 * (2 * i) + 1];
        odd[2 * i] = in[2 * (2 * i + 1)];
        odd[2 * i + 1] = in[2 * (2 * i + 1) + 1];
    }
    mel_cfft(even, ef, half, l + 1);
    mel_cfft(odd, of, half, l + 1);
    for (int k = 0; k < half; k++) {
        const float re = mel_t.lcos[l][k], im = mel_t.lnsin[l][k];
        const float re_odd = of[2 * k], im_odd = of[2 * k + 1];
        const float e_re = ef[2 * k], e_im = ef[2 * k + 1];
        out[2 * k] = e_re + re * re_odd - im * im_odd;
        out[2 * k + 1] = e_im + re * im_odd + im * re_odd;
        out[2 * (k + half)] = e_re - re * re_odd + im * im_odd;
        out[2 * (k + half) + 1] = e_im - re * im_odd - im * re_odd;
    }
}

/* fft_twoforone, mel.rs:648-695 (the default FFT path) */
void ref_mel_fft400(const float *in, float *out) {
    mel_tables_init();
    const int half = MEL_NFFT / 2;
    float z[400], zf[400];
    for (int m = 0; m < half; m++) {
        z[2 * m] = in[2 * m];
        z[2 * m + 1] = in[2 * m + 1];
    }
    mel_cfft(z, zf, half, 1);
    for (int k = 0; k < half; k++) {
        const int km = (half - k) % half;
        const float ar = zf[2 * k], ai = zf[2 * k + 1], br = zf[2 * km], bi = zf[2 * km + 1];
        const float e_re = 0.5f * (ar + br), e_im = 0.5f * (ai - bi);
        const float o_re = 0.5f * (ai + bi), o_im = 0.5f * (br - ar);
        const float re = mel_t.lcos[0][k], im = mel_t.lnsin[0][k];
        out[2 * k] = e_re + re * o_re - im * o_im;
        out[2 * k + 1] = e_im + re * o_im + im * o_re;
        out[2 * (k + half)] = e_re - re * o_re + im * o_im;
        out[2 * (k + half) + 1] = e_im - re * o_im - im * o_re;
    }
}

/* log10_floor_approx, mel.rs:1239-1249 */
float ref_log10_floor_approx(double x) {
    x = x > 1e-10 ? x : 1e-10;
    uint64_t bits;
    memcpy(&bits, &x, 8);
    const int64_t ex = (int64_t)((bits >> 52) & 0x7ff) - 1023;
    const uint64_t mb = (bits & 0x000fffffffffffffull) | 0x3ff0000000000000ull;
    double m;
    memcpy(&m, &mb, 8);
    const double t = (m - 1.0) / (m + 1.0);
    const double t2 = t * t;
    const double series = 1.0 + t2 * (1.0 / 3.0 + t2 * (1.0 / 5.0 + t2 * (1.0 / 7.0 + t2 * (1.0 / 9.0))));
    const double ln_m = 2.0 * t * series;
    return (float)(((double)ex * M_LN2 + ln_m) * (1.0 / M_LN10));
}

void ref_mel_hann(float *out400) {
    mel_tables_init();
    memcpy(out400, mel_t.hann, sizeof mel_t.hann);
}

int64_t ref_mel_frames(int64_t n_samples) {
    return (n_samples + MEL_PAD1 + 2 * MEL_PAD2 - MEL_NFFT) / MEL_HOP;
}

/* log_mel, mel.rs:1476-1660 (build_padded 1096-1125, compute_frame_column
 * 1167-1204, power_and_project 1206-1237, global clamp/normalize 1610-1650) */
void ref_log_mel(const float *samples, int64_t n, const float *filters, int n_mel, float *out) {
    mel_tables_init();
    const int64_t plen = n + MEL_PAD1 + 2 * MEL_PAD2;
    float *padded = (float *)calloc((size_t)plen, sizeof(float));
    memcpy(padded + MEL_PAD2, samples, sizeof(float) * (size_t)n);
    const int64_t refl = MEL_PAD2 < (n > 0 ? n - 1 : 0) ? MEL_PAD2 : (n > 0 ? n - 1 : 0);
    for (int64_t j = 1; j <= refl; j++) padded[MEL_PAD2 - j] = samples[j];
    const int64_t valid = n + MEL_PAD2;
    const int64_t nf = (plen - MEL_NFFT) / MEL_HOP;
    int *st = (int *)malloc(sizeof(int) * n_mel), *en = (int *)malloc(sizeof(int) * n_mel);
    for (int m = 0; m < n_mel; m++) { /* SparseMelFilters::new */
        const float *row = filters + (int64_t)m * MEL_NBINS;
        int a = -1, b = -1;
        for (int k = 0; k < MEL_NBINS; k++)
            if (row[k] != 0.0f) {
                if (a < 0) a = k;
                b = k;
            }
        st[m] = a < 0 ? 0 : a;
        en[m] = b < 0 ? 0 : b + 1;
    }
    const float floor10 = (float)log10(1e-10);
#pragma omp parallel for schedule(static)
    for (int64_t f = 0; f < nf; f++) {
        const int64_t off = f * MEL_HOP;
        if (off >= valid) {
            for (int m = 0; m < n_mel; m++) out[(int64_t)m * nf + f] = floor10;
            continue;
        }
        float in[MEL_NFFT], spec[2 * MEL_NFFT], pw[MEL_NBINS];
        const int64_t avail = valid - off < MEL_NFFT ? valid - off : MEL_NFFT;
        for (int j = 0; j < MEL_NFFT; j++) in[j] = j < avail ? mel_t.hann[j] * padded[off + j] : 0.0f;
        ref_mel_fft400(in, spec);
        for (int j = 0; j < MEL_NBINS; j++) {
            const float re = spec[2 * j], im = spec[2 * j + 1];
            pw[j] = re * re + im * im;
        }
        for (int m = 0; m < n_mel; m++) {
            const float *row = filters + (int64_t)m * MEL_NBINS;
            double sum = 0.0;
            for (int k = st[m]; k < en[m]; k++) sum += (double)pw[k] * (double)row[k];
            out[(int64_t)m * nf + f] = ref_log10_floor_approx(sum);
        }
    }
    const int64_t tot = (int64_t)n_mel * nf;
    float mx = -INFINITY;
    for (int64_t i = 0; i < tot; i++)
        if (out[i] > mx) mx = out[i];
    const float fl = mx - 8.0f;
    for (int64_t i = 0; i < tot; i++) {
        float v = out[i] < fl ? fl : out[i];
        out[i] = (v + 4.0f) / 4.0f;
    }
    free(st);
    free(en);
    free(padded);
}
