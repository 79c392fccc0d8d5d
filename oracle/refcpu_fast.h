/* refcpu_fast.h — register-blocked AVX2 / F16C kernels of the oracle's FAST
 * restatement (test infrastructure: the CPU baseline's timed leg).  Each
 * returns the same bits as the strict scalar loop it replaces in refcpu.c. */
#ifndef REFCPU_FAST_H
#define REFCPU_FAST_H

#include <stdint.h>

/* c[m x n] (row stride ldc) = a[m x k] (lda) . b[k x n] (ldb), every output
 * the ascending-k sequence of f32 mul then add from +0.0f. */
void rf_matmul(const float *a, int64_t lda, const float *b, int64_t ldb, float *c, int64_t ldc, int64_t m,
               int k, int n);
/* Epilogue of the int8 GEMMs, per output (r, o): acc = raw - 128 * wc[o]
 * (wc may be NULL: acc = raw); acc_out[r][o] = acc when acc_out;
 * y[r][o] = (f32)acc * xs[r] * ws[o], then + bias[o], or + 0.0f when bias is
 * NULL and add_zero. */
typedef struct {
    const float *xs, *ws, *bias;
    const int32_t *wc;
    float *y;
    int32_t *acc_out;
    int add_zero;
} rf_epi;
/* y[m x n] from the exact i32 x[m x k] . w[n x k]^T (w magnitudes <= 63). */
void rf_gemm_u8i8(const uint8_t *x, const int8_t *w, int64_t m, int k, int n, const rf_epi *e);
/* y[m x n] from the exact i32 x[m x k] . w[n x k]^T. */
void rf_gemm_i8i8(const int8_t *x, const int8_t *w, int64_t m, int k, int n, const rf_epi *e);
/* quantize_row_i7_u8 of one row (optionally of its GELU), vectorized; g is
 * scratch of n floats; returns the row's activation scale. */
float rf_quant_row_i7(const float *x, int n, const float *gelu_tab, uint16_t (*f2h)(float), float *g,
                      uint8_t *out);
float rf_dot_f16c(const uint16_t *w, const float *x, int n);
float rf_dot_i8w_f32(const int8_t *w, const float *x, int n);
int32_t rf_dot_i8(const int8_t *w, const int8_t *x, int n);
/* y[i] = expf(x[i]) by the platform expf's table method, 8 lanes at a time */
void rf_expf_n(const float *x, float *y, int64_t n);
/* softmax_row of refcpu.c, exponentials 8 at a time, sum in index order */
void rf_softmax_row(float *row, int cols);
/* decode-step self attention pieces: scores against keys stored transposed
 * [dh][ld], and the f16 value pass, both in the strict sequential orders */
void rf_scores_t(const float *qh, const float *kt, int ld, int dh, int tk, float *sc);
void rf_pv_f16(const float *p, const uint16_t *v, int64_t ldv, int tk, int dh, float *out);
void rf_pv_f32(const float *p, const float *v, int64_t ldv, int tk, int dh, float *out);

#endif
