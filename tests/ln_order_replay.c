/* CPU replay of the decoder LayerNorm's two summation orders (test
 * infrastructure, compiled by tests/test_ln_order.py with -ffp-contract=off).
 *
 *  - the reference (layer_norm, nn.rs:4425-4438): f64 sums in index order;
 *  - the kernels' fast mode (fw_ln_quant_core in fw_dec.h): lane l of a
 *    64-lane wave holds the float4 groups l, l + 64, ... of the row, sums
 *    ((x0 + x1) + (x2 + x3)) per group into its partial in group order, and
 *    the wave reduces the 64 partials as a balanced tree (DPP pair, quad,
 *    half-row and row steps, then (r0 + r1) + (r2 + r3));
 *  - the kernels' exact mode: the mean is the tree sum when fw_row_sum_exact
 *    says every partial sum is exact, else the sequential sum; the variance is
 *    always the sequential sum.
 *
 * usage: ln_order_replay <kind> <rows> <d> <seed> [slack [dump]]
 *   slack (default 0) loosens the exactness bound by that many binades, to
 *   show that a wrong bound is caught (exact_pred_wrong > 0);
 *   dump: a file that receives every row whose fast-mode output differs, as
 *   f32 x, w, b, reference output, fast-mode output (5 d floats per row).
 *   kind 0: Gaussian rows N(0, 1), gains 1 and biases 0;
 *   kind 1: Gaussian rows with random gains/biases and a random offset;
 *   kind 2: adversarial rows for the exactness predicate (exponent spans of
 *           0-60 binades, near-constant rows, zeros and subnormals).
 * prints one JSON object of counts. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static uint64_t rng_s;
static uint64_t rnext(void) {
    uint64_t z = (rng_s += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
static double runif(void) { return ((rnext() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
static int g_have;
static double g_next;
static double rgauss(void) { /* Box-Muller, both outputs used */
    if (g_have) {
        g_have = 0;
        return g_next;
    }
    const double u = runif(), v = runif(), r = sqrt(-2.0 * log(u));
    g_next = r * sin(6.283185307179586 * v);
    g_have = 1;
    return r * cos(6.283185307179586 * v);
}

static double tree64(const double *p) {
    double t[64];
    memcpy(t, p, sizeof t);
    for (int w = 64; w > 1; w >>= 1)
        for (int i = 0; i < w / 2; i++) t[i] = t[2 * i] + t[2 * i + 1];
    return t[0];
}

/* the kernels' fast-mode partials and tree */
static double tree_sum_x(const float *x, int d) {
    double part[64];
    const int n4 = d / 4;
    for (int l = 0; l < 64; l++) {
        double s = 0.0;
        for (int g = l; g < n4; g += 64) {
            const float *v = x + 4 * g;
            s += ((double)v[0] + (double)v[1]) + ((double)v[2] + (double)v[3]);
        }
        part[l] = s;
    }
    return tree64(part);
}
static double tree_sum_sq(const float *x, int d, double mean) {
    double part[64];
    const int n4 = d / 4;
    for (int l = 0; l < 64; l++) {
        double s = 0.0;
        for (int g = l; g < n4; g += 64) {
            const float *v = x + 4 * g;
            const double a = (double)v[0] - mean, b = (double)v[1] - mean;
            const double c = (double)v[2] - mean, e = (double)v[3] - mean;
            s += (a * a + b * b) + (c * c + e * e);
        }
        part[l] = s;
    }
    return tree64(part);
}
static double seq_sum_x(const float *x, int d) {
    double s = 0.0;
    for (int i = 0; i < d; i++) s += (double)x[i];
    return s;
}
static double seq_sum_sq(const float *x, int d, double mean) {
    double s = 0.0;
    for (int i = 0; i < d; i++) {
        const double t = (double)x[i] - mean;
        s += t * t;
    }
    return s;
}
/* fw_row_sum_exact */
static int g_slack;
static int row_sum_exact(const float *x, int d) {
    int emx = 0, emn = 255;
    for (int i = 0; i < d; i++) {
        uint32_t u;
        memcpy(&u, &x[i], 4);
        const uint32_t a = u & 0x7fffffffu;
        if (a) {
            int e = (int)(a >> 23);
            if (e < 1) e = 1;
            if (e > emx) emx = e;
            if (e < emn) emn = e;
        }
    }
    if (emx == 0) return 1;
    int lg = 0;
    while ((1 << lg) < d) lg++;
    return emx < 255 && emx - emn <= 29 - lg + g_slack;
}
static void ln_out(const float *x, int d, double mean, double var, const float *w, const float *b, float *y) {
    const double inv = 1.0 / sqrt(var + (double)1e-5f);
    for (int i = 0; i < d; i++) y[i] = (float)((((double)x[i] - mean) * inv) * (double)w[i] + (double)b[i]);
}
static int same_bits_d(double a, double b) { return memcmp(&a, &b, 8) == 0; }

int main(int argc, char **argv) {
    if (argc < 5) return 2;
    const int kind = atoi(argv[1]);
    const long rows = atol(argv[2]);
    const int d = atoi(argv[3]);
    rng_s = strtoull(argv[4], NULL, 10);
    g_slack = argc > 5 ? atoi(argv[5]) : 0;
    FILE *dump = argc > 6 ? fopen(argv[6], "ab") : NULL;
    if (d % 4 || d > 1 << 16) return 2;
    float *x = malloc(sizeof(float) * d), *w = malloc(sizeof(float) * d), *b = malloc(sizeof(float) * d);
    float *y0 = malloc(sizeof(float) * d), *y1 = malloc(sizeof(float) * d), *y2 = malloc(sizeof(float) * d);
    long mean_diff = 0, var_diff = 0, out_rows_diff = 0, out_elems_diff = 0, pred_true = 0, pred_wrong = 0,
         exact_mode_diff = 0;
    for (long r = 0; r < rows; r++) {
        if (kind == 0) {
            for (int i = 0; i < d; i++) {
                x[i] = (float)rgauss();
                w[i] = 1.0f;
                b[i] = 0.0f;
            }
        } else if (kind == 1) {
            const double off = rgauss() * 2.0, sc = exp(rgauss());
            for (int i = 0; i < d; i++) {
                x[i] = (float)(off + sc * rgauss());
                w[i] = (float)(1.0 + 0.1 * rgauss());
                b[i] = (float)(0.1 * rgauss());
            }
        } else {
            const int sub = (int)(rnext() % 4);
            const int span = (int)(rnext() % 61);
            for (int i = 0; i < d; i++) {
                double v;
                if (sub == 0) /* random exponents over `span` binades, random signs */
                    v = ldexp(1.0 + runif(), -(int)(rnext() % (span + 1))) * ((rnext() & 1) ? 1 : -1);
                else if (sub == 1) /* near-constant row (silence): c + tiny noise */
                    v = 0.75 + ldexp(rgauss(), -span);
                else if (sub == 2) /* many zeros, some huge, some tiny */
                    v = (rnext() % 3 == 0) ? 0.0 : ldexp(rgauss(), (int)(rnext() % (span + 1)) - span / 2);
                else /* subnormals next to normals */
                    v = (rnext() % 2) ? ldexp(rgauss(), -140 + (int)(rnext() % 10)) : ldexp(rgauss(), -(int)(rnext() % (span + 1)));
                x[i] = (float)v;
                w[i] = 1.0f;
                b[i] = 0.0f;
            }
        }
        /* reference */
        const double ms = seq_sum_x(x, d), mean = ms / d;
        const double var = seq_sum_sq(x, d, mean) / d;
        ln_out(x, d, mean, var, w, b, y0);
        /* fast mode */
        const double tms = tree_sum_x(x, d), tmean = tms / d;
        const double tvar = tree_sum_sq(x, d, tmean) / d;
        ln_out(x, d, tmean, tvar, w, b, y1);
        /* exact mode */
        const int pred = row_sum_exact(x, d);
        pred_true += pred;
        if (pred && !same_bits_d(tms, ms)) pred_wrong++;
        const double emean = (pred ? tms : ms) / d;
        const double evar = seq_sum_sq(x, d, emean) / d;
        ln_out(x, d, emean, evar, w, b, y2);
        if (memcmp(y2, y0, sizeof(float) * d)) exact_mode_diff++;
        mean_diff += !same_bits_d(tmean, mean);
        var_diff += !same_bits_d(tvar, var);
        int nd = 0;
        for (int i = 0; i < d; i++) nd += memcmp(&y0[i], &y1[i], 4) != 0;
        out_elems_diff += nd;
        out_rows_diff += nd != 0;
        if (nd && dump) {
            fwrite(x, 4, d, dump);
            fwrite(w, 4, d, dump);
            fwrite(b, 4, d, dump);
            fwrite(y0, 4, d, dump);
            fwrite(y1, 4, d, dump);
        }
    }
    if (dump) fclose(dump);
    printf("{\"rows\": %ld, \"d\": %d, \"kind\": %d, \"mean_bits_differ\": %ld, \"var_bits_differ\": %ld, "
           "\"rows_output_differs\": %ld, \"elements_output_differ\": %ld, \"exact_pred_true\": %ld, "
           "\"exact_pred_wrong\": %ld, \"exact_mode_rows_differ\": %ld}\n",
           rows, d, kind, mean_diff, var_diff, out_rows_diff, out_elems_diff, pred_true, pred_wrong,
           exact_mode_diff);
    free(x);
    free(w);
    free(b);
    free(y0);
    free(y1);
    free(y2);
    return 0;
}
