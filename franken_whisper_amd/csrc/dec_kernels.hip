// dec_kernels.hip — decoder kernels shared by both arms and the pure-f16
// arm's kernels (gfx950); the int8 arm's per-token kernels are in dec_fast.hip.
//
// Every kernel reproduces the reference's per-output reduction order wherever
// that order feeds a floating-point rounding:
//  - f16 GEMVs: dot_f16c's 4x8 FMA accumulators and fixed add tree
//    (nn.rs:1983-2051) mapped onto 4 lanes per output row;
//  - f16 cross-attention: the same dot order for scores and outputs,
//    softmax with glibc-exact expf and a sequential sum (nn.rs:4880-4963);
//  - the strict f32 GEMM of the cross K/V precompute: ascending-k sequential
//    mul+add per output (nn.rs:587-604).
#include "fw_kernels.h"

#define LN_EPS_F 1e-5f

// ---------------------------------------------------------------------------
// f16 GEMV in dot_f16c order (nn.rs:1983-2051), MAXS streams per block.
// Lane j (0..3) of a 4-lane group owns accumulator vector a_j (8 lanes of the
// AVX register); chunk c covers elements [32c, 32c+32).
// Block = 256 threads; 64 rows per block.
template <int MAXS, int U>
__global__ void __launch_bounds__(256) k_gemv_f16(const uint16_t *__restrict__ W, const float *__restrict__ bias,
                                                  const float *__restrict__ x, float *y, int N, int K, int ns,
                                                  int ldy, int mode, const float *__restrict__ gelu_tab) {
    // blockIdx.y selects the stream group [s0, s0 + MAXS)
    const int s0 = blockIdx.y * MAXS;
    x += (size_t)s0 * K;
    y += (size_t)s0 * ldy;
    ns = ns - s0 < MAXS ? ns - s0 : MAXS;
    int j = threadIdx.x & 3;
    int row = blockIdx.x * 64 + (threadIdx.x >> 2);
    bool ok = row < N;
    const uint16_t *wr = W + (size_t)(ok ? row : 0) * K;
    float a[MAXS][8];
#pragma unroll
    for (int s = 0; s < MAXS; s++)
#pragma unroll
        for (int l = 0; l < 8; l++) a[s][l] = 0.0f;
    const int nc = K >> 5;
    // fma of one 32-chunk (8 weights per lane) into the MAXS accumulators
    auto chunk = [&](const uint4 wv, const float4 (&xc)[MAXS][2]) {
        float wf[8];
        wf[0] = fw_h2f(wv.x & 0xffff); wf[1] = fw_h2f(wv.x >> 16);
        wf[2] = fw_h2f(wv.y & 0xffff); wf[3] = fw_h2f(wv.y >> 16);
        wf[4] = fw_h2f(wv.z & 0xffff); wf[5] = fw_h2f(wv.z >> 16);
        wf[6] = fw_h2f(wv.w & 0xffff); wf[7] = fw_h2f(wv.w >> 16);
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            if (s < ns) {
                const float4 x0 = xc[s][0], x1 = xc[s][1];
                a[s][0] = __builtin_fmaf(wf[0], x0.x, a[s][0]);
                a[s][1] = __builtin_fmaf(wf[1], x0.y, a[s][1]);
                a[s][2] = __builtin_fmaf(wf[2], x0.z, a[s][2]);
                a[s][3] = __builtin_fmaf(wf[3], x0.w, a[s][3]);
                a[s][4] = __builtin_fmaf(wf[4], x1.x, a[s][4]);
                a[s][5] = __builtin_fmaf(wf[5], x1.y, a[s][5]);
                a[s][6] = __builtin_fmaf(wf[6], x1.z, a[s][6]);
                a[s][7] = __builtin_fmaf(wf[7], x1.w, a[s][7]);
            }
        }
    };
    auto load_x = [&](int c, float4 (&xc)[MAXS][2]) {
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            const float4 *xp = (const float4 *)(x + (size_t)(s < ns ? s : ns - 1) * K + c * 32 + j * 8);
            xc[s][0] = xp[0];
            xc[s][1] = xp[1];
        }
    };
    // the weight chunks of the next U iterations are in flight while the
    // current ones are used (rows past N read row 0 and are never stored)
    uint4 wq[U];
#pragma unroll
    for (int u = 0; u < U; u++) wq[u] = *(const uint4 *)(wr + (u < nc ? u : nc - 1) * 32 + j * 8);
    int c = 0;
    for (; c + U <= nc; c += U) {
        uint4 wc[U];
        float4 xc[U][MAXS][2];
#pragma unroll
        for (int u = 0; u < U; u++) {
            wc[u] = wq[u];
            const int cn = c + U + u < nc ? c + U + u : nc - 1;
            wq[u] = *(const uint4 *)(wr + cn * 32 + j * 8);
        }
#pragma unroll
        for (int u = 0; u < U; u++) load_x(c + u, xc[u]);
#pragma unroll
        for (int u = 0; u < U; u++) chunk(wc[u], xc[u]);
    }
    for (; c < nc; c++) {
        float4 xc[MAXS][2];
        load_x(c, xc);
        chunk(*(const uint4 *)(wr + c * 32 + j * 8), xc);
    }
    int tail8 = nc * 32;
#pragma unroll
    for (int s = 0; s < MAXS; s++) {
        if (s >= ns) continue;
        float t[8];
#pragma unroll
        for (int l = 0; l < 8; l++) {
            float v = a[s][l];
            v = v + __shfl_xor(v, 1, 64); // (a0+a1) | (a2+a3)
            v = v + __shfl_xor(v, 2, 64); // (a0+a1)+(a2+a3)
            t[l] = v;
        }
        float acc = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
        if (j == 0 && ok) {
            const float *xr = x + (size_t)s * K;
            int i = tail8;
            for (; i + 8 <= K; i += 8) {
                float p[8];
                for (int l = 0; l < 8; l++) p[l] = fw_h2f(wr[i + l]) * xr[i + l];
                acc += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
            }
            for (; i < K; i++) acc += fw_h2f(wr[i]) * xr[i];
            float v = bias ? acc + bias[row] : acc;
            float *yp = y + (size_t)s * ldy + row;
            if (mode == 1) *yp = *yp + v;
            else if (mode == 2) *yp = fw_gelu(v, gelu_tab);
            else *yp = v;
        }
    }
}

// Cross-attention, f16 K/V (FRANKEN_WHISPER_INT8_CROSS_KV=0 arm): scores =
// gemv_f16(K_h, qh) and out = gemv_f16(Vt_h, p), both in dot_f16c order.
__global__ void __launch_bounds__(256) k_cross_attn_f16(const float *qc, const uint16_t *ck,
                                                        const uint16_t *cvt, float *att, int d, int T, int H,
                                                        int L, int layer, float scale) {
    extern __shared__ float scf[]; // [T]
    __shared__ float qh[64];
    __shared__ float red[4];
    __shared__ float bc[1];
    int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    size_t lh = ((size_t)s * L + layer) * H + h;
    const uint16_t *K = ck + lh * (size_t)T * 64;
    const uint16_t *V = cvt + lh * (size_t)T * 64;
    if (t < 64) qh[t] = qc[(size_t)s * d + h * 64 + t] * scale;
    __syncthreads();
    float mx = -INFINITY;
    for (int jj = t; jj < T; jj += 256) {
        const uint16_t *kr = K + (size_t)jj * 64;
        float a[4][8];
        for (int q = 0; q < 4; q++)
            for (int l = 0; l < 8; l++) a[q][l] = 0.0f;
        for (int c = 0; c < 2; c++)
            for (int q = 0; q < 4; q++)
                for (int l = 0; l < 8; l++) {
                    int i = c * 32 + q * 8 + l;
                    a[q][l] = __builtin_fmaf(fw_h2f(kr[i]), qh[i], a[q][l]);
                }
        float tt[8];
        for (int l = 0; l < 8; l++) tt[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
        float v = ((tt[0] + tt[1]) + (tt[2] + tt[3])) + ((tt[4] + tt[5]) + (tt[6] + tt[7]));
        scf[jj] = v;
        mx = fmaxf(mx, v);
    }
    mx = fw_block_max(mx, red);
    bool fin = isfinite(mx);
    if (fin)
        for (int jj = t; jj < T; jj += 256) {
            float e = fw_expf(scf[jj] - mx);
            scf[jj] = isfinite(e) ? e : 0.0f;
        }
    __syncthreads();
    if (t == 0) {
        float sum = 0.0f;
        if (fin) for (int jj = 0; jj < T; jj++) sum += scf[jj];
        bc[0] = (fin && sum > 0.0f) ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    float inv = bc[0];
    if (inv > 0.0f)
        for (int jj = t; jj < T; jj += 256) scf[jj] = scf[jj] * inv;
    __syncthreads();
    // out[dd] = dot_f16c(V[dd, :T], p): lane j of the 4-lane group owns a_j
    int dd = t >> 2, j = t & 3;
    const uint16_t *vr = V + (size_t)dd * T;
    float a[8];
    for (int l = 0; l < 8; l++) a[l] = 0.0f;
    int nc = T >> 5;
    for (int c = 0; c < nc; c++)
        for (int l = 0; l < 8; l++) {
            int i = c * 32 + j * 8 + l;
            a[l] = __builtin_fmaf(fw_h2f(vr[i]), scf[i], a[l]);
        }
    float tt[8];
    for (int l = 0; l < 8; l++) {
        float v = a[l];
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        tt[l] = v;
    }
    float acc = ((tt[0] + tt[1]) + (tt[2] + tt[3])) + ((tt[4] + tt[5]) + (tt[6] + tt[7]));
    if (j == 0) {
        int i = nc * 32;
        for (; i + 8 <= T; i += 8) {
            float p[8];
            for (int l = 0; l < 8; l++) p[l] = fw_h2f(vr[i + l]) * scf[i + l];
            acc += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
        }
        for (; i < T; i++) acc += fw_h2f(vr[i]) * scf[i];
        att[(size_t)s * d + h * 64 + dd] = acc;
    }
}

// ---------------------------------------------------------------------------
// Strict f32 GEMM C[m,n] = A[m,k] x B^T, B natural [n,k] f16: every output is
// the ascending-k sequential mul+add of FT_SGEMM_STRICT_PARITY (nn.rs:587-604),
// so it reproduces the reference's strict-parity matmul bit for bit.
// 64x64 tile per 256-thread block, 4x4 outputs per thread, k staged by 16.
// epi: 0 plain [m,n]; 1 cross-K (scale, f16, per-head natural layout);
//      2 cross-V (+bias, f16, per-head transposed layout).
__global__ void __launch_bounds__(256) k_gemm_strict(const float *__restrict__ A, const uint16_t *__restrict__ B,
                                                     int m, int n, int k, int epi, float *C,
                                                     const float *bias, float scale, uint16_t *out16,
                                                     int T, int H, int L, int layer, int ldc,
                                                     const float *gelu_tab, const float *pos) {
    __shared__ float As[16][65];
    __shared__ float Bs[16][65];
    int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;
    int m0 = blockIdx.y * 64, n0 = blockIdx.x * 64;
    float c[4][4];
    for (int i = 0; i < 4; i++)
        for (int jj = 0; jj < 4; jj++) c[i][jj] = 0.0f;
    for (int k0 = 0; k0 < k; k0 += 16) {
        for (int e = threadIdx.x; e < 64 * 16; e += 256) {
            int r = e >> 4, kk = e & 15;
            int gr = m0 + r, gk = k0 + kk;
            As[kk][r] = (gr < m && gk < k) ? A[(size_t)gr * k + gk] : 0.0f;
            int gn = n0 + r;
            Bs[kk][r] = (gn < n && gk < k) ? fw_h2f(B[(size_t)gn * k + gk]) : 0.0f;
        }
        __syncthreads();
        int kmax = min(16, k - k0);
        for (int kk = 0; kk < kmax; kk++) {
            float a[4], b[4];
            for (int i = 0; i < 4; i++) a[i] = As[kk][ty * 4 + i];
            for (int jj = 0; jj < 4; jj++) b[jj] = Bs[kk][tx * 4 + jj];
            for (int i = 0; i < 4; i++)
                for (int jj = 0; jj < 4; jj++) c[i][jj] = c[i][jj] + a[i] * b[jj];
        }
        __syncthreads();
    }
    for (int i = 0; i < 4; i++) {
        int gr = m0 + ty * 4 + i;
        if (gr >= m) continue;
        for (int jj = 0; jj < 4; jj++) {
            int gn = n0 + tx * 4 + jj;
            if (gn >= n) continue;
            float v = c[i][jj];
            if (epi == 0) {
                if (bias) v = v + bias[gn];
                C[(size_t)gr * ldc + gn] = v;
            } else if (epi == 3) { // matmul_bias then GELU (conv stem, gelu_add_bias)
                C[(size_t)gr * ldc + gn] = fw_gelu(v + bias[gn], gelu_tab);
            } else if (epi == 4) { // conv2: GELU then + pos_emb (encoder.rs:1557-1572)
                C[(size_t)gr * ldc + gn] = fw_gelu(v + bias[gn], gelu_tab) + pos[(size_t)(gr % T) * ldc + gn];
            } else if (epi == 5) { // residual x += (acc + b) (add_bias_residual, nn.rs:4741)
                float *p = C + (size_t)gr * ldc + gn;
                *p = *p + (v + bias[gn]);
            } else {
                int s = gr / T, row = gr % T, h = gn >> 6, dd = gn & 63;
                size_t lh = ((size_t)s * L + layer) * H + h;
                if (epi == 1) {
                    out16[lh * (size_t)T * 64 + (size_t)row * 64 + dd] = fw_f2h(v * scale);
                } else {
                    out16[lh * (size_t)T * 64 + (size_t)dd * T + row] = fw_f2h(v + bias[gn]);
                }
            }
        }
    }
}

// Per-row int8 quantization of f16 rows (quantize_f16_row_to_i8_into,
// nn.rs:2490-2555): one 64-thread block per row.
__global__ void __launch_bounds__(64) k_quant_f16_rows(const uint16_t *src, int8_t *q, float *s, int n) {
    size_t r = blockIdx.x;
    const uint16_t *row = src + r * n;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += 64) m = fmaxf(m, fabsf(fw_h2f(row[i])));
    m = fw_wave_max(m);
    float sc = fmaxf(m, 1e-9f) / 127.0f;
    float inv = 1.0f / sc;
    for (int i = threadIdx.x; i < n; i += 64) q[r * n + i] = fw_q8_avx(fw_h2f(row[i]), inv, i, n);
    if (threadIdx.x == 0) s[r] = sc;
}

// ---------------------------------------------------------------------------
// launch wrappers

// Each thread's sequential chunk loop is latency-bound (a row's K/32 chunks in
// order), so matrices up to 32 M weights run one stream per block row of the
// grid (grid.y = ns) with 8 chunks of weights in flight per thread; larger ones
// (the logits) keep 4 streams per block so the weights are read ns/4 times.
void fw_launch_gemv_f16(hipStream_t st, const uint16_t *W, const float *bias, const float *x, float *y, int N,
                        int K, int ns, int ldy, int mode, const float *gelu_tab) {
    if ((size_t)N * K <= ((size_t)32 << 20) || ns == 1)
        hipLaunchKernelGGL((k_gemv_f16<1, 8>), dim3((N + 63) / 64, ns), dim3(256), 0, st, W, bias, x, y, N, K, ns,
                           ldy, mode, gelu_tab);
    else
        hipLaunchKernelGGL((k_gemv_f16<4, 4>), dim3((N + 63) / 64, (ns + 3) / 4), dim3(256), 0, st, W, bias, x, y, N,
                           K, ns, ldy, mode, gelu_tab);
}

void fw_launch_cross_attn_f16(hipStream_t st, const float *qc, const uint16_t *ck, const uint16_t *cvt,
                              float *att, int d, int T, int H, int L, int layer, int ns, float scale) {
    hipLaunchKernelGGL(k_cross_attn_f16, dim3(H, ns), dim3(256), sizeof(float) * T, st, qc, ck, cvt, att, d, T,
                       H, L, layer, scale);
}

// Greedy bookkeeping after a sampling step: record the sampled tokens, advance
// the shared position, clear the first-step flag.
__global__ void k_step_book(int *posp, int *initialp, const int32_t *tok, int32_t *hist, int stride, int step,
                            int ns, int advance) {
    int s = threadIdx.x;
    if (s < ns && hist) hist[(size_t)s * stride + step] = tok[s];
    if (s == 0) {
        if (advance) *posp = *posp + 1;
        if (initialp) *initialp = 0;
    }
}
void fw_launch_step_bookkeeping(hipStream_t st, int *posp, int *initialp, const int32_t *tok, int32_t *hist,
                                int hist_stride, int step, int ns) {
    hipLaunchKernelGGL(k_step_book, dim3(1), dim3(64), 0, st, posp, initialp, tok, hist, hist_stride, step, ns,
                       1);
}

void fw_launch_gemm_strict(hipStream_t st, const float *A, const uint16_t *B, int m, int n, int k, int epi,
                           float *C, const float *bias, float scale, uint16_t *out16, int T, int H, int L,
                           int layer, int ldc, const float *gelu_tab, const float *pos) {
    dim3 grid((n + 63) / 64, (m + 63) / 64);
    hipLaunchKernelGGL(k_gemm_strict, grid, dim3(256), 0, st, A, B, m, n, k, epi, C, bias, scale, out16, T, H,
                       L, layer, ldc > 0 ? ldc : n, gelu_tab, pos);
}

void fw_launch_quant_f16_rows(hipStream_t st, const uint16_t *src, int8_t *q, float *s, int rows, int n) {
    hipLaunchKernelGGL(k_quant_f16_rows, dim3(rows), dim3(64), 0, st, src, q, s, n);
}
