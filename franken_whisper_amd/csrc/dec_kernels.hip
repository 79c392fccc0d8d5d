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
// f16 GEMV in dot_f16c order (nn.rs:1983-2051), every stream in one launch so
// the weights are read once.
//
// dot_f16c keeps 4 accumulator vectors of 8 lanes: chain ch = 8 * jv + l
// (vector jv, lane l) takes element 32c + ch of each 32-element chunk c, FMA,
// in chunk order.  Here LPR lanes share a row and lane q owns the CPL = 32/LPR
// chains q*CPL .. q*CPL + CPL - 1 (contiguous elements of every chunk), for
// every stream of the pass.  Then the reference's reduction: lane-wise
// (a0 + a1) + (a2 + a3) by butterflies over the lanes holding the same l of
// other vectors, the 8-lane tree ((t0+t1)+(t2+t3))+((t4+t5)+(t6+t7)) (in-lane
// over a lane's aligned block of t, then butterflies), then the K % 32 tail
// (8-element chunks, each reduced the same way, then scalar mul + add) by the
// row's first lane.  Every add is commutative, so a butterfly leaves the same
// bits on both lanes.  The streams' x rows are staged in LDS by K-slabs.
template <int LPR, int SG>
__global__ void __launch_bounds__(256) k_gemv_f16m(const uint16_t *__restrict__ W, const float *__restrict__ bias,
                                                   const float *__restrict__ x, float *y, int N, int K, int ns,
                                                   int ldy, int mode, const float *__restrict__ gelu_tab, int cps) {
    // U chunks of weights in flight per lane: narrow per-lane loads need more
    // of them to cover the memory latency
    constexpr int CPL = 32 / LPR, RPB = 256 / LPR, U = CPL <= 2 ? 16 : CPL == 4 ? 8 : 4, NW = (CPL + 1) / 2;
    // a K-slab of every stream of the pass, chunk-major [cps][SG][32], so the
    // streams of one chunk sit at small constant offsets from one address
    extern __shared__ __align__(16) float xs[];
    const int q = threadIdx.x % LPR;
    const int nc = K >> 5, nslab = (nc + cps - 1) / cps, ntile = (N + RPB - 1) / RPB;
    // stage chunks [c0, c0 + cn) of streams [s0, s0 + sn): every load of a round
    // is issued before its LDS stores
    // (streams past sn of the pass are staged as zeros: the FMA loop runs all SG)
    auto stage = [&](int s0, int sn, int c0, int cn) {
        const int n4 = cn * 8, tot = SG * n4;
        for (int b0 = 0; b0 < tot; b0 += 256 * 8) {
            // unconditional loads from clamped (valid) addresses, so all eight
            // are in flight before the first wait
            float4 tmp[8];
#pragma unroll
            for (int r = 0; r < 8; r++) {
                int i = b0 + r * 256 + (int)threadIdx.x;
                i = i < tot ? i : tot - 1;
                const int sl = i / n4, c4 = i - sl * n4;
                const int sv = sl < sn ? sl : sn - 1;
                const float4 v = ((const float4 *)(x + (size_t)(s0 + sv) * K + (size_t)c0 * 32))[c4];
                tmp[r] = sl < sn ? v : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int r = 0; r < 8; r++) {
                const int i = b0 + r * 256 + (int)threadIdx.x;
                if (i < tot) {
                    const int sl = i / n4, c4 = i - sl * n4;
                    ((float4 *)xs)[((c4 >> 3) * SG + sl) * 8 + (c4 & 7)] = tmp[r];
                }
            }
        }
    };
    for (int s0 = 0; s0 < ns; s0 += SG) {
        const int sn = ns - s0 < SG ? ns - s0 : SG;
        if (nslab == 1) {
            __syncthreads();
            stage(s0, sn, 0, nc);
            __syncthreads();
        }
        for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
            const int row = tile * RPB + threadIdx.x / LPR;
            const bool ok = row < N;
            const uint16_t *wr = W + (size_t)(ok ? row : 0) * K + q * CPL;
            // CPL f16 weights of chunk c (rows past N read row 0, never stored)
            auto ldw = [&](int c, uint32_t (&u)[NW]) {
                const uint16_t *p = wr + (size_t)c * 32;
                if constexpr (CPL == 8) {
                    const uint4 v = *(const uint4 *)p;
                    u[0] = v.x; u[1] = v.y; u[2] = v.z; u[3] = v.w;
                } else if constexpr (CPL == 4) {
                    const uint2 v = *(const uint2 *)p;
                    u[0] = v.x; u[1] = v.y;
                } else if constexpr (CPL == 2) {
                    u[0] = *(const uint32_t *)p;
                } else {
                    u[0] = *p;
                }
            };
            float a[SG][CPL];
#pragma unroll
            for (int sl = 0; sl < SG; sl++)
#pragma unroll
                for (int e = 0; e < CPL; e++) a[sl][e] = 0.0f;
            for (int sb = 0; sb < nslab; sb++) {
                const int c0 = sb * cps, cn = nc - c0 < cps ? nc - c0 : cps;
                if (nslab > 1) {
                    __syncthreads();
                    stage(s0, sn, c0, cn);
                    __syncthreads();
                }
                uint32_t wq[U][NW];
#pragma unroll
                for (int u = 0; u < U; u++) ldw(c0 + (u < cn ? u : cn - 1), wq[u]);
                for (int c = 0; c < cn; c += U) {
                    uint32_t wc[U][NW];
#pragma unroll
                    for (int u = 0; u < U; u++) {
#pragma unroll
                        for (int e = 0; e < NW; e++) wc[u][e] = wq[u][e];
                        ldw(c0 + (c + U + u < cn ? c + U + u : cn - 1), wq[u]);
                    }
#pragma unroll
                    for (int u = 0; u < U; u++) {
                        if (c + u < cn) {
                            float wf[CPL];
#pragma unroll
                            for (int e = 0; e < CPL; e++)
                                wf[e] = fw_h2f((uint16_t)(CPL == 1 ? wc[u][0] : (wc[u][e >> 1] >> ((e & 1) * 16))));
                            const float *xc = xs + (c + u) * SG * 32 + q * CPL;
                            float xv[SG][CPL];
#pragma unroll
                            for (int sl = 0; sl < SG; sl++) {
                                if constexpr (CPL >= 4) {
#pragma unroll
                                    for (int e = 0; e < CPL; e += 4) {
                                        const float4 t = *(const float4 *)(xc + sl * 32 + e);
                                        xv[sl][e] = t.x; xv[sl][e + 1] = t.y; xv[sl][e + 2] = t.z; xv[sl][e + 3] = t.w;
                                    }
                                } else if constexpr (CPL == 2) {
                                    const float2 t = *(const float2 *)(xc + sl * 32);
                                    xv[sl][0] = t.x; xv[sl][1] = t.y;
                                } else {
                                    xv[sl][0] = xc[sl * 32];
                                }
                            }
#pragma unroll
                            for (int sl = 0; sl < SG; sl++)
#pragma unroll
                                for (int e = 0; e < CPL; e++) a[sl][e] = __builtin_fmaf(wf[e], xv[sl][e], a[sl][e]);
                        }
                    }
                }
            }
#pragma unroll
            for (int sl = 0; sl < SG; sl++) {
                if (sl < sn) {
                    // (a0 + a1) + (a2 + a3): vectors jv and jv ^ 1 sit 8 / CPL lanes apart
                    float t[CPL];
#pragma unroll
                    for (int e = 0; e < CPL; e++) {
                        float v = a[sl][e];
                        v = v + __shfl_xor(v, 8 / CPL, 64);
                        v = v + __shfl_xor(v, 16 / CPL, 64);
                        t[e] = v;
                    }
                    // ((t0+t1)+(t2+t3))+((t4+t5)+(t6+t7)): in-lane over this lane's
                    // aligned block of CPL values, then across the 8 / CPL lanes
#pragma unroll
                    for (int w = 1; w < CPL; w <<= 1)
#pragma unroll
                        for (int e = 0; e < CPL; e += 2 * w) t[e] = t[e] + t[e + w];
                    float acc = t[0];
#pragma unroll
                    for (int m = 1; m < 8 / CPL; m <<= 1) acc = acc + __shfl_xor(acc, m, 64);
                    if (q == 0 && ok) {
                        const float *xr = x + (size_t)(s0 + sl) * K;
                        const uint16_t *w0 = W + (size_t)row * K;
                        int i = nc * 32;
                        for (; i + 8 <= K; i += 8) {
                            float p[8];
                            for (int l = 0; l < 8; l++) p[l] = fw_h2f(w0[i + l]) * xr[i + l];
                            acc += ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
                        }
                        for (; i < K; i++) acc += fw_h2f(w0[i]) * xr[i];
                        const float v = bias ? acc + bias[row] : acc;
                        float *yp = y + (size_t)(s0 + sl) * ldy + row;
                        if (mode == 1) *yp = *yp + v;
                        else if (mode == 2) *yp = fw_gelu(v, gelu_tab);
                        else *yp = v;
                    }
                }
            }
        }
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

// Lanes per row: enough waves for narrow matrices (N <= 2048: 32 lanes, up to
// 8192: 16), 8 for the vocabulary-wide logits; streams go 16 per pass.  The
// streams' x rows sit in LDS (at most 96 KB: a K-slab of cps 32-chunks); when
// the whole row fits, the grid is persistent (two blocks per CU walk the row
// tiles, x staged once per block), else each block takes one row tile and
// stages the slabs in turn.
void fw_launch_gemv_f16(hipStream_t st, const uint16_t *W, const float *bias, const float *x, float *y, int N,
                        int K, int ns, int ldy, int mode, const float *gelu_tab) {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    const int nc = K >> 5;
    // streams per pass: the next of 1, 2, 4, 8, 10, 12, 16 (padding rows are zeros)
    const int spass = ns > 12 ? 16 : ns > 10 ? 12 : ns > 8 ? 10 : ns > 4 ? 8 : ns > 2 ? 4 : ns;
    int cps = (96 * 1024) / (spass * 128);
    cps = cps < nc ? cps : (nc > 0 ? nc : 1);
    const size_t shm = sizeof(float) * (size_t)spass * cps * 32;
    const bool one = cps >= nc;
#define GF_GO(LPR, SG)                                                                                      \
    do {                                                                                                    \
        const int ntile = (N + 256 / LPR - 1) / (256 / LPR);                                                \
        const int grid = one && ntile > 2 * n_cu ? 2 * n_cu : ntile;                                       \
        hipLaunchKernelGGL((k_gemv_f16m<LPR, SG>), dim3(grid), dim3(256), shm, st, W, bias, x, y, N, K, ns, \
                           ldy, mode, gelu_tab, cps);                                                      \
    } while (0)
#define GF_SG(LPR)                      \
    do {                                \
        switch (spass) {                \
        case 1: GF_GO(LPR, 1); break;   \
        case 2: GF_GO(LPR, 2); break;   \
        case 4: GF_GO(LPR, 4); break;   \
        case 8: GF_GO(LPR, 8); break;   \
        case 10: GF_GO(LPR, 10); break; \
        case 12: GF_GO(LPR, 12); break; \
        default: GF_GO(LPR, 16); break; \
        }                               \
    } while (0)
    if (N <= 2048) GF_SG(32);
    else if (N <= 8192) GF_SG(16);
    else GF_SG(8);
#undef GF_SG
#undef GF_GO
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
