// enc_kernels.hip — encoder kernels for gfx950 (MFMA).
//
// The encoder is a dense contraction: every linear and the conv stem are one
// tiled MFMA GEMM template with two operand kinds:
//   KIND_I8   : i8 x i8 -> i32 (v_mfma_i32_32x32x32_i8).  The int8 path's
//               accumulators are exact integers, equal to the reference's
//               maddubs sum minus 128*colsum (nn.rs:1537-1771) or its i8 dot
//               (encoder.rs:2524-2606); epilogue ((f32)acc * s_x) * s_w (+ b).
//   KIND_F16S : f32 activations carried as an f16 pair (hi, lo = f16(a - hi))
//               against the f16 weights (exact: the reference dequantizes f16
//               weights to f32), two v_mfma_f32_32x32x16_f16 per product;
//               per-product error <= 2^-22 |a| + 2^-25, fp32 accumulation.
// Tile 128x128 per 256-thread block (2x2 waves of 64x64 = 2x2 MFMA 32x32
// tiles), K staged through LDS in 64-byte rows, double buffered.
//
// MFMA operand layouts (verified on gfx950): A lane l -> row l%32, k block
// (l/32)*16 bytes; B lane l -> col l%32, same k block; accumulator r of lane l
// -> row (r/4)*8 + (l/32)*4 + r%4, col l%32.
#include "fw_enc.h"

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

#define LDSR 80 // padded LDS row stride in bytes (64 data + 16 pad)

__device__ __forceinline__ void fw_split(float v, uint16_t &hi, uint16_t &lo) {
    asm volatile("" : "+v"(v));
    _Float16 h = (_Float16)v;
    float r = v - (float)h;
    asm volatile("" : "+v"(r));
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (_Float16)r);
}

template <int KIND>
__global__ void __launch_bounds__(256) k_gemm(FwGemm g) {
    constexpr int NA = KIND == FW_KIND_F16S ? 2 : 1;
    constexpr int ES = KIND == FW_KIND_I8 ? 1 : 2;
    constexpr int BM = 128, BN = 128;
    constexpr int TILE_BYTES = (NA * BM + BN) * LDSR;
    __shared__ __align__(16) unsigned char lds[2 * TILE_BYTES];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    // XCD-friendly tile order: consecutive blocks walk N first within a band
    // of row tiles so a band's A rows stay hot in one L2.
    const int gx = gridDim.x;
    const int bid = blockIdx.y * gx + blockIdx.x;
    const int n_tile = bid % gx, m_tile = bid / gx;
    const int m0 = m_tile * BM, n0 = n_tile * BN;
    const int kstep = 64 / ES; // k elements per stage
    const int nsteps = g.K / kstep;

    // global -> register staging: 512 16-byte chunks per operand tile, 2 per thread
    int4 ra[NA][2], rb[2];
    auto gload = [&](int s) {
#pragma unroll
        for (int q = 0; q < 2; q++) {
            int c = tid + q * 256;
            int row = c >> 2, cc = c & 3;
            size_t koff = (size_t)s * 64 + cc * 16; // bytes
            int gr = m0 + row;
#pragma unroll
            for (int a = 0; a < NA; a++) {
                const unsigned char *base = (const unsigned char *)(a == 0 ? g.A : g.A2);
                ra[a][q] = gr < g.M ? *(const int4 *)(base + (size_t)gr * g.lda * ES + koff) : make_int4(0, 0, 0, 0);
            }
            int gn = n0 + row;
            rb[q] = gn < g.N ? *(const int4 *)((const unsigned char *)g.B + (size_t)gn * g.ldb * ES + koff)
                             : make_int4(0, 0, 0, 0);
        }
    };
    auto lstore = [&](int buf) {
        unsigned char *t = lds + buf * TILE_BYTES;
#pragma unroll
        for (int q = 0; q < 2; q++) {
            int c = tid + q * 256;
            int row = c >> 2, cc = c & 3;
#pragma unroll
            for (int a = 0; a < NA; a++) *(int4 *)(t + (a * BM + row) * LDSR + cc * 16) = ra[a][q];
            *(int4 *)(t + (NA * BM + row) * LDSR + cc * 16) = rb[q];
        }
    };

    typedef typename std::conditional<KIND == FW_KIND_I8, v16i, v16f>::type accT;
    accT acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) acc[i][j][r] = 0;

    gload(0);
    lstore(0);
    __syncthreads();
    int buf = 0;
    for (int s = 0; s < nsteps; s++) {
        if (s + 1 < nsteps) gload(s + 1);
        const unsigned char *t = lds + buf * TILE_BYTES;
#pragma unroll
        for (int ks = 0; ks < 2; ks++) {
            int koff = ks * 32 + (lane >> 5) * 16;
            v4i af[NA][2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                int row = wm * 64 + i * 32 + (lane & 31);
#pragma unroll
                for (int a = 0; a < NA; a++) af[a][i] = *(const v4i *)(t + (a * BM + row) * LDSR + koff);
            }
#pragma unroll
            for (int j = 0; j < 2; j++) {
                int row = wn * 64 + j * 32 + (lane & 31);
                bf[j] = *(const v4i *)(t + (NA * BM + row) * LDSR + koff);
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    if constexpr (KIND == FW_KIND_I8) {
                        acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[0][i], bf[j], acc[i][j], 0, 0, 0);
                    } else {
                        v8h bh = __builtin_bit_cast(v8h, bf[j]);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, af[0][i]), bh,
                                                                           acc[i][j], 0, 0, 0);
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(v8h, af[1][i]), bh,
                                                                           acc[i][j], 0, 0, 0);
                    }
                }
        }
        if (s + 1 < nsteps) lstore(buf ^ 1);
        __syncthreads();
        buf ^= 1;
    }

    // epilogue
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            int col = n0 + wn * 64 + j * 32 + (lane & 31);
            if (col >= g.N) continue;
            float sw = g.sw ? g.sw[col] : 1.0f;
            float bias = g.bias ? g.bias[col] : 0.0f;
#pragma unroll
            for (int r = 0; r < 16; r++) {
                int row = m0 + wm * 64 + i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                if (row >= g.M) continue;
                if (g.epi == FW_EPI_ACC32) { // raw accumulator (per-GEMM parity)
                    if constexpr (KIND == FW_KIND_I8) ((int *)g.C)[(size_t)row * g.ldc + col] = acc[i][j][r];
                    else g.C[(size_t)row * g.ldc + col] = acc[i][j][r];
                    continue;
                }
                float v;
                if constexpr (KIND == FW_KIND_I8) {
                    v = (float)acc[i][j][r] * g.sx[row] * sw;
                } else {
                    v = acc[i][j][r];
                }
                if (g.bias) v = v + bias;
                switch (g.epi) {
                case FW_EPI_F32: g.C[(size_t)row * g.ldc + col] = v; break;
                case FW_EPI_RESID: {
                    float *p = g.C + (size_t)row * g.ldc + col;
                    *p = *p + v;
                    break;
                }
                case FW_EPI_GELU_F32: g.C[(size_t)row * g.ldc + col] = fw_gelu(v, g.gelu_tab); break;
                case FW_EPI_GELU_SPLIT: {
                    uint16_t hi, lo;
                    fw_split(fw_gelu(v, g.gelu_tab), hi, lo);
                    g.o16[0][(size_t)row * g.ldc + col] = hi;
                    g.o16[1][(size_t)row * g.ldc + col] = lo;
                    break;
                }
                case FW_EPI_CONV2: {
                    int t = row % g.T;
                    g.C[(size_t)row * g.ldc + col] = fw_gelu(v, g.gelu_tab) + g.pos[(size_t)t * g.ldc + col];
                    break;
                }
                case FW_EPI_QKV: {
                    // head-major split outputs: Q, K as [B, H, T, 64]; V as [B, H, 64, Tp]
                    int d = g.ldc, which = col / d, cc = col % d, h = cc >> 6, dd = cc & 63;
                    int b = row / g.T, t = row % g.T;
                    size_t bh = (size_t)b * g.H + h;
                    uint16_t hi, lo;
                    fw_split(v, hi, lo);
                    if (which < 2) {
                        size_t o = (bh * g.T + t) * 64 + dd;
                        g.o16[2 * which][o] = hi;
                        g.o16[2 * which + 1][o] = lo;
                    } else {
                        size_t o = (bh * 64 + dd) * g.Tp + t;
                        g.o16[4][o] = hi;
                        g.o16[5][o] = lo;
                    }
                    break;
                }
                default: break;
                }
            }
        }
}

// ---------------------------------------------------------------------------
// LayerNorm per row (nn.rs:4455-4545, f64 statistics) with the output the next
// GEMM consumes: mode F32 (ln_post), SPLIT (f16 hi/lo pair for the f32 path),
// I7 (quantize_act_i7, nn.rs:1443-1466: per-row amax/127, add-trunc body /
// exact tail, stored as the signed value q = u8 - 128).
#define FW_LN_MAXV 8
__global__ void __launch_bounds__(256) k_enc_ln(const float *x, const float *w, const float *b, int d, int mode,
                                                float *yf, uint16_t *hi, uint16_t *lo, int8_t *q, float *qs) {
    __shared__ double shd[4];
    __shared__ float shf[4];
    size_t r = blockIdx.x;
    const float *xr = x + r * d;
    float xv[FW_LN_MAXV];
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < FW_LN_MAXV; k++) {
        int i = threadIdx.x + k * 256;
        xv[k] = i < d ? xr[i] : 0.0f;
        if (i < d) s += (double)xv[k];
    }
    double mean = fw_block_sum(s, shd) / (double)d;
    double v = 0.0;
#pragma unroll
    for (int k = 0; k < FW_LN_MAXV; k++) {
        int i = threadIdx.x + k * 256;
        if (i < d) {
            double t = (double)xv[k] - mean;
            v += t * t;
        }
    }
    double var = fw_block_sum(v, shd) / (double)d;
    double inv = 1.0 / sqrt(var + (double)1e-5f);
    float yv[FW_LN_MAXV];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < FW_LN_MAXV; k++) {
        int i = threadIdx.x + k * 256;
        if (i < d) {
            double nrm = ((double)xv[k] - mean) * inv;
            yv[k] = (float)(nrm * (double)w[i] + (double)b[i]);
            amax = fmaxf(amax, fabsf(yv[k]));
        }
    }
    if (mode == FW_LN_F32) {
#pragma unroll
        for (int k = 0; k < FW_LN_MAXV; k++) {
            int i = threadIdx.x + k * 256;
            if (i < d) yf[r * d + i] = yv[k];
        }
    } else if (mode == FW_LN_SPLIT) {
#pragma unroll
        for (int k = 0; k < FW_LN_MAXV; k++) {
            int i = threadIdx.x + k * 256;
            if (i < d) fw_split(yv[k], hi[r * d + i], lo[r * d + i]);
        }
    } else {
        amax = fw_block_max(amax, shf);
        float sc = fmaxf(amax, 1e-9f) / 127.0f;
        float iv = 1.0f / sc;
#pragma unroll
        for (int k = 0; k < FW_LN_MAXV; k++) {
            int i = threadIdx.x + k * 256;
            if (i < d) q[r * d + i] = fw_q8_avx(yv[k], iv, i, d);
        }
        if (threadIdx.x == 0) qs[r] = sc;
    }
}

// Per-row exact-rounding i8 quantization of the attention output
// (matmul_bias_i8's quant_row_i8, encoder.rs:2468-2508, 2536-2551).
__global__ void __launch_bounds__(256) k_quant_exact_rows(const float *x, int n, int8_t *q, float *qs) {
    __shared__ float shf[4];
    size_t r = blockIdx.x;
    const float *xr = x + r * n;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, fabsf(xr[i]));
    m = fw_block_max(m, shf);
    float sc = fmaxf(m, 1e-9f) / 127.0f;
    float inv = 1.0f / sc;
    for (int i = threadIdx.x; i < n; i += 256)
        q[r * n + i] = (int8_t)(int)fw_clamp(fw_round_away(xr[i] * inv), -127.0f, 127.0f);
    if (threadIdx.x == 0) qs[r] = sc;
}

// quantize_act_i7_gelu (nn.rs:1791-1823): GELU (skipped when gelu_tab is
// NULL: quantize_act_i7, nn.rs:1443-1466), per-row amax/127, add-trunc body /
// exact tail, signed storage.
__global__ void __launch_bounds__(256) k_gelu_quant_i7_rows(const float *x, int n, const float *gelu_tab, int8_t *q,
                                                            float *qs) {
    __shared__ float shf[4];
    size_t r = blockIdx.x;
    const float *xr = x + r * n;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += 256) m = fmaxf(m, fabsf(gelu_tab ? fw_gelu(xr[i], gelu_tab) : xr[i]));
    m = fw_block_max(m, shf);
    float sc = fmaxf(m, 1e-9f) / 127.0f;
    float inv = 1.0f / sc;
    for (int i = threadIdx.x; i < n; i += 256)
        q[r * n + i] = fw_q8_avx(gelu_tab ? fw_gelu(xr[i], gelu_tab) : xr[i], inv, i, n);
    if (threadIdx.x == 0) qs[r] = sc;
}

// im2col for conv1d (kernel 3, pad 1; conv1d_wt nn.rs:5006-5103) into the f16
// pair the GEMM consumes.  Column order kk*Cin + ci (weights are reordered to
// match at load); columns >= 3*Cin are zero padding up to Kp.
__global__ void k_im2col(const float *x, int B, int Tin, int Cin, int stride, int Tout, int Kp, uint16_t *hi,
                         uint16_t *lo) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)B * Tout * Kp;
    if (idx >= total) return;
    int col = (int)(idx % Kp);
    size_t row = idx / Kp;
    int b = (int)(row / Tout), t = (int)(row % Tout);
    float v = 0.0f;
    if (col < 3 * Cin) {
        int kk = col / Cin, ci = col % Cin;
        int ti = t * stride + kk - 1;
        if (ti >= 0 && ti < Tin) v = x[((size_t)b * Tin + ti) * Cin + ci];
    }
    fw_split(v, hi[idx], lo[idx]);
}

// time_major_mel_window_from_full_mel (encoder.rs:684-714) for a batch of windows.
__global__ void k_mel_window(const float *mel, int n_mel, long long mel_frames, const long long *offs, int n_frames,
                             float *out, int B) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t total = (size_t)B * n_frames * n_mel;
    if (idx >= total) return;
    int m = (int)(idx % n_mel);
    size_t rf = idx / n_mel;
    int f = (int)(rf % n_frames), b = (int)(rf / n_frames);
    long long off = offs[b];
    long long avail = mel_frames - off;
    if (avail < 0) avail = 0;
    long long copy = avail < n_frames ? avail : n_frames;
    float fill = copy == n_frames ? 0.0f : -1.5f;
    out[idx] = f < copy ? mel[(size_t)m * mel_frames + off + f] : fill;
}

__global__ void k_fill_u16(uint16_t *p, size_t n, uint16_t v) {
    size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// ---------------------------------------------------------------------------
// Bidirectional attention, one block per (window b, head h, 128 queries):
// 4 waves x 32 queries.  Computes S^T = K Q^T per 64-key tile (A = K rows from
// LDS, B = this wave's Q^T held in registers) so each lane owns one query and
// the softmax max/sum over keys is in-register plus one cross-half shuffle; then
// O^T += V^T P^T with P^T taken straight from the S^T accumulators (their key
// order is matched by reading V^T in the same permuted order).  f16 pairs with
// three MFMAs per product (hh + hl + lh); scores scaled by 1/8 = 64^-0.5 (the
// SDPA scale, nn.rs:5867); online softmax in f32.
__global__ void __launch_bounds__(256) k_attention(const uint16_t *qh, const uint16_t *ql, const uint16_t *kh,
                                                   const uint16_t *kl, const uint16_t *vth, const uint16_t *vtl,
                                                   int T, int Tp, int H, int d, int out_mode, float *of,
                                                   uint16_t *oh, uint16_t *ol) {
    __shared__ __align__(16) uint16_t sK[2][64][72];  // [hi/lo][key][dim] (+pad)
    __shared__ __align__(16) uint16_t sV[2][64][72];  // [hi/lo][dim][key]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = blockIdx.y, b = blockIdx.z;
    const int q0 = blockIdx.x * 128 + wave * 32;
    const int myq = q0 + (lane & 31);
    const size_t bh = (size_t)b * H + h;
    // this lane's Q^T fragments: q = myq, dims (l/32)*8 + ks*16 .. +8, ks = 0..3
    v8h qfh[4], qfl[4];
#pragma unroll
    for (int ks = 0; ks < 4; ks++) {
        int dd = ks * 16 + (lane >> 5) * 8;
        if (myq < T) {
            qfh[ks] = *(const v8h *)(qh + (bh * T + myq) * 64 + dd);
            qfl[ks] = *(const v8h *)(ql + (bh * T + myq) * 64 + dd);
        } else {
#pragma unroll
            for (int e = 0; e < 8; e++) {
                qfh[ks][e] = (_Float16)0.0f;
                qfl[ks][e] = (_Float16)0.0f;
            }
        }
    }
    v16f o[2];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) o[j][r] = 0.0f;
    float m = -INFINITY, l = 0.0f;
    const float sl2 = 0.125f * 1.4426950408889634f;
    for (int k0 = 0; k0 < T; k0 += 64) {
        __syncthreads();
        // load K tile [64 keys][64 dims] and V^T tile [64 dims][64 keys] (hi, lo)
        for (int c = threadIdx.x; c < 2 * 64 * 8; c += 256) {
            int a = c >> 9, rr = (c >> 3) & 63, cc = c & 7;
            int key = k0 + rr;
            const uint16_t *ks_ = a ? kl : kh;
            int4 kv = key < T ? *(const int4 *)(ks_ + (bh * T + key) * 64 + cc * 8) : make_int4(0, 0, 0, 0);
            *(int4 *)&sK[a][rr][cc * 8] = kv;
            const uint16_t *vs_ = a ? vtl : vth;
            *(int4 *)&sV[a][rr][cc * 8] = *(const int4 *)(vs_ + (bh * 64 + rr) * Tp + k0 + cc * 8);
        }
        __syncthreads();
        // S^T tiles: keys 32t .. 32t+31 x this wave's 32 queries
        v16f st[2];
#pragma unroll
        for (int t = 0; t < 2; t++) {
#pragma unroll
            for (int r = 0; r < 16; r++) st[t][r] = 0.0f;
#pragma unroll
            for (int ks = 0; ks < 4; ks++) {
                int key = t * 32 + (lane & 31), dd = ks * 16 + (lane >> 5) * 8;
                v8h ah = *(const v8h *)&sK[0][key][dd];
                v8h al = *(const v8h *)&sK[1][key][dd];
                st[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qfh[ks], st[t], 0, 0, 0);
                st[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah, qfl[ks], st[t], 0, 0, 0);
                st[t] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al, qfh[ks], st[t], 0, 0, 0);
            }
        }
        // online softmax over this tile's keys for query myq
        float tmax = -INFINITY;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                int key = k0 + t * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                float s = key < T ? st[t][r] : -INFINITY;
                st[t][r] = s;
                tmax = fmaxf(tmax, s);
            }
        tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
        float mnew = fmaxf(m, tmax);
        float alpha = __builtin_amdgcn_exp2f((m - mnew) * sl2);
        float psum = 0.0f;
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                float p = __builtin_amdgcn_exp2f((st[t][r] - mnew) * sl2);
                st[t][r] = p;
                psum += p;
            }
        psum += __shfl_xor(psum, 32, 64);
        l = l * alpha + psum;
        m = mnew;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[j][r] *= alpha;
        // O^T[dim][q] += V^T[dim][key] P^T[key][q]; key substep (t, u) uses
        // accumulator regs 8u..8u+7 of S^T tile t: keys 32t+16u + (l/32)*4 + {0..3, 8..11}
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                v8h ph, pl;
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    float p = st[t][8 * u + e];
                    _Float16 hh = (_Float16)p;
                    ph[e] = hh;
                    pl[e] = (_Float16)(p - (float)hh);
                }
                int kb = t * 32 + u * 16 + (lane >> 5) * 4;
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    int dim = j * 32 + (lane & 31);
                    v8h vh, vl;
                    uint2 a0 = *(const uint2 *)&sV[0][dim][kb];
                    uint2 a1 = *(const uint2 *)&sV[0][dim][kb + 8];
                    uint2 b0 = *(const uint2 *)&sV[1][dim][kb];
                    uint2 b1 = *(const uint2 *)&sV[1][dim][kb + 8];
                    uint4 va = make_uint4(a0.x, a0.y, a1.x, a1.y), vb = make_uint4(b0.x, b0.y, b1.x, b1.y);
                    vh = __builtin_bit_cast(v8h, va);
                    vl = __builtin_bit_cast(v8h, vb);
                    o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, ph, o[j], 0, 0, 0);
                    o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh, pl, o[j], 0, 0, 0);
                    o[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl, ph, o[j], 0, 0, 0);
                }
            }
    }
    if (myq >= T) return;
    float inv = 1.0f / l;
    size_t orow = ((size_t)b * T + myq) * d + (size_t)h * 64;
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            int dim = j * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
            float v = o[j][r] * inv;
            if (out_mode == 0) of[orow + dim] = v;
            else fw_split(v, oh[orow + dim], ol[orow + dim]);
        }
}

// ---------------------------------------------------------------------------
// Exact mode: the reference's strict-parity arithmetic for the f32 parts of the
// encoder, for bit-exact parity checks (not the performance path).

// im2col in the reference column order ci*3 + kk (conv1d_wt, nn.rs:5060-5075).
__global__ void k_im2col_f32(const float *x, int B, int Tin, int Cin, int stride, int Tout, float *out) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t K = (size_t)3 * Cin, total = (size_t)B * Tout * K;
    if (idx >= total) return;
    int col = (int)(idx % K);
    size_t row = idx / K;
    int b = (int)(row / Tout), t = (int)(row % Tout);
    int ci = col / 3, kk = col % 3;
    int ti = t * stride + kk - 1;
    out[idx] = (ti >= 0 && ti < Tin) ? x[((size_t)b * Tin + ti) * Cin + ci] : 0.0f;
}

// Per-head attention of attention_raw (FW_ATTN_NO_SDPA=1, nn.rs:6035-6131):
// scores[i][j] = sum_d (q[i,d]*s) * (k[j,d]*s) in ascending d (strict matmul),
// s = 64^-0.25.  q, k, v rows of width ld starting at column offsets.
__global__ void k_attn_scores_exact(const float *qkv, int ld, int qoff, int koff, int T, int H, float scale,
                                    float *S) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    size_t TT = (size_t)T * T;
    int bh = blockIdx.y;
    if (idx >= TT) return;
    int b = bh / H, h = bh % H;
    int i = (int)(idx / T), j = (int)(idx % T);
    const float *q = qkv + ((size_t)b * T + i) * ld + qoff + h * 64;
    const float *k = qkv + ((size_t)b * T + j) * ld + koff + h * 64;
    float acc = 0.0f;
    for (int dd = 0; dd < 64; dd++) acc += (q[dd] * scale) * (k[dd] * scale);
    S[(size_t)bh * TT + idx] = acc;
}

// softmax_rows (nn.rs:4880-4963): max, glibc-exact expf, sequential sum, *= 1/sum.
__global__ void k_softmax_rows_exact(float *S, size_t rows, int n) {
    size_t r = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= rows) return;
    float *row = S + r * n;
    float mx = -INFINITY;
    for (int j = 0; j < n; j++) mx = fmaxf(mx, row[j]);
    if (!isfinite(mx)) return;
    float sum = 0.0f;
    for (int j = 0; j < n; j++) {
        float e = fw_expf(row[j] - mx);
        e = isfinite(e) ? e : 0.0f;
        row[j] = e;
        sum += e;
    }
    if (sum > 0.0f) {
        float inv = 1.0f / sum;
        for (int j = 0; j < n; j++) row[j] = row[j] * inv;
    }
}

// out[i, h*64+dd] = sum_j P[i][j] * v[j, dd] in ascending j (strict matmul).
__global__ void k_attn_pv_exact(const float *S, const float *qkv, int ld, int voff, int T, int H, int d, float *out) {
    size_t idx = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    int bh = blockIdx.y;
    if (idx >= (size_t)T * 64) return;
    int b = bh / H, h = bh % H;
    int i = (int)(idx / 64), dd = (int)(idx % 64);
    const float *p = S + ((size_t)bh * T + i) * T;
    const float *v = qkv + (size_t)b * T * ld + voff + h * 64 + dd;
    float acc = 0.0f;
    for (int j = 0; j < T; j++) acc += p[j] * v[(size_t)j * ld];
    out[((size_t)b * T + i) * d + h * 64 + dd] = acc;
}

void fw_launch_im2col_f32(hipStream_t st, const float *x, int B, int Tin, int Cin, int stride, int Tout, float *out) {
    size_t total = (size_t)B * Tout * 3 * Cin;
    hipLaunchKernelGGL(k_im2col_f32, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, B, Tin, Cin, stride,
                       Tout, out);
}
void fw_launch_attention_exact(hipStream_t st, const float *qkv, int ld, int qoff, int koff, int voff, int B, int T,
                               int H, int d, float *S, float *out) {
    float scale = powf(64.0f, -0.25f);
    size_t TT = (size_t)T * T;
    hipLaunchKernelGGL(k_attn_scores_exact, dim3((unsigned)((TT + 255) / 256), B * H), dim3(256), 0, st, qkv, ld,
                       qoff, koff, T, H, scale, S);
    size_t rows = (size_t)B * H * T;
    hipLaunchKernelGGL(k_softmax_rows_exact, dim3((unsigned)((rows + 63) / 64)), dim3(64), 0, st, S, rows, T);
    hipLaunchKernelGGL(k_attn_pv_exact, dim3((unsigned)(((size_t)T * 64 + 255) / 256), B * H), dim3(256), 0, st, S, qkv,
                       ld, voff, T, H, d, out);
}

// ---------------------------------------------------------------------------
void fw_launch_gemm(hipStream_t st, int kind, const FwGemm &g) {
    dim3 grid((g.N + 127) / 128, (g.M + 127) / 128);
    if (kind == FW_KIND_I8) hipLaunchKernelGGL(k_gemm<FW_KIND_I8>, grid, dim3(256), 0, st, g);
    else hipLaunchKernelGGL(k_gemm<FW_KIND_F16S>, grid, dim3(256), 0, st, g);
}
void fw_launch_enc_ln(hipStream_t st, const float *x, const float *w, const float *b, int rows, int d, int mode,
                      float *yf, uint16_t *hi, uint16_t *lo, int8_t *q, float *qs) {
    hipLaunchKernelGGL(k_enc_ln, dim3(rows), dim3(256), 0, st, x, w, b, d, mode, yf, hi, lo, q, qs);
}
void fw_launch_quant_exact_rows(hipStream_t st, const float *x, int rows, int n, int8_t *q, float *qs) {
    hipLaunchKernelGGL(k_quant_exact_rows, dim3(rows), dim3(256), 0, st, x, n, q, qs);
}
void fw_launch_gelu_quant_i7_rows(hipStream_t st, const float *x, int rows, int n, const float *tab, int8_t *q,
                                  float *qs) {
    hipLaunchKernelGGL(k_gelu_quant_i7_rows, dim3(rows), dim3(256), 0, st, x, n, tab, q, qs);
}
void fw_launch_im2col(hipStream_t st, const float *x, int B, int Tin, int Cin, int stride, int Tout, int Kp,
                      uint16_t *hi, uint16_t *lo) {
    size_t total = (size_t)B * Tout * Kp;
    hipLaunchKernelGGL(k_im2col, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, B, Tin, Cin, stride,
                       Tout, Kp, hi, lo);
}
void fw_launch_mel_window(hipStream_t st, const float *mel, int n_mel, long long mel_frames, const long long *offs,
                          int n_frames, float *out, int B) {
    size_t total = (size_t)B * n_frames * n_mel;
    hipLaunchKernelGGL(k_mel_window, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, mel, n_mel, mel_frames,
                       offs, n_frames, out, B);
}
void fw_launch_fill_u16(hipStream_t st, uint16_t *p, size_t n, uint16_t v) {
    hipLaunchKernelGGL(k_fill_u16, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, p, n, v);
}
void fw_launch_attention(hipStream_t st, const uint16_t *qh, const uint16_t *ql, const uint16_t *kh,
                         const uint16_t *kl, const uint16_t *vth, const uint16_t *vtl, int B, int T, int Tp, int H,
                         int d, int out_mode, float *of, uint16_t *oh, uint16_t *ol) {
    dim3 grid((T + 127) / 128, H, B);
    hipLaunchKernelGGL(k_attention, grid, dim3(256), 0, st, qh, ql, kh, kl, vth, vtl, T, Tp, H, d, out_mode, of, oh,
                       ol);
}
