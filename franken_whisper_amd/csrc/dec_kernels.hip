// dec_kernels.hip — decoder-step kernels for gfx950.
//
// The decoder step is HBM-bound GEMV work (~1 FLOP/byte).  Every kernel here
// reproduces the reference's per-output reduction order wherever that order
// feeds a floating-point rounding, so the int8 arm is bit-exact against the
// reference CPU path and the f16 arm reproduces dot_f16c's lane tree:
//  - int8 GEMVs: exact integer dot (v_dot4_i32_i8), reference epilogue
//    ((f32)acc * s_w) * s_x + b (nn.rs:3187-3188), activation quantized in the
//    kernel prologue exactly as quantize_act_i8_into (nn.rs:3020-3064);
//  - f16 GEMVs: dot_f16c's 4x8 FMA accumulators and fixed add tree
//    (nn.rs:1983-2051) mapped onto 4 lanes per output row;
//  - block-int8 GEMV: dot_i8w_f32 per 32-block then the sequential block fold
//    (nn.rs:3501-3564, 3756-3824);
//  - attention: per-key ascending-d dots, softmax with glibc-exact expf and a
//    sequential sum (nn.rs:4880-4963), per-output ascending-j accumulation
//    (nn.rs:6466-6540);
//  - LayerNorm in f64 (nn.rs:4386-4545) with a tree reduction (the one
//    documented deviation: f64 sums of f32 inputs are exact except below
//    2^-53 relative, where tree and sequential order may differ).
#include "fw_kernels.h"

#define LN_EPS_F 1e-5f

// ---------------------------------------------------------------------------
// embed_tokens (decoder.rs:1323-1385): x = f16(E[tok]) + P[pos]
__global__ void k_embed(const int32_t *tok, const int *posp, const uint16_t *emb, const float *pemb,
                        float *x, int d) {
    int s = blockIdx.x;
    int pos = *posp;
    const uint16_t *er = emb + (size_t)tok[s] * d;
    const float *pr = pemb + (size_t)pos * d;
    for (int i = threadIdx.x; i < d; i += blockDim.x) x[(size_t)s * d + i] = fw_h2f(er[i]) + pr[i];
}

// LayerNorm of one row per block (nn.rs:4455-4545): f64 mean/var, eps as f64
// of the f32 1e-5, ((x-mean)*inv)*w + b rounded to f32.
__global__ void k_layernorm(const float *x, float *y, const float *w, const float *b, int d) {
    __shared__ double sh[16];
    int r = blockIdx.x;
    const float *xr = x + (size_t)r * d;
    float *yr = y + (size_t)r * d;
    double s = 0.0;
    for (int i = threadIdx.x; i < d; i += blockDim.x) s += (double)xr[i];
    double mean = fw_block_sum(s, sh) / (double)d;
    double v = 0.0;
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        double t = (double)xr[i] - mean;
        v += t * t;
    }
    double var = fw_block_sum(v, sh) / (double)d;
    double inv = 1.0 / sqrt(var + (double)LN_EPS_F);
    for (int i = threadIdx.x; i < d; i += blockDim.x) {
        double nrm = ((double)xr[i] - mean) * inv;
        yr[i] = (float)(nrm * (double)w[i] + (double)b[i]);
    }
}

// ---------------------------------------------------------------------------
// int8 GEMV for S streams sharing one weight read (gemv_i8 nn.rs:3168-3231 per
// stream; gemv_i8_cohort nn.rs:3389-3477 is bit-identical per row).
// W [N,K] i8 row-major, sw [N], x [S,K] f32 (quantized here), y [S,ldy].
// mode: 0 store, 1 residual add (x += y, decoder.rs:2369), 2 GELU (nn.rs:4603).
// Block = 256 threads = 4 waves; 16 lanes per row; 16 rows per block.
template <int MAXS>
__global__ void __launch_bounds__(256) k_gemv_i8(const int8_t *__restrict__ W, const float *__restrict__ sw,
                                                 const float *__restrict__ bias, const float *__restrict__ x,
                                                 float *y, int N, int K, int ns, int ldy, int mode,
                                                 const float *__restrict__ gelu_tab) {
    extern __shared__ __align__(16) unsigned char smem[];
    int8_t *xq = (int8_t *)smem;                      // [MAXS][K]
    float *xs = (float *)(smem + MAXS * K);            // [MAXS]
    __shared__ float red[4];
    // prologue: per-stream activation quantization (identical in every block)
    for (int s = 0; s < ns; s++) {
        const float *xr = x + (size_t)s * K;
        float m = 0.0f;
        for (int i = threadIdx.x; i < K; i += 256) m = fmaxf(m, fabsf(xr[i]));
        m = fw_block_max(m, red);
        float sc = fmaxf(m, 1e-9f) / 127.0f;
        float inv = 1.0f / sc;
        for (int i = threadIdx.x; i < K; i += 256) xq[s * K + i] = fw_q8_avx(xr[i], inv, i, K);
        if (threadIdx.x == 0) xs[s] = sc;
        __syncthreads();
    }
    int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int sub = lane & 15;
    int row = blockIdx.x * 16 + wave * 4 + (lane >> 4);
    bool ok = row < N;
    int acc[MAXS];
#pragma unroll
    for (int s = 0; s < MAXS; s++) acc[s] = 0;
    int nch = K >> 4; // 16-byte chunks
    const int4 *wr = (const int4 *)(W + (size_t)(ok ? row : 0) * K);
    for (int c = sub; c < nch; c += 16) {
        int4 wv = ok ? wr[c] : make_int4(0, 0, 0, 0);
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            if (s < ns) {
                int4 xv = *(const int4 *)(xq + s * K + c * 16);
                int a = acc[s];
                a = fw_sdot4(wv.x, xv.x, a);
                a = fw_sdot4(wv.y, xv.y, a);
                a = fw_sdot4(wv.z, xv.z, a);
                a = fw_sdot4(wv.w, xv.w, a);
                acc[s] = a;
            }
        }
    }
#pragma unroll
    for (int s = 0; s < MAXS; s++) {
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) acc[s] += __shfl_xor(acc[s], o, 64);
    }
    if (ok) {
        float swr = sw[row];
        float b = bias ? bias[row] : 0.0f;
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            if (s < ns && s == sub) {
                float v = (float)acc[s] * swr * xs[s] + b;
                float *yp = y + (size_t)s * ldy + row;
                if (mode == 1) *yp = *yp + v;
                else if (mode == 2) *yp = fw_gelu(v, gelu_tab);
                else *yp = v;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// f16 GEMV in dot_f16c order (nn.rs:1983-2051), S streams per weight read.
// Lane j (0..3) of a 4-lane group owns accumulator vector a_j (8 lanes of the
// AVX register); chunk c covers elements [32c, 32c+32).
// Block = 256 threads; 64 rows per block.
template <int MAXS>
__global__ void __launch_bounds__(256) k_gemv_f16(const uint16_t *__restrict__ W, const float *__restrict__ bias,
                                                  const float *__restrict__ x, float *y, int N, int K, int ns,
                                                  int ldy, int mode, const float *__restrict__ gelu_tab) {
    int j = threadIdx.x & 3;
    int row = blockIdx.x * 64 + (threadIdx.x >> 2);
    bool ok = row < N;
    const uint16_t *wr = W + (size_t)(ok ? row : 0) * K;
    float a[MAXS][8];
#pragma unroll
    for (int s = 0; s < MAXS; s++)
#pragma unroll
        for (int l = 0; l < 8; l++) a[s][l] = 0.0f;
    int nc = K >> 5;
    for (int c = 0; c < nc; c++) {
        int off = c * 32 + j * 8;
        uint4 wv = ok ? *(const uint4 *)(wr + off) : make_uint4(0, 0, 0, 0);
        float wf[8];
        wf[0] = fw_h2f(wv.x & 0xffff); wf[1] = fw_h2f(wv.x >> 16);
        wf[2] = fw_h2f(wv.y & 0xffff); wf[3] = fw_h2f(wv.y >> 16);
        wf[4] = fw_h2f(wv.z & 0xffff); wf[5] = fw_h2f(wv.z >> 16);
        wf[6] = fw_h2f(wv.w & 0xffff); wf[7] = fw_h2f(wv.w >> 16);
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            if (s < ns) {
                const float4 *xp = (const float4 *)(x + (size_t)s * K + off);
                float4 x0 = xp[0], x1 = xp[1];
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

// ---------------------------------------------------------------------------
// Block-int8-weight x f32-activation GEMV (gemv_i8w_f32a_blocked,
// nn.rs:3756-3824) with block 32: one row per 64-thread block, 16 blocks per
// iteration (lane = 4*g + j), block dots in dot_i8w_f32's tree, then the
// sequential fold acc += dot_b * scale_b by lane s for stream s.
template <int MAXS>
__global__ void __launch_bounds__(64) k_gemv_blk(const int8_t *__restrict__ W, const float *__restrict__ sc,
                                                 const float *__restrict__ bias, const float *__restrict__ x,
                                                 float *y, int N, int K, int ns, int ldy, int mode) {
    __shared__ float part[MAXS][16];
    int lane = threadIdx.x, g = lane >> 2, j = lane & 3;
    int row = blockIdx.x;
    int nb = K >> 5;
    const int8_t *wr = W + (size_t)row * K;
    const float *sr = sc + (size_t)row * nb;
    float acc = 0.0f; // lane s < ns holds stream s's running fold
    for (int b0 = 0; b0 < nb; b0 += 16) {
        int b = b0 + g;
        bool okb = b < nb;
        int off = b * 32 + j * 8;
        int2 wv = okb ? *(const int2 *)(wr + off) : make_int2(0, 0);
        float wf[8];
#pragma unroll
        for (int l = 0; l < 4; l++) {
            wf[l] = (float)(int8_t)((wv.x >> (8 * l)) & 0xff);
            wf[4 + l] = (float)(int8_t)((wv.y >> (8 * l)) & 0xff);
        }
#pragma unroll
        for (int s = 0; s < MAXS; s++) {
            if (s < ns) {
                float t[8];
                if (okb) {
                    const float4 *xp = (const float4 *)(x + (size_t)s * K + off);
                    float4 x0 = xp[0], x1 = xp[1];
                    // _mm256_fmadd_ps(w, x, 0) of the single 32-wide chunk
                    t[0] = __builtin_fmaf(wf[0], x0.x, 0.0f); t[1] = __builtin_fmaf(wf[1], x0.y, 0.0f);
                    t[2] = __builtin_fmaf(wf[2], x0.z, 0.0f); t[3] = __builtin_fmaf(wf[3], x0.w, 0.0f);
                    t[4] = __builtin_fmaf(wf[4], x1.x, 0.0f); t[5] = __builtin_fmaf(wf[5], x1.y, 0.0f);
                    t[6] = __builtin_fmaf(wf[6], x1.z, 0.0f); t[7] = __builtin_fmaf(wf[7], x1.w, 0.0f);
                } else {
#pragma unroll
                    for (int l = 0; l < 8; l++) t[l] = 0.0f;
                }
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    float v = t[l];
                    v = v + __shfl_xor(v, 1, 64);
                    v = v + __shfl_xor(v, 2, 64);
                    t[l] = v;
                }
                float dsum = ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
                if (j == 0) part[s][g] = dsum;
            }
        }
        __syncthreads();
        if (lane < ns) {
            int gmax = nb - b0 < 16 ? nb - b0 : 16;
            for (int gg = 0; gg < gmax; gg++) acc = acc + part[lane][gg] * sr[b0 + gg];
        }
        __syncthreads();
    }
    if (lane < ns) {
        float v = acc + (bias ? bias[row] : 0.0f);
        float *yp = y + (size_t)lane * ldy + row;
        if (mode == 1) *yp = *yp + v;
        else *yp = v;
    }
}

// ---------------------------------------------------------------------------
// Self-attention over the f16 KV cache for one (head, stream), tq == 1
// (attention_with_cache nn.rs:6267-6337 -> KvCache::append nn.rs:5352 ->
// attention_decode_step_f16 nn.rs:6466-6540).  Appends this token's k/v (RNE
// to f16) at `pos` and attends over [0, pos].  64 threads.
__global__ void __launch_bounds__(64) k_self_attn(const float *qkv, uint16_t *kc, uint16_t *vc, float *att,
                                                  const int *posp, int d, int nctx, int L, int layer,
                                                  float scale) {
    extern __shared__ float sm[]; // [64 qh][64 knew][64 vnew][nctx scores]
    int pos = *posp;
    float *qh = sm, *kn = sm + 64, *vn = sm + 128, *sc = sm + 192;
    int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    int base = h * 64;
    const float *q = qkv + (size_t)s * 3 * d;
    size_t cbase = ((size_t)s * L + layer) * nctx * d;
    uint16_t kh = fw_f2h(q[d + base + t]), vh = fw_f2h(q[2 * d + base + t]);
    kc[cbase + (size_t)pos * d + base + t] = kh;
    vc[cbase + (size_t)pos * d + base + t] = vh;
    qh[t] = q[base + t] * scale;
    kn[t] = fw_h2f(kh);
    vn[t] = fw_h2f(vh);
    __syncthreads();
    int tk = pos + 1;
    float mx = -INFINITY;
    for (int jj = t; jj < tk; jj += 64) {
        float acc = 0.0f;
        if (jj == pos) {
            for (int i = 0; i < 64; i++) acc += qh[i] * (kn[i] * scale);
        } else {
            const uint4 *kr = (const uint4 *)(kc + cbase + (size_t)jj * d + base);
            for (int c = 0; c < 8; c++) {
                uint4 u = kr[c];
                uint32_t ww[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int e = 0; e < 4; e++) {
                    acc += qh[c * 8 + 2 * e] * (fw_h2f(ww[e] & 0xffff) * scale);
                    acc += qh[c * 8 + 2 * e + 1] * (fw_h2f(ww[e] >> 16) * scale);
                }
            }
        }
        sc[jj] = acc;
        mx = fmaxf(mx, acc);
    }
    mx = fw_wave_max(mx);
    bool fin = isfinite(mx);
    if (fin) {
        for (int jj = t; jj < tk; jj += 64) {
            float e = fw_expf(sc[jj] - mx);
            sc[jj] = isfinite(e) ? e : 0.0f;
        }
    }
    __syncthreads();
    __shared__ float inv_s;
    if (t == 0) {
        float sum = 0.0f;
        if (fin) for (int jj = 0; jj < tk; jj++) sum += sc[jj];
        inv_s = (fin && sum > 0.0f) ? 1.0f / sum : 0.0f;
        if (fin && !(sum > 0.0f)) inv_s = -1.0f; // leave as-is marker
    }
    __syncthreads();
    float inv = inv_s;
    if (fin && inv > 0.0f)
        for (int jj = t; jj < tk; jj += 64) sc[jj] = sc[jj] * inv;
    __syncthreads();
    float acc = 0.0f;
    for (int jj = 0; jj < tk; jj++) {
        float v = jj == pos ? vn[t] : fw_h2f(vc[cbase + (size_t)jj * d + base + t]);
        acc += sc[jj] * v;
    }
    att[(size_t)s * d + base + t] = acc;
}

// ---------------------------------------------------------------------------
// Cross-attention for one (head, stream), int8 K/V (cross_attention
// decoder.rs:1524-1716 with int8 cross K/V, the default): qh = q*s, quantized
// per vector; scores = gemv_i8(K_h, qh); softmax; p quantized per vector;
// out = gemv_i8(Vt_h, p).  256 threads; scores in LDS.
__global__ void __launch_bounds__(256) k_cross_attn_i8(const float *qc, const int8_t *ck, const float *cks,
                                                       const int8_t *cvt, const float *cvs, float *att,
                                                       int d, int T, int H, int L, int layer, float scale) {
    extern __shared__ __align__(16) unsigned char smc[];
    float *sc = (float *)smc;                       // [T]
    int8_t *p8 = (int8_t *)(smc + sizeof(float) * T); // [T] (padded)
    __shared__ float qh[64];
    __shared__ __align__(16) int8_t q8[64];
    __shared__ float red[4];
    __shared__ float bc[2];
    __shared__ int part[256];
    int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    size_t lh = ((size_t)s * L + layer) * H + h;
    const int8_t *K = ck + lh * (size_t)T * 64;
    const float *Ks = cks + lh * T;
    const int8_t *V = cvt + lh * (size_t)T * 64;
    const float *Vs = cvs + lh * 64;
    if (t < 64) qh[t] = qc[(size_t)s * d + h * 64 + t] * scale;
    __syncthreads();
    float m = t < 64 ? fabsf(qh[t]) : 0.0f;
    m = fw_block_max(m, red);
    float xs = fmaxf(m, 1e-9f) / 127.0f;
    float xinv = 1.0f / xs;
    if (t < 64) q8[t] = fw_q8_avx(qh[t], xinv, t, 64);
    __syncthreads();
    const int *qw = (const int *)q8;
    float mx = -INFINITY;
    for (int jj = t; jj < T; jj += 256) {
        const int4 *kr = (const int4 *)(K + (size_t)jj * 64);
        int acc = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            int4 kv = kr[c];
            acc = fw_sdot4(kv.x, qw[4 * c + 0], acc);
            acc = fw_sdot4(kv.y, qw[4 * c + 1], acc);
            acc = fw_sdot4(kv.z, qw[4 * c + 2], acc);
            acc = fw_sdot4(kv.w, qw[4 * c + 3], acc);
        }
        float v = (float)acc * Ks[jj] * xs + 0.0f;
        sc[jj] = v;
        mx = fmaxf(mx, v);
    }
    mx = fw_block_max(mx, red);
    bool fin = isfinite(mx);
    if (fin)
        for (int jj = t; jj < T; jj += 256) {
            float e = fw_expf(sc[jj] - mx);
            sc[jj] = isfinite(e) ? e : 0.0f;
        }
    __syncthreads();
    if (t == 0) {
        float sum = 0.0f;
        if (fin) for (int jj = 0; jj < T; jj++) sum += sc[jj];
        bc[0] = (fin && sum > 0.0f) ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    float inv = bc[0];
    float pm = 0.0f;
    for (int jj = t; jj < T; jj += 256) {
        float p = inv > 0.0f ? sc[jj] * inv : sc[jj];
        sc[jj] = p;
        pm = fmaxf(pm, fabsf(p));
    }
    pm = fw_block_max(pm, red);
    float ps = fmaxf(pm, 1e-9f) / 127.0f;
    float pinv = 1.0f / ps;
    for (int jj = t; jj < T; jj += 256) p8[jj] = fw_q8_avx(sc[jj], pinv, jj, T);
    for (int jj = T + t; jj < ((T + 15) & ~15); jj += 256) p8[jj] = 0;
    __syncthreads();
    // out[dd] = sum_j V[dd, j] * p8[j]: 4 threads per output, quarter ranges
    int dd = t >> 2, qq = t & 3;
    int nw = (T + 3) >> 2;          // 4-byte words per row (rows are T bytes)
    int per = (nw + 3) >> 2;
    int w0 = qq * per, w1 = min(nw, w0 + per);
    const int8_t *vr = V + (size_t)dd * T;
    int acc = 0;
    for (int wi = w0; wi < w1; wi++) {
        int jj = wi * 4;
        int vw;
        if (jj + 4 <= T && (((size_t)(vr + jj)) & 3) == 0) {
            vw = *(const int *)(vr + jj);
        } else {
            vw = 0;
            for (int e = 0; e < 4 && jj + e < T; e++) vw |= ((int)(uint8_t)vr[jj + e]) << (8 * e);
        }
        int pw = *(const int *)(p8 + jj);
        acc = fw_sdot4(vw, pw, acc);
    }
    part[t] = acc;
    __syncthreads();
    if (qq == 0) {
        int tot = part[t] + part[t + 1] + part[t + 2] + part[t + 3];
        att[(size_t)s * d + h * 64 + dd] = (float)tot * Vs[dd] * ps + 0.0f;
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
// Filtered first-index argmax (process_logits no-timestamps + argmax_idx,
// decode.rs:702-867, 1708-1790).  One block per stream.
__device__ __forceinline__ bool fw_masked(int i, const fwhip_filter &f, int initial) {
    if (initial && (i == f.eot || i == f.space_token)) return true;
    if (i >= f.timestamp_begin) return true;
    if (i == f.no_timestamps || i == f.sot || i == f.no_speech || i == f.solm || i == f.translate ||
        i == f.transcribe || i == f.sot_prev)
        return true;
    if (i >= f.sot + 1 && i <= f.sot + f.n_languages) return true;
    return false;
}

__global__ void __launch_bounds__(256) k_argmax(const float *logits, int V, fwhip_filter f, int use_filter,
                                                const int *initialp, int32_t *out) {
    __shared__ float bv[256];
    int initial = *initialp;
    __shared__ int bi[256];
    int s = blockIdx.x, t = threadIdx.x;
    const float *l = logits + (size_t)s * V;
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i = t; i < V; i += 256) {
        float v = l[i];
        if (use_filter && fw_masked(i, f, initial)) continue;
        if (v > best) { best = v; idx = i; }
    }
    bv[t] = best;
    bi[t] = idx;
    __syncthreads();
    for (int o = 128; o > 0; o >>= 1) {
        if (t < o) {
            float v2 = bv[t + o];
            int i2 = bi[t + o];
            if (v2 > bv[t] || (v2 == bv[t] && i2 < bi[t])) { bv[t] = v2; bi[t] = i2; }
        }
        __syncthreads();
    }
    if (t == 0) out[s] = bi[0] == 0x7fffffff ? 0 : bi[0];
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
#define FW_GEMV_DISPATCH(KER, MAXS_, ...)                                            \
    do {                                                                               \
        if (MAXS_ <= 1) hipLaunchKernelGGL(KER<1>, __VA_ARGS__);                     \
        else if (MAXS_ <= 4) hipLaunchKernelGGL(KER<4>, __VA_ARGS__);                \
        else if (MAXS_ <= 8) hipLaunchKernelGGL(KER<8>, __VA_ARGS__);                \
        else hipLaunchKernelGGL(KER<16>, __VA_ARGS__);                               \
    } while (0)

static int fw_round_maxs(int ns) { return ns <= 1 ? 1 : ns <= 4 ? 4 : ns <= 8 ? 8 : 16; }

void fw_launch_embed(hipStream_t st, const int32_t *tok, const int *posp, const uint16_t *emb,
                     const float *pemb, float *x, int d, int ns) {
    hipLaunchKernelGGL(k_embed, dim3(ns), dim3(256), 0, st, tok, posp, emb, pemb, x, d);
}

void fw_launch_layernorm(hipStream_t st, const float *x, float *y, const float *w, const float *b, int d,
                         int rows) {
    hipLaunchKernelGGL(k_layernorm, dim3(rows), dim3(256), 0, st, x, y, w, b, d);
}

void fw_launch_gemv_i8(hipStream_t st, const int8_t *W, const float *sw, const float *bias, const float *x,
                       float *y, int N, int K, int ns, int ldy, int mode, const float *gelu_tab) {
    for (int s0 = 0; s0 < ns; s0 += 16) {
        int n = ns - s0 < 16 ? ns - s0 : 16;
        int mx = fw_round_maxs(n);
        size_t shm = (size_t)mx * K + 16 * sizeof(float);
        FW_GEMV_DISPATCH(k_gemv_i8, mx, dim3((N + 15) / 16), dim3(256), shm, st, W, sw, bias,
                         x + (size_t)s0 * K, y + (size_t)s0 * ldy, N, K, n, ldy, mode, gelu_tab);
    }
}

void fw_launch_gemv_f16(hipStream_t st, const uint16_t *W, const float *bias, const float *x, float *y, int N,
                        int K, int ns, int ldy, int mode, const float *gelu_tab) {
    for (int s0 = 0; s0 < ns; s0 += 16) {
        int n = ns - s0 < 16 ? ns - s0 : 16;
        int mx = fw_round_maxs(n);
        FW_GEMV_DISPATCH(k_gemv_f16, mx, dim3((N + 63) / 64), dim3(256), 0, st, W, bias, x + (size_t)s0 * K,
                         y + (size_t)s0 * ldy, N, K, n, ldy, mode, gelu_tab);
    }
}

void fw_launch_gemv_blk(hipStream_t st, const int8_t *W, const float *sc, const float *bias, const float *x,
                        float *y, int N, int K, int ns, int ldy, int mode) {
    for (int s0 = 0; s0 < ns; s0 += 16) {
        int n = ns - s0 < 16 ? ns - s0 : 16;
        int mx = fw_round_maxs(n);
        FW_GEMV_DISPATCH(k_gemv_blk, mx, dim3(N), dim3(64), 0, st, W, sc, bias, x + (size_t)s0 * K,
                         y + (size_t)s0 * ldy, N, K, n, ldy, mode);
    }
}

void fw_launch_self_attn(hipStream_t st, const float *qkv, uint16_t *kc, uint16_t *vc, float *att,
                         const int *posp, int d, int H, int nctx, int L, int layer, int ns, float scale) {
    size_t shm = sizeof(float) * (192 + nctx);
    hipLaunchKernelGGL(k_self_attn, dim3(H, ns), dim3(64), shm, st, qkv, kc, vc, att, posp, d, nctx, L, layer,
                       scale);
}

void fw_launch_cross_attn_i8(hipStream_t st, const float *qc, const int8_t *ck, const float *cks,
                             const int8_t *cvt, const float *cvs, float *att, int d, int T, int H, int L,
                             int layer, int ns, float scale) {
    size_t shm = sizeof(float) * T + ((T + 15) & ~15) + 16;
    hipLaunchKernelGGL(k_cross_attn_i8, dim3(H, ns), dim3(256), shm, st, qc, ck, cks, cvt, cvs, att, d, T, H, L,
                       layer, scale);
}

void fw_launch_cross_attn_f16(hipStream_t st, const float *qc, const uint16_t *ck, const uint16_t *cvt,
                              float *att, int d, int T, int H, int L, int layer, int ns, float scale) {
    hipLaunchKernelGGL(k_cross_attn_f16, dim3(H, ns), dim3(256), sizeof(float) * T, st, qc, ck, cvt, att, d, T,
                       H, L, layer, scale);
}

void fw_launch_argmax(hipStream_t st, const float *logits, int V, const fwhip_filter *f, const int *initialp,
                      int32_t *out, int ns) {
    fwhip_filter ff;
    int use = f != nullptr;
    if (f) ff = *f;
    else memset(&ff, 0, sizeof ff);
    hipLaunchKernelGGL(k_argmax, dim3(ns), dim3(256), 0, st, logits, V, ff, use, initialp, out);
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
