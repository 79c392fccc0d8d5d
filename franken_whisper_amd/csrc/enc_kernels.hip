// enc_kernels.hip — encoder kernels for gfx950 other than the GEMM
// (enc_gemm.hip): LayerNorm/quantizer row kernels, im2col, attention.
//
// The f32 path carries activations as an f16 pair (hi, lo = f16(a - hi)) so
// that MFMA f16 products reproduce f32 products to within 2^-22 relative.
//
// MFMA operand layouts (gfx950): A lane l -> row l%32, k block (l/32)*8
// halves; B lane l -> col l%32, same k block; accumulator r of lane l -> row
// (r/4)*8 + (l/32)*4 + r%4, col l%32.
#include <cstdio>
#include <cstdlib>

#include "fw_enc.h"

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));

__device__ __forceinline__ void fw_split(float v, uint16_t &hi, uint16_t &lo) {
    asm volatile("" : "+v"(v));
    _Float16 h = (_Float16)v;
    float r = v - (float)h;
    asm volatile("" : "+v"(r));
    hi = __builtin_bit_cast(uint16_t, h);
    lo = __builtin_bit_cast(uint16_t, (_Float16)r);
}
// The same, or-ing into `of` whether the hi half overflows (|v| >= 65520).
__device__ __forceinline__ void fw_split(float v, uint16_t &hi, uint16_t &lo, uint32_t &of) {
    of |= fabsf(v) >= 65520.0f ? 1u : 0u;
    fw_split(v, hi, lo);
}

// ---------------------------------------------------------------------------
// LayerNorm per row (nn.rs:4455-4545, f64 statistics) with the output the next
// GEMM consumes: mode F32 (ln_post), SPLIT (f16 hi/lo pair for the f32 path),
// I7 (quantize_act_i7, nn.rs:1443-1466: per-row amax/127, add-trunc body /
// exact tail, stored as the signed value q = u8 - 128).  One wave per row (4
// rows per block), the row held in registers as NV float4s per lane (d <= 256
// NV, d % 4 == 0); every load is unconditional (clamped index) and issued
// before the first use: row, weight and bias together, so a row costs one
// memory round trip.
__device__ __forceinline__ double eln_wave_sum(double v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}
// With SEQ the row's mean and variance come from st [rows][2], the
// reference's sequential f64 loops (k_enc_ln_stats_seq); the wave's tree order
// differs from them in the last f64 bits, which the f32 result shows on rows
// of nearly equal values (silence).
template <int NV, bool SEQ>
__global__ void __launch_bounds__(256) k_enc_ln(const float *x, const float *w, const float *b, int rows, int d,
                                                int mode, float *yf, uint16_t *hi, uint16_t *lo, int8_t *q,
                                                float *qs, int *ovf, const double *st) {
    constexpr int ELN_V4 = NV;
    const int lane = threadIdx.x & 63;
    const size_t r = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= (size_t)rows) return;
    const int n4 = d >> 2; // float4 per row; lane owns float4 slots lane + 64k
    const float4 *xr = (const float4 *)(x + r * d);
    const float4 *wr = (const float4 *)w, *br = (const float4 *)b;
    float4 xv[ELN_V4], wv4[ELN_V4], bv4[ELN_V4];
    bool ok[ELN_V4];
#pragma unroll
    for (int k = 0; k < ELN_V4; k++) {
        const int c4 = lane + 64 * k;
        ok[k] = c4 < n4;
        xv[k] = xr[ok[k] ? c4 : 0];
    }
#pragma unroll
    for (int k = 0; k < ELN_V4; k++) {
        const int c4 = ok[k] ? lane + 64 * k : 0;
        wv4[k] = wr[c4];
        bv4[k] = br[c4];
    }
    double mean, var;
    if constexpr (SEQ) {
        mean = st[2 * r];
        var = st[2 * r + 1];
    } else {
        double s = 0.0;
#pragma unroll
        for (int k = 0; k < ELN_V4; k++)
            if (ok[k]) s += ((double)xv[k].x + (double)xv[k].y) + ((double)xv[k].z + (double)xv[k].w);
        mean = eln_wave_sum(s) / (double)d;
        double v = 0.0;
#pragma unroll
        for (int k = 0; k < ELN_V4; k++)
            if (ok[k]) {
                double t0 = (double)xv[k].x - mean, t1 = (double)xv[k].y - mean;
                double t2 = (double)xv[k].z - mean, t3 = (double)xv[k].w - mean;
                v += (t0 * t0 + t1 * t1) + (t2 * t2 + t3 * t3);
            }
        var = eln_wave_sum(v) / (double)d;
    }
    const double inv = 1.0 / sqrt(var + (double)1e-5f);
    float yv[ELN_V4][4];
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < ELN_V4; k++) {
        const float4 ww = wv4[k], bb = bv4[k];
        const float xs[4] = {xv[k].x, xv[k].y, xv[k].z, xv[k].w};
        const float wv[4] = {ww.x, ww.y, ww.z, ww.w}, bv[4] = {bb.x, bb.y, bb.z, bb.w};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            double nrm = ((double)xs[e] - mean) * inv;
            yv[k][e] = (float)(nrm * (double)wv[e] + (double)bv[e]);
            if (ok[k]) amax = fmaxf(amax, fabsf(yv[k][e]));
        }
    }
    if (mode == FW_LN_F32) {
#pragma unroll
        for (int k = 0; k < ELN_V4; k++)
            if (ok[k]) ((float4 *)(yf + r * d))[lane + 64 * k] = make_float4(yv[k][0], yv[k][1], yv[k][2], yv[k][3]);
    } else if (mode == FW_LN_SPLIT) {
        uint32_t of = 0;
#pragma unroll
        for (int k = 0; k < ELN_V4; k++)
            if (ok[k]) {
                uint16_t h[4], l[4];
#pragma unroll
                for (int e = 0; e < 4; e++) fw_split(yv[k][e], h[e], l[e], of);
                ((uint2 *)(hi + r * d))[lane + 64 * k] =
                    make_uint2(h[0] | ((uint32_t)h[1] << 16), h[2] | ((uint32_t)h[3] << 16));
                ((uint2 *)(lo + r * d))[lane + 64 * k] =
                    make_uint2(l[0] | ((uint32_t)l[1] << 16), l[2] | ((uint32_t)l[3] << 16));
            }
        if (of && ovf) *ovf = 1;
    } else {
        amax = fw_wave_max(amax);
        const float sc = fmaxf(amax, 1e-9f) / 127.0f;
        const float iv = 1.0f / sc;
#pragma unroll
        for (int k = 0; k < ELN_V4; k++)
            if (ok[k]) {
                const int i = (lane + 64 * k) * 4;
                uint32_t b0 = (uint8_t)fw_q8_avx(yv[k][0], iv, i, d), b1 = (uint8_t)fw_q8_avx(yv[k][1], iv, i + 1, d);
                uint32_t b2 = (uint8_t)fw_q8_avx(yv[k][2], iv, i + 2, d), b3 = (uint8_t)fw_q8_avx(yv[k][3], iv, i + 3, d);
                ((uint32_t *)(q + r * d))[lane + 64 * k] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            }
        if (lane == 0) qs[r] = sc;
    }
}

// The reference's sequential f64 LayerNorm statistics (nn.rs:4425-4438: the
// sum of (f64)x in index order, mean = sum / d, then the sum of
// ((f64)x - mean)^2 in index order, var = that / d) of 64 rows per block:
// 256-column chunks of the rows go through LDS (each of the 4 waves loads 16
// rows, one coalesced 256-byte run per row and load), and lane r of wave 0
// adds row r's chunk in index order, so one LDS read serves all 64 chains; the
// next chunk's loads are in flight while a chunk is added (double buffer).
// Two passes over the rows (the mean first).  st [rows][2] = mean, var.
#define LNS_CH 256
__global__ void __launch_bounds__(256) k_enc_ln_stats_seq(const float *x, int rows, int d, double *st) {
    __shared__ float xs[2][64][LNS_CH + 1];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const size_t r0 = (size_t)blockIdx.x * 64;
    const int nr = rows - r0 < 64 ? (int)(rows - r0) : 64;
    const int nch = (d + LNS_CH - 1) / LNS_CH;
    // thread t loads columns c0 + lane + 64 i (i < 4) of rows w + 4 k (k < 16)
    float v[16][4];
    auto load = [&](int c0) {
#pragma unroll
        for (int k = 0; k < 16; k++) {
            const int r = w + 4 * k;
            const float *row = x + (r0 + (r < nr ? r : 0)) * d;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int c = c0 + lane + 64 * i;
                v[k][i] = c < d ? row[c] : 0.0f;
            }
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int k = 0; k < 16; k++)
#pragma unroll
            for (int i = 0; i < 4; i++) xs[buf][w + 4 * k][lane + 64 * i] = v[k][i];
    };
    double mean = 0.0;
    for (int pass = 0; pass < 2; pass++) {
        double s = 0.0;
        load(0);
        for (int ch = 0; ch < nch; ch++) {
            const int buf = ch & 1, c0 = ch * LNS_CH;
            stash(buf);
            __syncthreads();
            if (ch + 1 < nch) load(c0 + LNS_CH);
            if (w == 0) {
                const float *xr = xs[buf][lane];
                const int cn = d - c0 < LNS_CH ? d - c0 : LNS_CH;
                int j = 0;
                // 16 values requested ahead of their 16 adds
                for (; j + 16 <= cn; j += 16) {
                    float e[16];
#pragma unroll
                    for (int u = 0; u < 16; u++) e[u] = xr[j + u];
                    if (pass == 0) {
#pragma unroll
                        for (int u = 0; u < 16; u++) s += (double)e[u];
                    } else {
#pragma unroll
                        for (int u = 0; u < 16; u++) {
                            const double dv = (double)e[u] - mean;
                            s += dv * dv;
                        }
                    }
                }
                for (; j < cn; j++) {
                    if (pass == 0) {
                        s += (double)xr[j];
                    } else {
                        const double dv = (double)xr[j] - mean;
                        s += dv * dv;
                    }
                }
            }
        }
        // wave 0 has added the last chunk before the next pass restages buffer 0
        __syncthreads();
        if (pass == 0) mean = s / (double)d;
        else if (w == 0 && lane < nr) {
            st[2 * (r0 + lane)] = mean;
            st[2 * (r0 + lane) + 1] = s / (double)d;
        }
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
// exact tail, signed storage.  One wave per row (4 rows per block); rows of up
// to 64 * 4 * GQ_V4 values (n % 4 == 0) are read once into registers with
// unconditional loads, longer rows take two passes.
#define GQ_V4 24
__global__ void __launch_bounds__(256) k_gelu_quant_i7_rows(const float *x, int rows, int n, const float *gelu_tab,
                                                            int8_t *q, float *qs) {
    const int lane = threadIdx.x & 63;
    const size_t r = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= (size_t)rows) return;
    const float *xr = x + r * n;
    const int n4 = n >> 2;
    if ((n & 3) == 0 && n4 <= 64 * GQ_V4) {
        float4 v[GQ_V4];
#pragma unroll
        for (int k = 0; k < GQ_V4; k++) {
            const int c4 = lane + 64 * k;
            v[k] = ((const float4 *)xr)[c4 < n4 ? c4 : 0];
        }
        // all table reads first (groups past the row hold clamped, valid
        // data), then the row max
        if (gelu_tab) {
#pragma unroll
            for (int k = 0; k < GQ_V4; k++) {
                v[k].x = fw_gelu(v[k].x, gelu_tab);
                v[k].y = fw_gelu(v[k].y, gelu_tab);
                v[k].z = fw_gelu(v[k].z, gelu_tab);
                v[k].w = fw_gelu(v[k].w, gelu_tab);
            }
        }
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < GQ_V4; k++)
            if (lane + 64 * k < n4)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v[k].x), fabsf(v[k].y)), fmaxf(fabsf(v[k].z), fabsf(v[k].w))));
        m = fw_dpp_wave_max(m);
        const float sc = fmaxf(m, 1e-9f) / 127.0f;
        const float inv = 1.0f / sc;
#pragma unroll
        for (int k = 0; k < GQ_V4; k++) {
            const int c4 = lane + 64 * k;
            if (c4 < n4) {
                const int i = c4 * 4;
                uint32_t b0 = (uint8_t)fw_q8_avx(v[k].x, inv, i, n), b1 = (uint8_t)fw_q8_avx(v[k].y, inv, i + 1, n);
                uint32_t b2 = (uint8_t)fw_q8_avx(v[k].z, inv, i + 2, n), b3 = (uint8_t)fw_q8_avx(v[k].w, inv, i + 3, n);
                ((uint32_t *)(q + r * n))[c4] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            }
        }
        if (lane == 0) qs[r] = sc;
        return;
    }
    float m = 0.0f;
    for (int i = lane; i < n; i += 64) m = fmaxf(m, fabsf(gelu_tab ? fw_gelu(xr[i], gelu_tab) : xr[i]));
    m = fw_wave_max(m);
    const float sc = fmaxf(m, 1e-9f) / 127.0f;
    const float inv = 1.0f / sc;
    for (int i = lane; i < n; i += 64) q[r * n + i] = fw_q8_avx(gelu_tab ? fw_gelu(xr[i], gelu_tab) : xr[i], inv, i, n);
    if (lane == 0) qs[r] = sc;
}

// The same quantization with one wave per row (4 rows per block) for rows of
// n % 4 == 0 values, n <= 256 * NV: lane l holds float4 groups l, l + 64, ...,
// all loads issued before the first use, a DPP max, and 4-byte stores.
template <int NV>
__global__ void __launch_bounds__(256) k_quant_exact_rows_w(const float *x, int rows, int n, int8_t *q, float *qs) {
    const int lane = threadIdx.x & 63;
    const size_t r = (size_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= (size_t)rows) return;
    const int n4 = n >> 2;
    const float4 *xr = (const float4 *)(x + r * n);
    float4 v[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) v[k] = xr[lane + 64 * k < n4 ? lane + 64 * k : 0];
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; k++)
        if (lane + 64 * k < n4) m = fmaxf(m, fmaxf(fmaxf(fabsf(v[k].x), fabsf(v[k].y)), fmaxf(fabsf(v[k].z), fabsf(v[k].w))));
    m = fw_dpp_wave_max(m);
    const float sc = fmaxf(m, 1e-9f) / 127.0f;
    const float inv = 1.0f / sc;
    auto qe = [&](float t) { return (uint32_t)(uint8_t)(int8_t)(int)fw_clamp(fw_round_away(t * inv), -127.0f, 127.0f); };
#pragma unroll
    for (int k = 0; k < NV; k++)
        if (lane + 64 * k < n4)
            ((uint32_t *)(q + r * n))[lane + 64 * k] =
                qe(v[k].x) | (qe(v[k].y) << 8) | (qe(v[k].z) << 16) | (qe(v[k].w) << 24);
    if (lane == 0) qs[r] = sc;
}

// GELU + quantize_act of fc1 rows (the same arithmetic as the kernel above)
// with the reference's f16-indexed GELU table held in LDS as f16 (its values
// are f16-rounded): 64K x 2 B = 128 KB, loaded once per block.  The grid is
// persistent (one block per CU, grid-stride over rows), one wave per row, NV4
// float4 groups per lane; rows of n % 8 == 0 values use the add-trunc rounding
// throughout.
#define GQ_TAB_N 65536
// The f16 GELU table into LDS: 16 bytes per thread and load, every load issued
// before the first store (blockDim.x == 1024).
__device__ __forceinline__ void fw_gtab_fill(uint16_t *gtab, const uint16_t *tab16) {
    const uint4 *s = (const uint4 *)tab16;
    uint4 *d = (uint4 *)gtab;
    uint4 v[GQ_TAB_N / 8 / 1024];
#pragma unroll
    for (int u = 0; u < GQ_TAB_N / 8 / 1024; u++) v[u] = s[threadIdx.x + u * 1024];
#pragma unroll
    for (int u = 0; u < GQ_TAB_N / 8 / 1024; u++) d[threadIdx.x + u * 1024] = v[u];
}
template <int NV4, bool FULL>
__global__ void __launch_bounds__(1024) k_gelu_quant_rows_lds(const float *x, int rows, int n, const uint16_t *tab16,
                                                             int8_t *q, float *qs) {
    extern __shared__ uint16_t gtab[]; // [65536]
    fw_gtab_fill(gtab, tab16);
    __syncthreads();
    const int lane = threadIdx.x & 63, wpb = blockDim.x >> 6;
    const int n4 = n >> 2;
    auto load = [&](float4 (&v)[NV4], int r) {
        const float4 *xr = (const float4 *)(x + (size_t)r * n);
#pragma unroll
        for (int k = 0; k < NV4; k++) {
            const int c4 = lane + 64 * k;
            v[k] = xr[c4 < n4 ? c4 : 0];
        }
    };
    auto row = [&](float4 (&v)[NV4], int r) {
        // a row with every |x| < 10 (the usual case, decided for the whole
        // wave) needs no clamp selects: GELU is the table value
        float ax = 0.0f;
#pragma unroll
        for (int k = 0; k < NV4; k++)
            if (FULL || lane + 64 * k < n4)
                ax = fmaxf(ax, fmaxf(fmaxf(fabsf(v[k].x), fabsf(v[k].y)), fmaxf(fabsf(v[k].z), fabsf(v[k].w))));
        const bool inner = fw_dpp_wave_max(ax) < 10.0f;
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < NV4; k++) {
            float *e = &v[k].x;
            if (inner) {
#pragma unroll
                for (int c = 0; c < 4; c++) e[c] = fw_h2f(gtab[fw_f2h(e[c])]);
            } else {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float a = e[c];
                    const float t = fw_h2f(gtab[fw_f2h(a)]);
                    e[c] = a <= -10.0f ? 0.0f : (a >= 10.0f ? a : t);
                }
            }
            if (FULL || lane + 64 * k < n4)
                m = fmaxf(m, fmaxf(fmaxf(fabsf(v[k].x), fabsf(v[k].y)), fmaxf(fabsf(v[k].z), fabsf(v[k].w))));
        }
        m = fw_dpp_wave_max(m);
        const float sc = fmaxf(m, 1e-9f) / 127.0f;
        const float inv = 1.0f / sc;
#pragma unroll
        for (int k = 0; k < NV4; k++) {
            const int c4 = lane + 64 * k;
            if (FULL || c4 < n4) {
                const uint32_t b0 = fw_q8_body(v[k].x, inv), b1 = fw_q8_body(v[k].y, inv);
                const uint32_t b2 = fw_q8_body(v[k].z, inv), b3 = fw_q8_body(v[k].w, inv);
                ((uint32_t *)(q + (size_t)r * n))[c4] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
            }
        }
        if (lane == 0) qs[r] = sc;
    };
    for (int r = blockIdx.x * wpb + (threadIdx.x >> 6); r < rows; r += gridDim.x * wpb) {
        float4 v[NV4];
        load(v, r);
        row(v, r);
    }
}

// The same GELU + quantization from rows of f16 table indices (the
// FW_EPI_F16IDX epilogue of the fc1 GEMM): an index h is the f16 rounding of
// an fc1 value v with |v| < FW_GIDX_LIM, whose GELU is the table entry
// gtab[h] (the clamp cases need |v| >= 10); the sentinel marks a value whose
// exact f32 sits at the same index of `side`, which takes the full
// clamp-or-table path.  Half the bytes of the f32 rows; the output is the same.
// One wave per row, persistent over rows; lane l holds the 8-index groups l,
// l + 64, ... (NV8 of them: n == 512 * NV8).
template <int NV8>
__global__ void __launch_bounds__(1024) k_gelu_quant_h16(const uint16_t *hx, const float *side, int rows, int n,
                                                        const uint16_t *tab16, int8_t *q, float *qs) {
    extern __shared__ uint16_t gtab[]; // [65536]
    fw_gtab_fill(gtab, tab16);
    __syncthreads();
    const int lane = threadIdx.x & 63, wpb = blockDim.x >> 6;
    for (int r = blockIdx.x * wpb + (threadIdx.x >> 6); r < rows; r += gridDim.x * wpb) {
        const uint4 *hr = (const uint4 *)(hx + (size_t)r * n);
        uint4 hv[NV8];
#pragma unroll
        for (int k = 0; k < NV8; k++) hv[k] = hr[lane + 64 * k];
        float g[NV8][8];
        bool sent = false;
#pragma unroll
        for (int k = 0; k < NV8; k++) {
            const uint32_t w[4] = {hv[k].x, hv[k].y, hv[k].z, hv[k].w};
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t lo = w[c] & 0xffffu, hi = w[c] >> 16;
                sent |= lo == FW_GIDX_SENT || hi == FW_GIDX_SENT;
                g[k][2 * c] = fw_h2f(gtab[lo]);
                g[k][2 * c + 1] = fw_h2f(gtab[hi]);
            }
        }
        if (__builtin_amdgcn_ballot_w64(sent)) {
            // rare: values with |v| >= FW_GIDX_LIM, read back exactly
#pragma unroll
            for (int k = 0; k < NV8; k++) {
                const uint32_t w[4] = {hv[k].x, hv[k].y, hv[k].z, hv[k].w};
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const uint32_t h = (w[e >> 1] >> (16 * (e & 1))) & 0xffffu;
                    if (h == FW_GIDX_SENT) {
                        const float a = side[(size_t)r * n + (lane + 64 * k) * 8 + e];
                        const float t = fw_h2f(gtab[fw_f2h(a)]);
                        g[k][e] = a <= -10.0f ? 0.0f : (a >= 10.0f ? a : t);
                    }
                }
            }
        }
        float m = 0.0f;
#pragma unroll
        for (int k = 0; k < NV8; k++)
#pragma unroll
            for (int e = 0; e < 8; e++) m = fmaxf(m, fabsf(g[k][e]));
        m = fw_dpp_wave_max(m);
        const float sc = fmaxf(m, 1e-9f) / 127.0f;
        const float inv = 1.0f / sc;
#pragma unroll
        for (int k = 0; k < NV8; k++) {
            uint32_t b[8];
#pragma unroll
            for (int e = 0; e < 8; e++) b[e] = fw_q8_body(g[k][e], inv);
            ((uint2 *)(q + (size_t)r * n))[lane + 64 * k] =
                make_uint2(b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24), b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24));
        }
        if (lane == 0) qs[r] = sc;
    }
}

// im2col for conv1d (kernel 3, pad 1; conv1d_wt nn.rs:5006-5103) into the f16
// pair the GEMM consumes.  Column order kk*Cin + ci (weights are reordered to
// match at load); columns >= 3*Cin are zero padding up to Kp.
__global__ void k_im2col(const float *x, int B, int Tin, int Cin, int stride, int Tout, int Kp, uint16_t *hi,
                         uint16_t *lo, int *ovf) {
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
    uint32_t of = 0;
    fw_split(v, hi[idx], lo[idx], of);
    if (of && ovf) *ovf = 1;
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
// Attention on f16 pairs (S^T = K Q^T, online softmax over 64-key tiles,
// O^T += V^T P^T), with 8 waves (256 queries) per block sharing each K/V tile, and the tiles (K hi/lo, V^T hi/lo:
// 4 x 8 KB) fed global -> LDS directly through an AT_NS-stage ring, one
// barrier per tile.  Rows are 128 bytes; 16-byte chunk c of row r sits at
// chunk c ^ (r & 7), which keeps the fragment reads free of bank conflicts.
// QPW 32-query sub-tiles per wave share each K / V^T fragment read from LDS
// (the fragment reads, not the MFMAs, set the LDS traffic per query), every
// query's arithmetic the same whatever QPW is.  Measured on MI355X (16
// large-v3-turbo windows, per launch): 8 waves x 2 sub-tiles with a 2-stage
// ring 550 us; 8 x 1 with 3 stages 620 us; 8 x 1 with 2 stages 608 us;
// 4 x 2 with 2 stages 601 us; 4 x 2 with 3 stages 724 us.
#ifndef AT_QW
#define AT_QW 8
#endif
#ifndef AT_NSTAGE
#define AT_NSTAGE 2
#endif
#ifndef AT_QPW
#define AT_QPW 2
#endif
template <int AT_QW_, int AT_NS, int QPW>
__global__ void __launch_bounds__(64 * AT_QW_, 2) k_attention2(const uint16_t *qh, const uint16_t *ql, const uint16_t *kh,
                                                           const uint16_t *kl, const uint16_t *vth, const uint16_t *vtl,
                                                           int T, int Tp, int H, int d, int out_mode, float *of,
                                                           uint16_t *oh, uint16_t *ol) {
    __shared__ __align__(1024) uint16_t sm[AT_NS][4][64 * 64]; // [stage][K hi, K lo, V^T hi, V^T lo][row][64]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int h = blockIdx.y, b = blockIdx.z;
    const size_t bh = (size_t)b * H + h;
    const int q0 = (blockIdx.x * AT_QW_ + wave) * 32 * QPW;
    const int nt = (T + 63) >> 6;
    // this lane's Q^T fragments: q = q0 + 32 qs + l % 32, dims ks*16 + (l/32)*8 .. +8
    v8h qfh[QPW][4], qfl[QPW][4];
#pragma unroll
    for (int qs = 0; qs < QPW; qs++) {
        const int myq = q0 + qs * 32 + (lane & 31);
        const int qc = myq < T ? myq : T - 1;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            const int dd = ks * 16 + (lane >> 5) * 8;
            v8h a = *(const v8h *)(qh + (bh * T + qc) * 64 + dd), c = *(const v8h *)(ql + (bh * T + qc) * 64 + dd);
#pragma unroll
            for (int e = 0; e < 8; e++) {
                qfh[qs][ks][e] = myq < T ? a[e] : (_Float16)0.0f;
                qfl[qs][ks][e] = myq < T ? c[e] : (_Float16)0.0f;
            }
        }
    }
    // loader: 32 instructions of 1 KB per tile, AT_QW_ waves share them
    constexpr int LPW = 32 / AT_QW_;
    const uint16_t *src[LPW];
    int dsto[LPW];
#pragma unroll
    for (int qq = 0; qq < LPW; qq++) {
        const int ii = wave * LPW + qq, arr = ii >> 3, r = ((ii & 7) << 3) + (lane >> 3);
        const int c = (lane & 7) ^ (r & 7);
        dsto[qq] = arr * 64 * 64 + ((ii & 7) << 3) * 64; // halves, wave-uniform
        if (arr < 2) src[qq] = (arr ? kl : kh) + (bh * T) * 64 + (size_t)r * 64 + c * 8;  // + key0*64 per tile
        else src[qq] = (arr == 3 ? vtl : vth) + (bh * 64 + r) * (size_t)Tp + c * 8;       // + key0 per tile
    }
    auto issue = [&](int it) {
        const int itc = it < nt ? it : nt - 1;
        const int k0 = itc * 64;
        uint16_t *base = &sm[it % AT_NS][0][0];
#pragma unroll
        for (int qq = 0; qq < LPW; qq++) {
            const int ii = wave * LPW + qq, arr = ii >> 3;
            const uint16_t *g;
            if (arr < 2) {
                // key rows past T reload row T-1 (masked in the softmax)
                const int r = ((ii & 7) << 3) + (lane >> 3);
                const int kr = k0 + r < T ? k0 : T - 1 - r;
                g = src[qq] + (size_t)kr * 64;
            } else {
                g = src[qq] + k0; // V^T rows are zero padded to Tp >= 64 * nt
            }
            __builtin_amdgcn_global_load_lds((const void *)g,
                                             (void __attribute__((address_space(3))) *)(base + dsto[qq]), 16, 0, 0);
        }
    };
    // Each accumulator takes all three f16-pair products in turn (hi*hi,
    // lo*hi, hi*lo); the two 32-key (or 32-dim) halves and the sub-tiles are
    // independent chains, interleaved so consecutive MFMAs never depend on
    // each other.
    v16f o[QPW][2];
    float m[QPW], l[QPW];
#pragma unroll
    for (int qs = 0; qs < QPW; qs++) {
        m[qs] = -INFINITY;
        l[qs] = 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) o[qs][j][r] = 0.0f;
    }
    const float sl2 = 0.125f * 1.4426950408889634f;
#pragma unroll
    for (int p = 0; p < AT_NS - 1; p++) issue(p);
    for (int it = 0; it < nt; it++) {
        FW_WAIT_VM_LGKM0(LPW * (AT_NS - 2)); // this wave's loads of tile `it` have landed
        asm volatile("s_barrier" ::: "memory");
        issue(it + AT_NS - 1);
        const uint16_t *sK = &sm[it % AT_NS][0][0];
        const int k0 = it * 64;
        // the first MFMA of each chain takes a zero accumulator operand
        const v16f zero = {};
        v16f st[QPW][2];
#pragma unroll
        for (int qs = 0; qs < QPW; qs++) st[qs][0] = st[qs][1] = zero;
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            v8h ah[2], al[2];
#pragma unroll
            for (int t = 0; t < 2; t++) {
                const int kr = t * 32 + (lane & 31), c = ks * 2 + (lane >> 5);
                const int off = kr * 64 + ((c ^ (kr & 7)) << 3);
                ah[t] = *(const v8h *)(sK + off);
                al[t] = *(const v8h *)(sK + 64 * 64 + off);
            }
#pragma unroll
            for (int qs = 0; qs < QPW; qs++) {
                st[qs][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0], qfh[qs][ks], st[qs][0], 0, 0, 0);
                st[qs][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1], qfh[qs][ks], st[qs][1], 0, 0, 0);
            }
#pragma unroll
            for (int qs = 0; qs < QPW; qs++) {
                st[qs][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[0], qfh[qs][ks], st[qs][0], 0, 0, 0);
                st[qs][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[1], qfh[qs][ks], st[qs][1], 0, 0, 0);
            }
#pragma unroll
            for (int qs = 0; qs < QPW; qs++) {
                st[qs][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0], qfl[qs][ks], st[qs][0], 0, 0, 0);
                st[qs][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1], qfl[qs][ks], st[qs][1], 0, 0, 0);
            }
        }
        // keys past T exist only in the last tile
        if (k0 + 64 > T) {
#pragma unroll
            for (int qs = 0; qs < QPW; qs++)
#pragma unroll
                for (int t = 0; t < 2; t++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int key = k0 + t * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                        if (key >= T) st[qs][t][r] = -INFINITY;
                    }
        }
#pragma unroll
        for (int qs = 0; qs < QPW; qs++) {
            float tmax = -INFINITY;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) tmax = fmaxf(tmax, st[qs][t][r]);
            tmax = fmaxf(tmax, __shfl_xor(tmax, 32, 64));
            const float mnew = fmaxf(m[qs], tmax);
            // exp2((s - mnew) * sl2) as one fma per score
            const float nms = -mnew * sl2;
            float psum = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; t++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(st[qs][t][r], sl2, nms));
                    st[qs][t][r] = pv;
                    psum += pv;
                }
            psum += __shfl_xor(psum, 32, 64);
            // rescale only when some row's running max moved (wave-uniform test)
            if (__builtin_amdgcn_ballot_w64(mnew != m[qs])) {
                const float alpha = __builtin_amdgcn_exp2f((m[qs] - mnew) * sl2);
                l[qs] *= alpha;
#pragma unroll
                for (int j = 0; j < 2; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) o[qs][j][r] *= alpha;
            }
            l[qs] += psum;
            m[qs] = mnew;
        }
        const uint16_t *sV = &sm[it % AT_NS][2][0];
#pragma unroll
        for (int t = 0; t < 2; t++)
#pragma unroll
            for (int u = 0; u < 2; u++) {
                // P holds keys {G + 4h + 0..3, G + 8 + 4h + 0..3} (G = 32t + 16u,
                // h = lane / 32); V^T stores each 16-key group with bits 2 and 3
                // of the key swapped, so these 8 keys are one 16-byte chunk
                const int c = t * 4 + u * 2 + (lane >> 5);
                v8h vh[2], vl[2];
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int dim = j * 32 + (lane & 31);
                    const int a = dim * 64 + ((c ^ (dim & 7)) << 3);
                    vh[j] = *(const v8h *)(sV + a);
                    vl[j] = *(const v8h *)(sV + 64 * 64 + a);
                }
#pragma unroll
                for (int qs = 0; qs < QPW; qs++) {
                    // f16 pair of P, two values per conversion
                    v8h ph, pl;
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        const v2f pv = {st[qs][t][8 * u + e], st[qs][t][8 * u + e + 1]};
                        const v2h hh = __builtin_convertvector(pv, v2h);
                        const v2h lo = __builtin_convertvector(pv - __builtin_convertvector(hh, v2f), v2h);
                        ph[e] = hh[0];
                        ph[e + 1] = hh[1];
                        pl[e] = lo[0];
                        pl[e + 1] = lo[1];
                    }
                    o[qs][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh[0], ph, o[qs][0], 0, 0, 0);
                    o[qs][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh[1], ph, o[qs][1], 0, 0, 0);
                    o[qs][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl[0], ph, o[qs][0], 0, 0, 0);
                    o[qs][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vl[1], ph, o[qs][1], 0, 0, 0);
                    o[qs][0] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh[0], pl, o[qs][0], 0, 0, 0);
                    o[qs][1] = __builtin_amdgcn_mfma_f32_32x32x16_f16(vh[1], pl, o[qs][1], 0, 0, 0);
                }
            }
    }
    FW_WAIT_VM(0); // dummy tiles landed before the block exits
#pragma unroll
    for (int qs = 0; qs < QPW; qs++) {
        const int myq = q0 + qs * 32 + (lane & 31);
        if (myq >= T) continue;
        const float inv = 1.0f / l[qs];
        const size_t orow = ((size_t)b * T + myq) * d + (size_t)h * 64;
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) {
                const int dim = j * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                const float v = o[qs][j][r] * inv;
                if (out_mode == 0) of[orow + dim] = v;
                else fw_split(v, oh[orow + dim], ol[orow + dim]);
            }
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

// Per-head attention of attention_raw (FW_ATTN_NO_SDPA=1, nn.rs:6035-6131),
// in three tiled launches whose every output keeps the reference's own
// operation sequence (only the scheduling is tiled):
//   scores[i][j] = sum_d (q[i,d]*s) * (k[j,d]*s) in ascending d (strict matmul),
//     s = 64^-0.25, each scaled operand rounded once as in the reference;
//   softmax_rows (nn.rs:4880-4963): max, glibc-exact expf, the sequential sum,
//     *= 1/sum (a row whose max is not finite is left as it is);
//   out[i, h*64+dd] = sum_j p[i][j] * v[j, dd] in ascending j (strict matmul).
// q, k, v rows of width ld at column offsets; S [B*H, T, T].

// 64 x 64 score tile of one (window, head): 256 threads, 4 x 4 outputs each.
// Also leaves each row's maximum over the tile's columns in pm[row][tile]
// (the max fold of softmax_rows ignores NaN and is order-free).
__global__ void __launch_bounds__(256) k_attn_scores_exact(const float *qkv, int ld, int qoff, int koff, int T, int H,
                                                           float scale, float *S, float *pm) {
    __shared__ float qs[64][65], ks[64][65];
    const int bh = blockIdx.z, b = bh / H, h = bh % H;
    const int i0 = blockIdx.y * 64, j0 = blockIdx.x * 64, t = threadIdx.x;
    // stage the scaled rows (rows past T read row T - 1; their results are dropped)
    for (int e = t; e < 64 * 64; e += 256) {
        const int r = e >> 6, c = e & 63;
        const int qi = min(i0 + r, T - 1), kj = min(j0 + r, T - 1);
        qs[r][c] = qkv[((size_t)b * T + qi) * ld + qoff + h * 64 + c] * scale;
        ks[r][c] = qkv[((size_t)b * T + kj) * ld + koff + h * 64 + c] * scale;
    }
    __syncthreads();
    const int ti = t >> 4, tj = t & 15; // rows ti + 16 a, columns tj + 16 c
    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[a][c] = 0.0f;
    for (int dd = 0; dd < 64; dd++) {
        float qv[4], kv[4];
#pragma unroll
        for (int a = 0; a < 4; a++) qv[a] = qs[ti + 16 * a][dd];
#pragma unroll
        for (int c = 0; c < 4; c++) kv[c] = ks[tj + 16 * c][dd];
#pragma unroll
        for (int a = 0; a < 4; a++)
#pragma unroll
            for (int c = 0; c < 4; c++) acc[a][c] += qv[a] * kv[c];
    }
    const size_t TT = (size_t)T * T;
    const int nt = gridDim.x;
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int i = i0 + ti + 16 * a;
        float m = -INFINITY;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int j = j0 + tj + 16 * c;
            if (j < T) m = fmaxf(m, acc[a][c]);
        }
        // the 16 lanes holding row i's columns
#pragma unroll
        for (int o = 8; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o, 16));
        if (i >= T) continue;
        if (tj == 0) pm[((size_t)bh * T + i) * nt + blockIdx.x] = m;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int j = j0 + tj + 16 * c;
            if (j < T) S[(size_t)bh * TT + (size_t)i * T + j] = acc[a][c];
        }
    }
}

// softmax_rows over 64 rows per block (4 waves).  Each row's max folds the
// score tiles' partial maxima pm; then 64-column chunks of the 64 rows go
// through LDS (double-buffered: the next chunk's loads are in flight while the
// current one is summed), each exp written back to S in place, and lane r of
// wave 0 adds row r's exps in index order.  The scaling p = e * (1 / sum) is
// left to the value pass, which multiplies each staged value by the row's
// factor sf: 1 / sum, or exactly 1.0 for a row softmax_rows leaves unscaled
// (a max that is not finite keeps the raw scores; a zero sum keeps the exps).
#define SMX_CH 64
__global__ void __launch_bounds__(256) k_softmax_rows_exact(float *S, const float *pm, int nt, size_t rows, int n,
                                                            float *sf) {
    __shared__ float ech[2][64][SMX_CH + 1];
    __shared__ float rmx[64];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const size_t r0 = (size_t)blockIdx.x * 64;
    const int nr = rows - r0 < 64 ? (int)(rows - r0) : 64;
    if (t < nr) {
        const float *p = pm + (r0 + t) * nt;
        float m = -INFINITY;
        for (int k = 0; k < nt; k++) m = fmaxf(m, p[k]);
        rmx[t] = m;
    }
    __syncthreads();
    // thread t stages column c0 + lane of rows w + 4 i
    float v[16];
    auto load = [&](int c0) {
        const int c = c0 + lane;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = w + 4 * i;
            v[i] = (r < nr && c < n) ? S[(r0 + r) * n + c] : 0.0f;
        }
    };
    auto stash = [&](int c0, int buf) {
        const int c = c0 + lane;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            const int r = w + 4 * i;
            if (r >= nr || c >= n) continue;
            const float m = rmx[r];
            if (!isfinite(m)) continue; // the row is left as it is
            float e = fw_expf(v[i] - m);
            e = isfinite(e) ? e : 0.0f;
            S[(r0 + r) * n + c] = e;
            ech[buf][r][lane] = e;
        }
    };
    const bool fin = w == 0 && lane < nr && isfinite(rmx[lane]);
    const int nch = (n + SMX_CH - 1) / SMX_CH;
    float sum = 0.0f;
    load(0);
    for (int ch = 0; ch < nch; ch++) {
        const int c0 = ch * SMX_CH, buf = ch & 1;
        stash(c0, buf);
        __syncthreads();
        if (ch + 1 < nch) load(c0 + SMX_CH);
        if (fin) {
            const int cn = n - c0 < SMX_CH ? n - c0 : SMX_CH;
            if (cn == SMX_CH) {
                float e[SMX_CH];
#pragma unroll
                for (int j = 0; j < SMX_CH; j++) e[j] = ech[buf][lane][j];
#pragma unroll
                for (int j = 0; j < SMX_CH; j++) sum += e[j];
            } else {
                for (int j = 0; j < cn; j++) sum += ech[buf][lane][j];
            }
        }
    }
    if (w == 0 && lane < nr) sf[r0 + lane] = (fin && sum > 0.0f) ? 1.0f / sum : 1.0f;
}

// 64 queries x 64 dims of one (window, head): 256 threads, 4 x 4 outputs
// each, keys in chunks of 32 through LDS in ascending order
__global__ void __launch_bounds__(256) k_attn_pv_exact(const float *S, const float *sf, const float *qkv, int ld,
                                                       int voff, int T, int H, int d, float *out) {
    __shared__ float ps[64][33], vs[32][65];
    const int bh = blockIdx.y, b = bh / H, h = bh % H;
    const int i0 = blockIdx.x * 64, t = threadIdx.x;
    const int ti = t >> 4, tj = t & 15; // queries ti + 16 a, dims tj + 16 c
    const float *P = S + (size_t)bh * T * T;
    float acc[4][4];
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[a][c] = 0.0f;
    for (int k0 = 0; k0 < T; k0 += 32) {
        const int kn = T - k0 < 32 ? T - k0 : 32;
        for (int e = t; e < 64 * 32; e += 256) {
            const int r = e >> 5, c = e & 31;
            const int qi = min(i0 + r, T - 1);
            ps[r][c] = c < kn ? P[(size_t)qi * T + k0 + c] * sf[(size_t)bh * T + qi] : 0.0f;
        }
        for (int e = t; e < 32 * 64; e += 256) {
            const int r = e >> 6, c = e & 63;
            vs[r][c] = r < kn ? qkv[((size_t)b * T + k0 + r) * ld + voff + h * 64 + c] : 0.0f;
        }
        __syncthreads();
        for (int j = 0; j < kn; j++) {
            float pv[4], vv[4];
#pragma unroll
            for (int a = 0; a < 4; a++) pv[a] = ps[ti + 16 * a][j];
#pragma unroll
            for (int c = 0; c < 4; c++) vv[c] = vs[j][tj + 16 * c];
#pragma unroll
            for (int a = 0; a < 4; a++)
#pragma unroll
                for (int c = 0; c < 4; c++) acc[a][c] += pv[a] * vv[c];
        }
        __syncthreads();
    }
#pragma unroll
    for (int a = 0; a < 4; a++) {
        const int i = i0 + ti + 16 * a;
        if (i >= T) continue;
#pragma unroll
        for (int c = 0; c < 4; c++) out[((size_t)b * T + i) * d + h * 64 + tj + 16 * c] = acc[a][c];
    }
}

void fw_launch_im2col_f32(hipStream_t st, const float *x, int B, int Tin, int Cin, int stride, int Tout, float *out) {
    size_t total = (size_t)B * Tout * 3 * Cin;
    hipLaunchKernelGGL(k_im2col_f32, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, B, Tin, Cin, stride,
                       Tout, out);
}
void fw_launch_attention_exact(hipStream_t st, const float *qkv, int ld, int qoff, int koff, int voff, int B, int T,
                               int H, int d, float *S, float *sf, float *out) {
    float scale = powf(64.0f, -0.25f);
    const unsigned nt = (unsigned)((T + 63) / 64);
    const size_t rows = (size_t)B * H * T;
    float *pm = sf + rows; // [rows][nt] partial maxima
    hipLaunchKernelGGL(k_attn_scores_exact, dim3(nt, nt, B * H), dim3(256), 0, st, qkv, ld, qoff, koff, T, H, scale,
                       S, pm);
    hipLaunchKernelGGL(k_softmax_rows_exact, dim3((unsigned)((rows + 63) / 64)), dim3(256), 0, st, S, pm, (int)nt,
                       rows, T, sf);
    hipLaunchKernelGGL(k_attn_pv_exact, dim3(nt, B * H), dim3(256), 0, st, S, sf, qkv, ld, voff, T, H, d, out);
}

// ---------------------------------------------------------------------------
void fw_launch_enc_ln(hipStream_t st, const float *x, const float *w, const float *b, int rows, int d, int mode,
                      float *yf, uint16_t *hi, uint16_t *lo, int8_t *q, float *qs, int *ovf, double *stats) {
    const dim3 g((rows + 3) / 4), blk(256);
    const bool seq = (mode & FW_LN_SEQ) != 0;
    mode &= ~FW_LN_SEQ;
    if (seq) {
        if (!stats) { // a caller's mistake in this library, never an input's
            fprintf(stderr, "fw_launch_enc_ln: FW_LN_SEQ without the statistics scratch\n");
            abort();
        }
        hipLaunchKernelGGL(k_enc_ln_stats_seq, dim3((rows + 63) / 64), dim3(256), 0, st, x, rows, d, stats);
    }
#define ELN_CASE(NV)                                                                                              \
    if (seq)                                                                                                    \
        hipLaunchKernelGGL((k_enc_ln<NV, true>), g, blk, 0, st, x, w, b, rows, d, mode, yf, hi, lo, q, qs, ovf,   \
                           (const double *)stats);                                                              \
    else hipLaunchKernelGGL((k_enc_ln<NV, false>), g, blk, 0, st, x, w, b, rows, d, mode, yf, hi, lo, q, qs, ovf,  \
                            (const double *)nullptr);                                                           \
    break;
    switch ((d + 255) / 256) {
    case 1: ELN_CASE(1)
    case 2: ELN_CASE(2)
    case 3: ELN_CASE(3)
    case 4: ELN_CASE(4)
    case 5: ELN_CASE(5)
    case 6: ELN_CASE(6)
    case 7: ELN_CASE(7)
    default: ELN_CASE(8)
    }
#undef ELN_CASE
}
void fw_launch_quant_exact_rows(hipStream_t st, const float *x, int rows, int n, int8_t *q, float *qs) {
    const dim3 g4((rows + 3) / 4), b4(256);
    if (n % 4 == 0 && n > 0) {
        switch ((n + 255) / 256) {
        case 1: hipLaunchKernelGGL(k_quant_exact_rows_w<1>, g4, b4, 0, st, x, rows, n, q, qs); return;
        case 2: hipLaunchKernelGGL(k_quant_exact_rows_w<2>, g4, b4, 0, st, x, rows, n, q, qs); return;
        case 3: hipLaunchKernelGGL(k_quant_exact_rows_w<3>, g4, b4, 0, st, x, rows, n, q, qs); return;
        case 4: hipLaunchKernelGGL(k_quant_exact_rows_w<4>, g4, b4, 0, st, x, rows, n, q, qs); return;
        case 5: hipLaunchKernelGGL(k_quant_exact_rows_w<5>, g4, b4, 0, st, x, rows, n, q, qs); return;
        case 6: hipLaunchKernelGGL(k_quant_exact_rows_w<6>, g4, b4, 0, st, x, rows, n, q, qs); return;
        case 7: hipLaunchKernelGGL(k_quant_exact_rows_w<7>, g4, b4, 0, st, x, rows, n, q, qs); return;
        case 8: hipLaunchKernelGGL(k_quant_exact_rows_w<8>, g4, b4, 0, st, x, rows, n, q, qs); return;
        default: break;
        }
    }
    hipLaunchKernelGGL(k_quant_exact_rows, dim3(rows), dim3(256), 0, st, x, n, q, qs);
}
void fw_launch_gelu_quant_i7_rows(hipStream_t st, const float *x, int rows, int n, const float *tab, int8_t *q,
                                  float *qs) {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    const size_t shm = sizeof(uint16_t) * GQ_TAB_N;
    const dim3 grid(n_cu), blk(1024);
    // the MLP widths of the Whisper sizes (4 x 384 ... 4 x 1280) are whole
    // multiples of 256: every lane's groups are in the row
    if (tab && (n & 255) == 0) {
        const uint16_t *t16 = fw_gelu_tab16(tab);
        switch (n / 256) {
        case 6: hipLaunchKernelGGL((k_gelu_quant_rows_lds<6, true>), grid, blk, shm, st, x, rows, n, t16, q, qs); return;
        case 8: hipLaunchKernelGGL((k_gelu_quant_rows_lds<8, true>), grid, blk, shm, st, x, rows, n, t16, q, qs); return;
        case 12:
            hipLaunchKernelGGL((k_gelu_quant_rows_lds<12, true>), grid, blk, shm, st, x, rows, n, t16, q, qs);
            return;
        case 16:
            hipLaunchKernelGGL((k_gelu_quant_rows_lds<16, true>), grid, blk, shm, st, x, rows, n, t16, q, qs);
            return;
        case 20:
            hipLaunchKernelGGL((k_gelu_quant_rows_lds<20, true>), grid, blk, shm, st, x, rows, n, t16, q, qs);
            return;
        default: break;
        }
    }
    hipLaunchKernelGGL(k_gelu_quant_i7_rows, dim3((rows + 3) / 4), dim3(256), 0, st, x, rows, n, tab, q, qs);
}
bool fw_launch_gelu_quant_h16(hipStream_t st, const uint16_t *hx, const float *side, int rows, int n,
                              const float *tab, int8_t *q, float *qs) {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    if (!tab || n <= 0 || n % 512) return false;
    const size_t shm = sizeof(uint16_t) * GQ_TAB_N;
    const dim3 grid(n_cu), blk(1024);
#define GQH(NV8)                                                                                                     \
    case NV8:                                                                                                        \
        hipLaunchKernelGGL((k_gelu_quant_h16<NV8>), grid, blk, shm, st, hx, side, rows, n, fw_gelu_tab16(tab), q, qs); \
        return true;
    switch (n / 512) {
        GQH(1)
        GQH(2)
        GQH(3)
        GQH(4)
        GQH(5)
        GQH(6)
        GQH(7)
        GQH(8)
        GQH(10)
        GQH(12)
        GQH(16)
    default: return false;
    }
#undef GQH
}
void fw_launch_im2col(hipStream_t st, const float *x, int B, int Tin, int Cin, int stride, int Tout, int Kp,
                      uint16_t *hi, uint16_t *lo, int *ovf) {
    size_t total = (size_t)B * Tout * Kp;
    hipLaunchKernelGGL(k_im2col, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, x, B, Tin, Cin, stride,
                       Tout, Kp, hi, lo, ovf);
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
    // the largest query tile whose launch still covers every CU (one window:
    // 20 heads x 12 blocks of 128 queries; ten: 20 x 10 x 3 of 512); every
    // tile gives the same bits
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    auto nblk = [&](int qb) { return (long long)B * H * ((T + qb - 1) / qb); };
#define AT_GO(QW_, QPW_)                                                                                           \
    hipLaunchKernelGGL((k_attention2<QW_, AT_NSTAGE, QPW_>), dim3((T + 32 * QW_ * QPW_ - 1) / (32 * QW_ * QPW_), H, B), \
                       dim3(64 * QW_), 0, st, qh, ql, kh, kl, vth, vtl, T, Tp, H, d, out_mode, of, oh, ol)
    if (nblk(32 * AT_QPW * AT_QW) >= n_cu) AT_GO(AT_QW, AT_QPW);
    else if (nblk(256) >= n_cu) AT_GO(8, 1);
    else AT_GO(4, 1);
#undef AT_GO
}
