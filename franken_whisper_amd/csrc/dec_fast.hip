// dec_fast.hip — the int8 decoder arm's per-token kernels (gfx950).
//
// Decode is HBM-bound: per step the cohort reads every weight once (161 MB
// int8 at large-v3-turbo) plus each stream's cross K/V (15.9 MB int8) and
// self-attention cache.  The kernels here keep the reference's arithmetic
// exactly (integer dots are exact in any order; every floating-point rounding
// is reproduced in the reference's order) while spreading the bytes over the
// whole chip:
//  - activations are quantized once per use (quantize_act_i8_into,
//    nn.rs:3020-3064) — in the LayerNorm kernel or a row kernel — instead of in
//    every GEMV block;
//  - int8 GEMVs run on v_mfma_i32_16x16x64_i8 with the cohort's (up to 16)
//    quantized activation rows as the A operand and 16 weight rows as B: one
//    16-byte weight load per lane per MFMA, K split over the block's 4 waves,
//    exact i32 partial sums added in LDS, then gemv_i8's epilogue
//    ((f32)acc * s_w) * s_x + b (nn.rs:3187-3188);
//  - the logits GEMV also emits per-block (value, index) argmax keys over the
//    filtered logits (process_logits no-timestamps masks, decode.rs:702-867;
//    first-index strict '>' argmax, decode.rs:1708-1780); a one-block kernel
//    finishes the argmax and the greedy bookkeeping on the device.
#include <cstdlib>

#include "fw_kernels.h"

typedef int v4i __attribute__((ext_vector_type(4)));

#include <type_traits>

#include "fw_dec.h"

template <int NV, bool SEQ>
__global__ void __launch_bounds__(256) k_ln_quant(const float *x, float *y, const float *w, const float *b, int d,
                                                  int rows, int8_t *xq, float *xs) {
    const int lane = threadIdx.x & 63;
    const int r = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int n4 = d >> 2;
    const float4 *xr = (const float4 *)(x + (size_t)r * d);
    float4 xv[NV];
    bool ok[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int i = lane + k * 64;
        ok[k] = i < n4;
        xv[k] = xr[ok[k] ? i : 0];
    }
    fw_ln_quant_vals<NV, SEQ>(xv, ok, y, w, b, d, r, xq, xs, lane);
}

// embed_tokens (decoder.rs:1323-1385: x = f16(E[tok]) + P[pos]) of one stream
// per block (one wave), followed, when w is given, by the first layer's
// attention LayerNorm of the row (into ln_y and/or the int8 activation rows,
// as k_ln_quant).
// Row s sits at position *posp + s / rps (rps: rows per position, the streams
// of a prefill chunk whose rows are [position][stream]).
template <int NV, bool SEQ>
__global__ void __launch_bounds__(64) k_embed_ln(const int32_t *tok, const int *posp, const uint16_t *emb,
                                                 const float *pemb, float *x, int d, const float *w, const float *b,
                                                 float *ln_y, int8_t *xq, float *xs, int rps) {
    const int s = blockIdx.x, lane = threadIdx.x;
    const int n4 = d >> 2;
    const uint2 *er = (const uint2 *)(emb + (size_t)tok[s] * d);
    const float4 *pr = (const float4 *)(pemb + (size_t)(*posp + s / rps) * d);
    float4 xv[NV];
    bool ok[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int i = lane + k * 64;
        ok[k] = i < n4;
        const int c = ok[k] ? i : 0;
        const uint2 e = er[c];
        const float4 p = pr[c];
        xv[k] = make_float4(fw_h2f(e.x & 0xffff) + p.x, fw_h2f(e.x >> 16) + p.y, fw_h2f(e.y & 0xffff) + p.z,
                            fw_h2f(e.y >> 16) + p.w);
        if (ok[k]) ((float4 *)(x + (size_t)s * d))[i] = xv[k];
    }
    if (w) fw_ln_quant_vals<NV, SEQ>(xv, ok, ln_y, w, b, d, s, xq, xs, lane);
}

// ---------------------------------------------------------------------------
// The same GEMV on weights repacked so each lane's share of a row is
// contiguous ("fragment order", fw_launch_pack_gemv_f16): lane q of the LPR
// lanes of a row owns lane-local elements li = c * CPL + e (chunk c, element e
// of its CPL), stored in 16-byte groups g = li / 8 at row offset
// (g * LPR + q) * 8 + li % 8.  Wave load g then reads LPR * 16 contiguous bytes
// of each of its rows, and a lane issues R = 8 groups per round, the next round
// in flight while the current one is used (a row of 1280 needs one round at 32
// lanes per row).  Needs K % (8 * LPR) == 0.
template <int LPR, int SG, bool LN>
__global__ void __launch_bounds__(256) k_gemv_f16f(const uint16_t *__restrict__ Wf, const float *__restrict__ bias,
                                                   const float *__restrict__ x, float *y, int N, int K, int ns,
                                                   int ldy, int mode, const float *__restrict__ gelu_tab, int cps,
                                                   int spb, const float *__restrict__ lnw,
                                                   const float *__restrict__ lnb) {
    constexpr int CPL = 32 / LPR, RPB = 256 / LPR, R = 8, CPG = 8 / CPL;
    extern __shared__ __align__(16) float xs[]; // [cps][SG][32]
    const int q = threadIdx.x % LPR;
    const int nc = K >> 5, G = K / (8 * LPR), nslab = (nc + cps - 1) / cps, ntile = (N + RPB - 1) / RPB;
    auto stage = [&](int s0, int sn, int c0, int cn) {
        const int n4 = cn * 8, tot = SG * n4;
        for (int b0 = 0; b0 < tot; b0 += 256 * 8) {
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
    // this block's streams [sb0, sb1), SG per pass; with lnw the staged rows are
    // LayerNorm(x) (k_ln_quant's arithmetic: one wave per row, whole rows of
    // K <= 1280 in one slab)
    const int sb0 = blockIdx.y * spb, sb1 = ns < sb0 + spb ? ns : sb0 + spb;
    auto stage_ln = [&](int s0, int sn) {
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, n4 = K >> 2;
        for (int sl = wave; sl < SG; sl += 4) {
            float4 xv[5];
            bool okk[5];
#pragma unroll
            for (int kk = 0; kk < 5; kk++) {
                const int i = lane + kk * 64;
                okk[kk] = i < n4;
                xv[kk] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (sl < sn) xv[kk] = ((const float4 *)(x + (size_t)(s0 + sl) * K))[okk[kk] ? i : 0];
            }
            if (sl < sn) fw_ln_quant_vals<5>(xv, okk, nullptr, lnw, lnb, K, 0, nullptr, nullptr, lane);
#pragma unroll
            for (int kk = 0; kk < 5; kk++) {
                if (okk[kk]) {
                    const int i = (lane + kk * 64) * 4;
                    *(float4 *)(xs + ((i >> 5) * SG + sl) * 32 + (i & 31)) =
                        sl < sn ? xv[kk] : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
            }
        }
    };
    for (int s0 = sb0; s0 < sb1; s0 += SG) {
        const int sn = sb1 - s0 < SG ? sb1 - s0 : SG;
        bool staged = false;
        for (int tile = blockIdx.x; tile < ntile; tile += gridDim.x) {
            const int row = tile * RPB + threadIdx.x / LPR;
            const bool ok = row < N;
            const uint4 *wl = (const uint4 *)(Wf + (size_t)(ok ? row : 0) * K) + q;
            float a[SG][CPL];
#pragma unroll
            for (int sl = 0; sl < SG; sl++)
#pragma unroll
                for (int e = 0; e < CPL; e++) a[sl][e] = 0.0f;
            for (int sb = 0; sb < nslab; sb++) {
                const int c0 = sb * cps, cn = nc - c0 < cps ? nc - c0 : cps;
                const int gs0 = c0 / CPG, gn = cn / CPG;
                uint4 nxt[R];
#pragma unroll
                for (int i = 0; i < R; i++) nxt[i] = wl[(size_t)(gs0 + i < G ? gs0 + i : G - 1) * LPR];
                if (nslab > 1 || !staged) {
                    __syncthreads();
                    if constexpr (LN) stage_ln(s0, sn);
                    else stage(s0, sn, c0, cn);
                    __syncthreads();
                    staged = true;
                }
                for (int gg = 0; gg < gn; gg += R) {
                    uint4 cur[R];
#pragma unroll
                    for (int i = 0; i < R; i++) {
                        cur[i] = nxt[i];
                        const int gx = gs0 + gg + R + i;
                        nxt[i] = wl[(size_t)(gx < G ? gx : G - 1) * LPR];
                    }
#pragma unroll
                    for (int i = 0; i < R; i++) {
                        if (gg + i < gn) {
                            const uint32_t u[4] = {cur[i].x, cur[i].y, cur[i].z, cur[i].w};
#pragma unroll
                            for (int cc = 0; cc < CPG; cc++) {
                                float wf[CPL];
#pragma unroll
                                for (int e = 0; e < CPL; e++) {
                                    const int f = cc * CPL + e;
                                    wf[e] = fw_h2f((uint16_t)(u[f >> 1] >> ((f & 1) * 16)));
                                }
                                const float *xc = xs + ((gg + i) * CPG + cc) * SG * 32 + q * CPL;
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
            }
#pragma unroll
            for (int sl = 0; sl < SG; sl++) {
                if (sl < sn) {
                    float t[CPL];
#pragma unroll
                    for (int e = 0; e < CPL; e++) {
                        float v = a[sl][e];
                        v = v + __shfl_xor(v, 8 / CPL, 64);
                        v = v + __shfl_xor(v, 16 / CPL, 64);
                        t[e] = v;
                    }
#pragma unroll
                    for (int w = 1; w < CPL; w <<= 1)
#pragma unroll
                        for (int e = 0; e < CPL; e += 2 * w) t[e] = t[e] + t[e + w];
                    float acc = t[0];
#pragma unroll
                    for (int m = 1; m < 8 / CPL; m <<= 1) acc = acc + __shfl_xor(acc, m, 64);
                    if (q == 0 && ok) {
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

int fw_gemv_f16_lpr(int N) { return N <= 2048 ? 32 : N <= 8192 ? 16 : 8; }
bool fw_gemv_f16_frag_ok(int N, int K) { return K > 0 && K % (8 * fw_gemv_f16_lpr(N)) == 0; }

__global__ void __launch_bounds__(256) k_pack_gemv_f16(const uint16_t *W, uint16_t *Wf, int N, int K, int LPR) {
    const int CPL = 32 / LPR;
    const size_t total = (size_t)N * K;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < total; i += (size_t)gridDim.x * 256) {
        const size_t r = i / K;
        const int k = (int)(i - r * K);
        const int c = k >> 5, within = k & 31, q = within / CPL, e = within % CPL;
        const int li = c * CPL + e;
        Wf[r * K + (size_t)((li >> 3) * LPR + q) * 8 + (li & 7)] = W[i];
    }
}

void fw_launch_pack_gemv_f16(hipStream_t st, const uint16_t *W, uint16_t *Wf, int N, int K) {
    const size_t total = (size_t)N * K;
    size_t g = (total + 255) / 256;
    g = g < 65536 ? g : 65536;
    hipLaunchKernelGGL(k_pack_gemv_f16, dim3((unsigned)g), dim3(256), 0, st, W, Wf, N, K, fw_gemv_f16_lpr(N));
}

// W in fragment order (fw_launch_pack_gemv_f16); K % (8 * lanes per row) == 0
void fw_launch_gemv_f16f(hipStream_t st, const uint16_t *Wf, const float *bias, const float *x, float *y, int N,
                         int K, int ns, int ldy, int mode, const float *gelu_tab, const float *lnw,
                         const float *lnb) {
    static int n_cu = 0;
    if (!n_cu) {
        int dev = 0;
        (void)hipGetDevice(&dev);
        if (hipDeviceGetAttribute(&n_cu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n_cu <= 0)
            n_cu = 256;
    }
    const int LPR = fw_gemv_f16_lpr(N), CPG = LPR / 4;
    const int nc = K >> 5;
    // streams per block: all of them when their rows fit the LDS budget in one
    // slab, else split over grid.y (fc2's 5120-wide rows)
    constexpr size_t LDS_BUDGET = 128 * 1024;
    int spb = ns < 16 ? ns : 16;
    while (spb > 1 && (size_t)spb * nc * 128 > LDS_BUDGET) spb = (spb + 1) / 2;
    const int nby = (ns + spb - 1) / spb;
    const int spass = spb > 12 ? 16 : spb > 10 ? 12 : spb > 8 ? 10 : spb > 5 ? 8 : spb > 4 ? 5 : spb > 2 ? 4 : spb;
    int cps = (int)(LDS_BUDGET / ((size_t)spass * 128));
    cps = cps / CPG * CPG; // whole weight groups per slab
    cps = cps < nc ? cps : nc;
    const size_t shm = sizeof(float) * (size_t)spass * cps * 32;
    const bool one = cps >= nc;
    if (lnw && (!one || K > 1280)) return; // LayerNorm staging needs the whole row (callers check)
#define GF_GO(LPR_, SG)                                                                                      \
    do {                                                                                                     \
        const int ntile = (N + 256 / LPR_ - 1) / (256 / LPR_);                                               \
        const int grid = one && ntile > 2 * n_cu ? 2 * n_cu : ntile;                                        \
        if (lnw)                                                                                            \
            hipLaunchKernelGGL((k_gemv_f16f<LPR_, SG, true>), dim3(grid, nby), dim3(256), shm, st, Wf, bias, x,   \
                               y, N, K, ns, ldy, mode, gelu_tab, cps, spb, lnw, lnb);                       \
        else                                                                                                \
            hipLaunchKernelGGL((k_gemv_f16f<LPR_, SG, false>), dim3(grid, nby), dim3(256), shm, st, Wf, bias, x,  \
                               y, N, K, ns, ldy, mode, gelu_tab, cps, spb, lnw, lnb);                       \
    } while (0)
#define GF_SG(LPR_)                      \
    do {                                 \
        switch (spass) {                 \
        case 1: GF_GO(LPR_, 1); break;   \
        case 2: GF_GO(LPR_, 2); break;   \
        case 4: GF_GO(LPR_, 4); break;   \
        case 5: GF_GO(LPR_, 5); break;   \
        case 8: GF_GO(LPR_, 8); break;   \
        case 10: GF_GO(LPR_, 10); break; \
        case 12: GF_GO(LPR_, 12); break; \
        default: GF_GO(LPR_, 16); break; \
        }                                \
    } while (0)
    if (LPR == 32) GF_SG(32);
    else if (LPR == 16) GF_SG(16);
    else GF_SG(8);
#undef GF_SG
#undef GF_GO
}


// ---------------------------------------------------------------------------
// int8 GEMV on MFMA.  W [N, K] i8 in fragment order (below), sw [N]; xq [16,
// K] i8 (rows >= ns are zero), xs [ns]; y [ns, ldy].  Block = 4 waves over
// 16*RG rows; wave w takes the 64-wide k blocks kb = w, w+4, ...
//
// Fragment order: the 16 x 64 operand of row group rg (rows 16*rg ..
// 16*rg+15) and k block kb is one contiguous KB at (rg * K/64 + kb) * 1024,
// lane l's 16 bytes (row 16*rg + l%16, columns kb*64 + (l/16)*16 ..) at l*16,
// so every wave load reads 8 whole 128-byte lines; rows past N (the last
// group) are zero.  Row-major rows put 16 half lines in each wave load
// (measured on the 51866 x 1280 logits: 21.6 us row-major, 15.8 us in
// fragment order, 12.6 us for a plain read of the same bytes).
// mode 0 store, 1 residual add (add_into, decoder.rs:2369), 2 GELU
// (nn.rs:4603), 3 logits: store + per-block argmax keys keys[s*nblk + block],
// 4 GELU stored in the block-interleaved order of the block GEMV's input.
#define GV_KPW 5 // k blocks per wave held in registers (K <= 1280 in one pass)
//
// XF = 1: the activations arrive as f32 rows xf [ns, K] together with per-head
// partial maxima pmax [ns, H] of |xf| (written by the attention kernel that
// produced them); the block forms each row's quantize_act_i8_into scale from
// the partial maxima and quantizes its own operand chunks, so no separate
// quantization pass over the rows is needed.
// 16 elements of a row whose length is a multiple of 8: all in the add-trunc
// body of the quantizer.
__device__ __forceinline__ v4i fw_q8_chunk16(const float4 (&v)[4], float iv) {
    v4i q;
#pragma unroll
    for (int c = 0; c < 4; c++)
        q[c] = (int)(fw_q8_body(v[c].x, iv) | (fw_q8_body(v[c].y, iv) << 8) | (fw_q8_body(v[c].z, iv) << 16) |
                     (fw_q8_body(v[c].w, iv) << 24));
    return q;
}
template <int RG, int XF>
__global__ void __launch_bounds__(256) k_gemv_i8m(const int8_t *__restrict__ W, const float *__restrict__ sw,
                                                  const float *__restrict__ bias, const int8_t *__restrict__ xq,
                                                  const float *__restrict__ xs, float *y, int N, int K, int ns,
                                                  int ldy, int mode, const float *__restrict__ gelu_tab,
                                                  fwhip_filter filt, int use_filter, const int *initialp,
                                                  unsigned long long *keys, const float *__restrict__ xf,
                                                  const float *__restrict__ pmax, int H) {
    static_assert(RG <= 4, "one row group per wave in the epilogue");
    __shared__ int red[4][RG * 4][64];
    __shared__ unsigned long long ksh[RG][16];
    __shared__ int smax[16];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int row_base = blockIdx.x * 16 * RG;
    const int nkb = K >> 6;
    const int ko = (lane >> 4) * 16;
    v4i acc[RG];
#pragma unroll
    for (int g = 0; g < RG; g++) acc[g] = (v4i){0, 0, 0, 0};
    const int8_t *xrow = xq + (size_t)(lane & 15) * K + ko;
    const int sa = lane & 15;
    const float *frow = xf + (size_t)(sa < ns ? sa : 0) * K + ko;
    // epilogue operands of the row group this wave finishes (g = wave < RG),
    // loaded now so their latency overlaps the operand loads and MFMAs
    const int ge = wave;
    const int erow = row_base + ge * 16 + (lane & 15);
    const bool eok = ge < RG && erow < N;
    const int erc = eok ? erow : 0;
    const float e_sw = sw[erc];
    const float e_b = bias ? bias[erc] : 0.0f;
    const int initial = (mode == 3 && use_filter) ? *initialp : 0;
    float e_xs[4], e_y[4];
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int s = (lane >> 4) * 4 + r;
        const int sc_ = s < ns ? s : 0;
        e_xs[r] = XF ? 0.0f : xs[sc_]; // XF: from the row scales below
        e_y[r] = mode == 1 ? y[(size_t)sc_ * ldy + erc] : 0.0f;
    }
    // XF: the head maxima are loaded first, so waiting for them does not wait
    // for the operand loads behind them (ns * H <= 512)
    float pm[2] = {0.0f, 0.0f};
    if (XF == 1) {
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int e = threadIdx.x + u * 256;
            pm[u] = pmax[e < ns * H ? e : 0];
        }
    }
    // weight fragments of this wave's k blocks kb = wave + 4*i, i < GV_KPW
    // (row groups past the last one clamped to it)
    const int ngrp = (N + 15) >> 4;
    const int8_t *wl = W + lane * 16;
    auto wfrag = [&](int g, int kb) -> const v4i * {
        const int rg = blockIdx.x * RG + g;
        return (const v4i *)(wl + ((size_t)(rg < ngrp ? rg : ngrp - 1) * nkb + kb) * 1024);
    };
    v4i xa[GV_KPW], wb[GV_KPW][RG];
#pragma unroll
    for (int i = 0; i < GV_KPW; i++) {
        const int kb = wave + 4 * i;
        const int kbc = kb < nkb ? kb : nkb - 1;
#pragma unroll
        for (int g = 0; g < RG; g++) wb[i][g] = *wfrag(g, kbc);
    }
    float4 xfv[XF == 1 ? GV_KPW : 1][4];
    if (XF == 1) {
        // operand chunks first (they are the long loads), then the row scales
#pragma unroll
        for (int i = 0; i < GV_KPW; i++) {
            const int kb = wave + 4 * i;
            const float4 *fp = (const float4 *)(frow + (kb < nkb ? kb : nkb - 1) * 64);
#pragma unroll
            for (int c = 0; c < 4; c++) xfv[i][c] = fp[c];
        }
        if (threadIdx.x < 16) smax[threadIdx.x] = 0;
        __syncthreads();
#pragma unroll
        for (int u = 0; u < 2; u++) {
            const int e = threadIdx.x + u * 256;
            // m >= 0, so int order is float order; NaN never wins (as fmaxf)
            if (e < ns * H && pm[u] == pm[u]) atomicMax(&smax[e / H], __float_as_int(pm[u]));
        }
        __syncthreads();
    }
    if (XF == 1) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int st_ = (lane >> 4) * 4 + r;
            e_xs[r] = fmaxf(__int_as_float(smax[st_ < ns ? st_ : 0]), 1e-9f) / 127.0f;
        }
    }
    const float a_iv = XF == 1 ? 1.0f / (fmaxf(__int_as_float(smax[sa]), 1e-9f) / 127.0f) : 0.0f;
    // activation operands (every operand load is issued before the first
    // MFMA; addresses clamped, unused blocks never multiplied)
#pragma unroll
    for (int i = 0; i < GV_KPW; i++) {
        const int kb = wave + 4 * i;
        const int kbc = kb < nkb ? kb : nkb - 1;
        if (XF == 1) {
            xa[i] = fw_q8_chunk16(xfv[i], a_iv);
            if (sa >= ns) xa[i] = (v4i){0, 0, 0, 0};
        } else {
            xa[i] = *(const v4i *)(xrow + kbc * 64);
        }
    }
#pragma unroll
    for (int i = 0; i < GV_KPW; i++) {
        if (wave + 4 * i < nkb) {
#pragma unroll
            for (int g = 0; g < RG; g++) acc[g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(xa[i], wb[i][g], acc[g], 0, 0, 0);
        }
    }
    // K beyond 4 * GV_KPW * 64
    for (int kb = wave + 4 * GV_KPW; kb < nkb; kb += 4) {
        v4i x1;
        if (XF == 1) {
            float4 v[4];
#pragma unroll
            for (int c = 0; c < 4; c++) v[c] = ((const float4 *)(frow + kb * 64))[c];
            x1 = sa < ns ? fw_q8_chunk16(v, a_iv) : (v4i){0, 0, 0, 0};
        } else {
            x1 = *(const v4i *)(xrow + kb * 64);
        }
#pragma unroll
        for (int g = 0; g < RG; g++) acc[g] = __builtin_amdgcn_mfma_i32_16x16x64_i8(x1, *wfrag(g, kb), acc[g], 0, 0, 0);
    }
#pragma unroll
    for (int g = 0; g < RG; g++)
#pragma unroll
        for (int r = 0; r < 4; r++) red[wave][g * 4 + r][lane] = acc[g][r];
    __syncthreads();
    if (ge < RG) {
        const int g = ge, row = erow;
        const bool okr = eok;
        const bool masked = mode == 3 && use_filter && okr && dec_masked(row, filt, initial);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int s = (lane >> 4) * 4 + r;
            const int tot = red[0][g * 4 + r][lane] + red[1][g * 4 + r][lane] + red[2][g * 4 + r][lane] +
                            red[3][g * 4 + r][lane];
            unsigned long long key = 0ull;
            if (okr && s < ns) {
                const float v = (float)tot * e_sw * e_xs[r] + e_b;
                float *yp = y + (size_t)s * ldy + (mode == 4 ? fw_blk_perm(row, ldy >> 5) : row);
                if (mode == 1) *yp = e_y[r] + v;
                else if (mode == 2 || mode == 4) *yp = fw_gelu(v, gelu_tab);
                else *yp = v;
                if (mode == 3 && !masked) key = am_key(v, row);
            }
            if (mode == 3) {
                // max over the 16 lanes holding stream s (same lane>>4)
                key = row16_max_u64(key);
                if ((lane & 15) == 0) ksh[g][s] = key;
            }
        }
    }
    if (mode != 3) return;
    __syncthreads();
    if (threadIdx.x < ns) {
        unsigned long long k = 0ull;
#pragma unroll
        for (int g = 0; g < RG; g++) k = ksh[g][threadIdx.x] > k ? ksh[g][threadIdx.x] : k;
        keys[(size_t)threadIdx.x * gridDim.x + blockIdx.x] = k;
    }
}

// Finish the argmax from the per-block keys and do the greedy bookkeeping:
// tok[s] = argmax, hist[s*cap + *stepp] = tok[s], advance the position, clear
// the first-step flag, advance the step counter.  One block of 16 waves, wave
// w reduces streams w, w+16, ...
__global__ void __launch_bounds__(1024) k_argmax_finish(const unsigned long long *keys, int nblk, int ns,
                                                        int32_t *tok, int32_t *hist, int hist_cap, int *posp,
                                                        int *initialp, int *stepp, int advance) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int step = stepp ? *stepp : 0;
    for (int s = wave; s < ns; s += 16) {
        const unsigned long long *ks = keys + (size_t)s * nblk;
        unsigned long long k = 0ull;
        int i = lane;
        for (; i + 192 < nblk; i += 256) {
            unsigned long long a0 = ks[i], a1 = ks[i + 64], a2 = ks[i + 128], a3 = ks[i + 192];
            a0 = a0 > a1 ? a0 : a1;
            a2 = a2 > a3 ? a2 : a3;
            a0 = a0 > a2 ? a0 : a2;
            k = a0 > k ? a0 : k;
        }
        for (; i < nblk; i += 64) k = ks[i] > k ? ks[i] : k;
        k = wave_max_u64(k);
        if (lane == 0) {
            int t = k ? (int)(0xffffffffu - (uint32_t)(k & 0xffffffffull)) : 0;
            tok[s] = t;
            if (hist) hist[(size_t)s * hist_cap + step] = t;
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        if (advance) *posp = *posp + 1;
        if (initialp) *initialp = 0;
        if (stepp) *stepp = step + 1;
    }
}

// ---------------------------------------------------------------------------
// Block-int8-weight x f32-activation GEMV with 32-wide blocks
// (gemv_i8w_f32a_blocked, nn.rs:3756-3824): for each (row, stream) the block
// dots dot_i8w_f32 (nn.rs:3501-3564; one 32-chunk: products, lane-wise
// (a0+a1)+(a2+a3), then ((t0+t1)+(t2+t3))+((t4+t5)+(t6+t7))) are folded in
// ascending block order, acc = acc + dot_b * s_b, then + bias.
//
// A block owns R consecutive rows (R = ceil(N / CUs): one block per CU).
// Thread c owns the (32-block b, stream group g) pair c = g * nb + b and holds
// the activation chunks x[g*SG .. g*SG+SG)[b*32 .. b*32+32) in registers for
// all R rows; per row it converts the weight chunk once and forms SG block
// dots, writing dot_b * s_b to LDS; one thread per (row, stream) then folds
// the products in ascending b.
//
// The activations arrive block-interleaved (fw_blk_perm: 16-byte chunk q of
// block b at chunk index q*nb + b, written so by the producing GEMV), so the
// q-th load of the lanes owning consecutive blocks reads consecutive 16-byte
// chunks; in natural order every wave load would touch 64 cache lines.
#define B7_RP 5
template <int SG>
__global__ void __launch_bounds__(512) k_gemv_blk7(const int8_t *__restrict__ W, const float *__restrict__ sc,
                                                   const float *__restrict__ bias, const float *__restrict__ x,
                                                   float *y, int N, int K, int ns, int ldy, int mode, int R) {
    extern __shared__ __align__(16) float b7_sm[]; // P[R][ns][ldp]
    const int nb = K >> 5, ldp = nb + 4;
    const int row0 = blockIdx.x * R;
    const int nr = N - row0 < R ? N - row0 : R;
    const int nsg = (ns + SG - 1) / SG, combos = nb * nsg;
    const int tid = threadIdx.x;
    if (tid < combos) {
        const int g = tid / nb, b = tid - g * nb;
        int4 wr[B7_RP][2];
        float sr[B7_RP];
        auto load_rows = [&](int rc) {
            const int nc = nr - rc < B7_RP ? nr - rc : B7_RP;
#pragma unroll
            for (int u = 0; u < B7_RP; u++) {
                const int row = row0 + rc + (u < nc ? u : nc - 1);
                const int4 *wq = (const int4 *)(W + (size_t)row * K + (size_t)b * 32);
                wr[u][0] = wq[0];
                wr[u][1] = wq[1];
                sr[u] = sc[(size_t)row * nb + b];
            }
        };
        load_rows(0);
        float xv[SG][32];
#pragma unroll
        for (int j = 0; j < SG; j++) {
            const int sj = g * SG + j < ns ? g * SG + j : ns - 1;
            const float4 *xp = (const float4 *)(x + (size_t)sj * K) + b;
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const float4 v = xp[(size_t)q * nb];
                xv[j][q * 4 + 0] = v.x;
                xv[j][q * 4 + 1] = v.y;
                xv[j][q * 4 + 2] = v.z;
                xv[j][q * 4 + 3] = v.w;
            }
        }
        for (int rc = 0; rc < nr; rc += B7_RP) {
            const int nc = nr - rc < B7_RP ? nr - rc : B7_RP;
            if (rc > 0) load_rows(rc);
#pragma unroll
            for (int u = 0; u < B7_RP; u++) {
                if (u < nc) {
                    const int r = rc + u;
                    const int wv[8] = {wr[u][0].x, wr[u][0].y, wr[u][0].z, wr[u][0].w,
                                       wr[u][1].x, wr[u][1].y, wr[u][1].z, wr[u][1].w};
                    // element q*4+e sits in accumulation lane (q%2)*4+e of
                    // group q/2
                    float tl[SG][8];
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        float wf[16]; // words h, h+2, h+4, h+6 -> lanes h*4 .. h*4+3
#pragma unroll
                        for (int gq = 0; gq < 4; gq++)
#pragma unroll
                            for (int e = 0; e < 4; e++)
                                wf[gq * 4 + e] = (float)(int8_t)((wv[gq * 2 + h] >> (8 * e)) & 0xff);
#pragma unroll
                        for (int j = 0; j < SG; j++)
#pragma unroll
                            for (int e = 0; e < 4; e++) {
                                const int l = h * 4 + e;
                                const float p0 = __builtin_fmaf(wf[0 * 4 + e], xv[j][l], 0.0f);
                                const float p1 = __builtin_fmaf(wf[1 * 4 + e], xv[j][8 + l], 0.0f);
                                const float p2 = __builtin_fmaf(wf[2 * 4 + e], xv[j][16 + l], 0.0f);
                                const float p3 = __builtin_fmaf(wf[3 * 4 + e], xv[j][24 + l], 0.0f);
                                tl[j][l] = (p0 + p1) + (p2 + p3);
                            }
                    }
                    float *pr = b7_sm + (size_t)r * ns * ldp + b;
#pragma unroll
                    for (int j = 0; j < SG; j++) {
                        const float dot = ((tl[j][0] + tl[j][1]) + (tl[j][2] + tl[j][3])) +
                                          ((tl[j][4] + tl[j][5]) + (tl[j][6] + tl[j][7]));
                        if (g * SG + j < ns) pr[(size_t)(g * SG + j) * ldp] = dot * sr[u];
                    }
                }
            }
        }
    }
    __syncthreads();
    for (int i = tid; i < nr * ns; i += blockDim.x) {
        const int r = i / ns, s = i - r * ns, row = row0 + r;
        const float4 *pp = (const float4 *)(b7_sm + (size_t)i * ldp);
        float acc = 0.0f;
#pragma unroll 20
        for (int q = 0; q < (nb >> 2); q++) {
            const float4 v = pp[q];
            acc = acc + v.x;
            acc = acc + v.y;
            acc = acc + v.z;
            acc = acc + v.w;
        }
        const float v = acc + (bias ? bias[row] : 0.0f);
        float *yp = y + (size_t)s * ldy + row;
        if (mode == 1) *yp = *yp + v;
        else *yp = v;
    }
}

// ---------------------------------------------------------------------------
// 1 / (sequential f32 sum of v[0..n)) (softmax_rows' sum, nn.rs:4880-4963), 0
// when the sum is not positive; one thread.  The dependent adds bound the
// loop; reading 64 values per LDS round trip keeps the waits between batches
// few.
__device__ __forceinline__ float fw_seq_sum_inv(const float *v, int n) {
    const float4 *v4 = (const float4 *)v;
    const int n4 = n >> 2, n16 = n4 & ~15;
    float sum = 0.0f;
    for (int q = 0; q < n16; q += 16) {
        float4 c[16];
#pragma unroll
        for (int u = 0; u < 16; u++) c[u] = v4[q + u];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            sum += c[u].x;
            sum += c[u].y;
            sum += c[u].z;
            sum += c[u].w;
        }
    }
    {
        // the last n4 % 16 groups and n % 4 values, read in one round trip
        float4 c[16];
        float t[3];
#pragma unroll
        for (int u = 0; u < 16; u++) c[u] = v4[n16 + u < n4 ? n16 + u : 0];
#pragma unroll
        for (int u = 0; u < 3; u++) t[u] = v[n4 * 4 + u < n ? n4 * 4 + u : 0];
#pragma unroll
        for (int u = 0; u < 16; u++) {
            if (n16 + u < n4) {
                sum += c[u].x;
                sum += c[u].y;
                sum += c[u].z;
                sum += c[u].w;
            }
        }
#pragma unroll
        for (int u = 0; u < 3; u++)
            if (n4 * 4 + u < n) sum += t[u];
    }
    return sum > 0.0f ? 1.0f / sum : 0.0f;
}


// ---------------------------------------------------------------------------
// Cross-attention for one (head, stream) with f16 K/V (cross_attention,
// decoder.rs:1524-1716, FRANKEN_WHISPER_INT8_CROSS_KV=0): qh = q*s; scores =
// gemv_f16(K_h, qh) and out = gemv_f16(Vt_h, p), both in dot_f16c order
// (nn.rs:1983-2051); softmax with glibc-exact expf and the sequential sum
// (nn.rs:4880-4963), formed by one wave (fw_seq_sum_wave) when T <= 1536.
// 512 threads.  Scores: a key row (64 f16) per thread per round, read as eight
// 16-byte loads.  Values: 8 lanes per output column dd, lane q owning chains
// 4q .. 4q+3 of each 32-key chunk (vector q/2, lanes 4(q%2) .. +3), then the
// dot_f16c reduction by butterflies; V^T rows need T % 4 == 0 for 8-byte loads
// (VEC), else they are read element by element.
#define XA_MAXC 48 // 32-key chunks of V^T a thread holds in registers (T <= 1536)
template <bool VEC>
__global__ void __launch_bounds__(512) k_cross_attn_f16v2(const float *qc, const uint16_t *ck, const uint16_t *cvt,
                                                          float *att, int d, int T, int H, int L, int layer,
                                                          float scale) {
    extern __shared__ __align__(16) float scf[]; // [(T + 3) & ~3]
    __shared__ float qh[64];
    __shared__ float red[8];
    __shared__ float inv_s;
    const int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    const size_t lh = ((size_t)s * L + layer) * H + h;
    const uint16_t *K = ck + lh * (size_t)T * 64;
    const uint16_t *V = cvt + lh * (size_t)T * 64;
    // VEC: this thread's V^T chunks (row dd = t / 8, 4 keys at 32c + 4(t % 8))
    // requested first, so they arrive under the scores and the softmax
    const int nc = T >> 5;
    uint2 vreg[VEC ? XA_MAXC : 1];
    if constexpr (VEC) {
        const uint16_t *vr0 = V + (size_t)(t >> 3) * T + (t & 7) * 4;
#pragma unroll
        for (int c = 0; c < XA_MAXC; c++) vreg[c] = *(const uint2 *)(vr0 + (size_t)(c < nc ? c : 0) * 32);
    }
    if (t < 64) qh[t] = qc[(size_t)s * d + h * 64 + t] * scale;
    __syncthreads();
    float mx = -INFINITY;
    for (int j = t; j < T; j += 512) {
        const uint4 *kr = (const uint4 *)(K + (size_t)j * 64);
        uint4 kv[8];
#pragma unroll
        for (int i = 0; i < 8; i++) kv[i] = kr[i];
        float a[4][8];
#pragma unroll
        for (int jv = 0; jv < 4; jv++)
#pragma unroll
            for (int l = 0; l < 8; l++) a[jv][l] = 0.0f;
#pragma unroll
        for (int c = 0; c < 2; c++)
#pragma unroll
            for (int jv = 0; jv < 4; jv++) {
                const uint4 u = kv[c * 4 + jv];
                const uint32_t uw[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
                for (int l = 0; l < 8; l++)
                    a[jv][l] = __builtin_fmaf(fw_h2f((uint16_t)(uw[l >> 1] >> ((l & 1) * 16))),
                                              qh[c * 32 + jv * 8 + l], a[jv][l]);
            }
        float tt[8];
#pragma unroll
        for (int l = 0; l < 8; l++) tt[l] = (a[0][l] + a[1][l]) + (a[2][l] + a[3][l]);
        const float v = ((tt[0] + tt[1]) + (tt[2] + tt[3])) + ((tt[4] + tt[5]) + (tt[6] + tt[7]));
        scf[j] = v;
        mx = fmaxf(mx, v);
    }
    mx = fw_block_max(mx, red);
    const bool fin = isfinite(mx);
    if (fin)
        for (int j = t; j < T; j += 512) {
            const float e = fw_expf(scf[j] - mx);
            scf[j] = isfinite(e) ? e : 0.0f;
        }
    __syncthreads();
    if (t < 64) {
        float sum = 0.0f;
        if (fin) {
            if (T <= 64 * SW_MAXC) {
                sum = fw_seq_sum_wave(scf, T);
            } else if (t == 0) {
                for (int j = 0; j < T; j++) sum += scf[j];
            }
        }
        if (t == 0) inv_s = (fin && sum > 0.0f) ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    const float inv = inv_s;
    if (inv > 0.0f)
        for (int j = t; j < T; j += 512) scf[j] = scf[j] * inv;
    __syncthreads();
    const int dd = t >> 3, q = t & 7;
    const uint16_t *vr = V + (size_t)dd * T;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (VEC) {
#pragma unroll
        for (int c = 0; c < XA_MAXC; c++) {
            if (c < nc) {
                const float4 p = *(const float4 *)(scf + c * 32 + q * 4);
                const uint2 u = vreg[c];
                a[0] = __builtin_fmaf(fw_h2f((uint16_t)(u.x & 0xffff)), p.x, a[0]);
                a[1] = __builtin_fmaf(fw_h2f((uint16_t)(u.x >> 16)), p.y, a[1]);
                a[2] = __builtin_fmaf(fw_h2f((uint16_t)(u.y & 0xffff)), p.z, a[2]);
                a[3] = __builtin_fmaf(fw_h2f((uint16_t)(u.y >> 16)), p.w, a[3]);
            }
        }
    } else {
        for (int c = 0; c < nc; c++) {
            const int i0 = c * 32 + q * 4;
            const float4 p = *(const float4 *)(scf + i0);
            a[0] = __builtin_fmaf(fw_h2f(vr[i0]), p.x, a[0]);
            a[1] = __builtin_fmaf(fw_h2f(vr[i0 + 1]), p.y, a[1]);
            a[2] = __builtin_fmaf(fw_h2f(vr[i0 + 2]), p.z, a[2]);
            a[3] = __builtin_fmaf(fw_h2f(vr[i0 + 3]), p.w, a[3]);
        }
    }
    // (a0 + a1) + (a2 + a3): vectors 2 lanes apart; then the 8-lane tree
#pragma unroll
    for (int e = 0; e < 4; e++) {
        a[e] = a[e] + __shfl_xor(a[e], 2, 64);
        a[e] = a[e] + __shfl_xor(a[e], 4, 64);
    }
    float acc = (a[0] + a[1]) + (a[2] + a[3]);
    acc = acc + __shfl_xor(acc, 1, 64);
    if (q == 0) {
        int i = nc * 32;
        for (; i + 8 <= T; i += 8) {
            float pp[8];
            for (int l = 0; l < 8; l++) pp[l] = fw_h2f(vr[i + l]) * scf[i + l];
            acc += ((pp[0] + pp[1]) + (pp[2] + pp[3])) + ((pp[4] + pp[5]) + (pp[6] + pp[7]));
        }
        for (; i < T; i++) acc += fw_h2f(vr[i]) * scf[i];
        att[(size_t)s * d + h * 64 + dd] = acc;
    }
}

void fw_launch_cross_attn_f16(hipStream_t st, const float *qc, const uint16_t *ck, const uint16_t *cvt, float *att,
                              int d, int T, int H, int L, int layer, int ns, float scale) {
    const size_t shm = sizeof(float) * (size_t)((T + 3) & ~3);
    if ((T & 3) == 0 && (T >> 5) <= XA_MAXC)
        hipLaunchKernelGGL(k_cross_attn_f16v2<true>, dim3(H, ns), dim3(512), shm, st, qc, ck, cvt, att, d, T, H, L,
                           layer, scale);
    else
        hipLaunchKernelGGL(k_cross_attn_f16v2<false>, dim3(H, ns), dim3(512), shm, st, qc, ck, cvt, att, d, T, H, L,
                           layer, scale);
}

// ---------------------------------------------------------------------------
// The same cross attention on K and V^T stored in slot order
// (fw_launch_pack_cross_f16): in a 64-wide group of a row, element
// 32cc + 8k + l sits at l*8 + cc*4 + k, so lane l of an 8-lane row group reads
// its four dot_f16c slots (k = 0..3, lane l) of two chunks as one 16-byte load
// and a row group's load is one whole 128-byte line.  Key rows are one group
// (64 values: the score chains are lane-local, then the slot tree's last
// three steps are lane exchanges).  V^T rows (stride Tv = T rounded up to 64)
// hold nc / 2 groups, an odd last chunk as l*4 + k, and the n % 32 tail in
// natural order.  512 threads: the value pass gives each of the 64 output
// rows one row group.  A lane requests all its key rows at entry (T <= 1536:
// 24 rounds of 64 keys) and its V^T groups after its scores; every request is
// a whole 128-byte line.
#define XP_MAXG 24 // full 64-key groups of V^T a lane holds in registers
__device__ __forceinline__ int fw_xp_pos(int e) { return (e & 7) * 8 + (e >> 5) * 4 + ((e >> 3) & 3); }

// FQ: the cross LayerNorm and this head's q rows are formed in the block
// (gemv_f16 of LN(x_s), nn.rs:2346-2460, on the slot-order matrix of
// fw_launch_pack_gemv16 at 16 lanes per row, d == 1280): wave 0 normalizes
// the stream's residual row into LDS (the GEMV's one-wave LayerNorm), then
// every lane carries 2 of the 64 rows for its 2 dot_f16c slots, the slot tree
// runs over the 16 lanes of a row, and the bias is added; so q holds the bits
// the separate GEMV writes.
#define XQ_D 1280
#ifndef XQ_EARLY
#define XQ_EARLY 8 // 64-key rounds requested before the q projection
#endif
// The cross LayerNorm of x_s (wave 0, the GEMV's one-wave arithmetic) into xl
// and the head's 64 q rows (gemv_f16 on the slot-order matrix at 16 lanes per
// row, then the bias) into qf; 512 threads, d == XQ_D.  issue_early runs once
// the weight rows are requested (key rows that stream in meanwhile),
// issue_late once the q rows are stored, before the caller's barrier.
template <bool SEQ, typename E, typename F>
__device__ __forceinline__ void xq_rows(const uint16_t *__restrict__ wq, const float *__restrict__ bq,
                                        const float *__restrict__ x, const float *__restrict__ lnw,
                                        const float *__restrict__ lnb, int h, int s, float *xl, float *qf,
                                        E &&issue_early, F &&issue_late) {
    constexpr int NV = XQ_D / 256, G = XQ_D / 128; // float4s per lane of a row; 16-byte groups per weight row
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int p = lane & 15, rq = lane >> 4; // lane of the row group, row group of the wave
    float4 lv[NV], lw[NV], lb[NV];
    bool lok[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        lok[k] = true;
        lv[k] = ((const float4 *)(x + (size_t)s * XQ_D))[lane + k * 64];
    }
    fw_ln_load_wb<NV>(lok, lnw, lnb, lw, lb, lane);
    // rows h * 64 + wave * 8 + r * 4 + rq, r = 0, 1
    uint4 wv[2][G];
#pragma unroll
    for (int r = 0; r < 2; r++) {
        const uint4 *wr = (const uint4 *)(wq + (size_t)(h * 64 + wave * 8 + r * 4 + rq) * XQ_D) + p;
#pragma unroll
        for (int g = 0; g < G; g++) wv[r][g] = wr[g * 16];
    }
    const float bv0 = bq ? bq[h * 64 + wave * 8 + rq] : 0.0f, bv1 = bq ? bq[h * 64 + wave * 8 + 4 + rq] : 0.0f;
    issue_early();
    if (wave == 0) fw_ln_quant_core<NV, SEQ>(lv, lok, lw, lb, xl, XQ_D, 0, nullptr, nullptr, lane);
    __syncthreads();
    // lane p = kh * 8 + l holds slots 8 (2 kh + kk) + l; a group is 4 chunks
    float acc[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
    const int kh = p >> 3, pl = p & 7;
#pragma unroll
    for (int g = 0; g < G; g++) {
#pragma unroll
        for (int cc = 0; cc < 4; cc++) {
            const int c = g * 4 + cc;
            const float x0 = xl[c * 32 + 8 * (2 * kh) + pl], x1 = xl[c * 32 + 8 * (2 * kh + 1) + pl];
#pragma unroll
            for (int r = 0; r < 2; r++) {
                const uint32_t u[4] = {wv[r][g].x, wv[r][g].y, wv[r][g].z, wv[r][g].w};
                const float w0 = fw_h2f((uint16_t)(u[cc] & 0xffffu)), w1 = fw_h2f((uint16_t)(u[cc] >> 16));
                acc[r][0] = __builtin_fmaf(w0, x0, acc[r][0]);
                acc[r][1] = __builtin_fmaf(w1, x1, acc[r][1]);
            }
        }
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
        float v = acc[r][0] + acc[r][1];
        v = v + __shfl_xor(v, 8, 64);
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 4, 64);
        if (bq) v = v + (r ? bv1 : bv0);
        if (p == 0) qf[wave * 8 + r * 4 + rq] = v;
    }
    issue_late();
}

template <bool FQ, bool SEQ>
__global__ void __launch_bounds__(512) k_cross_attn_f16p(const float *qc, const uint16_t *ckp, const uint16_t *cvtp,
                                                         float *att, int d, int T, int Tv, int H, int L, int layer,
                                                         float scale, const uint16_t *__restrict__ wq,
                                                         const float *__restrict__ bq, const float *__restrict__ x,
                                                         const float *__restrict__ lnw, const float *__restrict__ lnb,
                                                         int ns) {
    extern __shared__ __align__(16) float scf[]; // [Tv]: scores, then p in the value pass order
    __shared__ float red[8];
    __shared__ float inv_s;
    __shared__ uint64_t etab[32]; // fw_expf's table, in LDS: its lookups then wait on no global load
    // row s = blockIdx.y attends with the cross K/V of stream s % ns (a prefill
    // chunk's rows are [position][stream])
    const int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6, l = lane & 7, rg = lane >> 3;
    const size_t lh = ((size_t)(s % ns) * L + layer) * H + h;
    const uint16_t *K = ckp + lh * (size_t)T * 64;
    const uint16_t *V = cvtp + lh * (size_t)Tv * 64;
    const int nc = T >> 5, ng = nc >> 1, ntail = T - nc * 32;
    if (t < 32) {
        const uint64_t tb[32] = FW_EXP2F_TAB;
        etab[t] = tb[t];
    }
    float q0[4], q1[4];
    // (no load sits behind a branch: addresses past the end are clamped to
    // the last row and the values unused, so the waits count loads exactly)
    const int nr = (T + 63) >> 6;
    uint4 kv[XP_MAXG];
    auto load_keys = [&](auto lo_tag, auto hi_tag) {
        constexpr int LO = decltype(lo_tag)::value, HI = decltype(hi_tag)::value;
#pragma unroll
        for (int r = LO; r < HI; r++) {
            const int j = r * 64 + wave * 8 + rg;
            kv[r] = fw_ld_stream(K + (size_t)(j < T ? j : T - 1) * 64 + l * 8);
        }
    };
    using k0 = std::integral_constant<int, 0>;
    using kE = std::integral_constant<int, XQ_EARLY>;
    using kN = std::integral_constant<int, XP_MAXG>;
    if constexpr (FQ) {
        __shared__ __align__(16) float xl[XQ_D];
        __shared__ float qf[64];
        // the first key rows stream in while q is formed (all of them would
        // not fit the registers beside the q operands)
        xq_rows<SEQ>(wq, bq, x, lnw, lnb, h, s, xl, qf, [&] { load_keys(k0{}, kE{}); }, [&] { load_keys(kE{}, kN{}); });
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 4; k++) {
            q0[k] = qf[8 * k + l];
            q1[k] = qf[32 + 8 * k + l];
        }
    } else {
        // loads retire in order (vmcnt), so the first requests are the ones
        // used first: q, then every key row this lane multiplies (key j =
        // r * 64 + wave * 8 + rg)
        const float *qs = qc + (size_t)s * d + h * 64;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            q0[k] = qs[8 * k + l];
            q1[k] = qs[32 + 8 * k + l];
        }
        load_keys(k0{}, kN{});
    }
    // qh = q * s, this lane's slots of both chunks
#pragma unroll
    for (int k = 0; k < 4; k++) {
        q0[k] = q0[k] * scale;
        q1[k] = q1[k] * scale;
    }
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < XP_MAXG; r++) {
        if (r < nr) {
            const int j = r * 64 + wave * 8 + rg;
            const uint32_t u[4] = {kv[r].x, kv[r].y, kv[r].z, kv[r].w};
            float a[4];
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float w0 = fw_h2f((uint16_t)(u[k >> 1] >> ((k & 1) * 16)));
                const float w1 = fw_h2f((uint16_t)(u[2 + (k >> 1)] >> ((k & 1) * 16)));
                a[k] = __builtin_fmaf(w1, q1[k], __builtin_fmaf(w0, q0[k], 0.0f));
            }
            float v = (a[0] + a[1]) + (a[2] + a[3]);
            v = v + __shfl_xor(v, 1, 64);
            v = v + __shfl_xor(v, 2, 64);
            v = v + __shfl_xor(v, 4, 64);
            if (j < T) {
                if (l == 0) scf[j] = v;
                mx = fmaxf(mx, v);
            }
        }
    }
    // the value rows are requested once this wave's scores are formed: a
    // CU's memory queue serves the block's key rows first, and the softmax
    // (with its 1500-long sequential sum) runs while the values stream in
    __builtin_amdgcn_sched_barrier(0);
    const int dd = wave * 8 + rg;
    const uint16_t *vr = V + (size_t)dd * Tv;
    uint4 vreg[XP_MAXG];
#pragma unroll
    for (int g = 0; g < XP_MAXG; g++) vreg[g] = fw_ld_stream(vr + (g < ng ? g : 0) * 64 + l * 8);
    // the odd last chunk (when nc is odd, ng * 64 + 32 <= nc * 32 <= Tv)
    const uint2 vodd = *(const uint2 *)(vr + ((nc & 1) ? ng * 64 : 0) + l * 4);
    // the n % 32 tail (rows are Tv >= nc * 32 + 32 long; used by lane 0 only)
    uint4 vtail[4];
#pragma unroll
    for (int i = 0; i < 4; i++) vtail[i] = fw_ld_stream(vr + (ntail > 0 ? nc * 32 : 0) + i * 8);
    mx = fw_block_max(mx, red);
    const bool fin = isfinite(mx);
    // (the value rows are in flight: reads clamped to the scores, the table
    // in LDS, so the exps wait on no global load)
    if (fin) {
        float sv[3];
#pragma unroll
        for (int u = 0; u < 3; u++) sv[u] = scf[min(t + u * 512, T - 1)];
#pragma unroll
        for (int u = 0; u < 3; u++) {
            const float e = fw_expf_tab(sv[u] - mx, etab);
            if (t + u * 512 < T) scf[t + u * 512] = isfinite(e) ? e : 0.0f;
        }
    }
    __syncthreads();
    if (t < 64) {
        float sum = 0.0f;
        if (fin) {
            if (T <= 64 * SW_MAXC) {
                sum = fw_seq_sum_wave(scf, T);
            } else if (t == 0) {
                for (int j = 0; j < T; j++) sum += scf[j];
            }
        }
        if (t == 0) inv_s = (fin && sum > 0.0f) ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    // p (normalized when the sum is positive; a non-finite max leaves the raw
    // scores, as softmax_rows does), moved to the value pass order: within
    // chunk c, element 8k + l to 4l + k; the tail stays in place
    const float inv = inv_s;
    float pv[3];
#pragma unroll
    for (int u = 0; u < 3; u++) {
        const int j = t + u * 512;
        pv[u] = j < T ? (inv > 0.0f ? scf[j] * inv : scf[j]) : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < 3; u++) {
        const int j = t + u * 512;
        if (j < T) {
            const int e = j & 31;
            scf[j < nc * 32 ? (j & ~31) + (e & 7) * 4 + (e >> 3) : j] = pv[u];
        }
    }
    __syncthreads();
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < XP_MAXG; g++) {
        if (g < ng) {
            const float4 p0 = *(const float4 *)(scf + g * 64 + l * 4);
            const float4 p1 = *(const float4 *)(scf + g * 64 + 32 + l * 4);
            const uint32_t u[4] = {vreg[g].x, vreg[g].y, vreg[g].z, vreg[g].w};
            const float pa[4] = {p0.x, p0.y, p0.z, p0.w}, pb[4] = {p1.x, p1.y, p1.z, p1.w};
#pragma unroll
            for (int k = 0; k < 4; k++)
                a[k] = __builtin_fmaf(fw_h2f((uint16_t)(u[k >> 1] >> ((k & 1) * 16))), pa[k], a[k]);
#pragma unroll
            for (int k = 0; k < 4; k++)
                a[k] = __builtin_fmaf(fw_h2f((uint16_t)(u[2 + (k >> 1)] >> ((k & 1) * 16))), pb[k], a[k]);
        }
    }
    if (nc & 1) {
        const float4 p0 = *(const float4 *)(scf + (nc - 1) * 32 + l * 4);
        const float pa[4] = {p0.x, p0.y, p0.z, p0.w};
        const uint32_t u[2] = {vodd.x, vodd.y};
#pragma unroll
        for (int k = 0; k < 4; k++) a[k] = __builtin_fmaf(fw_h2f((uint16_t)(u[k >> 1] >> ((k & 1) * 16))), pa[k], a[k]);
    }
    float acc = (a[0] + a[1]) + (a[2] + a[3]);
    acc = acc + __shfl_xor(acc, 1, 64);
    acc = acc + __shfl_xor(acc, 2, 64);
    acc = acc + __shfl_xor(acc, 4, 64);
    if (l == 0) {
        // dot_f16c's tails: whole 8-wide chunks (products, then their tree), then scalars
        const uint32_t tw[16] = {vtail[0].x, vtail[0].y, vtail[0].z, vtail[0].w, vtail[1].x, vtail[1].y,
                                 vtail[1].z, vtail[1].w, vtail[2].x, vtail[2].y, vtail[2].z, vtail[2].w,
                                 vtail[3].x, vtail[3].y, vtail[3].z, vtail[3].w};
        const float *pt = scf + nc * 32;
        int i = 0;
#pragma unroll
        for (int c8 = 0; c8 < 4; c8++) {
            if (i + 8 <= ntail) {
                float pp[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int ii = c8 * 8 + e;
                    pp[e] = fw_h2f((uint16_t)(tw[ii >> 1] >> ((ii & 1) * 16))) * pt[ii];
                }
                acc += ((pp[0] + pp[1]) + (pp[2] + pp[3])) + ((pp[4] + pp[5]) + (pp[6] + pp[7]));
                i += 8;
            }
        }
#pragma unroll
        for (int ii = 0; ii < 32; ii++)
            if (ii >= i && ii < ntail) acc += fw_h2f((uint16_t)(tw[ii >> 1] >> ((ii & 1) * 16))) * pt[ii];
        att[(size_t)s * d + h * 64 + dd] = acc;
    }
}

// The same cross attention in two launches for cohorts too small to fill the
// CUs with one block per (head, stream): k_cross_scores_f16p spreads a head's
// keys over XS_KC blocks (the per-key dot_f16c of k_cross_attn_f16p, and each
// block's maximum), k_cross_pv_f16p gives each of XS_DC blocks 64 / XS_DC of
// the head's output dims, every one forming the same softmax (the maximum of
// the chunk maxima, expf, the sequential sum by one wave, p in the value pass
// order) before its value pass.  Every value has the one-launch kernel's bits.
#define XS_KC 8
#define XS_DC 4
__global__ void __launch_bounds__(256) k_cross_scores_f16p(const float *qc, const uint16_t *ckp, float *sbuf,
                                                           float *mbuf, int d, int T, int Tv, int H, int L, int layer,
                                                           int ns, float scale) {
    __shared__ float red[4];
    const int h = blockIdx.x, kc = blockIdx.y, r = blockIdx.z, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6, l = lane & 7, rg = lane >> 3;
    const size_t lh = ((size_t)(r % ns) * L + layer) * H + h;
    const uint16_t *K = ckp + lh * (size_t)T * 64;
    const int CH = ((T + XS_KC * 64 - 1) / (XS_KC * 64)) * 64, j0 = kc * CH, j1 = min(T, j0 + CH);
    const float *qs = qc + (size_t)r * d + h * 64;
    float q0[4], q1[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        q0[k] = qs[8 * k + l] * scale;
        q1[k] = qs[32 + 8 * k + l] * scale;
    }
    constexpr int NR = 1536 / XS_KC / 32; // 32-key rounds a block holds at most (T <= 1536)
    uint4 kv[NR];
#pragma unroll
    for (int q = 0; q < NR; q++) {
        const int j = j0 + q * 32 + wave * 8 + rg;
        kv[q] = fw_ld_stream(K + (size_t)(j < j1 ? j : (j1 > j0 ? j1 - 1 : 0)) * 64 + l * 8);
    }
    float mx = -INFINITY;
    float *sc = sbuf + ((size_t)r * H + h) * Tv;
#pragma unroll
    for (int q = 0; q < NR; q++) {
        const int j = j0 + q * 32 + wave * 8 + rg;
        const uint32_t u[4] = {kv[q].x, kv[q].y, kv[q].z, kv[q].w};
        float a[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float w0 = fw_h2f((uint16_t)(u[k >> 1] >> ((k & 1) * 16)));
            const float w1 = fw_h2f((uint16_t)(u[2 + (k >> 1)] >> ((k & 1) * 16)));
            a[k] = __builtin_fmaf(w1, q1[k], __builtin_fmaf(w0, q0[k], 0.0f));
        }
        float v = (a[0] + a[1]) + (a[2] + a[3]);
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 4, 64);
        if (j < j1) {
            if (l == 0) sc[j] = v;
            mx = fmaxf(mx, v);
        }
    }
    mx = fw_block_max(mx, red);
    if (t == 0) mbuf[((size_t)r * H + h) * XS_KC + kc] = mx;
}

// k_cross_scores_f16p with the cross LayerNorm and the head's q rows formed
// in the block (xq_rows; the separate LN + q GEMV's bits), 512 threads: each
// of a head's XS_KC blocks forms the same q, its three 64-key rounds
// requested while q is formed.  For cohorts that fill few CUs: it saves the
// q GEMV's launch at the price of XS_KC reads of the head's q rows from L2.
template <bool SEQ>
__global__ void __launch_bounds__(512) k_cross_scores_f16pq(const uint16_t *__restrict__ wq,
                                                            const float *__restrict__ bq, const float *__restrict__ x,
                                                            const float *__restrict__ lnw,
                                                            const float *__restrict__ lnb, const uint16_t *ckp,
                                                            float *sbuf, float *mbuf, int T, int Tv, int H, int L,
                                                            int layer, int ns, float scale) {
    __shared__ __align__(16) float xl[XQ_D];
    __shared__ float qf[64];
    __shared__ float red[8];
    const int h = blockIdx.x, kc = blockIdx.y, r = blockIdx.z, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6, l = lane & 7, rg = lane >> 3;
    const size_t lh = ((size_t)(r % ns) * L + layer) * H + h;
    const uint16_t *K = ckp + lh * (size_t)T * 64;
    const int CH = ((T + XS_KC * 64 - 1) / (XS_KC * 64)) * 64, j0 = kc * CH, j1 = min(T, j0 + CH);
    constexpr int NR = 1536 / XS_KC / 64; // 64-key rounds a block holds at most (T <= 1536)
    uint4 kv[NR];
    xq_rows<SEQ>(
        wq, bq, x, lnw, lnb, h, r, xl, qf,
        [&] {
#pragma unroll
            for (int q = 0; q < NR; q++) {
                const int j = j0 + q * 64 + wave * 8 + rg;
                kv[q] = fw_ld_stream(K + (size_t)(j < j1 ? j : (j1 > j0 ? j1 - 1 : 0)) * 64 + l * 8);
            }
        },
        [] {});
    __syncthreads();
    float q0[4], q1[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        q0[k] = qf[8 * k + l] * scale;
        q1[k] = qf[32 + 8 * k + l] * scale;
    }
    float mx = -INFINITY;
    float *sc = sbuf + ((size_t)r * H + h) * Tv;
#pragma unroll
    for (int q = 0; q < NR; q++) {
        const int j = j0 + q * 64 + wave * 8 + rg;
        const uint32_t u[4] = {kv[q].x, kv[q].y, kv[q].z, kv[q].w};
        float a[4];
#pragma unroll
        for (int k = 0; k < 4; k++) {
            const float w0 = fw_h2f((uint16_t)(u[k >> 1] >> ((k & 1) * 16)));
            const float w1 = fw_h2f((uint16_t)(u[2 + (k >> 1)] >> ((k & 1) * 16)));
            a[k] = __builtin_fmaf(w1, q1[k], __builtin_fmaf(w0, q0[k], 0.0f));
        }
        float v = (a[0] + a[1]) + (a[2] + a[3]);
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 4, 64);
        if (j < j1) {
            if (l == 0) sc[j] = v;
            mx = fmaxf(mx, v);
        }
    }
    mx = fw_block_max(mx, red);
    if (t == 0) mbuf[((size_t)r * H + h) * XS_KC + kc] = mx;
}

__global__ void __launch_bounds__(256) k_cross_pv_f16p(const float *sbuf, const float *mbuf, const uint16_t *cvtp,
                                                       float *att, int d, int T, int Tv, int H, int L, int layer,
                                                       int ns) {
    // [Tv] the exponentials in key order (the sum's input), then [Tv] the
    // same in the value pass order: within chunk c element 8k + l sits at
    // 4l + k, the n % 32 tail in place
    extern __shared__ __align__(16) float scf[];
    float *sp = scf + Tv;
    __shared__ float inv_s;
    __shared__ uint64_t etab[32]; // fw_expf's table, in LDS: its lookups then wait on no global load
    const int h = blockIdx.x, dc = blockIdx.y, r = blockIdx.z, t = threadIdx.x;
    if (t < 32) {
        const uint64_t tb[32] = FW_EXP2F_TAB;
        etab[t] = tb[t];
    }
    const int lane = t & 63, l = lane & 7;
    const size_t lh = ((size_t)(r % ns) * L + layer) * H + h;
    const uint16_t *V = cvtp + lh * (size_t)Tv * 64;
    const int nc = T >> 5, ng = nc >> 1, ntail = T - nc * 32;
    constexpr int DPB = 64 / XS_DC; // dims of this block: threads [0, 8 * DPB) hold one each
    const bool pvt = t < 8 * DPB;
    const int dd = dc * DPB + (pvt ? t >> 3 : 0);
    // this thread's scores and the block maxima first (loads retire in order),
    // then the value rows, which stream in while the softmax is formed; no
    // load sits behind a branch (addresses clamped)
    constexpr int PU = 1536 / 256;
    const float *sc = sbuf + ((size_t)r * H + h) * Tv;
    float sv[PU], mk[XS_KC];
#pragma unroll
    for (int u = 0; u < PU; u++) sv[u] = sc[min(t + u * 256, T - 1)];
#pragma unroll
    for (int k = 0; k < XS_KC; k++) mk[k] = mbuf[((size_t)r * H + h) * XS_KC + k];
    const uint16_t *vr = V + (size_t)dd * Tv;
    uint4 vreg[XP_MAXG];
#pragma unroll
    for (int g = 0; g < XP_MAXG; g++) vreg[g] = fw_ld_stream(vr + (g < ng ? g : 0) * 64 + l * 8);
    const uint2 vodd = *(const uint2 *)(vr + ((nc & 1) ? ng * 64 : 0) + l * 4);
    uint4 vtail[4];
#pragma unroll
    for (int i = 0; i < 4; i++) vtail[i] = fw_ld_stream(vr + (ntail > 0 ? nc * 32 : 0) + i * 8);
    float mx = -INFINITY;
#pragma unroll
    for (int k = 0; k < XS_KC; k++) mx = fmaxf(mx, mk[k]);
    const bool fin = isfinite(mx);
    __syncthreads();
    // expf of every held score (any input keeps fw_expf's table index in
    // range); a non-finite max keeps the raw scores
#pragma unroll
    for (int u = 0; u < PU; u++) {
        const float e = fw_expf_tab(sv[u] - mx, etab);
        const float v = fin ? (isfinite(e) ? e : 0.0f) : sv[u];
        const int j = t + u * 256, ee = j & 31;
        if (j < T) {
            scf[j] = v;
            sp[j < nc * 32 ? (j & ~31) + (ee & 7) * 4 + (ee >> 3) : j] = v;
        }
    }
    __syncthreads();
    if (t < 64) {
        float sum = 0.0f;
        if (fin) {
            if (T <= 64 * SW_MAXC) {
                sum = fw_seq_sum_wave(scf, T);
            } else if (t == 0) {
                for (int j = 0; j < T; j++) sum += scf[j];
            }
        }
        if (t == 0) inv_s = (fin && sum > 0.0f) ? 1.0f / sum : 0.0f;
    }
    __syncthreads();
    // p = e * inv when the sum is positive, else e (x * 1 is x): the bits of
    // the one-launch kernel's p
    const float pm = inv_s > 0.0f ? inv_s : 1.0f;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int g = 0; g < XP_MAXG; g++) {
        if (g < ng) {
            const float4 p0 = *(const float4 *)(sp + g * 64 + l * 4);
            const float4 p1 = *(const float4 *)(sp + g * 64 + 32 + l * 4);
            const uint32_t u[4] = {vreg[g].x, vreg[g].y, vreg[g].z, vreg[g].w};
            const float pa[4] = {p0.x * pm, p0.y * pm, p0.z * pm, p0.w * pm};
            const float pb[4] = {p1.x * pm, p1.y * pm, p1.z * pm, p1.w * pm};
#pragma unroll
            for (int k = 0; k < 4; k++)
                a[k] = __builtin_fmaf(fw_h2f((uint16_t)(u[k >> 1] >> ((k & 1) * 16))), pa[k], a[k]);
#pragma unroll
            for (int k = 0; k < 4; k++)
                a[k] = __builtin_fmaf(fw_h2f((uint16_t)(u[2 + (k >> 1)] >> ((k & 1) * 16))), pb[k], a[k]);
        }
    }
    // the odd last chunk and the tail's p (rows of sp are Tv >= nc * 32 + 32
    // long: read whole, used where in range)
    const float4 po = *(const float4 *)(sp + (nc & 1 ? (nc - 1) * 32 : 0) + l * 4);
    float pt[32];
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 q = *(const float4 *)(sp + nc * 32 + i * 4);
        pt[4 * i] = q.x * pm;
        pt[4 * i + 1] = q.y * pm;
        pt[4 * i + 2] = q.z * pm;
        pt[4 * i + 3] = q.w * pm;
    }
    if (nc & 1) {
        const float pa[4] = {po.x * pm, po.y * pm, po.z * pm, po.w * pm};
        const uint32_t u[2] = {vodd.x, vodd.y};
#pragma unroll
        for (int k = 0; k < 4; k++) a[k] = __builtin_fmaf(fw_h2f((uint16_t)(u[k >> 1] >> ((k & 1) * 16))), pa[k], a[k]);
    }
    float acc = (a[0] + a[1]) + (a[2] + a[3]);
    acc = acc + __shfl_xor(acc, 1, 64);
    acc = acc + __shfl_xor(acc, 2, 64);
    acc = acc + __shfl_xor(acc, 4, 64);
    if (pvt && l == 0) {
        // dot_f16c's tails: whole 8-wide chunks (products, then their tree), then scalars
        const uint32_t tw[16] = {vtail[0].x, vtail[0].y, vtail[0].z, vtail[0].w, vtail[1].x, vtail[1].y,
                                 vtail[1].z, vtail[1].w, vtail[2].x, vtail[2].y, vtail[2].z, vtail[2].w,
                                 vtail[3].x, vtail[3].y, vtail[3].z, vtail[3].w};
        const int n8 = ntail >> 3;
#pragma unroll
        for (int c8 = 0; c8 < 4; c8++) {
            if (c8 < n8) {
                float pp[8];
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    const int ii = c8 * 8 + e;
                    pp[e] = fw_h2f((uint16_t)(tw[ii >> 1] >> ((ii & 1) * 16))) * pt[ii];
                }
                acc += ((pp[0] + pp[1]) + (pp[2] + pp[3])) + ((pp[4] + pp[5]) + (pp[6] + pp[7]));
            }
        }
#pragma unroll
        for (int ii = 0; ii < 32; ii++)
            if (ii >= n8 * 8 && ii < ntail) acc += fw_h2f((uint16_t)(tw[ii >> 1] >> ((ii & 1) * 16))) * pt[ii];
        att[(size_t)r * d + h * 64 + dd] = acc;
    }
}

size_t fw_cross_split_floats(int T, int H, int ns) {
    return (size_t)ns * H * (fw_cross_f16p_tv(T) + XS_KC);
}

// the same with the cross LayerNorm of x and the q projection in the scores
// launch (wq in fw_launch_pack_gemv16's slot order at 16 lanes per row; needs
// fw_cross_f16pq_ok(d, T, H))
void fw_launch_cross_attn_f16pq_split(hipStream_t st, const uint16_t *wq, const float *bq, const float *x,
                                      const float *lnw, const float *lnb, const uint16_t *ckp, const uint16_t *cvtp,
                                      float *att, int d, int T, int H, int L, int layer, int ns, float scale,
                                      float *scratch, int lnseq) {
    const int Tv = fw_cross_f16p_tv(T);
    float *sbuf = scratch, *mbuf = scratch + (size_t)ns * H * Tv;
    if (lnseq)
        hipLaunchKernelGGL(k_cross_scores_f16pq<true>, dim3(H, XS_KC, ns), dim3(512), 0, st, wq, bq, x, lnw, lnb, ckp,
                           sbuf, mbuf, T, Tv, H, L, layer, ns, scale);
    else
        hipLaunchKernelGGL(k_cross_scores_f16pq<false>, dim3(H, XS_KC, ns), dim3(512), 0, st, wq, bq, x, lnw, lnb, ckp,
                           sbuf, mbuf, T, Tv, H, L, layer, ns, scale);
    hipLaunchKernelGGL(k_cross_pv_f16p, dim3(H, XS_DC, ns), dim3(256), sizeof(float) * 2 * (size_t)Tv, st, sbuf, mbuf,
                       cvtp, att, d, T, Tv, H, L, layer, ns);
}

// scratch: fw_cross_split_floats(T, H, ns) floats
void fw_launch_cross_attn_f16p_split(hipStream_t st, const float *qc, const uint16_t *ckp, const uint16_t *cvtp,
                                     float *att, int d, int T, int H, int L, int layer, int ns, float scale,
                                     float *scratch) {
    const int Tv = fw_cross_f16p_tv(T);
    float *sbuf = scratch, *mbuf = scratch + (size_t)ns * H * Tv;
    hipLaunchKernelGGL(k_cross_scores_f16p, dim3(H, XS_KC, ns), dim3(256), 0, st, qc, ckp, sbuf, mbuf, d, T, Tv, H,
                       L, layer, ns, scale);
    hipLaunchKernelGGL(k_cross_pv_f16p, dim3(H, XS_DC, ns), dim3(256), sizeof(float) * 2 * (size_t)Tv, st, sbuf, mbuf,
                       cvtp, att, d, T, Tv, H, L, layer, ns);
}

// K [rows_k, 64] and V^T [rows_v, T] (natural order) to the slot order of
// k_cross_attn_f16p; V^T rows take stride Tv (pad left as it is).
__global__ void __launch_bounds__(256) k_pack_cross_f16(const uint16_t *ck, const uint16_t *cvt, uint16_t *ckp,
                                                        uint16_t *cvtp, size_t rows_k, size_t rows_v, int T, int Tv) {
    const size_t nk = rows_k * 64, nv = rows_v * (size_t)T;
    const int nc = T >> 5, ng = nc >> 1;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < nk + nv; i += (size_t)gridDim.x * 256) {
        if (i < nk) {
            ckp[(i & ~(size_t)63) + fw_xp_pos((int)(i & 63))] = ck[i];
        } else {
            const size_t iv = i - nk, r = iv / T;
            const int e = (int)(iv - r * T);
            int pos;
            if (e < ng * 64) pos = (e & ~63) + fw_xp_pos(e & 63);
            else if (e < nc * 32) pos = ng * 64 + ((e - ng * 64) & 7) * 4 + ((e - ng * 64) >> 3);
            else pos = e;
            cvtp[r * Tv + pos] = cvt[iv];
        }
    }
}

// the value pass holds <= XP_MAXG groups per lane and p in 3 values per thread;
// the sum needs T <= 64 * SW_MAXC
bool fw_cross_f16p_ok(int T) { return T > 0 && T <= 1536 && T <= 64 * SW_MAXC && T <= 64 * XP_MAXG; }
int fw_cross_f16p_tv(int T) { return (T + 63) & ~63; }

void fw_launch_pack_cross_f16(hipStream_t st, const uint16_t *ck, const uint16_t *cvt, uint16_t *ckp, uint16_t *cvtp,
                              size_t rows_k, size_t rows_v, int T) {
    const size_t tot = rows_k * 64 + rows_v * (size_t)T;
    size_t g = (tot + 255) / 256;
    g = g < 65536 ? g : 65536;
    hipLaunchKernelGGL(k_pack_cross_f16, dim3((unsigned)g), dim3(256), 0, st, ck, cvt, ckp, cvtp, rows_k, rows_v, T,
                       fw_cross_f16p_tv(T));
}

void fw_launch_cross_attn_f16p(hipStream_t st, const float *qc, const uint16_t *ckp, const uint16_t *cvtp, float *att,
                               int d, int T, int H, int L, int layer, int ns, float scale, int rows) {
    const int Tv = fw_cross_f16p_tv(T);
    hipLaunchKernelGGL((k_cross_attn_f16p<false, false>), dim3(H, rows > 0 ? rows : ns), dim3(512),
                       sizeof(float) * (size_t)Tv, st, qc, ckp, cvtp, att, d, T, Tv, H, L, layer, scale, nullptr,
                       nullptr, nullptr, nullptr, nullptr, ns);
}

bool fw_cross_f16pq_ok(int d, int T, int H) { return d == XQ_D && H * 64 == d && fw_cross_f16p_ok(T); }

// the same with the cross LayerNorm of x and the q projection (wq: the cross
// q weights in fw_launch_pack_gemv16's slot order, 16 lanes per row) inside
void fw_launch_cross_attn_f16pq(hipStream_t st, const uint16_t *wq, const float *bq, const float *x, const float *lnw,
                                const float *lnb, const uint16_t *ckp, const uint16_t *cvtp, float *att, int d, int T,
                                int H, int L, int layer, int ns, float scale, int lnseq) {
    const int Tv = fw_cross_f16p_tv(T);
    if (lnseq)
        hipLaunchKernelGGL((k_cross_attn_f16p<true, true>), dim3(H, ns), dim3(512), sizeof(float) * (size_t)Tv, st,
                           nullptr, ckp, cvtp, att, d, T, Tv, H, L, layer, scale, wq, bq, x, lnw, lnb, ns);
    else
        hipLaunchKernelGGL((k_cross_attn_f16p<true, false>), dim3(H, ns), dim3(512), sizeof(float) * (size_t)Tv, st,
                           nullptr, ckp, cvtp, att, d, T, Tv, H, L, layer, scale, wq, bq, x, lnw, lnb, ns);
}

// ---------------------------------------------------------------------------
// sum_j p[j] * v[j*64 + t] (f16 values) in ascending j, one f32 chain per
// thread (the attention value pass of one output column); the operands of 32
// keys are read before their adds, so LDS latency is paid once per 32 keys.
// The self-attention KV cache element: f16 (FW_KV_F16: the row rounded to
// f16 on append, read back exactly) or f32 (the reference's default cache, the
// row as computed).  Attention reads either as f32 with the same arithmetic
// (attention_decode_step / _f16, nn.rs:6340-6523).
template <typename KV>
struct KvT;
template <>
struct KvT<uint16_t> {
    static __device__ __forceinline__ float val(uint16_t x) { return fw_h2f(x); }
    static __device__ __forceinline__ void put(uint16_t *p, size_t i, float v) { p[i] = fw_f2h(v); }
};
template <>
struct KvT<float> {
    static __device__ __forceinline__ float val(float x) { return x; }
    static __device__ __forceinline__ void put(float *p, size_t i, float v) { p[i] = v; }
};

template <typename KV>
__device__ __forceinline__ float fw_pv_chain(const float *p, const KV *v, int tk, int t) {
    float acc = 0.0f;
    int j = 0;
    for (; j + 32 <= tk; j += 32) {
        float pv[32], vv[32];
#pragma unroll
        for (int u = 0; u < 32; u++) {
            pv[u] = p[j + u];
            vv[u] = KvT<KV>::val(v[(j + u) * 64 + t]);
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < 32; u++) acc += pv[u] * vv[u];
    }
    for (; j + 8 <= tk; j += 8) {
        float pv[8], vv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            pv[u] = p[j + u];
            vv[u] = KvT<KV>::val(v[(j + u) * 64 + t]);
        }
#pragma unroll
        for (int u = 0; u < 8; u++) acc += pv[u] * vv[u];
    }
    for (; j < tk; j++) acc += p[j] * KvT<KV>::val(v[j * 64 + t]);
    return acc;
}

// ---------------------------------------------------------------------------
// Self-attention over the f16 KV cache for one (head, stream), tq == 1
// (attention_with_cache nn.rs:6267-6337 -> KvCache::append nn.rs:5352 ->
// attention_decode_step_f16 nn.rs:6466-6540).  Appends this token's k/v (RNE
// to f16) at pos and attends over [0, pos]: per-key ascending-d scores of
// (q*s)*(k*s), softmax with glibc-exact expf and a sequential sum, then per
// output the ascending-j sum of p_j * v_j.  256 threads: one key per thread
// for the scores; the cache rows of this head are staged in LDS for the
// value pass.
#define SA_STG 4
// A head's cache row is KW 16-byte chunks (8 for f16, 16 for f32)
template <typename KV>
struct SaRow {
    static constexpr int KW = 64 * (int)sizeof(KV) / 16, EPC = 16 / (int)sizeof(KV);
};
// score = sequential sum over the head's 64 dims of qh[i] * (k[i] * s)
// (attention_decode_step / _f16, nn.rs:6340-6523)
template <typename KV>
__device__ __forceinline__ float sa_score(const float *qh, const uint4 (&kk)[SaRow<KV>::KW], float scale) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < SaRow<KV>::KW; c++) {
        const uint32_t ww[4] = {kk[c].x, kk[c].y, kk[c].z, kk[c].w};
        if constexpr (sizeof(KV) == 2) {
#pragma unroll
            for (int e = 0; e < 4; e++) {
                acc += qh[c * 8 + 2 * e] * (fw_h2f(ww[e] & 0xffff) * scale);
                acc += qh[c * 8 + 2 * e + 1] * (fw_h2f(ww[e] >> 16) * scale);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; e++) acc += qh[c * 4 + e] * (__uint_as_float(ww[e]) * scale);
        }
    }
    return acc;
}

// The attention of one (head, stream) over cache rows [0, tk) once the
// token's own row is in the cache and qh (= q * s, LDS) is set; NT threads.
template <int NT, typename KV>
__device__ __forceinline__ void sa_attend(const float *qh, const KV *kc, const KV *vc, size_t cbase, int base, int d,
                                          int tk, float scale, float *sc, KV *vs, float *red, float *inv_s,
                                          float *out, float *pmax_slot) {
    constexpr int KW = SaRow<KV>::KW, EPC = SaRow<KV>::EPC;
    const int t = threadIdx.x;
    // this thread's first key row is requested ahead of the value rows (clamped
    // address, used when t < tk), so keys and values share one round trip
    uint4 kpre[KW];
    {
        const uint4 *kr = (const uint4 *)(kc + cbase + (size_t)(t < tk ? t : tk - 1) * d + base);
#pragma unroll
        for (int c = 0; c < KW; c++) kpre[c] = kr[c];
    }
    // stage V rows [0, tk) of this head (KW x 16 bytes per row), SA_STG chunks
    // per thread per round, loads issued before the LDS stores
    for (int c0 = 0; c0 < tk * KW; c0 += NT * SA_STG) {
        uint4 v[SA_STG];
#pragma unroll
        for (int u = 0; u < SA_STG; u++) {
            int c = c0 + t + u * NT;
            int cc = c < tk * KW ? c : tk * KW - 1;
            v[u] = *(const uint4 *)(vc + cbase + (size_t)((unsigned)cc / KW) * d + base + ((unsigned)cc % KW) * EPC);
        }
#pragma unroll
        for (int u = 0; u < SA_STG; u++) {
            int c = c0 + t + u * NT;
            if (c < tk * KW) ((uint4 *)vs)[c] = v[u];
        }
    }
    float mx = -INFINITY;
    auto score = [&](const uint4 (&kk)[KW]) { return sa_score<KV>(qh, kk, scale); };
    if (t < tk) {
        const float acc = score(kpre);
        sc[t] = acc;
        mx = fmaxf(mx, acc);
    }
    for (int j = t + NT; j < tk; j += NT) {
        const uint4 *kr = (const uint4 *)(kc + cbase + (size_t)j * d + base);
        uint4 kk[KW];
#pragma unroll
        for (int c = 0; c < KW; c++) kk[c] = kr[c];
        const float acc = score(kk);
        sc[j] = acc;
        mx = fmaxf(mx, acc);
    }
    mx = fw_block_max(mx, red);
    const bool fin = isfinite(mx);
    if (fin)
        for (int j = t; j < tk; j += NT) {
            float e = fw_expf(sc[j] - mx);
            sc[j] = isfinite(e) ? e : 0.0f;
        }
    __syncthreads();
    if (t == 0) *inv_s = fin ? fw_seq_sum_inv(sc, tk) : 0.0f;
    __syncthreads();
    const float inv = *inv_s;
    if (inv > 0.0f)
        for (int j = t; j < tk; j += NT) sc[j] = sc[j] * inv;
    __syncthreads();
    if (t < 64) {
        const float acc = fw_pv_chain(sc, vs, tk, t);
        out[t] = acc;
        // this head's share of the row amax the int8 consumer needs
        const float m = fw_dpp_wave_max(fabsf(acc));
        if (pmax_slot && t == 0) *pmax_slot = m;
    }
}

// Row r = blockIdx.y is stream r % ns at position *posp + r / ns (a prefill
// chunk's rows are [position][stream]; a step has one row per stream).  With
// `append` the row's own k/v go into the cache first; a prefill chunk appends
// every row beforehand (k_kv_append16), so a row sees the earlier rows of its
// chunk.
template <typename KV>
__global__ void __launch_bounds__(256) k_self_attn2(const float *qkv, KV *kc, KV *vc, float *att, const int *posp,
                                                    int d, int nctx, int L, int layer, float scale, float *pmax,
                                                    int ns, int append) {
    extern __shared__ __align__(16) unsigned char sm2[];
    float *sc = (float *)sm2;                                    // [nctx]
    KV *vs = (KV *)(sm2 + sizeof(float) * ((nctx + 3) & ~3));   // [nctx][64]
    __shared__ float qh[64];
    __shared__ float red[4];
    __shared__ float inv_s;
    const int h = blockIdx.x, r = blockIdx.y, t = threadIdx.x;
    const int s = r % ns, pos = *posp + r / ns;
    const int base = h * 64;
    const float *q = qkv + (size_t)r * 3 * d;
    const size_t cbase = ((size_t)s * L + layer) * nctx * d;
    if (t < 64) {
        if (append) {
            KvT<KV>::put(kc, cbase + (size_t)pos * d + base + t, q[d + base + t]);
            KvT<KV>::put(vc, cbase + (size_t)pos * d + base + t, q[2 * d + base + t]);
        }
        qh[t] = q[base + t] * scale;
    }
    __syncthreads(); // this block's own cache row is visible to its threads
    sa_attend<256, KV>(qh, kc, vc, cbase, base, d, pos + 1, scale, sc, vs, red, &inv_s, att + (size_t)r * d + base,
                   pmax ? pmax + (size_t)r * gridDim.x + h : nullptr);
}

// The k/v of every row of a prefill chunk into the cache (KvCache::append,
// nn.rs:5352-5416: RNE to f16 for an f16 cache), row r = stream r % ns at
// position *posp + r / ns.
template <typename KV>
__global__ void __launch_bounds__(256) k_kv_append(const float *qkv, KV *kc, KV *vc, const int *posp, int d, int nctx,
                                                   int L, int layer, int ns) {
    const int r = blockIdx.x, s = r % ns, pos = *posp + r / ns;
    const float *q = qkv + (size_t)r * 3 * d;
    const size_t o = ((size_t)s * L + layer) * nctx * d + (size_t)pos * d;
    for (int c = threadIdx.x; c < d; c += 256) {
        KvT<KV>::put(kc, o + c, q[d + c]);
        KvT<KV>::put(vc, o + c, q[2 * d + c]);
    }
}

// ---------------------------------------------------------------------------
// The f16 arm's self-attention sublayer for one (head, stream), d == 1280: the
// head's 192 rows of the fused q/k/v projection (gemv_f16, nn.rs:2346-2460,
// bias [q_b | 0 | v_b]) of LN(x_s) (LN: the attention LayerNorm of the
// residual row, wave 0, the GEMV's one-wave arithmetic; else x is the already
// normalized row), then k_self_attn2's attention with this token's k/v
// appended.  The projection runs on the slot-order matrix of
// fw_launch_pack_gemv16 (16 lanes per row): lane p = kh * 8 + l of a row
// group holds the normalized row's values of its two dot_f16c slots
// 8 (2 kh + kk) + l of all 40 chunks in registers, so a 32-row batch (8 waves
// x 4 row groups) is 10 weight loads and 80 FMAs per lane; the six batches
// (q, k, v halves) are double-buffered.  The slot tree and the bias are the
// GEMV's, so q/k/v hold its bits.
//
// EMB (layer 0): the row is first formed as the token embedding
// f16(emb[tok]) + pemb[pos] (embed_tokens, decoder.rs:1323-1385, k_embed_ln's
// arithmetic) and the head-0 block stores it to xo, the residual.
template <bool LN, bool EMB, bool SEQ, typename KV>
__global__ void __launch_bounds__(512) k_self_attn_f16q(const uint16_t *__restrict__ wqkv,
                                                        const float *__restrict__ bqkv, const float *__restrict__ x,
                                                        const float *__restrict__ lnw, const float *__restrict__ lnb,
                                                        KV *kc, KV *vc, float *att, const int *posp,
                                                        int nctx, int L, int layer, float scale,
                                                        const int32_t *__restrict__ tok,
                                                        const uint16_t *__restrict__ emb,
                                                        const float *__restrict__ pemb, float *xo) {
    constexpr int D = XQ_D, NV = D / 256, G = D / 128, NC = D / 32;
    extern __shared__ __align__(16) unsigned char sm4[];
    float *sc = (float *)sm4;                                  // [nctx]
    KV *vs = (KV *)(sm4 + sizeof(float) * ((nctx + 3) & ~3)); // [nctx][64]
    __shared__ __align__(16) float xl[D];
    __shared__ float qkvl[192];
    __shared__ float qh[64];
    __shared__ float red[8];
    __shared__ float inv_s;
    const int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int p = lane & 15, rq = lane >> 4, kh = p >> 3, pl = p & 7;
    const int base = h * 64;
    float4 lv[NV], lw[NV], lb[NV];
    bool lok[NV];
    if (wave == 0) {
        if constexpr (EMB) {
            const uint2 *er = (const uint2 *)(emb + (size_t)tok[s] * D);
            const float4 *pr = (const float4 *)(pemb + (size_t)*posp * D);
#pragma unroll
            for (int k = 0; k < NV; k++) {
                lok[k] = true;
                const uint2 e = er[lane + k * 64];
                const float4 pp = pr[lane + k * 64];
                lv[k] = make_float4(fw_h2f(e.x & 0xffff) + pp.x, fw_h2f(e.x >> 16) + pp.y,
                                    fw_h2f(e.y & 0xffff) + pp.z, fw_h2f(e.y >> 16) + pp.w);
                if (h == 0) ((float4 *)(xo + (size_t)s * D))[lane + k * 64] = lv[k];
            }
        } else {
#pragma unroll
            for (int k = 0; k < NV; k++) {
                lok[k] = true;
                lv[k] = ((const float4 *)(x + (size_t)s * D))[lane + k * 64];
            }
        }
        if constexpr (LN) fw_ln_load_wb<NV>(lok, lnw, lnb, lw, lb, lane);
    }
    // row of batch b for this lane: local row 32 b + 4 wave + rq of the head's
    // 192 (q rows 0-63, k 64-127, v 128-191), global row part * d + base + i
    auto grow = [&](int b) {
        const int r = 32 * b + 4 * wave + rq;
        return (r >> 6) * D + base + (r & 63);
    };
    uint4 wv[2][G];
    auto loadw = [&](int set, int b) {
        const uint4 *wr = (const uint4 *)(wqkv + (size_t)grow(b) * D) + p;
#pragma unroll
        for (int g = 0; g < G; g++) wv[set][g] = wr[g * 16];
    };
    loadw(0, 0);
    loadw(1, 1);
    if (wave == 0) {
        if constexpr (LN) fw_ln_quant_core<NV, SEQ>(lv, lok, lw, lb, xl, D, 0, nullptr, nullptr, lane);
        else {
#pragma unroll
            for (int k = 0; k < NV; k++) ((float4 *)xl)[lane + k * 64] = lv[k];
        }
    }
    __syncthreads();
    float xr[NC][2];
#pragma unroll
    for (int c = 0; c < NC; c++) {
        xr[c][0] = xl[c * 32 + 8 * (2 * kh) + pl];
        xr[c][1] = xl[c * 32 + 8 * (2 * kh + 1) + pl];
    }
    auto rowdot = [&](int set, int b) {
        float a0 = 0.0f, a1 = 0.0f;
#pragma unroll
        for (int g = 0; g < G; g++) {
            const uint32_t u[4] = {wv[set][g].x, wv[set][g].y, wv[set][g].z, wv[set][g].w};
#pragma unroll
            for (int cc = 0; cc < 4; cc++) {
                a0 = __builtin_fmaf(fw_h2f((uint16_t)(u[cc] & 0xffffu)), xr[g * 4 + cc][0], a0);
                a1 = __builtin_fmaf(fw_h2f((uint16_t)(u[cc] >> 16)), xr[g * 4 + cc][1], a1);
            }
        }
        float v = a0 + a1;
        v = v + __shfl_xor(v, 8, 64);
        v = v + __shfl_xor(v, 1, 64);
        v = v + __shfl_xor(v, 2, 64);
        v = v + __shfl_xor(v, 4, 64);
        const int gr = grow(b);
        if (bqkv) v = v + bqkv[gr];
        if (p == 0) qkvl[32 * b + 4 * wave + rq] = v;
    };
#pragma unroll
    for (int b = 0; b < 6; b++) {
        rowdot(b & 1, b);
        if (b + 2 < 6) loadw(b & 1, b + 2);
    }
    __syncthreads();
    const int pos = *posp;
    const size_t cbase = ((size_t)s * L + layer) * nctx * D;
    if (t < 64) {
        KvT<KV>::put(kc, cbase + (size_t)pos * D + base + t, qkvl[64 + t]);
        KvT<KV>::put(vc, cbase + (size_t)pos * D + base + t, qkvl[128 + t]);
        qh[t] = qkvl[t] * scale;
    }
    __threadfence_block();
    __syncthreads(); // this block's own cache row is visible to its threads
    sa_attend<512, KV>(qh, kc, vc, cbase, base, D, pos + 1, scale, sc, vs, red, &inv_s, att + (size_t)s * D + base,
                   nullptr);
}

// ---------------------------------------------------------------------------
// The int8 arm's whole self-attention sublayer for one (head, stream), up to
// the output projection: the attention LayerNorm of stream s's residual row
// (wave 0, k_ln_quant's arithmetic, into LDS), the head's 192 rows of the fused
// q/k/v projection (gemv_i8, nn.rs:3168-3231: exact i32 dots,
// ((f32)acc * s_w) * s_x + b, bias [q_b | 0 | v_b]), then k_self_attn2's
// attention over the f16 cache with this token's k/v appended.  512 threads;
// wave w computes projection rows 24w .. 24w+23 in three 8-row batches (a
// batch never straddles the q/k/v boundary), lane c taking 16-byte chunks c
// and c + 64 of each row (d <= 2048).  The LayerNorm operands are requested
// first and two batches of weight rows right behind them; the third batch is
// requested once the first has been used.
//
// EMB (layer 0): the residual row is the token embedding first (embed_tokens,
// decoder.rs:1323-1385: x = f16(E[tok]) + P[pos], as k_embed_ln), which every
// block forms for its stream and the head-0 block also stores as x.
template <int NV, bool EMB, bool SEQ, typename KV>
__global__ void __launch_bounds__(512) k_self_attn_fused(const int8_t *__restrict__ wqkv, const float *__restrict__ sqkv,
                                                         const float *__restrict__ bqkv, float *x,
                                                         const float *__restrict__ lnw, const float *__restrict__ lnb,
                                                         KV *kc, KV *vc, float *att, const int *posp, int d, int nctx,
                                                         int L, int layer, float scale, float *pmax, const int32_t *tok,
                                                         const uint16_t *emb, const float *pemb) {
    extern __shared__ __align__(16) unsigned char sm3[];
    float *sc = (float *)sm3;                                  // [nctx]
    KV *vs = (KV *)(sm3 + sizeof(float) * ((nctx + 3) & ~3)); // [nctx][64]
    __shared__ float qkvl[192];
    __shared__ float qh[64];
    __shared__ __align__(16) int8_t xql[256 * NV];
    __shared__ float xsl;
    __shared__ float red[8];
    __shared__ float inv_s;
    const int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const int base = h * 64;
    float4 lv[NV], lw[NV], lb[NV];
    bool lok[NV];
    if constexpr (EMB) {
        const uint2 *er = (const uint2 *)(emb + (size_t)tok[s] * d);
        const float4 *pr = (const float4 *)(pemb + (size_t)(*posp) * d);
#pragma unroll
        for (int k = 0; k < NV; k++) {
            lok[k] = lane + k * 64 < (d >> 2);
            const int c = lok[k] ? lane + k * 64 : 0;
            const uint2 e = er[c];
            const float4 p = pr[c];
            lv[k] = make_float4(fw_h2f(e.x & 0xffff) + p.x, fw_h2f(e.x >> 16) + p.y, fw_h2f(e.y & 0xffff) + p.z,
                                fw_h2f(e.y >> 16) + p.w);
        }
    } else {
#pragma unroll
        for (int k = 0; k < NV; k++) {
            lok[k] = lane + k * 64 < (d >> 2);
            lv[k] = ((const float4 *)(x + (size_t)s * d))[lok[k] ? lane + k * 64 : 0];
        }
    }
    fw_ln_load_wb<NV>(lok, lnw, lnb, lw, lb, lane);
    if (d < 0) {
        // never taken: a use outside wave 0's LayerNorm branch, so the compiler
        // issues these loads here, ahead of the weight rows, instead of moving
        // them into that branch behind everything else
#pragma unroll
        for (int k = 0; k < NV; k++) qkvl[k] = lv[k].x + lw[k].y + lb[k].z;
    }
    if constexpr (EMB) {
        if (h == 0 && wave == 0) {
#pragma unroll
            for (int k = 0; k < NV; k++)
                if (lok[k]) ((float4 *)(x + (size_t)s * d))[lane + k * 64] = lv[k];
        }
    }
    const int nq = d >> 4;
    const int qc0 = lane < nq ? lane : 0, qc1 = lane + 64 < nq ? lane + 64 : 0;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    // first global row of batch b of this wave (rows 24w + 8b .. +7 of the 192)
    auto brow = [&](int b) {
        const int r = wv * 24 + 8 * b;
        return (r >> 6) * d + base + (r & 63);
    };
    int4 wa[2][8], wb[2][8];
    auto loadb = [&](int set, int b) {
        const int r0 = brow(b);
#pragma unroll
        for (int rr = 0; rr < 8; rr++) {
            const int8_t *wr = wqkv + (size_t)(r0 + rr) * d;
            wa[set][rr] = *(const int4 *)(wr + qc0 * 16);
            wb[set][rr] = *(const int4 *)(wr + qc1 * 16);
        }
    };
    loadb(0, 0);
    loadb(1, 1);
    // row scales and biases: wave-uniform, scalar loads
    float rsc[3][8], rbi[3][8];
#pragma unroll
    for (int b = 0; b < 3; b++)
#pragma unroll
        for (int rr = 0; rr < 8; rr++) {
            rsc[b][rr] = sqkv[brow(b) + rr];
            rbi[b][rr] = bqkv[brow(b) + rr];
        }
    const int pos = *posp;
    if (wave == 0) fw_ln_quant_core<NV, SEQ>(lv, lok, lw, lb, nullptr, d, 0, xql, &xsl, lane);
    __syncthreads();
    {
        // chunks past the row read as zero
        const int4 xa = lane < nq ? *(const int4 *)(xql + qc0 * 16) : make_int4(0, 0, 0, 0);
        const int4 xb = lane + 64 < nq ? *(const int4 *)(xql + qc1 * 16) : make_int4(0, 0, 0, 0);
        const float sx = xsl;
        auto rows = [&](int set, int b) {
#pragma unroll
            for (int rr = 0; rr < 8; rr++) {
                int acc = 0;
                acc = fw_sdot4(wa[set][rr].x, xa.x, acc);
                acc = fw_sdot4(wa[set][rr].y, xa.y, acc);
                acc = fw_sdot4(wa[set][rr].z, xa.z, acc);
                acc = fw_sdot4(wa[set][rr].w, xa.w, acc);
                acc = fw_sdot4(wb[set][rr].x, xb.x, acc);
                acc = fw_sdot4(wb[set][rr].y, xb.y, acc);
                acc = fw_sdot4(wb[set][rr].z, xb.z, acc);
                acc = fw_sdot4(wb[set][rr].w, xb.w, acc);
                acc = fw_dpp_wave_sum_i32(acc);
                if (lane == 0) qkvl[wv * 24 + 8 * b + rr] = (float)acc * rsc[b][rr] * sx + rbi[b][rr];
            }
        };
        rows(0, 0);
        loadb(0, 2);
        rows(1, 1);
        rows(0, 2);
    }
    __syncthreads();
    const size_t cbase = ((size_t)s * L + layer) * nctx * d;
    if (t < 64) {
        KvT<KV>::put(kc, cbase + (size_t)pos * d + base + t, qkvl[64 + t]);
        KvT<KV>::put(vc, cbase + (size_t)pos * d + base + t, qkvl[128 + t]);
        qh[t] = qkvl[t] * scale;
    }
    __syncthreads(); // this block's own cache row is visible to its threads
    constexpr int KW = SaRow<KV>::KW, EPC = SaRow<KV>::EPC;
    const int tk = pos + 1;
    // stage V rows [0, tk) of this head (KW x 16 bytes per row), loads issued
    // before the LDS stores
    for (int c0 = 0; c0 < tk * KW; c0 += 512 * 2) {
        uint4 v[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            int c = c0 + t + u * 512;
            int cc = c < tk * KW ? c : tk * KW - 1;
            v[u] = *(const uint4 *)(vc + cbase + (size_t)((unsigned)cc / KW) * d + base + ((unsigned)cc % KW) * EPC);
        }
#pragma unroll
        for (int u = 0; u < 2; u++) {
            int c = c0 + t + u * 512;
            if (c < tk * KW) ((uint4 *)vs)[c] = v[u];
        }
    }
    float mx = -INFINITY;
    for (int j = t; j < tk; j += 512) {
        const uint4 *kr = (const uint4 *)(kc + cbase + (size_t)j * d + base);
        uint4 kk[KW];
#pragma unroll
        for (int c = 0; c < KW; c++) kk[c] = kr[c];
        const float acc = sa_score<KV>(qh, kk, scale);
        sc[j] = acc;
        mx = fmaxf(mx, acc);
    }
    mx = fw_block_max(mx, red);
    const bool fin = isfinite(mx);
    if (fin)
        for (int j = t; j < tk; j += 512) {
            float e = fw_expf(sc[j] - mx);
            sc[j] = isfinite(e) ? e : 0.0f;
        }
    __syncthreads();
    if (t == 0) inv_s = fin ? fw_seq_sum_inv(sc, tk) : 0.0f;
    __syncthreads();
    const float inv = inv_s;
    if (inv > 0.0f)
        for (int j = t; j < tk; j += 512) sc[j] = sc[j] * inv;
    __syncthreads();
    if (t < 64) {
        const float acc = fw_pv_chain(sc, vs, tk, t);
        att[(size_t)s * d + base + t] = acc;
        // this head's share of the row amax the int8 consumer needs
        const float m = fw_dpp_wave_max(fabsf(acc));
        if (pmax && t == 0) pmax[(size_t)s * gridDim.x + h] = m;
    }
}

// ---------------------------------------------------------------------------
// Cross-attention for one (head, stream) with int8 K/V (cross_attention,
// decoder.rs:1524-1716, int8 cross K/V — the default), including the head's
// rows of the cross q projection: q = gemv_i8(Wq_h, xq) (+ bias); qh = q*s
// quantized per vector; scores = gemv_i8(K_h, qh); softmax; p quantized per
// vector; out = gemv_i8(Vt_h, p).  512 threads.  Vt rows have stride Tq (T
// rounded up to 16, zero padded).
//
// The register operands are requested at entry, in the order they are
// consumed, so each phase waits only for its own (vector memory returns in
// order): the LayerNorm row, weight and bias; the head's 64 q-projection rows;
// the keys (CA_KPT per thread).  The head's Vt rows go straight into LDS (64 x
// Tq bytes, global -> LDS without registers), issued by waves 1-7 while wave 0
// forms the softmax's sequential sum (fw_seq_sum_wave).
#define CA_KPT 3
#define CA_VKB 16 // 1 KB Vt loads per wave (7 waves): 64 * ca_vstride(Tq) <= 7 * CA_VKB KB
// LDS row stride of the staged Vt rows: Tq rounded up to 16 mod 256
__host__ __device__ __forceinline__ int ca_vstride(int Tq) { return Tq + ((16 - Tq % 256) + 256) % 256; }
// Block barrier for LDS data (a plain barrier: __syncthreads would also wait
// for the global -> LDS loads still in flight)
#define CA_SYNC()                                                                                  \
    do {                                                                                           \
        FW_WAIT_LGKM0();                                                                           \
        asm volatile("s_barrier" ::: "memory");                                                    \
    } while (0)
//
// VB (FW_CROSS_V_BLOCK, decoder.rs:1605-1608): cvt holds the block-int8 V^T
// (32-frame blocks, scales vbs [.., 64, nb]) and the value pass is
// gemv_i8w_f32a_blocked (nn.rs:3756-3824) on the f32 softmax weights: no p
// quantization; per output dim the blocks' dot_i8w_f32 (nn.rs:3479-3564)
// times their scale, summed in block order.
template <int NV, bool SEQ, bool VB = false>
__global__ void __launch_bounds__(512) k_cross_attn_i8v2(const int8_t *__restrict__ wq, const float *__restrict__ swq,
                                                         const float *__restrict__ bq, const float *__restrict__ x,
                                                         const float *__restrict__ lnw, const float *__restrict__ lnb,
                                                         const int8_t *ck, const float *cks, const int8_t *cvt,
                                                         const float *cvs, float *att, int d, int T, int Tq, int H,
                                                         int L, int layer, float scale, float *pmax,
                                                         const float *vbs, int nb) {
    extern __shared__ __align__(16) unsigned char smc2[];
    const int vst = ca_vstride(Tq);                                               // LDS row stride of Vt
    int8_t *vl = (int8_t *)smc2;                                                  // [64, vst]
    float *sc = (float *)(smc2 + (size_t)64 * vst);                               // [T]
    int8_t *p8 = (int8_t *)(smc2 + (size_t)64 * vst + sizeof(float) * ((T + 3) & ~3)); // [Tq]
    __shared__ __align__(16) int8_t q8[64];
    __shared__ float red[16];
    __shared__ float bc[2];
    const int h = blockIdx.x, s = blockIdx.y, t = threadIdx.x;
    const int lane = t & 63, wave = t >> 6;
    const size_t lh = ((size_t)s * L + layer) * H + h;
    const int8_t *Kp = ck + lh * (size_t)T * 64;
    const float *Ks = cks + lh * T;
    const int8_t *Vp = cvt + lh * (size_t)Tq * 64;
    const float *Vs = cvs + lh * 64;
    const int nch = Tq >> 4;
    // The cross LayerNorm of stream s's residual row (wave 0, k_ln_quant's
    // arithmetic, into LDS), then this head's 64 rows of the cross q
    // projection (gemv_i8, nn.rs:3168-3231: exact i32 dots,
    // ((f32)acc * s_w) * s_x + b), 8 rows per wave, lane c taking 16-byte
    // chunks c and c + 64 of the row (d <= 2048).
    __shared__ float qf[64];
    __shared__ __align__(16) int8_t xql[256 * NV];
    __shared__ float xsl;
    float4 lv[NV], lw[NV], lb[NV];
    bool lok[NV];
#pragma unroll
    for (int k = 0; k < NV; k++) {
        lok[k] = lane + k * 64 < (d >> 2);
        lv[k] = ((const float4 *)(x + (size_t)s * d))[lok[k] ? lane + k * 64 : 0];
    }
    fw_ln_load_wb<NV>(lok, lnw, lnb, lw, lb, lane);
    if (d < 0) {
        // never taken: a use outside wave 0's LayerNorm branch, so the compiler
        // issues these loads here, ahead of the other operands, instead of
        // moving them into that branch behind everything else
#pragma unroll
        for (int k = 0; k < NV; k++) qf[k] = lv[k].x + lw[k].y + lb[k].z;
    }
    const int nq = d >> 4;
    const int qc0 = lane < nq ? lane : 0, qc1 = lane + 64 < nq ? lane + 64 : 0;
    int4 wa[8], wb[8];
#pragma unroll
    for (int rr = 0; rr < 8; rr++) {
        const int8_t *wr = wq + (size_t)(h * 64 + wave * 8 + rr) * d;
        wa[rr] = *(const int4 *)(wr + qc0 * 16);
        wb[rr] = *(const int4 *)(wr + qc1 * 16);
    }
    // per-row scales and biases are wave-uniform: scalar loads, which leave the
    // vector-memory count (at most 63 outstanding) to the operands above and below
    const float *bqp = bq ? bq : swq; // unconditional loads; the bias is added only when present
    const int wrow0 = h * 64 + __builtin_amdgcn_readfirstlane(wave) * 8;
    float qsw[8], qb[8];
#pragma unroll
    for (int rr = 0; rr < 8; rr++) {
        qsw[rr] = swq[wrow0 + rr];
        qb[rr] = bqp[wrow0 + rr];
    }
    int4 kr[CA_KPT][4];
    float ksc[CA_KPT];
#pragma unroll
    for (int u = 0; u < CA_KPT; u++) {
        const int j = t + u * 512;
        const int jc = j < T ? j : T - 1; // clamped: unconditional loads
        const int4 *kp = (const int4 *)(Kp + (size_t)jc * 64);
#pragma unroll
        for (int c = 0; c < 4; c++) kr[u][c] = kp[c];
        ksc[u] = Ks[jc];
    }
    if (wave == 0) fw_ln_quant_core<NV, SEQ>(lv, lok, lw, lb, nullptr, d, 0, xql, &xsl, lane);
    CA_SYNC();
    {
        // chunks past the row read as zero
        const int4 xa = lane < nq ? *(const int4 *)(xql + qc0 * 16) : make_int4(0, 0, 0, 0);
        const int4 xb = lane + 64 < nq ? *(const int4 *)(xql + qc1 * 16) : make_int4(0, 0, 0, 0);
        const float sx = xsl;
#pragma unroll
        for (int rr = 0; rr < 8; rr++) {
            int acc = 0;
            acc = fw_sdot4(wa[rr].x, xa.x, acc);
            acc = fw_sdot4(wa[rr].y, xa.y, acc);
            acc = fw_sdot4(wa[rr].z, xa.z, acc);
            acc = fw_sdot4(wa[rr].w, xa.w, acc);
            acc = fw_sdot4(wb[rr].x, xb.x, acc);
            acc = fw_sdot4(wb[rr].y, xb.y, acc);
            acc = fw_sdot4(wb[rr].z, xb.z, acc);
            acc = fw_sdot4(wb[rr].w, xb.w, acc);
            acc = fw_dpp_wave_sum_i32(acc);
            if (lane == 0) {
                float q = (float)acc * qsw[rr] * sx;
                if (bq) q = q + qb[rr];
                qf[wave * 8 + rr] = q;
            }
        }
    }
    CA_SYNC();
    if (wave == 0) {
        float v = qf[lane] * scale;
        float m = fw_dpp_wave_max(fabsf(v));
        float xs = fmaxf(m, 1e-9f) / 127.0f;
        q8[lane] = fw_q8_avx(v, 1.0f / xs, lane, 64);
        if (lane == 0) bc[0] = xs;
    }
    CA_SYNC();
    const float xs = bc[0];
    const int *qw = (const int *)q8;
    float mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < CA_KPT; u++) {
        const int j = t + u * 512;
        if (j < T) {
            int acc = 0;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                acc = fw_sdot4(kr[u][c].x, qw[4 * c + 0], acc);
                acc = fw_sdot4(kr[u][c].y, qw[4 * c + 1], acc);
                acc = fw_sdot4(kr[u][c].z, qw[4 * c + 2], acc);
                acc = fw_sdot4(kr[u][c].w, qw[4 * c + 3], acc);
            }
            float v = (float)acc * ksc[u] * xs + 0.0f;
            sc[j] = v;
            mx = fmaxf(mx, v);
        }
    }
    // keys beyond the prefetched range (T > CA_KPT * 512)
    for (int j = t + CA_KPT * 512; j < T; j += 512) {
        const int4 *kp = (const int4 *)(Kp + (size_t)j * 64);
        int acc = 0;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            int4 kv = kp[c];
            acc = fw_sdot4(kv.x, qw[4 * c + 0], acc);
            acc = fw_sdot4(kv.y, qw[4 * c + 1], acc);
            acc = fw_sdot4(kv.z, qw[4 * c + 2], acc);
            acc = fw_sdot4(kv.w, qw[4 * c + 3], acc);
        }
        float v = (float)acc * Ks[j] * xs + 0.0f;
        sc[j] = v;
        mx = fmaxf(mx, v);
    }
    mx = fw_dpp_wave_max(mx);
    if (lane == 0) red[wave] = mx;
    CA_SYNC();
    mx = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7])));
    const bool fin = isfinite(mx);
    // exp pass; am = max |stored value| (the exps, or the raw scores when the
    // max is not finite and softmax leaves them as they are)
    float am = 0.0f;
    for (int j = t; j < T; j += 512) {
        float v = sc[j];
        if (fin) {
            const float e = fw_expf(v - mx);
            v = isfinite(e) ? e : 0.0f;
            sc[j] = v;
        }
        am = fmaxf(am, fabsf(v));
    }
    am = fw_dpp_wave_max(am);
    if (lane == 0) red[8 + wave] = am;
    CA_SYNC();
    if (wave == 0) {
        // softmax_rows' sequential sum (nn.rs:4880-4963), T <= 64 * SW_MAXC
        const float sum = fin ? fw_seq_sum_wave(sc, T) : 0.0f;
        if (t == 0) bc[1] = sum > 0.0f ? 1.0f / sum : 0.0f;
    } else {
        // meanwhile waves 1-7 bring the head's Vt rows into LDS rows of stride
        // vst, 1 KB of LDS per wave instruction: lane slot (row, col) takes
        // Vt[row, col], pad slots (col >= Tq) an in-bounds dummy; the tail
        // rewrites the last KB with the same bytes.  The loads are non-temporal
        // (read once per step): the step's weights then stay in the last-level
        // cache (measured: logits 23 -> 20 us, cross attention 17.4 -> 16.1 us).
        const int nkb = (64 * vst + 1023) >> 10;
#pragma unroll
        for (int u = 0; u < CA_VKB; u++) {
            const int kb = (wave - 1) + 7 * u, kc = kb < nkb ? kb : nkb - 1;
            const int off = kc * 1024 + lane * 16, row = off / vst, col = off - row * vst;
            const int8_t *src = row < 64 && col < Tq ? Vp + (size_t)row * Tq + col : Vp;
            __builtin_amdgcn_global_load_lds((const void *)src,
                                             (void __attribute__((address_space(3))) *)(vl + (size_t)kc * 1024), 16,
                                             0, 2);
        }
        FW_WAIT_VM(0);
    }
    CA_SYNC();
    const float inv = bc[1];
    if constexpr (VB) {
        // p_j = e_j * inv as softmax_rows leaves it (the raw scores when the
        // maximum is not finite); block dots (dim dd, block b) over the 512
        // threads into LDS, then one lane per dim sums its blocks in order
        float *bd = (float *)(smc2 + (((size_t)64 * vst + sizeof(float) * ((T + 3) & ~3) + Tq + 15) & ~(size_t)15));
        const float *Vbs = vbs + lh * 64 * nb;
        auto pj = [&](int j) { return inv > 0.0f ? sc[j] * inv : sc[j]; };
        for (int i = t; i < 64 * nb; i += 512) {
            const int dd = i / nb, b = i - dd * nb, j0 = b * 32, n = T - j0 < 32 ? T - j0 : 32;
            const int8_t *vr = vl + (size_t)dd * vst + j0;
            float sd;
            if (n == 32) {
                // one 32-wide step: four 8-lane accumulators from +0, then
                // (a0 + a1) + (a2 + a3) per lane and the lanes' tree
                float tt[8];
#pragma unroll
                for (int l = 0; l < 8; l++) {
                    const float a0 = __builtin_fmaf((float)vr[l], pj(j0 + l), 0.0f);
                    const float a1 = __builtin_fmaf((float)vr[8 + l], pj(j0 + 8 + l), 0.0f);
                    const float a2 = __builtin_fmaf((float)vr[16 + l], pj(j0 + 16 + l), 0.0f);
                    const float a3 = __builtin_fmaf((float)vr[24 + l], pj(j0 + 24 + l), 0.0f);
                    tt[l] = (a0 + a1) + (a2 + a3);
                }
                sd = ((tt[0] + tt[1]) + (tt[2] + tt[3])) + ((tt[4] + tt[5]) + (tt[6] + tt[7]));
            } else {
                // the last, short block: 8-wide product trees, then scalars
                sd = 0.0f;
                int i8 = 0;
                for (; i8 + 8 <= n; i8 += 8) {
                    float pp[8];
#pragma unroll
                    for (int l = 0; l < 8; l++) pp[l] = (float)vr[i8 + l] * pj(j0 + i8 + l);
                    sd += ((pp[0] + pp[1]) + (pp[2] + pp[3])) + ((pp[4] + pp[5]) + (pp[6] + pp[7]));
                }
                for (; i8 < n; i8++) sd += (float)vr[i8] * pj(j0 + i8);
            }
            bd[i] = sd * Vbs[i];
        }
        CA_SYNC();
        float om = 0.0f;
        if (wave == 0) {
            float acc = 0.0f;
            for (int b = 0; b < nb; b++) acc += bd[lane * nb + b];
            const float o = acc + 0.0f;
            att[(size_t)s * d + h * 64 + lane] = o;
            om = fw_dpp_wave_max(fabsf(o));
        }
        if (pmax && t == 0) pmax[(size_t)s * H + h] = om;
        return;
    }
    am = fmaxf(fmaxf(fmaxf(red[8], red[9]), fmaxf(red[10], red[11])),
               fmaxf(fmaxf(red[12], red[13]), fmaxf(red[14], red[15])));
    // max_j |p_j| of p_j = e_j * inv: rounding is monotonic and sign-symmetric,
    // so it is (max_j |e_j|) * inv rounded once
    const float pm = inv > 0.0f ? am * inv : am;
    const float ps = fmaxf(pm, 1e-9f) / 127.0f;
    const float pinv = 1.0f / ps;
    for (int j = t; j < Tq; j += 512) {
        int8_t q = 0;
        if (j < T) {
            const float p = inv > 0.0f ? sc[j] * inv : sc[j];
            q = fw_q8_avx(p, pinv, j, T);
        }
        p8[j] = q;
    }
    CA_SYNC();
    // out[dd] = sum_j Vt[dd, j] * p8[j] (exact i32 in any order): lane dd owns
    // row dd, wave w the 16-byte chunks w, w + 8, ...  The row stride vst is 16
    // mod 256, so the 16 lanes of a read group hit 16 different bank groups, and
    // the p8 chunk is one broadcast address.  Partial sums meet in LDS.
    __shared__ int pvp[8][64];
    {
        int acc = 0;
        for (int ck = wave; ck < nch; ck += 8) {
            const int4 vv = *(const int4 *)(vl + (size_t)lane * vst + ck * 16);
            const int4 q4 = *(const int4 *)(p8 + ck * 16);
            acc = fw_sdot4(vv.x, q4.x, acc);
            acc = fw_sdot4(vv.y, q4.y, acc);
            acc = fw_sdot4(vv.z, q4.z, acc);
            acc = fw_sdot4(vv.w, q4.w, acc);
        }
        pvp[wave][lane] = acc;
    }
    CA_SYNC();
    float om = 0.0f; // max |out| over the head's 64 rows (wave 0)
    if (wave == 0) {
        int acc = 0;
#pragma unroll
        for (int w = 0; w < 8; w++) acc += pvp[w][lane];
        const float o = (float)acc * Vs[lane] * ps + 0.0f;
        att[(size_t)s * d + h * 64 + lane] = o;
        om = fw_dpp_wave_max(fabsf(o));
    }
    if (pmax && t == 0) pmax[(size_t)s * H + h] = om;
}

// Per-row int8 quantization of f16 rows into a row stride ldq >= n (zero
// padded; quantize_f16_row_to_i8_into, nn.rs:2490-2555).  One 64-thread block
// per row.
__global__ void __launch_bounds__(64) k_quant_f16_rows_ld(const uint16_t *src, int8_t *q, float *s, int n, int ldq) {
    size_t r = blockIdx.x;
    const uint16_t *row = src + r * n;
    float m = 0.0f;
    for (int i = threadIdx.x; i < n; i += 64) m = fmaxf(m, fabsf(fw_h2f(row[i])));
    m = fw_wave_max(m);
    float sc = fmaxf(m, 1e-9f) / 127.0f;
    float inv = 1.0f / sc;
    for (int i = threadIdx.x; i < ldq; i += 64) q[r * ldq + i] = i < n ? fw_q8_avx(fw_h2f(row[i]), inv, i, n) : 0;
    if (threadIdx.x == 0) s[r] = sc;
}

// ---------------------------------------------------------------------------
// launch wrappers
// Row kernels hold ceil(d/256) float4 groups per lane; d % 4 == 0 and
// d <= 2048 are checked when the decoder is loaded.
#define FW_ROWS_DISPATCH1(KERNEL, SEQ, d, ...)                                                     \
    switch ((d + 255) / 256) {                                                                      \
    case 1: hipLaunchKernelGGL((KERNEL<1, SEQ>), __VA_ARGS__); break;                               \
    case 2: hipLaunchKernelGGL((KERNEL<2, SEQ>), __VA_ARGS__); break;                               \
    case 3: hipLaunchKernelGGL((KERNEL<3, SEQ>), __VA_ARGS__); break;                               \
    case 4: hipLaunchKernelGGL((KERNEL<4, SEQ>), __VA_ARGS__); break;                               \
    case 5: hipLaunchKernelGGL((KERNEL<5, SEQ>), __VA_ARGS__); break;                               \
    case 6: hipLaunchKernelGGL((KERNEL<6, SEQ>), __VA_ARGS__); break;                               \
    case 7: hipLaunchKernelGGL((KERNEL<7, SEQ>), __VA_ARGS__); break;                               \
    default: hipLaunchKernelGGL((KERNEL<8, SEQ>), __VA_ARGS__); break;                              \
    }
// KERNEL<rows of d floats, SEQ = seq != 0>
#define FW_ROWS_DISPATCH(KERNEL, seq, d, ...)                                                      \
    do {                                                                                            \
        if (seq) {                                                                                  \
            FW_ROWS_DISPATCH1(KERNEL, true, d, __VA_ARGS__)                                         \
        } else {                                                                                    \
            FW_ROWS_DISPATCH1(KERNEL, false, d, __VA_ARGS__)                                        \
        }                                                                                           \
    } while (0)

// (seq: one row per block, so that the rows' sequential sums, bound by their
// LDS reads, each have a CU's LDS to themselves)
void fw_launch_ln_quant(hipStream_t st, const float *x, float *y, const float *w, const float *b, int d, int rows,
                        int8_t *xq, float *xs, int seq) {
    if (seq) FW_ROWS_DISPATCH1(k_ln_quant, true, d, dim3(rows), dim3(64), 0, st, x, y, w, b, d, rows, xq, xs)
    else FW_ROWS_DISPATCH1(k_ln_quant, false, d, dim3((rows + 3) / 4), dim3(256), 0, st, x, y, w, b, d, rows, xq, xs)
}

void fw_launch_embed_ln(hipStream_t st, const int32_t *tok, const int *posp, const uint16_t *emb, const float *pemb,
                        float *x, int d, int ns, const float *w, const float *b, float *ln_y, int8_t *xq, float *xs,
                        int rps, int seq) {
    FW_ROWS_DISPATCH(k_embed_ln, seq, d, dim3(ns), dim3(64), 0, st, tok, posp, emb, pemb, x, d, w, b, ln_y, xq, xs,
                     rps > 0 ? rps : ns);
}

int fw_gemv_i8m_blocks(int N) { return N >= 16384 ? (N + 63) / 64 : (N + 15) / 16; }

// Row-major [N, K] int8 -> the GEMV's fragment order, one 16-byte piece per
// thread (rows past N written as zero).
__global__ void __launch_bounds__(256) k_pack_gemv_frags(const int8_t *W, int8_t *Wf, int N, int K, size_t npieces) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= npieces) return;
    const int nkb = K >> 6, l = (int)(i & 63);
    const size_t f = i >> 6;
    const int kb = (int)(f % nkb), rg = (int)(f / nkb);
    const int row = rg * 16 + (l & 15), k = kb * 64 + (l >> 4) * 16;
    v4i v = (v4i){0, 0, 0, 0};
    if (row < N) v = *(const v4i *)(W + (size_t)row * K + k);
    *(v4i *)(Wf + i * 16) = v;
}
size_t fw_gemv_frag_bytes(int N, int K) { return (size_t)((N + 15) / 16) * 16 * K; }
void fw_launch_pack_gemv_frags(hipStream_t st, const int8_t *W, int8_t *Wf, int N, int K) {
    const size_t np = fw_gemv_frag_bytes(N, K) / 16;
    hipLaunchKernelGGL(k_pack_gemv_frags, dim3((unsigned)((np + 255) / 256)), dim3(256), 0, st, W, Wf, N, K, np);
}

void fw_launch_gemv_i8m(hipStream_t st, const int8_t *W, const float *sw, const float *bias, const int8_t *xq,
                        const float *xs, float *y, int N, int K, int ns, int ldy, int mode, const float *gelu_tab,
                        const fwhip_filter *filt, const int *initialp, unsigned long long *keys, const float *xf,
                        const float *pmax, int H) {
    fwhip_filter ff;
    int use = filt != nullptr;
    if (filt) ff = *filt;
    else memset(&ff, 0, sizeof ff);
    int nblk = fw_gemv_i8m_blocks(N);
#define GV_ARGS dim3(nblk), dim3(256), 0, st, W, sw, bias, xq, xs, y, N, K, ns, ldy, mode, gelu_tab, ff, use, initialp, \
                keys, xf, pmax, H
    if (xf) hipLaunchKernelGGL((k_gemv_i8m<1, 1>), GV_ARGS);
    else if (N >= 16384) hipLaunchKernelGGL((k_gemv_i8m<4, 0>), GV_ARGS);
    else hipLaunchKernelGGL((k_gemv_i8m<1, 0>), GV_ARGS);
#undef GV_ARGS
}

// The same argmax and bookkeeping with one block per stream: every key is
// requested at entry (clamped addresses: a repeated key leaves the maximum
// unchanged), so the stream's keys cost one round trip instead of a dependent
// walk.  The block that counts last (cnt, zero between launches) advances the
// position, clears initial and the step counter; every block has read the
// step before it counts.
#define AM_U 16
__global__ void __launch_bounds__(256) k_argmax_rows(const unsigned long long *keys, int nblk, int ns, int32_t *tok,
                                                     int32_t *hist, int hist_cap, int *posp, int *initialp,
                                                     int *stepp, int advance, int *cnt) {
    __shared__ unsigned long long red[4];
    const int s = blockIdx.x, t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int step = stepp ? *stepp : 0;
    const unsigned long long *ks = keys + (size_t)s * nblk;
    unsigned long long kv[AM_U];
#pragma unroll
    for (int u = 0; u < AM_U; u++) kv[u] = ks[min(t + u * 256, nblk - 1)];
    unsigned long long k = 0ull;
#pragma unroll
    for (int u = 0; u < AM_U; u++) k = kv[u] > k ? kv[u] : k;
    k = wave_max_u64(k);
    if (lane == 0) red[wave] = k;
    __syncthreads();
    if (t == 0) {
#pragma unroll
        for (int w = 1; w < 4; w++) k = red[w] > k ? red[w] : k;
        const int tk = k ? (int)(0xffffffffu - (uint32_t)(k & 0xffffffffull)) : 0;
        tok[s] = tk;
        if (hist) hist[(size_t)s * hist_cap + step] = tk;
        if (atomicAdd(cnt, 1) == ns - 1) {
            if (advance) *posp = *posp + 1;
            if (initialp) *initialp = 0;
            if (stepp) *stepp = step + 1;
            *cnt = 0;
        }
    }
}

void fw_launch_argmax_finish(hipStream_t st, const unsigned long long *keys, int nblk, int ns, int32_t *tok,
                             int32_t *hist, int hist_cap, int *posp, int *initialp, int *stepp, int advance,
                             int *cnt) {
    if (cnt && nblk > 0 && nblk <= 256 * AM_U)
        hipLaunchKernelGGL(k_argmax_rows, dim3(ns), dim3(256), 0, st, keys, nblk, ns, tok, hist, hist_cap, posp,
                           initialp, stepp, advance, cnt);
    else
        hipLaunchKernelGGL(k_argmax_finish, dim3(1), dim3(1024), 0, st, keys, nblk, ns, tok, hist, hist_cap, posp,
                           initialp, stepp, advance);
}

// Streams go in chunks of SG * floor(512 / nb) (one (block, group) pair per
// thread).  x is block-interleaved (fw_blk_perm).
int fw_launch_gemv_blk2(hipStream_t st, const int8_t *W, const float *sc, const float *bias, const float *x, float *y,
                        int N, int K, int ns, int ldy, int mode, int n_cu) {
    constexpr int SG = 4;
    const int nb = K >> 5, ldp = nb + 4;
    if ((K & 31) || nb > 512) return -1;
    const int chunk = SG * (512 / nb);
    for (int s0 = 0; s0 < ns; s0 += chunk) {
        const int n = ns - s0 < chunk ? ns - s0 : chunk;
        int R = (N + n_cu - 1) / n_cu;
        const int rmax = (64 * 1024) / (int)(sizeof(float) * n * ldp);
        if (R > rmax) R = rmax;
        if (R < 1) return -1;
        const int nsg = (n + SG - 1) / SG;
        const int threads = ((nb * nsg + 63) / 64) * 64;
        const size_t shm = sizeof(float) * (size_t)R * n * ldp;
        hipLaunchKernelGGL(k_gemv_blk7<SG>, dim3((N + R - 1) / R), dim3(threads), shm, st, W, sc, bias,
                           x + (size_t)s0 * K, y + (size_t)s0 * ldy, N, K, n, ldy, mode, R);
    }
    return 0;
}

// LDS of the self-attention blocks: the scores [nctx] and the head's V rows [nctx][64]
static size_t sa_shm(int nctx, int kv32) {
    return sizeof(float) * (size_t)((nctx + 3) & ~3) + (kv32 ? 4 : 2) * 64 * (size_t)nctx;
}

void fw_launch_self_attn2(hipStream_t st, const float *qkv, void *kc, void *vc, float *att, const int *posp, int d,
                          int H, int nctx, int L, int layer, int ns, float scale, float *pmax, int rows, int append,
                          int kv32) {
    const dim3 g(H, rows > 0 ? rows : ns);
    if (kv32)
        hipLaunchKernelGGL(k_self_attn2<float>, g, dim3(256), sa_shm(nctx, 1), st, qkv, (float *)kc, (float *)vc, att,
                           posp, d, nctx, L, layer, scale, pmax, ns, append);
    else
        hipLaunchKernelGGL(k_self_attn2<uint16_t>, g, dim3(256), sa_shm(nctx, 0), st, qkv, (uint16_t *)kc,
                           (uint16_t *)vc, att, posp, d, nctx, L, layer, scale, pmax, ns, append);
}

void fw_launch_kv_append(hipStream_t st, const float *qkv, void *kc, void *vc, const int *posp, int d, int nctx,
                         int L, int layer, int ns, int rows, int kv32) {
    if (kv32)
        hipLaunchKernelGGL(k_kv_append<float>, dim3(rows), dim3(256), 0, st, qkv, (float *)kc, (float *)vc, posp, d,
                           nctx, L, layer, ns);
    else
        hipLaunchKernelGGL(k_kv_append<uint16_t>, dim3(rows), dim3(256), 0, st, qkv, (uint16_t *)kc, (uint16_t *)vc,
                           posp, d, nctx, L, layer, ns);
}

bool fw_self_attn_f16q_ok(int d, int H) { return d == XQ_D && H * 64 == d; }

// q/k/v projection (wqkv in fw_launch_pack_gemv16's slot order at 16 lanes per
// row, bias bqkv) of LN(x) (or of x itself when lnw is null: an already
// normalized row) and the self-attention of k_self_attn2, one launch
template <typename KV>
static void launch_self_attn_f16q(hipStream_t st, const uint16_t *wqkv, const float *bqkv, const float *x,
                                  const float *lnw, const float *lnb, KV *kc, KV *vc, float *att, const int *posp,
                                  int H, int nctx, int L, int layer, int ns, float scale, const int32_t *tok,
                                  const uint16_t *emb, const float *pemb, float *xo, int lnseq) {
    const size_t shm = sa_shm(nctx, sizeof(KV) == 4);
#define SAQ(LN_, EMB_, SEQ_, ...)                                                                                     \
    hipLaunchKernelGGL((k_self_attn_f16q<LN_, EMB_, SEQ_, KV>), dim3(H, ns), dim3(512), shm, st, wqkv, bqkv, x, lnw,   \
                       lnb, kc, vc, att, posp, nctx, L, layer, scale, __VA_ARGS__)
    if (tok && lnseq) SAQ(true, true, true, tok, emb, pemb, xo);
    else if (tok) SAQ(true, true, false, tok, emb, pemb, xo);
    else if (lnw && lnseq) SAQ(true, false, true, nullptr, nullptr, nullptr, nullptr);
    else if (lnw) SAQ(true, false, false, nullptr, nullptr, nullptr, nullptr);
    else SAQ(false, false, false, nullptr, nullptr, nullptr, nullptr);
#undef SAQ
}

void fw_launch_self_attn_f16q(hipStream_t st, const uint16_t *wqkv, const float *bqkv, const float *x,
                              const float *lnw, const float *lnb, void *kc, void *vc, float *att,
                              const int *posp, int H, int nctx, int L, int layer, int ns, float scale,
                              const int32_t *tok, const uint16_t *emb, const float *pemb, float *xo, int lnseq,
                              int kv32) {
    if (kv32)
        launch_self_attn_f16q(st, wqkv, bqkv, x, lnw, lnb, (float *)kc, (float *)vc, att, posp, H, nctx, L, layer, ns,
                              scale, tok, emb, pemb, xo, lnseq);
    else
        launch_self_attn_f16q(st, wqkv, bqkv, x, lnw, lnb, (uint16_t *)kc, (uint16_t *)vc, att, posp, H, nctx, L,
                              layer, ns, scale, tok, emb, pemb, xo, lnseq);
}

template <int NV, typename KV>
using k_self_attn_fused_e = void (*)(const int8_t *, const float *, const float *, float *, const float *,
                                     const float *, KV *, KV *, float *, const int *, int, int, int, int, float,
                                     float *, const int32_t *, const uint16_t *, const float *);
template <int NV, typename KV>
static void launch_self_attn_fused_t(hipStream_t st, bool embed, dim3 grid, const int8_t *wqkv, const float *sqkv,
                                     const float *bqkv, float *x, const float *lnw, const float *lnb, KV *kc, KV *vc,
                                     float *att, const int *posp, int d, int nctx, int L, int layer, float scale,
                                     float *pmax, const int32_t *tok, const uint16_t *emb, const float *pemb,
                                     int lnseq) {
    const k_self_attn_fused_e<NV, KV> k = embed ? (lnseq ? k_self_attn_fused<NV, true, true, KV>
                                                         : k_self_attn_fused<NV, true, false, KV>)
                                                : (lnseq ? k_self_attn_fused<NV, false, true, KV>
                                                         : k_self_attn_fused<NV, false, false, KV>);
    hipLaunchKernelGGL(k, grid, dim3(512), sa_shm(nctx, sizeof(KV) == 4), st, wqkv, sqkv, bqkv, x, lnw, lnb, kc, vc,
                       att, posp, d, nctx, L, layer, scale, pmax, tok, emb, pemb);
}
template <int NV>
static void launch_self_attn_fused(hipStream_t st, bool embed, dim3 grid, int kv32, const int8_t *wqkv,
                                   const float *sqkv, const float *bqkv, float *x, const float *lnw,
                                   const float *lnb, void *kc, void *vc, float *att, const int *posp, int d,
                                   int nctx, int L, int layer, float scale, float *pmax, const int32_t *tok,
                                   const uint16_t *emb, const float *pemb, int lnseq) {
    if (kv32)
        launch_self_attn_fused_t<NV, float>(st, embed, grid, wqkv, sqkv, bqkv, x, lnw, lnb, (float *)kc, (float *)vc,
                                            att, posp, d, nctx, L, layer, scale, pmax, tok, emb, pemb, lnseq);
    else
        launch_self_attn_fused_t<NV, uint16_t>(st, embed, grid, wqkv, sqkv, bqkv, x, lnw, lnb, (uint16_t *)kc,
                                               (uint16_t *)vc, att, posp, d, nctx, L, layer, scale, pmax, tok, emb,
                                               pemb, lnseq);
}

void fw_launch_self_attn_fused(hipStream_t st, const int8_t *wqkv, const float *sqkv, const float *bqkv, float *x,
                               const float *lnw, const float *lnb, void *kc, void *vc, float *att,
                               const int *posp, int d, int H, int nctx, int L, int layer, int ns, float scale,
                               float *pmax, const int32_t *tok, const uint16_t *emb, const float *pemb, int lnseq,
                               int kv32) {
    const bool e = emb != nullptr;
    const dim3 grid(H, ns);
    switch ((d + 255) / 256) {
#define SAF(NV)                                                                                                      \
    case NV:                                                                                                         \
        launch_self_attn_fused<NV>(st, e, grid, kv32, wqkv, sqkv, bqkv, x, lnw, lnb, kc, vc, att, posp, d, nctx, L,   \
                                   layer, scale, pmax, tok, emb, pemb, lnseq);                                        \
        break;
        SAF(1)
        SAF(2)
        SAF(3)
        SAF(4)
        SAF(5)
        SAF(6)
        SAF(7)
    default: launch_self_attn_fused<8>(st, e, grid, kv32, wqkv, sqkv, bqkv, x, lnw, lnb, kc, vc, att, posp, d, nctx,
                                       L, layer, scale, pmax, tok, emb, pemb, lnseq);
        break;
#undef SAF
    }
}

void fw_launch_cross_attn_i8v2(hipStream_t st, const int8_t *wq, const float *swq, const float *bq, const float *x,
                               const float *lnw, const float *lnb, const int8_t *ck, const float *cks, const int8_t *cvt,
                               const float *cvs, float *att, int d, int T, int Tq, int H, int L, int layer, int ns,
                               float scale, float *pmax, int lnseq, const float *vbs) {
    if (64 * ca_vstride(Tq) > 7 * CA_VKB * 1024) return; // refused where the decoder is loaded (T <= 1536)
    size_t shm = (size_t)64 * ca_vstride(Tq) + sizeof(float) * ((T + 3) & ~3) + Tq;
    const int nb = (T + 31) / 32;
    if (vbs) {
        // + the block dots [64, nb], 16-byte aligned
        shm = ((shm + 15) & ~(size_t)15) + sizeof(float) * 64 * (size_t)nb;
#define CA_VBL(NV_)                                                                                                 \
    case NV_:                                                                                                       \
        if (lnseq)                                                                                                  \
            hipLaunchKernelGGL((k_cross_attn_i8v2<NV_, true, true>), dim3(H, ns), dim3(512), shm, st, wq, swq, bq, x, \
                               lnw, lnb, ck, cks, cvt, cvs, att, d, T, Tq, H, L, layer, scale, pmax, vbs, nb);        \
        else                                                                                                        \
            hipLaunchKernelGGL((k_cross_attn_i8v2<NV_, false, true>), dim3(H, ns), dim3(512), shm, st, wq, swq, bq,   \
                               x, lnw, lnb, ck, cks, cvt, cvs, att, d, T, Tq, H, L, layer, scale, pmax, vbs, nb);     \
        break;
        switch ((d + 255) / 256) {
            CA_VBL(1)
            CA_VBL(2)
            CA_VBL(3)
            CA_VBL(4)
            CA_VBL(5)
            CA_VBL(6)
            CA_VBL(7)
            CA_VBL(8)
        default: break;
        }
#undef CA_VBL
        return;
    }
    FW_ROWS_DISPATCH(k_cross_attn_i8v2, lnseq, d, dim3(H, ns), dim3(512), shm, st, wq, swq, bq, x, lnw, lnb, ck, cks,
                     cvt, cvs, att, d, T, Tq, H, L, layer, scale, pmax, nullptr, 0);
}

void fw_launch_quant_f16_rows_ld(hipStream_t st, const uint16_t *src, int8_t *q, float *s, int rows, int n, int ldq) {
    hipLaunchKernelGGL(k_quant_f16_rows_ld, dim3(rows), dim3(64), 0, st, src, q, s, n, ldq);
}

// Per-block argmax keys over already computed logits [ns, V] (the f16 arm's
// logits GEMV has no fused key epilogue): block (b, s) covers 2048 logits.
__global__ void __launch_bounds__(256) k_logits_keys(const float *logits, int V, fwhip_filter filt, int use_filter,
                                                     const int *initialp, unsigned long long *keys) {
    __shared__ unsigned long long wk[4];
    const int b = blockIdx.x, s = blockIdx.y, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int initial = use_filter ? *initialp : 0;
    const float *l = logits + (size_t)s * V;
    unsigned long long k = 0ull;
    for (int i = b * 2048 + threadIdx.x; i < V && i < (b + 1) * 2048; i += 256) {
        if (use_filter && dec_masked(i, filt, initial)) continue;
        unsigned long long c = am_key(l[i], i);
        k = c > k ? c : k;
    }
    k = wave_max_u64(k);
    if (lane == 0) wk[wave] = k;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long m = wk[0];
        for (int w = 1; w < 4; w++) m = wk[w] > m ? wk[w] : m;
        keys[(size_t)s * gridDim.x + b] = m;
    }
}

int fw_logits_keys_blocks(int V) { return (V + 2047) / 2048; }

void fw_launch_logits_keys(hipStream_t st, const float *logits, int V, int ns, const fwhip_filter *filt,
                           const int *initialp, unsigned long long *keys) {
    fwhip_filter ff;
    int use = filt != nullptr;
    if (filt) ff = *filt;
    else memset(&ff, 0, sizeof ff);
    hipLaunchKernelGGL(k_logits_keys, dim3(fw_logits_keys_blocks(V), ns), dim3(256), 0, st, logits, V, ff, use,
                       initialp, keys);
}
