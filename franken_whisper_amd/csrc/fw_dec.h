// fw_dec.h — device helpers shared by the decoder kernels: the decoder
// LayerNorm (+ int8 activation quantizer) of one row per wave, and the
// argmax keys and suppress mask of process_logits.
#pragma once
#include "fw_kernels.h"

// ---------------------------------------------------------------------------
// LayerNorm (nn.rs:4455-4545: f64 mean/var, ((x-mean)*inv)*w + b rounded to
// f32) of one stream row per wave, then the decoder activation quantizer of
// the normalized row (per-row amax/127, add-trunc body, exact n%8 tail) into
// the int8 activation buffer.  y may be NULL (int8-only consumers), xq may be
// NULL (f32-only consumers).  4 rows per block; lane l holds the float4
// groups l, l+64, ... (NV of them, d <= 256*NV, d % 4 == 0).  Every load of
// x, w and b is issued before the first use, so the row costs one memory
// round trip; the reductions run on DPP lane moves.
// Row r whose values xv (lane l: float4 groups l, l+64, ...; ok = in range)
// are already loaded or in flight.
// LayerNorm weight and bias groups of lane l (as the row values).
template <int NV>
__device__ __forceinline__ void fw_ln_load_wb(const bool (&ok)[NV], const float *w, const float *b, float4 (&wv)[NV],
                                              float4 (&bv)[NV], int lane) {
    const float4 *w4 = (const float4 *)w, *b4 = (const float4 *)b;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        const int c = ok[k] ? lane + k * 64 : 0;
        wv[k] = w4[c];
        bv[k] = b4[c];
    }
}

// The same with the weight and bias groups already loaded (or in flight).
template <int NV>
__device__ __forceinline__ void fw_ln_quant_core(float4 (&xv)[NV], const bool (&ok)[NV], const float4 (&wv)[NV],
                                                 const float4 (&bv)[NV], float *y, int d, int r, int8_t *xq,
                                                 float *xs, int lane) {
    double s = 0.0;
#pragma unroll
    for (int k = 0; k < NV; k++)
        if (ok[k]) s += ((double)xv[k].x + (double)xv[k].y) + ((double)xv[k].z + (double)xv[k].w);
    const double mean = fw_dpp_wave_sum_f64(s) / (double)d;
    double v = 0.0;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if (ok[k]) {
            const double a = (double)xv[k].x - mean, bb = (double)xv[k].y - mean;
            const double c = (double)xv[k].z - mean, e = (double)xv[k].w - mean;
            v += (a * a + bb * bb) + (c * c + e * e);
        }
    }
    const double var = fw_dpp_wave_sum_f64(v) / (double)d;
    const double inv = 1.0 / sqrt(var + (double)1e-5f);
    float m = 0.0f;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        float4 o;
        o.x = (float)((((double)xv[k].x - mean) * inv) * (double)wv[k].x + (double)bv[k].x);
        o.y = (float)((((double)xv[k].y - mean) * inv) * (double)wv[k].y + (double)bv[k].y);
        o.z = (float)((((double)xv[k].z - mean) * inv) * (double)wv[k].z + (double)bv[k].z);
        o.w = (float)((((double)xv[k].w - mean) * inv) * (double)wv[k].w + (double)bv[k].w);
        xv[k] = o;
        if (ok[k]) {
            m = fmaxf(m, fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w))));
            if (y) ((float4 *)(y + (size_t)r * d))[lane + k * 64] = o;
        }
    }
    if (!xq) return;
    m = fw_dpp_wave_max(m);
    const float sc = fmaxf(m, 1e-9f) / 127.0f;
    const float iv = 1.0f / sc;
#pragma unroll
    for (int k = 0; k < NV; k++) {
        if (ok[k]) {
            const int i = (lane + k * 64) * 4;
            const uint32_t q = (uint32_t)(uint8_t)fw_q8_avx(xv[k].x, iv, i, d) |
                               ((uint32_t)(uint8_t)fw_q8_avx(xv[k].y, iv, i + 1, d) << 8) |
                               ((uint32_t)(uint8_t)fw_q8_avx(xv[k].z, iv, i + 2, d) << 16) |
                               ((uint32_t)(uint8_t)fw_q8_avx(xv[k].w, iv, i + 3, d) << 24);
            *(uint32_t *)(xq + (size_t)r * d + i) = q;
        }
    }
    if (lane == 0) xs[r] = sc;
}

template <int NV>
__device__ __forceinline__ void fw_ln_quant_vals(float4 (&xv)[NV], const bool (&ok)[NV], float *y, const float *w,
                                                 const float *b, int d, int r, int8_t *xq, float *xs, int lane) {
    float4 wv[NV], bv[NV];
    fw_ln_load_wb<NV>(ok, w, b, wv, bv, lane);
    fw_ln_quant_core<NV>(xv, ok, wv, bv, y, d, r, xq, xs, lane);
}


// ---------------------------------------------------------------------------
// Order-preserving argmax key: larger value first, then smaller index; 0 means
// "no candidate" (masked, -inf or NaN never compare greater, as in the
// reference's strict '>' scan).  -0.0 and +0.0 compare equal under '>', so the
// first of them wins (argmax_idx, decode.rs:1708-1770): both map to one key.
__device__ __forceinline__ unsigned long long am_key(float v, int idx) {
    if (!(v > -INFINITY)) return 0ull;
    uint32_t u = v == 0.0f ? 0u : __float_as_uint(v);
    u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    return ((unsigned long long)u << 32) | (unsigned long long)(0xffffffffu - (uint32_t)idx);
}
template <int CTRL>
__device__ __forceinline__ unsigned long long dpp_max_u64(unsigned long long k) {
    const uint32_t lo = __builtin_amdgcn_mov_dpp((int)(uint32_t)k, CTRL, 0xf, 0xf, false);
    const uint32_t hi = __builtin_amdgcn_mov_dpp((int)(uint32_t)(k >> 32), CTRL, 0xf, 0xf, false);
    const unsigned long long o = ((unsigned long long)hi << 32) | lo;
    return o > k ? o : k;
}
// max over each 16-lane row (every lane of the row gets it), DPP moves only
__device__ __forceinline__ unsigned long long row16_max_u64(unsigned long long k) {
    k = dpp_max_u64<FW_DPP_XOR1>(k);
    k = dpp_max_u64<FW_DPP_XOR2>(k);
    k = dpp_max_u64<FW_DPP_HALF_MIRROR>(k);
    return dpp_max_u64<FW_DPP_MIRROR>(k);
}
// max over the wave (every lane gets it)
__device__ __forceinline__ unsigned long long wave_max_u64(unsigned long long k) {
    k = row16_max_u64(k);
    const unsigned long long r0 = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), 0) << 32) |
                                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 0);
    const unsigned long long r1 = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), 16) << 32) |
                                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 16);
    const unsigned long long r2 = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), 32) << 32) |
                                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 32);
    const unsigned long long r3 = ((unsigned long long)(uint32_t)__builtin_amdgcn_readlane((int)(k >> 32), 48) << 32) |
                                  (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 48);
    const unsigned long long a = r0 > r1 ? r0 : r1, b = r2 > r3 ? r2 : r3;
    return a > b ? a : b;
}

// The suppress set of process_logits in no-timestamps mode (decode.rs:702-867).
__device__ __forceinline__ bool dec_masked(int i, const fwhip_filter &f, int initial) {
    if (initial && (i == f.eot || i == f.space_token)) return true;
    if (i >= f.timestamp_begin) return true;
    if (i == f.no_timestamps || i == f.sot || i == f.no_speech || i == f.solm || i == f.translate ||
        i == f.transcribe || i == f.sot_prev)
        return true;
    if (i >= f.sot + 1 && i <= f.sot + f.n_languages) return true;
    return false;
}
