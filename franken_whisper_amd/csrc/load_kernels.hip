// load_kernels.hip — load-time weight preparation on the device: the
// reference quantizers run once per weight, one thread (error-feedback chain)
// or one wave (per-row amax) per output row, with the reference's exact f32
// arithmetic (-ffp-contract=off keeps w*inv + err a mul then an add).
#include "fw_kernels.h"

// quantize_f16_to_i8 (nn.rs:2576-2633, FW_DEC_EF off): per-row amax/127 with
// add-trunc rounding in the 8-wide body and exact rounding in the tail.
// (k_quant_f16_rows in dec_kernels.hip is the same operation.)

// quantize_f16_to_i8_blocked (nn.rs:3583, 3619-3720): per-32-block amax/127;
// output rows of stride ldq.
__global__ void k_quant_blocked(const uint16_t *w, int8_t *q, float *s, int64_t out, int inp, int block, int ldq) {
    int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    int nb = (inp + block - 1) / block;
    if (idx >= out * nb) return;
    int64_t o = idx / nb;
    int b = (int)(idx % nb);
    const uint16_t *wr = w + o * inp;
    int st = b * block, e = min(inp, st + block);
    float amax = 0.0f;
    for (int i = st; i < e; i++) amax = fmaxf(amax, fabsf(fw_h2f(wr[i])));
    float sc = fmaxf(amax, 1e-9f) / 127.0f;
    float inv = 1.0f / sc;
    int e8 = st + ((e - st) / 8) * 8;
    for (int i = st; i < e; i++) {
        float v = fw_h2f(wr[i]) * inv;
        float r = i < e8 ? fw_round_add_trunc(v) : fw_round_away(v);
        q[o * ldq + i] = (int8_t)(int)fw_clamp(r, -127.0f, 127.0f);
    }
    s[o * nb + b] = sc;
}

// quantize_rows_to_i7 (nn.rs:869-927): amax folded from 1e-9, scale amax/63,
// error-feedback rounding when ef (FW_ENC_EF_QUANT default on), colsum.
__global__ void k_quant_i7(const uint16_t *w, int8_t *q, float *s, int32_t *cs, int64_t out, int inp, int ef) {
    int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= out) return;
    const uint16_t *wr = w + o * inp;
    float amax = 1e-9f;
    for (int i = 0; i < inp; i++) amax = fmaxf(amax, fabsf(fw_h2f(wr[i])));
    float sc = amax / 63.0f;
    float inv = 1.0f / sc;
    int32_t acc = 0;
    float err = 0.0f;
    for (int i = 0; i < inp; i++) {
        float qq;
        if (ef) {
            float target = fw_h2f(wr[i]) * inv + err;
            qq = fw_clamp(fw_round_away(target), -63.0f, 63.0f);
            err = target - qq;
        } else {
            qq = fw_clamp(fw_round_away(fw_h2f(wr[i]) * inv), -63.0f, 63.0f);
        }
        int qi = (int)qq;
        q[o * inp + i] = (int8_t)qi;
        acc += qi;
    }
    s[o] = sc;
    cs[o] = acc;
}

// quantize_enc_i8_rows (encoder.rs:2235-2263): amax folded from 1e-9, /127,
// exact rounding.
__global__ void k_quant_enc_i8(const uint16_t *w, int8_t *q, float *s, int64_t out, int inp) {
    int64_t o = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (o >= out) return;
    const uint16_t *wr = w + o * inp;
    float amax = 1e-9f;
    for (int i = 0; i < inp; i++) amax = fmaxf(amax, fabsf(fw_h2f(wr[i])));
    float sc = amax / 127.0f;
    float inv = 1.0f / sc;
    for (int i = 0; i < inp; i++)
        q[o * inp + i] = (int8_t)(int)fw_clamp(fw_round_away(fw_h2f(wr[i]) * inv), -127.0f, 127.0f);
    s[o] = sc;
}

void fw_launch_quant_blocked(hipStream_t st, const uint16_t *w, int8_t *q, float *s, int64_t out, int inp,
                             int block, int ldq) {
    int64_t n = out * ((inp + block - 1) / block);
    hipLaunchKernelGGL(k_quant_blocked, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, w, q, s, out, inp,
                       block, ldq > 0 ? ldq : inp);
}
void fw_launch_quant_i7(hipStream_t st, const uint16_t *w, int8_t *q, float *s, int32_t *cs, int64_t out,
                        int inp, int ef) {
    hipLaunchKernelGGL(k_quant_i7, dim3((unsigned)((out + 63) / 64)), dim3(64), 0, st, w, q, s, cs, out, inp, ef);
}
void fw_launch_quant_enc_i8(hipStream_t st, const uint16_t *w, int8_t *q, float *s, int64_t out, int inp) {
    hipLaunchKernelGGL(k_quant_enc_i8, dim3((unsigned)((out + 63) / 64)), dim3(64), 0, st, w, q, s, out, inp);
}
