// fw_device.h — device-side helpers shared by the decoder and encoder kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "fw_math.h"

#define FW_WAVE 64

__device__ __forceinline__ float fw_h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}
// RNE f32 -> f16 of an f32 value.  The empty asm pins `f` as a materialized f32
// register: without it the backend may fold a producing multiply into a
// mixed-precision mad (v_mad_mixlo_f16), rounding the exact product straight to
// f16 — a double-rounding difference from Rust's Float16::from_f32(a * b).
__device__ __forceinline__ uint16_t fw_f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// f32::round: half away from zero (trunc and v - trunc(v) are exact).
__device__ __forceinline__ float fw_round_away(float v) {
    float t = truncf(v);
    return fabsf(v - t) >= 0.5f ? t + copysignf(1.0f, v) : t;
}
// AVX2 add-trunc rounding trunc(v + copysign(0.5, v)) (nn.rs:3036-3038).
__device__ __forceinline__ float fw_round_add_trunc(float v) {
    return truncf(v + copysignf(0.5f, v));
}
__device__ __forceinline__ float fw_clamp(float v, float lo, float hi) {
    return fminf(fmaxf(v, lo), hi);
}
// i8 quantization of one element at index i of an n-long vector whose 8-wide
// body uses add-trunc and whose n % 8 tail uses exact rounding.
__device__ __forceinline__ int8_t fw_q8_avx(float v, float inv, int i, int n) {
    float t = v * inv;
    float r = i < n - (n & 7) ? fw_round_add_trunc(t) : fw_round_away(t);
    return (int8_t)(int)fw_clamp(r, -127.0f, 127.0f);
}

__device__ __forceinline__ float fw_expf(float x) {
    const uint64_t tab[32] = FW_EXP2F_TAB;
    return fw_expf_tab(x, tab);
}

// GELU of the reference (nn.rs:4603-4673): clamp +-10, else f16-indexed table.
__device__ __forceinline__ float fw_gelu(float v, const float *tab) {
    return v <= -10.0f ? 0.0f : (v >= 10.0f ? v : tab[fw_f2h(v)]);
}

// ---- wave / block reductions -------------------------------------------
template <typename T>
__device__ __forceinline__ T fw_wave_sum(T v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, FW_WAVE);
    return v;
}
__device__ __forceinline__ float fw_wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, FW_WAVE));
    return v;
}

// Block-wide sum/max (all threads get the result).  `sh` needs blockDim/64 slots.
template <typename T>
__device__ __forceinline__ T fw_block_sum(T v, T *sh) {
    v = fw_wave_sum(v);
    int w = threadIdx.x / FW_WAVE, l = threadIdx.x % FW_WAVE, nw = blockDim.x / FW_WAVE;
    __syncthreads();
    if (l == 0) sh[w] = v;
    __syncthreads();
    T r = 0;
    for (int i = 0; i < nw; i++) r += sh[i];
    return r;
}
__device__ __forceinline__ float fw_block_max(float v, float *sh) {
    v = fw_wave_max(v);
    int w = threadIdx.x / FW_WAVE, l = threadIdx.x % FW_WAVE, nw = blockDim.x / FW_WAVE;
    __syncthreads();
    if (l == 0) sh[w] = v;
    __syncthreads();
    float r = -INFINITY;
    for (int i = 0; i < nw; i++) r = fmaxf(r, sh[i]);
    return r;
}

__device__ __forceinline__ int fw_sdot4(int a, int b, int c) {
    return __builtin_amdgcn_sdot4(a, b, c, false);
}
