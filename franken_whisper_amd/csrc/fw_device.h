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

// fw_q8_avx for an element of the add-trunc body (rows of n % 8 == 0), as an
// unsigned byte ready for packing.
__device__ __forceinline__ uint32_t fw_q8_body(float v, float inv) {
    return (uint32_t)(uint8_t)(int8_t)(int)fw_clamp(fw_round_add_trunc(v * inv), -127.0f, 127.0f);
}

__device__ __forceinline__ float fw_expf(float x) {
    const uint64_t tab[32] = FW_EXP2F_TAB;
    return fw_expf_tab(x, tab);
}

__device__ __forceinline__ float fw_logf(float x) {
    const double tab[32] = FW_LOGF_TAB;
    return fw_logf_tab(x, tab);
}

// GELU of the reference (nn.rs:4603-4673): clamp +-10, else f16-indexed table.
__device__ __forceinline__ float fw_gelu(float v, const float *tab) {
    // The table read is unconditional (every f16 pattern is a valid index) and
    // the clamp cases are merged with bit masks the compiler cannot see
    // through: written as a select, the read gets moved behind a branch of its
    // own and each element waits for its data in turn.
    const uint32_t t = __float_as_uint(tab[fw_f2h(v)]);
    const bool lo = v <= -10.0f, hi = v >= 10.0f;
    uint32_t mt = (!lo && !hi) ? 0xffffffffu : 0u, mv = hi ? 0xffffffffu : 0u;
    asm volatile("" : "+v"(mt), "+v"(mv));
    return __uint_as_float((t & mt) | (__float_as_uint(v) & mv));
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

// Block-interleaved position of feature k in a row of nb 32-wide blocks:
// 16-byte chunk q of block b goes to chunk index q * nb + b.
__device__ __forceinline__ int fw_blk_perm(int k, int nb) {
    return ((((k & 31) >> 2) * nb + (k >> 5)) << 2) | (k & 3);
}

// Explicit s_waitcnt (gfx9 encoding: vmcnt bits 3:0 and 15:14, expcnt 6:4,
// lgkmcnt 11:8); the counters not named are not waited on.
#define FW_WAIT_VM(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (15 << 8) | (((n) >> 4) << 14))
#define FW_WAIT_LGKM0() __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (3 << 14))
#define FW_WAIT_VM_LGKM0(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (7 << 4) | (((n) >> 4) << 14))

// Whole-wave reductions over DPP lane moves (no LDS round trips): pair, quad,
// half-row and row butterflies, then the four 16-lane row results are read
// into scalars and combined as (r0 + r1) + (r2 + r3).  Every lane returns the
// same value.
template <int CTRL>
__device__ __forceinline__ float fw_dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xf, 0xf, false));
}
template <int CTRL>
__device__ __forceinline__ double fw_dpp_f64(double v) {
    const int lo = __builtin_amdgcn_mov_dpp(__double2loint(v), CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_mov_dpp(__double2hiint(v), CTRL, 0xf, 0xf, false);
    return __hiloint2double(hi, lo);
}
#define FW_DPP_XOR1 0xB1      // quad_perm [1,0,3,2]
#define FW_DPP_XOR2 0x4E      // quad_perm [2,3,0,1]
#define FW_DPP_HALF_MIRROR 0x141
#define FW_DPP_MIRROR 0x140
__device__ __forceinline__ double fw_rl_f64(double v, int lane) {
    return __hiloint2double(__builtin_amdgcn_readlane(__double2hiint(v), lane),
                            __builtin_amdgcn_readlane(__double2loint(v), lane));
}
__device__ __forceinline__ double fw_dpp_wave_sum_f64(double v) {
    v = v + fw_dpp_f64<FW_DPP_XOR1>(v);
    v = v + fw_dpp_f64<FW_DPP_XOR2>(v);
    v = v + fw_dpp_f64<FW_DPP_HALF_MIRROR>(v);
    v = v + fw_dpp_f64<FW_DPP_MIRROR>(v);
    return (fw_rl_f64(v, 0) + fw_rl_f64(v, 16)) + (fw_rl_f64(v, 32) + fw_rl_f64(v, 48));
}
__device__ __forceinline__ float fw_dpp_wave_max(float v) {
    v = fmaxf(v, fw_dpp_f32<FW_DPP_XOR1>(v));
    v = fmaxf(v, fw_dpp_f32<FW_DPP_XOR2>(v));
    v = fmaxf(v, fw_dpp_f32<FW_DPP_HALF_MIRROR>(v));
    v = fmaxf(v, fw_dpp_f32<FW_DPP_MIRROR>(v));
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float c = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float d = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return fmaxf(fmaxf(a, b), fmaxf(c, d));
}

__device__ __forceinline__ int fw_dpp_wave_sum_i32(int v) {
    v = v + __builtin_amdgcn_mov_dpp(v, FW_DPP_XOR1, 0xf, 0xf, false);
    v = v + __builtin_amdgcn_mov_dpp(v, FW_DPP_XOR2, 0xf, 0xf, false);
    v = v + __builtin_amdgcn_mov_dpp(v, FW_DPP_HALF_MIRROR, 0xf, 0xf, false);
    v = v + __builtin_amdgcn_mov_dpp(v, FW_DPP_MIRROR, 0xf, 0xf, false);
    return (__builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16)) +
           (__builtin_amdgcn_readlane(v, 32) + __builtin_amdgcn_readlane(v, 48));
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
