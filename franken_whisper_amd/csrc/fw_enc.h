// fw_enc.h — encoder kernel interface.
#pragma once
#include <type_traits>

#include "fw_kernels.h"

#define FW_KIND_I8 0
#define FW_KIND_F16S 1

#define FW_EPI_F32 0
#define FW_EPI_RESID 1
#define FW_EPI_GELU_F32 2
#define FW_EPI_GELU_SPLIT 3
#define FW_EPI_CONV2 4
#define FW_EPI_QKV 5
#define FW_EPI_ACC32 6
// int8 only: v = (acc * s_x) * s_w + b stored as its f16 bits (the index of
// the f16 GELU table) when |v| < FW_GIDX_LIM, else FW_GIDX_SENT with the exact
// v written at the same index of the f32 side array C
#define FW_EPI_F16IDX 7
#define FW_GIDX_LIM 9.98f
#define FW_GIDX_SENT 0xffffu
// f16-pair only: the decoder's cross K/V of every layer from one GEMM
// (DecoderState::new, decoder.rs:1040-1222).  Column col = (l * 2 + kv) * d + c
// (d = ldc, head h = c / 64, dd = c % 64), row = s * T + t: K (kv 0) goes to
// o16[0] at [s, l, h, t, dd] as f16(v * scale), V (kv 1) to o16[1] at
// [s, l, h, dd, t] as f16(v + bias[col]).
#define FW_EPI_XKV 8

// Position of key t in a V^T row: bits 2 and 3 swapped, so the keys
// {16g + 4h + 0..3, 16g + 8 + 4h + 0..3} one attention MFMA lane multiplies
// sit together at 16g + 8h + 0..7.
__host__ __device__ __forceinline__ int fw_vt_pos(int t) { return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1); }

#define FW_LN_F32 0
#define FW_LN_SPLIT 1
#define FW_LN_I7 2
// or-ed into the mode: the f64 statistics summed in index order, as the
// reference's loops do (exact mode), instead of the wave's tree order
#define FW_LN_SEQ 0x100

struct FwGemm {
    const void *A;  // [M, lda] i8, or f16 hi
    const void *A2; // f16 lo (KIND_F16S)
    const void *B;  // [N, ldb] i8 or f16
    int M, N, K, lda, ldb;
    const float *sx, *sw, *bias;
    int epi;
    float *C;
    int ldc;
    uint16_t *o16[6];
    const float *pos;
    const float *gelu_tab;
    int T, H, Tp;
    int L;       // FW_EPI_XKV: decoder layers
    float scale; // FW_EPI_XKV: the key scale
    int map;     // tile order (set by fw_launch_gemm)
    // f16-pair epilogues (QKV, GELU split): set to 1 when a finite or infinite
    // value reaches |v| >= 65520, where the pair's hi half overflows (nullable)
    int *ovf;
};

// false when the operand kind / epilogue pair has no kernel (nothing launched)
bool fw_launch_gemm(hipStream_t st, int kind, const FwGemm &g);
// ovf (nullable): as FwGemm::ovf, for the SPLIT output.  With FW_LN_SEQ,
// stats [rows][2] (f64) is scratch for the sequential statistics (required).
void fw_launch_enc_ln(hipStream_t st, const float *x, const float *w, const float *b, int rows, int d, int mode,
                      float *yf, uint16_t *hi, uint16_t *lo, int8_t *q, float *qs, int *ovf = nullptr,
                      double *stats = nullptr);
void fw_launch_quant_exact_rows(hipStream_t st, const float *x, int rows, int n, int8_t *q, float *qs);
// The f16 copy of the GELU table that follows the f32 one (65536 entries) in
// the context's allocation; tab is the context's f32 table.
inline const uint16_t *fw_gelu_tab16(const float *tab) { return (const uint16_t *)(tab + 65536); }
void fw_launch_gelu_quant_i7_rows(hipStream_t st, const float *x, int rows, int n, const float *tab, int8_t *q,
                                  float *qs);
// The same GELU + quantization from FW_EPI_F16IDX rows (f16 table indices hx,
// exact values of the sentinel elements in side); false when n is not a
// supported width (a multiple of 512 up to 8192).
bool fw_launch_gelu_quant_h16(hipStream_t st, const uint16_t *hx, const float *side, int rows, int n,
                              const float *tab, int8_t *q, float *qs);
void fw_launch_im2col(hipStream_t st, const float *x, int B, int Tin, int Cin, int stride, int Tout, int Kp,
                      uint16_t *hi, uint16_t *lo, int *ovf = nullptr);
void fw_launch_mel_window(hipStream_t st, const float *mel, int n_mel, long long mel_frames, const long long *offs,
                          int n_frames, float *out, int B);
void fw_launch_fill_u16(hipStream_t st, uint16_t *p, size_t n, uint16_t v);
// f32 -> f16 pair (hi = f16(x), lo = f16(x - hi)): the A operand of an f16-pair GEMM
void fw_launch_split_f16(hipStream_t st, const float *x, size_t n, uint16_t *hi, uint16_t *lo, int *ovf = nullptr);
void fw_launch_attention(hipStream_t st, const uint16_t *qh, const uint16_t *ql, const uint16_t *kh,
                         const uint16_t *kl, const uint16_t *vth, const uint16_t *vtl, int B, int T, int Tp, int H,
                         int d, int out_mode, float *of, uint16_t *oh, uint16_t *ol);
void fw_launch_im2col_f32(hipStream_t st, const float *x, int B, int Tin, int Cin, int stride, int Tout, float *out);
// S [B*H, T, T] and sf [B*H*T * (1 + ceil(T / 64))] are scratch (the scores,
// then the exps; each row's scale factor, then the score tiles' row maxima)
void fw_launch_attention_exact(hipStream_t st, const float *qkv, int ld, int qoff, int koff, int voff, int B, int T,
                               int H, int d, float *S, float *sf, float *out);
// ToMe (enc_tome.hip): merge x [B, T, d] into xm [B, T - r', d] with the
// unmerge map umap [B, T] (workspace fw_tome_ws_bytes(B, T)); returns T - r'
bool fw_tome_ok(int T, int d);
size_t fw_tome_ws_bytes(int B, int T);
int fw_launch_tome_merge(hipStream_t st, const float *x, int B, int T, int d, int r, void *ws, float *xm,
                         int32_t *umap);
void fw_launch_tome_unmerge(hipStream_t st, const float *xm, int B, int Tm, const int32_t *umap, int T, int d,
                            float *out);
void fw_launch_tome_vpad(hipStream_t st, uint16_t *vt, size_t rows, int T, int Tp);
// cum [B, T0] = step[cum] per window (step [B, Tprev]): the unmerge map through one more merge
void fw_launch_tome_compose(hipStream_t st, int32_t *cum, const int32_t *step, int B, int T0, int Tprev);
