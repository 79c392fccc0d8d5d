/*
 * refcpu.h — CPU restatement of franken_whisper's native Whisper engine hot
 * path, written from the reference's Rust sources (src/native_engine/) as
 * TEST INFRASTRUCTURE: the parity oracle for the HIP library and the CPU
 * baseline timed beside it.  Nothing in the product links or calls this.
 *
 * Flag set restated (the "PINNED" mode, which makes every operation in-tree
 * Rust or IEEE/glibc and therefore restatable bit for bit):
 *   FT_SGEMM_STRICT_PARITY=1 (nn.rs:535-541, 587-604): every f32 matmul is an
 *       ascending-k sequential mul+add per output, no FMA;
 *   FW_ATTN_NO_SDPA=1 (nn.rs:5917-5921): encoder attention is the per-head
 *       matmul -> softmax -> matmul of attention_raw (nn.rs:6035-6131);
 *   FW_ENC_QKV_FUSED=0, FW_TOME_R=0, FW_SDPA_POLY_EXP=0, FW_KV_F16=1;
 *   x86-64-v3 build (.cargo/config.toml:37): the AVX2/F16C/FMA kernels are the
 *       ones restated (their lane orders and add-trunc rounding), with their
 *       scalar tails where the Rust has them.
 * Default-mode FrankenTorch arithmetic (ft sgemm tile order, ft SDPA, poly-exp)
 * is NOT restated: it lives in the absent ft-kernel-cpu 0.1.2 crate.
 *
 * Build: -O2 -ffp-contract=off (Rust never contracts a*b+c), -mfma -mf16c only
 * for the explicit FMA/F16C the reference itself uses.
 */
#ifndef REFCPU_H
#define REFCPU_H
#include <stdint.h>
#include "../include/fwhip.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar primitives ---- */
float ref_f16_to_f32(uint16_t h);
uint16_t ref_f32_to_f16(float f);
void ref_f16_to_f32_n(const uint16_t *h, float *f, int64_t n);
void ref_f32_to_f16_n(const float *f, uint16_t *h, int64_t n);
float ref_gelu_scalar(float x);
const float *ref_gelu_table(void);

/* ---- quantizers ---- */
void ref_quantize_act_i8(const float *x, int n, float xinv, int8_t *out);
void ref_quantize_row_i7_u8(const float *x, int n, float inv, uint8_t *out);
void ref_quant_row_i8_exact(const float *x, int n, float inv, int8_t *out);
float ref_quantize_f16_row_to_i8(const uint16_t *w, int n, int8_t *out);
void ref_quantize_f16_to_i8(const uint16_t *w, int64_t out, int inp, int8_t *q, float *s);
void ref_quantize_f16_to_i8_blocked(const uint16_t *w, int64_t out, int inp, int block,
                                    int8_t *q, float *s);
void ref_quantize_rows_to_i7(const uint16_t *w, int64_t out, int inp, int ef, int8_t *q,
                             float *s, int32_t *colsum);
void ref_quantize_enc_i8_rows(const uint16_t *w, int64_t out, int inp, int8_t *q, float *s);
float ref_act_scale(const float *x, int n); /* max(max|x|,1e-9)/127 */

/* ---- GEMV / dots ---- */
int32_t ref_dot_i8(const int8_t *w, const int8_t *x, int n);
float ref_dot_f16c(const uint16_t *w, const float *x, int n);
float ref_dot_i8w_f32(const int8_t *w, const float *x, int n);
void ref_gemv_i8(const int8_t *W, const float *s_w, int64_t out, int inp, const float *x,
                 const float *bias, float *y);
void ref_gemv_f16(const uint16_t *W, int64_t out, int inp, const float *x, const float *bias,
                  float *y);
void ref_gemv_i8w_f32a_blocked(const int8_t *W, const float *s, int64_t out, int inp, int block,
                               const float *x, const float *bias, float *y);

/* ---- row ops ---- */
void ref_layer_norm(const float *x, float *y, int64_t rows, int cols, const float *w,
                    const float *b, float eps);
void ref_gelu_inplace(float *x, int64_t n);
void ref_softmax_rows(float *x, int64_t rows, int cols);
void ref_matmul_strict(const float *a, const float *b, float *c, int64_t m, int k, int n);
int ref_argmax_first(const float *l, int n);

/* ---- attention (exported for the reference's attention invariants) ---- */
void ref_attention(const float *q, int tq, const float *k, const float *v, int tk, int n_state,
                   int n_head, int causal, int cache_len, float *out);
void ref_attention_decode_f16(const float *q, const uint16_t *kc, const uint16_t *vc, int tk, int d,
                              int H, float *out);
void ref_attention_decode_f32(const float *q, const float *kc, const float *vc, int tk, int d, int H, float *out);

/* ---- encoder ---- */
typedef struct ref_encoder ref_encoder;
ref_encoder *ref_encoder_new(const fwhip_encoder_weights *w, int precision);
void ref_encoder_free(ref_encoder *e);
/* x: time-major [n_frames, n_mels]; out: [n_frames/2, d].  n_layers_run < 0
 * runs every block (encoder_layer_limit semantics otherwise). */
int ref_encoder_forward(const ref_encoder *e, const float *x, int n_frames, float *out,
                        int n_layers_run);
int ref_encoder_forward_tome(const ref_encoder *e, const float *x, int n_frames, float *out, int n_layers_run,
                             int tome_r, int tome_after);
int ref_encoder_forward_tome2(const ref_encoder *e, const float *x, int n_frames, float *out, int n_layers_run,
                              int tome_r, int tome_after, int tome_every, int tome_floor);
int ref_tome_merge(const float *x, int seq, int d, int r, float *merged, int32_t *umap);
void ref_tome_unmerge(const float *merged, const int32_t *umap, int seq, int d, float *out);
void ref_mel_window(const float *full_mel, int n_mel, int64_t mel_frames, int64_t frame_offset,
                    int n_frames, float *out);
/* one encoder int8 GEMM, for per-GEMM parity: i32 accumulators and epilogue */
void ref_enc_i7_gemm(const ref_encoder *e, int layer, int which, const float *x, int64_t m,
                     int32_t *acc_out, float *y_out);

/* ---- decoder ---- */
typedef struct ref_decoder ref_decoder;
void ref_decoder_set_kv_f16(ref_decoder *dd, int on); /* FW_KV_F16 for the states made next */
void ref_decoder_set_cross_v_block(ref_decoder *dd, int on); /* FW_CROSS_V_BLOCK, likewise */
typedef struct ref_dstate ref_dstate;
ref_decoder *ref_decoder_new(const fwhip_decoder_weights *w, int arm);
void ref_decoder_free(ref_decoder *d);
ref_dstate *ref_dstate_new(const ref_decoder *d, const float *enc, int enc_frames);
void ref_dstate_free(ref_dstate *s);
void ref_dstate_reset(ref_dstate *s);
int ref_dstate_len(const ref_dstate *s);
/* cross K/V accessors (layer-major then head) for parity of the precompute */
const uint16_t *ref_dstate_cross_k_f16(const ref_dstate *s);
const uint16_t *ref_dstate_cross_vt_f16(const ref_dstate *s);
int ref_decoder_step(const ref_decoder *d, ref_dstate *s, const int32_t *tokens, int tq,
                     float *logits);
int ref_process_argmax(const fwhip_filter *f, const float *logits, int n_vocab, int initial);
/* FilterConfig (decode.rs:671-693); -1 is None for max_initial_tid / max_tokens */
typedef struct ref_filter_cfg {
    int suppress_blank, no_timestamps, max_initial_tid, max_tokens;
} ref_filter_cfg;
void ref_compute_logprobs(const float *logits, int n, float *lp);
int ref_process_logits(const fwhip_filter *f, const ref_filter_cfg *cfg, float *logits, float *logprobs, int n,
                       const int32_t *prev, int n_prev, int has_ts, int64_t seek_delta_cs, int tokens_in_window);
int ref_decode_greedy(const ref_decoder *d, ref_dstate *s, const int32_t *prompt, int n_prompt,
                      int n_max, const fwhip_filter *f, int32_t *out_tokens, int32_t *out_len);

/* ---- log-mel frontend (mel.rs:81-1660) ---- */
int64_t ref_mel_frames(int64_t n_samples); /* n_frames_for, mel.rs:1127 */
/* log_mel (mel.rs:1476): mel-major out [n_mel, ref_mel_frames(n)], clamped to
 * max - 8 and normalized (x + 4) / 4.  filters: [n_mel, 201] f32. */
void ref_log_mel(const float *samples, int64_t n_samples, const float *filters, int n_mel, float *out);
/* pieces, for pinning: the default two-for-one real FFT of one 400-sample
 * frame (out: 400 interleaved complex bins), the log10 approximation, and the
 * Hann window */
void ref_mel_fft400(const float *in, float *out);
float ref_log10_floor_approx(double x);
void ref_mel_hann(float *out400);

int ref_num_threads(void);
void ref_set_num_threads(int n);
/* FAST restatement on/off (refcpu_fast.c: register-blocked AVX2 / F16C
 * kernels giving the same bits as the scalar loops). */
void ref_set_fast(int on);
int ref_get_fast(void);

#ifdef __cplusplus
}
#endif
#endif
