// fw_kernels.h — kernel launch wrappers shared between translation units.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "fw_device.h"
#include "fwhip.h"

// decoder (dec_kernels.hip)
void fw_launch_gemv_f16(hipStream_t st, const uint16_t *W, const float *bias, const float *x, float *y, int N,
                        int K, int ns, int ldy, int mode, const float *gelu_tab);
// f16 GEMV on weights in fragment order (repacked once by
// fw_launch_pack_gemv_f16 when fw_gemv_f16_frag_ok(N, K)); same results
int fw_gemv_f16_lpr(int N);
bool fw_gemv_f16_frag_ok(int N, int K);
void fw_launch_pack_gemv_f16(hipStream_t st, const uint16_t *W, uint16_t *Wf, int N, int K);
// With lnw / lnb (K <= 1280) the rows x are first put through LayerNorm
// (k_ln_quant's arithmetic), so the GEMV consumes LN(x).
void fw_launch_gemv_f16f(hipStream_t st, const uint16_t *Wf, const float *bias, const float *x, float *y, int N,
                         int K, int ns, int ldy, int mode, const float *gelu_tab, const float *lnw = nullptr,
                         const float *lnb = nullptr);
// The f16 GEMV for a cohort in slot order (dec_gemv16.hip): weights packed
// once by fw_launch_pack_gemv16 (needs fw_gemv16_ok(N, K)); bit-identical to
// fw_launch_gemv_f16.  keys (logits head): per-tile argmax keys
// [ns, fw_gemv16_key_blocks(N, K)] of the filtered rows.
bool fw_gemv16_ok(int N, int K);
int fw_gemv16_lpr(int N, int K);
int fw_gemv16_key_blocks(int N, int K);
void fw_launch_pack_gemv16(hipStream_t st, const uint16_t *W, uint16_t *Wp, int N, int K);
void fw_launch_gemv16(hipStream_t st, const uint16_t *Wp, const float *bias, const float *x, float *y, int N, int K,
                      int ns, int ldy, int mode, const float *gelu_tab, const float *lnw = nullptr,
                      const float *lnb = nullptr, const fwhip_filter *filt = nullptr, const int *initialp = nullptr,
                      unsigned long long *keys = nullptr, int r = 0, int sb_cap = 0, int grid_cap = 0);
void fw_launch_cross_attn_f16(hipStream_t st, const float *qc, const uint16_t *ck, const uint16_t *cvt,
                              float *att, int d, int T, int H, int L, int layer, int ns, float scale);
// The f16 arm's cross attention on slot-order K / V^T copies (dec_fast.hip):
// fw_launch_pack_cross_f16 repacks natural-order K [rows_k, 64] and V^T
// [rows_v, T] once per DecoderState::new (V^T rows at stride fw_cross_f16p_tv(T)).
bool fw_cross_f16p_ok(int T);
int fw_cross_f16p_tv(int T);
void fw_launch_pack_cross_f16(hipStream_t st, const uint16_t *ck, const uint16_t *cvt, uint16_t *ckp, uint16_t *cvtp,
                              size_t rows_k, size_t rows_v, int T);
// rows > 0: a prefill chunk of `rows` rows ([position][stream], the q rows and
// outputs indexed by row, the cross K/V by row % ns); else one row per stream
void fw_launch_cross_attn_f16p(hipStream_t st, const float *qc, const uint16_t *ckp, const uint16_t *cvtp, float *att,
                               int d, int T, int H, int L, int layer, int ns, float scale, int rows = 0);
// fw_launch_cross_attn_f16p (one row per stream) in two launches that spread
// each head's keys and output dims over more blocks, for cohorts whose
// (head, stream) blocks fill few CUs or more than one round of them; the same
// bits.  scratch: fw_cross_split_floats(T, H, ns) floats.
size_t fw_cross_split_floats(int T, int H, int ns);
void fw_launch_cross_attn_f16p_split(hipStream_t st, const float *qc, const uint16_t *ckp, const uint16_t *cvtp,
                                     float *att, int d, int T, int H, int L, int layer, int ns, float scale,
                                     float *scratch);
// the same with the cross LayerNorm of x [ns, d] and the q projection (wq in
// fw_launch_pack_gemv16's slot order at 16 lanes per row, bias bq) formed in
// each scores block; needs fw_cross_f16pq_ok(d, T, H)
void fw_launch_cross_attn_f16pq_split(hipStream_t st, const uint16_t *wq, const float *bq, const float *x,
                                      const float *lnw, const float *lnb, const uint16_t *ckp, const uint16_t *cvtp,
                                      float *att, int d, int T, int H, int L, int layer, int ns, float scale,
                                      float *scratch, int lnseq = 0);
// fw_launch_cross_attn_f16p with the cross LayerNorm of x [ns, d] and the q
// projection inside (wq in fw_launch_pack_gemv16's slot order at 16 lanes per
// row, bq the bias); needs fw_cross_f16pq_ok(d, T, H)
// the f16 arm's attention LayerNorm (lnw null: x already normalized), q/k/v
// projection (wqkv in fw_launch_pack_gemv16's slot order at 16 lanes per row)
// and self-attention in one launch; needs fw_self_attn_f16q_ok(d, H).  With
// tok (layer 0, lnw given) the rows are the token embeddings f16(emb[tok]) +
// pemb[*posp], stored to xo (x unused).
bool fw_self_attn_f16q_ok(int d, int H);
// (kc / vc: the self-attention caches, f16 or, with kv32, f32, in every
// launcher that takes them)
void fw_launch_self_attn_f16q(hipStream_t st, const uint16_t *wqkv, const float *bqkv, const float *x,
                              const float *lnw, const float *lnb, void *kc, void *vc, float *att,
                              const int *posp, int H, int nctx, int L, int layer, int ns, float scale,
                              const int32_t *tok = nullptr, const uint16_t *emb = nullptr,
                              const float *pemb = nullptr, float *xo = nullptr, int lnseq = 0, int kv32 = 0);
bool fw_cross_f16pq_ok(int d, int T, int H);
void fw_launch_cross_attn_f16pq(hipStream_t st, const uint16_t *wq, const float *bq, const float *x, const float *lnw,
                                const float *lnb, const uint16_t *ckp, const uint16_t *cvtp, float *att, int d, int T,
                                int H, int L, int layer, int ns, float scale, int lnseq = 0);
void fw_launch_gemm_strict(hipStream_t st, const float *A, const uint16_t *B, int m, int n, int k, int epi,
                           float *C, const float *bias, float scale, uint16_t *out16, int T, int H, int L,
                           int layer, int ldc = 0, const float *gelu_tab = nullptr, const float *pos = nullptr);
void fw_launch_quant_f16_rows(hipStream_t st, const uint16_t *src, int8_t *q, float *s, int rows, int n);
void fw_launch_step_bookkeeping(hipStream_t st, int *posp, int *initialp, const int32_t *tok, int32_t *hist,
                                int hist_stride, int step, int ns);

// lnseq (the kernels with a LayerNorm inside): nonzero sums the LayerNorm's
// mean and variance in the reference's sequential f64 order (exact mode)

// the window decode loop (dec_window.hip): process_logits in full + argmax +
// the loop's state per stream, and the post-loop log-probabilities
#define WIN_MAXTS 1536 // timestamp tokens the forcing rule's sequential sum takes
struct FwWinCfg {
    int V, beg, eot, sot, sot_prev, solm, no_speech, no_ts, translate, transcribe, space, n_lang;
    int timestamps;      // 0: no-timestamps mode (every timestamp masked)
    int max_initial_tid; // < 0: no initial-timestamp cap
    int max_tokens;      // the user token budget (min with n_max); <= 0: none
    int n_max;           // sampled-token cap of the loop
    int exact;           // decide the forcing rule from the exact log-sum-exp every step
    int ldr;             // row stride (floats) of the stored rows
};
struct FwWinStream {
    int seek_cs, seek_end_cs, has_prior;                               // set by the host
    int n_dec, has_ts, seek_delta_cs, result_len, done, n_exact;       // loop state
};
// one stream's row is filtered by WIN_NB blocks, each leaving its partial
// results in a slot; the last block to count (cnt[s], zero between launches)
// merges them
#ifndef WIN_NB
#define WIN_NB 16
#endif
// the last block merges the slots one per lane of a 64-wide wave
static_assert(WIN_NB >= 1 && WIN_NB <= 64, "WIN_NB must be in 1..64");
struct FwWinPart {
    unsigned long long ka, kt;  // argmax keys: every lane, the timestamp lanes
    float mall, mtxt, mts, sb;  // maxima (all, text, timestamp lanes); sum of expf(u - mall) over the block's lanes
};
bool fw_win_select_ok(int V);
void fw_launch_win_select(hipStream_t st, const float *logits, int ldl, const FwWinCfg &c, FwWinStream *ws,
                          int32_t *hist, int hist_cap, float *rows, uint8_t *forced, float *scratch, int32_t *tok,
                          int *posp, int *ndone, FwWinPart *part, int *cnt, int ns);
void fw_launch_win_plogs(hipStream_t st, const float *rows, const float *nsrow, const FwWinCfg &c,
                         const FwWinStream *ws, const int32_t *hist, int hist_cap, const uint8_t *forced,
                         float *plogs, float *nslp, int ns);

// int8 decoder arm (dec_fast.hip)
// seq: the LayerNorm's mean and variance are the reference's sequential f64
// sums (bit for bit on every row; exact mode), else the wave's tree sums
void fw_launch_ln_quant(hipStream_t st, const float *x, float *y, const float *w, const float *b, int d, int rows,
                        int8_t *xq, float *xs, int seq = 0);
// rps > 0: row s sits at position *posp + s / rps (a prefill chunk of rps
// streams); else every row at *posp
void fw_launch_embed_ln(hipStream_t st, const int32_t *tok, const int *posp, const uint16_t *emb, const float *pemb,
                        float *x, int d, int ns, const float *w, const float *b, float *ln_y, int8_t *xq, float *xs,
                        int rps = 0, int seq = 0);
int fw_gemv_i8m_blocks(int N);
// W of fw_launch_gemv_i8m is stored as MFMA operand fragments: bytes needed
// for an [N, K] matrix (K % 64 == 0), and the repacking of a row-major one
size_t fw_gemv_frag_bytes(int N, int K);
void fw_launch_pack_gemv_frags(hipStream_t st, const int8_t *W, int8_t *Wf, int N, int K);
void fw_launch_gemv_i8m(hipStream_t st, const int8_t *W, const float *sw, const float *bias, const int8_t *xq,
                        const float *xs, float *y, int N, int K, int ns, int ldy, int mode, const float *gelu_tab,
                        const fwhip_filter *filt, const int *initialp, unsigned long long *keys,
                        const float *xf = nullptr, const float *pmax = nullptr, int H = 0);
// cnt (an int that is zero between launches): one block per stream, the last
// to finish doing the bookkeeping; else one block walks every stream
void fw_launch_argmax_finish(hipStream_t st, const unsigned long long *keys, int nblk, int ns, int32_t *tok,
                             int32_t *hist, int hist_cap, int *posp, int *initialp, int *stepp, int advance,
                             int *cnt = nullptr);
int fw_launch_gemv_blk2(hipStream_t st, const int8_t *W, const float *sc, const float *bias, const float *x, float *y,
                        int N, int K, int ns, int ldy, int mode, int n_cu);
// pmax (nullable): [ns, H] max |output| of each head block, for a consumer
// that quantizes the rows itself (fw_launch_gemv_i8m with xf)
// rows > 0: a prefill chunk of `rows` rows, row r = stream r % ns at position
// *posp + r / ns, its k/v already appended (append = 0, fw_launch_kv_append)
void fw_launch_self_attn2(hipStream_t st, const float *qkv, void *kc, void *vc, float *att, const int *posp, int d,
                          int H, int nctx, int L, int layer, int ns, float scale, float *pmax = nullptr, int rows = 0,
                          int append = 1, int kv32 = 0);
// the k/v of every row of a prefill chunk into the caches
void fw_launch_kv_append(hipStream_t st, const float *qkv, void *kc, void *vc, const int *posp, int d, int nctx,
                         int L, int layer, int ns, int rows, int kv32);
// The int8 arm's self-attention sublayer: attention LayerNorm of the residual
// rows x, the fused q/k/v projection (int8 rows wqkv [3d, d], row scales sqkv,
// bias bqkv), cache append and attention; per-head output maxima into pmax.
// With emb (layer 0) the rows are first formed as the token embeddings
// f16(emb[tok]) + pemb[pos] and stored to x.
void fw_launch_self_attn_fused(hipStream_t st, const int8_t *wqkv, const float *sqkv, const float *bqkv, float *x,
                               const float *lnw, const float *lnb, void *kc, void *vc, float *att,
                               const int *posp, int d, int H, int nctx, int L, int layer, int ns, float scale,
                               float *pmax, const int32_t *tok = nullptr, const uint16_t *emb = nullptr,
                               const float *pemb = nullptr, int lnseq = 0, int kv32 = 0);
// q = Wq LN(x): the cross LayerNorm (lnw, lnb) of the residual rows x and the
// int8 cross q projection [d, d] (row scales swq, bias bq) run in the kernel.
// With vbs (FW_CROSS_V_BLOCK) cvt is the block-int8 V^T (rows of stride Tq,
// 32-frame blocks, scales vbs [.., 64, ceil(T / 32)]) and p stays f32.
void fw_launch_cross_attn_i8v2(hipStream_t st, const int8_t *wq, const float *swq, const float *bq, const float *x,
                               const float *lnw, const float *lnb, const int8_t *ck, const float *cks, const int8_t *cvt,
                               const float *cvs, float *att, int d, int T, int Tq, int H, int L, int layer, int ns,
                               float scale, float *pmax = nullptr, int lnseq = 0, const float *vbs = nullptr);
void fw_launch_quant_f16_rows_ld(hipStream_t st, const uint16_t *src, int8_t *q, float *s, int rows, int n, int ldq);
int fw_logits_keys_blocks(int V);
void fw_launch_logits_keys(hipStream_t st, const float *logits, int V, int ns, const fwhip_filter *filt,
                           const int *initialp, unsigned long long *keys);

// load-time quantizers (load_kernels.hip); ldq: output row stride (0: inp)
void fw_launch_quant_blocked(hipStream_t st, const uint16_t *w, int8_t *q, float *s, int64_t out, int inp,
                             int block, int ldq = 0);
void fw_launch_quant_i7(hipStream_t st, const uint16_t *w, int8_t *q, float *s, int32_t *cs, int64_t out,
                        int inp, int ef);
void fw_launch_quant_enc_i8(hipStream_t st, const uint16_t *w, int8_t *q, float *s, int64_t out, int inp);
