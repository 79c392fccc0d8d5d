/*
 * fwhip.h — C ABI of the MI355X (gfx950) Whisper engine hot path.
 *
 * This is the drop-in boundary for franken_whisper's native engine
 * (src/native_engine/): the encoder forward and the greedy decoder step run on
 * one GPU behind these entry points, and the Rust engine (or any other host)
 * binds them through a thin FFI crate.  Every entry point names the reference
 * interface it replaces (file:line under the reference tree).
 *
 * Conventions
 *  - Plain C types only: pointers, sizes, int32/int64, float.  No GPU-runtime
 *    types cross the boundary.
 *  - "dev" pointers are device addresses obtained from fwhip_malloc (or any
 *    allocation on the context's device); "host" pointers are ordinary memory.
 *  - Weights are passed as host pointers in ggml layout ([out, in] row-major for
 *    linears, f16 stored as raw IEEE binary16 bits in uint16_t, f32 otherwise).
 *    The library copies, quantizes (with the reference quantizers) and uploads
 *    them once; the caller keeps ownership of its buffers.
 *  - Status codes mirror fw-ios/include/fw_ios.h:8-12 and FwError
 *    (src/error.rs:75-115): FWHIP_ERR_INVALID ~ FwError::InvalidRequest,
 *    FWHIP_ERR_CANCELLED ~ FwError::Cancelled, FWHIP_ERR_UNSUPPORTED tells the
 *    caller to fall back to its CPU route with a named reason (the pattern of
 *    encoder.rs:1700-1725 / 1993-2003).
 *  - fwhip_last_error() returns a thread-local message for the last failing call
 *    on the calling thread (fw_ios.h:14-20 pattern).
 *  - Threading: a context owns one HIP stream.  Calls on one context must be
 *    serialized by the caller; separate contexts may run concurrently.
 */
#ifndef FWHIP_H
#define FWHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FWHIP_ABI_VERSION 2

typedef int32_t fwhip_status;
#define FWHIP_OK 0
#define FWHIP_ERR_GENERIC 1
#define FWHIP_ERR_INVALID 2
#define FWHIP_ERR_UNSUPPORTED 5
#define FWHIP_ERR_CANCELLED 6

typedef struct fwhip_ctx fwhip_ctx;
typedef struct fwhip_encoder fwhip_encoder;
typedef struct fwhip_decoder fwhip_decoder;
typedef struct fwhip_dstate fwhip_dstate;

/* Model hyper-parameters: the eleven ggml header fields of WhisperHParams
 * (src/native_engine/mod.rs:56-77), minus ftype. */
typedef struct fwhip_hparams {
    int32_t n_vocab;
    int32_t n_audio_ctx;
    int32_t n_audio_state;
    int32_t n_audio_head;
    int32_t n_audio_layer;
    int32_t n_text_ctx;
    int32_t n_text_state;
    int32_t n_text_head;
    int32_t n_text_layer;
    int32_t n_mels;
} fwhip_hparams;

/* One encoder block, ggml tensor names encoder.blocks.{i}.* (encoder.rs:78-120). */
typedef struct fwhip_enc_layer {
    const float *attn_ln_w, *attn_ln_b;         /* [d] */
    const uint16_t *q_w; const float *q_b;       /* [d,d] f16, [d] */
    const uint16_t *k_w;                         /* [d,d] f16, no bias */
    const uint16_t *v_w; const float *v_b;
    const uint16_t *o_w; const float *o_b;
    const float *mlp_ln_w, *mlp_ln_b;
    const uint16_t *fc1_w; const float *fc1_b;   /* [4d,d] f16, [4d] */
    const uint16_t *fc2_w; const float *fc2_b;   /* [d,4d] f16, [d]  */
} fwhip_enc_layer;

/* Encoder weights (EncoderWeights, encoder.rs:129-161; load encoder.rs:772-1029). */
typedef struct fwhip_encoder_weights {
    fwhip_hparams hp;
    const uint16_t *conv1_w; const float *conv1_b;  /* [d, n_mels, 3] f16 */
    const uint16_t *conv2_w; const float *conv2_b;  /* [d, d, 3] f16 */
    const float *pos_emb;                           /* [n_audio_ctx, d] f32 */
    const fwhip_enc_layer *layers;                  /* n_audio_layer entries */
    const float *ln_post_w, *ln_post_b;
} fwhip_encoder_weights;

/* One decoder block, ggml names decoder.blocks.{i}.* (decoder.rs:487-512). */
typedef struct fwhip_dec_layer {
    const float *attn_ln_w, *attn_ln_b;
    const uint16_t *q_w; const float *q_b;
    const uint16_t *k_w;                         /* no bias */
    const uint16_t *v_w; const float *v_b;
    const uint16_t *o_w; const float *o_b;
    const float *cross_ln_w, *cross_ln_b;
    const uint16_t *cq_w; const float *cq_b;
    const uint16_t *ck_w;                        /* no bias */
    const uint16_t *cv_w; const float *cv_b;
    const uint16_t *co_w; const float *co_b;
    const float *mlp_ln_w, *mlp_ln_b;
    const uint16_t *fc1_w; const float *fc1_b;
    const uint16_t *fc2_w; const float *fc2_b;
} fwhip_dec_layer;

/* Decoder weights (DecoderWeights, decoder.rs:514-545; load decoder.rs:752-932). */
typedef struct fwhip_decoder_weights {
    fwhip_hparams hp;
    const uint16_t *tok_emb;                     /* [n_vocab, d] f16 (tied logits head) */
    const float *pos_emb;                        /* [n_text_ctx, d] f32 */
    const fwhip_dec_layer *layers;               /* n_text_layer entries */
    const float *ln_w, *ln_b;
} fwhip_decoder_weights;

/* Encoder precision plan (encoder.rs:474-512, mod.rs:777-841). */
#define FWHIP_ENC_F32 0   /* default f32 path: every linear f32 */
#define FWHIP_ENC_INT8 1  /* FW_ENC_ATTN_OUT_I8I32 quality-safe plan: q/k/v/fc1/fc2 i7
                             (error-feedback weight quant), attn.out full i8 */

/* Decoder arm (Appendix-A flag sets; mod.rs:335-1110, decoder.rs:776-892). */
#define FWHIP_DEC_INT8 0  /* reference default: int8 fused QKV, attn_out, cross_q,
                             cross_out, mlp_0, block-int8 mlp_2, int8 cross K/V,
                             int8 tied logits; f16 KV cache */
#define FWHIP_DEC_F16 1   /* pure-f16 arm: every GEMV f16 (dot_f16c order),
                             f16 cross K/V, f16 tied logits; f16 KV cache */

/* Greedy filter for the no-timestamps decode (process_logits, decode.rs:702-867,
 * with FilterConfig decode.rs:3031-3040 and no_timestamps = true).  Special ids
 * as derived by Tokenizer::from_vocab (tokenizer.rs:230-300). */
typedef struct fwhip_filter {
    int32_t eot, sot, sot_prev, solm, no_speech, no_timestamps;
    int32_t translate, transcribe, timestamp_begin;
    int32_t space_token;      /* id of " " (suppress_blank), -1 if absent */
    int32_t n_languages;      /* language tokens sot+1 .. sot+n_languages are masked */
} fwhip_filter;

/* The arithmetic one encoder GEMM family ran in one forward (GemmPrecision,
 * encoder.rs:1885-1927).  fwhip_gemm_precision_str gives the reference's
 * stable report strings, plus "f16_pair" for this engine's MFMA form of f32. */
#define FWHIP_PREC_F32 0          /* "f32": f32 operands and accumulation (exact mode: the
                                     reference's strict-parity order) */
#define FWHIP_PREC_I7 1           /* "i7": 7-bit weights x u8 activations, i32 accumulation */
#define FWHIP_PREC_I8 2           /* "i8": i8 weights x i8 activations, i32 accumulation */
#define FWHIP_PREC_F16 3          /* "f16" (reference values; not run by this engine) */
#define FWHIP_PREC_F16_WEIGHTS 4  /* "f16_weights" */
#define FWHIP_PREC_Q8_0_WEIGHTS 5 /* "q8_0_weights" */
#define FWHIP_PREC_F16_KV 6       /* "f16_kv" */
#define FWHIP_PREC_MIXED 7        /* "mixed" */
#define FWHIP_PREC_F16_PAIR 8     /* "f16_pair": each f32 operand carried as an f16 hi/lo
                                     pair, three f16 MFMA products (hi*hi + hi*lo + lo*hi)
                                     accumulated in f32, about 2^-21 relative of f32 */
/* GEMM families, in EncoderPrecision::families order (encoder.rs:1929-1985). */
#define FWHIP_FAM_CONV_STEM 0
#define FWHIP_FAM_ATTN_QKV 1
#define FWHIP_FAM_ATTENTION 2
#define FWHIP_FAM_ATTN_OUT 3
#define FWHIP_FAM_MLP_FC1 4
#define FWHIP_FAM_MLP_FC2 5
#define FWHIP_N_FAM 6

/* Per-forward execution record (EncoderExecution, encoder.rs:1987-2003):
 * what computed this forward, returned by the forward itself.
 *  - route: "hip:gfx950:int8" / "hip:gfx950:f32", with ":exact" when the
 *    strict-parity arithmetic ran;
 *  - family[f]: FWHIP_PREC_* of family FWHIP_FAM_f (EncoderPrecision): on the
 *    int8 plan in fast mode conv_stem and attention are f16_pair, q/k/v and
 *    the MLP i7, attn_out i8; exact mode runs f32 where fast mode runs
 *    f16_pair; the f32 plan is f16_pair (fast) or f32 (exact) throughout;
 *  - precision_source: what chose family[] (EncoderExecution::
 *    precision_source): "fwhip_encoder_load" (the plan, fast mode),
 *    "fwhip_encoder_set_exact" (exact mode), or "f16_pair_range" when a fast
 *    forward met a value past the f16 range (|v| >= 65520, where an f16 pair
 *    cannot carry it) and ran again in exact mode, whose results it returns. */
typedef struct fwhip_exec_record {
    char route[48];
    int32_t precision;        /* FWHIP_ENC_* (the load-time plan) */
    int32_t n_windows;
    double device_ms;         /* stream time of the forward */
    int32_t family[FWHIP_N_FAM];
    char precision_source[32];
} fwhip_exec_record;

/* ---- context, memory ---------------------------------------------------- */

/* Open device `device` and create a context with its own stream.
 * FWHIP_ERR_UNSUPPORTED when no gfx950 device is visible. */
fwhip_status fwhip_init(int32_t device, fwhip_ctx **out);
void fwhip_destroy(fwhip_ctx *ctx);
const char *fwhip_last_error(void);
int32_t fwhip_abi_version(void);

fwhip_status fwhip_malloc(fwhip_ctx *ctx, size_t bytes, void **dev);
fwhip_status fwhip_free(fwhip_ctx *ctx, void *dev);
fwhip_status fwhip_upload(fwhip_ctx *ctx, void *dev, const void *host, size_t bytes);
fwhip_status fwhip_download(fwhip_ctx *ctx, void *host, const void *dev, size_t bytes);
fwhip_status fwhip_synchronize(fwhip_ctx *ctx);

/* GemmPrecision::as_str (encoder.rs:1912-1927) of a FWHIP_PREC_* value
 * ("f16_pair" for FWHIP_PREC_F16_PAIR), NULL for an unknown value. */
const char *fwhip_gemm_precision_str(int32_t prec);

/* Cancellation between layers and tokens, the checkpoint() contract of
 * nn.rs:29-37 / encoder.rs:1628 / decoder.rs:1877: the next layer boundary
 * returns FWHIP_ERR_CANCELLED and clears the flag. */
fwhip_status fwhip_request_cancel(fwhip_ctx *ctx);

/* Kernel timing: when enabled, the library brackets every launch of kernel
 * class `kclass` with events on its stream; fwhip_kernel_stats returns the
 * launch count and summed device milliseconds since the last reset. */
#define FWHIP_K_ENC_GEMM_I8 1
#define FWHIP_K_ENC_GEMM_F32 2
#define FWHIP_K_ENC_ATTN 3
#define FWHIP_K_DEC_GEMV 4
#define FWHIP_K_DEC_LOGITS 5
#define FWHIP_K_DEC_CROSS 6  /* cross K/V precompute (fast mode) */
#define FWHIP_K_DEC_STEP 7   /* one sampled decoder step of the greedy loop, or a one-token
                                fwhip_decoder_step (forward, logits and argmax) */
#define FWHIP_K_DEQUANT 8    /* ggml payload decode (fwhip_dequant, fwhip_ggml_tensor_f32) */
#define FWHIP_K_DEC_XATTN 9  /* the fused cross-attention sublayer (LayerNorm, q, attention over the
                                cross K/V) of a one-token fwhip_decoder_step */
fwhip_status fwhip_kernel_timing(fwhip_ctx *ctx, int32_t enable);
fwhip_status fwhip_kernel_stats(fwhip_ctx *ctx, int32_t kclass, int64_t *launches,
                                double *total_ms, double *work_units);

/* ---- encoder ------------------------------------------------------------ */

/* Replaces EncoderWeights::from_ggml (encoder.rs:764) + the quant plan
 * (encoder.rs:838-843).  precision = FWHIP_ENC_F32 | FWHIP_ENC_INT8. */
fwhip_status fwhip_encoder_load(fwhip_ctx *ctx, const fwhip_encoder_weights *w,
                                int32_t precision, fwhip_encoder **out);
void fwhip_encoder_free(fwhip_encoder *enc);

/* Replaces encoder::forward_from_full_mel_window (encoder.rs:1224-1238) for a
 * batch of windows: window b is frames [frame_offsets[b], +n_frames) of the
 * mel-major log-mel `mel_dev` ([n_mels, mel_frames] f32), padded with -1.5 past
 * the end (encoder.rs:684-714).  Output `out_dev` is [n_windows, n_frames/2, d]
 * f32 (after ln_post).  n_frames must be even and <= 2*n_audio_ctx
 * (encoder.rs:716-737).  rec may be NULL. */
fwhip_status fwhip_encoder_forward(fwhip_encoder *enc, const float *mel_dev, int64_t mel_frames,
                                   const int64_t *frame_offsets, int32_t n_windows,
                                   int32_t n_frames, float *out_dev, fwhip_exec_record *rec);

/* Exact mode (exact = 1): reproduce the reference's strict-parity arithmetic
 * (FT_SGEMM_STRICT_PARITY=1, FW_ATTN_NO_SDPA=1; nn.rs:587-604, 6035-6131)
 * for every f32 operation of the forward — sequential-k f32 GEMMs for the
 * conv stem (and every linear on the f32 plan), per-head attention with a
 * glibc-exact softmax — so encoder states are bit-identical to the reference
 * CPU path.  A parity mode, orders of magnitude slower than the default fast
 * mode (exact = 0: MFMA f16-pair GEMMs and flash attention, within the 1e-3
 * tolerance; int8 accumulators are exact in both). */
fwhip_status fwhip_encoder_set_exact(fwhip_encoder *enc, int32_t exact);

/* ToMe token merging (FW_TOME_R / FW_TOME_LAYER, encoder.rs:1264-1337 and
 * 1590-1632; the single-shot schedule unless fwhip_encoder_set_tome_schedule
 * says otherwise): merge r of the rows of every window after block `after`
 * (0-based) by bipartite soft matching (tome_merge, encoder.rs:1403-1506), run
 * the later blocks on the merged rows and unmerge before ln_post
 * (tome_unmerge, encoder.rs:1509-1517).  The merge runs when rows > r + 2 and
 * rows - r >= the floor (128 unless set).  r = 0 (the initial setting) is the
 * un-merged encoder, FW_TOME_R=0; r < 0 applies the reference's default for
 * the model (tome_r_for: 500 after block 3 on the 20-head large class for full
 * 1500-row windows, none otherwise).  The merge itself is computed in the
 * strict-parity arithmetic in both modes (its similarity GEMM in ascending-k
 * sequential f32), so in exact mode the whole forward stays bit-identical to
 * the reference's strict mode with the same FW_TOME_R. */
fwhip_status fwhip_encoder_set_tome(fwhip_encoder *enc, int32_t r, int32_t after);

/* Replaces FW_TOME_EVERY / FW_TOME_FLOOR (tome_every_layers / tome_floor,
 * encoder.rs:1379-1402; defaults 0 and 128, the initial setting here).
 * every = 0: the single-shot schedule (one merge after block `after`).
 * every > 0: the progressive schedule, a merge after block `after` and again
 * after every `every` blocks, the unmerge map composed through each merge
 * (one unmerge before ln_post).  A merge is skipped when it would leave fewer
 * than `floor` rows.  Negative values are FWHIP_ERR_INVALID. */
fwhip_status fwhip_encoder_set_tome_schedule(fwhip_encoder *enc, int32_t every, int32_t floor);

/* tome_merge of rows x_dev [n_windows, T, d] (f32) per window: merged rows
 * into merged_dev [n_windows, T - r', d] (r' = min(r, ceil(T/2), T - 1)) and
 * the unmerge map umap_dev [n_windows, T] (original row -> merged row);
 * *out_rows = T - r'.  A parity entry point for the encoder's merge step; it
 * allocates its workspace per call. */
fwhip_status fwhip_tome_merge(fwhip_ctx *ctx, const float *x_dev, int32_t n_windows, int32_t T, int32_t d, int32_t r,
                              float *merged_dev, int32_t *umap_dev, int32_t *out_rows);

/* Same contract, time-major input already windowed: `x_dev` is
 * [n_windows, n_frames, n_mels] (the Mat that forward_time_major consumes,
 * encoder.rs:1520). */
fwhip_status fwhip_encoder_forward_time_major(fwhip_encoder *enc, const float *x_dev,
                                              int32_t n_windows, int32_t n_frames,
                                              float *out_dev, fwhip_exec_record *rec);

/* Per-GEMM parity of the int8 plan: quantize f32 rows x_dev [m, in] with the
 * reference quantizer for linear `which` of block `layer` (0 q, 1 k, 2 v:
 * quantize_act_i7 nn.rs:1443; 3 attn.out: quant_row_i8 encoder.rs:2468; 4 fc1:
 * quantize_act_i7; 5 fc2: quantize_act_i7_gelu nn.rs:1791), run the i8 GEMM
 * and write the exact i32 accumulators acc_dev [m, out] (= the reference's
 * maddubs sum - 128*colsum, nn.rs:1660-1700, or its i8 dot, encoder.rs:2573)
 * and the epilogue output y_dev [m, out] ((f32)acc*s_x*s_w + b). */
fwhip_status fwhip_encoder_gemm_i8(fwhip_encoder *enc, int32_t layer, int32_t which, const float *x_dev,
                                   int32_t m, int32_t *acc_dev, float *y_dev);

/* Per-GEMM parity of the fused epilogues the int8 forward runs, on rows x_dev
 * [n_windows * n_tokens, d] quantized with quantize_act_i7 (nn.rs:1443):
 *   which 0: the fused q/k/v GEMM (matmul_bias_i7_quantized nn.rs:1537-1771,
 *     fused head-major as attention_from_i7_qkv nn.rs:5836-5877) with each
 *     epilogue value v split into f16 hi = f16(v), lo = f16(v - hi).  out16_dev
 *     receives Q hi, Q lo, K hi, K lo, each [n_windows, H, n_tokens, 64], then
 *     V^T hi, V^T lo, each [n_windows, H, 64, Tp] (Tp = n_tokens rounded up to
 *     64, zero padded; key t of a 16-key group at position t with bits 2 and 3
 *     swapped).
 *   which 4: fc1 in GELU-index form: out16_dev [m, 4d] holds the f16 bits of v
 *     (the reference GELU's table index, nn.rs:4603-4687) when |v| < 9.98, else
 *     0xffff with v itself in side_dev [m, 4d].
 * A test entry point: it allocates its quantized operand per call. */
fwhip_status fwhip_encoder_gemm_i8_fused(fwhip_encoder *enc, int32_t layer, int32_t which, const float *x_dev,
                                         int32_t n_windows, int32_t n_tokens, uint16_t *out16_dev, float *side_dev);

/* ---- decoder ------------------------------------------------------------ */

/* Replaces DecoderWeights::from_ggml (decoder.rs:752-932).  arm = FWHIP_DEC_*. */
fwhip_status fwhip_decoder_load(fwhip_ctx *ctx, const fwhip_decoder_weights *w, int32_t arm,
                                fwhip_decoder **out);
void fwhip_decoder_free(fwhip_decoder *dec);

/* Exact mode (exact = 1): the cross K/V precompute of fwhip_dstate_set_cross
 * (DecoderState::new, decoder.rs:1049-1069) is the strict-parity sequential-k
 * f32 GEMM (FT_SGEMM_STRICT_PARITY=1, nn.rs:587-604), so logits are
 * bit-identical to the reference's strict mode.  Fast mode (exact = 0, the
 * default) makes every layer's cross K and V in one f16-pair MFMA GEMM (each
 * K/V value within ~1e-7 relative before its f16 rounding; the reference's
 * default ft sgemm has no pinned summation order either).  In exact mode every
 * LayerNorm of the token step also sums its f64 mean and variance in the
 * reference's sequential index order (layer_norm, nn.rs:4425-4438), so logits
 * and tokens are bit-identical whatever the rows; fast mode sums them in a
 * wave tree, whose variance differs in its last f64 bits in most rows (an
 * f32 output moved by it in 6 of 1.2 M Gaussian rows of width 1280).  The
 * kernels are the same in both modes apart from that sum. */
fwhip_status fwhip_decoder_set_exact(fwhip_decoder *dec, int32_t exact);

/* Replaces FW_KV_F16 (kv_f16_enabled, nn.rs:5097-5109), read when a state is
 * made (KvCache::new): the self-attention cache of the states that
 * fwhip_dstate_new makes after this call.  on = 1 (this library's initial
 * setting): K/V rows rounded to f16 on append (KvCache::append,
 * nn.rs:5352-5416); on = 0: f32 rows as computed, the reference's default
 * (FW_KV_F16 unset; attention_decode_step, nn.rs:6340-6400).  Attention reads
 * either as f32 with the same arithmetic, so the two differ only by the f16
 * rounding of the cached rows; the f32 cache takes twice the memory
 * (4 x n_layer x n_text_ctx x d x 2 bytes per stream). */
fwhip_status fwhip_decoder_set_kv_f16(fwhip_decoder *dec, int32_t on);

/* Replaces FW_CROSS_V_BLOCK (cross_v_block_enabled, decoder.rs:1496-1520; off
 * by default), read when a state is made: on the int8 arm, the states that
 * fwhip_dstate_new makes after fwhip_decoder_set_cross_v_block(dec, 1) keep
 * each head's cross V^T block-quantized along the encoder frames
 * (quantize_f16_to_i8_blocked, 32 frames per scale, decoder.rs:1249-1263) and
 * run the cross attention's value pass as gemv_i8w_f32a_blocked on the f32
 * softmax weights (decoder.rs:1605-1608) instead of gemv_i8.  No effect on the
 * f16 arm. */
fwhip_status fwhip_decoder_set_cross_v_block(fwhip_decoder *dec, int32_t on);

/* A cohort of n_streams independent DecoderStates (decoder.rs:980-1027), each
 * with its own f16 self-attention KV cache (KvCache, nn.rs:5138) of
 * n_text_ctx tokens and its own cross K/V over enc_frames encoder rows
 * (FWHIP_DEC_INT8: enc_frames <= 1536; Whisper's encoder emits 1500). */
fwhip_status fwhip_dstate_new(fwhip_decoder *dec, int32_t n_streams, int32_t enc_frames,
                              fwhip_dstate **out);
void fwhip_dstate_free(fwhip_dstate *st);

/* Replaces DecoderState::new (decoder.rs:1040-1285): cross K/V precompute for
 * every stream from `enc_dev` ([n_streams, enc_frames, d] f32), then reset the
 * self-attention caches. */
fwhip_status fwhip_dstate_set_cross(fwhip_dstate *st, const float *enc_dev);

/* DecoderState::reset (decoder.rs:1289): clear the self-attention caches. */
fwhip_status fwhip_dstate_reset(fwhip_dstate *st);
int32_t fwhip_dstate_len(const fwhip_dstate *st, int32_t stream);

/* Replaces decoder::forward_step (decoder.rs:2048-2085) and, for n_streams > 1,
 * forward_step_batch (decoder.rs:1907-2046): every stream consumes `tq` tokens
 * (host `tokens`, [n_streams, tq]); tq > 1 is the prompt prefill.  Writes the
 * last position's logits to `logits_dev` ([n_streams, n_vocab] f32, may be NULL)
 * and, when `argmax_host` is non-NULL, the filtered first-index argmax
 * (process_logits + argmax, decode.rs:702-867, 1727-1790) per stream; `filter`
 * may be NULL for the raw argmax.  `initial` marks the first sampling step
 * (suppress_blank). */
fwhip_status fwhip_decoder_step(fwhip_dstate *st, const int32_t *tokens, int32_t tq,
                                float *logits_dev, int32_t *argmax_host,
                                const fwhip_filter *filter, int32_t initial);

/* Read back decoder-state buffers for stream `stream` into host memory
 * (the cross K/V built by DecoderState::new and the self-attention cache, for
 * parity checks; decoder.rs:1129-1245 layouts):
 *   FWHIP_DS_CROSS_K_F16   [n_layer, n_head, enc_frames, 64] f16 (scaled keys)
 *   FWHIP_DS_CROSS_VT_F16  [n_layer, n_head, 64, enc_frames] f16
 *   FWHIP_DS_KV_K, _KV_V   [n_layer, n_text_ctx, d] f16, or f32 for a state made
 *                          with fwhip_decoder_set_kv_f16(dec, 0)
 * `bytes` must equal the buffer size. */
#define FWHIP_DS_CROSS_K_F16 1
#define FWHIP_DS_CROSS_VT_F16 2
#define FWHIP_DS_KV_K 3
#define FWHIP_DS_KV_V 4
fwhip_status fwhip_dstate_read(const fwhip_dstate *st, int32_t what, int32_t stream, void *host,
                               size_t bytes);

/* Greedy no-timestamps decode of every stream (the loop of
 * transcribe_samples_uncached, decode.rs:3429-3566, with max_context = 0):
 * prefill `prompt` (n_prompt tokens, shared by all streams), then argmax ->
 * step until eot or n_max_tokens sampled tokens.  out_tokens is host
 * [n_streams, n_max_tokens]; out_len[s] receives the sampled count including a
 * final eot. */
fwhip_status fwhip_decode_greedy(fwhip_dstate *st, const int32_t *prompt, int32_t n_prompt,
                                 int32_t n_max_tokens, const fwhip_filter *filter,
                                 int32_t *out_tokens, int32_t *out_len);

/* The window decode loop (the greedy loop of transcribe_samples_uncached,
 * decode.rs:3456-3566, beam 1, temperature 0) with process_logits in full
 * (decode.rs:702-867: blank/eot at the first step, control, task and language
 * tokens, timestamps in no-timestamps mode, the user token budget, timestamp
 * pairing, the initial-timestamp cap, the monotone timestamp floor and the
 * timestamp-mass forcing rule).  FilterConfig (decode.rs:671-693) beyond the
 * filter's ids; suppress_blank is on, suppress_nst off, as the driver sets
 * them. */
typedef struct fwhip_window_cfg {
    int32_t timestamps;      /* 0: no-timestamps mode */
    int32_t max_initial_tid; /* round(1.0 / (30 / n_audio_ctx)); < 0: no cap */
    int32_t max_tokens;      /* the user token budget; <= 0: none (min with n_max is applied) */
    int32_t n_max;           /* sampled-token cap: n_text_ctx / 2 - 4 */
    int32_t exact;           /* 1: decide the forcing rule from the exact log-softmax on
                                every step (the default recomputes it only when the
                                decision is within 1e-3 of its threshold) */
} fwhip_window_cfg;

/* One stream of the window loop: seek_cs / seek_end_cs / has_prior_segments
 * in; the rest out (the loop's decoded, result_len, has_ts, seek_delta_cs;
 * no_speech_logprob: the no-speech token's log-probability on the prefill
 * logits, compute_logprobs decode.rs:1437-1448; n_exact: steps that took the
 * exact forcing decision). */
typedef struct fwhip_window_stream {
    int32_t seek_cs, seek_end_cs, has_prior_segments;
    int32_t n_tokens, result_len, has_ts, seek_delta_cs, n_exact;
    float no_speech_logprob;
} fwhip_window_stream;

/* Run the window loop for every stream of `st` (cross K/V already set by
 * fwhip_dstate_set_cross): prefill `prompt` (n_prompt tokens, shared by the
 * streams), then process_logits + argmax -> step on the device until every
 * stream ends.  out_tokens / out_plogs are host [n_streams, cfg->n_max]: the
 * decoded tokens (decoded, decode.rs:3476) and each token's log-probability
 * (plogs: compute_logprobs of the filtered logits at the chosen token). */
fwhip_status fwhip_decode_window(fwhip_dstate *st, const int32_t *prompt, int32_t n_prompt,
                                 const fwhip_filter *filter, const fwhip_window_cfg *cfg,
                                 fwhip_window_stream *streams, int32_t *out_tokens, float *out_plogs);

/* ---- the window driver ---------------------------------------------------- */

/* A byte-level vocabulary (Tokenizer's token bytes, tokenizer.rs:230-300):
 * token i is bytes[offsets[i] .. offsets[i + 1]); offsets has n_tokens + 1
 * entries.  Tokens >= eot are special and never rendered. */
typedef struct fwhip_vocab {
    int32_t n_tokens;
    const uint8_t *bytes;
    const uint64_t *offsets;
} fwhip_vocab;

/* The DecodeParams fields (decode.rs:239-447) and process switches the greedy
 * driver reads. */
typedef struct fwhip_transcribe_params {
    int32_t timestamps;           /* DecodeParams.timestamps (segment timestamps) */
    int32_t max_context;          /* DecodeParams.max_context when max_context_set:
                                     < 0 the default (n_text_ctx / 2), 0 no carried prompt, n a cap */
    int32_t max_context_set;      /* 0: max_context is None */
    int32_t max_tokens;           /* DecodeParams.max_text_ctx, the user token budget; <= 0: none */
    int32_t no_context;           /* FW_NO_CONTEXT: never condition on previous text */
    int32_t retry_failed_window;  /* FW_RETRY_FAILED_WINDOW (the reference's default: 1) */
    int32_t tiny_en_ts_context;   /* FW_TINY_EN_TS_CONTEXT: keep tiny.en's carried context with timestamps */
    int32_t carry_initial_prompt; /* DecodeParams.carry_initial_prompt */
    const int32_t *initial_prompt;  /* Tokenizer::encode of DecodeParams.initial_prompt (may be NULL) */
    int32_t n_initial_prompt;
    const int32_t *sot_sequence;    /* Tokenizer::sot_sequence(language, translate, timestamps) */
    int32_t n_sot;
    double no_speech_threshold;   /* the quality gates (decode.rs:1082-1104): 0.6 */
    double logprob_threshold;     /* -1.0 */
    int32_t exact_forcing;        /* fwhip_window_cfg.exact */
} fwhip_transcribe_params;

typedef struct fwhip_transcript fwhip_transcript;

/* TranscriptionSegment: centisecond bounds, trimmed text (UTF-8, owned by the
 * transcript), text confidence (NaN when the reference gives None). */
typedef struct fwhip_segment_info {
    int64_t start_cs, end_cs;
    const char *text;
    double confidence;
} fwhip_segment_info;

/* WindowStats plus the window's decode: every accepted window in order;
 * `dropped` marks the reference's DroppedWindow records (a later window that
 * closed no timestamp and is not silence), `retried` a window decoded again
 * without its carried prompt; tokens / plogs (owned by the transcript) are the
 * window's decoded tokens and their log-probabilities. */
typedef struct fwhip_window_info {
    int64_t seek_cs;
    double avg_logprob, no_speech_prob;
    int32_t result_len, n_tokens, has_ts, seek_delta_cs, no_speech, dropped, retried;
    const int32_t *tokens;
    const float *plogs;
} fwhip_window_info;

/* Replaces transcribe_samples (decode.rs:2880-2955 -> 2956-3960) on its
 * greedy path (beam 1, no temperature fallback, no word timestamps, the
 * language given by the sot sequence, full 30 s windows): the log-mel of the
 * whole audio (samples_dev, n_samples 16 kHz f32 on the device; filters_dev
 * [n_mel, 201]), then window by window the encoder at the seek, the window
 * loop (fwhip_decode_window) and the rules between windows — prompt carry,
 * the short-tail prompt clear, the no-speech gate, the failed-window retry,
 * the single-timestamp-ending skip, segment building, the seek advance.
 * Without timestamps and without a carried prompt the windows are
 * independent and run as batched cohorts, with the same results.  enc and dec
 * must belong to ctx; FWHIP_ERR_INVALID "transcribe_samples: empty audio" for
 * n_samples == 0.  Release the result with fwhip_transcript_free. */
fwhip_status fwhip_transcribe(fwhip_ctx *ctx, fwhip_encoder *enc, fwhip_decoder *dec, const float *samples_dev,
                              int64_t n_samples, const float *filters_dev, int32_t n_mel, const fwhip_filter *filter,
                              const fwhip_vocab *vocab, const fwhip_transcribe_params *params,
                              fwhip_transcript **out);
int32_t fwhip_transcript_n_segments(const fwhip_transcript *t);
fwhip_status fwhip_transcript_segment(const fwhip_transcript *t, int32_t i, fwhip_segment_info *out);
int32_t fwhip_transcript_n_windows(const fwhip_transcript *t);
fwhip_status fwhip_transcript_window(const fwhip_transcript *t, int32_t i, fwhip_window_info *out);
void fwhip_transcript_free(fwhip_transcript *t);

/* process_logits in no-timestamps mode + argmax (decode.rs:702-867,
 * 1708-1790) for `n_rows` rows of logits on the device (`logits_dev`
 * [n_rows, n_vocab] f32): the suppress set of `filter` (NULL: raw argmax; with
 * `initial` the first-step eot/blank suppression too), then the first index of
 * the maximum under the reference's strict '>' (NaN and -inf never win, -0.0
 * and +0.0 tie, a row with no candidate gives 0).  argmax_host is [n_rows]. */
fwhip_status fwhip_argmax_logits(fwhip_ctx *ctx, const float *logits_dev, int32_t n_rows, int32_t n_vocab,
                                 const fwhip_filter *filter, int32_t initial, int32_t *argmax_host);

/* layer_norm (src/native_engine/nn.rs:4351-4545: f64 mean and variance,
 * ((x - mean) * inv) * w + b rounded to f32, eps 1e-5) of n_rows rows of d
 * floats on the device (x_dev, y_dev [n_rows, d]; w_dev, b_dev [d]), with
 * the decoder's LayerNorm kernel.  exact = 1: the sums run in the reference's
 * sequential index order (nn.rs:4425-4438), bit-identical to it on every row;
 * exact = 0: the fast mode's wave-tree sums (fwhip_decoder_set_exact).  A
 * parity entry for the LayerNorm inside the decoder's kernels.  Needs
 * d % 4 == 0 and d <= 2048. */
fwhip_status fwhip_layer_norm(fwhip_ctx *ctx, const float *x_dev, const float *w_dev, const float *b_dev,
                              int64_t n_rows, int32_t d, float *y_dev, int32_t exact);

/* ---- log-mel frontend ---------------------------------------------------- */

/* n_frames_for (src/native_engine/mel.rs:1127-1131): frames log_mel produces
 * for n_samples raw 16 kHz samples, (n + 480000 + 400 - 400) / 160. */
int64_t fwhip_mel_frames(int64_t n_samples);

/* log_mel (src/native_engine/mel.rs:1476-1660, default two-for-one FFT path).
 * samples_dev: n_samples f32 PCM on the device; filters_dev: the filterbank
 * [n_mel, n_fft_bins] row-major f32 on the device (MelFilterbank,
 * src/native_engine/mod.rs:143); mel_dev receives [n_mel, fwhip_mel_frames(n)]
 * mel-major f32, bit-identical to the reference.  FWHIP_ERR_INVALID when
 * n_fft_bins != 201 or n_mel == 0 (the reference's InvalidRequest cases), or
 * n_mel > 256.  Enqueued on the context stream; fwhip_synchronize waits. */
fwhip_status fwhip_log_mel(fwhip_ctx *ctx, const float *samples_dev, int64_t n_samples,
                           const float *filters_dev, int32_t n_mel, int32_t n_fft_bins,
                           float *mel_dev);

/* fwhip_log_mel without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * Same arguments, result and errors as fwhip_log_mel, bit for bit; its scratch
 * (filter ranges, per-block maxima, the floor: 512 KiB) is a device array each
 * GPU holds from fwhip_init until the process ends, so inputs are limited to
 * 1,043,968 frames (about 166 M samples, 2.9 hours at 16 kHz); longer inputs
 * return FWHIP_ERR_INVALID.  All calls on one GPU share that scratch: calls that
 * overlap on one GPU (two contexts, two threads) race. */
fwhip_status fwhip_log_mel_noalloc(fwhip_ctx *ctx, const float *samples_dev, int64_t n_samples,
                                   const float *filters_dev, int32_t n_mel, int32_t n_fft_bins, float *mel_dev);

/* ---- ggml model files ---------------------------------------------------- */

/* A whisper.cpp ggml model file (src/native_engine/ggml.rs:1-47 layout: magic,
 * eleven i32 hparams, mel filterbank, byte-level vocab, tensor directory with
 * ggml-order dims, no padding).  Opening scans the directory only; payloads
 * stay in the file and are read when a tensor is asked for. */
typedef struct fwhip_ggml fwhip_ggml;

/* Tensor element types (the file's ttype codes, ggml.rs:1068-1087). */
#define FWHIP_GGML_F32 0
#define FWHIP_GGML_F16 1
#define FWHIP_GGML_Q4_0 2
#define FWHIP_GGML_Q4_1 3
#define FWHIP_GGML_Q5_0 6
#define FWHIP_GGML_Q5_1 7
#define FWHIP_GGML_Q8_0 8
#define FWHIP_GGML_Q2_K 10
#define FWHIP_GGML_Q3_K 11
#define FWHIP_GGML_Q4_K 12
#define FWHIP_GGML_Q5_K 13
#define FWHIP_GGML_Q6_K 14

/* Replaces GgmlModel::load (ggml.rs:903-950, the streamed pread scan of
 * 1160-1220): FWHIP_ERR_INVALID with the reference's message for a bad magic,
 * a truncated or malformed structure (negative counts, n_dims outside 1..=4,
 * element counts that are not a multiple of the type's block), and
 * FWHIP_ERR_UNSUPPORTED for an ftype or tensor type the reference does not
 * decode; FWHIP_ERR_GENERIC ("io: ...") when the file cannot be opened.  A
 * file the reference would load but whose tensor names hold a NUL byte (valid
 * UTF-8 there, not a C string here) is refused with FWHIP_ERR_UNSUPPORTED
 * ("cpu:ggml-nul-in-tensor-name"). */
fwhip_status fwhip_ggml_open(const char *path, fwhip_ggml **out);
/* GgmlModel::from_bytes (ggml.rs:953-955): the same parse over a copy of `len`
 * bytes of caller memory. */
fwhip_status fwhip_ggml_open_bytes(const void *data, uint64_t len, fwhip_ggml **out);
void fwhip_ggml_close(fwhip_ggml *g);

/* hparams11: n_vocab, n_audio_ctx, n_audio_state, n_audio_head, n_audio_layer,
 * n_text_ctx, n_text_state, n_text_head, n_text_layer, n_mels, ftype
 * (WhisperHParams, mod.rs:56-77). */
fwhip_status fwhip_ggml_header(const fwhip_ggml *g, int32_t *hparams11);
/* GgmlModel::filters (MelFilterbank, [n_mel, n_fft_bins] row-major); `data`
 * stays valid until fwhip_ggml_close. */
fwhip_status fwhip_ggml_filters(const fwhip_ggml *g, int32_t *n_mel, int32_t *n_fft_bins, const float **data);
/* GgmlModel::vocab_tokens: the count stored in the file and token `id`'s raw
 * bytes (valid until fwhip_ggml_close). */
int32_t fwhip_ggml_vocab_count(const fwhip_ggml *g);
fwhip_status fwhip_ggml_vocab_token(const fwhip_ggml *g, int32_t id, const uint8_t **bytes, uint32_t *len);
/* GgmlModel::tensor_names (ggml.rs:1416, sorted) and tensor (ggml.rs:1424):
 * logical row-major shape (ggml's ne[] reversed; unused trailing entries 1),
 * element type and payload bytes.  Unknown names: FWHIP_ERR_INVALID
 * "unknown tensor '<name>'". */
int32_t fwhip_ggml_tensor_count(const fwhip_ggml *g);
const char *fwhip_ggml_tensor_name(const fwhip_ggml *g, int32_t i);
fwhip_status fwhip_ggml_tensor_info(const fwhip_ggml *g, const char *name, int32_t *dtype, int32_t *n_dims,
                                    int64_t *shape4, uint64_t *byte_len);
/* The payload bytes as stored (TensorBytes, ggml.rs:689-740) into `host` (cap
 * bytes at least byte_len). */
fwhip_status fwhip_ggml_tensor_raw(const fwhip_ggml *g, const char *name, void *host, uint64_t cap);

/* GgmlModel::tensor_f32 (ggml.rs:1478-1632) on the GPU: the payload is read
 * into pinned staging, copied to the device and decoded there into out_dev
 * (n_elements f32, 4-byte aligned) in the reference's arithmetic, bit for bit. */
fwhip_status fwhip_ggml_tensor_f32(fwhip_ctx *ctx, const fwhip_ggml *g, const char *name, float *out_dev,
                                   int64_t n_elements);
/* The decode step alone: `raw_dev` holds a payload of element type `dtype`
 * already on the device (raw_bytes must equal the type's byte length for
 * n_elements, ggml_byte_len ggml.rs:386-474; both pointers 4-byte aligned).
 * Enqueued on the context stream. */
fwhip_status fwhip_dequant(fwhip_ctx *ctx, int32_t dtype, const void *raw_dev, uint64_t raw_bytes,
                           int64_t n_elements, float *out_dev);

/* EncoderWeights::from_ggml (encoder.rs:764-1029) into fwhip_encoder_load:
 * the reference's tensor names, shapes and messages.  Vectors may be stored in
 * any type (decoded as tensor_f32 does).  Linears and conv kernels are taken
 * as binary16: f16-stored ones as they are, others when every value is a
 * binary16 value (the reference then computes on the same numbers), else
 * FWHIP_ERR_UNSUPPORTED "cpu:ggml-<type>-linear: ..." (the caller's CPU route).
 * Cancellation (fwhip_request_cancel) is checked between blocks. */
fwhip_status fwhip_encoder_load_ggml(fwhip_ctx *ctx, const fwhip_ggml *g, int32_t precision, fwhip_encoder **out);
/* DecoderWeights::from_ggml (decoder.rs:752-932) into fwhip_decoder_load.  The
 * GPU arms are the reference's f16-stored arms (load_linear / load_embedding,
 * decoder.rs:599-720), so every linear and the token embedding must be stored
 * as f16 (else FWHIP_ERR_UNSUPPORTED "cpu:ggml-<type>-linear: ..."). */
fwhip_status fwhip_decoder_load_ggml(fwhip_ctx *ctx, const fwhip_ggml *g, int32_t arm, fwhip_decoder **out);

#ifdef __cplusplus
}
#endif
#endif /* FWHIP_H */
