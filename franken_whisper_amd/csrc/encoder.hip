// encoder.hip — encoder load and forward (C ABI): EncoderWeights::from_ggml
// (encoder.rs:772-1029) and forward_time_major / forward_from_full_mel_window
// (encoder.rs:1224-1677), batched over windows.
#include <cmath>
#include <string>
#include <vector>

#include "fw_enc.h"
#include "fw_internal.h"

#define HIP_TRY(expr)                                                                         \
    do {                                                                                      \
        hipError_t _e = (expr);                                                               \
        if (_e != hipSuccess)                                                                 \
            return fw_fail(FWHIP_ERR_GENERIC, std::string(#expr ": ") + hipGetErrorString(_e)); \
    } while (0)

struct EncLayerDev {
    const float *attn_ln_w, *attn_ln_b, *mlp_ln_w, *mlp_ln_b;
    const float *qkv_b, *o_b, *fc1_b, *fc2_b;
    // f32 plan: f16 weights [N, K]
    const uint16_t *qkv16 = nullptr, *o16 = nullptr, *fc1_16 = nullptr, *fc2_16 = nullptr;
    // int8 plan: i7 (q/k/v/fc1/fc2) and i8 (attn.out), per-row scales
    const int8_t *qkv7 = nullptr, *o8 = nullptr, *fc1_7 = nullptr, *fc2_7 = nullptr;
    const float *qkv7s = nullptr, *o8s = nullptr, *fc1_7s = nullptr, *fc2_7s = nullptr;
};

struct EncBufs {
    int B = 0, nf = 0;
    float *mel_tm, *a1, *x, *att, *ff;
    uint16_t *a1h, *a1l, *a2h, *a2l, *hh, *hl, *qh, *ql, *kh, *kl, *vth, *vtl, *ath, *atl, *gh, *gl;
    int8_t *hq, *aq, *gq;
    float *hs, *as, *gs;
    long long *offs;
    // ToMe: merged rows, unmerge map, merge workspace
    float *xm;
    int32_t *umap, *umap2; // original row -> current row; the latest merge's map
    void *tws;
    std::vector<void *> owned;
};

struct EncExactBufs {
    int B = 0, nf = 0;
    float *c1, *a1, *c2, *h, *qkv, *S, *sf, *att, *ff; // sf: the softmax rows' scale factors
    double *lnst;                                       // [rows][2] sequential LayerNorm statistics
    std::vector<void *> owned;
};

struct fwhip_encoder {
    fwhip_ctx *ctx;
    int precision;
    int exact = 0;
    // ToMe (FW_TOME_R / FW_TOME_LAYER): merge tome_r rows after block
    // tome_after; 0 = the un-merged encoder (the strict-parity setting)
    int tome_r = 0, tome_after = 3;
    int tome_min_rows = 0; // the default rule merges full 30 s windows only (1500 rows)
    int tome_every = 0, tome_floor = 128; // FW_TOME_EVERY (0: single shot) / FW_TOME_FLOOR
    const uint16_t *conv1n = nullptr, *conv2n = nullptr; // natural [d, Cin*3] (exact mode)
    EncExactBufs xbuf;
    fwhip_hparams hp;
    int d, H, L, nmel, nctx, dff, Kp1;
    const uint16_t *conv1w, *conv2w; // reordered [d, kk*Cin + ci] (conv1 padded to Kp1)
    const float *conv1b, *conv2b, *pos, *lnpw, *lnpb;
    std::vector<EncLayerDev> layers;
    std::vector<void *> owned;
    EncBufs buf;
};

static bool enc_quant_i7(fwhip_ctx *c, std::vector<void *> &own, const uint16_t *host, int64_t out, int inp,
                         const int8_t **q, const float **s) {
    uint16_t *tmp = nullptr;
    size_t bytes = sizeof(uint16_t) * (size_t)out * inp;
    if (hipMalloc(&tmp, bytes) != hipSuccess) return false;
    if (hipMemcpy(tmp, host, bytes, hipMemcpyHostToDevice) != hipSuccess) return false;
    int8_t *qq = (int8_t *)fw_dalloc(own, (size_t)out * inp);
    float *ss = (float *)fw_dalloc(own, sizeof(float) * out);
    int32_t *cs = nullptr;
    if (hipMalloc(&cs, sizeof(int32_t) * out) != hipSuccess || !qq || !ss) return false;
    fw_launch_quant_i7(c->stream, tmp, qq, ss, cs, out, inp, 1); // FW_ENC_EF_QUANT on
    if (hipStreamSynchronize(c->stream) != hipSuccess) return false;
    hipFree(tmp);
    hipFree(cs);
    *q = qq;
    *s = ss;
    return true;
}

static bool enc_quant_i8(fwhip_ctx *c, std::vector<void *> &own, const uint16_t *host, int64_t out, int inp,
                         const int8_t **q, const float **s) {
    uint16_t *tmp = nullptr;
    size_t bytes = sizeof(uint16_t) * (size_t)out * inp;
    if (hipMalloc(&tmp, bytes) != hipSuccess) return false;
    if (hipMemcpy(tmp, host, bytes, hipMemcpyHostToDevice) != hipSuccess) return false;
    int8_t *qq = (int8_t *)fw_dalloc(own, (size_t)out * inp);
    float *ss = (float *)fw_dalloc(own, sizeof(float) * out);
    if (!qq || !ss) return false;
    fw_launch_quant_enc_i8(c->stream, tmp, qq, ss, out, inp);
    if (hipStreamSynchronize(c->stream) != hipSuccess) return false;
    hipFree(tmp);
    *q = qq;
    *s = ss;
    return true;
}

// conv weight [Cout, Cin, 3] -> [Cout, Kp] with column kk*Cin + ci (zero padded)
static std::vector<uint16_t> conv_reorder(const uint16_t *w, int cout, int cin, int kp) {
    std::vector<uint16_t> r((size_t)cout * kp, 0);
    for (int co = 0; co < cout; co++)
        for (int ci = 0; ci < cin; ci++)
            for (int kk = 0; kk < 3; kk++) r[(size_t)co * kp + kk * cin + ci] = w[((size_t)co * cin + ci) * 3 + kk];
    return r;
}

fwhip_ctx *fw_encoder_ctx(const fwhip_encoder *e) { return e->ctx; }
fwhip_hparams fw_encoder_hparams(const fwhip_encoder *e) { return e->hp; }

extern "C" fwhip_status fwhip_encoder_load(fwhip_ctx *c, const fwhip_encoder_weights *w, int32_t precision,
                                           fwhip_encoder **out) {
    if (!c || !w || !out) return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_load: NULL argument");
    *out = nullptr;
    if (precision != FWHIP_ENC_F32 && precision != FWHIP_ENC_INT8)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_load: unknown precision");
    const fwhip_hparams &hp = w->hp;
    if (hp.n_audio_state <= 0 || hp.n_audio_head <= 0 || hp.n_audio_layer <= 0 || hp.n_mels <= 0 ||
        hp.n_audio_ctx <= 0)
        return fw_fail(FWHIP_ERR_INVALID, "encoder: non-positive hparam");
    if (hp.n_audio_state % hp.n_audio_head || hp.n_audio_state / hp.n_audio_head != 64)
        return fw_fail(FWHIP_ERR_INVALID, "encoder: d_head must be 64");
    if (hp.n_audio_state % 128 || hp.n_audio_state > 2048)
        return fw_fail(FWHIP_ERR_INVALID, "encoder: n_audio_state must be a multiple of 128 and <= 2048");
    HIP_TRY(hipSetDevice(c->device));
    fwhip_encoder *e = new fwhip_encoder();
    e->ctx = c;
    e->precision = precision;
    e->hp = hp;
    e->d = hp.n_audio_state;
    e->H = hp.n_audio_head;
    e->L = hp.n_audio_layer;
    e->nmel = hp.n_mels;
    e->nctx = hp.n_audio_ctx;
    e->dff = 4 * e->d;
    e->Kp1 = ((3 * e->nmel + 63) / 64) * 64;
    int d = e->d, dff = e->dff;
    auto &own = e->owned;
    bool ok = true;
    auto up32 = [&](const float *p, size_t n) -> const float * {
        const float *r = (const float *)fw_dupload(own, p, sizeof(float) * n);
        ok = ok && r;
        return r;
    };
    auto up16 = [&](const uint16_t *p, size_t n) -> const uint16_t * {
        const uint16_t *r = (const uint16_t *)fw_dupload(own, p, sizeof(uint16_t) * n);
        ok = ok && r;
        return r;
    };
    std::vector<uint16_t> c1 = conv_reorder(w->conv1_w, d, e->nmel, e->Kp1);
    std::vector<uint16_t> c2 = conv_reorder(w->conv2_w, d, d, 3 * d);
    e->conv1w = up16(c1.data(), c1.size());
    e->conv2w = up16(c2.data(), c2.size());
    e->conv1n = up16(w->conv1_w, (size_t)d * e->nmel * 3);
    e->conv2n = up16(w->conv2_w, (size_t)d * d * 3);
    e->conv1b = up32(w->conv1_b, d);
    e->conv2b = up32(w->conv2_b, d);
    e->pos = up32(w->pos_emb, (size_t)e->nctx * d);
    e->lnpw = up32(w->ln_post_w, d);
    e->lnpb = up32(w->ln_post_b, d);
    for (int li = 0; ok && li < e->L; li++) {
        const fwhip_enc_layer &s = w->layers[li];
        EncLayerDev l;
        l.attn_ln_w = up32(s.attn_ln_w, d);
        l.attn_ln_b = up32(s.attn_ln_b, d);
        l.mlp_ln_w = up32(s.mlp_ln_w, d);
        l.mlp_ln_b = up32(s.mlp_ln_b, d);
        std::vector<uint16_t> qkv((size_t)3 * d * d);
        memcpy(qkv.data(), s.q_w, sizeof(uint16_t) * d * d);
        memcpy(qkv.data() + (size_t)d * d, s.k_w, sizeof(uint16_t) * d * d);
        memcpy(qkv.data() + (size_t)2 * d * d, s.v_w, sizeof(uint16_t) * d * d);
        std::vector<float> qb((size_t)3 * d, 0.0f);
        memcpy(qb.data(), s.q_b, sizeof(float) * d);
        memcpy(qb.data() + 2 * d, s.v_b, sizeof(float) * d);
        l.qkv_b = up32(qb.data(), 3 * d);
        l.o_b = up32(s.o_b, d);
        l.fc1_b = up32(s.fc1_b, dff);
        l.fc2_b = up32(s.fc2_b, d);
        if (precision == FWHIP_ENC_INT8) {
            // quality-safe plan (encoder.rs:474-512): q/k/v/fc1/fc2 i7 with
            // error-feedback rounding (per-row quantization, so quantizing the
            // fused [q; k; v] equals quantizing each), attn.out full i8
            ok = ok && enc_quant_i7(c, own, qkv.data(), 3 * d, d, &l.qkv7, &l.qkv7s);
            ok = ok && enc_quant_i8(c, own, s.o_w, d, d, &l.o8, &l.o8s);
            ok = ok && enc_quant_i7(c, own, s.fc1_w, dff, d, &l.fc1_7, &l.fc1_7s);
            ok = ok && enc_quant_i7(c, own, s.fc2_w, d, dff, &l.fc2_7, &l.fc2_7s);
        } else {
            l.qkv16 = up16(qkv.data(), qkv.size());
            l.o16 = up16(s.o_w, (size_t)d * d);
            l.fc1_16 = up16(s.fc1_w, (size_t)dff * d);
            l.fc2_16 = up16(s.fc2_w, (size_t)d * dff);
        }
        e->layers.push_back(l);
    }
    if (!ok || hipDeviceSynchronize() != hipSuccess) {
        fw_free_all(own);
        delete e;
        return fw_fail(FWHIP_ERR_GENERIC, "fwhip_encoder_load: device allocation or upload failed");
    }
    *out = e;
    return FWHIP_OK;
}

extern "C" void fwhip_encoder_free(fwhip_encoder *e) {
    if (!e) return;
    hipSetDevice(e->ctx->device);
    hipStreamSynchronize(e->ctx->stream);
    fw_free_all(e->buf.owned);
    fw_free_all(e->xbuf.owned);
    fw_free_all(e->owned);
    delete e;
}

static bool ensure_bufs(fwhip_encoder *e, int B, int nf) {
    EncBufs &b = e->buf;
    if (b.B >= B && b.nf >= nf) return true;
    hipStreamSynchronize(e->ctx->stream);
    fw_free_all(b.owned);
    b = EncBufs();
    b.B = B;
    b.nf = nf;
    int d = e->d, H = e->H, dff = e->dff;
    size_t T1 = nf, T2 = nf / 2, Tp = (T2 + 63) / 64 * 64;
    size_t M1 = (size_t)B * T1, M = (size_t)B * T2;
    auto &o = b.owned;
    auto A = [&](size_t bytes) { return fw_dalloc(o, bytes); };
    b.mel_tm = (float *)A(sizeof(float) * M1 * e->nmel);
    b.a1h = (uint16_t *)A(2 * M1 * e->Kp1);
    b.a1l = (uint16_t *)A(2 * M1 * e->Kp1);
    b.a1 = (float *)A(4 * M1 * d);
    b.a2h = (uint16_t *)A(2 * M * 3 * d);
    b.a2l = (uint16_t *)A(2 * M * 3 * d);
    b.x = (float *)A(4 * M * d);
    b.hh = (uint16_t *)A(2 * M * d);
    b.hl = (uint16_t *)A(2 * M * d);
    b.hq = (int8_t *)A(M * d);
    b.hs = (float *)A(4 * M);
    size_t qk = (size_t)B * H * T2 * 64, vt = (size_t)B * H * 64 * Tp;
    b.qh = (uint16_t *)A(2 * qk);
    b.ql = (uint16_t *)A(2 * qk);
    b.kh = (uint16_t *)A(2 * qk);
    b.kl = (uint16_t *)A(2 * qk);
    b.vth = (uint16_t *)A(2 * vt);
    b.vtl = (uint16_t *)A(2 * vt);
    b.att = (float *)A(4 * M * d);
    b.ath = (uint16_t *)A(2 * M * d);
    b.atl = (uint16_t *)A(2 * M * d);
    b.aq = (int8_t *)A(M * d);
    b.as = (float *)A(4 * M);
    b.ff = (float *)A(4 * M * dff);
    b.gh = (uint16_t *)A(2 * M * dff);
    b.gl = (uint16_t *)A(2 * M * dff);
    b.gq = (int8_t *)A(M * dff);
    b.gs = (float *)A(4 * M);
    b.offs = (long long *)A(sizeof(long long) * B);
    b.xm = (float *)A(4 * M * d);
    b.umap = (int32_t *)A(sizeof(int32_t) * M);
    b.umap2 = (int32_t *)A(sizeof(int32_t) * M);
    b.tws = A(fw_tome_ws_bytes(B, (int)T2));
    for (void *p : o)
        if (!p) return false;
    // V^T padding columns (keys >= T) must be finite zeros
    fw_launch_fill_u16(e->ctx->stream, b.vth, vt, 0);
    fw_launch_fill_u16(e->ctx->stream, b.vtl, vt, 0);
    return hipStreamSynchronize(e->ctx->stream) == hipSuccess;
}

// MLP widths the index-form GELU quantizer handles (multiples of 512 up to 8192)
static bool enc_h16_ok(int n) {
    const int k = n / 512;
    return n > 0 && n % 512 == 0 && (k <= 8 || k == 10 || k == 12 || k == 16);
}

// The ToMe schedule of forward_time_major (encoder.rs:1590-1632): a merge is
// due after block li when, single shot (tome_every 0), none ran yet and
// li == tome_after, or, progressive, li >= tome_after and (li - tome_after) is
// a multiple of tome_every; it runs when rows > r + 2 and rows - r >= the
// floor.  The default rule's full-window test (tome_r_for) looks at the
// window's rows before any merge (T0).
static bool tome_due(const fwhip_encoder *e, int li, int rows, int T0, int n_merges) {
    if (e->tome_r <= 0 || T0 < e->tome_min_rows) return false;
    const bool due = e->tome_every == 0 ? (n_merges == 0 && li == e->tome_after)
                                        : (li >= e->tome_after && (li - e->tome_after) % e->tome_every == 0);
    return due && rows > e->tome_r + 2 && rows - e->tome_r >= e->tome_floor && fw_tome_ok(rows, e->d);
}

// One merge of the current rows X [B, Tc, d] into the other of b.x / b.xm
// (b.x is free once the first merge has read it); the first merge writes the
// original-row map b.umap, later ones their own map into b.umap2, composed
// into b.umap.  Returns the merged rows; Tc becomes their count.
static float *tome_step(hipStream_t st, EncBufs &b, float *X, int B, int T0, int &Tc, int d, int r, int n_merges) {
    float *dst = X == b.xm ? b.x : b.xm;
    const int Tprev = Tc;
    Tc = fw_launch_tome_merge(st, X, B, Tprev, d, r, b.tws, dst, n_merges ? b.umap2 : b.umap);
    if (n_merges) fw_launch_tome_compose(st, b.umap, b.umap2, B, T0, Tprev);
    return dst;
}

// tome_unmerge before ln_post (encoder.rs:1629-1631): the full rows, in b.x
// or, when the merged rows are there, in b.att (free after the last block)
static float *tome_finish(hipStream_t st, EncBufs &b, float *X, int B, int Tc, int T0, int d, int n_merges) {
    if (!n_merges) return X;
    float *fin = X == b.x ? b.att : b.x;
    fw_launch_tome_unmerge(st, X, B, Tc, b.umap, T0, d, fin);
    return fin;
}

static FwGemm gemm_args(const void *A, const void *A2, const void *B, int M, int N, int K, const float *sx,
                        const float *sw, const float *bias, int epi, float *C, int ldc) {
    FwGemm g;
    memset(&g, 0, sizeof g);
    g.A = A;
    g.A2 = A2;
    g.B = B;
    g.M = M;
    g.N = N;
    g.K = K;
    g.lda = K;
    g.ldb = K;
    g.sx = sx;
    g.sw = sw;
    g.bias = bias;
    g.epi = epi;
    g.C = C;
    g.ldc = ldc;
    return g;
}

// EncoderExecution of a forward (encoder.rs:1987-2003): the route, the
// arithmetic of each GEMM family and what chose it.
static void fill_record(fwhip_exec_record *rec, const fwhip_encoder *e, int B, double ms, bool exact,
                        const char *source) {
    if (!rec) return;
    const bool i8 = e->precision == FWHIP_ENC_INT8;
    snprintf(rec->route, sizeof rec->route, "hip:gfx950:%s%s", i8 ? "int8" : "f32", exact ? ":exact" : "");
    rec->precision = e->precision;
    rec->n_windows = B;
    rec->device_ms = ms;
    // the f32 parts: strict f32 in exact mode, f16-pair MFMA in fast mode
    const int f = exact ? FWHIP_PREC_F32 : FWHIP_PREC_F16_PAIR;
    rec->family[FWHIP_FAM_CONV_STEM] = f;
    rec->family[FWHIP_FAM_ATTENTION] = f;
    rec->family[FWHIP_FAM_ATTN_QKV] = i8 ? FWHIP_PREC_I7 : f;
    rec->family[FWHIP_FAM_ATTN_OUT] = i8 ? FWHIP_PREC_I8 : f;
    rec->family[FWHIP_FAM_MLP_FC1] = i8 ? FWHIP_PREC_I7 : f;
    rec->family[FWHIP_FAM_MLP_FC2] = i8 ? FWHIP_PREC_I7 : f;
    snprintf(rec->precision_source, sizeof rec->precision_source, "%s", source);
}

static fwhip_status enc_run(fwhip_encoder *e, int B, int nf, float *out_dev, fwhip_exec_record *rec) {
    fwhip_ctx *c = e->ctx;
    hipStream_t st = c->stream;
    EncBufs &b = e->buf;
    int d = e->d, H = e->H, dff = e->dff;
    int T1 = nf, T2 = nf / 2, Tp = (T2 + 63) / 64 * 64;
    int M1 = B * T1, M = B * T2;
    bool i8 = e->precision == FWHIP_ENC_INT8;
    const float *gt = c->gelu_tab;
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    hipEventRecord(e0, st);
    fw_event_pair ev;
    // every f16-pair split reports a value past the f16 range into c->ovf_dev
    int *ovf = c->ovf_dev;
    fw_ovf_clear(c);
    // conv stem (encoder.rs:1550-1572): conv1 + GELU, conv2 (stride 2) + GELU, + pos_emb
    fw_launch_im2col(st, b.mel_tm, B, T1, e->nmel, 1, T1, e->Kp1, b.a1h, b.a1l, ovf);
    {
        FwGemm g = gemm_args(b.a1h, b.a1l, e->conv1w, M1, d, e->Kp1, nullptr, nullptr, e->conv1b, FW_EPI_GELU_F32,
                             b.a1, d);
        g.gelu_tab = gt;
        fw_timed_begin(c, FWHIP_K_ENC_GEMM_F32, 2.0 * M1 * d * 3.0 * e->nmel, &ev);
        fw_launch_gemm(st, FW_KIND_F16S, g);
        fw_timed_end(c, &ev);
    }
    fw_launch_im2col(st, b.a1, B, T1, d, 2, T2, 3 * d, b.a2h, b.a2l, ovf);
    {
        FwGemm g = gemm_args(b.a2h, b.a2l, e->conv2w, M, d, 3 * d, nullptr, nullptr, e->conv2b, FW_EPI_CONV2, b.x, d);
        g.gelu_tab = gt;
        g.pos = e->pos;
        g.T = T2;
        fw_timed_begin(c, FWHIP_K_ENC_GEMM_F32, 2.0 * M * d * 3.0 * d, &ev);
        fw_launch_gemm(st, FW_KIND_F16S, g);
        fw_timed_end(c, &ev);
    }
    int gcls = i8 ? FWHIP_K_ENC_GEMM_I8 : FWHIP_K_ENC_GEMM_F32;
    // the current rows: b.x [B, T2, d], or after a ToMe merge b.xm [B, Tc, d]
    float *X = b.x;
    int Tc = T2, Mc = M, Tpc = Tp;
    int n_merges = 0;
    int kind = i8 ? FW_KIND_I8 : FW_KIND_F16S;
    for (int li = 0; li < e->L; li++) {
        const EncLayerDev &l = e->layers[li];
        // self-attention residual (encoder_block, encoder.rs:2608-2681)
        fw_launch_enc_ln(st, X, l.attn_ln_w, l.attn_ln_b, Mc, d, i8 ? FW_LN_I7 : FW_LN_SPLIT, nullptr, b.hh, b.hl,
                         b.hq, b.hs, ovf);
        FwGemm g = i8 ? gemm_args(b.hq, nullptr, l.qkv7, Mc, 3 * d, d, b.hs, l.qkv7s, l.qkv_b, FW_EPI_QKV, nullptr, d)
                      : gemm_args(b.hh, b.hl, l.qkv16, Mc, 3 * d, d, nullptr, nullptr, l.qkv_b, FW_EPI_QKV, nullptr, d);
        g.ovf = ovf;
        g.o16[0] = b.qh;
        g.o16[1] = b.ql;
        g.o16[2] = b.kh;
        g.o16[3] = b.kl;
        g.o16[4] = b.vth;
        g.o16[5] = b.vtl;
        g.T = Tc;
        g.H = H;
        g.Tp = Tpc;
        fw_timed_begin(c, gcls, 2.0 * Mc * 3.0 * d * d, &ev);
        fw_launch_gemm(st, kind, g);
        fw_timed_end(c, &ev);
        fw_timed_begin(c, FWHIP_K_ENC_ATTN, 4.0 * B * H * (double)Tc * Tc * 64, &ev);
        fw_launch_attention(st, b.qh, b.ql, b.kh, b.kl, b.vth, b.vtl, B, Tc, Tpc, H, d, i8 ? 0 : 1, b.att, b.ath,
                            b.atl);
        fw_timed_end(c, &ev);
        if (i8) {
            fw_launch_quant_exact_rows(st, b.att, Mc, d, b.aq, b.as);
            g = gemm_args(b.aq, nullptr, l.o8, Mc, d, d, b.as, l.o8s, l.o_b, FW_EPI_RESID, X, d);
        } else {
            g = gemm_args(b.ath, b.atl, l.o16, Mc, d, d, nullptr, nullptr, l.o_b, FW_EPI_RESID, X, d);
        }
        fw_timed_begin(c, gcls, 2.0 * Mc * (double)d * d, &ev);
        fw_launch_gemm(st, kind, g);
        fw_timed_end(c, &ev);
        // MLP residual (encoder.rs:2684-2735)
        fw_launch_enc_ln(st, X, l.mlp_ln_w, l.mlp_ln_b, Mc, d, i8 ? FW_LN_I7 : FW_LN_SPLIT, nullptr, b.hh, b.hl,
                         b.hq, b.hs, ovf);
        if (i8) {
            // fc1 as f16 GELU-table indices (half the bytes of f32 rows; the
            // rare |v| >= 9.98 values exactly in b.ff), then GELU + quantization;
            // f32 rows where the index form has no kernel
            g = gemm_args(b.hq, nullptr, l.fc1_7, Mc, dff, d, b.hs, l.fc1_7s, l.fc1_b, FW_EPI_F16IDX, b.ff, dff);
            g.o16[0] = b.gh;
            fw_timed_begin(c, gcls, 2.0 * Mc * (double)dff * d, &ev);
            bool idx = enc_h16_ok(dff) && fw_launch_gemm(st, kind, g);
            if (!idx) {
                g.epi = FW_EPI_F32;
                fw_launch_gemm(st, kind, g);
            }
            fw_timed_end(c, &ev);
            if (!idx || !fw_launch_gelu_quant_h16(st, b.gh, b.ff, Mc, dff, gt, b.gq, b.gs))
                fw_launch_gelu_quant_i7_rows(st, b.ff, Mc, dff, gt, b.gq, b.gs);
            g = gemm_args(b.gq, nullptr, l.fc2_7, Mc, d, dff, b.gs, l.fc2_7s, l.fc2_b, FW_EPI_RESID, X, d);
        } else {
            g = gemm_args(b.hh, b.hl, l.fc1_16, Mc, dff, d, nullptr, nullptr, l.fc1_b, FW_EPI_GELU_SPLIT, nullptr,
                          dff);
            g.gelu_tab = gt;
            g.o16[0] = b.gh;
            g.o16[1] = b.gl;
            g.ovf = ovf;
            fw_timed_begin(c, gcls, 2.0 * Mc * (double)dff * d, &ev);
            fw_launch_gemm(st, kind, g);
            fw_timed_end(c, &ev);
            g = gemm_args(b.gh, b.gl, l.fc2_16, Mc, d, dff, nullptr, nullptr, l.fc2_b, FW_EPI_RESID, X, d);
        }
        fw_timed_begin(c, gcls, 2.0 * Mc * (double)d * dff, &ev);
        fw_launch_gemm(st, kind, g);
        fw_timed_end(c, &ev);
        if (tome_due(e, li, Tc, T2, n_merges)) {
            X = tome_step(st, b, X, B, T2, Tc, d, e->tome_r, n_merges++);
            Mc = B * Tc;
            Tpc = (Tc + 63) / 64 * 64;
            // V^T rows now have stride Tpc: their padding keys must be finite
            fw_launch_tome_vpad(st, b.vth, (size_t)B * H * 64, Tc, Tpc);
            fw_launch_tome_vpad(st, b.vtl, (size_t)B * H * 64, Tc, Tpc);
        }
        if (c->cancel.exchange(0)) {
            hipStreamSynchronize(st);
            hipEventDestroy(e0);
            hipEventDestroy(e1);
            return fw_fail(FWHIP_ERR_CANCELLED, "cancelled");
        }
    }
    X = tome_finish(st, b, X, B, Tc, T2, d, n_merges);
    // ln_post (encoder.rs:1636)
    fw_launch_enc_ln(st, X, e->lnpw, e->lnpb, M, d, FW_LN_F32, out_dev, nullptr, nullptr, nullptr, nullptr);
    hipEventRecord(e1, st);
    fw_ovf_fetch(c);
    hipError_t err = hipStreamSynchronize(st);
    float ms = 0.0f;
    hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (err != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, std::string("encoder: ") + hipGetErrorString(err));
    err = hipGetLastError();
    if (err != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, std::string("encoder launch: ") + hipGetErrorString(err));
    fill_record(rec, e, B, ms, false, "fwhip_encoder_load");
    return FWHIP_OK;
}

static bool ensure_exact_bufs(fwhip_encoder *e, int B, int nf) {
    EncExactBufs &x = e->xbuf;
    if (x.B >= B && x.nf >= nf) return true;
    hipStreamSynchronize(e->ctx->stream);
    fw_free_all(x.owned);
    x = EncExactBufs();
    x.B = B;
    x.nf = nf;
    int d = e->d;
    size_t T1 = nf, T2 = nf / 2, M1 = (size_t)B * T1, M = (size_t)B * T2;
    auto A = [&](size_t n) { return (float *)fw_dalloc(x.owned, sizeof(float) * n); };
    x.c1 = A(M1 * 3 * e->nmel);
    x.a1 = A(M1 * d);
    x.c2 = A(M * 3 * d);
    x.h = A(M * d);
    x.qkv = A(M * 3 * d);
    x.S = A((size_t)B * e->H * T2 * T2);
    x.sf = A((size_t)B * e->H * T2 * (1 + (T2 + 63) / 64));
    x.att = A(M * d);
    x.ff = A(M * e->dff);
    x.lnst = (double *)fw_dalloc(x.owned, sizeof(double) * 2 * M);
    for (void *p : x.owned)
        if (!p) return false;
    return true;
}

// Exact mode: the reference's strict-parity arithmetic end to end — strict
// sequential-k f32 GEMMs for the conv stem (and, on the f32 plan, every
// linear), the per-head attention of attention_raw with glibc-exact softmax,
// and on the int8 plan the same int8 GEMMs as the fast mode.
static fwhip_status enc_run_exact(fwhip_encoder *e, int B, int nf, float *out_dev, fwhip_exec_record *rec,
                                  const char *source) {
    fwhip_ctx *c = e->ctx;
    hipStream_t st = c->stream;
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    hipEventRecord(e0, st);
    EncBufs &b = e->buf;
    EncExactBufs &x = e->xbuf;
    int d = e->d, H = e->H, dff = e->dff;
    int T1 = nf, T2 = nf / 2, M1 = B * T1, M = B * T2;
    bool i8 = e->precision == FWHIP_ENC_INT8;
    const float *gt = c->gelu_tab;
    fw_launch_im2col_f32(st, b.mel_tm, B, T1, e->nmel, 1, T1, x.c1);
    fw_launch_gemm_strict(st, x.c1, e->conv1n, M1, d, 3 * e->nmel, 3, x.a1, e->conv1b, 1.0f, nullptr, T1, 0, 0, 0, d,
                          gt, nullptr);
    fw_launch_im2col_f32(st, x.a1, B, T1, d, 2, T2, x.c2);
    fw_launch_gemm_strict(st, x.c2, e->conv2n, M, d, 3 * d, 4, b.x, e->conv2b, 1.0f, nullptr, T2, 0, 0, 0, d, gt,
                          e->pos);
    float *X = b.x;
    int Tc = T2, Mc = M;
    int n_merges = 0;
    for (int li = 0; li < e->L; li++) {
        const EncLayerDev &l = e->layers[li];
        if (i8) {
            fw_launch_enc_ln(st, X, l.attn_ln_w, l.attn_ln_b, Mc, d, FW_LN_I7 | FW_LN_SEQ, nullptr, nullptr, nullptr, b.hq, b.hs,
                             nullptr, x.lnst);
            FwGemm g = gemm_args(b.hq, nullptr, l.qkv7, Mc, 3 * d, d, b.hs, l.qkv7s, l.qkv_b, FW_EPI_F32, x.qkv, 3 * d);
            fw_launch_gemm(st, FW_KIND_I8, g);
        } else {
            fw_launch_enc_ln(st, X, l.attn_ln_w, l.attn_ln_b, Mc, d, FW_LN_F32 | FW_LN_SEQ, x.h, nullptr, nullptr, nullptr,
                             nullptr, nullptr, x.lnst);
            fw_launch_gemm_strict(st, x.h, l.qkv16, Mc, 3 * d, d, 0, x.qkv, l.qkv_b, 1.0f, nullptr, Tc, 0, 0, 0,
                                  3 * d, nullptr, nullptr);
        }
        fw_launch_attention_exact(st, x.qkv, 3 * d, 0, d, 2 * d, B, Tc, H, d, x.S, x.sf, x.att);
        if (i8) {
            fw_launch_quant_exact_rows(st, x.att, Mc, d, b.aq, b.as);
            FwGemm g = gemm_args(b.aq, nullptr, l.o8, Mc, d, d, b.as, l.o8s, l.o_b, FW_EPI_RESID, X, d);
            fw_launch_gemm(st, FW_KIND_I8, g);
            fw_launch_enc_ln(st, X, l.mlp_ln_w, l.mlp_ln_b, Mc, d, FW_LN_I7 | FW_LN_SEQ, nullptr, nullptr, nullptr, b.hq, b.hs,
                             nullptr, x.lnst);
            g = gemm_args(b.hq, nullptr, l.fc1_7, Mc, dff, d, b.hs, l.fc1_7s, l.fc1_b, FW_EPI_F32, b.ff, dff);
            fw_launch_gemm(st, FW_KIND_I8, g);
            fw_launch_gelu_quant_i7_rows(st, b.ff, Mc, dff, gt, b.gq, b.gs);
            g = gemm_args(b.gq, nullptr, l.fc2_7, Mc, d, dff, b.gs, l.fc2_7s, l.fc2_b, FW_EPI_RESID, X, d);
            fw_launch_gemm(st, FW_KIND_I8, g);
        } else {
            fw_launch_gemm_strict(st, x.att, l.o16, Mc, d, d, 5, X, l.o_b, 1.0f, nullptr, Tc, 0, 0, 0, d, nullptr,
                                  nullptr);
            fw_launch_enc_ln(st, X, l.mlp_ln_w, l.mlp_ln_b, Mc, d, FW_LN_F32 | FW_LN_SEQ, x.h, nullptr, nullptr, nullptr, nullptr,
                             nullptr, x.lnst);
            fw_launch_gemm_strict(st, x.h, l.fc1_16, Mc, dff, d, 3, x.ff, l.fc1_b, 1.0f, nullptr, Tc, 0, 0, 0, dff, gt,
                                  nullptr);
            fw_launch_gemm_strict(st, x.ff, l.fc2_16, Mc, d, dff, 5, X, l.fc2_b, 1.0f, nullptr, Tc, 0, 0, 0, d,
                                  nullptr, nullptr);
        }
        if (tome_due(e, li, Tc, T2, n_merges)) {
            X = tome_step(st, b, X, B, T2, Tc, d, e->tome_r, n_merges++);
            Mc = B * Tc;
        }
        if (c->cancel.exchange(0)) {
            hipStreamSynchronize(st);
            hipEventDestroy(e0);
            hipEventDestroy(e1);
            return fw_fail(FWHIP_ERR_CANCELLED, "cancelled");
        }
    }
    X = tome_finish(st, b, X, B, Tc, T2, d, n_merges);
    fw_launch_enc_ln(st, X, e->lnpw, e->lnpb, M, d, FW_LN_F32 | FW_LN_SEQ, out_dev, nullptr, nullptr, nullptr, nullptr,
                     nullptr, x.lnst);
    hipEventRecord(e1, st);
    hipError_t err = hipStreamSynchronize(st);
    float ms = 0.0f;
    hipEventElapsedTime(&ms, e0, e1);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    if (err == hipSuccess) err = hipGetLastError();
    if (err != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, std::string("encoder (exact): ") + hipGetErrorString(err));
    fill_record(rec, e, B, ms, true, source);
    return FWHIP_OK;
}

// A fast forward whose f16-pair operands met a value past the f16 range
// (the device flag) is run again in exact mode, which has no f16 pairs; the
// record says so.
static fwhip_status enc_dispatch(fwhip_encoder *e, int B, int nf, float *out_dev, fwhip_exec_record *rec) {
    if (!e->exact) {
        fwhip_status r = enc_run(e, B, nf, out_dev, rec);
        if (r != FWHIP_OK || !*e->ctx->ovf_host) return r;
    }
    if (!ensure_exact_bufs(e, B, nf)) return fw_fail(FWHIP_ERR_GENERIC, "encoder: exact buffers failed");
    return enc_run_exact(e, B, nf, out_dev, rec, e->exact ? "fwhip_encoder_set_exact" : "f16_pair_range");
}

extern "C" fwhip_status fwhip_encoder_set_exact(fwhip_encoder *e, int32_t exact) {
    if (!e) return fw_fail(FWHIP_ERR_INVALID, "NULL encoder");
    if (exact && e->precision == FWHIP_ENC_F32 && e->layers.size() && !e->layers[0].qkv16)
        return fw_fail(FWHIP_ERR_INVALID, "exact f32 mode needs the f32 plan's weights");
    e->exact = exact != 0;
    return FWHIP_OK;
}

// FW_TOME_R / FW_TOME_LAYER (encoder.rs:1264-1337): merge r rows after block
// `after` (0-based) of every full window; r = 0 restores the un-merged
// encoder; r < 0 takes the reference's default for the model (tome_r_for:
// 500 after block 3 on the 20-head large class, else 0).
extern "C" fwhip_status fwhip_encoder_set_tome(fwhip_encoder *e, int32_t r, int32_t after) {
    if (!e) return fw_fail(FWHIP_ERR_INVALID, "NULL encoder");
    int min_rows = 0;
    if (r < 0) {
        r = e->H >= 20 ? 500 : 0;
        after = 3;
        min_rows = 1500; // shorter (tail) windows keep every row
    }
    if (r > 0 && (after < 0 || after >= e->L)) return fw_fail(FWHIP_ERR_INVALID, "ToMe layer out of range");
    e->tome_r = r;
    e->tome_after = after;
    e->tome_min_rows = min_rows;
    return FWHIP_OK;
}

// FW_TOME_EVERY / FW_TOME_FLOOR (encoder.rs:1379-1402): every = 0 keeps the
// single-shot schedule, every > 0 merges again after every `every` blocks from
// the first; no merge leaves fewer than `floor` rows.
extern "C" fwhip_status fwhip_encoder_set_tome_schedule(fwhip_encoder *e, int32_t every, int32_t floor) {
    if (!e) return fw_fail(FWHIP_ERR_INVALID, "NULL encoder");
    if (every < 0 || floor < 0) return fw_fail(FWHIP_ERR_INVALID, "ToMe schedule: every and floor must be >= 0");
    e->tome_every = every;
    e->tome_floor = floor;
    return FWHIP_OK;
}

extern "C" fwhip_status fwhip_tome_merge(fwhip_ctx *c, const float *x_dev, int32_t n_windows, int32_t T, int32_t d,
                                         int32_t r, float *merged_dev, int32_t *umap_dev, int32_t *out_rows) {
    if (!c || !x_dev || !merged_dev || !umap_dev || !out_rows) return fw_fail(FWHIP_ERR_INVALID, "fwhip_tome_merge: NULL argument");
    if (n_windows <= 0 || r < 0 || !fw_tome_ok(T, d))
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_tome_merge: needs n_windows > 0, r >= 0, 2 <= T <= 4096, d % 32 == 0");
    HIP_TRY(hipSetDevice(c->device));
    void *ws = nullptr;
    HIP_TRY(hipMalloc(&ws, fw_tome_ws_bytes(n_windows, T)));
    *out_rows = fw_launch_tome_merge(c->stream, x_dev, n_windows, T, d, r, ws, merged_dev, umap_dev);
    hipError_t e = hipStreamSynchronize(c->stream);
    if (e == hipSuccess) e = hipGetLastError();
    hipFree(ws);
    if (e != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, std::string("fwhip_tome_merge: ") + hipGetErrorString(e));
    return FWHIP_OK;
}

static fwhip_status check_frames(fwhip_encoder *e, int n_windows, int n_frames) {
    if (n_windows <= 0) return fw_fail(FWHIP_ERR_INVALID, "encoder: n_windows must be > 0");
    // validate_mel_window_shape (encoder.rs:716-737)
    if (n_frames <= 0 || n_frames % 2 || n_frames > 2 * e->nctx)
        return fw_fail(FWHIP_ERR_INVALID, "encoder: mel window has " + std::to_string(n_frames) +
                                              " frames, expected a positive even count <= " +
                                              std::to_string(2 * e->nctx));
    return FWHIP_OK;
}

extern "C" fwhip_status fwhip_encoder_forward_time_major(fwhip_encoder *e, const float *x_dev, int32_t n_windows,
                                                         int32_t n_frames, float *out_dev, fwhip_exec_record *rec) {
    if (!e || !x_dev || !out_dev) return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_forward_time_major: NULL argument");
    fwhip_status r = check_frames(e, n_windows, n_frames);
    if (r != FWHIP_OK) return r;
    HIP_TRY(hipSetDevice(e->ctx->device));
    if (!ensure_bufs(e, n_windows, n_frames)) return fw_fail(FWHIP_ERR_GENERIC, "encoder: buffer allocation failed");
    HIP_TRY(hipMemcpyAsync(e->buf.mel_tm, x_dev, sizeof(float) * (size_t)n_windows * n_frames * e->nmel,
                           hipMemcpyDeviceToDevice, e->ctx->stream));
    return enc_dispatch(e, n_windows, n_frames, out_dev, rec);
}

extern "C" fwhip_status fwhip_encoder_forward(fwhip_encoder *e, const float *mel_dev, int64_t mel_frames,
                                              const int64_t *frame_offsets, int32_t n_windows, int32_t n_frames,
                                              float *out_dev, fwhip_exec_record *rec) {
    if (!e || !mel_dev || !frame_offsets || !out_dev)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_forward: NULL argument");
    fwhip_status r = check_frames(e, n_windows, n_frames);
    if (r != FWHIP_OK) return r;
    for (int i = 0; i < n_windows; i++)
        if (frame_offsets[i] < 0) return fw_fail(FWHIP_ERR_INVALID, "encoder: negative frame offset");
    HIP_TRY(hipSetDevice(e->ctx->device));
    if (!ensure_bufs(e, n_windows, n_frames)) return fw_fail(FWHIP_ERR_GENERIC, "encoder: buffer allocation failed");
    HIP_TRY(hipStreamSynchronize(e->ctx->stream));
    HIP_TRY(hipMemcpy(e->buf.offs, frame_offsets, sizeof(long long) * n_windows, hipMemcpyHostToDevice));
    fw_launch_mel_window(e->ctx->stream, mel_dev, e->nmel, mel_frames, e->buf.offs, n_frames, e->buf.mel_tm,
                         n_windows);
    return enc_dispatch(e, n_windows, n_frames, out_dev, rec);
}

// Per-GEMM parity: run one encoder int8 linear (which: 0 q, 1 k, 2 v, 3 attn.out,
// 4 fc1, 5 fc2 with the GELU-fused quantizer) of `layer` on f32 input rows
// x_dev [m, in] and write the i32 accumulators and the epilogue output.
extern "C" fwhip_status fwhip_encoder_gemm_i8(fwhip_encoder *e, int32_t layer, int32_t which, const float *x_dev,
                                              int32_t m, int32_t *acc_dev, float *y_dev) {
    if (!e || !x_dev || !acc_dev || !y_dev) return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_gemm_i8: NULL argument");
    if (e->precision != FWHIP_ENC_INT8) return fw_fail(FWHIP_ERR_INVALID, "encoder is not on the int8 plan");
    if (layer < 0 || layer >= e->L || which < 0 || which > 5 || m <= 0)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_gemm_i8: bad layer/which/m");
    fwhip_ctx *c = e->ctx;
    HIP_TRY(hipSetDevice(c->device));
    int d = e->d, dff = e->dff;
    const EncLayerDev &l = e->layers[layer];
    int inp = which == 5 ? dff : d, out = which == 4 ? dff : d;
    std::vector<void *> tmp;
    int8_t *xq = (int8_t *)fw_dalloc(tmp, (size_t)m * inp);
    float *xs = (float *)fw_dalloc(tmp, sizeof(float) * m);
    if (!xq || !xs) {
        fw_free_all(tmp);
        return fw_fail(FWHIP_ERR_GENERIC, "allocation failed");
    }
    hipStream_t st = c->stream;
    if (which == 3) fw_launch_quant_exact_rows(st, x_dev, m, inp, xq, xs);
    else if (which == 5) fw_launch_gelu_quant_i7_rows(st, x_dev, m, inp, c->gelu_tab, xq, xs);
    else {
        // quantize_act_i7 of the (already normalized) rows: LN-free row quant
        fw_launch_gelu_quant_i7_rows(st, x_dev, m, inp, nullptr, xq, xs);
    }
    const int8_t *W = nullptr;
    const float *Ws = nullptr, *bias = nullptr;
    size_t dd = (size_t)d * d;
    switch (which) {
    case 0: W = l.qkv7; Ws = l.qkv7s; bias = l.qkv_b; break;
    case 1: W = l.qkv7 + dd; Ws = l.qkv7s + d; bias = nullptr; break;
    case 2: W = l.qkv7 + 2 * dd; Ws = l.qkv7s + 2 * d; bias = l.qkv_b + 2 * d; break;
    case 3: W = l.o8; Ws = l.o8s; bias = l.o_b; break;
    case 4: W = l.fc1_7; Ws = l.fc1_7s; bias = l.fc1_b; break;
    default: W = l.fc2_7; Ws = l.fc2_7s; bias = l.fc2_b; break;
    }
    FwGemm g = gemm_args(xq, nullptr, W, m, out, inp, xs, Ws, nullptr, FW_EPI_ACC32, (float *)acc_dev, out);
    fw_launch_gemm(st, FW_KIND_I8, g);
    g = gemm_args(xq, nullptr, W, m, out, inp, xs, Ws, bias, FW_EPI_F32, y_dev, out);
    fw_launch_gemm(st, FW_KIND_I8, g);
    hipError_t err = hipStreamSynchronize(st);
    fw_free_all(tmp);
    if (err != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, hipGetErrorString(err));
    return FWHIP_OK;
}

// Per-GEMM parity of the two fused int8 epilogues the forward runs (see
// include/fwhip.h): the QKV GEMM's head-major f16 hi/lo split with V
// transposed, and fc1 as f16 GELU-table indices with exact side values.
extern "C" fwhip_status fwhip_encoder_gemm_i8_fused(fwhip_encoder *e, int32_t layer, int32_t which,
                                                    const float *x_dev, int32_t n_windows, int32_t n_tokens,
                                                    uint16_t *out16_dev, float *side_dev) {
    if (!e || !x_dev || !out16_dev) return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_gemm_i8_fused: NULL argument");
    if (e->precision != FWHIP_ENC_INT8) return fw_fail(FWHIP_ERR_INVALID, "encoder is not on the int8 plan");
    if (layer < 0 || layer >= e->L || (which != 0 && which != 4) || n_windows <= 0 || n_tokens <= 0 ||
        (int64_t)n_windows * n_tokens > (1 << 30) / e->dff)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_gemm_i8_fused: bad layer/which/size");
    if (which == 4 && (!side_dev || !enc_h16_ok(e->dff)))
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_encoder_gemm_i8_fused: fc1 index form needs side_dev and a "
                                          "supported MLP width");
    fwhip_ctx *c = e->ctx;
    HIP_TRY(hipSetDevice(c->device));
    const int d = e->d, H = e->H, dff = e->dff, T = n_tokens, Tp = (T + 63) / 64 * 64, m = n_windows * n_tokens;
    const EncLayerDev &l = e->layers[layer];
    std::vector<void *> tmp;
    int8_t *xq = (int8_t *)fw_dalloc(tmp, (size_t)m * d);
    float *xs = (float *)fw_dalloc(tmp, sizeof(float) * m);
    if (!xq || !xs) {
        fw_free_all(tmp);
        return fw_fail(FWHIP_ERR_GENERIC, "allocation failed");
    }
    hipStream_t st = c->stream;
    fw_launch_gelu_quant_i7_rows(st, x_dev, m, d, nullptr, xq, xs); // quantize_act_i7
    bool ok;
    if (which == 0) {
        const size_t qk = (size_t)n_windows * H * T * 64, vt = (size_t)n_windows * H * 64 * Tp;
        FwGemm g = gemm_args(xq, nullptr, l.qkv7, m, 3 * d, d, xs, l.qkv7s, l.qkv_b, FW_EPI_QKV, nullptr, d);
        for (int i = 0; i < 4; i++) g.o16[i] = out16_dev + i * qk;
        g.o16[4] = out16_dev + 4 * qk;
        g.o16[5] = out16_dev + 4 * qk + vt;
        g.T = T;
        g.H = H;
        g.Tp = Tp;
        fw_launch_fill_u16(st, g.o16[4], 2 * vt, 0);
        ok = fw_launch_gemm(st, FW_KIND_I8, g);
    } else {
        FwGemm g = gemm_args(xq, nullptr, l.fc1_7, m, dff, d, xs, l.fc1_7s, l.fc1_b, FW_EPI_F16IDX, side_dev, dff);
        g.o16[0] = out16_dev;
        ok = fw_launch_gemm(st, FW_KIND_I8, g);
    }
    hipError_t err = hipStreamSynchronize(st);
    fw_free_all(tmp);
    if (!ok) return fw_fail(FWHIP_ERR_UNSUPPORTED, "fwhip_encoder_gemm_i8_fused: no kernel for this shape");
    if (err != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, hipGetErrorString(err));
    return FWHIP_OK;
}
