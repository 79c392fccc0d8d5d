// fwhip.hip — C ABI of the gfx950 Whisper hot path (include/fwhip.h).
//
// Host-side orchestration only: weight upload and load-time quantization,
// decoder state, per-token step, greedy loop, encoder forward.  All arithmetic
// runs in the kernels of dec_kernels.hip / enc_kernels.hip / load_kernels.hip.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "fw_enc.h"
#include "fw_internal.h"
#include "fw_kernels.h"

static thread_local std::string g_err;

fwhip_status fw_fail(fwhip_status code, const std::string &msg) {
    g_err = msg;
    return code;
}

#define HIP_TRY(expr)                                                                         \
    do {                                                                                      \
        hipError_t _e = (expr);                                                               \
        if (_e != hipSuccess)                                                                 \
            return fw_fail(FWHIP_ERR_GENERIC, std::string(#expr ": ") + hipGetErrorString(_e)); \
    } while (0)

extern "C" const char *fwhip_last_error(void) { return g_err.c_str(); }
extern "C" int32_t fwhip_abi_version(void) { return FWHIP_ABI_VERSION; }

// ---------------------------------------------------------------------------
// context
extern "C" fwhip_status fwhip_init(int32_t device, fwhip_ctx **out) {
    if (!out) return fw_fail(FWHIP_ERR_INVALID, "fwhip_init: out is NULL");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fw_fail(FWHIP_ERR_UNSUPPORTED, "cpu:no-hip-device");
    if (device < 0 || device >= n) return fw_fail(FWHIP_ERR_INVALID, "fwhip_init: device out of range");
    hipDeviceProp_t prop;
    HIP_TRY(hipGetDeviceProperties(&prop, device));
    if (std::string(prop.gcnArchName).find("gfx950") == std::string::npos)
        return fw_fail(FWHIP_ERR_UNSUPPORTED, std::string("cpu:unsupported-arch:") + prop.gcnArchName);
    HIP_TRY(hipSetDevice(device));
    fw_mel_noalloc_setup(device);
    fwhip_ctx *c = new fwhip_ctx();
    c->device = device;
    c->n_cu = prop.multiProcessorCount;
    if (hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking) != hipSuccess) {
        delete c;
        return fw_fail(FWHIP_ERR_GENERIC, "hipStreamCreate failed");
    }
    // GELU table (gelu_table, nn.rs:4561-4575) built on the host with the
    // platform tanhf, exactly as the reference builds it.
    // The f32 values are f16-exact; their f16 copy follows them in the same
    // allocation (fw_gelu_tab16) for the kernels that keep the table in LDS.
    std::vector<float> tab(1 << 16);
    std::vector<uint16_t> tab16(1 << 16);
    for (int i = 0; i < (1 << 16); i++) {
        float f = fw_host_h2f((uint16_t)i);
        float g = 0.5f * f * (1.0f + tanhf(0.7978846f * f * (1.0f + 0.044715f * f * f)));
        tab16[i] = fw_host_f2h(g);
        tab[i] = fw_host_h2f(tab16[i]);
    }
    const size_t tb = sizeof(float) * tab.size();
    if (hipMalloc(&c->gelu_tab, tb + sizeof(uint16_t) * tab16.size()) != hipSuccess ||
        hipMemcpy(c->gelu_tab, tab.data(), tb, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy((char *)c->gelu_tab + tb, tab16.data(), sizeof(uint16_t) * tab16.size(), hipMemcpyHostToDevice) !=
            hipSuccess) {
        fwhip_destroy(c);
        return fw_fail(FWHIP_ERR_GENERIC, "gelu table upload failed");
    }
    if (hipMalloc(&c->ovf_dev, 256) != hipSuccess || hipHostMalloc(&c->ovf_host, 256) != hipSuccess ||
        hipMemset(c->ovf_dev, 0, 256) != hipSuccess) {
        fwhip_destroy(c);
        return fw_fail(FWHIP_ERR_GENERIC, "flag allocation failed");
    }
    *c->ovf_host = 0;
    *out = c;
    return FWHIP_OK;
}

void fw_ovf_clear(fwhip_ctx *c) { fw_launch_fill_u16(c->stream, (uint16_t *)c->ovf_dev, 2, 0); }
void fw_ovf_fetch(fwhip_ctx *c) {
    (void)hipMemcpyAsync(c->ovf_host, c->ovf_dev, sizeof(int), hipMemcpyDeviceToHost, c->stream);
}

extern "C" const char *fwhip_gemm_precision_str(int32_t p) {
    static const char *const names[] = {"f32", "i7", "i8", "f16", "f16_weights", "q8_0_weights", "f16_kv",
                                        "mixed", "f16_pair"};
    return p >= 0 && p < (int32_t)(sizeof names / sizeof names[0]) ? names[p] : nullptr;
}

extern "C" void fwhip_destroy(fwhip_ctx *c) {
    if (!c) return;
    hipSetDevice(c->device);
    hipStreamSynchronize(c->stream);
    for (auto &e : c->pending) {
        hipEventDestroy(e.a);
        hipEventDestroy(e.b);
    }
    for (hipEvent_t e : c->ev_pool) hipEventDestroy(e);
    if (c->gelu_tab) hipFree(c->gelu_tab);
    if (c->mel_tab) hipFree(c->mel_tab);
    if (c->mel_scratch) hipFree(c->mel_scratch);
    if (c->am_scratch) hipFree(c->am_scratch);
    if (c->ovf_dev) hipFree(c->ovf_dev);
    if (c->ovf_host) hipHostFree(c->ovf_host);
    hipStreamDestroy(c->stream);
    delete c;
}

extern "C" fwhip_status fwhip_malloc(fwhip_ctx *c, size_t bytes, void **dev) {
    if (!c || !dev) return fw_fail(FWHIP_ERR_INVALID, "fwhip_malloc: NULL argument");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipMalloc(dev, bytes ? bytes : 1));
    return FWHIP_OK;
}
extern "C" fwhip_status fwhip_free(fwhip_ctx *c, void *dev) {
    if (!c) return fw_fail(FWHIP_ERR_INVALID, "fwhip_free: NULL ctx");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (dev) HIP_TRY(hipFree(dev));
    return FWHIP_OK;
}
extern "C" fwhip_status fwhip_upload(fwhip_ctx *c, void *dev, const void *host, size_t bytes) {
    if (!c || (!dev && bytes) || (!host && bytes)) return fw_fail(FWHIP_ERR_INVALID, "fwhip_upload: NULL");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipMemcpyAsync(dev, host, bytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return FWHIP_OK;
}
extern "C" fwhip_status fwhip_download(fwhip_ctx *c, void *host, const void *dev, size_t bytes) {
    if (!c || (!dev && bytes) || (!host && bytes)) return fw_fail(FWHIP_ERR_INVALID, "fwhip_download: NULL");
    HIP_TRY(hipSetDevice(c->device));
    HIP_TRY(hipMemcpyAsync(host, dev, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return FWHIP_OK;
}
extern "C" fwhip_status fwhip_synchronize(fwhip_ctx *c) {
    if (!c) return fw_fail(FWHIP_ERR_INVALID, "NULL ctx");
    HIP_TRY(hipStreamSynchronize(c->stream));
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, std::string("kernel error: ") + hipGetErrorString(e));
    return FWHIP_OK;
}
extern "C" fwhip_status fwhip_request_cancel(fwhip_ctx *c) {
    if (!c) return fw_fail(FWHIP_ERR_INVALID, "NULL ctx");
    c->cancel.store(1);
    return FWHIP_OK;
}

// ---- kernel timing ---------------------------------------------------------
void fw_timed_begin(fwhip_ctx *c, int cls, double units, fw_event_pair *ev) {
    ev->active = c->timing;
    if (!ev->active) return;
    ev->cls = cls;
    ev->units = units;
    hipEvent_t *e[2] = {&ev->a, &ev->b};
    for (hipEvent_t *p : e) {
        if (!c->ev_pool.empty()) {
            *p = c->ev_pool.back();
            c->ev_pool.pop_back();
        } else {
            hipEventCreate(p);
        }
    }
    hipEventRecord(ev->a, c->stream);
}
void fw_timed_end(fwhip_ctx *c, fw_event_pair *ev) {
    if (!ev->active) return;
    hipEventRecord(ev->b, c->stream);
    c->pending.push_back(*ev);
}
static void fw_drain_events(fwhip_ctx *c) {
    if (c->pending.empty()) return;
    hipStreamSynchronize(c->stream);
    for (auto &e : c->pending) {
        float ms = 0.0f;
        hipEventElapsedTime(&ms, e.a, e.b);
        auto &s = c->stats[e.cls];
        s.launches += 1;
        s.ms += ms;
        s.units += e.units;
        c->ev_pool.push_back(e.a);
        c->ev_pool.push_back(e.b);
    }
    c->pending.clear();
}
extern "C" fwhip_status fwhip_kernel_timing(fwhip_ctx *c, int32_t enable) {
    if (!c) return fw_fail(FWHIP_ERR_INVALID, "NULL ctx");
    fw_drain_events(c);
    c->stats.clear();
    c->timing = enable != 0;
    return FWHIP_OK;
}
extern "C" fwhip_status fwhip_kernel_stats(fwhip_ctx *c, int32_t cls, int64_t *launches, double *total_ms,
                                           double *units) {
    if (!c) return fw_fail(FWHIP_ERR_INVALID, "NULL ctx");
    fw_drain_events(c);
    auto it = c->stats.find(cls);
    if (launches) *launches = it == c->stats.end() ? 0 : it->second.launches;
    if (total_ms) *total_ms = it == c->stats.end() ? 0.0 : it->second.ms;
    if (units) *units = it == c->stats.end() ? 0.0 : it->second.units;
    return FWHIP_OK;
}

// ---------------------------------------------------------------------------
// device buffers owned by a model/state
void *fw_dalloc(std::vector<void *> &owned, size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) return nullptr;
    owned.push_back(p);
    return p;
}
void *fw_dupload(std::vector<void *> &owned, const void *host, size_t bytes) {
    void *p = fw_dalloc(owned, bytes);
    if (p && host && bytes) {
        if (hipMemcpy(p, host, bytes, hipMemcpyHostToDevice) != hipSuccess) return nullptr;
    }
    return p;
}
void fw_free_all(std::vector<void *> &owned) {
    for (void *p : owned) hipFree(p);
    owned.clear();
}

// ---------------------------------------------------------------------------
// decoder
struct DecLayerDev {
    const float *attn_ln_w, *attn_ln_b, *cross_ln_w, *cross_ln_b, *mlp_ln_w, *mlp_ln_b;
    const float *qkv_b, *o_b, *cq_b, *co_b, *fc1_b, *fc2_b, *cv_b;
    // o8, co8, fc1_8 (and the decoder's emb8) are in the int8 GEMV's fragment
    // order; qkv8 and cq8 (read by the attention kernels) are row-major
    const int8_t *qkv8 = nullptr, *o8 = nullptr, *cq8 = nullptr, *co8 = nullptr, *fc1_8 = nullptr,
                 *fc2_b8 = nullptr;
    const float *qkv8s = nullptr, *o8s = nullptr, *cq8s = nullptr, *co8s = nullptr, *fc1_8s = nullptr,
                *fc2_b8s = nullptr;
    const uint16_t *qkv16 = nullptr, *o16 = nullptr, *cq16 = nullptr, *co16 = nullptr, *fc1_16 = nullptr,
                   *fc2_16 = nullptr, *ck16w = nullptr, *cv16w = nullptr;
};

struct fwhip_decoder {
    fwhip_ctx *ctx;
    int arm;
    fwhip_hparams hp;
    int d, H, L, V, nctx, dff;
    const uint16_t *emb16 = nullptr;  // natural order (the token embedding gather)
    const uint16_t *emb16f = nullptr; // f16 arm: the tied logits head in GEMV fragment order
    const int8_t *emb8 = nullptr;
    const float *emb8s = nullptr;
    const float *pos_emb = nullptr, *ln_w = nullptr, *ln_b = nullptr;
    // cross K and V weights of every layer, [L][K rows; V rows][d] f16, and the
    // matching bias [L][0 | cv_b] (one f16-pair GEMM makes every layer's cross K/V)
    const uint16_t *ckv16 = nullptr;
    const float *ckv_b = nullptr;
    // 1: strict sequential-k cross K/V precompute, and every LayerNorm's mean
    // and variance summed in the reference's sequential order
    int exact = 0;
    // self-attention cache of the states made next: f16 (FW_KV_F16) or f32
    // (the reference's default), read when a state is made, as KvCache::new does
    int kv_f16 = 1;
    // FW_CROSS_V_BLOCK (the int8 arm; default off): read when a state is made
    int cross_v_block = 0;
    std::vector<DecLayerDev> layers;
    std::vector<void *> owned;
};

struct fwhip_dstate {
    fwhip_decoder *dec;
    int S, T, Tq, Sp, len;
    void *kv_k, *kv_v; // [S][L][nctx][d] f16, or f32 when kv32
    int kv32 = 0;
    uint16_t *ck16, *cvt16;
    uint16_t *ck16p = nullptr, *cvt16p = nullptr; // f16 arm: slot-order copies for the cross attention
    float *xsplit = nullptr; // f16 arm: scores and block maxima of the two-launch cross attention
    int *am_cnt = nullptr;   // argmax blocks counted in (zero between launches)
    int8_t *ck8 = nullptr, *cvt8 = nullptr; // cvt8 rows have stride Tq (T rounded up to 16)
    float *ck8s = nullptr, *cvt8s = nullptr;
    int8_t *cvb8 = nullptr; // FW_CROSS_V_BLOCK: block-int8 V^T, rows of stride Tq
    float *cvbs = nullptr;  // its scales [S, L, H, 64, ceil(T / 32)]
    float *x, *h, *qkv, *att, *y, *ff, *logits;
    int8_t *xq;             // [Sp, d] quantized activation rows (rows >= S stay zero)
    float *xs;              // [Sp]
    unsigned long long *keys; // [S, nkeys] per-block argmax keys
    int nkeys;
    int32_t *tok, *hist, *rows;
    int *pos, *initial, *stepc;
    float *pmax;            // [S, H] per-head max |attention output|
    uint16_t *ench, *encl;  // [S * T, d] f16 pair of the encoder states (fast cross K/V)
    int hist_cap;
    // captured sampling step (forward of st->tok + argmax + bookkeeping)
    hipGraphExec_t graph = nullptr;
    fwhip_filter graph_filter;
    int graph_lnseq = 0, wgraph_lnseq = 0; // the decoder's exact flag when each graph was captured
    std::vector<void *> owned;
    // the window loop (fwhip_decode_window): filtered rows of every step, the
    // raw prefill rows, per-stream loop state, forced flags, exact-sum scratch,
    // log-probabilities; allocated on first use for n_max steps
    float *w_rows = nullptr, *w_nsrow = nullptr, *w_scratch = nullptr, *w_plogs = nullptr, *w_nslp = nullptr;
    FwWinStream *w_ws = nullptr;
    uint8_t *w_forced = nullptr;
    int *w_ndone = nullptr;
    // pinned host buffer the loops' end-of-text polls copy into: the newest
    // columns of the token history, or the done count (allocated on first use)
    int32_t *poll_host = nullptr;
    int poll_cap = 0;
    // batched prompt prefill (f16 arm): activation rows of a chunk of
    // PF_CHUNK positions x S streams, allocated on first use
    std::vector<void *> pf_owned;
    float *pf_x = nullptr, *pf_h = nullptr, *pf_qkv = nullptr, *pf_att = nullptr, *pf_y = nullptr, *pf_ff = nullptr;
    FwWinPart *w_part = nullptr; // [S][WIN_NB] partial results of the select blocks
    int *w_cnt = nullptr;        // [S] select blocks counted in (zero between launches)
    int w_nmax = 0, w_ldr = 0;
    std::vector<void *> w_owned;
    hipGraphExec_t wgraph = nullptr;
    FwWinCfg wgraph_cfg;
};

// Quantize a host f16 [out, inp] matrix to per-row int8 on the device; with
// `frag` the int8 matrix is kept in the int8 GEMV's fragment order
// (fw_launch_pack_gemv_frags) instead of row-major.
static bool dev_quant_rows(fwhip_ctx *c, std::vector<void *> &owned, const uint16_t *host, int64_t out, int inp,
                           const int8_t **q, const float **s, bool frag = false) {
    uint16_t *tmp = nullptr;
    int8_t *rm = nullptr;
    size_t bytes = sizeof(uint16_t) * (size_t)out * inp;
    bool ok = hipMalloc(&tmp, bytes) == hipSuccess;
    ok = ok && hipMemcpy(tmp, host, bytes, hipMemcpyHostToDevice) == hipSuccess;
    int8_t *qq = nullptr;
    float *ss = ok ? (float *)fw_dalloc(owned, sizeof(float) * out) : nullptr;
    if (ok && frag) {
        qq = (int8_t *)fw_dalloc(owned, fw_gemv_frag_bytes((int)out, inp));
        ok = qq && hipMalloc(&rm, (size_t)out * inp) == hipSuccess;
    } else if (ok) {
        rm = qq = (int8_t *)fw_dalloc(owned, (size_t)out * inp);
    }
    ok = ok && ss && rm;
    if (ok) {
        fw_launch_quant_f16_rows(c->stream, tmp, rm, ss, (int)out, inp);
        if (frag) fw_launch_pack_gemv_frags(c->stream, rm, qq, (int)out, inp);
        ok = hipStreamSynchronize(c->stream) == hipSuccess;
    }
    if (tmp) hipFree(tmp);
    if (frag && rm) hipFree(rm);
    if (!ok) return false;
    *q = qq;
    *s = ss;
    return true;
}

static bool dev_quant_blocked(fwhip_ctx *c, std::vector<void *> &owned, const uint16_t *host, int64_t out,
                              int inp, const int8_t **q, const float **s) {
    uint16_t *tmp = nullptr;
    size_t bytes = sizeof(uint16_t) * (size_t)out * inp;
    if (hipMalloc(&tmp, bytes) != hipSuccess) return false;
    if (hipMemcpy(tmp, host, bytes, hipMemcpyHostToDevice) != hipSuccess) return false;
    int nb = (inp + 31) / 32;
    int8_t *qq = (int8_t *)fw_dalloc(owned, (size_t)out * inp);
    float *ss = (float *)fw_dalloc(owned, sizeof(float) * out * nb);
    if (!qq || !ss) return false;
    fw_launch_quant_blocked(c->stream, tmp, qq, ss, out, inp, 32);
    if (hipStreamSynchronize(c->stream) != hipSuccess) return false;
    hipFree(tmp);
    *q = qq;
    *s = ss;
    return true;
}

// The f16 arm's logits head forms its argmax keys inside the GEMV when that
// GEMV takes the shape (slot order, the final LayerNorm fused: d <= 1280).
static bool f16_fused_keys(const fwhip_decoder *dd) {
    return dd->arm == FWHIP_DEC_F16 && fw_gemv16_ok(dd->V, dd->d) && dd->d <= 1280;
}

// An f16 GEMV weight [N, K] repacked for the cohort GEMV: slot order when
// fw_gemv16_ok(N, K) (dec_gemv16.hip), else the fragment order of
// fw_gemv_f16_frag_ok, else natural order; fw_gemv16 launches the matching
// kernel.  `nat` (device, natural order) is freed when repacked unless keep_nat.
static const uint16_t *frag16(fwhip_ctx *c, std::vector<void *> &owned, const uint16_t *nat, int N, int K,
                              bool keep_nat = false) {
    const bool slot = fw_gemv16_ok(N, K);
    if (!nat || (!slot && !fw_gemv_f16_frag_ok(N, K))) return nat;
    uint16_t *f = (uint16_t *)fw_dalloc(owned, sizeof(uint16_t) * (size_t)N * K);
    if (!f) return nullptr;
    if (slot) fw_launch_pack_gemv16(c->stream, nat, f, N, K);
    else fw_launch_pack_gemv_f16(c->stream, nat, f, N, K);
    if (hipStreamSynchronize(c->stream) != hipSuccess) return nullptr;
    if (!keep_nat) {
        for (auto it = owned.begin(); it != owned.end(); ++it)
            if (*it == (const void *)nat) {
                owned.erase(it);
                break;
            }
        hipFree((void *)nat);
    }
    return f;
}
static void fw_gemv16(hipStream_t st, const uint16_t *W, const float *bias, const float *x, float *y, int N, int K,
                      int ns, int ldy, int mode, const float *gelu_tab) {
    if (fw_gemv16_ok(N, K)) fw_launch_gemv16(st, W, bias, x, y, N, K, ns, ldy, mode, gelu_tab);
    else if (fw_gemv_f16_frag_ok(N, K)) fw_launch_gemv_f16f(st, W, bias, x, y, N, K, ns, ldy, mode, gelu_tab);
    else fw_launch_gemv_f16(st, W, bias, x, y, N, K, ns, ldy, mode, gelu_tab);
}
// y = W LayerNorm(x) (+ bias): the LayerNorm inside the GEMV where its kernel
// stages whole rows (K <= 1280), else a LayerNorm pass into h.
// seq: the LayerNorm's sums in the reference's sequential order (exact mode),
// always as a pass of its own (one row per block) ahead of the plain GEMV: the
// GEMV's blocks would each run every sequential sum of their rows, several to
// a CU (10 streams: 72 against 20 us for fc1), for the same normalized values.
static void fw_gemv16_ln(hipStream_t st, const uint16_t *W, const float *bias, const float *x, float *h,
                         const float *lnw, const float *lnb, float *y, int N, int K, int ns, int ldy, int mode,
                         const float *gelu_tab, int seq = 0) {
    if (seq) {
        fw_launch_ln_quant(st, x, h, lnw, lnb, K, ns, nullptr, nullptr, 1);
        fw_gemv16(st, W, bias, h, y, N, K, ns, ldy, mode, gelu_tab);
    } else if (fw_gemv16_ok(N, K) && K <= 1280) {
        fw_launch_gemv16(st, W, bias, x, y, N, K, ns, ldy, mode, gelu_tab, lnw, lnb);
    } else if (fw_gemv_f16_frag_ok(N, K) && K <= 1280) {
        fw_launch_gemv_f16f(st, W, bias, x, y, N, K, ns, ldy, mode, gelu_tab, lnw, lnb);
    } else {
        fw_launch_ln_quant(st, x, h, lnw, lnb, K, ns, nullptr, nullptr, seq);
        fw_gemv16(st, W, bias, h, y, N, K, ns, ldy, mode, gelu_tab);
    }
}

static bool hp_decoder_ok(const fwhip_hparams &hp, std::string &why) {
    if (hp.n_text_state <= 0 || hp.n_text_head <= 0 || hp.n_text_layer <= 0 || hp.n_vocab <= 0 ||
        hp.n_text_ctx <= 0) {
        why = "non-positive decoder hparam";
        return false;
    }
    if (hp.n_text_state % hp.n_text_head) {
        why = "n_text_head must divide n_text_state";
        return false;
    }
    if (hp.n_text_state / hp.n_text_head != 64) {
        why = "d_head must be 64";
        return false;
    }
    // The row LayerNorm/quantize kernels keep one row per wave in registers.
    if (hp.n_text_state > 2048) {
        why = "n_text_state must be at most 2048";
        return false;
    }
    return true;
}

fwhip_ctx *fw_decoder_ctx(const fwhip_decoder *d) { return d->ctx; }
fwhip_hparams fw_decoder_hparams(const fwhip_decoder *d) { return d->hp; }

extern "C" fwhip_status fwhip_decoder_load(fwhip_ctx *c, const fwhip_decoder_weights *w, int32_t arm,
                                           fwhip_decoder **out) {
    if (!c || !w || !out) return fw_fail(FWHIP_ERR_INVALID, "fwhip_decoder_load: NULL argument");
    *out = nullptr;
    if (arm != FWHIP_DEC_INT8 && arm != FWHIP_DEC_F16) return fw_fail(FWHIP_ERR_INVALID, "unknown decoder arm");
    std::string why;
    if (!hp_decoder_ok(w->hp, why)) return fw_fail(FWHIP_ERR_INVALID, "fwhip_decoder_load: " + why);
    HIP_TRY(hipSetDevice(c->device));
    fwhip_decoder *dd = new fwhip_decoder();
    dd->ctx = c;
    dd->arm = arm;
    dd->hp = w->hp;
    dd->d = w->hp.n_text_state;
    dd->H = w->hp.n_text_head;
    dd->L = w->hp.n_text_layer;
    dd->V = w->hp.n_vocab;
    dd->nctx = w->hp.n_text_ctx;
    dd->dff = 4 * dd->d;
    int d = dd->d, dff = dd->dff;
    auto &own = dd->owned;
    bool ok = true;
    auto up32 = [&](const float *p, size_t n) -> const float * {
        if (!p) return nullptr;
        const float *r = (const float *)fw_dupload(own, p, sizeof(float) * n);
        ok = ok && r;
        return r;
    };
    auto up16 = [&](const uint16_t *p, size_t n) -> const uint16_t * {
        const uint16_t *r = (const uint16_t *)fw_dupload(own, p, sizeof(uint16_t) * n);
        ok = ok && r;
        return r;
    };
    dd->emb16 = up16(w->tok_emb, (size_t)dd->V * d);
    dd->pos_emb = up32(w->pos_emb, (size_t)dd->nctx * d);
    dd->ln_w = up32(w->ln_w, d);
    dd->ln_b = up32(w->ln_b, d);
    {
        std::vector<uint16_t> ckv((size_t)dd->L * 2 * d * d);
        std::vector<float> ckvb((size_t)dd->L * 2 * d, 0.0f);
        for (int li = 0; li < dd->L; li++) {
            memcpy(ckv.data() + (size_t)li * 2 * d * d, w->layers[li].ck_w, sizeof(uint16_t) * d * d);
            memcpy(ckv.data() + ((size_t)li * 2 + 1) * d * d, w->layers[li].cv_w, sizeof(uint16_t) * d * d);
            memcpy(ckvb.data() + ((size_t)li * 2 + 1) * d, w->layers[li].cv_b, sizeof(float) * d);
        }
        dd->ckv16 = up16(ckv.data(), ckv.size());
        dd->ckv_b = up32(ckvb.data(), ckvb.size());
    }
    if (ok && arm == FWHIP_DEC_INT8) ok = dev_quant_rows(c, own, w->tok_emb, dd->V, d, &dd->emb8, &dd->emb8s, true);
    if (ok && arm == FWHIP_DEC_F16) {
        dd->emb16f = frag16(c, own, dd->emb16, dd->V, d, true);
        ok = dd->emb16f != nullptr;
    }
    for (int li = 0; ok && li < dd->L; li++) {
        const fwhip_dec_layer &s = w->layers[li];
        DecLayerDev l;
        l.attn_ln_w = up32(s.attn_ln_w, d);
        l.attn_ln_b = up32(s.attn_ln_b, d);
        l.cross_ln_w = up32(s.cross_ln_w, d);
        l.cross_ln_b = up32(s.cross_ln_b, d);
        l.mlp_ln_w = up32(s.mlp_ln_w, d);
        l.mlp_ln_b = up32(s.mlp_ln_b, d);
        // fuse_qkv (decoder.rs:2245-2289): [q; k; v] rows, bias [q_b | 0 | v_b]
        std::vector<uint16_t> qkv((size_t)3 * d * d);
        memcpy(qkv.data(), s.q_w, sizeof(uint16_t) * d * d);
        memcpy(qkv.data() + (size_t)d * d, s.k_w, sizeof(uint16_t) * d * d);
        memcpy(qkv.data() + (size_t)2 * d * d, s.v_w, sizeof(uint16_t) * d * d);
        std::vector<float> qkvb((size_t)3 * d, 0.0f);
        memcpy(qkvb.data(), s.q_b, sizeof(float) * d);
        memcpy(qkvb.data() + 2 * d, s.v_b, sizeof(float) * d);
        l.qkv_b = up32(qkvb.data(), 3 * d);
        l.o_b = up32(s.o_b, d);
        l.cq_b = up32(s.cq_b, d);
        l.co_b = up32(s.co_b, d);
        l.fc1_b = up32(s.fc1_b, dff);
        l.fc2_b = up32(s.fc2_b, d);
        l.cv_b = up32(s.cv_b, d);
        l.ck16w = dd->ckv16 ? dd->ckv16 + (size_t)li * 2 * d * d : nullptr;
        l.cv16w = dd->ckv16 ? dd->ckv16 + ((size_t)li * 2 + 1) * d * d : nullptr;
        l.fc2_16 = frag16(c, own, up16(s.fc2_w, (size_t)d * dff), d, dff); // prefill arm of mlp_2 in both arms
        if (arm == FWHIP_DEC_INT8) {
            ok = ok && dev_quant_rows(c, own, qkv.data(), 3 * d, d, &l.qkv8, &l.qkv8s);
            ok = ok && dev_quant_rows(c, own, s.o_w, d, d, &l.o8, &l.o8s, true);
            ok = ok && dev_quant_rows(c, own, s.cq_w, d, d, &l.cq8, &l.cq8s);
            ok = ok && dev_quant_rows(c, own, s.co_w, d, d, &l.co8, &l.co8s, true);
            ok = ok && dev_quant_rows(c, own, s.fc1_w, dff, d, &l.fc1_8, &l.fc1_8s, true);
            ok = ok && dev_quant_blocked(c, own, s.fc2_w, d, dff, &l.fc2_b8, &l.fc2_b8s);
        } else {
            l.qkv16 = frag16(c, own, up16(qkv.data(), (size_t)3 * d * d), 3 * d, d);
            l.o16 = frag16(c, own, up16(s.o_w, (size_t)d * d), d, d);
            l.cq16 = frag16(c, own, up16(s.cq_w, (size_t)d * d), d, d);
            l.co16 = frag16(c, own, up16(s.co_w, (size_t)d * d), d, d);
            l.fc1_16 = frag16(c, own, up16(s.fc1_w, (size_t)dff * d), dff, d);
            ok = ok && l.qkv16 && l.o16 && l.cq16 && l.co16 && l.fc1_16;
        }
        dd->layers.push_back(l);
    }
    if (!ok || hipDeviceSynchronize() != hipSuccess) {
        fw_free_all(own);
        delete dd;
        return fw_fail(FWHIP_ERR_GENERIC, "fwhip_decoder_load: device allocation or upload failed");
    }
    *out = dd;
    return FWHIP_OK;
}

extern "C" void fwhip_decoder_free(fwhip_decoder *dd) {
    if (!dd) return;
    hipSetDevice(dd->ctx->device);
    hipStreamSynchronize(dd->ctx->stream);
    fw_free_all(dd->owned);
    delete dd;
}

extern "C" fwhip_status fwhip_dstate_new(fwhip_decoder *dd, int32_t S, int32_t T, fwhip_dstate **out) {
    if (!dd || !out) return fw_fail(FWHIP_ERR_INVALID, "fwhip_dstate_new: NULL argument");
    *out = nullptr;
    if (S <= 0 || T <= 0) return fw_fail(FWHIP_ERR_INVALID, "fwhip_dstate_new: n_streams and enc_frames must be > 0");
    // the int8 cross-attention kernel stages a head's Vt rows (64 x T bytes) in LDS
    if (dd->arm == FWHIP_DEC_INT8 && T > 1536)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_dstate_new: enc_frames must be at most 1536 on the int8 arm");
    fwhip_ctx *c = dd->ctx;
    HIP_TRY(hipSetDevice(c->device));
    fwhip_dstate *st = new fwhip_dstate();
    st->dec = dd;
    st->S = S;
    st->T = T;
    st->Tq = (T + 15) & ~15;
    st->Sp = (S + 15) & ~15;
    st->len = 0;
    int d = dd->d, L = dd->L, nctx = dd->nctx;
    auto &own = st->owned;
    size_t kvn = (size_t)S * L * nctx * d;
    size_t crn = (size_t)S * L * T * d;
    st->kv32 = dd->kv_f16 ? 0 : 1;
    st->kv_k = fw_dalloc(own, kvn * (st->kv32 ? 4 : 2));
    st->kv_v = fw_dalloc(own, kvn * (st->kv32 ? 4 : 2));
    st->ck16 = (uint16_t *)fw_dalloc(own, crn * 2);
    st->cvt16 = (uint16_t *)fw_dalloc(own, crn * 2);
    bool ok = st->kv_k && st->kv_v && st->ck16 && st->cvt16;
    if (dd->arm == FWHIP_DEC_F16 && fw_cross_f16p_ok(T)) {
        st->ck16p = (uint16_t *)fw_dalloc(own, crn * 2);
        const size_t vpn = (size_t)S * L * dd->H * 64 * fw_cross_f16p_tv(T);
        st->cvt16p = (uint16_t *)fw_dalloc(own, vpn * 2);
        st->xsplit = (float *)fw_dalloc(own, sizeof(float) * fw_cross_split_floats(T, dd->H, S));
        ok = ok && st->ck16p && st->cvt16p && st->xsplit;
        if (ok) ok = hipMemset(st->cvt16p, 0, vpn * 2) == hipSuccess;
    }
    if (dd->arm == FWHIP_DEC_INT8) {
        st->ck8 = (int8_t *)fw_dalloc(own, crn);
        st->cvt8 = (int8_t *)fw_dalloc(own, (size_t)S * L * dd->H * 64 * st->Tq);
        st->ck8s = (float *)fw_dalloc(own, sizeof(float) * (size_t)S * L * dd->H * T);
        st->cvt8s = (float *)fw_dalloc(own, sizeof(float) * (size_t)S * L * d);
        ok = ok && st->ck8 && st->cvt8 && st->ck8s && st->cvt8s;
        if (dd->cross_v_block) {
            st->cvb8 = (int8_t *)fw_dalloc(own, (size_t)S * L * dd->H * 64 * st->Tq);
            st->cvbs = (float *)fw_dalloc(own, sizeof(float) * (size_t)S * L * dd->H * 64 * ((T + 31) / 32));
            ok = ok && st->cvb8 && st->cvbs;
        }
    }
    st->x = (float *)fw_dalloc(own, sizeof(float) * S * d);
    st->h = (float *)fw_dalloc(own, sizeof(float) * S * d);
    st->qkv = (float *)fw_dalloc(own, sizeof(float) * S * 3 * d);
    st->att = (float *)fw_dalloc(own, sizeof(float) * S * d);
    st->y = (float *)fw_dalloc(own, sizeof(float) * S * d);
    st->ff = (float *)fw_dalloc(own, sizeof(float) * S * dd->dff);
    st->logits = (float *)fw_dalloc(own, sizeof(float) * (size_t)S * dd->V);
    st->xq = (int8_t *)fw_dalloc(own, (size_t)st->Sp * d);
    st->xs = (float *)fw_dalloc(own, sizeof(float) * st->Sp);
    st->nkeys = dd->arm == FWHIP_DEC_INT8 ? fw_gemv_i8m_blocks(dd->V)
                : f16_fused_keys(dd)         ? fw_gemv16_key_blocks(dd->V, d)
                                             : fw_logits_keys_blocks(dd->V);
    st->keys = (unsigned long long *)fw_dalloc(own, sizeof(unsigned long long) * (size_t)S * st->nkeys);
    st->tok = (int32_t *)fw_dalloc(own, sizeof(int32_t) * S);
    st->rows = (int32_t *)fw_dalloc(own, sizeof(int32_t) * (size_t)S * nctx);
    st->hist_cap = nctx;
    st->hist = (int32_t *)fw_dalloc(own, sizeof(int32_t) * (size_t)S * nctx);
    st->pos = (int *)fw_dalloc(own, sizeof(int) * 5);
    st->initial = st->pos + 1;
    st->stepc = st->pos + 2;
    st->am_cnt = st->pos + 4;
    st->pmax = (float *)fw_dalloc(own, sizeof(float) * (size_t)S * dd->H);
    st->ench = (uint16_t *)fw_dalloc(own, sizeof(uint16_t) * (size_t)S * T * d);
    st->encl = (uint16_t *)fw_dalloc(own, sizeof(uint16_t) * (size_t)S * T * d);
    ok = ok && st->x && st->h && st->qkv && st->att && st->y && st->ff && st->logits && st->xq && st->xs &&
         st->keys && st->tok && st->rows && st->hist && st->pos && st->pmax && st->ench && st->encl;
    // padding rows of the quantized activations must read as zeros
    ok = ok && hipMemset(st->xq, 0, (size_t)st->Sp * d) == hipSuccess && hipMemset(st->pos, 0, sizeof(int) * 5) == hipSuccess;
    if (!ok) {
        fw_free_all(own);
        delete st;
        return fw_fail(FWHIP_ERR_GENERIC, "fwhip_dstate_new: device allocation failed");
    }
    *out = st;
    return FWHIP_OK;
}

extern "C" void fwhip_dstate_free(fwhip_dstate *st) {
    if (!st) return;
    hipSetDevice(st->dec->ctx->device);
    hipStreamSynchronize(st->dec->ctx->stream);
    if (st->graph) hipGraphExecDestroy(st->graph);
    if (st->wgraph) hipGraphExecDestroy(st->wgraph);
    fw_free_all(st->w_owned);
    fw_free_all(st->pf_owned);
    fw_free_all(st->owned);
    if (st->poll_host) hipHostFree(st->poll_host);
    delete st;
}

extern "C" fwhip_status fwhip_dstate_reset(fwhip_dstate *st) {
    if (!st) return fw_fail(FWHIP_ERR_INVALID, "NULL state");
    st->len = 0;
    return FWHIP_OK;
}
extern "C" int32_t fwhip_dstate_len(const fwhip_dstate *st, int32_t) { return st ? st->len : -1; }

extern "C" fwhip_status fwhip_dstate_read(const fwhip_dstate *st, int32_t what, int32_t stream, void *host,
                                          size_t bytes) {
    if (!st || !host) return fw_fail(FWHIP_ERR_INVALID, "fwhip_dstate_read: NULL argument");
    if (stream < 0 || stream >= st->S) return fw_fail(FWHIP_ERR_INVALID, "fwhip_dstate_read: stream out of range");
    const fwhip_decoder *dd = st->dec;
    HIP_TRY(hipSetDevice(dd->ctx->device));
    size_t cr = (size_t)dd->L * st->T * dd->d * 2, kv = (size_t)dd->L * dd->nctx * dd->d * (st->kv32 ? 4 : 2);
    const void *src = nullptr;
    size_t n = 0;
    switch (what) {
    case FWHIP_DS_CROSS_K_F16: src = (const char *)st->ck16 + stream * cr; n = cr; break;
    case FWHIP_DS_CROSS_VT_F16: src = (const char *)st->cvt16 + stream * cr; n = cr; break;
    case FWHIP_DS_KV_K: src = (const char *)st->kv_k + stream * kv; n = kv; break;
    case FWHIP_DS_KV_V: src = (const char *)st->kv_v + stream * kv; n = kv; break;
    default: return fw_fail(FWHIP_ERR_INVALID, "fwhip_dstate_read: unknown buffer");
    }
    if (bytes != n) return fw_fail(FWHIP_ERR_INVALID, "fwhip_dstate_read: size mismatch, need " + std::to_string(n));
    HIP_TRY(hipStreamSynchronize(dd->ctx->stream));
    HIP_TRY(hipMemcpy(host, src, n, hipMemcpyDeviceToHost));
    return FWHIP_OK;
}

extern "C" fwhip_status fwhip_decoder_set_exact(fwhip_decoder *dd, int32_t exact) {
    if (!dd) return fw_fail(FWHIP_ERR_INVALID, "NULL decoder");
    dd->exact = exact != 0;
    return FWHIP_OK;
}

// FW_CROSS_V_BLOCK (cross_v_block_enabled, decoder.rs:1496-1520): states made
// after this call on the int8 arm keep a block-int8 copy of the cross V
// (quantize_f16_to_i8_blocked along the frames, 32 per scale,
// decoder.rs:1249-1263) for a value pass on f32 softmax weights
extern "C" fwhip_status fwhip_decoder_set_cross_v_block(fwhip_decoder *dd, int32_t on) {
    if (!dd) return fw_fail(FWHIP_ERR_INVALID, "NULL decoder");
    dd->cross_v_block = on != 0;
    return FWHIP_OK;
}

// FW_KV_F16 (kv_f16_enabled, nn.rs:5097-5109): the cache type of the states
// made after this call (1: f16, this library's initial setting; 0: f32, the
// reference's default)
extern "C" fwhip_status fwhip_decoder_set_kv_f16(fwhip_decoder *dd, int32_t on) {
    if (!dd) return fw_fail(FWHIP_ERR_INVALID, "NULL decoder");
    dd->kv_f16 = on != 0;
    return FWHIP_OK;
}

// DecoderState::new (decoder.rs:1040-1285) for every stream: the cross K/V
// projections written as per-head f16 K (scaled) and transposed f16 V, then
// per-row int8 copies for the default arm.  Exact mode: the strict
// sequential-k f32 GEMM, layer by layer; fast mode: every layer's K and V in
// one f16-pair MFMA GEMM over the states split into f16 (hi, lo) pairs.  A
// state past the f16 range (|v| >= 65520, which a pair cannot carry) sets the
// range flag, and the strict GEMM then replaces the fast one's results.
static bool cross_kv(fwhip_dstate *st, const float *enc_dev, bool strict) {
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    const int d = dd->d, H = dd->H, L = dd->L, T = st->T, S = st->S;
    const float kscale = powf(64.0f, -0.25f);
    fw_event_pair ev;
    if (strict) {
        for (int li = 0; li < L; li++) {
            const DecLayerDev &l = dd->layers[li];
            fw_timed_begin(c, FWHIP_K_DEC_GEMV, 2.0 * S * T * (double)d * d, &ev);
            fw_launch_gemm_strict(c->stream, enc_dev, l.ck16w, S * T, d, d, 1, nullptr, nullptr, kscale, st->ck16,
                                  T, H, L, li);
            fw_timed_end(c, &ev);
            fw_launch_gemm_strict(c->stream, enc_dev, l.cv16w, S * T, d, d, 2, nullptr, l.cv_b, 1.0f, st->cvt16, T,
                                  H, L, li);
        }
    } else {
        fw_ovf_clear(c);
        fw_launch_split_f16(c->stream, enc_dev, (size_t)S * T * d, st->ench, st->encl, c->ovf_dev);
        FwGemm g;
        memset(&g, 0, sizeof g);
        g.A = st->ench;
        g.A2 = st->encl;
        g.B = dd->ckv16;
        g.M = S * T;
        g.N = L * 2 * d;
        g.K = d;
        g.lda = d;
        g.ldb = d;
        g.bias = dd->ckv_b;
        g.epi = FW_EPI_XKV;
        g.ldc = d;
        g.o16[0] = st->ck16;
        g.o16[1] = st->cvt16;
        g.T = T;
        g.H = H;
        g.L = L;
        g.scale = kscale;
        fw_timed_begin(c, FWHIP_K_DEC_CROSS, 2.0 * 2.0 * S * T * (double)L * d * d, &ev);
        const bool ok = fw_launch_gemm(c->stream, FW_KIND_F16S, g);
        fw_timed_end(c, &ev);
        if (!ok) return false;
        fw_ovf_fetch(c);
    }
    if (st->ck16p)
        fw_launch_pack_cross_f16(c->stream, st->ck16, st->cvt16, st->ck16p, st->cvt16p, (size_t)S * L * H * T,
                                 (size_t)S * L * H * 64, T);
    if (dd->arm == FWHIP_DEC_INT8) {
        fw_launch_quant_f16_rows(c->stream, st->ck16, st->ck8, st->ck8s, S * L * H * T, 64);
        fw_launch_quant_f16_rows_ld(c->stream, st->cvt16, st->cvt8, st->cvt8s, S * L * H * 64, T, st->Tq);
        if (st->cvb8) fw_launch_quant_blocked(c->stream, st->cvt16, st->cvb8, st->cvbs, (int64_t)S * L * H * 64, T, 32,
                                              st->Tq);
    }
    return true;
}

extern "C" fwhip_status fwhip_dstate_set_cross(fwhip_dstate *st, const float *enc_dev) {
    if (!st || !enc_dev) return fw_fail(FWHIP_ERR_INVALID, "fwhip_dstate_set_cross: NULL argument");
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    HIP_TRY(hipSetDevice(c->device));
    if (!cross_kv(st, enc_dev, dd->exact)) return fw_fail(FWHIP_ERR_GENERIC, "cross K/V GEMM has no kernel");
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (!dd->exact && *c->ovf_host) {
        cross_kv(st, enc_dev, true);
        HIP_TRY(hipGetLastError());
        HIP_TRY(hipStreamSynchronize(c->stream));
    }
    st->len = 0;
    return FWHIP_OK;
}

static fwhip_status check_cancel(fwhip_ctx *c) {
    if (c->cancel.exchange(0)) return fw_fail(FWHIP_ERR_CANCELLED, "cancelled");
    return FWHIP_OK;
}

// int8 GEMV over every stream, 16 streams per launch (the MFMA tile height).
// xf (nullable): quantize the f32 rows xf inside the GEMV, with st->pmax
// holding the per-head maxima of those rows
static void gemv_i8_all(fwhip_dstate *st, hipStream_t s, const int8_t *W, const float *sw, const float *bias, float *y,
                        int N, int K, int ldy, int mode, const fwhip_filter *filt, const float *xf = nullptr) {
    const float *gt = st->dec->ctx->gelu_tab;
    const int H = st->dec->H;
    int nblk = fw_gemv_i8m_blocks(N);
    for (int s0 = 0; s0 < st->S; s0 += 16) {
        int n = st->S - s0 < 16 ? st->S - s0 : 16;
        fw_launch_gemv_i8m(s, W, sw, bias, st->xq + (size_t)s0 * K, st->xs + s0, y + (size_t)s0 * ldy, N, K, n, ldy,
                           mode, gt, filt, st->initial, mode == 3 ? st->keys + (size_t)s0 * nblk : nullptr,
                           xf ? xf + (size_t)s0 * K : nullptr, xf ? st->pmax + (size_t)s0 * H : nullptr, H);
    }
}
static bool gemv_blk_all(fwhip_dstate *st, hipStream_t s, const int8_t *W, const float *sc, const float *bias,
                         const float *x, float *y, int N, int K, int ldy) {
    return fw_launch_gemv_blk2(s, W, sc, bias, x, y, N, K, st->S, ldy, 1, st->dec->ctx->n_cu) == 0;
}

// One token row for every stream at the device-side position *st->pos
// (forward_step_hidden decoder.rs:1754-1906 + logits_last 2087-2147).  With
// want_logits the final LayerNorm, the logits and the per-block argmax keys
// over the filtered logits (filt may be NULL: raw argmax) are produced too.
// `timed` brackets the logits GEMV with events (never inside a graph capture).
static void dec_logits_f16(fwhip_dstate *st, const float *x, float *h, const fwhip_filter *filt, bool timed);
// Exact mode (dd->exact): every LayerNorm, wherever it is fused, sums its
// statistics in the reference's sequential order (the kernels' lnseq).
static fwhip_status dec_forward_row(fwhip_dstate *st, const int32_t *tok, bool prefill, bool want_logits,
                                    const fwhip_filter *filt, bool timed) {
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    hipStream_t s = c->stream;
    int d = dd->d, H = dd->H, L = dd->L, T = st->T, S = st->S, dff = dd->dff;
    bool i8 = dd->arm == FWHIP_DEC_INT8;
    float scale = powf(64.0f, -0.25f);
    const float *gt = c->gelu_tab;
    const int sq = dd->exact;
    // a one-token step times its fused cross-attention sublayer launches
    // (algorithmic bytes: the cohort's cross K/V of the layer and the q weights)
    const bool xt = timed && !prefill;
    fw_event_pair xev;
    xev.active = false;
    const double xbytes = i8 ? (double)S * (2.0 * T * d + 4.0 * H * T + 4.0 * d) + (double)d * d + 4.0 * d
                             : (double)S * 4.0 * T * d + 2.0 * d * d + 4.0 * d;
    // The f16 arm's projections fold into the attention kernels when the
    // cohort's (head, stream) blocks fill one round of the CUs: with fewer
    // streams a head's rows would be multiplied on that many CUs only (one
    // stream: 332 against 316 us per step), with more the second round costs
    // more than the two launches saved (16 streams: 611 against 606 us); 10
    // streams: 420 against 443 us.
    const bool fold = !i8 && S >= 4 && H * S <= c->n_cu;
    const bool sa_fold = fold && fw_self_attn_f16q_ok(d, H) && fw_gemv16_ok(3 * d, d) && fw_gemv16_lpr(3 * d, d) == 16;
    // embedding + layer 0's attention LayerNorm (the int8 arm, and the f16
    // arm's folded self-attention, form both inside layer 0's kernel)
    if (!i8 && !sa_fold)
        fw_launch_embed_ln(s, tok, st->pos, dd->emb16, dd->pos_emb, st->x, d, S, dd->layers[0].attn_ln_w,
                           dd->layers[0].attn_ln_b, st->h, nullptr, nullptr, 0, sq);
    for (int li = 0; li < L; li++) {
        const DecLayerDev &l = dd->layers[li];
        if (i8) {
            // (the cross LayerNorm runs inside the cross-attention kernel; the
            // GEMVs' 80-320 blocks would each redo a whole LayerNorm, which
            // measured slower than this one-wave-per-row kernel)
            // attention LayerNorm, q/k/v projection and attention in one kernel;
            // it writes per-head maxima; the o / co GEMVs quantize att themselves
            fw_launch_self_attn_fused(s, l.qkv8, l.qkv8s, l.qkv_b, st->x, l.attn_ln_w, l.attn_ln_b, st->kv_k,
                                      st->kv_v, st->att, st->pos, d, H, dd->nctx, L, li, S, scale, st->pmax,
                                      li == 0 ? tok : nullptr, li == 0 ? dd->emb16 : nullptr,
                                      li == 0 ? dd->pos_emb : nullptr, sq, st->kv32);
            gemv_i8_all(st, s, l.o8, l.o8s, l.o_b, st->x, d, d, d, 1, nullptr, st->att);
            // the cross LayerNorm and q projection run inside the cross-attention kernel
            if (xt) fw_timed_begin(c, FWHIP_K_DEC_XATTN, xbytes, &xev);
            fw_launch_cross_attn_i8v2(s, l.cq8, l.cq8s, l.cq_b, st->x, l.cross_ln_w, l.cross_ln_b, st->ck8, st->ck8s,
                                      st->cvb8 ? st->cvb8 : st->cvt8, st->cvt8s, st->att, d, T, st->Tq, H, L, li, S,
                                      scale, st->pmax, sq, st->cvbs);
            if (xt) fw_timed_end(c, &xev);
            gemv_i8_all(st, s, l.co8, l.co8s, l.co_b, st->x, d, d, d, 1, nullptr, st->att);
            // mode 4: GELU written block-interleaved for the block GEMV; prefill
            // rows take the f16 mlp_2 (the block-int8 arm has no batch form),
            // which reads natural order
            fw_launch_ln_quant(s, st->x, nullptr, l.mlp_ln_w, l.mlp_ln_b, d, S, st->xq, st->xs, sq);
            gemv_i8_all(st, s, l.fc1_8, l.fc1_8s, l.fc1_b, st->ff, dff, d, dff, prefill ? 2 : 4, nullptr);
            if (prefill) fw_gemv16(s, l.fc2_16, l.fc2_b, st->ff, st->x, d, dff, S, d, 1, gt);
            else if (!gemv_blk_all(st, s, l.fc2_b8, l.fc2_b8s, l.fc2_b, st->ff, st->x, d, dff, d))
                return fw_fail(FWHIP_ERR_INVALID, "block GEMV: unsupported mlp width");
        } else {
            if (sa_fold) {
                // the LayerNorm, q/k/v projection and attention in one kernel
                // (layer 0: the embedding too)
                if (li > 0)
                    fw_launch_self_attn_f16q(s, l.qkv16, l.qkv_b, st->x, l.attn_ln_w, l.attn_ln_b, st->kv_k,
                                             st->kv_v, st->att, st->pos, H, dd->nctx, L, li, S, scale, nullptr,
                                             nullptr, nullptr, nullptr, sq, st->kv32);
                else
                    fw_launch_self_attn_f16q(s, l.qkv16, l.qkv_b, nullptr, l.attn_ln_w, l.attn_ln_b, st->kv_k,
                                             st->kv_v, st->att, st->pos, H, dd->nctx, L, li, S, scale, tok,
                                             dd->emb16, dd->pos_emb, st->x, sq, st->kv32);
            } else {
                // (layer 0's attention LayerNorm ran with the embedding, into h)
                if (li > 0)
                    fw_gemv16_ln(s, l.qkv16, l.qkv_b, st->x, st->h, l.attn_ln_w, l.attn_ln_b, st->qkv, 3 * d, d, S,
                                 3 * d, 0, gt, sq);
                else
                    fw_gemv16(s, l.qkv16, l.qkv_b, st->h, st->qkv, 3 * d, d, S, 3 * d, 0, gt);
                fw_launch_self_attn2(s, st->qkv, st->kv_k, st->kv_v, st->att, st->pos, d, H, dd->nctx, L, li, S,
                                     scale, nullptr, 0, 1, st->kv32);
            }
            fw_gemv16(s, l.o16, l.o_b, st->att, st->x, d, d, S, d, 1, gt);
            if (fold && st->ck16p && fw_cross_f16pq_ok(d, T, H) && fw_gemv16_ok(d, d) && fw_gemv16_lpr(d, d) == 16) {
                // the cross LayerNorm and q projection run inside the cross-attention kernel
                if (xt) fw_timed_begin(c, FWHIP_K_DEC_XATTN, xbytes, &xev);
                fw_launch_cross_attn_f16pq(s, l.cq16, l.cq_b, st->x, l.cross_ln_w, l.cross_ln_b, st->ck16p,
                                           st->cvt16p, st->att, d, T, H, L, li, S, scale, sq);
                if (xt) fw_timed_end(c, &xev);
            } else {
                // a cohort whose (head, stream) blocks fill under half the CUs
                // (one stream: 20 blocks for 1,500 keys) or need more than one
                // round of them (16 streams: 320 blocks; 591 against 606 us per
                // step) spreads each head over more blocks in two launches; under
                // half, the scores launch also forms the LayerNorm and q rows
                const long long hs = (long long)S * H;
                const bool xsplit = st->ck16p && (hs * 2 <= c->n_cu || hs > c->n_cu);
                if (xsplit && hs * 2 <= c->n_cu && fw_cross_f16pq_ok(d, T, H) && fw_gemv16_ok(d, d) &&
                    fw_gemv16_lpr(d, d) == 16) {
                    fw_launch_cross_attn_f16pq_split(s, l.cq16, l.cq_b, st->x, l.cross_ln_w, l.cross_ln_b, st->ck16p,
                                                     st->cvt16p, st->att, d, T, H, L, li, S, scale, st->xsplit, sq);
                } else {
                    fw_gemv16_ln(s, l.cq16, l.cq_b, st->x, st->h, l.cross_ln_w, l.cross_ln_b, st->y, d, d, S, d, 0,
                                 gt, sq);
                    if (xsplit)
                        fw_launch_cross_attn_f16p_split(s, st->y, st->ck16p, st->cvt16p, st->att, d, T, H, L, li, S,
                                                        scale, st->xsplit);
                    else if (st->ck16p)
                        fw_launch_cross_attn_f16p(s, st->y, st->ck16p, st->cvt16p, st->att, d, T, H, L, li, S, scale);
                    else fw_launch_cross_attn_f16(s, st->y, st->ck16, st->cvt16, st->att, d, T, H, L, li, S, scale);
                }
            }
            fw_gemv16(s, l.co16, l.co_b, st->att, st->x, d, d, S, d, 1, gt);
            fw_gemv16_ln(s, l.fc1_16, l.fc1_b, st->x, st->h, l.mlp_ln_w, l.mlp_ln_b, st->ff, dff, d, S, dff, 2, gt,
                         sq);
            fw_gemv16(s, l.fc2_16, l.fc2_b, st->ff, st->x, d, dff, S, d, 1, gt);
        }
    }
    if (want_logits) {
        fw_event_pair ev;
        ev.active = false;
        if (i8) {
            fw_launch_ln_quant(s, st->x, nullptr, dd->ln_w, dd->ln_b, d, S, st->xq, st->xs, sq);
            if (timed) fw_timed_begin(c, FWHIP_K_DEC_LOGITS, (double)dd->V * d, &ev);
            gemv_i8_all(st, s, dd->emb8, dd->emb8s, nullptr, st->logits, dd->V, d, dd->V, 3, filt);
            if (timed) fw_timed_end(c, &ev);
        } else {
            dec_logits_f16(st, st->x, st->h, filt, timed);
        }
    }
    return FWHIP_OK;
}

// The f16 arm's final LayerNorm and tied logits head of the S rows x (h:
// LayerNorm scratch), with the per-tile argmax keys of the filtered rows.
static void dec_logits_f16(fwhip_dstate *st, const float *x, float *h, const fwhip_filter *filt, bool timed) {
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    hipStream_t s = c->stream;
    const int d = dd->d, S = st->S;
    const float *gt = c->gelu_tab;
    fw_event_pair ev;
    ev.active = false;
    if (timed) fw_timed_begin(c, FWHIP_K_DEC_LOGITS, (double)dd->V * d * 2.0, &ev);
    if (f16_fused_keys(dd)) {
        // final LayerNorm, tied f16 logits head and per-tile argmax keys in one
        // kernel (exact mode: the LayerNorm as a pass of its own, as fw_gemv16_ln)
        if (dd->exact) {
            fw_launch_ln_quant(s, x, h, dd->ln_w, dd->ln_b, d, S, nullptr, nullptr, 1);
            fw_launch_gemv16(s, dd->emb16f, nullptr, h, st->logits, dd->V, d, S, dd->V, 0, gt, nullptr, nullptr, filt,
                             st->initial, st->keys);
        } else {
            fw_launch_gemv16(s, dd->emb16f, nullptr, x, st->logits, dd->V, d, S, dd->V, 0, gt, dd->ln_w, dd->ln_b,
                             filt, st->initial, st->keys);
        }
        if (timed) fw_timed_end(c, &ev);
    } else {
        fw_gemv16_ln(s, dd->emb16f, nullptr, x, h, dd->ln_w, dd->ln_b, st->logits, dd->V, d, S, dd->V, 0, gt,
                     dd->exact);
        if (timed) fw_timed_end(c, &ev);
        fw_launch_logits_keys(s, st->logits, dd->V, S, filt, st->initial, st->keys);
    }
}

// Batched prompt prefill (f16 arm): the rows of PF_CHUNK positions of every
// stream go through each layer together, [position][stream] order, row r at
// stream r % S and position *pos + r / S.  Every projection is row-local
// (gemv_f16 per row), so a batch gives each row the bits of its own forward;
// the self attention appends every row's k/v first and then lets row r see
// positions [0, *pos + r / S] of its stream, exactly the keys the row-by-row
// forward gives it (decoder.rs:1754-1906).
#define PF_CHUNK 32
static bool prefill_batch_ok(const fwhip_dstate *st) {
    const fwhip_decoder *dd = st->dec;
    return dd->arm == FWHIP_DEC_F16 && st->ck16p && fw_cross_f16p_ok(st->T) && dd->d == dd->H * 64 &&
           fw_gemv16_ok(3 * dd->d, dd->d) && fw_gemv16_ok(dd->d, dd->d) && fw_gemv16_ok(dd->dff, dd->d) &&
           fw_gemv16_ok(dd->d, dd->dff);
}
static fwhip_status prefill_buffers(fwhip_dstate *st) {
    if (st->pf_x) return FWHIP_OK;
    const fwhip_decoder *dd = st->dec;
    const size_t R = (size_t)st->S * PF_CHUNK, d = dd->d;
    st->pf_x = (float *)fw_dalloc(st->pf_owned, sizeof(float) * R * d);
    st->pf_h = (float *)fw_dalloc(st->pf_owned, sizeof(float) * R * dd->dff);
    st->pf_qkv = (float *)fw_dalloc(st->pf_owned, sizeof(float) * R * 3 * d);
    st->pf_att = (float *)fw_dalloc(st->pf_owned, sizeof(float) * R * d);
    st->pf_y = (float *)fw_dalloc(st->pf_owned, sizeof(float) * R * d);
    st->pf_ff = (float *)fw_dalloc(st->pf_owned, sizeof(float) * R * dd->dff);
    if (!st->pf_x || !st->pf_h || !st->pf_qkv || !st->pf_att || !st->pf_y || !st->pf_ff) {
        fw_free_all(st->pf_owned);
        st->pf_x = nullptr;
        return fw_fail(FWHIP_ERR_GENERIC, "prefill: device allocation failed");
    }
    return FWHIP_OK;
}
static fwhip_status dec_forward_chunk(fwhip_dstate *st, const int32_t *tok, int n_pos, bool want_logits,
                                      const fwhip_filter *filt, bool timed) {
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    hipStream_t s = c->stream;
    const int d = dd->d, H = dd->H, L = dd->L, T = st->T, S = st->S, dff = dd->dff, R = S * n_pos;
    const float scale = powf(64.0f, -0.25f);
    const float *gt = c->gelu_tab;
    float *x = st->pf_x, *h = st->pf_h, *qkv = st->pf_qkv, *att = st->pf_att, *y = st->pf_y, *ff = st->pf_ff;
    const int sq = dd->exact;
    fw_launch_embed_ln(s, tok, st->pos, dd->emb16, dd->pos_emb, x, d, R, dd->layers[0].attn_ln_w,
                       dd->layers[0].attn_ln_b, h, nullptr, nullptr, S, sq);
    for (int li = 0; li < L; li++) {
        const DecLayerDev &l = dd->layers[li];
        if (li > 0)
            fw_gemv16_ln(s, l.qkv16, l.qkv_b, x, h, l.attn_ln_w, l.attn_ln_b, qkv, 3 * d, d, R, 3 * d, 0, gt, sq);
        else fw_gemv16(s, l.qkv16, l.qkv_b, h, qkv, 3 * d, d, R, 3 * d, 0, gt);
        fw_launch_kv_append(s, qkv, st->kv_k, st->kv_v, st->pos, d, dd->nctx, L, li, S, R, st->kv32);
        fw_launch_self_attn2(s, qkv, st->kv_k, st->kv_v, att, st->pos, d, H, dd->nctx, L, li, S, scale, nullptr, R,
                             0, st->kv32);
        fw_gemv16(s, l.o16, l.o_b, att, x, d, d, R, d, 1, gt);
        fw_gemv16_ln(s, l.cq16, l.cq_b, x, h, l.cross_ln_w, l.cross_ln_b, y, d, d, R, d, 0, gt, sq);
        fw_launch_cross_attn_f16p(s, y, st->ck16p, st->cvt16p, att, d, T, H, L, li, S, scale, R);
        fw_gemv16(s, l.co16, l.co_b, att, x, d, d, R, d, 1, gt);
        fw_gemv16_ln(s, l.fc1_16, l.fc1_b, x, h, l.mlp_ln_w, l.mlp_ln_b, ff, dff, d, R, dff, 2, gt, sq);
        fw_gemv16(s, l.fc2_16, l.fc2_b, ff, x, d, dff, R, d, 1, gt);
    }
    // the last position's rows of every stream
    if (want_logits) dec_logits_f16(st, x + (size_t)(n_pos - 1) * S * d, h, filt, timed);
    return FWHIP_OK;
}

// Host values are staged with a synchronous copy ordered after the queued work,
// so no host buffer is read after the call returns.
static fwhip_status set_dev_ints(fwhip_ctx *c, int *dst, const int *v, int n) {
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipMemcpy(dst, v, sizeof(int) * n, hipMemcpyHostToDevice));
    return FWHIP_OK;
}

// Run `tq` token rows ([S, tq] host tokens) through the decoder for every
// stream: the token matrix is uploaded once (position-major) and each row reads
// its column; the device position starts at st->len and advances between rows.
// The last row produces the logits and argmax keys.
static double dec_step_bytes(const fwhip_dstate *st, int tk);

// Forward of tq rows per stream from position st->len.  With `ev` (tq == 1,
// the step in isolation) the forward is bracketed as a FWHIP_K_DEC_STEP launch
// from its first kernel; the caller ends the pair.
static fwhip_status stage_rows(fwhip_dstate *st, const int32_t *tokens, int tq, const fwhip_filter *filt,
                               fw_event_pair *ev = nullptr) {
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    int S = st->S;
    std::vector<int32_t> pm((size_t)S * tq);
    for (int t = 0; t < tq; t++)
        for (int s = 0; s < S; s++) pm[(size_t)t * S + s] = tokens[(size_t)s * tq + t];
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipMemcpy(st->rows, pm.data(), sizeof(int32_t) * pm.size(), hipMemcpyHostToDevice));
    int p0 = st->len;
    fwhip_status r = set_dev_ints(c, st->pos, &p0, 1);
    if (r != FWHIP_OK) return r;
    if (tq > 1 && prefill_batch_ok(st)) {
        r = prefill_buffers(st);
        if (r != FWHIP_OK) return r;
        for (int c0 = 0; c0 < tq; c0 += PF_CHUNK) {
            const int n = tq - c0 < PF_CHUNK ? tq - c0 : PF_CHUNK, p = p0 + c0;
            r = set_dev_ints(c, st->pos, &p, 1);
            if (r != FWHIP_OK) return r;
            r = dec_forward_chunk(st, st->rows + (size_t)c0 * S, n, c0 + n == tq, filt, true);
            if (r != FWHIP_OK) return r;
            r = check_cancel(c);
            if (r != FWHIP_OK) {
                hipStreamSynchronize(c->stream);
                return r;
            }
        }
        // the position of the last row, where the row-by-row forward leaves it
        const int pl = p0 + tq - 1;
        r = set_dev_ints(c, st->pos, &pl, 1);
        if (r != FWHIP_OK) return r;
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, std::string("launch failed: ") + hipGetErrorString(e));
        return FWHIP_OK;
    }
    for (int t = 0; t < tq; t++) {
        if (ev && tq == 1) fw_timed_begin(c, FWHIP_K_DEC_STEP, dec_step_bytes(st, p0 + 1), ev);
        r = dec_forward_row(st, st->rows + (size_t)t * S, tq > 1, t == tq - 1, filt, true);
        if (r != FWHIP_OK) return r;
        if (t + 1 < tq) fw_launch_step_bookkeeping(c->stream, st->pos, nullptr, st->rows, nullptr, 0, 0, S);
        r = check_cancel(c);
        if (r != FWHIP_OK) {
            hipStreamSynchronize(c->stream);
            return r;
        }
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fw_fail(FWHIP_ERR_GENERIC, std::string("launch failed: ") + hipGetErrorString(e));
    return FWHIP_OK;
}

extern "C" fwhip_status fwhip_decoder_step(fwhip_dstate *st, const int32_t *tokens, int32_t tq, float *logits_dev,
                                           int32_t *argmax_host, const fwhip_filter *filter, int32_t initial) {
    if (!st || !tokens) return fw_fail(FWHIP_ERR_INVALID, "fwhip_decoder_step: NULL argument");
    if (tq <= 0) return fw_fail(FWHIP_ERR_INVALID, "forward_step: empty token batch");
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    HIP_TRY(hipSetDevice(c->device));
    int S = st->S;
    for (int i = 0; i < S * tq; i++)
        if (tokens[i] < 0 || tokens[i] >= dd->V)
            return fw_fail(FWHIP_ERR_INVALID, "token id " + std::to_string(tokens[i]) + " out of range");
    if (st->len + tq > dd->nctx)
        return fw_fail(FWHIP_ERR_INVALID, "decode position " + std::to_string(st->len + tq - 1) +
                                              " >= n_text_ctx " + std::to_string(dd->nctx));
    int init = initial ? 1 : 0;
    fwhip_status r = set_dev_ints(c, st->initial, &init, 1);
    if (r != FWHIP_OK) return r;
    // a one-token step (forward, logits, argmax) is timed as FWHIP_K_DEC_STEP
    fw_event_pair ev;
    ev.active = false;
    r = stage_rows(st, tokens, tq, filter, &ev);
    if (r != FWHIP_OK) {
        fw_timed_end(c, &ev);
        return r;
    }
    st->len += tq;
    if (argmax_host)
        fw_launch_argmax_finish(c->stream, st->keys, st->nkeys, S, st->tok, nullptr, 0, st->pos, nullptr, nullptr, 0);
    fw_timed_end(c, &ev);
    if (logits_dev)
        HIP_TRY(hipMemcpyAsync(logits_dev, st->logits, sizeof(float) * (size_t)S * dd->V, hipMemcpyDeviceToDevice,
                               c->stream));
    if (argmax_host)
        HIP_TRY(hipMemcpyAsync(argmax_host, st->tok, sizeof(int32_t) * S, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipGetLastError());
    return FWHIP_OK;
}

// The sampling step after the first: forward of the sampled tokens st->tok,
// logits + argmax keys, then argmax + bookkeeping on the device.
static fwhip_status greedy_step(fwhip_dstate *st, const fwhip_filter *filt, bool timed) {
    fwhip_status r = dec_forward_row(st, st->tok, false, true, filt, timed);
    if (r != FWHIP_OK) return r;
    fw_launch_argmax_finish(st->dec->ctx->stream, st->keys, st->nkeys, st->S, st->tok, st->hist, st->hist_cap, st->pos,
                            st->initial, st->stepc, 1, st->am_cnt);
    return FWHIP_OK;
}

// Capture greedy_step into a HIP graph (its kernels read the position, the
// sampled tokens and the step counter from device memory, so one capture
// replays for every step of this state).  Returns false when capture is
// unavailable; the loop then launches the same kernels directly.
static bool capture_step_impl(fwhip_dstate *st, const fwhip_filter *filt);
// Graph capture is skipped under a profiler that intercepts the HIP runtime
// (rocprofv3 preloads librocprofiler-sdk-tool): a kernel trace of replayed
// graphs has ended in a SIGSEGV inside the runtime's graph launch path, so
// profiled runs launch the same kernels directly.
static bool profiler_preloaded() {
    const char *p = getenv("LD_PRELOAD");
    return p && strstr(p, "rocprofiler-sdk") != nullptr;
}
static bool capture_step(fwhip_dstate *st, const fwhip_filter *filt) {
    static int disabled = -1, debug = -1;
    if (disabled < 0) disabled = getenv("FWHIP_NO_GRAPH") != nullptr || profiler_preloaded();
    if (debug < 0) debug = getenv("FWHIP_DEBUG") != nullptr;
    if (disabled) return false;
    bool ok = capture_step_impl(st, filt);
    if (debug) fprintf(stderr, "fwhip: greedy step graph %s\n", ok ? "captured" : "unavailable (direct launches)");
    return ok;
}
static bool capture_step_impl(fwhip_dstate *st, const fwhip_filter *filt) {
    if (st->graph && !memcmp(&st->graph_filter, filt, sizeof *filt) && st->graph_lnseq == st->dec->exact)
        return true;
    if (st->graph) {
        hipGraphExecDestroy(st->graph);
        st->graph = nullptr;
    }
    hipStream_t s = st->dec->ctx->stream;
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return false;
    greedy_step(st, filt, false);
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture(s, &g) != hipSuccess || !g) {
        (void)hipGetLastError();
        return false;
    }
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    st->graph = ge;
    st->graph_filter = *filt;
    st->graph_lnseq = st->dec->exact;
    return true;
}

// Algorithmic HBM bytes of one sampled decoder step of every stream at cache
// length tk: the weights once (int8 rows + f32 row scales, mlp_2 as 32-blocks
// with an f32 scale each, or f16), and per stream its cross K/V (int8 + scales,
// or f16) and self-attention cache (K and V rows [0, tk) read, one row each
// written, f16 or f32).
static double dec_step_bytes(const fwhip_dstate *st, int tk) {
    const fwhip_decoder *dd = st->dec;
    const double d = dd->d, L = dd->L, V = dd->V, T = st->T, S = st->S, H = dd->H;
    double w, cross;
    if (dd->arm == FWHIP_DEC_INT8) {
        w = L * (3 * d * d + 3 * d * d + 4 * d * d + 4 * (3 * d + d + d + d + 4 * d) + 4 * d * d * (1.0 + 4.0 / 32.0)) +
            V * d + 4 * V;
        cross = L * (2 * T * d + 4 * H * T + 4 * d);
    } else {
        // per layer: self q/k/v (3 d^2), o, cross q, cross o (3 d^2), fc1 and
        // fc2 (8 d^2), f16; the tied head V x d
        w = 2.0 * (L * 14 * d * d + V * d);
        cross = L * 2 * T * d * 2;
    }
    const double kv = L * 2 * ((double)tk + 1) * d * (st->kv32 ? 4 : 2);
    return w + S * (cross + kv);
}

// Greedy no-timestamps loop (decode.rs:3429-3566): prefill the prompt, then
// argmax -> step.  Sampled tokens, the position and the step count live on the
// device; each step after the first replays one captured graph; the host polls
// for end-of-text every few steps, so steps stream without a per-token sync.
// The pinned poll buffer of a state, at least n int32 (a poll copies a few
// hundred bytes; pageable copies cost ~100 us of idle GPU each).
static int32_t *poll_buffer(fwhip_dstate *st, int n) {
    if (st->poll_cap < n) {
        if (st->poll_host) {
            hipStreamSynchronize(st->dec->ctx->stream);
            hipHostFree(st->poll_host);
            st->poll_host = nullptr;
            st->poll_cap = 0;
        }
        if (hipHostMalloc((void **)&st->poll_host, sizeof(int32_t) * (size_t)n, hipHostMallocDefault) != hipSuccess) {
            st->poll_host = nullptr;
            return nullptr;
        }
        st->poll_cap = n;
    }
    return st->poll_host;
}

extern "C" fwhip_status fwhip_decode_greedy(fwhip_dstate *st, const int32_t *prompt, int32_t n_prompt,
                                            int32_t n_max, const fwhip_filter *filter, int32_t *out_tokens,
                                            int32_t *out_len) {
    if (!st || !prompt || !filter || !out_tokens || !out_len)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_decode_greedy: NULL argument");
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    HIP_TRY(hipSetDevice(c->device));
    int S = st->S;
    if (n_prompt <= 0 || n_max <= 0) return fw_fail(FWHIP_ERR_INVALID, "empty prompt or n_max <= 0");
    if (st->len + n_prompt + n_max - 1 > dd->nctx)
        return fw_fail(FWHIP_ERR_INVALID, "prompt + n_max exceeds n_text_ctx");
    if (n_max > st->hist_cap) return fw_fail(FWHIP_ERR_INVALID, "n_max exceeds n_text_ctx");
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= dd->V) return fw_fail(FWHIP_ERR_INVALID, "prompt token out of range");
    std::vector<int32_t> rows((size_t)S * n_prompt);
    for (int s = 0; s < S; s++)
        for (int t = 0; t < n_prompt; t++) rows[(size_t)s * n_prompt + t] = prompt[t];
    const int init[2] = {1, 0}; // initial = 1, step counter = 0
    fwhip_status r = set_dev_ints(c, st->initial, init, 2);
    if (r != FWHIP_OK) return r;
    r = stage_rows(st, rows.data(), n_prompt, filter);
    if (r != FWHIP_OK) return r;
    // first sampled token: from the prefill's logits
    fw_launch_argmax_finish(c->stream, st->keys, st->nkeys, S, st->tok, st->hist, st->hist_cap, st->pos, st->initial,
                            st->stepc, 1, st->am_cnt);
    std::vector<int32_t> hist((size_t)S * n_max, -1);
    int steps = 1;
    const int poll = 8;
    // each poll copies the history's newest `poll` columns into pinned memory
    // and keeps which streams have produced end-of-text so far
    int32_t *ph = poll_buffer(st, S * poll);
    if (!ph) return fw_fail(FWHIP_ERR_GENERIC, "pinned poll buffer");
    std::vector<uint8_t> done(S, 0);
    int polled = 0; // history columns already examined
    bool use_graph = n_max > 1 && capture_step(st, filter);
    for (int i = 1; i < n_max; i++) {
        r = check_cancel(c);
        if (r != FWHIP_OK) {
            hipStreamSynchronize(c->stream);
            st->len += n_prompt + steps - 1;
            return r;
        }
        fw_event_pair ev;
        fw_timed_begin(c, FWHIP_K_DEC_STEP, dec_step_bytes(st, st->len + n_prompt + i), &ev);
        if (use_graph) HIP_TRY(hipGraphLaunch(st->graph, c->stream));
        else {
            r = greedy_step(st, filter, false);
            if (r != FWHIP_OK) return r;
        }
        fw_timed_end(c, &ev);
        steps = i + 1;
        if (steps % poll == 0 && steps < n_max) {
            const int nc = steps - polled; // <= poll
            HIP_TRY(hipMemcpy2DAsync(ph, sizeof(int32_t) * poll, st->hist + polled, sizeof(int32_t) * st->hist_cap,
                                     sizeof(int32_t) * nc, S, hipMemcpyDeviceToHost, c->stream));
            HIP_TRY(hipStreamSynchronize(c->stream));
            bool all = true;
            for (int s = 0; s < S; s++) {
                for (int k = 0; k < nc && !done[s]; k++)
                    if (ph[(size_t)s * poll + k] == filter->eot) done[s] = 1;
                all = all && done[s];
            }
            polled = steps;
            if (all) break;
        }
    }
    HIP_TRY(hipMemcpy2DAsync(hist.data(), sizeof(int32_t) * n_max, st->hist, sizeof(int32_t) * st->hist_cap,
                             sizeof(int32_t) * steps, S, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipGetLastError());
    for (int s = 0; s < S; s++) {
        int n = steps;
        for (int k = 0; k < steps; k++)
            if (hist[(size_t)s * n_max + k] == filter->eot) {
                n = k + 1;
                break;
            }
        out_len[s] = n;
        for (int k = 0; k < n_max; k++) out_tokens[(size_t)s * n_max + k] = k < n ? hist[(size_t)s * n_max + k] : 0;
    }
    st->len += n_prompt + steps - 1;
    return FWHIP_OK;
}

// ---------------------------------------------------------------------------
// The window loop on the device (decode.rs:3429-3566 with the full
// process_logits): prefill, then per step the forward of the sampled tokens,
// the logits and k_win_select (filter, forcing rule, argmax, the loop state);
// the host only polls for every stream being done.

static fwhip_status win_buffers(fwhip_dstate *st, int n_max) {
    const fwhip_decoder *dd = st->dec;
    const int ldr = ((dd->V + 63) / 64) * 64;
    if (st->w_nmax >= n_max && st->w_ldr == ldr) return FWHIP_OK;
    HIP_TRY(hipStreamSynchronize(dd->ctx->stream));
    fw_free_all(st->w_owned);
    const size_t S = st->S;
    st->w_rows = (float *)fw_dalloc(st->w_owned, sizeof(float) * S * n_max * ldr);
    st->w_nsrow = (float *)fw_dalloc(st->w_owned, sizeof(float) * S * ldr);
    st->w_scratch = (float *)fw_dalloc(st->w_owned, sizeof(float) * S * ldr);
    st->w_plogs = (float *)fw_dalloc(st->w_owned, sizeof(float) * S * n_max);
    st->w_nslp = (float *)fw_dalloc(st->w_owned, sizeof(float) * S);
    st->w_ws = (FwWinStream *)fw_dalloc(st->w_owned, sizeof(FwWinStream) * S);
    st->w_forced = (uint8_t *)fw_dalloc(st->w_owned, S * n_max);
    st->w_ndone = (int *)fw_dalloc(st->w_owned, sizeof(int));
    st->w_part = (FwWinPart *)fw_dalloc(st->w_owned, sizeof(FwWinPart) * S * WIN_NB);
    st->w_cnt = (int *)fw_dalloc(st->w_owned, sizeof(int) * S);
    if (!st->w_rows || !st->w_nsrow || !st->w_scratch || !st->w_plogs || !st->w_nslp || !st->w_ws || !st->w_forced ||
        !st->w_ndone || !st->w_part || !st->w_cnt) {
        fw_free_all(st->w_owned);
        st->w_nmax = 0;
        return fw_fail(FWHIP_ERR_GENERIC, "fwhip_decode_window: device allocation failed");
    }
    HIP_TRY(hipMemsetAsync(st->w_cnt, 0, sizeof(int) * S, dd->ctx->stream)); // (outside any capture)
    st->w_nmax = n_max;
    st->w_ldr = ldr;
    if (st->wgraph) {
        hipGraphExecDestroy(st->wgraph);
        st->wgraph = nullptr;
    }
    return FWHIP_OK;
}

static fwhip_status win_step(fwhip_dstate *st, const FwWinCfg &cfg) {
    fwhip_status r = dec_forward_row(st, st->tok, false, true, nullptr, false);
    if (r != FWHIP_OK) return r;
    fw_launch_win_select(st->dec->ctx->stream, st->logits, st->dec->V, cfg, st->w_ws, st->hist, st->hist_cap,
                         st->w_rows, st->w_forced, st->w_scratch, st->tok, st->pos, st->w_ndone, st->w_part, st->w_cnt,
                         st->S);
    return FWHIP_OK;
}

static bool win_capture(fwhip_dstate *st, const FwWinCfg &cfg) {
    static int disabled = -1;
    if (disabled < 0) disabled = getenv("FWHIP_NO_GRAPH") != nullptr || profiler_preloaded();
    if (disabled) return false;
    if (st->wgraph && !memcmp(&st->wgraph_cfg, &cfg, sizeof cfg) && st->wgraph_lnseq == st->dec->exact) return true;
    if (st->wgraph) {
        hipGraphExecDestroy(st->wgraph);
        st->wgraph = nullptr;
    }
    hipStream_t s = st->dec->ctx->stream;
    if (hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal) != hipSuccess) return false;
    win_step(st, cfg);
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture(s, &g) != hipSuccess || !g) {
        (void)hipGetLastError();
        return false;
    }
    hipGraphExec_t ge = nullptr;
    hipError_t e = hipGraphInstantiate(&ge, g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    st->wgraph = ge;
    st->wgraph_cfg = cfg;
    st->wgraph_lnseq = st->dec->exact;
    return true;
}

extern "C" fwhip_status fwhip_decode_window(fwhip_dstate *st, const int32_t *prompt, int32_t n_prompt,
                                            const fwhip_filter *filter, const fwhip_window_cfg *wc,
                                            fwhip_window_stream *streams, int32_t *out_tokens, float *out_plogs) {
    if (!st || !prompt || !filter || !wc || !streams || !out_tokens || !out_plogs)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_decode_window: NULL argument");
    fwhip_decoder *dd = st->dec;
    fwhip_ctx *c = dd->ctx;
    HIP_TRY(hipSetDevice(c->device));
    const int S = st->S, n_max = wc->n_max;
    if (n_prompt <= 0 || n_max <= 0) return fw_fail(FWHIP_ERR_INVALID, "empty prompt or n_max <= 0");
    if (st->len + n_prompt + n_max - 1 > dd->nctx) return fw_fail(FWHIP_ERR_INVALID, "prompt + n_max exceeds n_text_ctx");
    if (n_max > st->hist_cap) return fw_fail(FWHIP_ERR_INVALID, "n_max exceeds n_text_ctx");
    for (int i = 0; i < n_prompt; i++)
        if (prompt[i] < 0 || prompt[i] >= dd->V) return fw_fail(FWHIP_ERR_INVALID, "prompt token out of range");
    if (filter->timestamp_begin <= 0 || filter->timestamp_begin > dd->V || dd->V - filter->timestamp_begin > WIN_MAXTS ||
        filter->eot <= 0 || filter->eot > filter->timestamp_begin)
        return fw_fail(FWHIP_ERR_UNSUPPORTED, "fwhip_decode_window: the vocabulary's timestamp range is not supported");
    if (!fw_win_select_ok(dd->V))
        return fw_fail(FWHIP_ERR_UNSUPPORTED, "fwhip_decode_window: vocabulary larger than the select kernel covers");
    fwhip_status r = win_buffers(st, n_max);
    if (r != FWHIP_OK) return r;
    FwWinCfg cfg;
    memset(&cfg, 0, sizeof cfg);
    cfg.V = dd->V;
    cfg.beg = filter->timestamp_begin;
    cfg.eot = filter->eot;
    cfg.sot = filter->sot;
    cfg.sot_prev = filter->sot_prev;
    cfg.solm = filter->solm;
    cfg.no_speech = filter->no_speech;
    cfg.no_ts = filter->no_timestamps;
    cfg.translate = filter->translate;
    cfg.transcribe = filter->transcribe;
    cfg.space = filter->space_token;
    cfg.n_lang = filter->n_languages;
    cfg.timestamps = wc->timestamps ? 1 : 0;
    cfg.max_initial_tid = wc->max_initial_tid;
    cfg.max_tokens = wc->max_tokens > 0 ? (wc->max_tokens < n_max ? wc->max_tokens : n_max) : 0;
    cfg.n_max = n_max;
    cfg.exact = wc->exact ? 1 : 0;
    cfg.ldr = st->w_ldr;
    std::vector<FwWinStream> ws(S);
    for (int s = 0; s < S; s++) {
        memset(&ws[s], 0, sizeof ws[s]);
        ws[s].seek_cs = streams[s].seek_cs;
        ws[s].seek_end_cs = streams[s].seek_end_cs;
        ws[s].has_prior = streams[s].has_prior_segments ? 1 : 0;
        ws[s].seek_delta_cs = 3000;
    }
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipMemcpy(st->w_ws, ws.data(), sizeof(FwWinStream) * S, hipMemcpyHostToDevice));
    HIP_TRY(hipMemsetAsync(st->w_ndone, 0, sizeof(int), c->stream));
    std::vector<int32_t> rows((size_t)S * n_prompt);
    for (int s = 0; s < S; s++)
        for (int t = 0; t < n_prompt; t++) rows[(size_t)s * n_prompt + t] = prompt[t];
    r = stage_rows(st, rows.data(), n_prompt, nullptr);
    if (r != FWHIP_OK) return r;
    HIP_TRY(hipMemcpy2DAsync(st->w_nsrow, sizeof(float) * cfg.ldr, st->logits, sizeof(float) * dd->V,
                             sizeof(float) * dd->V, S, hipMemcpyDeviceToDevice, c->stream));
    fw_launch_win_select(c->stream, st->logits, dd->V, cfg, st->w_ws, st->hist, st->hist_cap, st->w_rows,
                         st->w_forced, st->w_scratch, st->tok, st->pos, st->w_ndone, st->w_part, st->w_cnt, S);
    int steps = 1;
    const int poll = 8;
    int32_t *pnd = poll_buffer(st, 1); // the done count, copied to pinned memory
    if (!pnd) return fw_fail(FWHIP_ERR_GENERIC, "pinned poll buffer");
    bool use_graph = n_max > 1 && win_capture(st, cfg);
    for (int i = 1; i < n_max; i++) {
        if (i % poll == 1 || poll == 1) {
            HIP_TRY(hipMemcpyAsync(pnd, st->w_ndone, sizeof(int), hipMemcpyDeviceToHost, c->stream));
            HIP_TRY(hipStreamSynchronize(c->stream));
            if (*pnd >= S) break;
        }
        r = check_cancel(c);
        if (r != FWHIP_OK) {
            hipStreamSynchronize(c->stream);
            st->len += n_prompt + steps - 1;
            return r;
        }
        fw_event_pair ev;
        fw_timed_begin(c, FWHIP_K_DEC_STEP, dec_step_bytes(st, st->len + n_prompt + i), &ev);
        if (use_graph) HIP_TRY(hipGraphLaunch(st->wgraph, c->stream));
        else {
            r = win_step(st, cfg);
            if (r != FWHIP_OK) return r;
        }
        fw_timed_end(c, &ev);
        steps = i + 1;
    }
    fw_launch_win_plogs(c->stream, st->w_rows, st->w_nsrow, cfg, st->w_ws, st->hist, st->hist_cap, st->w_forced,
                        st->w_plogs, st->w_nslp, S);
    std::vector<int32_t> hist((size_t)S * n_max);
    std::vector<float> nslp(S);
    HIP_TRY(hipMemcpyAsync(ws.data(), st->w_ws, sizeof(FwWinStream) * S, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipMemcpy2DAsync(hist.data(), sizeof(int32_t) * n_max, st->hist, sizeof(int32_t) * st->hist_cap,
                             sizeof(int32_t) * n_max, S, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipMemcpyAsync(out_plogs, st->w_plogs, sizeof(float) * S * n_max, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipMemcpyAsync(nslp.data(), st->w_nslp, sizeof(float) * S, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipGetLastError());
    for (int s = 0; s < S; s++) {
        const int n = ws[s].n_dec;
        fwhip_window_stream &o = streams[s];
        o.n_tokens = n;
        o.result_len = ws[s].result_len;
        o.has_ts = ws[s].has_ts;
        o.seek_delta_cs = ws[s].seek_delta_cs;
        o.n_exact = ws[s].n_exact;
        o.no_speech_logprob = nslp[s];
        for (int k = 0; k < n_max; k++) {
            out_tokens[(size_t)s * n_max + k] = k < n ? hist[(size_t)s * n_max + k] : 0;
            if (k >= n) out_plogs[(size_t)s * n_max + k] = 0.0f;
        }
    }
    st->len += n_prompt + steps - 1;
    return FWHIP_OK;
}

// process_logits (no-timestamps mode) + argmax (decode.rs:702-867, 1708-1790)
// over rows of logits already on the device: per-block keys, then the
// first-index maximum of each row.
extern "C" fwhip_status fwhip_argmax_logits(fwhip_ctx *c, const float *logits_dev, int32_t n_rows, int32_t n_vocab,
                                            const fwhip_filter *filter, int32_t initial, int32_t *argmax_host) {
    if (!c || !logits_dev || !argmax_host) return fw_fail(FWHIP_ERR_INVALID, "fwhip_argmax_logits: NULL argument");
    if (n_rows <= 0 || n_rows > 65535 || n_vocab <= 0)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_argmax_logits: n_rows must be in 1..65535 and n_vocab > 0");
    HIP_TRY(hipSetDevice(c->device));
    const int nblk = fw_logits_keys_blocks(n_vocab);
    const size_t kb = sizeof(unsigned long long) * (size_t)n_rows * nblk;
    const size_t need = kb + sizeof(int32_t) * (size_t)n_rows + 256;
    if (need > c->am_scratch_bytes) {
        HIP_TRY(hipStreamSynchronize(c->stream));
        if (c->am_scratch) HIP_TRY(hipFree(c->am_scratch));
        c->am_scratch = nullptr;
        c->am_scratch_bytes = 0;
        HIP_TRY(hipMalloc(&c->am_scratch, need));
        c->am_scratch_bytes = need;
    }
    unsigned long long *keys = (unsigned long long *)c->am_scratch;
    int32_t *tok = (int32_t *)((char *)c->am_scratch + kb);
    int *initp = (int *)(tok + n_rows);
    int init = initial ? 1 : 0;
    fwhip_status r = set_dev_ints(c, initp, &init, 1);
    if (r != FWHIP_OK) return r;
    fw_launch_logits_keys(c->stream, logits_dev, n_vocab, n_rows, filter, initp, keys);
    fw_launch_argmax_finish(c->stream, keys, nblk, n_rows, tok, nullptr, 0, nullptr, nullptr, nullptr, 0);
    HIP_TRY(hipMemcpyAsync(argmax_host, tok, sizeof(int32_t) * n_rows, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipGetLastError());
    return FWHIP_OK;
}

// layer_norm (nn.rs:4351-4545) of n_rows rows of d f32 on the device, with the
// decoder's one-wave-per-row kernel: exact = 1 sums the mean and variance in
// the reference's sequential order, exact = 0 in the wave's tree order.
extern "C" fwhip_status fwhip_layer_norm(fwhip_ctx *c, const float *x_dev, const float *w_dev, const float *b_dev,
                                         int64_t n_rows, int32_t d, float *y_dev, int32_t exact) {
    if (!c || !x_dev || !w_dev || !b_dev || !y_dev) return fw_fail(FWHIP_ERR_INVALID, "fwhip_layer_norm: NULL argument");
    if (d <= 0 || d % 4 != 0 || d > 2048 || n_rows <= 0 || n_rows > (int64_t)4 * 65535 * 1024)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_layer_norm: need d % 4 == 0, 0 < d <= 2048, 0 < n_rows <= 268M");
    HIP_TRY(hipSetDevice(c->device));
    for (int64_t r0 = 0; r0 < n_rows; r0 += (int64_t)4 * 65535) {
        const int n = (int)(n_rows - r0 < (int64_t)4 * 65535 ? n_rows - r0 : (int64_t)4 * 65535);
        fw_launch_ln_quant(c->stream, x_dev + r0 * d, y_dev + r0 * d, w_dev, b_dev, d, n, nullptr, nullptr,
                           exact ? 1 : 0);
    }
    HIP_TRY(hipGetLastError());
    HIP_TRY(hipStreamSynchronize(c->stream));
    return FWHIP_OK;
}
