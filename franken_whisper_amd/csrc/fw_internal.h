// fw_internal.h — host-side internals shared by the API translation units.
#pragma once
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "fwhip.h"

struct fw_event_pair {
    hipEvent_t a, b;
    int cls;
    double units;
    bool active;
};

struct fw_kstat {
    int64_t launches = 0;
    double ms = 0.0;
    double units = 0.0;
};

struct fwhip_ctx {
    int device = 0;
    int n_cu = 0;
    hipStream_t stream = nullptr;
    std::atomic<int> cancel{0};
    bool timing = false;
    std::vector<fw_event_pair> pending;
    std::vector<hipEvent_t> ev_pool; // events of drained timings, reused
    std::map<int, fw_kstat> stats;
    // device: the GELU table [65536] f32, followed in the same allocation by
    // the same values as f16 (fw_gelu_tab16)
    float *gelu_tab = nullptr;
    // log-mel: window and FFT twiddles (built on first use) and a scratch
    // buffer grown on demand (filter ranges, per-block maxima, the floor)
    void *mel_tab = nullptr;
    void *mel_scratch = nullptr;
    size_t mel_scratch_bytes = 0;
    // fwhip_argmax_logits: per-block keys, tokens and the first-step flag
    void *am_scratch = nullptr;
    size_t am_scratch_bytes = 0;
    // f16-pair range flag: set on the device by a split whose value reaches
    // |v| >= 65520; copied to pinned host memory before a forward's final sync
    int *ovf_dev = nullptr, *ovf_host = nullptr;
};
// clear the f16-pair range flag (a fill kernel) / queue its copy to the host
void fw_ovf_clear(fwhip_ctx *c);
void fw_ovf_fetch(fwhip_ctx *c);

fwhip_status fw_fail(fwhip_status code, const std::string &msg);
void fw_timed_begin(fwhip_ctx *c, int cls, double units, fw_event_pair *ev);
void fw_timed_end(fwhip_ctx *c, fw_event_pair *ev);
void *fw_dalloc(std::vector<void *> &owned, size_t bytes);
void *fw_dupload(std::vector<void *> &owned, const void *host, size_t bytes);
void fw_free_all(std::vector<void *> &owned);
// The context and model shape of a loaded encoder / decoder (encoder.hip,
// fwhip.hip), for the window driver.
fwhip_ctx *fw_encoder_ctx(const fwhip_encoder *e);
fwhip_hparams fw_encoder_hparams(const fwhip_encoder *e);
fwhip_ctx *fw_decoder_ctx(const fwhip_decoder *d);
fwhip_hparams fw_decoder_hparams(const fwhip_decoder *d);
// Resolve the allocation-free log-mel's device scratch and tables on `device`
// (the current device), once per device; called by fwhip_init.
void fw_mel_noalloc_setup(int device);

// IEEE binary16 <-> binary32 on the host (round-to-nearest-even).
static inline float fw_host_h2f(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16, ex = (h >> 10) & 0x1fu, man = h & 0x3ffu, bits;
    if (ex == 0) {
        if (man == 0) bits = sign;
        else {
            int e = -1;
            do {
                e++;
                man <<= 1;
            } while (!(man & 0x400u));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((man & 0x3ffu) << 13);
        }
    } else if (ex == 31) bits = sign | 0x7f800000u | (man << 13) | (man ? 0x400000u : 0u);
    else bits = sign | ((ex + 112u) << 23) | (man << 13);
    float f;
    memcpy(&f, &bits, 4);
    return f;
}
static inline uint16_t fw_host_f2h(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t a = x & 0x7fffffffu;
    if (a > 0x7f800000u) return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a == 0x7f800000u) return (uint16_t)(sign | 0x7c00u);
    if (a >= 0x38800000u) {
        uint32_t r = a - (112u << 23);
        r += 0xfffu + ((r >> 13) & 1u);
        r >>= 13;
        return (uint16_t)(sign | (r >= 0x7c00u ? 0x7c00u : r));
    }
    uint32_t e = a >> 23;
    if (e < 102) return sign;
    uint32_t m = (a & 0x7fffffu) | 0x800000u, s = 126u - e;
    uint32_t q = m >> s, rem = m & ((1u << s) - 1u), half = 1u << (s - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}
