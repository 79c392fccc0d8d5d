// transcribe.hip — the window driver (transcribe_samples_uncached,
// decode.rs:2956-3960, on its greedy path: beam 1, no temperature fallback, no
// word timestamps, explicit language, full-context windows — the reference's
// defaults).  Host code over the library's own entry points: the log-mel of
// the whole audio on the device, one encoder window at the seek, the window
// loop on the device (fwhip_decode_window), and the host-side rules between
// windows — prompt carry, the short-tail prompt clear, the no-speech gate, the
// failed-window retry, the single-timestamp-ending skip, segment building and
// the seek advance.
//
// Windows depend on each other through the carried prompt and, with
// timestamps, through the seek, so they run one at a time.  With no
// timestamps and no carried prompt they are independent (the fixed 30 s seek
// of decode_independent_no_timestamp_windows, decode.rs:2706-2822): then up
// to COHORT windows encode as one batch and decode as one cohort of streams,
// with the same results.
#include <algorithm>
#include <cmath>
#include <memory>
#include <string>
#include <vector>

#include "fw_internal.h"

namespace {

constexpr int64_t CHUNK_CS = 3000;
constexpr int64_t DELTA_MIN = 10;
constexpr double EMPTY_WINDOW_AVG_LOGPROB = -999.0;
constexpr int COHORT = 16;

struct Segment {
    int64_t start_cs, end_cs;
    std::string text;
    double confidence; // NaN: none
};

struct Window {
    int64_t seek_cs;
    double avg_logprob, no_speech_prob;
    int32_t result_len, has_ts, seek_delta_cs, no_speech, dropped, retried;
    std::vector<int32_t> tokens;
    std::vector<float> plogs;
};

struct Run {
    std::vector<int32_t> tokens;
    std::vector<float> plogs;
    int32_t result_len, has_ts, seek_delta_cs;
    float ns_lp;
};

// String::from_utf8_lossy: each maximal ill-formed subsequence -> U+FFFD
std::string utf8_lossy(const std::string &b) {
    std::string o;
    o.reserve(b.size());
    const size_t n = b.size();
    size_t i = 0;
    auto cont = [&](size_t k) { return k < n && ((unsigned char)b[k] & 0xc0) == 0x80; };
    while (i < n) {
        const unsigned char c = (unsigned char)b[i];
        if (c < 0x80) {
            o += (char)c;
            i++;
            continue;
        }
        size_t need = 0;
        unsigned char lo = 0x80, hi = 0xbf;
        if (c >= 0xc2 && c <= 0xdf) need = 1;
        else if (c >= 0xe0 && c <= 0xef) {
            need = 2;
            if (c == 0xe0) lo = 0xa0;
            if (c == 0xed) hi = 0x9f;
        } else if (c >= 0xf0 && c <= 0xf4) {
            need = 3;
            if (c == 0xf0) lo = 0x90;
            if (c == 0xf4) hi = 0x8f;
        }
        if (!need) { // not a lead byte
            o += "\xef\xbf\xbd";
            i++;
            continue;
        }
        size_t k = 1;
        bool ok = true;
        for (; k <= need; k++) {
            if (i + k >= n) {
                ok = false;
                break;
            }
            const unsigned char x = (unsigned char)b[i + k];
            const bool good = k == 1 ? (x >= lo && x <= hi) : cont(i + k);
            if (!good) {
                ok = false;
                break;
            }
        }
        if (ok) {
            o.append(b, i, need + 1);
            i += need + 1;
        } else {
            o += "\xef\xbf\xbd"; // the lead and the continuation bytes that fit
            i += k;
        }
    }
    return o;
}

// char::is_whitespace (White_Space) at the front / back of valid UTF-8
bool is_ws(uint32_t c) {
    return (c >= 0x09 && c <= 0x0d) || c == 0x20 || c == 0x85 || c == 0xa0 || c == 0x1680 ||
           (c >= 0x2000 && c <= 0x200a) || c == 0x2028 || c == 0x2029 || c == 0x202f || c == 0x205f || c == 0x3000;
}
uint32_t decode_at(const std::string &s, size_t i, size_t *len) {
    const unsigned char c = (unsigned char)s[i];
    if (c < 0x80) {
        *len = 1;
        return c;
    }
    const int n = c >= 0xf0 ? 4 : c >= 0xe0 ? 3 : 2;
    uint32_t v = c & (0x7f >> n);
    for (int k = 1; k < n; k++) v = (v << 6) | ((unsigned char)s[i + k] & 0x3f);
    *len = (size_t)n;
    return v;
}
std::string rust_trim(const std::string &s) {
    size_t a = 0, b = s.size();
    while (a < b) {
        size_t l;
        if (!is_ws(decode_at(s, a, &l))) break;
        a += l;
    }
    while (b > a) {
        size_t st = b - 1;
        while (st > a && ((unsigned char)s[st] & 0xc0) == 0x80) st--;
        size_t l;
        if (!is_ws(decode_at(s, st, &l))) break;
        b = st;
    }
    return s.substr(a, b - a);
}

struct Tok {
    const fwhip_vocab *v;
    int32_t eot, beg;
    // Tokenizer::decode (tokenizer.rs:548-567) + str::trim
    std::string text(const int32_t *t, size_t n) const {
        std::string b;
        for (size_t i = 0; i < n; i++)
            if (t[i] < eot && t[i] >= 0 && t[i] < v->n_tokens)
                b.append((const char *)v->bytes + v->offsets[t[i]], (size_t)(v->offsets[t[i] + 1] - v->offsets[t[i]]));
        return rust_trim(utf8_lossy(b));
    }
    // text_confidence (decode.rs:2019-2046)
    double confidence(const int32_t *t, const float *p, size_t n) const {
        double sum = 0.0;
        size_t cnt = 0;
        for (size_t i = 0; i < n; i++)
            if (t[i] < beg && t[i] < eot && std::isfinite(p[i])) {
                sum += (double)p[i];
                cnt++;
            }
        if (!cnt) return NAN;
        const double c = std::exp(sum / (double)cnt);
        return std::isfinite(c) ? (c < 0.0 ? 0.0 : c > 1.0 ? 1.0 : c) : 0.0;
    }
};

// build_segments (decode.rs:1877-1977)
void build_segments(const Tok &tk, const int32_t *t, const float *p, size_t n, int64_t seek, int64_t delta,
                    int64_t seek_end, bool split, std::vector<Segment> &out) {
    const int64_t hi = seek_end > seek ? seek_end : seek;
    auto clamp = [&](int64_t x) { return x < seek ? seek : x > hi ? hi : x; };
    if (!split) {
        std::string text = tk.text(t, n);
        if (!text.empty()) out.push_back({clamp(seek), clamp(seek + delta), text, tk.confidence(t, p, n)});
        return;
    }
    size_t i0 = 0, i = 0;
    int64_t t0 = clamp(seek + (n && t[0] >= tk.beg ? 2 * (int64_t)(t[0] - tk.beg) : 0));
    while (i < n) {
        if (t[i] > tk.beg) {
            const int64_t t1 = clamp(seek + 2 * (int64_t)(t[i] - tk.beg));
            std::string text = tk.text(t + i0, i + 1 - i0);
            if (!text.empty()) out.push_back({t0, t1, text, tk.confidence(t + i0, p + i0, i + 1 - i0)});
            t0 = t1;
            while (i + 1 < n && t[i + 1] > tk.beg) i++;
            i0 = i + 1;
        }
        i++;
    }
    if (i0 < n) {
        std::string text = tk.text(t + i0, n - i0);
        if (!text.empty()) out.push_back({t0, clamp(seek + delta), text, tk.confidence(t + i0, p + i0, n - i0)});
    }
}

bool single_timestamp_ending(const std::vector<int32_t> &d, size_t n, int32_t beg, bool ts, int32_t budget) {
    const bool forced = ts && budget > 0 && n > (size_t)budget;
    return n > 1 && !forced && d[n - 2] < beg && d[n - 1] > beg;
}

bool is_tiny_en(const fwhip_hparams &h) {
    return h.n_vocab == 51864 && h.n_audio_ctx == 1500 && h.n_audio_state == 384 && h.n_audio_head == 6 &&
           h.n_audio_layer == 4 && h.n_text_ctx == 448 && h.n_text_state == 384 && h.n_text_head == 6 &&
           h.n_text_layer == 4 && h.n_mels == 80;
}

} // namespace

struct fwhip_transcript {
    std::vector<Segment> segments;
    std::vector<Window> windows;
};

#define TR_TRY(expr)                                                                                              \
    do {                                                                                                          \
        fwhip_status _r = (expr);                                                                                 \
        if (_r != FWHIP_OK) return _r;                                                                            \
    } while (0)

namespace {

struct Driver {
    fwhip_ctx *c;
    fwhip_encoder *enc;
    fwhip_decoder *dec;
    fwhip_hparams hp;
    const fwhip_filter *f;
    const fwhip_transcribe_params *p;
    Tok tk;
    const float *mel = nullptr;
    int64_t mel_frames = 0;
    float *encbuf = nullptr;
    fwhip_dstate *st = nullptr;
    int st_streams = 0;
    fwhip_window_cfg wc;

    ~Driver() {
        if (st) fwhip_dstate_free(st);
        if (encbuf) fwhip_free(c, encbuf);
    }

    fwhip_status state(int S) {
        if (st && st_streams == S) return FWHIP_OK;
        if (st) fwhip_dstate_free(st);
        st = nullptr;
        TR_TRY(fwhip_dstate_new(dec, S, hp.n_audio_ctx, &st));
        st_streams = S;
        return FWHIP_OK;
    }

    // encode windows at `seeks` and run the window loop over them as one cohort
    fwhip_status run(const std::vector<int64_t> &seeks, const std::vector<int32_t> &prompt, int64_t seek_end,
                     int has_prior, std::vector<Run> &out) {
        const int S = (int)seeks.size();
        fwhip_exec_record rec;
        TR_TRY(fwhip_encoder_forward(enc, mel, mel_frames, seeks.data(), S, 2 * hp.n_audio_ctx, encbuf, &rec));
        TR_TRY(state(S));
        TR_TRY(fwhip_dstate_set_cross(st, encbuf));
        std::vector<fwhip_window_stream> ws(S);
        for (int s = 0; s < S; s++) {
            memset(&ws[s], 0, sizeof ws[s]);
            ws[s].seek_cs = (int32_t)seeks[s];
            ws[s].seek_end_cs = (int32_t)seek_end;
            ws[s].has_prior_segments = has_prior;
        }
        std::vector<int32_t> toks((size_t)S * wc.n_max);
        std::vector<float> plogs((size_t)S * wc.n_max);
        TR_TRY(fwhip_decode_window(st, prompt.data(), (int32_t)prompt.size(), f, &wc, ws.data(), toks.data(),
                                   plogs.data()));
        out.resize(S);
        for (int s = 0; s < S; s++) {
            Run &r = out[s];
            const int n = ws[s].n_tokens;
            r.tokens.assign(toks.begin() + (size_t)s * wc.n_max, toks.begin() + (size_t)s * wc.n_max + n);
            r.plogs.assign(plogs.begin() + (size_t)s * wc.n_max, plogs.begin() + (size_t)s * wc.n_max + n);
            r.result_len = ws[s].result_len;
            r.has_ts = ws[s].has_ts;
            r.seek_delta_cs = ws[s].seek_delta_cs;
            r.ns_lp = ws[s].no_speech_logprob;
        }
        return FWHIP_OK;
    }
};

} // namespace

extern "C" fwhip_status fwhip_transcribe(fwhip_ctx *c, fwhip_encoder *enc, fwhip_decoder *dec, const float *samples_dev,
                                         int64_t n_samples, const float *filters_dev, int32_t n_mel,
                                         const fwhip_filter *filter, const fwhip_vocab *vocab,
                                         const fwhip_transcribe_params *p, fwhip_transcript **out) {
    if (!c || !enc || !dec || !filters_dev || !filter || !vocab || !p || !out || (!samples_dev && n_samples))
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_transcribe: NULL argument");
    *out = nullptr;
    if (fw_encoder_ctx(enc) != c || fw_decoder_ctx(dec) != c)
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_transcribe: encoder and decoder must belong to the context");
    if (n_samples <= 0) return fw_fail(FWHIP_ERR_INVALID, "transcribe_samples: empty audio");
    if (!p->sot_sequence || p->n_sot <= 0) return fw_fail(FWHIP_ERR_INVALID, "fwhip_transcribe: empty sot sequence");
    if (vocab->n_tokens < 0 || (vocab->n_tokens && (!vocab->bytes || !vocab->offsets)))
        return fw_fail(FWHIP_ERR_INVALID, "fwhip_transcribe: malformed vocab");
    Driver D;
    D.c = c;
    D.enc = enc;
    D.dec = dec;
    D.hp = fw_decoder_hparams(dec);
    const fwhip_hparams ehp = fw_encoder_hparams(enc);
    D.hp.n_audio_ctx = ehp.n_audio_ctx;
    D.hp.n_audio_state = ehp.n_audio_state;
    D.hp.n_audio_head = ehp.n_audio_head;
    D.hp.n_audio_layer = ehp.n_audio_layer;
    D.hp.n_mels = ehp.n_mels;
    D.f = filter;
    D.p = p;
    D.tk = Tok{vocab, filter->eot, filter->timestamp_begin};
    if (n_mel != ehp.n_mels) return fw_fail(FWHIP_ERR_INVALID, "fwhip_transcribe: n_mel differs from the encoder's");
    const fwhip_hparams &hp = D.hp;
    const bool ts = p->timestamps != 0;

    // the log-mel of the whole audio (mel.rs:1476), once
    D.mel_frames = fwhip_mel_frames(n_samples);
    void *mel = nullptr;
    TR_TRY(fwhip_malloc(c, sizeof(float) * (size_t)n_mel * D.mel_frames, &mel));
    struct Free {
        fwhip_ctx *c;
        void *p;
        ~Free() { fwhip_free(c, p); }
    } free_mel{c, mel};
    D.mel = (const float *)mel;
    TR_TRY(fwhip_log_mel(c, samples_dev, n_samples, filters_dev, n_mel, 201, (float *)mel));

    // run constants (decode.rs:2985-3044)
    const int64_t seek_end = std::max<int64_t>(1 + std::max<int64_t>(n_samples + 200 - 400, 0) / 160, DELTA_MIN);
    const float prec = 30.0f / (float)std::max(hp.n_audio_ctx, 1);
    const int32_t mit = (int32_t)std::round(1.0f / prec);
    const int32_t n_max = std::max(hp.n_text_ctx / 2 - 4, 1);
    const int32_t user_mt = p->max_tokens > 0 ? std::min(p->max_tokens, n_max) : 0;
    const int32_t max_prompt =
        (p->max_context_set && p->max_context >= 0) ? p->max_context : hp.n_text_ctx / 2;
    const bool tiny_policy = is_tiny_en(hp) && ts && !p->max_context_set && !p->tiny_en_ts_context;
    D.wc.timestamps = ts ? 1 : 0;
    D.wc.max_initial_tid = mit;
    D.wc.max_tokens = user_mt;
    D.wc.n_max = n_max;
    D.wc.exact = p->exact_forcing ? 1 : 0;
    const std::vector<int32_t> sot(p->sot_sequence, p->sot_sequence + p->n_sot);

    // split_carried_prompt (decode.rs:997-1011)
    std::vector<int32_t> st_prompt, past;
    {
        std::vector<int32_t> ip(p->initial_prompt, p->initial_prompt + (p->initial_prompt ? p->n_initial_prompt : 0));
        if (p->carry_initial_prompt && !ip.empty()) {
            const size_t keep = (size_t)std::max(max_prompt - 1, 1);
            st_prompt.assign(ip.end() - (ip.size() > keep ? keep : ip.size()), ip.end());
        } else {
            past = ip;
        }
    }
    fwhip_transcript *T = new fwhip_transcript();
    std::unique_ptr<fwhip_transcript> guard(T);
    const size_t ENC_WINDOWS = COHORT;
    {
        void *eb = nullptr;
        TR_TRY(fwhip_malloc(c, sizeof(float) * ENC_WINDOWS * hp.n_audio_ctx * hp.n_audio_state, &eb));
        D.encbuf = (float *)eb;
    }
    auto gate = [&](const Run &r, double *avg, double *nsp) {
        const float x = expf(r.ns_lp);
        *nsp = std::isfinite(x) ? (double)x : 0.0;
        const size_t rl = (size_t)r.result_len;
        const size_t n = (rl > 0 && rl <= r.plogs.size()) ? rl : r.plogs.size();
        double a = EMPTY_WINDOW_AVG_LOGPROB;
        if (n) {
            double sum = 0.0;
            for (size_t i = 0; i < n; i++) sum += (double)r.plogs[i];
            a = sum / (double)n;
        }
        *avg = std::isfinite(a) ? a : EMPTY_WINDOW_AVG_LOGPROB;
        return *nsp > p->no_speech_threshold && *avg < p->logprob_threshold;
    };
    auto accept = [&](int64_t seek, const Run &r, double avg, double nsp, bool no_speech, bool dropped, bool retried) {
        Window w;
        w.seek_cs = seek;
        w.avg_logprob = avg;
        w.no_speech_prob = nsp;
        w.result_len = r.result_len;
        w.has_ts = r.has_ts;
        w.seek_delta_cs = r.seek_delta_cs;
        w.no_speech = no_speech;
        w.dropped = dropped;
        w.retried = retried;
        w.tokens = r.tokens;
        w.plogs = r.plogs;
        T->windows.push_back(std::move(w));
        const size_t take = std::min((size_t)r.result_len, r.tokens.size());
        if (!no_speech && !r.tokens.empty()) {
            build_segments(D.tk, r.tokens.data(), r.plogs.data(), take, seek, r.seek_delta_cs, seek_end, ts,
                           T->segments);
            past.clear();
            for (size_t i = 0; i < take; i++)
                if (r.tokens[i] < filter->eot) past.push_back(r.tokens[i]);
            if (past.size() > (size_t)max_prompt) past.erase(past.begin(), past.end() - max_prompt);
        } else if (no_speech) {
            past.clear();
        }
    };

    const bool carry_off = max_prompt <= 1 || p->no_context;
    if (!ts && carry_off) {
        // independent windows (decode.rs:2706-2822): fixed 30 s seeks, the
        // bare sot sequence as prompt, cohorts of COHORT windows
        std::vector<int64_t> seeks;
        for (int64_t s = 0; s + DELTA_MIN < seek_end; s += CHUNK_CS) seeks.push_back(s);
        for (size_t b = 0; b < seeks.size(); b += ENC_WINDOWS) {
            std::vector<int64_t> part(seeks.begin() + b, seeks.begin() + std::min(seeks.size(), b + ENC_WINDOWS));
            std::vector<Run> runs;
            TR_TRY(D.run(part, sot, seek_end, 0, runs));
            for (size_t k = 0; k < part.size(); k++) {
                double avg, nsp;
                const bool ns = gate(runs[k], &avg, &nsp);
                accept(part[k], runs[k], avg, nsp, ns, runs[k].result_len == 0 && !ns && part[k] > 0, false);
            }
        }
        *out = guard.release();
        return FWHIP_OK;
    }

    int64_t seek = 0;
    bool force_empty = false;
    while (seek + DELTA_MIN < seek_end) {
        if (seek > 0 && seek + 500 >= seek_end) { // short tail: drop the carried prompt (decode.rs:3383-3386)
            st_prompt.clear();
            past.clear();
        }
        const std::vector<int32_t> none;
        const std::vector<int32_t> &rolling = (tiny_policy && seek > 0) ? none : past;
        const bool carried = !p->no_context && !force_empty && (!rolling.empty() || !st_prompt.empty()) && max_prompt > 1;
        std::vector<int32_t> prompt;
        if (carried) { // carried_prompt_tokens (decode.rs:1013-1029)
            const size_t budget = (size_t)std::max<int64_t>((int64_t)max_prompt - 1 - (int64_t)st_prompt.size(), 0);
            const size_t take = std::min(rolling.size(), budget);
            prompt.push_back(filter->sot_prev);
            prompt.insert(prompt.end(), st_prompt.begin(), st_prompt.end());
            prompt.insert(prompt.end(), rolling.end() - take, rolling.end());
        }
        prompt.insert(prompt.end(), sot.begin(), sot.end());
        std::vector<Run> runs;
        TR_TRY(D.run({seek}, prompt, seek_end, T->segments.empty() ? 0 : 1, runs));
        const Run &r = runs[0];
        double avg, nsp;
        const bool ns = gate(r, &avg, &nsp);
        if (p->retry_failed_window && r.result_len == 0 && !ns && !force_empty && carried) {
            force_empty = true; // the same seek once more with no carried prompt
            continue;
        }
        const bool retried = force_empty;
        force_empty = false;
        const size_t take = std::min((size_t)r.result_len, r.tokens.size());
        const bool ste = single_timestamp_ending(r.tokens, take, filter->timestamp_begin, ts, user_mt);
        const int64_t advance = ste ? std::min(seek_end - seek, CHUNK_CS) : (int64_t)r.seek_delta_cs;
        accept(seek, r, avg, nsp, ns, r.result_len == 0 && !ns && seek > 0, retried);
        seek += std::max(advance, DELTA_MIN);
        if (c->cancel.exchange(0)) return fw_fail(FWHIP_ERR_CANCELLED, "cancelled");
    }
    *out = guard.release();
    return FWHIP_OK;
}

extern "C" int32_t fwhip_transcript_n_segments(const fwhip_transcript *t) { return t ? (int32_t)t->segments.size() : -1; }
extern "C" fwhip_status fwhip_transcript_segment(const fwhip_transcript *t, int32_t i, fwhip_segment_info *o) {
    if (!t || !o) return fw_fail(FWHIP_ERR_INVALID, "fwhip_transcript_segment: NULL argument");
    if (i < 0 || (size_t)i >= t->segments.size()) return fw_fail(FWHIP_ERR_INVALID, "segment index out of range");
    const Segment &s = t->segments[i];
    o->start_cs = s.start_cs;
    o->end_cs = s.end_cs;
    o->text = s.text.c_str();
    o->confidence = s.confidence;
    return FWHIP_OK;
}
extern "C" int32_t fwhip_transcript_n_windows(const fwhip_transcript *t) { return t ? (int32_t)t->windows.size() : -1; }
extern "C" fwhip_status fwhip_transcript_window(const fwhip_transcript *t, int32_t i, fwhip_window_info *o) {
    if (!t || !o) return fw_fail(FWHIP_ERR_INVALID, "fwhip_transcript_window: NULL argument");
    if (i < 0 || (size_t)i >= t->windows.size()) return fw_fail(FWHIP_ERR_INVALID, "window index out of range");
    const Window &w = t->windows[i];
    o->seek_cs = w.seek_cs;
    o->avg_logprob = w.avg_logprob;
    o->no_speech_prob = w.no_speech_prob;
    o->result_len = w.result_len;
    o->n_tokens = (int32_t)w.tokens.size();
    o->has_ts = w.has_ts;
    o->seek_delta_cs = w.seek_delta_cs;
    o->no_speech = w.no_speech;
    o->dropped = w.dropped;
    o->retried = w.retried;
    o->tokens = w.tokens.data();
    o->plogs = w.plogs.data();
    return FWHIP_OK;
}
extern "C" void fwhip_transcript_free(fwhip_transcript *t) { delete t; }
