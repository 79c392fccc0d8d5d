"""Restatement of the reference's window driver over the oracle's decoder.

TEST INFRASTRUCTURE: imported only by tests/ as the checker of the library's
window loop (fwhip_decode_window) and driver (fwhip_transcribe) — never by the
product package.

Follows transcribe_samples_uncached (src/native_engine/decode.rs:2956-3960) on
its greedy path (beam 1, no temperature fallback, no word timestamps, explicit
language, no tail truncation, which are its defaults), step by step:

- `window_loop`           the per-window prefill + greedy loop   decode.rs:3405-3566
- `process_logits`        via the C restatement (refcpu.c)       decode.rs:702-867
- `build_segments`        timestamp-paired / single segments     decode.rs:1877-1977
- `text_confidence`                                              decode.rs:2019-2046
- `single_timestamp_ending`, `should_rescue_unclosed_window`     decode.rs:2376-2416
- `carried_prompt_tokens`, `split_carried_prompt`                decode.rs:997-1029
- `should_clear_short_tail_prompt`                               decode.rs:1980-1982
- `suppress_tiny_en_ts_context`                                  decode.rs:939-966
- `transcribe`            the window loop over the audio         decode.rs:2956-3960

Pinned by the reference's own unit cases for these functions
(decode.rs:5305-5811), restated in tests/test_oracle_window.py.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass, field

import numpy as np

from oracle import oracle as O

CHUNK_CS = 3000
DELTA_MIN = 10
EMPTY_WINDOW_AVG_LOGPROB = -999.0

_libm = C.CDLL("libm.so.6")
_libm.expf.restype = C.c_float
_libm.expf.argtypes = [C.c_float]

# char::is_whitespace (the White_Space property), which str::trim strips
RUST_WHITESPACE = "".join(map(chr, [*range(0x09, 0x0E), 0x20, 0x85, 0xA0, 0x1680, *range(0x2000, 0x200B), 0x2028,
                                    0x2029, 0x202F, 0x205F, 0x3000]))


@dataclass
class Params:
    """The DecodeParams fields the greedy driver reads (decode.rs:239-447)."""
    timestamps: bool = False
    max_context: int | None = None   # None: n_text_ctx / 2; 0: no carry; n: cap
    max_tokens: int | None = None    # max_text_ctx, the user token budget
    no_context: bool = False         # FW_NO_CONTEXT
    retry_failed_window: bool = True  # FW_RETRY_FAILED_WINDOW (default on)
    tiny_en_ts_context: bool = False  # FW_TINY_EN_TS_CONTEXT
    carry_initial_prompt: bool = False
    initial_prompt: list = field(default_factory=list)  # token ids of the user prompt
    no_speech_threshold: float = 0.6
    logprob_threshold: float = -1.0


def seek_end_cs(n_samples: int) -> int:
    """n_len_org in centiseconds (decode.rs:2985-2995)."""
    return max(1 + max(n_samples + 200 - 400, 0) // 160, DELTA_MIN)


def max_initial_tid(n_audio_ctx: int) -> int:
    """(1.0 / (30 / n_audio_ctx)).round() in f32 (decode.rs:3004-3009)."""
    q = np.float32(1.0) / (np.float32(30.0) / np.float32(max(n_audio_ctx, 1)))
    return int(math.floor(float(q) + 0.5))


def filter_cfg(timestamps: bool, mit: int, max_tokens: int | None) -> O.RefFilterCfg:
    return O.RefFilterCfg(1, 0 if timestamps else 1, mit, max_tokens if max_tokens else -1)


def window_loop(st, prompt, filt, timestamps, mit, n_max, user_max_tokens, seek_cs, seek_end, has_prior):
    """Prefill + the greedy loop of one window (decode.rs:3405-3566)."""
    beg, eot = filt.timestamp_begin, filt.eot
    logits = st.step(np.asarray(prompt, np.int32))
    lp0 = O.compute_logprobs(logits)
    ns_lp = float(lp0[filt.no_speech])
    cfg = filter_cfg(timestamps, mit, user_max_tokens)
    decoded, plogs = [], []
    has_ts, delta, rl = False, CHUNK_CS, 0
    for i in range(n_max):
        flt, lp, _ = O.process_logits(filt, cfg, logits, decoded, has_ts, delta, len(decoded))
        tok = O.argmax_first(flt)
        decoded.append(tok)
        plogs.append(np.float32(lp[tok]))
        if tok > beg:
            nd = 2 * (tok - beg)
            if has_ts and delta > nd and rl < i:
                break
            delta, rl, has_ts = nd, i + 1, True
        budget = user_max_tokens is not None and i >= user_max_tokens
        covers = seek_cs + delta + DELTA_MIN >= seek_end
        if tok == eot or budget or (has_ts and covers):
            if rl == 0 and timestamps:
                if covers and (seek_cs == 0 or not has_prior):
                    rl = i + 1
                else:
                    break
            if not timestamps:
                rl, delta = i + 1, CHUNK_CS
            break
        if i + 1 == n_max:
            break  # the reference's last forward is never sampled
        logits = st.step(np.asarray([tok], np.int32))
    return {"tokens": decoded, "plogs": np.array(plogs, np.float32), "result_len": rl, "has_ts": has_ts,
            "seek_delta_cs": delta, "no_speech_lp": np.float32(ns_lp)}


def carried_prompt_tokens(sot_prev, static, past, max_ctx):
    take = min(len(past), max(max_ctx - (1 + len(static)), 0))
    return [sot_prev] + list(static) + list(past[len(past) - take:])


def split_carried_prompt(tokens, carry_initial, max_ctx):
    if not carry_initial or not tokens:
        return [], list(tokens)
    keep = max(max_ctx - 1, 1)
    return list(tokens[max(len(tokens) - keep, 0):]), []


def is_tiny_en(hp) -> bool:
    return (hp.n_vocab, hp.n_audio_ctx, hp.n_audio_state, hp.n_audio_head, hp.n_audio_layer, hp.n_text_ctx,
            hp.n_text_state, hp.n_text_head, hp.n_text_layer, hp.n_mels) == (51864, 1500, 384, 6, 4, 448, 384, 6,
                                                                              4, 80)


def suppress_tiny_en_ts_context(hp, p: Params) -> bool:
    return is_tiny_en(hp) and p.timestamps and p.max_context is None and not p.tiny_en_ts_context


def single_timestamp_ending(decoded, beg, timestamps, budget):
    forced = timestamps and budget is not None and len(decoded) > budget
    return len(decoded) > 1 and not forced and decoded[-2] < beg and decoded[-1] > beg


def should_rescue_unclosed_window(seek_cs, covers, has_prior):
    return covers and (seek_cs == 0 or not has_prior)


def should_clear_short_tail_prompt(seek_cs, seek_end):
    return seek_cs > 0 and seek_cs + 500 >= seek_end


def ts_offset_cs(tok, beg):
    return 2 * (tok - beg) if tok is not None and tok >= beg else 0


def decode_text(vocab, tokens, eot) -> str:
    """Tokenizer::decode (tokenizer.rs:548-567): the bytes of the non-special
    tokens, lossy UTF-8; then str::trim."""
    b = b"".join(vocab[t] for t in tokens if t < eot and 0 <= t < len(vocab))
    return b.decode("utf-8", errors="replace").strip(RUST_WHITESPACE)


def text_confidence(tokens, plogs, beg, eot):
    vals = [float(p) for t, p in zip(tokens, plogs) if t < beg and t < eot and math.isfinite(float(p))]
    if not vals:
        return None
    c = math.exp(sum(vals) / len(vals))
    return min(max(c, 0.0), 1.0) if math.isfinite(c) else 0.0


def build_segments(vocab, tokens, plogs, seek_cs, delta, seek_end, split, beg, eot):
    def clamp(t):
        return min(max(t, seek_cs), max(seek_end, seek_cs))
    segs = []
    if not split:
        text = decode_text(vocab, tokens, eot)
        if text:
            segs.append((clamp(seek_cs), clamp(seek_cs + delta), text, text_confidence(tokens, plogs, beg, eot)))
        return segs
    i0 = 0
    t0 = clamp(seek_cs + ts_offset_cs(tokens[0] if tokens else None, beg))
    i = 0
    while i < len(tokens):
        tok = tokens[i]
        if tok > beg:
            t1 = clamp(seek_cs + 2 * (tok - beg))
            text = decode_text(vocab, tokens[i0:i + 1], eot)
            if text:
                segs.append((t0, t1, text, text_confidence(tokens[i0:i + 1], plogs[i0:i + 1], beg, eot)))
            t0 = t1
            while i + 1 < len(tokens) and tokens[i + 1] > beg:
                i += 1
            i0 = i + 1
        i += 1
    if i0 < len(tokens):
        text = decode_text(vocab, tokens[i0:], eot)
        if text:
            segs.append((t0, clamp(seek_cs + delta), text, text_confidence(tokens[i0:], plogs[i0:], beg, eot)))
    return segs


def transcribe(encode, dec, hp, n_samples, filt, sot_seq, vocab, p: Params):
    """transcribe_samples_uncached (decode.rs:2956-3960), greedy path.
    encode(seek_cs) -> the encoder states of the window at that mel frame."""
    beg, eot = filt.timestamp_begin, filt.eot
    seek_end = seek_end_cs(n_samples)
    mit = max_initial_tid(hp.n_audio_ctx)
    n_max = max(hp.n_text_ctx // 2 - 4, 1)
    user_mt = min(p.max_tokens, n_max) if p.max_tokens and p.max_tokens > 0 else None
    max_prompt = p.max_context if (p.max_context is not None and p.max_context >= 0) else hp.n_text_ctx // 2
    tiny_policy = suppress_tiny_en_ts_context(hp, p)
    static, past = split_carried_prompt(list(p.initial_prompt), p.carry_initial_prompt, max_prompt)
    segments, windows = [], []
    seek = 0
    force_empty = False
    enc_cache = None
    while seek + DELTA_MIN < seek_end:
        if enc_cache is not None and enc_cache[0] == seek:
            enc = enc_cache[1]
        else:
            enc = encode(seek)
        enc_cache = None
        st = dec.state(enc)
        if should_clear_short_tail_prompt(seek, seek_end):
            static, past = [], []
        rolling = [] if (tiny_policy and seek > 0) else past
        carried = (not p.no_context and not force_empty and (len(rolling) > 0 or len(static) > 0)
                   and max_prompt > 1)
        prompt = carried_prompt_tokens(filt.sot_prev, static, rolling, max_prompt) if carried else []
        prompt = prompt + list(sot_seq)
        w = window_loop(st, prompt, filt, p.timestamps, mit, n_max, user_mt, seek, seek_end, len(segments) > 0)
        del st
        decoded, plogs, rl = w["tokens"], w["plogs"], w["result_len"]
        x = float(_libm.expf(float(w["no_speech_lp"])))
        nsp = x if math.isfinite(x) else 0.0
        rp = plogs[:rl] if 0 < rl <= len(plogs) else plogs
        avg = sum(float(v) for v in rp) / len(rp) if len(rp) else EMPTY_WINDOW_AVG_LOGPROB
        if not math.isfinite(avg):
            avg = EMPTY_WINDOW_AVG_LOGPROB
        no_speech = nsp > p.no_speech_threshold and avg < p.logprob_threshold
        if p.retry_failed_window and rl == 0 and not no_speech and not force_empty and carried:
            force_empty = True
            enc_cache = (seek, enc)
            continue
        retried = force_empty
        force_empty = False
        dropped = rl == 0 and not no_speech and seek > 0
        res = decoded[:min(rl, len(decoded))]
        ste = single_timestamp_ending(res, beg, p.timestamps, user_mt)
        advance = min(seek_end - seek, CHUNK_CS) if ste else w["seek_delta_cs"]
        windows.append({"seek_cs": seek, "avg_logprob": avg, "no_speech_prob": nsp, "result_len": rl,
                        "tokens": decoded, "plogs": plogs, "dropped": dropped, "retried": retried,
                        "no_speech": no_speech, "seek_delta_cs": w["seek_delta_cs"], "has_ts": w["has_ts"]})
        if not no_speech and decoded:
            take = min(rl, len(decoded))
            segments += build_segments(vocab, decoded[:take], plogs[:take], seek, w["seek_delta_cs"], seek_end,
                                       p.timestamps, beg, eot)
            past = [t for t in decoded[:take] if t < eot]
            if len(past) > max_prompt:
                past = past[len(past) - max_prompt:]
        elif no_speech:
            past = []
        seek += max(advance, DELTA_MIN)
    return {"segments": segments, "windows": windows}
