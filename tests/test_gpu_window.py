"""The window loop on the device (fwhip_decode_window: process_logits in full,
argmax, the loop state of decode.rs:3456-3566) against the oracle's
restatement of the same loop (oracle/transcribe_ref.window_loop over
ref_decoder_step and ref_process_logits): sampled tokens, their
log-probabilities, result_len, has_ts, the seek delta and the no-speech
log-probability bit for bit, in timestamp and no-timestamps mode, with the
initial-timestamp cap, the user token budget, seeks that reach the end of the
audio (rescue / end rules), prior segments, cohorts of streams, both decoder
arms, and the exact forcing decision on every step (exact = 1) giving the same
windows as the default."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from oracle import oracle as O
from oracle import transcribe_ref as R
from tests.helpers import assert_bitexact

pytestmark = pytest.mark.gpu

MICRO_ML = synth.MICRO_ML


def _run(ctx, cfgm, arm, seed, streams, timestamps, max_tokens=None, exact=0):
    m = synth.Model(cfgm, seed=seed)
    tk = m.tokens
    filt = tk.filter()
    T = cfgm.n_audio_ctx
    enc = synth.encoder_states(seed + 1, len(streams), T, cfgm.n_text_state)
    n_max = cfgm.n_text_ctx // 2 - 4
    mit = R.max_initial_tid(cfgm.n_audio_ctx)
    prompt = tk.sot_sequence(language_id=0, timestamps=timestamps)
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(True)
    st = dec.state(len(streams), T)
    st.set_cross(ctx.array(enc))
    wc = abi.WindowCfg(1 if timestamps else 0, mit, max_tokens or 0, n_max, exact)
    got = st.window(prompt, filt, wc, streams)
    st.close()
    dec.close()
    od = O.Decoder(m, arm)
    user_mt = min(max_tokens, n_max) if max_tokens else None
    want = []
    for s, (sk, se, hp) in enumerate(streams):
        ost = od.state(enc[s])
        want.append(R.window_loop(ost, prompt, filt, timestamps, mit, n_max, user_mt, sk, se, hp))
    return got, want


def _same(got, want, label):
    for s, (g, w) in enumerate(zip(got, want)):
        tag = f"{label} stream {s}"
        assert g["tokens"] == w["tokens"], f"{tag}: tokens {g['tokens']} vs {w['tokens']}"
        assert_bitexact(g["plogs"], w["plogs"], f"{tag} plogs")
        for k in ("result_len", "has_ts", "seek_delta_cs"):
            assert g[k] == w[k], f"{tag} {k}: {g[k]} vs {w[k]}"
        assert_bitexact(np.float32(g["no_speech_lp"]), np.float32(w["no_speech_lp"]), f"{tag} no-speech")


CASES = [
    ("ts-one-window", abi.DEC_F16, 3, [(0, 100000, False)], True, None),
    ("ts-cohort-seeks", abi.DEC_F16, 4, [(0, 100000, False), (3000, 3400, True), (6000, 6100, False)], True, None),
    ("ts-int8-arm", abi.DEC_INT8, 5, [(0, 100000, False), (1200, 2000, True)], True, None),
    ("ts-budget", abi.DEC_F16, 6, [(0, 100000, False), (0, 100000, True)], True, 5),
    ("no-ts-cohort", abi.DEC_F16, 7, [(0, 100000, False), (3000, 6000, True), (6000, 6400, False)], False, None),
    ("no-ts-budget", abi.DEC_INT8, 8, [(0, 100000, False)], False, 3),
]


@pytest.mark.parametrize("name,arm,seed,streams,ts,mt", CASES, ids=[c[0] for c in CASES])
def test_window_loop_matches_oracle(ctx, name, arm, seed, streams, ts, mt):
    print(f"window loop {name}", flush=True)
    got, want = _run(ctx, MICRO_ML, arm, seed, streams, ts, mt)
    _same(got, want, name)
    print(name, [(len(g["tokens"]), g["result_len"], g["has_ts"], g["n_exact"]) for g in got], flush=True)


def test_window_loop_exact_decision_mode_gives_the_same_windows(ctx):
    streams = [(0, 100000, False), (3000, 5000, True)]
    a, want = _run(ctx, MICRO_ML, abi.DEC_F16, 9, streams, True)
    b, _ = _run(ctx, MICRO_ML, abi.DEC_F16, 9, streams, True, exact=1)
    _same(a, want, "default")
    _same(b, want, "exact")
    assert all(x["n_exact"] == len(x["tokens"]) or x["n_exact"] <= len(x["tokens"]) for x in b)


def test_window_loop_english_only_model(ctx):
    got, want = _run(ctx, synth.MICRO, abi.DEC_F16, 10, [(0, 100000, False), (0, 800, False)], True)
    _same(got, want, "micro.en")
