"""The window driver (fwhip_transcribe) against the oracle's restatement of
transcribe_samples_uncached (oracle/transcribe_ref.transcribe over the
oracle's log-mel, encoder and decoder): every accepted window — seek, decoded
tokens, their log-probabilities, result_len, avg_logprob, no-speech
probability, the gate, dropped / retried marks — and every segment — bounds,
text and confidence — identical, for no-timestamps decoding with and without
the carried prompt (the batched independent windows and the sequential loop),
segment timestamps with prompt carry, a user token budget, a carried initial
prompt, and a no-speech threshold that gates windows out.

The model is a seeded random-init Whisper with a 1500-row audio context (full
30 s windows), two encoder blocks and a 96-token text context; the audio is
seeded synthetic speech-like noise with silent gaps; the vocabulary is the
synthetic byte-level one of the seeded model file (its single-byte tokens
make invalid UTF-8, exercising the lossy text decode).  Both sides run the
strict-parity arithmetic (exact encoder and cross K/V)."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from franken_whisper_amd import ggml as W
from oracle import oracle as O
from oracle import transcribe_ref as R

pytestmark = pytest.mark.gpu

DRV = synth.Config("drv", 51864, 1500, 128, 2, 2, 96, 128, 2, 2, 80)
DRV_ML = synth.Config("drv-ml", 51866, 1500, 128, 2, 2, 96, 128, 2, 2, 80)


@pytest.fixture(scope="module")
def setup(ctx):
    out = {}
    for cfg in (DRV, DRV_ML):
        m = synth.Model(cfg, seed=21)
        # make end-of-text and the raw high bytes (invalid UTF-8 alone) likely
        # now and then, so windows end, segments carry text and the lossy
        # decode is exercised
        emb = m.t["decoder.token_embedding.weight"].view(np.float16)
        emb[m.tokens.eot] *= np.float16(10.0)
        emb[128:256] *= np.float16(2.0)
        audio = synth.audio(5, 71.3, gaps=True)
        fb = synth.mel_filterbank(cfg.n_mels)
        enc = native.Encoder(ctx, m, abi.ENC_F32)
        enc.set_exact(True)
        dec = native.Decoder(ctx, m, abi.DEC_F16)
        dec.set_exact(True)
        mel = O.log_mel(audio, fb)
        oenc = O.Encoder(m, abi.ENC_F32)
        cache = {}

        def encode(seek, oenc=oenc, mel=mel, cache=cache, cfg=cfg):
            if seek not in cache:
                cache[seek] = oenc.forward(O.mel_window(mel, seek, 2 * cfg.n_audio_ctx))
            return cache[seek]
        out[cfg.name] = dict(m=m, audio=audio, audio_dev=ctx.array(audio), fb_dev=ctx.array(fb), enc=enc, dec=dec,
                             odec=O.Decoder(m, abi.DEC_F16), encode=encode,
                             vocab=W.synthetic_vocab(m.tokens.eot))
    yield out
    for v in out.values():
        v["enc"].close()
        v["dec"].close()


def _compare(got, want, label):
    gw, ww = got["windows"], want["windows"]
    assert [w["seek_cs"] for w in gw] == [w["seek_cs"] for w in ww], label
    for k, (g, w) in enumerate(zip(gw, ww)):
        tag = f"{label} window {k} (seek {w['seek_cs']})"
        assert g["tokens"] == list(w["tokens"]), tag
        np.testing.assert_array_equal(g["plogs"].view(np.uint32), np.asarray(w["plogs"], np.float32).view(np.uint32),
                                      err_msg=tag)
        for key in ("result_len", "has_ts", "seek_delta_cs", "no_speech", "dropped", "retried"):
            assert g[key] == w[key], f"{tag} {key}: {g[key]} vs {w[key]}"
        assert g["avg_logprob"] == w["avg_logprob"] and g["no_speech_prob"] == w["no_speech_prob"], tag
    assert len(got["segments"]) == len(want["segments"]), label
    for g, w in zip(got["segments"], want["segments"]):
        assert g[:3] == w[:3], f"{label}: {g} vs {w}"
        assert (g[3] is None and w[3] is None) or g[3] == w[3], f"{label}: {g} vs {w}"


CASES = [
    ("no-ts-independent", "drv", dict(timestamps=False, max_context=0)),
    ("no-ts-carry", "drv", dict(timestamps=False)),
    ("ts-carry", "drv-ml", dict(timestamps=True)),
    ("ts-budget", "drv", dict(timestamps=True, max_tokens=6)),
    ("ts-initial-prompt", "drv-ml", dict(timestamps=True, carry_initial_prompt=True,
                                         initial_prompt=[300, 301, 302, 303, 304])),
    ("no-ts-prompt-retry", "drv", dict(timestamps=False, initial_prompt=[300, 301, 302, 303, 304])),
    ("no-ts-gated", "drv", dict(timestamps=False, no_speech_threshold=-1.0, logprob_threshold=50.0)),
    ("ts-no-context", "drv", dict(timestamps=True, no_context=True)),
]


@pytest.mark.parametrize("name,model,kw", CASES, ids=[c[0] for c in CASES])
def test_transcribe_matches_oracle(ctx, setup, name, model, kw):
    s = setup[model]
    m = s["m"]
    tk = m.tokens
    filt = tk.filter()
    sot = tk.sot_sequence(language_id=0, timestamps=kw.get("timestamps", False))
    print(f"transcribe {name}", flush=True)
    got = native.transcribe(ctx, s["enc"], s["dec"], s["audio_dev"], s["audio"].size, s["fb_dev"], m.cfg.n_mels, filt,
                            s["vocab"], sot, **kw)
    p = R.Params(**{k: v for k, v in kw.items()})
    want = R.transcribe(s["encode"], s["odec"], m.cfg, s["audio"].size, filt, sot, s["vocab"], p)
    print(name, [(w["seek_cs"], len(w["tokens"]), w["result_len"], w["no_speech"], w["retried"]) for w in
                 got["windows"]], len(got["segments"]), flush=True)
    _compare(got, want, name)
    assert got["windows"], name


def test_transcribe_rejects_empty_audio(ctx, setup):
    s = setup["drv"]
    tk = s["m"].tokens
    with pytest.raises(native.FwhipError) as e:
        native.transcribe(ctx, s["enc"], s["dec"], s["audio_dev"], 0, s["fb_dev"], 80, tk.filter(), s["vocab"],
                          tk.sot_sequence())
    assert e.value.code == abi.ERR_INVALID and "empty audio" in str(e.value)


@pytest.mark.parametrize("prec", [abi.ENC_F32, abi.ENC_INT8], ids=["f32", "int8"])
def test_exact_encoder_on_silent_gaps_bitexact(ctx, setup, prec):
    """Exact-mode encoder states of the gapped audio's windows against the
    oracle: nearly constant rows (silence) make LayerNorm's f64 statistics
    sensitive to their summation order, which must be the reference's."""
    s = setup["drv"]
    m = s["m"]
    enc = native.Encoder(ctx, m, prec)
    enc.set_exact(True)
    mel = O.log_mel(s["audio"], synth.mel_filterbank(80))
    out = ctx.empty((3, 1500, 128), np.float32)
    enc.forward_mel(ctx.array(mel), mel.shape[1], [0, 3000, 6000], 3000, out)
    got = out.download()
    enc.close()
    oe = O.Encoder(m, prec)
    for w, seek in enumerate((0, 3000, 6000)):
        np.testing.assert_array_equal(got[w].view(np.uint32),
                                      oe.forward(O.mel_window(mel, seek, 3000)).view(np.uint32), err_msg=f"seek {seek}")


@pytest.mark.parametrize("defaults", [False, True], ids=["f16-arm", "reference-defaults"])
def test_transcribe_turbo_timestamps_matches_oracle(ctx, defaults):
    """The window driver at large-v3-turbo scale (32 encoder blocks on the
    int8 plan, 4 decoder layers, both in exact mode): 65 s of seeded audio with
    silent gaps, segment timestamps with the carried prompt (the reference's
    defaults), every window and segment identical to the oracle's
    transcribe_samples_uncached.  On the f16 arm, and with the reference's
    default configuration: ToMe by its rule (500 of 1500 rows after block 3),
    the int8 decoder arm and the f32 self-attention cache."""
    import os

    cfg = synth.TURBO
    m = synth.Model(cfg, seed=4)
    tk = m.tokens
    filt = tk.filter()
    sot = tk.sot_sequence(language_id=0, timestamps=True)
    audio = synth.audio(17, 65.0, gaps=True)
    fb = synth.mel_filterbank(cfg.n_mels)
    vocab = W.synthetic_vocab(tk.eot)
    arm = abi.DEC_INT8 if defaults else abi.DEC_F16
    enc = native.Encoder(ctx, m, abi.ENC_INT8)
    enc.set_exact(True)
    if defaults:
        enc.set_tome(-1, 3)
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(True)
    if defaults:
        dec.set_kv_f16(False)
    print("turbo transcribe", "reference defaults" if defaults else "f16 arm", flush=True)
    try:
        got = native.transcribe(ctx, enc, dec, ctx.array(audio), audio.size, ctx.array(fb), cfg.n_mels, filt, vocab,
                                sot, timestamps=True)
    finally:
        enc.close()
        dec.close()
    lib = O.lib()
    lib.ref_set_num_threads(min(os.cpu_count() or 1, 16))
    try:
        lib.ref_set_fast(1)
        mel = O.log_mel(audio, fb)
        oenc = O.Encoder(m, abi.ENC_INT8)
        odec = O.Decoder(m, arm)
        if defaults:
            odec.set_kv_f16(False)
        cache = {}

        def encode(seek):
            if seek not in cache:
                win = O.mel_window(mel, seek, 2 * cfg.n_audio_ctx)
                cache[seek] = oenc.forward(win, tome_r=500, tome_after=3) if defaults else oenc.forward(win)
            return cache[seek]
        want = R.transcribe(encode, odec, cfg, audio.size, filt, sot, vocab, R.Params(timestamps=True))
    finally:
        lib.ref_set_fast(0)
    print([(w["seek_cs"], len(w["tokens"]), w["result_len"], w["no_speech"], w["retried"]) for w in got["windows"]],
          len(got["segments"]), flush=True)
    _compare(got, want, "turbo ts-carry" + (" reference defaults" if defaults else ""))
    assert got["windows"]
