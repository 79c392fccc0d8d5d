"""The benchmarked whole job at large-v3-turbo scale, as bench.py runs it
(transcribe_samples_uncached on its greedy path, decode.rs:2956-3600, with the
windows batched): 300 s of seeded synthetic 16 kHz audio with silent gaps ->
GPU log-mel (128 bins) -> 10 x 30 s windows -> int8-plan encoder in fast mode
-> cross K/V -> a 10-stream greedy decode of 220 tokens on the f16 decoder arm.

Checks:
  - the GPU log-mel of the whole 300 s equals the oracle's bit for bit;
  - every window's tokens equal the job's exact mode (encoder, cross K/V and
    every LayerNorm in the reference's strict-parity arithmetic);
  - windows 0 and 9 in exact mode equal the oracle (its FAST restatement,
    which gives the strict restatement's bits): encoder states bit for bit and
    the 220 tokens;
  - the fast int8 encoder's drift from the oracle after all 32 layers stays
    within 5e-2 relative max-abs and 4e-2 relative RMS (every GEMM
    re-quantizes its input, so fast mode's sub-ulp differences move int8
    rounding steps and grow with depth; measured 3.2e-2 and 2.4e-2 on
    window 0) while the tokens stay identical."""
import os

import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from oracle import oracle as O
from tests.helpers import assert_bitexact, rel_maxabs

pytestmark = pytest.mark.gpu

AUDIO_SEED = 1234
W = 10
N_TOKENS = 220


def _rel_rms(got, want):
    g, w = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.sqrt(np.mean((g - w) ** 2)) / np.sqrt(np.mean(w ** 2)))


def test_turbo_whole_job(ctx):
    cfg = synth.TURBO
    model = synth.Model(cfg, seed=0)
    nf = 2 * cfg.n_audio_ctx
    tk = model.tokens
    filt = tk.filter()
    prompt = tk.sot_sequence(language_id=0)

    samples = synth.audio(AUDIO_SEED, 30.0 * W, gaps=True)
    filters = synth.mel_filterbank(cfg.n_mels)
    mel_frames = native.mel_frames(samples.size)
    mel_dev = ctx.empty((cfg.n_mels, mel_frames), np.float32)
    ctx.log_mel(ctx.array(samples), samples.size, ctx.array(filters), cfg.n_mels, mel_dev)
    offsets = np.arange(W, dtype=np.int64) * nf

    def job(exact):
        enc = native.Encoder(ctx, model, abi.ENC_INT8)
        enc.set_exact(exact)
        states = ctx.empty((W, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
        enc.forward_mel(mel_dev, mel_frames, offsets, nf, states)
        enc.close()
        dec = native.Decoder(ctx, model, abi.DEC_F16)
        dec.set_exact(exact)
        st = dec.state(W, cfg.n_audio_ctx)
        st.set_cross(states)
        toks = st.greedy(prompt, N_TOKENS, filt)
        st.close()
        dec.close()
        host = states.download()
        states.free()
        return host, toks

    fast_states, fast_toks = job(False)
    exact_states, exact_toks = job(True)
    print(f"\nwindow token counts: {[len(t) for t in fast_toks]}")
    for w in range(W):
        assert np.array_equal(fast_toks[w], exact_toks[w]), f"window {w}: fast-mode tokens differ from exact mode"

    lib = O.lib()
    lib.ref_set_num_threads(min(os.cpu_count() or 1, 16))
    try:
        lib.ref_set_fast(1)
        mel = O.log_mel(samples, filters)
        assert_bitexact(mel_dev.download(), mel, "log-mel of 300 s")
        oenc = O.Encoder(model, abi.ENC_INT8)
        odec = O.Decoder(model, abi.DEC_F16)
        for w in (0, W - 1):
            win = np.ascontiguousarray(mel[:, w * nf:(w + 1) * nf].T)
            y = oenc.forward(win)
            assert_bitexact(exact_states[w], y, f"exact-mode encoder states, window {w}")
            drift, rms = rel_maxabs(fast_states[w], y), _rel_rms(fast_states[w], y)
            print(f"window {w}: fast int8 encoder vs oracle after {cfg.n_audio_layer} layers: "
                  f"rel max-abs {drift:.3e}, rel RMS {rms:.3e}")
            assert drift <= 5e-2 and rms <= 4e-2, (w, drift, rms)
            toks = odec.state(y).greedy(prompt, N_TOKENS, filt)
            assert np.array_equal(np.asarray(toks), exact_toks[w]), f"window {w}: tokens differ from the oracle"
    finally:
        lib.ref_set_fast(0)


def test_turbo_job_reference_defaults_exact(ctx):
    """The same job with the reference's defaults together (ToMe by the
    reference's rule, 500 of 1500 rows merged after block 3, tome_r_for in
    encoder.rs:1264-1337; the int8 decoder arm; the f32 self-attention cache,
    FW_KV_F16 unset) in exact mode: windows 0 and 9 equal the oracle's
    encoder states bit for bit and its 220 tokens."""
    cfg = synth.TURBO
    model = synth.Model(cfg, seed=0)
    nf = 2 * cfg.n_audio_ctx
    tk = model.tokens
    filt = tk.filter()
    prompt = tk.sot_sequence(language_id=0)

    samples = synth.audio(AUDIO_SEED, 30.0 * W, gaps=True)
    filters = synth.mel_filterbank(cfg.n_mels)
    mel_frames = native.mel_frames(samples.size)
    mel_dev = ctx.empty((cfg.n_mels, mel_frames), np.float32)
    ctx.log_mel(ctx.array(samples), samples.size, ctx.array(filters), cfg.n_mels, mel_dev)
    offsets = np.arange(W, dtype=np.int64) * nf

    enc = native.Encoder(ctx, model, abi.ENC_INT8)
    enc.set_exact(True)
    enc.set_tome(-1, 3)
    states = ctx.empty((W, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    enc.forward_mel(mel_dev, mel_frames, offsets, nf, states)
    enc.close()
    dec = native.Decoder(ctx, model, abi.DEC_INT8)
    dec.set_exact(True)
    dec.set_kv_f16(False)
    st = dec.state(W, cfg.n_audio_ctx)
    st.set_cross(states)
    toks = st.greedy(prompt, N_TOKENS, filt)
    st.close()
    dec.close()
    host = states.download()
    states.free()
    print(f"\nwindow token counts: {[len(t) for t in toks]}")

    lib = O.lib()
    lib.ref_set_num_threads(min(os.cpu_count() or 1, 16))
    try:
        lib.ref_set_fast(1)
        mel = O.log_mel(samples, filters)
        oenc = O.Encoder(model, abi.ENC_INT8)
        odec = O.Decoder(model, abi.DEC_INT8)
        odec.set_kv_f16(False)
        for w in (0, W - 1):
            win = np.ascontiguousarray(mel[:, w * nf:(w + 1) * nf].T)
            y = oenc.forward(win, tome_r=500, tome_after=3)
            assert_bitexact(host[w], y, f"exact-mode ToMe encoder states, window {w}")
            otoks = odec.state(y).greedy(prompt, N_TOKENS, filt)
            assert np.array_equal(np.asarray(otoks), toks[w]), f"window {w}: tokens differ from the oracle"
    finally:
        lib.ref_set_fast(0)
