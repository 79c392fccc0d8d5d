"""GPU parity of the log-mel frontend (fwhip_log_mel, mel.hip) against the
oracle's restatement of log_mel (src/native_engine/mel.rs:1476-1660): the whole
[n_mel, frames] output bit-exact, on the reference's own edge cases (silence,
5 ms, tiny inputs with partial reflection) and on seeded synthetic speech-like
audio with silent gaps, 30 s and 300 s long, through the C ABI."""
import numpy as np
import pytest

from franken_whisper_amd import native, synth
from oracle import oracle as O
from tests.helpers import assert_bitexact

pytestmark = pytest.mark.gpu


def _run(ctx, samples, filters):
    n = samples.size
    nf = native.mel_frames(n)
    assert nf == O.mel_frames(n)
    s_dev = ctx.array(samples if n else np.zeros(1, np.float32))
    f_dev = ctx.array(filters)
    out = ctx.empty((filters.shape[0], nf), np.float32)
    ctx.log_mel(s_dev, n, f_dev, filters.shape[0], out)
    ctx.synchronize()
    got = out.download()
    for a in (s_dev, f_dev, out):
        a.free()
    return got


@pytest.mark.parametrize("n", [0, 1, 2, 80, 200, 201, 207, 16000])
def test_log_mel_tiny_and_short_inputs_bitexact(ctx, n):
    print(f"log_mel n={n}", flush=True)
    samples = ((np.arange(n) + 1.0) / max(n, 1)).astype(np.float32) if n <= 207 else \
        synth.audio(11, n / 16000.0)
    filters = synth.mel_filterbank(128)
    assert_bitexact(_run(ctx, samples, filters), O.log_mel(samples, filters), f"log_mel n={n}")


def test_log_mel_silence_is_the_floor(ctx):
    filters = np.zeros((80, 201), np.float32)
    for m in range(80):
        filters[m, min(m * 201 // 80, 200)] = 1.0
    got = _run(ctx, np.zeros(16000, np.float32), filters)
    assert np.all(got == np.float32(-1.5))


@pytest.mark.parametrize("seconds,n_mel", [(30.0, 128), (30.0, 80), (300.0, 128)])
def test_log_mel_audio_with_gaps_bitexact(ctx, seconds, n_mel):
    print(f"log_mel {seconds}s n_mel={n_mel}", flush=True)
    samples = synth.audio(23, seconds, gaps=True)
    filters = synth.mel_filterbank(n_mel)
    assert_bitexact(_run(ctx, samples, filters), O.log_mel(samples, filters), f"log_mel {seconds}s")


def test_log_mel_rejects_what_the_reference_rejects(ctx):
    s_dev = ctx.array(np.zeros(100, np.float32))
    f_dev = ctx.array(np.zeros((8, 201), np.float32))
    out = ctx.empty((8, native.mel_frames(100)), np.float32)
    with pytest.raises(native.FwhipError):
        ctx.log_mel(s_dev, 100, f_dev, 8, out, n_fft_bins=200)
    with pytest.raises(native.FwhipError):
        ctx.log_mel(s_dev, 100, f_dev, 0, out)
    for a in (s_dev, f_dev, out):
        a.free()


@pytest.mark.parametrize("cfg", [synth.MICRO, synth.Config("tiny-2L", 51864, 1500, 384, 6, 2, 448, 384, 6, 4, 80)],
                         ids=lambda c: c.name)
def test_audio_to_encoder_states_bitexact(ctx, cfg):
    """The job's seam: audio -> fwhip_log_mel -> fwhip_encoder_forward on windows
    sliced from the device mel (the last one past the end, padded with -1.5) ->
    bit-identical to the oracle's log_mel, window slice and exact-mode encoder."""
    import ctypes

    from franken_whisper_amd import abi

    print(f"audio->encoder {cfg.name}", flush=True)
    m = synth.Model(cfg, seed=5, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    samples = synth.audio(31, 2.0, gaps=True)
    filters = synth.mel_filterbank(cfg.n_mels)
    total = native.mel_frames(samples.size)
    offs = [0, nf, total - nf // 2]
    mel_dev = ctx.empty((cfg.n_mels, total), np.float32)
    ctx.log_mel(ctx.array(samples), samples.size, ctx.array(filters), cfg.n_mels, mel_dev)
    enc = native.Encoder(ctx, m, abi.ENC_INT8)
    enc.set_exact(True)
    out = ctx.empty((len(offs), cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    enc.forward_mel(mel_dev, total, offs, nf, out)
    got = out.download()
    mel = O.log_mel(samples, filters)
    oenc = O.Encoder(m, abi.ENC_INT8)
    for b, off in enumerate(offs):
        win = np.empty((nf, cfg.n_mels), np.float32)
        O.lib().ref_mel_window(abi.ptr(mel, ctypes.c_float), cfg.n_mels, total, off, nf,
                               abi.ptr(win, ctypes.c_float))
        assert_bitexact(got[b], oenc.forward(win), f"{cfg.name} window at frame {off}")
    enc.close()
