"""Pins the oracle's log-mel restatement (CPU; src/native_engine/mel.rs).

Each check is fixed by the mathematics or by the reference's own tests, and is
chosen so a plausible restatement mistake fails it:
  - the 400-point two-for-one FFT against numpy's f64 FFT on random, impulse,
    DC and pure-tone frames (a wrong twiddle sign, a swapped even/odd split or
    a dropped term moves some bin by O(1)), and Parseval;
  - log10_floor_approx against log10, exact on powers of two (where the series
    term is 0) and at the 1e-10 floor;
  - the periodic Hann window's closed form and symmetry;
  - n_frames_for values (mel.rs:1127) and the 5 ms / tiny-input cases of
    tiny_inputs_reflect_only_existing_samples and
    log_mel_accepts_a_five_millisecond_window (mel.rs:2473-2498);
  - silence_collapses_to_floor (mel.rs:2283-2297): every value -1.5;
  - sine_440_argmax_matches_analytic_filter_projection (mel.rs:2406): a 440 Hz
    tone peaks in the mel bin with the largest weight on FFT bin 11;
  - the whole pipeline against an independent numpy f64 computation of the
    documented algorithm (reflective lead, 30 s + 200 zero tail, partial frames
    zero-filled past valid_len, floor frames, max - 8 clamp, (x + 4) / 4)."""
import numpy as np
import pytest

from franken_whisper_amd import synth
from oracle import oracle as O

SILENCE = np.float32(-1.5)


def _dummy_filters(n_mel):
    """dummy_filters (mel.rs:2266-2281): one unit weight per mel row."""
    f = np.zeros((n_mel, 201), dtype=np.float32)
    for m in range(n_mel):
        f[m, min(m * 201 // n_mel, 200)] = 1.0
    return f


def test_fft400_matches_numpy_dft():
    rng = np.random.default_rng(5)
    frames = [rng.standard_normal(400).astype(np.float32) for _ in range(6)]
    imp = np.zeros(400, np.float32)
    imp[37] = 1.0
    frames += [imp, np.ones(400, np.float32),
               np.cos(2 * np.pi * 11 * np.arange(400) / 400).astype(np.float32),
               np.sin(2 * np.pi * 173 * np.arange(400) / 400).astype(np.float32)]
    for x in frames:
        got = O.mel_fft400(x)
        want = np.fft.fft(x.astype(np.float64))
        err = np.max(np.abs(got - want)) / max(1.0, np.max(np.abs(want)))
        assert err < 2e-6, err
        # Parseval
        e_t = 400.0 * np.sum(x.astype(np.float64) ** 2)
        e_f = np.sum(np.abs(got) ** 2)
        assert abs(e_f - e_t) <= 1e-5 * e_t + 1e-9


def test_log10_floor_approx():
    xs = np.exp(np.linspace(np.log(1e-10), np.log(1e12), 4001))
    for x in xs:
        got = float(O.log10_floor_approx(x))
        assert abs(got - np.log10(x)) < 1e-6 * max(1.0, abs(np.log10(x))), x
    for k in range(-33, 40):
        x = 2.0 ** k
        if x < 1e-10:
            continue
        want = np.float32(k * 0.6931471805599453 * (1.0 / 2.302585092994046))
        assert O.log10_floor_approx(x) == want, k
    floor = np.float32(np.log10(1e-10))
    assert floor == np.float32(-10.0)
    for x in (0.0, 1e-30, 1e-11, 1e-10):
        assert O.log10_floor_approx(x) == floor


def test_hann_window_periodic():
    h = O.mel_hann()
    i = np.arange(400)
    want = (0.5 * (1.0 - np.cos(2.0 * np.pi * i / 400.0))).astype(np.float32)
    assert np.max(np.abs(h - want)) <= 6e-8
    assert h[0] == 0.0 and h[200] == 1.0
    assert np.array_equal(h[1:200], h[399:200:-1])


@pytest.mark.parametrize("n,frames", [(0, 3000), (1, 3000), (159, 3000), (160, 3001), (80, 3000),
                                      (480000, 6000), (4800000, 33000)])
def test_mel_frames(n, frames):
    assert O.mel_frames(n) == frames


def test_silence_collapses_to_floor():
    out = O.log_mel(np.zeros(16000, np.float32), _dummy_filters(80))
    assert out.shape == (80, O.mel_frames(16000))
    assert np.all(out == SILENCE)
    assert (np.float32(np.log10(1e-10)) + np.float32(4)) / np.float32(4) == SILENCE


def test_sine_440_peaks_in_the_analytic_bin():
    filters = synth.mel_filterbank(80)
    t = np.arange(16000) / 16000.0
    x = (0.5 * np.sin(2 * np.pi * 440.0 * t)).astype(np.float32)
    out = O.log_mel(x, filters)
    want = int(np.argmax(filters[:, 11]))
    for f in range(5, 95):
        assert int(np.argmax(out[:, f])) == want, f


def _numpy_log_mel(samples, filters):
    """The documented algorithm in numpy f64 (an independent restatement)."""
    n = samples.size
    pad = 200
    padded = np.zeros(n + 480000 + 2 * pad, np.float64)
    padded[pad:pad + n] = samples
    refl = min(pad, max(n - 1, 0))
    for j in range(1, refl + 1):
        padded[pad - j] = samples[j]
    valid = n + pad
    nf = (padded.size - 400) // 160
    hann = 0.5 * (1.0 - np.cos(2.0 * np.pi * np.arange(400) / 400.0))
    out = np.full((filters.shape[0], nf), -10.0)
    live = [f for f in range(nf) if f * 160 < valid]
    frames = np.zeros((len(live), 400))
    for i, f in enumerate(live):
        off = f * 160
        avail = min(400, valid - off)
        frames[i, :avail] = hann[:avail] * padded[off:off + avail]
    pw = np.abs(np.fft.rfft(frames, axis=1)) ** 2
    proj = pw @ filters.astype(np.float64).T
    out[:, live] = np.log10(np.maximum(proj, 1e-10)).T
    out = np.maximum(out, out.max() - 8.0)
    return (out + 4.0) / 4.0


@pytest.mark.parametrize("n", [0, 1, 2, 80, 200, 201, 207, 16000, 40000])
def test_log_mel_matches_numpy_pipeline(n):
    rng = np.random.default_rng(n + 3)
    samples = (np.arange(n) + 1.0).astype(np.float32) / max(n, 1) if n <= 207 else \
        (0.3 * rng.standard_normal(n)).astype(np.float32)
    filters = synth.mel_filterbank(128)
    got = O.log_mel(samples, filters)
    want = _numpy_log_mel(samples, filters)
    assert got.shape == want.shape
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) < 2e-4


def test_numpy_pipeline_catches_a_wrong_reflection():
    """Including sample 0 in the reflection (a plausible mistake) is caught."""
    rng = np.random.default_rng(9)
    x = (0.3 * rng.standard_normal(4000)).astype(np.float32)
    filters = synth.mel_filterbank(128)
    got = O.log_mel(x, filters)
    bad = x.copy()
    # shifting the audio one sample right reproduces a reflection that starts at sample 0
    bad = np.concatenate([bad[:1], bad])[: x.size + 1]
    alt = _numpy_log_mel(bad, filters)[:, :4]
    assert np.max(np.abs(got[:, :4] - alt)) > 1e-2
