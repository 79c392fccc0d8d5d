"""The decoder's fast mode (the default, and the benchmarked route): the cross
K/V precompute of DecoderState::new (decoder.rs:1040-1222) as one f16-pair
MFMA GEMM over every layer instead of the strict sequential-k f32 GEMM, and
the fragment-order f16 GEMVs with the LayerNorms fused into their staging.

- Cross K/V: more than 99% of the f16 values equal the exact mode's (which is
  bit-identical to the oracle), and every value is within one f16 ulp of it
  plus 1e-3 of the stream's rms.  The f32 sums differ by ~1e-7 of the sum of
  |terms| before the f16 rounding, which is more than one ulp only for values
  near zero.
- The f16 arm: greedy tokens in fast mode identical to the oracle's for the
  micro shapes, tiny.en and the large-v3-turbo decoder with 16 streams.
- The int8 arm re-quantizes every linear's input to int8 (absmax / 127, round
  half away), so a sub-ulp f32 difference upstream moves a rounding boundary
  and greedy tokens can part from the exact ones after a near-tie.  Its fast
  mode is checked by teacher forcing: both modes step along the exact mode's
  token path, and at every position the fast logits are within 3e-2 rms of
  the exact logits and the fast argmax agrees with the exact token at >= 95%
  of the positions (measured 97.7% at turbo with 16 streams, 98.4% on
  tiny.en; the micro model's fast logits are bit-identical to exact mode's,
  which the test requires).  Exact mode itself is bit-identical to the oracle
  on this arm (the deep-cache and greedy tests run it).
"""
import numpy as np
import pytest

from franken_whisper_amd import abi, native
from oracle import oracle as O
from tests.helpers import enc_states, model

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["micro", "large-v3-turbo"])
def test_fast_cross_kv_close_to_exact(ctx, name):
    m = model(name, seed=2, encoder=False)
    cfg = m.cfg
    S = 3
    enc = ctx.array(enc_states(17, S, cfg.n_audio_ctx, cfg.n_text_state))
    out = {}
    for exact in (True, False):
        dec = native.Decoder(ctx, m, abi.DEC_INT8)
        dec.set_exact(exact)
        st = dec.state(S, cfg.n_audio_ctx)
        st.set_cross(enc)
        out[exact] = [(st.read(abi.DS_CROSS_K_F16, s), st.read(abi.DS_CROSS_VT_F16, s)) for s in range(S)]
        st.close()
        dec.close()
    for s in range(S):
        for which in (0, 1):
            e16 = out[True][s][which].view(np.float16)
            f16 = out[False][s][which].view(np.float16)
            e, f = e16.astype(np.float64), f16.astype(np.float64)
            assert np.all(np.isfinite(f))
            same = float(np.mean(out[True][s][which] == out[False][s][which]))
            rms = float(np.sqrt(np.mean(e * e)))
            bound = np.abs(np.spacing(e16)).astype(np.float64) + 1e-3 * rms
            worst = float(np.max(np.abs(f - e) / bound))
            print(f"{name} stream {s} {'KV'[which]}: {same:.5f} identical, worst |d|/bound {worst:.3f}", flush=True)
            assert same > 0.99 and worst <= 1.0


CASES = [("micro-ml", 3, 28), ("tiny.en", 2, 64), ("large-v3-turbo", 16, 48)]


@pytest.mark.parametrize("name,S,n_max", CASES)
def test_fast_mode_f16_arm_greedy_matches_oracle(ctx, name, S, n_max):
    m = model(name, seed=5, encoder=False)
    cfg, tk = m.cfg, m.tokens
    enc = enc_states(23, S, cfg.n_audio_ctx, cfg.n_text_state)
    dec = native.Decoder(ctx, m, abi.DEC_F16)
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(ctx.array(enc))
    got = st.greedy(tk.sot_sequence(), n_max, tk.filter())
    odec = O.Decoder(m, abi.DEC_F16)
    for s in sorted({0, S // 2, S - 1}):
        want = odec.state(enc[s]).greedy(tk.sot_sequence(), n_max, tk.filter())
        print(f"{name} f16 arm stream {s}: {len(want)} tokens", flush=True)
        np.testing.assert_array_equal(got[s], want, err_msg=f"stream {s}")
    st.close()
    dec.close()


def _teacher_forced(ctx, m, arm, exact, enc_dev, S, prompt, path, filt):
    """Step a state of the given mode along token rows path [S, n]; returns the
    logits [n, S, V] and the filtered argmax [n, S] at every position."""
    cfg = m.cfg
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(exact)
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(enc_dev)
    lg = ctx.empty((S, cfg.n_vocab), np.float32)
    logits, am = [], []
    am.append(st.step(np.tile(prompt, (S, 1)), lg, filt, True))
    logits.append(lg.download())
    for i in range(path.shape[1] - 1):
        am.append(st.step(path[:, i:i + 1], lg, filt, False))
        logits.append(lg.download())
    st.close()
    dec.close()
    return np.stack(logits), np.stack(am)


@pytest.mark.parametrize("name,S,n_max", CASES)
def test_fast_mode_int8_arm_teacher_forced(ctx, name, S, n_max):
    m = model(name, seed=5, encoder=False)
    cfg, tk = m.cfg, m.tokens
    enc = enc_states(23, S, cfg.n_audio_ctx, cfg.n_text_state)
    enc_dev = ctx.array(enc)
    filt = tk.filter()
    prompt = np.asarray(tk.sot_sequence(), np.int32)
    # the exact mode's own greedy path, padded with end-of-text after a stream ends
    dec = native.Decoder(ctx, m, abi.DEC_INT8)
    dec.set_exact(True)
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(enc_dev)
    ref = st.greedy(prompt, n_max, filt)
    st.close()
    dec.close()
    n = max(len(r) for r in ref)
    path = np.full((S, n), tk.eot, np.int32)
    for s, r in enumerate(ref):
        path[s, :len(r)] = r
    le, ae = _teacher_forced(ctx, m, abi.DEC_INT8, True, enc_dev, S, prompt, path, filt)
    lf, af = _teacher_forced(ctx, m, abi.DEC_INT8, False, enc_dev, S, prompt, path, filt)
    agree, total, worst = 0, 0, 0.0
    for s, r in enumerate(ref):
        k = len(r)
        # exact mode reproduces its own greedy path under teacher forcing
        np.testing.assert_array_equal(ae[:k, s], r, err_msg=f"stream {s} exact replay")
        for i in range(k):
            e, f = le[i, s].astype(np.float64), lf[i, s].astype(np.float64)
            worst = max(worst, float(np.sqrt(np.mean((f - e) ** 2)) / np.sqrt(np.mean(e * e))))
        agree += int(np.sum(af[:k, s] == r))
        total += k
    print(f"{name} int8 arm fast vs exact: rel rms of logits <= {worst:.2e}; "
          f"argmax agreement {agree}/{total}", flush=True)
    # measured: micro-ml bit-identical (d 128: the fast cross K/V and LayerNorm
    # sums land on the same f32 values), tiny.en 126/128 at 1.3e-2, turbo
    # 750/768 at 2.0e-2 (every linear re-quantizes its input, so sub-ulp
    # differences move int8 rounding steps; exact mode is bit-identical)
    if name == "micro-ml":
        assert np.array_equal(lf.view(np.uint32), le.view(np.uint32))
    assert worst <= 3e-2
    assert agree >= 0.95 * total
