"""GPU parity of the decoder step against the oracle (the CPU restatement of
the reference's decoder, src/native_engine/decoder.rs + nn.rs).

Both arms are built to reproduce the reference's per-output arithmetic order,
so logits are compared BIT-EXACTLY in exact mode (the strict cross K/V
precompute, and every LayerNorm's f64 sums in the reference's sequential
order)."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native
from oracle import oracle as O
from tests.helpers import assert_bitexact, enc_states, model

pytestmark = pytest.mark.gpu


def _run_steps(ctx, name, arm, n_streams, n_steps, seed=0, T=None):
    m = model(name, seed=seed, encoder=False)
    cfg = m.cfg
    T = T or cfg.n_audio_ctx
    enc = enc_states(seed + 7, n_streams, T, cfg.n_text_state)
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(True)
    st = dec.state(n_streams, T)
    st.set_cross(ctx.array(enc))
    logits_dev = ctx.empty((n_streams, cfg.n_vocab), np.float32)
    odec = O.Decoder(m, arm)
    ostates = [odec.state(enc[s]) for s in range(n_streams)]
    tk = m.tokens
    prompt = tk.sot_sequence()
    rng = np.random.default_rng(seed)
    filt = tk.filter()
    # prefill (tq > 1)
    am = st.step(np.tile(prompt, (n_streams, 1)), logits_dev, filt, initial=True)
    got = logits_dev.download()
    for s in range(n_streams):
        want = ostates[s].step(prompt)
        print(f"{name} arm={arm} stream={s} prefill", flush=True)
        assert_bitexact(got[s], want, f"{name} arm={arm} stream {s} prefill logits")
        assert am[s] == O.process_argmax(filt, want, True)
    for k in range(n_steps):
        toks = rng.integers(0, cfg.n_vocab, size=n_streams).astype(np.int32)
        am = st.step(toks[:, None], logits_dev, filt, initial=False)
        got = logits_dev.download()
        for s in range(n_streams):
            want = ostates[s].step([int(toks[s])])
            assert_bitexact(got[s], want, f"{name} arm={arm} stream {s} step {k}")
            assert am[s] == O.process_argmax(filt, want, False)
    for x in (st, dec):
        x.close()


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16])
def test_micro_step_bitexact(ctx, arm):
    _run_steps(ctx, "micro", arm, n_streams=1, n_steps=6)


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16])
def test_micro_multilingual_cohort_bitexact(ctx, arm):
    _run_steps(ctx, "micro-ml", arm, n_streams=3, n_steps=4, seed=3)


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16])
def test_tiny_en_step_bitexact(ctx, arm):
    _run_steps(ctx, "tiny.en", arm, n_streams=2, n_steps=3, seed=1)


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16])
def test_micro_wide_cohort_bitexact(ctx, arm):
    # 18 streams: the per-call stream chunking (16) and several stream groups
    # of the block GEMV
    _run_steps(ctx, "micro", arm, n_streams=18, n_steps=2, seed=4)


@pytest.mark.parametrize("n_streams", [1, 10])
def test_turbo_step_bitexact_int8(ctx, n_streams):
    _run_steps(ctx, "large-v3-turbo", abi.DEC_INT8, n_streams=n_streams, n_steps=2, seed=2)


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16])
def test_greedy_tokens_match(ctx, arm):
    m = model("micro-ml", seed=5, encoder=False)
    cfg = m.cfg
    S, T = 3, cfg.n_audio_ctx
    enc = enc_states(11, S, T, cfg.n_text_state)
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(True)
    st = dec.state(S, T)
    st.set_cross(ctx.array(enc))
    tk = m.tokens
    n_max = cfg.n_text_ctx // 2 - 4
    got = st.greedy(tk.sot_sequence(), n_max, tk.filter())
    odec = O.Decoder(m, arm)
    for s in range(S):
        want = odec.state(enc[s]).greedy(tk.sot_sequence(), n_max, tk.filter())
        np.testing.assert_array_equal(got[s], want, err_msg=f"stream {s}")
    st.close()
    dec.close()


def test_step_rejects_bad_token_and_overflow(ctx):
    m = model("micro", seed=0, encoder=False)
    dec = native.Decoder(ctx, m, abi.DEC_INT8)
    st = dec.state(1, m.cfg.n_audio_ctx)
    st.set_cross(ctx.array(enc_states(1, 1, m.cfg.n_audio_ctx, m.cfg.n_text_state)))
    with pytest.raises(native.FwhipError) as e:
        st.step([[m.cfg.n_vocab]])
    assert e.value.code == abi.ERR_INVALID
    with pytest.raises(native.FwhipError) as e:
        st.step([list(range(m.cfg.n_text_ctx + 1))])
    assert e.value.code == abi.ERR_INVALID
    st.close()
    dec.close()
