"""GPU tests of the boundary's smaller contracts: process_logits + argmax over
device logits (decode.rs:702-867, 1708-1790) on adversarial rows, and
cancellation of decoder calls (checkpoint() between prompt rows and sampled
tokens, decode.rs:3566)."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from oracle import oracle as O
from tests.helpers import enc_states, model

pytestmark = pytest.mark.gpu


def _rows(V, rng):
    rows = []
    r = rng.standard_normal(V).astype(np.float32)
    rows.append(r)
    z = np.full(V, -np.inf, np.float32)
    z[100], z[5000] = -0.0, 0.0  # the signed zeros tie: the first index wins
    rows.append(z)
    z = np.full(V, -np.inf, np.float32)
    z[7], z[40000] = 0.0, -0.0
    rows.append(z)
    rows.append(np.full(V, -np.inf, np.float32))  # no candidate: 0
    n = np.full(V, np.nan, np.float32)
    n[33333] = -1e30
    rows.append(n)  # NaN never wins
    t = rng.standard_normal(V).astype(np.float32)
    t[[3000, 2999, 40000]] = 50.0  # a tie across key blocks
    rows.append(t)
    a = rng.standard_normal(V).astype(np.float32)
    a[50257] = 1e9  # a suppressed special token holds the maximum
    rows.append(a)
    return np.stack(rows)


@pytest.mark.parametrize("initial", [False, True])
def test_argmax_logits_edge_cases(ctx, initial):
    tk = synth.Tokens(synth.TURBO)
    V = synth.TURBO.n_vocab
    rows = _rows(V, np.random.default_rng(1))
    rows[-1, tk.eot] = 1e10 if initial else rows[-1, tk.eot]  # eot wins only after the first step
    dev = ctx.array(rows)
    filt = tk.filter()
    got = ctx.argmax_logits(dev, filt, initial)
    want = [O.process_argmax(filt, r, initial) for r in rows]
    assert got.tolist() == want
    raw = ctx.argmax_logits(dev, None, initial)
    assert raw.tolist() == [O.argmax_first(r) for r in rows]
    assert raw[1] == 100 and raw[2] == 7 and raw[3] == 0 and raw[4] == 33333 and raw[5] == 2999


def test_argmax_logits_rejects_bad_shapes(ctx):
    dev = ctx.empty((1, 8), np.float32)
    for n_rows, n_vocab in ((0, 8), (1, 0), (70000, 8)):
        out = np.zeros(max(n_rows, 1), np.int32)
        rc = native.lib().fwhip_argmax_logits(ctx.h, dev.ptr, n_rows, n_vocab, None, 0,
                                              out.ctypes.data_as(native._i32p))
        assert rc == abi.ERR_INVALID


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16], ids=["int8", "f16"])
def test_decoder_cancel_then_resume(ctx, arm):
    m = model("micro", seed=0, encoder=False)
    cfg, tk = m.cfg, m.tokens
    enc = enc_states(3, 2, cfg.n_audio_ctx, cfg.n_text_state)
    dec = native.Decoder(ctx, m, arm)
    st = dec.state(2, cfg.n_audio_ctx)
    st.set_cross(ctx.array(enc))
    want = st.greedy(tk.sot_sequence(), 20, tk.filter())
    # a cancelled greedy call stops between tokens and clears the flag
    st.set_cross(ctx.array(enc))
    ctx.cancel()
    with pytest.raises(native.FwhipError) as e:
        st.greedy(tk.sot_sequence(), 20, tk.filter())
    assert e.value.code == abi.ERR_CANCELLED
    st.set_cross(ctx.array(enc))
    got = st.greedy(tk.sot_sequence(), 20, tk.filter())
    for g, w in zip(got, want):
        np.testing.assert_array_equal(g, w)
    # a cancelled prefill leaves the state at its previous length
    st.reset()
    ctx.cancel()
    with pytest.raises(native.FwhipError) as e:
        st.step(np.tile(tk.sot_sequence(), (2, 1)))
    assert e.value.code == abi.ERR_CANCELLED
    assert st.len == 0
    st.step(np.tile(tk.sot_sequence(), (2, 1)))
    assert st.len == len(tk.sot_sequence())
    st.close()
    dec.close()
