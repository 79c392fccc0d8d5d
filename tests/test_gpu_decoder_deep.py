"""GPU decoder parity at the large-v3-turbo decoder shape (4 layers, d 1280,
20 heads, vocab 51866, n_text_ctx 448) deep into the KV cache, on both arms
(the int8 default and the pure-f16 arm with the f16 tied logits head), with 1,
3, 10 and 16 concurrent streams (the f16 arm folds the q/k/v and cross q
projections into its attention kernels at 10 streams and not at 1, 3 or 16, and
runs its cross attention in two launches at 1, 3 and 16 streams, so the
cohort-vs-alone comparison below also holds the folded kernels to the separate
ones bit for bit).

Each stream's cache is filled by prompt prefills through fwhip_decoder_step
(tq > 1) and single steps are checked at cache depths 65, 129, 224 and 447, so
the self-attention kernels run their multi-chunk key loops (more than 64 and
128 keys) and the sequential softmax sums at every length class.  Streams 0 and
S-1 are compared BIT-EXACTLY with the oracle (exact mode: the strict cross
K/V precompute); every stream of the cohort is
compared bit for bit with the same stream decoded alone (the cohort invariant
forward_step_batch_matches_independent_states, decoder.rs:2680, including the
continuation of each stream's private cache)."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from oracle import oracle as O
from tests.helpers import assert_bitexact, enc_states, model

pytestmark = pytest.mark.gpu

# (prefill rows before the checked step, checked step's row index): the step at
# row r attends to r + 1 cached positions
PLAN = [(64, 64), (63, 128), (94, 223), (222, 446)]


def _tokens(seed, S, n, V):
    return synth.uniform_i32(seed, "deep_tokens", 0, V, S * n).reshape(S, n)


def _drive(step, toks):
    """Run PLAN over token rows toks [S, 447]; returns the checked logits."""
    out, r = [], 0
    for n_pre, row in PLAN:
        assert r + n_pre == row
        step(toks[:, r:row])
        out.append(step(toks[:, row:row + 1]))
        r = row + 1
    return out


def _gpu_run(ctx, dec, enc, toks):
    S = toks.shape[0]
    cfg = dec.cfg
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(ctx.array(enc))
    logits = ctx.empty((S, cfg.n_vocab), np.float32)

    def step(rows):
        st.step(rows, logits)
        return logits.download()
    out = _drive(step, toks)
    st.close()
    return out


@pytest.mark.parametrize("S", [1, 3, 10, 16])
@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16], ids=["int8", "f16"])
def test_turbo_deep_cache_bitexact(ctx, arm, S):
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg = m.cfg
    enc = enc_states(21, S, cfg.n_audio_ctx, cfg.n_text_state)
    toks = _tokens(5 + S, S, 447, cfg.n_vocab)
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(True)
    got = _gpu_run(ctx, dec, enc, toks)
    odec = O.Decoder(m, arm)
    for s in sorted({0, S - 1}):
        ost = odec.state(enc[s])
        want = _drive(lambda rows: ost.step(rows[0]), toks[s:s + 1])
        for (n_pre, row), g, w in zip(PLAN, got, want):
            print(f"arm {arm} S={S} stream {s} depth {row + 1}", flush=True)
            assert_bitexact(g[s], w, f"arm {arm} stream {s} cache depth {row + 1}")
    if S > 1:
        for s in range(1, S - 1):
            alone = _gpu_run(ctx, dec, enc[s:s + 1], toks[s:s + 1])
            for (n_pre, row), g, a in zip(PLAN, got, alone):
                assert_bitexact(g[s], a[0], f"arm {arm} cohort stream {s} vs alone, depth {row + 1}")
    dec.close()


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16], ids=["int8", "f16"])
def test_turbo_greedy_16_streams_match_oracle(ctx, arm):
    """Config 3's cohort through the greedy loop: 16 streams, the turbo prompt
    [sot, en, transcribe, notimestamps], 32 sampled tokens; streams 0, 7 and 15
    against the oracle token for token."""
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg, tk = m.cfg, m.tokens
    S = 16
    enc = enc_states(33, S, cfg.n_audio_ctx, cfg.n_text_state)
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(True)
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(ctx.array(enc))
    got = st.greedy(tk.sot_sequence(), 32, tk.filter())
    odec = O.Decoder(m, arm)
    for s in (0, 7, 15):
        want = odec.state(enc[s]).greedy(tk.sot_sequence(), 32, tk.filter())
        print(f"arm {arm} stream {s}: {len(want)} tokens", flush=True)
        np.testing.assert_array_equal(got[s], want, err_msg=f"stream {s}")
    st.close()
    dec.close()


def test_cohort_continuation_after_batched_step(ctx):
    """decoder.rs:2680 second half: after a batched step, each stream's private
    cache continues exactly as a stream that stepped alone."""
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg = m.cfg
    S = 3
    enc = enc_states(41, S, cfg.n_audio_ctx, cfg.n_text_state)
    dec = native.Decoder(ctx, m, abi.DEC_INT8)
    dec.set_exact(True)
    coh = dec.state(S, cfg.n_audio_ctx)
    coh.set_cross(ctx.array(enc))
    lg = ctx.empty((S, cfg.n_vocab), np.float32)
    coh.step(np.array([[3], [5], [7]]), lg)
    coh.step(np.full((S, 1), 11), lg)
    got = lg.download()
    for s, t in enumerate((3, 5, 7)):
        one = dec.state(1, cfg.n_audio_ctx)
        one.set_cross(ctx.array(enc[s:s + 1]))
        l1 = ctx.empty((1, cfg.n_vocab), np.float32)
        one.step([[t]], l1)
        one.step([[11]], l1)
        assert_bitexact(got[s], l1.download()[0], f"stream {s} continuation")
        one.close()
    coh.close()
    dec.close()
