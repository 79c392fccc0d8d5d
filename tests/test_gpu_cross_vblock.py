"""GPU parity of the block-int8 cross V (FW_CROSS_V_BLOCK: fwhip_decoder_set_cross_v_block;
decoder.rs:1249-1263, 1605-1608) on the int8 arm at the large-v3-turbo decoder
shape, against the oracle's arm:

- exact mode, single steps at cache depths 65, 129, 224 and 447 after
  prefills, bit for bit, with 1 and 10 streams (1500 frames: 46 full 32-frame
  blocks and a 28-frame tail block, so the value pass takes both dot shapes);
- 16 streams through the greedy loop, token for token;
- fast mode (the block copy made from the fast cross K/V precompute): the
  prompt's logits within the int8 arm's fast-mode bound (3e-2 rms) of exact
  mode's."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native
from oracle import oracle as O
from tests.helpers import assert_bitexact, enc_states, model
from tests.test_gpu_decoder_deep import PLAN, _drive, _tokens

pytestmark = pytest.mark.gpu


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


@pytest.mark.parametrize("S", [1, 10])
def test_turbo_block_v_deep_bitexact(ctx, S):
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg = m.cfg
    enc = enc_states(25, S, cfg.n_audio_ctx, cfg.n_text_state)
    toks = _tokens(12 + S, S, 447, cfg.n_vocab)
    dec = native.Decoder(ctx, m, abi.DEC_INT8)
    dec.set_exact(True)
    dec.set_cross_v_block(True)
    got = _gpu_run(ctx, dec, enc, toks)
    odec = O.Decoder(m, abi.DEC_INT8)
    odec.set_cross_v_block(True)
    lib = O.lib()
    lib.ref_set_fast(1)
    try:
        for s in sorted({0, S - 1}):
            ost = odec.state(enc[s])
            want = _drive(lambda rows: ost.step(rows[0]), toks[s:s + 1])
            for (n_pre, row), g, w in zip(PLAN, got, want):
                print(f"block V S={S} stream {s} depth {row + 1}", flush=True)
                assert_bitexact(g[s], w, f"block V stream {s} depth {row + 1}")
    finally:
        lib.ref_set_fast(0)
    # and the arm is live: the per-row int8 V gives other logits
    dec2 = native.Decoder(ctx, m, abi.DEC_INT8)
    dec2.set_exact(True)
    other = _gpu_run(ctx, dec2, enc, toks)
    assert any(not np.array_equal(a, b) for a, b in zip(got, other))
    dec.close()
    dec2.close()


def test_turbo_block_v_greedy_16_streams(ctx):
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg, tk = m.cfg, m.tokens
    S = 16
    enc = enc_states(37, S, cfg.n_audio_ctx, cfg.n_text_state)
    dec = native.Decoder(ctx, m, abi.DEC_INT8)
    dec.set_exact(True)
    dec.set_cross_v_block(True)
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(ctx.array(enc))
    got = st.greedy(tk.sot_sequence(), 32, tk.filter())
    st.close()
    odec = O.Decoder(m, abi.DEC_INT8)
    odec.set_cross_v_block(True)
    for s in (0, 15):
        want = odec.state(enc[s]).greedy(tk.sot_sequence(), 32, tk.filter())
        print(f"block V stream {s}: {len(want)} tokens", flush=True)
        np.testing.assert_array_equal(got[s], want, err_msg=f"stream {s}")
    # fast mode (the f16-pair cross K/V precompute, tree LayerNorm sums): the
    # prompt's logits within the int8 arm's fast-mode bound of exact mode's
    lg = {}
    for exact in (True, False):
        dec.set_exact(exact)
        st = dec.state(S, cfg.n_audio_ctx)
        st.set_cross(ctx.array(enc))
        out = ctx.empty((S, cfg.n_vocab), np.float32)
        st.step(np.tile(np.asarray(tk.sot_sequence(), np.int32), (S, 1)), out)
        lg[exact] = out.download().astype(np.float64)
        st.close()
    rel = np.sqrt(np.mean((lg[False] - lg[True]) ** 2)) / np.sqrt(np.mean(lg[True] ** 2))
    print(f"block V fast vs exact prompt logits: rel rms {rel:.2e}", flush=True)
    assert rel <= 3e-2
    dec.close()
