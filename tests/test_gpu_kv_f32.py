"""GPU parity of the f32 self-attention cache (the reference's default,
FW_KV_F16 unset: fwhip_decoder_set_kv_f16(dec, 0); KvCache nn.rs:5097-5416,
attention_decode_step nn.rs:6340-6400) against the oracle's f32 cache, in
exact mode, at the large-v3-turbo decoder shape:

- single steps at cache depths 65, 129, 224 and 447 after prefills (the f16
  arm's batched prefill appends and attends through k_kv_append /
  k_self_attn2), bit for bit with the oracle on both arms, with 1 stream (the
  separate q/k/v GEMV and k_self_attn2) and 10 (the folded k_self_attn_f16q;
  the int8 arm's k_self_attn_fused in both);
- 16 streams through the greedy loop (graph replay) token for token;
- a cohort of 3 against each stream alone;
- the cache itself: layer 0's first row is the k/v projection of the
  embedding, identical in both cache types up to the f16 rounding — the f32
  cache holds values f16 does not represent, and rounding them gives the f16
  cache's bits."""
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
@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16], ids=["int8", "f16"])
def test_turbo_f32_cache_deep_bitexact(ctx, arm, S):
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg = m.cfg
    enc = enc_states(23, S, cfg.n_audio_ctx, cfg.n_text_state)
    toks = _tokens(9 + S, S, 447, cfg.n_vocab)
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(True)
    dec.set_kv_f16(False)
    got = _gpu_run(ctx, dec, enc, toks)
    odec = O.Decoder(m, arm)
    odec.set_kv_f16(False)
    lib = O.lib()
    lib.ref_set_fast(1)
    try:
        for s in sorted({0, S - 1}):
            ost = odec.state(enc[s])
            want = _drive(lambda rows: ost.step(rows[0]), toks[s:s + 1])
            for (n_pre, row), g, w in zip(PLAN, got, want):
                print(f"f32 cache arm {arm} S={S} stream {s} depth {row + 1}", flush=True)
                assert_bitexact(g[s], w, f"f32 cache arm {arm} stream {s} depth {row + 1}")
    finally:
        lib.ref_set_fast(0)
    dec.close()


def test_turbo_f32_cache_greedy_16_streams(ctx):
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg, tk = m.cfg, m.tokens
    S = 16
    enc = enc_states(35, S, cfg.n_audio_ctx, cfg.n_text_state)
    dec = native.Decoder(ctx, m, abi.DEC_F16)
    dec.set_exact(True)
    dec.set_kv_f16(False)
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(ctx.array(enc))
    got = st.greedy(tk.sot_sequence(), 32, tk.filter())
    odec = O.Decoder(m, abi.DEC_F16)
    odec.set_kv_f16(False)
    for s in (0, 15):
        want = odec.state(enc[s]).greedy(tk.sot_sequence(), 32, tk.filter())
        print(f"f32 cache stream {s}: {len(want)} tokens", flush=True)
        np.testing.assert_array_equal(got[s], want, err_msg=f"stream {s}")
    st.close()
    dec.close()


def test_turbo_f32_cache_cohort_matches_alone(ctx):
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg = m.cfg
    S = 3
    enc = enc_states(43, S, cfg.n_audio_ctx, cfg.n_text_state)
    toks = _tokens(4, S, 447, cfg.n_vocab)
    dec = native.Decoder(ctx, m, abi.DEC_F16)
    dec.set_exact(True)
    dec.set_kv_f16(False)
    got = _gpu_run(ctx, dec, enc, toks)
    for s in range(S):
        alone = _gpu_run(ctx, dec, enc[s:s + 1], toks[s:s + 1])
        for (n_pre, row), g, a in zip(PLAN, got, alone):
            assert_bitexact(g[s], a[0], f"f32 cache cohort stream {s} vs alone, depth {row + 1}")
    dec.close()


def test_f32_cache_rows_round_to_the_f16_cache(ctx):
    m = model("large-v3-turbo", seed=2, encoder=False)
    cfg = m.cfg
    enc = enc_states(45, 1, cfg.n_audio_ctx, cfg.n_text_state)
    rows = {}
    for kv16 in (True, False):
        dec = native.Decoder(ctx, m, abi.DEC_F16)
        dec.set_exact(True)
        dec.set_kv_f16(kv16)
        st = dec.state(1, cfg.n_audio_ctx)
        st.set_cross(ctx.array(enc))
        st.step([m.tokens.sot])
        d = cfg.n_text_state
        rows[kv16] = (st.read(abi.DS_KV_K)[:d].copy(), st.read(abi.DS_KV_V)[:d].copy())
        st.close()
        dec.close()
    for (f16, f32) in zip(rows[True], rows[False]):
        assert f32.dtype == np.float32 and f16.dtype == np.uint16
        np.testing.assert_array_equal(f32.astype(np.float16).view(np.uint16), f16)
        assert np.any(f32 != f32.astype(np.float16).astype(np.float32))
