"""Pins how the oracle composes its primitives (CPU only).

The primitives are pinned in test_oracle_primitives.py.  Here the composed
functions — ref_encoder_forward (conv stem, blocks, ln_post), ref_dstate_new
(cross K/V), ref_decoder_step (embedding, causal self-attention over the f16
cache, cross-attention, MLP, final LayerNorm, tied logits) and ref_decode_greedy
— are compared against tests/textbook.py, an independent float64 Whisper written
from the published architecture.  Tolerances:

  f32 encoder / f16 decoder arm: max-abs <= 1e-3 relative (the tolerance the
      parity contract uses for f32 outputs) and RMS <= 3e-4 relative; identical
      argmax and greedy tokens.  The residual is the reference GELU's f16 table
      turning sub-ulp f32-vs-f64 differences into one-f16-ulp steps.
  int8 arms: RMS <= 6e-2 relative (int8 quantization noise), identical argmax
      and greedy tokens on these seeds.

test_planted_mistakes_are_detected shows the comparison is sensitive: the
textbook with one named mistake (a dropped bias, a misplaced attention scale,
reversed conv taps, a missing causal mask, ...) lands far outside the
tolerance.  Two mistakes are invisible by construction and are asserted to be
so (a key bias adds a per-query constant to every score, which the softmax
cancels; an erf GELU differs from the tanh GELU by less than the f16 table's
rounding and is pinned instead by the table's known values).

Then the reference's own invariants, restated against the oracle:
  nn.rs:8472  attention_matches_single_head_reference (and the multi-head merge
              and causal-mask properties next to it);
  nn.rs:8559  kv_cache_incremental_equals_full_recompute;
  decoder.rs:2726  incremental_equals_batch_for_last_logits;
  decoder.rs:2997  qkv_fusion_bit_identity_int8_decode_and_f16_prefill.
(decoder.rs:2680, cohort == independent states, is a property of a batched
step, which the oracle does not have; the GPU tests hold the cohort step to it.)
"""
import numpy as np
import pytest

from franken_whisper_amd import abi, synth
from oracle import oracle as O
from tests import textbook as TB
from tests.helpers import rel_maxabs

TINY2 = synth.Config("tiny-2L", 51864, 1500, 384, 6, 2, 448, 384, 6, 4, 80)
ENC_CFGS = [synth.MICRO, TINY2]
DEC_CASES = [("micro", 3), ("micro-ml", 5), ("tiny.en", 1)]


def rms(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.sqrt(np.mean((got - want) ** 2)) / np.sqrt(np.mean(want ** 2)))


# ---- encoder -------------------------------------------------------------------
_enc_cache = {}


def _enc_case(cfg):
    if cfg.name not in _enc_cache:
        m = synth.Model(cfg, seed=2, decoder=False)
        x = synth.mel_input(3, 1, 2 * cfg.n_audio_ctx, cfg.n_mels)[0]
        _enc_cache[cfg.name] = (m, x, O.Encoder(m, abi.ENC_F32).forward(x),
                                O.Encoder(m, abi.ENC_INT8).forward(x))
    return _enc_cache[cfg.name]


@pytest.mark.parametrize("cfg", ENC_CFGS, ids=lambda c: c.name)
def test_encoder_f32_matches_textbook(cfg):
    m, x, want, _ = _enc_case(cfg)
    tb = TB.Encoder(m).forward(x)
    e_max, e_rms = rel_maxabs(want, tb), rms(want, tb)
    print(f"{cfg.name} f32 encoder vs textbook: max-abs {e_max:.2e} rms {e_rms:.2e}")
    assert e_max <= 1e-3 and e_rms <= 3e-4


@pytest.mark.parametrize("cfg", ENC_CFGS, ids=lambda c: c.name)
def test_encoder_int8_matches_textbook_within_int8_noise(cfg):
    m, x, want32, want8 = _enc_case(cfg)
    tb = TB.Encoder(m).forward(x)
    e8 = rms(want8, tb)
    print(f"{cfg.name} int8 encoder vs textbook: rms {e8:.2e}")
    assert e8 <= 6e-2
    # the int8 plan is a quantization of the same network, not another one
    assert rms(want8, want32) <= 6e-2


@pytest.mark.parametrize("cfg", ENC_CFGS, ids=lambda c: c.name)
def test_encoder_partial_depth_matches_textbook(cfg):
    """conv stem + ln_post alone (no blocks), then one block: the stem's tap
    order, stride and GELU, and the positional embedding, without the blocks
    averaging anything out."""
    m, x, _, _ = _enc_case(cfg)
    oe = O.Encoder(m, abi.ENC_F32)
    for n in (0, 1):
        want = oe.forward(x, n)
        tb = TB.Encoder(m).forward(x, n_layers=n)
        assert rel_maxabs(want, tb) <= 1e-3 and rms(want, tb) <= 3e-4, n


# ---- decoder -------------------------------------------------------------------
def _dec_case(name, seed):
    m = synth.Model(synth.CONFIGS[name], seed=seed, encoder=False)
    enc = synth.encoder_states(seed + 7, 1, m.cfg.n_audio_ctx, m.cfg.n_text_state)[0]
    toks = np.random.default_rng(seed).integers(0, m.cfg.n_vocab, size=6)
    return m, enc, toks


def _logit_run(state, prompt, toks):
    out = [state.step(prompt)]
    for t in toks:
        out.append(state.step([int(t)]))
    return out


@pytest.mark.parametrize("name,seed", DEC_CASES)
@pytest.mark.parametrize("arm", [abi.DEC_F16, abi.DEC_INT8], ids=["f16", "int8"])
def test_decoder_steps_match_textbook(name, seed, arm):
    m, enc, toks = _dec_case(name, seed)
    prompt = m.tokens.sot_sequence()
    want = _logit_run(O.Decoder(m, arm).state(enc), prompt, toks)
    got = _logit_run(TB.Decoder(m).state(enc), prompt, toks)
    for i, (w, g) in enumerate(zip(want, got)):
        e_max, e_rms = rel_maxabs(w, g), rms(w, g)
        print(f"{name} arm {arm} row {i}: max-abs {e_max:.2e} rms {e_rms:.2e}")
        if arm == abi.DEC_F16:
            assert e_max <= 1e-3 and e_rms <= 3e-4, i
            assert int(np.argmax(w)) == int(np.argmax(g)), i
        else:
            assert e_rms <= 6e-2, i
            # argmax agrees up to the int8 noise: the oracle's pick is within
            # three noise standard deviations of the textbook's maximum
            noise = np.sqrt(np.mean((np.asarray(w, np.float64) - g) ** 2))
            assert g[int(np.argmax(w))] >= np.max(g) - 3 * noise, i


def test_cross_kv_precompute_matches_textbook():
    """DecoderState::new: K scaled by d_head^-1/4 and V + bias, per head, as f16
    (K [L, H, T, 64], V transposed [L, H, 64, T]) — within one f16 rounding of
    the float64 values."""
    m, enc, _ = _dec_case("micro", 3)
    cfg = m.cfg
    st = O.Decoder(m, abi.DEC_F16).state(enc)
    L, H, T, d = cfg.n_text_layer, cfg.n_text_head, cfg.n_audio_ctx, cfg.n_text_state
    dh = d // H
    ck = TB.w16(st.cross_k_f16()).reshape(L, H, T, dh)
    cvt = TB.w16(st.cross_vt_f16()).reshape(L, H, dh, T)
    tbd = TB.Decoder(m, TB.Numerics(cross_f16=False))
    for li in range(L):
        p = f"decoder.blocks.{li}.cross_attn"
        k = tbd.linear(np.asarray(enc, np.float64), p + ".key", bias=False) * dh ** -0.25
        v = tbd.linear(np.asarray(enc, np.float64), p + ".value")
        for h in range(H):
            kk, vv = k[:, h * dh:(h + 1) * dh], v[:, h * dh:(h + 1) * dh].T
            for got, want in ((ck[li, h], kk), (cvt[li, h], vv)):
                ulp = np.spacing(np.abs(want).astype(np.float16)).astype(np.float64)
                assert np.all(np.abs(got - want) <= ulp), (li, h)
                assert np.mean(got == TB.f16(want)) > 0.995, (li, h)


@pytest.mark.parametrize("name,seed", [("micro-ml", 5), ("tiny.en", 1)])
@pytest.mark.parametrize("arm", [abi.DEC_F16, abi.DEC_INT8], ids=["f16", "int8"])
def test_greedy_tokens_match_textbook(name, seed, arm):
    m, enc, _ = _dec_case(name, seed)
    tk, cfg = m.tokens, m.cfg
    n_max = 24 if name == "tiny.en" else cfg.n_text_ctx // 2 - 4
    want = O.Decoder(m, arm).state(enc).greedy(tk.sot_sequence(), n_max, tk.filter())
    got = TB.Decoder(m).state(enc).greedy(tk.sot_sequence(), n_max, TB.NoTimestampsFilter(tk, cfg.n_vocab))
    np.testing.assert_array_equal(want, got)


# ---- sensitivity: planted mistakes in the textbook ----------------------------------
ENC_MUTATIONS = ["no_q_bias", "no_v_bias", "no_o_bias", "no_fc1_bias", "no_fc2_bias", "attn_unscaled",
                 "attn_scale_full_k", "conv_taps_reversed", "conv2_stride1_even", "no_pos_emb", "no_ln_post",
                 "ln_eps_1e-3"]
DEC_MUTATIONS = ["no_q_bias", "no_v_bias", "no_o_bias", "no_fc1_bias", "no_fc2_bias", "attn_unscaled",
                 "attn_scale_full_k", "no_causal_mask", "cross_k_unscaled", "no_cross_v_bias", "no_final_ln",
                 "pos_emb_shift", "ln_eps_1e-3"]
INVISIBLE = ["k_bias_from_q", "gelu_erf"]


@pytest.mark.parametrize("mutation", ENC_MUTATIONS)
def test_planted_mistakes_are_detected_encoder(mutation):
    m, x, want, _ = _enc_case(TINY2)
    base = rms(want, TB.Encoder(m).forward(x))
    bad = rms(want, TB.Encoder(m, TB.Numerics(mutate=mutation)).forward(x))
    print(f"{mutation}: rms {bad:.2e} vs correct {base:.2e}")
    assert bad > max(3 * base, 9e-4)


@pytest.mark.parametrize("mutation", DEC_MUTATIONS)
def test_planted_mistakes_are_detected_decoder(mutation):
    m, enc, toks = _dec_case("micro", 3)
    prompt = m.tokens.sot_sequence()
    want = _logit_run(O.Decoder(m, abi.DEC_F16).state(enc), prompt, toks[:2])
    base = max(rms(w, g) for w, g in zip(want, _logit_run(TB.Decoder(m).state(enc), prompt, toks[:2])))
    got = _logit_run(TB.Decoder(m, TB.Numerics(mutate=mutation)).state(enc), prompt, toks[:2])
    bad = max(rms(w, g) for w, g in zip(want, got))
    print(f"{mutation}: rms {bad:.2e} vs correct {base:.2e}")
    assert bad > max(3 * base, 9e-4)


@pytest.mark.parametrize("mutation", INVISIBLE)
def test_invisible_mutations_stay_within_tolerance(mutation):
    m, x, want, _ = _enc_case(TINY2)
    tb = TB.Encoder(m, TB.Numerics(mutate=mutation)).forward(x)
    assert rel_maxabs(want, tb) <= 1e-3


# ---- the reference's invariants, restated against the oracle ------------------------
def _max_rel_err(a, b):
    """The reference tests' max_rel_err (nn.rs:7142-7157): 0 within an absolute
    floor of 1e-5, else |a-b| / max(|a|, |b|, 1e-6)."""
    a, b = np.asarray(a, np.float32).ravel(), np.asarray(b, np.float32).ravel()
    d = np.abs(a - b)
    den = np.maximum(np.maximum(np.abs(a), np.abs(b)), 1e-6)
    return float(np.max(np.where(d <= 1e-5, 0.0, d / den)))


def _naive_attention(q, k, v, n_head, causal=False, cache_len=0):
    """Single-head-by-head float64 attention, softmax(q k^T / sqrt(dh)) v."""
    return TB.mha(np.asarray(q, np.float64), np.asarray(k, np.float64), np.asarray(v, np.float64), n_head,
                  TB.Numerics(), causal_offset=cache_len if causal else None)


def test_attention_matches_single_head_reference():
    """nn.rs:8472 (single head, 5 x 7 x 8) and nn.rs:8482 (4 heads of 6)."""
    rng = np.random.default_rng(6)
    q, k, v = (rng.uniform(-1, 1, (n, 8)).astype(np.float32) for n in (5, 7, 7))
    assert _max_rel_err(O.attention(q, k, v, 1), _naive_attention(q, k, v, 1)) < 1e-4
    q, k, v = (rng.uniform(-1, 1, (n, 24)).astype(np.float32) for n in (3, 5, 5))
    assert _max_rel_err(O.attention(q, k, v, 4), _naive_attention(q, k, v, 4)) < 1e-4
    # Whisper's head width, a long key axis
    q, k, v = (rng.standard_normal((n, 128)).astype(np.float32) for n in (9, 300, 300))
    assert _max_rel_err(O.attention(q, k, v, 2), _naive_attention(q, k, v, 2)) < 1e-4


def test_attention_causal_mask_property():
    """nn.rs:8520: perturbing the last key/value changes only the last query's
    row; and the masked result equals the float64 causal attention."""
    rng = np.random.default_rng(8)
    q, k, v = (rng.uniform(-1, 1, (4, 8)).astype(np.float32) for _ in range(3))
    a = O.attention(q, k, v, 2, causal=True)
    assert _max_rel_err(a, _naive_attention(q, k, v, 2, causal=True)) < 1e-4
    k2, v2 = k.copy(), v.copy()
    k2[-1] += 5.0
    v2[-1] += 5.0
    b = O.attention(q, k2, v2, 2, causal=True)
    assert np.all(np.abs(a[:-1] - b[:-1]) < 1e-6)
    assert np.any(np.abs(a[-1] - b[-1]) > 1e-4)


def test_kv_cache_incremental_equals_full_recompute():
    """nn.rs:8559: one row at a time through the f16 cache == causal attention
    over all rows at once.  K and V are f16-representable so the cache's f16
    storage loses nothing; the bound is the reference test's 1e-4."""
    rng = np.random.default_rng(9)
    n_head, dh, n = 3, 64, 5
    d = n_head * dh
    q = rng.uniform(-1, 1, (n, d)).astype(np.float32)
    k = TB.f16(rng.uniform(-1, 1, (n, d))).astype(np.float32)
    v = TB.f16(rng.uniform(-1, 1, (n, d))).astype(np.float32)
    full = O.attention(q, k, v, n_head, causal=True)
    k16, v16 = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    inc = np.stack([O.attention_decode_f16(q[t], k16[: t + 1], v16[: t + 1], n_head) for t in range(n)])
    assert _max_rel_err(inc, full) < 1e-4


@pytest.mark.parametrize("arm", [abi.DEC_F16, abi.DEC_INT8], ids=["f16", "int8"])
def test_incremental_equals_batch_for_last_logits(arm):
    """decoder.rs:2726: [a] then [b] vs [a, b] in one call — the last logits
    within 1e-4.  On the int8 arm a prompt's mlp_2 takes the f16 batch weights
    (the block-int8 GEMV has no batch form) while a single step takes the block
    int8 ones, so the two differ by int8 noise there; the f16 arm is bit-equal."""
    m, enc, _ = _dec_case("micro", 3)
    dec = O.Decoder(m, arm)
    a, b = 3, 5
    s1 = dec.state(enc)
    s1.step([a])
    inc = s1.step([b])
    batch = dec.state(enc).step([a, b])
    if arm == abi.DEC_F16:
        assert np.max(np.abs(inc - batch)) < 1e-4
        assert np.array_equal(inc.view(np.uint32), batch.view(np.uint32))
    else:
        assert rms(inc, batch) < 6e-2


def test_qkv_fusion_bit_identity():
    """decoder.rs:2997: the fused [q; k; v] projection (rows quantized together,
    bias [q_b | 0 | v_b]) equals the three separate projections bit for bit, on
    the int8 GEMV and the f16 GEMV, at width 64 and 384."""
    for n, tag in ((64, 1), (384, 11)):
        rng = np.random.default_rng(tag)
        ws = [TB.f16(rng.uniform(-0.05, 0.05, (n, n))).astype(np.float16).view(np.uint16) for _ in range(3)]
        bq, bv = rng.uniform(-0.05, 0.05, n).astype(np.float32), rng.uniform(-0.05, 0.05, n).astype(np.float32)
        fused = np.concatenate(ws)
        fb = np.concatenate([bq, np.zeros(n, np.float32), bv])
        qf, sf = O.quantize_f16_to_i8(fused)
        parts = [O.quantize_f16_to_i8(w) for w in ws]
        for _ in range(3):
            x = rng.uniform(-0.5, 0.5, n).astype(np.float32)
            yf = O.gemv_i8(qf, sf, x, fb)
            ys = np.concatenate([O.gemv_i8(q, s, x, b) for (q, s), b in zip(parts, (bq, None, bv))])
            assert np.array_equal(yf.view(np.uint32), ys.view(np.uint32))
            yf = O.gemv_f16(fused, x, fb)
            ys = np.concatenate([O.gemv_f16(w, x, b) for w, b in zip(ws, (bq, None, bv))])
            assert np.array_equal(yf.view(np.uint32), ys.view(np.uint32))
