"""The encoder's execution record (EncoderExecution, encoder.rs:1987-2003)
and the f16-pair range guard.

- The record names the route, the arithmetic of each GEMM family
  (EncoderPrecision, encoder.rs:1929-1985) and what chose it, in both modes
  and on both plans: fast mode runs the conv stem and attention (and on the
  f32 plan every linear) as f16-pair MFMA products, and says so.
- A fast forward whose f16-pair operands meet a value past the f16 range
  (|v| >= 65520: a conv activation, an f32-plan LayerNorm output, a q/k/v
  value) runs again in exact mode: the record says "f16_pair_range" and the
  states are bit-identical to the oracle's strict-parity encoder, where an
  unguarded pair would have produced inf / NaN.
- The decoder's fast cross K/V precompute falls back to the strict GEMM on
  encoder states past the f16 range: its K / V^T equal exact mode's."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from oracle import oracle as O
from tests.helpers import assert_bitexact, enc_states

pytestmark = pytest.mark.gpu

F16P, F32, I7, I8 = abi.PREC_F16_PAIR, abi.PREC_F32, abi.PREC_I7, abi.PREC_I8
EXPECT = {  # (plan, exact) -> conv_stem, attn_qkv, attention, attn_out, mlp_fc1, mlp_fc2
    (abi.ENC_INT8, False): [F16P, I7, F16P, I8, I7, I7],
    (abi.ENC_INT8, True): [F32, I7, F32, I8, I7, I7],
    (abi.ENC_F32, False): [F16P] * 6,
    (abi.ENC_F32, True): [F32] * 6,
}


def _forward(ctx, m, precision, exact, n_windows=2, seed=3):
    cfg = m.cfg
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(seed, n_windows, nf, cfg.n_mels)
    enc = native.Encoder(ctx, m, precision)
    enc.set_exact(exact)
    out = ctx.empty((n_windows, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    rec = enc.forward_time_major(ctx.array(x), n_windows, nf, out)
    got = out.download()
    enc.close()
    return x, got, rec


def test_gemm_precision_strings():
    lib = native.lib()
    names = [lib.fwhip_gemm_precision_str(i).decode() for i in range(9)]
    # GemmPrecision::as_str (encoder.rs:1912-1927), then this engine's f16 pair
    assert names == ["f32", "i7", "i8", "f16", "f16_weights", "q8_0_weights", "f16_kv", "mixed", "f16_pair"]
    assert lib.fwhip_gemm_precision_str(9) is None and lib.fwhip_gemm_precision_str(-1) is None


@pytest.mark.parametrize("exact", [False, True], ids=["fast", "exact"])
@pytest.mark.parametrize("precision", [abi.ENC_INT8, abi.ENC_F32], ids=["int8", "f32"])
def test_exec_record_families(ctx, precision, exact):
    m = synth.Model(synth.MICRO, seed=2, decoder=False)
    _, _, rec = _forward(ctx, m, precision, exact)
    plan = "int8" if precision == abi.ENC_INT8 else "f32"
    assert rec.route.decode() == f"hip:gfx950:{plan}" + (":exact" if exact else "")
    assert list(rec.family) == EXPECT[(precision, exact)]
    assert rec.precision == precision and rec.n_windows == 2 and rec.device_ms > 0
    assert rec.precision_source.decode() == ("fwhip_encoder_set_exact" if exact else "fwhip_encoder_load")
    print(dict(zip(abi.FAMILIES, (native.lib().fwhip_gemm_precision_str(f).decode() for f in rec.family))))


def _big(m, where):
    """Push one f16-pair operand of the fast forward past 65520."""
    t = m.t
    if where == "conv":       # conv1 output (after GELU) -> conv2's im2col pairs
        t["encoder.conv1.bias"][:6] = 1.0e5
    elif where == "qkv":      # layer 0 queries -> the QKV epilogue's pairs
        t["encoder.blocks.0.attn.query.bias"][:4] = 7.0e4
    elif where == "ln":       # f32 plan: layer 0's attention LayerNorm output pairs
        t["encoder.blocks.0.attn_ln.weight"][:3] = 4.0e4
    return m


@pytest.mark.parametrize("where,precision", [("conv", abi.ENC_INT8), ("qkv", abi.ENC_INT8), ("conv", abi.ENC_F32),
                                             ("ln", abi.ENC_F32)])
def test_f16_pair_range_falls_back_to_exact(ctx, where, precision):
    m = _big(synth.Model(synth.MICRO, seed=2, decoder=False), where)
    x, got, rec = _forward(ctx, m, precision, exact=False)
    assert rec.precision_source.decode() == "f16_pair_range", rec.precision_source
    assert rec.route.decode().endswith(":exact")
    assert list(rec.family) == EXPECT[(precision, True)]
    assert np.all(np.isfinite(got))
    oenc = O.Encoder(m, precision)
    want = np.stack([oenc.forward(x[b]) for b in range(x.shape[0])])
    assert_bitexact(got, want, f"{where} fallback")
    # the same model without the large values stays on the fast route
    _, _, rec2 = _forward(ctx, synth.Model(synth.MICRO, seed=2, decoder=False), precision, exact=False)
    assert rec2.precision_source.decode() == "fwhip_encoder_load"


def test_cross_kv_range_falls_back_to_strict(ctx):
    m = synth.Model(synth.MICRO, seed=5, encoder=False)
    cfg = m.cfg
    S, T = 2, cfg.n_audio_ctx
    states = enc_states(11, S, T, cfg.n_text_state)
    states[1, 7, :5] = 9.0e4
    states[0, 3, 2] = -7.0e4
    got = {}
    for exact in (False, True):
        dec = native.Decoder(ctx, m, abi.DEC_F16)
        dec.set_exact(exact)
        st = dec.state(S, T)
        st.set_cross(ctx.array(states))
        got[exact] = [(st.read(abi.DS_CROSS_K_F16, s), st.read(abi.DS_CROSS_VT_F16, s)) for s in range(S)]
        st.close()
        dec.close()
    for s in range(S):
        for a, b in zip(got[False][s], got[True][s]):
            np.testing.assert_array_equal(a.view(np.uint16), b.view(np.uint16))
