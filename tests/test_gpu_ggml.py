"""GPU side of the ggml model files:

- fwhip_dequant / fwhip_ggml_tensor_f32 — every element type the reference
  decodes (tensor_f32, ggml.rs:1478-1632) — bit for bit against the oracle's
  restatement, from one block to tensors the size of large-v3-turbo's token
  embedding (51866 x 1280), with partial tiles and unaligned block counts;
- encoder and decoder loaded from the seeded-weight model file
  (fwhip_encoder_load_ggml / fwhip_decoder_load_ggml) give the same bits as the
  same weights loaded from memory, on both encoder plans and decoder arms;
- stored types other than f16: vectors decoded like tensor_f32, f32 linears
  that hold binary16 values accepted by the encoder, everything else refused
  with the CPU-route status and the tensor's name."""
import struct

import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from franken_whisper_amd import ggml as W
from oracle import ggml_ref as G
from tests.helpers import assert_bitexact
from tests.test_oracle_ggml import header, random_payload

pytestmark = pytest.mark.gpu

ALL = [G.F32, G.F16, G.Q4_0, G.Q4_1, G.Q5_0, G.Q5_1, G.Q8_0, G.Q2_K, G.Q3_K, G.Q4_K, G.Q5_K, G.Q6_K]


def payload(t, n, seed):
    if t == G.F32:
        return np.random.default_rng(seed).standard_normal(n).astype("<f4").tobytes()
    if t == G.F16:
        return np.random.default_rng(seed).standard_normal(n).astype("<f2").tobytes()
    return random_payload(t, n, seed)


def sizes(t):
    qk = G.BLOCKS[t][0]
    return [qk, 7 * qk, 1024 + qk, 40 * 1024 + 3 * qk]


@pytest.mark.parametrize("t", ALL, ids=lambda t: G.BLOCKS[t][2])
def test_dequant_bitexact(ctx, t):
    for n in sizes(t):
        raw = payload(t, n, n + t)
        print(f"dequant {G.BLOCKS[t][2]} n={n}", flush=True)
        dev = ctx.array(np.frombuffer(raw + bytes(-len(raw) % 4), np.uint8).copy())
        out = ctx.empty((n,), np.float32)
        native.dequant(ctx, t, dev, len(raw), n, out)
        got = out.download()
        np.testing.assert_array_equal(got.view(np.uint32), G.dequant(t, raw, n).view(np.uint32),
                                      err_msg=f"{G.BLOCKS[t][2]} n={n}")


@pytest.mark.parametrize("t", [G.Q8_0, G.Q4_K, G.F16], ids=lambda t: G.BLOCKS[t][2])
def test_dequant_turbo_token_embedding_size(ctx, t):
    n = 51866 * 1280
    raw = payload(t, n, 11)
    print(f"dequant {G.BLOCKS[t][2]} n={n}", flush=True)
    dev = ctx.array(np.frombuffer(raw, np.uint8).copy())
    out = ctx.empty((n,), np.float32)
    native.dequant(ctx, t, dev, len(raw), n, out)
    np.testing.assert_array_equal(out.download().view(np.uint32), G.dequant(t, raw, n).view(np.uint32))


def test_dequant_argument_checks(ctx):
    raw = ctx.array(np.zeros(68, np.uint8))
    out = ctx.empty((64,), np.float32)
    with pytest.raises(native.FwhipError) as e:
        native.dequant(ctx, G.Q8_0, raw, 67, 64, out)
    assert e.value.code == abi.ERR_INVALID and "q8_0 byte length 67 != 68" in str(e.value)
    with pytest.raises(native.FwhipError) as e:
        native.dequant(ctx, G.Q8_0, raw, 68, 40, out)
    assert e.value.code == abi.ERR_INVALID and "not a multiple of 32" in str(e.value)
    with pytest.raises(native.FwhipError) as e:
        native.dequant(ctx, 4, raw, 68, 64, out)
    assert e.value.code == abi.ERR_UNSUPPORTED


def mixed_file(tmp_path):
    blob = header(1) + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0)
    for t in ALL:
        qk = G.BLOCKS[t][0]
        name = f"w.{G.BLOCKS[t][2]}"
        blob += struct.pack("<5i", 2, len(name), t, 2 * qk, 5) + name.encode() + payload(t, 10 * qk, t)
    p = tmp_path / "mixed.bin"
    p.write_bytes(blob)
    return p, G.parse(blob)


def test_tensor_f32_from_file(ctx, tmp_path):
    p, m = mixed_file(tmp_path)
    g = native.GgmlFile(str(p))
    for name in m.names():
        got = g.tensor_f32(ctx, name).download()
        shape, want = G.tensor_f32(m, name)
        assert list(got.shape) == shape
        np.testing.assert_array_equal(got.reshape(-1).view(np.uint32), want.view(np.uint32), err_msg=name)
    g.close()


# ------------------------------------------------------------- model loads

def _enc_out(ctx, model, prec, x, exact):
    enc = native.Encoder(ctx, model, prec)
    enc.set_exact(exact)
    cfg = enc.cfg
    out = ctx.empty((x.shape[0], x.shape[1] // 2, cfg.n_audio_state), np.float32)
    enc.forward_time_major(ctx.array(x), x.shape[0], x.shape[1], out)
    got = out.download()
    enc.close()
    return got


@pytest.mark.parametrize("prec", [abi.ENC_F32, abi.ENC_INT8], ids=["f32", "int8"])
def test_encoder_from_seeded_file_matches_memory_load(ctx, tmp_path, prec):
    m = synth.Model(synth.MICRO, seed=5)
    p = tmp_path / "ggml-micro.bin"
    W.write_model(p, m)
    g = native.GgmlFile(str(p))
    x = synth.mel_input(2, 2, 2 * m.cfg.n_audio_ctx, m.cfg.n_mels)
    for exact in (True, False):
        print(f"encoder from file prec={prec} exact={exact}", flush=True)
        assert_bitexact(_enc_out(ctx, g, prec, x, exact), _enc_out(ctx, m, prec, x, exact), f"exact={exact}")
    g.close()


def _greedy(ctx, model, arm, enc, n_max):
    dec = native.Decoder(ctx, model, arm)
    dec.set_exact(True)
    st = dec.state(enc.shape[0], enc.shape[1])
    st.set_cross(ctx.array(enc))
    tk = synth.Tokens(synth.MICRO)
    toks = st.greedy(tk.sot_sequence(), n_max, tk.filter())
    st.reset()
    logits = ctx.empty((enc.shape[0], synth.MICRO.n_vocab), np.float32)
    st.step(np.tile(np.int32(tk.sot_sequence()), (enc.shape[0], 1)), logits)
    lg = logits.download()
    st.close()
    dec.close()
    return toks, lg


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16], ids=["int8", "f16"])
def test_decoder_from_seeded_file_matches_memory_load(ctx, tmp_path, arm):
    m = synth.Model(synth.MICRO, seed=6)
    p = tmp_path / "ggml-micro.bin"
    W.write_model(p, m)
    g = native.GgmlFile(str(p))
    enc = synth.encoder_states(7, 3, m.cfg.n_audio_ctx, m.cfg.n_text_state)
    print(f"decoder from file arm={arm}", flush=True)
    a = _greedy(ctx, g, arm, enc, 24)
    b = _greedy(ctx, m, arm, enc, 24)
    for s in range(enc.shape[0]):
        np.testing.assert_array_equal(a[0][s], b[0][s], err_msg=f"stream {s} tokens")
    assert_bitexact(a[1], b[1], "prefill logits")
    g.close()


def _rewrite(m, tmp_path, convert):
    """The seeded file with tensors re-stored by convert(name, array) ->
    (ttype, payload) or None (keep)."""
    def tensors():
        for name, t, shape, pl in W.model_tensors(m):
            r = convert(name, m.t[name])
            if r is not None:
                t, pl = r
            yield name, t, shape, pl
    p = tmp_path / "ggml-mixed.bin"
    with open(p, "wb") as f:
        W.write(f, W.hparams11(m.cfg, 1), synth.mel_filterbank(m.cfg.n_mels), W.synthetic_vocab(m.tokens.eot),
                tensors())
    return p


def test_encoder_accepts_f32_stored_binary16_linears_and_other_vector_types(ctx, tmp_path):
    m = synth.Model(synth.MICRO, seed=8)

    def convert(name, a):
        if a.dtype == np.uint16:  # linears and conv kernels as f32 values
            return G.F32, a.view(np.float16).astype("<f4").tobytes()
        if name.endswith("attn_ln.weight") or name.endswith(".bias") and "blocks.0" in name:
            return G.F16, a.astype("<f2").tobytes()  # vectors as f16
        return None
    p = _rewrite(m, tmp_path, convert)
    g = native.GgmlFile(str(p))
    o = G.parse(p.read_bytes())
    # the same weights from memory, vectors as tensor_f32 decodes them
    for name in m.t:
        if m.t[name].dtype == np.float32:
            m.t[name] = G.tensor_f32(o, name)[1].reshape(m.t[name].shape)
    x = synth.mel_input(4, 1, 2 * m.cfg.n_audio_ctx, m.cfg.n_mels)
    for prec in (abi.ENC_F32, abi.ENC_INT8):
        assert_bitexact(_enc_out(ctx, g, prec, x, True), _enc_out(ctx, m, prec, x, True), f"prec {prec}")
    with pytest.raises(native.FwhipError) as e:
        native.Decoder(ctx, g, abi.DEC_F16)
    assert e.value.code == abi.ERR_UNSUPPORTED and "cpu:ggml-f32-linear" in str(e.value)
    assert "decoder.token_embedding.weight" in str(e.value)
    g.close()


def test_quantized_linears_take_the_cpu_route(ctx, tmp_path):
    m = synth.Model(synth.MICRO, seed=9)
    name = "encoder.blocks.1.mlp.0.weight"

    def convert(n, a):
        if n == name:
            return G.Q8_0, random_payload(G.Q8_0, a.size, 3)
        return None
    g = native.GgmlFile(str(_rewrite(m, tmp_path, convert)))
    with pytest.raises(native.FwhipError) as e:
        native.Encoder(ctx, g, abi.ENC_INT8)
    assert e.value.code == abi.ERR_UNSUPPORTED
    assert "cpu:ggml-q8_0-linear" in str(e.value) and name in str(e.value)
    g.close()


def test_shape_and_name_errors_match_the_reference(ctx, tmp_path):
    m = synth.Model(synth.MICRO, seed=10)
    m.t["encoder.ln_post.bias"] = np.zeros(127, np.float32)
    del m.t["decoder.blocks.1.cross_attn.value.bias"]
    p = tmp_path / "bad.bin"
    W.write_model(p, m)
    g = native.GgmlFile(str(p))
    with pytest.raises(native.FwhipError) as e:
        native.Encoder(ctx, g, abi.ENC_F32)
    assert str(e.value).endswith("encoder tensor 'encoder.ln_post.bias' has shape [127], expected a length-128 vector")
    with pytest.raises(native.FwhipError) as e:
        native.Decoder(ctx, g, abi.DEC_INT8)
    assert str(e.value).endswith("unknown tensor 'decoder.blocks.1.cross_attn.value.bias'")
    g.close()


def test_cancel_during_load(ctx, tmp_path):
    m = synth.Model(synth.MICRO, seed=11)
    p = tmp_path / "ggml-micro.bin"
    W.write_model(p, m)
    g = native.GgmlFile(str(p))
    ctx.cancel()
    with pytest.raises(native.FwhipError) as e:
        native.Encoder(ctx, g, abi.ENC_F32)
    assert e.value.code == abi.ERR_CANCELLED
    enc = native.Encoder(ctx, g, abi.ENC_F32)  # the flag was consumed
    enc.close()
    g.close()
