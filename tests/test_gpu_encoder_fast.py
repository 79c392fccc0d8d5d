"""GPU parity of the encoder path the benchmark runs (the int8 plan in fast
mode) and of the configs' own workloads.

- The persistent int8 GEMM at the benchmark's M (10 windows x 1500 = 15,000
  rows), where every block walks several tiles: i32 accumulators and
  epilogues BIT-EXACT against the oracle for all six linears of a
  large-v3-turbo block.
- The two fused epilogues only the forward uses, against the oracle's values
  on the same quantized rows: the QKV GEMM's head-major f16 hi/lo split with
  V transposed (hi = f16(v) and lo = f16(v - hi) bit for bit), and fc1 in
  GELU-index form (f16 bits of v where |v| < 9.98, else the sentinel with v
  itself in the side array).
- The 32-layer large-v3-turbo int8 encoder in exact mode: bit-identical to the
  oracle on one window.
- Fast mode (the benchmarked route) end to end: greedy tokens of the f16
  decoder arm in fast mode, from the fast-mode encoder states, identical to
  the oracle's (oracle encoder + oracle decoder) for tiny.en and for one
  large-v3-turbo window.  (The int8 decoder arm re-quantizes every linear's
  input, so its tokens follow the encoder states' last bits; its fast mode is
  checked by teacher forcing in the decoder's fast-mode tests.)
- Config 0: tiny.en (4 + 4 layers) f32 encoder within max-abs 1e-3 relative,
  and 64 greedy tokens identical on both decoder arms.
- The attention's query tile follows the launch size (128, 256 or 512 queries
  per block); a window's encoder states are bit-identical whichever tile its
  batch gets.
"""
import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from oracle import oracle as O
from tests.helpers import assert_bitexact, rel_maxabs

pytestmark = pytest.mark.gpu

TURBO1 = synth.Config("turbo-1L", 51866, 1500, 1280, 20, 1, 448, 1280, 20, 4, 128)


def _vt_pos(t):
    """Key t's position in a V^T row: bits 2 and 3 swapped."""
    t = np.asarray(t)
    return (t & ~12) | ((t & 4) << 1) | ((t & 8) >> 1)


def _split(y):
    y = np.asarray(y, np.float32)
    hi = y.astype(np.float16)
    lo = (y - hi.astype(np.float32)).astype(np.float16)
    return hi.view(np.uint16), lo.view(np.uint16)


@pytest.fixture(scope="module")
def turbo1():
    m = synth.Model(TURBO1, seed=4, decoder=False)
    return m, O.Encoder(m, abi.ENC_INT8)


def test_int8_gemm_multitile_bitexact(ctx, turbo1):
    """All six int8 GEMMs of a turbo block at M = 15,000 (fc1: 1,180 tiles on
    256 persistent blocks)."""
    m, oenc = turbo1
    enc = native.Encoder(ctx, m, abi.ENC_INT8)
    rng = np.random.default_rng(11)
    d, M = TURBO1.n_audio_state, 15000
    for which in range(6):
        inp = 4 * d if which == 5 else d
        out = 4 * d if which == 4 else d
        x = (rng.standard_normal((M, inp)) * (2.6 if which == 5 else 1.3)).astype(np.float32)
        xd = ctx.array(x)
        acc, y = ctx.empty((M, out), np.int32), ctx.empty((M, out), np.float32)
        print(f"turbo gemm {which} M={M}", flush=True)
        enc.gemm_i8(0, which, xd, acc, y)
        want_acc, want_y = oenc.gemm(0, which, x)
        np.testing.assert_array_equal(acc.download(), want_acc, err_msg=f"acc which {which}")
        assert_bitexact(y.download(), want_y, f"epilogue which {which}")
        for a in (xd, acc, y):
            a.free()
    enc.close()


def test_qkv_split_epilogue_matches_oracle(ctx, turbo1):
    m, oenc = turbo1
    enc = native.Encoder(ctx, m, abi.ENC_INT8)
    d, H, T, B = TURBO1.n_audio_state, TURBO1.n_audio_head, 1500, 10
    Tp = (T + 63) // 64 * 64
    x = (np.random.default_rng(12).standard_normal((B * T, d)) * 1.3).astype(np.float32)
    qk, vt = B * H * T * 64, B * H * 64 * Tp
    out = ctx.empty((4 * qk + 2 * vt,), np.uint16)
    print("qkv split epilogue, 10 windows", flush=True)
    enc.gemm_i8_fused(0, 0, ctx.array(x), B, T, out)
    got = out.download()
    planes = [got[i * qk:(i + 1) * qk].reshape(B, H, T, 64) for i in range(4)]
    vth = got[4 * qk:4 * qk + vt].reshape(B, H, 64, Tp)
    vtl = got[4 * qk + vt:].reshape(B, H, 64, Tp)
    for which in range(3):
        _, y = oenc.gemm(0, which, x)
        hi, lo = _split(y)
        hi, lo = hi.reshape(B, T, H, 64), lo.reshape(B, T, H, 64)
        if which < 2:
            np.testing.assert_array_equal(planes[2 * which], hi.transpose(0, 2, 1, 3), err_msg=f"{which} hi")
            np.testing.assert_array_equal(planes[2 * which + 1], lo.transpose(0, 2, 1, 3), err_msg=f"{which} lo")
        else:
            pos = _vt_pos(np.arange(T))
            np.testing.assert_array_equal(vth[:, :, :, pos], hi.transpose(0, 2, 3, 1), err_msg="V^T hi")
            np.testing.assert_array_equal(vtl[:, :, :, pos], lo.transpose(0, 2, 3, 1), err_msg="V^T lo")
            pad = np.setdiff1d(np.arange(Tp), pos)
            assert not vth[:, :, :, pad].any() and not vtl[:, :, :, pad].any()
    enc.close()


def test_fc1_index_epilogue_matches_oracle(ctx, turbo1):
    m, oenc = turbo1
    enc = native.Encoder(ctx, m, abi.ENC_INT8)
    d, M = TURBO1.n_audio_state, 15000
    rng = np.random.default_rng(13)
    x = (rng.standard_normal((M, d)) * 1.3).astype(np.float32)
    x[::97] *= 40.0  # rows whose fc1 values pass +-10: the sentinel path
    xd = ctx.array(x)
    idx, side = ctx.empty((M, 4 * d), np.uint16), ctx.empty((M, 4 * d), np.float32)
    print("fc1 index epilogue, M=15000", flush=True)
    enc.gemm_i8_fused(0, 4, xd, 1, M, idx, side)
    _, y = oenc.gemm(0, 4, x)
    gi, gs = idx.download(), side.download()
    inside = np.abs(y) < np.float32(9.98)
    assert (~inside).sum() > 1000, "the sentinel path did not run"
    np.testing.assert_array_equal(gi[inside], y[inside].astype(np.float16).view(np.uint16))
    assert np.all(gi[~inside] == 0xFFFF)
    assert_bitexact(gs[~inside], y[~inside], "fc1 side values")
    enc.close()


def _greedy_pair(ctx, cfg, seed, n_max, arm=abi.DEC_INT8, precision=abi.ENC_INT8, exact=False):
    m = synth.Model(cfg, seed=seed)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(seed + 1, 1, nf, cfg.n_mels) * np.float32(0.5)
    enc = native.Encoder(ctx, m, precision)
    if exact:
        enc.set_exact(True)
    out = ctx.empty((1, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    enc.forward_time_major(ctx.array(x), 1, nf, out)
    states = out.download()
    enc.close()
    want_states = O.Encoder(m, precision).forward(x[0])
    tk = m.tokens
    dec = native.Decoder(ctx, m, arm)
    st = dec.state(1, cfg.n_audio_ctx)
    st.set_cross(out)
    got = st.greedy(tk.sot_sequence(), n_max, tk.filter())[0]
    st.close()
    dec.close()
    want = O.Decoder(m, arm).state(want_states[0]).greedy(tk.sot_sequence(), n_max, tk.filter())
    return states[0], want_states, got, want


def test_turbo_int8_encoder_exact_full_depth_bitexact(ctx):
    """Config 2's encoder arithmetic, all 32 layers, one window: exact mode is
    bit-identical to the oracle."""
    cfg = synth.TURBO
    m = synth.Model(cfg, seed=6, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(7, 1, nf, cfg.n_mels) * np.float32(0.5)
    enc = native.Encoder(ctx, m, abi.ENC_INT8)
    enc.set_exact(True)
    out = ctx.empty((1, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    print("turbo int8 exact, 32 layers", flush=True)
    enc.forward_time_major(ctx.array(x), 1, nf, out)
    got = out.download()[0]
    enc.close()
    assert_bitexact(got, O.Encoder(m, abi.ENC_INT8).forward(x[0]), "turbo int8 exact 32 layers")


@pytest.mark.parametrize("name,n_max", [("tiny.en", 64), ("large-v3-turbo", 48)])
def test_fast_mode_int8_encoder_tokens_match_oracle(ctx, name, n_max):
    """The benchmarked route: int8 plan in fast mode (MFMA f16-pair conv and
    attention), then the f16 decoder arm in fast mode; greedy tokens identical
    to the oracle's encoder + decoder."""
    cfg = synth.CONFIGS[name]
    print(f"{name} fast int8 encoder -> f16 arm greedy {n_max}", flush=True)
    states, want_states, got, want = _greedy_pair(ctx, cfg, seed=8, n_max=n_max, arm=abi.DEC_F16)
    print(f"{name}: state rel max-abs {rel_maxabs(states, want_states):.2e}; tokens {got.tolist()}", flush=True)
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("arm", [abi.DEC_INT8, abi.DEC_F16], ids=["int8", "f16"])
def test_config0_tiny_en_f32_encoder_and_64_tokens(ctx, arm):
    """Config 0: tiny.en, one 30 s window, f32 encoder (fast mode) within
    max-abs 1e-3 relative of the oracle, then 64 greedy tokens from the SOT
    prefix identical to the oracle's (its decoder run on its own encoder
    states).  The harness drives up to 64 sampled tokens, stopping early at
    end-of-text as the reference loop does."""
    cfg = synth.TINY_EN
    states, want_states, got, want = _greedy_pair(ctx, cfg, seed=9, n_max=64, arm=arm, precision=abi.ENC_F32)
    err = rel_maxabs(states, want_states)
    print(f"tiny.en f32 encoder rel max-abs {err:.2e}; {len(got)} tokens", flush=True)
    assert err < 1e-3
    np.testing.assert_array_equal(got, want)


def test_encoder_cancel_then_resume(ctx):
    """A cancel requested before a forward stops it at the next layer boundary
    with FWHIP_ERR_CANCELLED and clears the flag (checkpoint(), encoder.rs:1628);
    the next forward runs to completion with the same result as an
    uncancelled one."""
    cfg = synth.MICRO
    m = synth.Model(cfg, seed=3, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = ctx.array(synth.mel_input(4, 1, nf, cfg.n_mels))
    enc = native.Encoder(ctx, m, abi.ENC_INT8)
    out = ctx.empty((1, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    enc.forward_time_major(x, 1, nf, out)
    ref = out.download()
    ctx.cancel()
    with pytest.raises(native.FwhipError) as e:
        enc.forward_time_major(x, 1, nf, out)
    assert e.value.code == abi.ERR_CANCELLED
    enc.forward_time_major(x, 1, nf, out)
    assert_bitexact(out.download(), ref, "forward after a cancelled one")
    enc.close()


@pytest.mark.parametrize("precision", [abi.ENC_INT8, abi.ENC_F32], ids=["int8", "f32"])
def test_attention_tiles_bit_identical_across_batch_sizes(ctx, precision):
    """large-v3-turbo: one window (128-query tiles), four (256) and six (512)
    give window 0 the same encoder states bit for bit, in both plans."""
    cfg = synth.TURBO
    m = synth.Model(cfg, seed=11, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(12, 6, nf, cfg.n_mels) * 0.5
    enc = native.Encoder(ctx, m, precision)
    outs = {}
    for B in (1, 4, 6):
        print(f"attention tiles: batch {B}", flush=True)
        out = ctx.empty((B, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
        enc.forward_time_major(ctx.array(np.ascontiguousarray(x[:B])), B, nf, out)
        outs[B] = out.download()
    enc.close()
    for B in (1, 4):
        assert_bitexact(outs[B][0], outs[6][0], f"window 0 at batch {B} vs 6")
