"""The FAST restatement of the oracle (oracle/refcpu_fast.c: register-blocked
AVX2 / F16C kernels, the CPU baseline's timed leg) gives the strict scalar
restatement's bits: primitive by primitive on ragged shapes and special
values, and end to end (encoder forward in both plans, with and without ToMe,
cross K/V, prefill logits and greedy tokens on both decoder arms)."""
import contextlib

import numpy as np
import pytest

from franken_whisper_amd import abi, synth
from oracle import oracle as O


@contextlib.contextmanager
def fast():
    O.lib().ref_set_fast(1)
    try:
        yield
    finally:
        O.lib().ref_set_fast(0)


def both(fn):
    a = fn()
    with fast():
        b = fn()
    return a, b


def same_bits(a, b, what):
    a, b = np.asarray(a), np.asarray(b)
    assert a.shape == b.shape, what
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.view(np.uint32)
    bad = np.flatnonzero(a.ravel() != b.ravel())
    assert bad.size == 0, f"{what}: {bad.size} differ, first at {bad[:5]}"


def rng(seed):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (5, 7, 16), (13, 64, 37), (97, 33, 48), (6, 200, 17), (200, 5, 130)])
def test_matmul_strict_order(m, k, n):
    r = rng(m * 1000 + k * 10 + n)
    a = r.standard_normal((m, k)).astype(np.float32)
    b = r.standard_normal((k, n)).astype(np.float32)
    a[0, 0] = -0.0
    b[:, 0] = -0.0  # column 0 sums -0.0 products from +0.0: the start value shows
    a, b = np.ascontiguousarray(a), np.ascontiguousarray(b)
    x, y = both(lambda: O.matmul_strict(a, b))
    same_bits(x, y, "matmul")
    assert np.all(np.signbit(x[:, 0]) == False)  # noqa: E712


def test_dot_f16c_and_i8w_lane_order():
    r = rng(1)
    for n in list(range(0, 70)) + [255, 256, 1280, 1500, 5120]:
        w = synth.normal_f16(n, "w", (n,), std=0.5) if n else np.zeros(0, np.uint16)
        x = r.standard_normal(n).astype(np.float32) * 3
        q = r.integers(-127, 128, n).astype(np.int8)
        a, b = both(lambda: O.dot_f16c(w, x))
        same_bits(np.float32(a), np.float32(b), f"dot_f16c n={n}")
        a, b = both(lambda: O.dot_i8w_f32(q, x))
        same_bits(np.float32(a), np.float32(b), f"dot_i8w_f32 n={n}")


def test_gemv_i8_exact_integer_dot():
    r = rng(2)
    for inp in (1, 15, 16, 17, 64, 100, 1280):
        q = r.integers(-127, 128, (37, inp)).astype(np.int8)
        s = r.random(37).astype(np.float32)
        x = r.standard_normal(inp).astype(np.float32)
        a, b = both(lambda: O.gemv_i8(q, s, x))
        same_bits(a, b, f"gemv_i8 inp={inp}")
        qb = O.quantize_f16_to_i8_blocked(synth.normal_f16(inp, "b", (9, inp)), 32)
        a, b = both(lambda: O.gemv_i8w_f32a_blocked(qb[0], qb[1], x))
        same_bits(a, b, f"gemv_i8w_f32a_blocked inp={inp}")


def test_softmax_rows_special_values():
    r = rng(3)
    rows = []
    for cols in (1, 7, 8, 9, 31, 64, 1500):
        x = (r.standard_normal((6, cols)) * 20).astype(np.float32)
        x[1, :] = -np.inf  # max not finite: row untouched
        x[2, ::3] = -np.inf  # masked lanes
        x[3, cols // 2] = np.nan  # NaN lane: ignored by the max, exp -> 0
        x[4, :] = 0.0
        x[5, 0] = 200.0  # everything else underflows
        rows.append(x)
    for x in rows:
        a, b = both(lambda: O.softmax_rows(x))
        same_bits(a, b, f"softmax cols={x.shape[1]}")


@pytest.mark.parametrize("tq,tk,d,h,causal,cache", [(5, 9, 24, 2, True, 4), (33, 33, 64, 4, True, 0),
                                                    (70, 51, 128, 2, False, 0), (1, 17, 16, 1, True, 16)])
def test_attention_per_head(tq, tk, d, h, causal, cache):
    r = rng(tq + tk + d)
    q = r.standard_normal((tq, d)).astype(np.float32)
    k = r.standard_normal((tk, d)).astype(np.float32)
    v = r.standard_normal((tk, d)).astype(np.float32)
    a, b = both(lambda: O.attention(q, k, v, h, causal, cache))
    same_bits(a, b, "attention")


@pytest.mark.parametrize("m", [1, 37, 130])
def test_encoder_int8_gemms(m):
    model = synth.Model(synth.MICRO_ML, seed=4, decoder=False)
    e = O.Encoder(model, abi.ENC_INT8)
    d = synth.MICRO_ML.n_audio_state
    r = rng(m)
    for which in range(6):
        x = r.standard_normal((m, 4 * d if which == 5 else d)).astype(np.float32)
        (aa, ay), (ba, by) = both(lambda: e.gemm(0, which, x))
        same_bits(aa, ba, f"gemm {which} acc")
        same_bits(ay, by, f"gemm {which} y")


@pytest.mark.parametrize("cfg", [synth.MICRO_ML, synth.TINY_EN], ids=lambda c: c.name)
@pytest.mark.parametrize("plan", [abi.ENC_F32, abi.ENC_INT8], ids=["f32", "int8"])
def test_encoder_forward(cfg, plan):
    model = synth.Model(cfg, seed=5, decoder=False)
    e = O.Encoder(model, plan)
    mel = synth.mel_input(5, 1, 2 * cfg.n_audio_ctx, cfg.n_mels)[0] * 0.5
    nl = 2 if cfg is synth.TINY_EN else -1
    a, b = both(lambda: e.forward(mel, n_layers=nl))
    same_bits(a, b, "encoder")
    a, b = both(lambda: e.forward(mel, n_layers=nl, tome_r=cfg.n_audio_ctx // 4, tome_after=0))
    same_bits(a, b, "encoder with ToMe")


@pytest.mark.parametrize("cfg", [synth.MICRO_ML, synth.TINY_EN], ids=lambda c: c.name)
@pytest.mark.parametrize("arm", [abi.DEC_F16, abi.DEC_INT8], ids=["f16", "int8"])
def test_decoder_greedy(cfg, arm):
    model = synth.Model(cfg, seed=6)
    enc = synth.encoder_states(7, 1, cfg.n_audio_ctx, cfg.n_text_state)[0]
    tk = model.tokens
    prompt = tk.sot_sequence(language_id=0)
    dec = O.Decoder(model, arm)

    def run():
        st = dec.state(enc)
        ck = st.cross_k_f16().copy()
        lg = st.step(prompt).copy()
        st2 = dec.state(enc)
        toks = st2.greedy(prompt, 12, tk.filter())
        return ck, lg, np.asarray(toks)

    (ak, al, at), (bk, bl, bt) = both(run)
    same_bits(ak, bk, "cross K")
    same_bits(al, bl, "prefill logits")
    same_bits(at, bt, "greedy tokens")


@pytest.mark.parametrize("arm", [abi.DEC_F16, abi.DEC_INT8], ids=["f16", "int8"])
def test_decoder_deep_cache_reset_and_mode_switch(arm):
    """Steps to the end of the text context (the transposed key copy grows row
    by row), a reset and replay, and a state that switches from strict to FAST
    half way (the copy is filled from the f16 cache): every step's logits are
    the strict ones."""
    cfg = synth.MICRO_ML
    model = synth.Model(cfg, seed=8)
    enc = synth.encoder_states(9, 1, cfg.n_audio_ctx, cfg.n_text_state)[0]
    dec = O.Decoder(model, arm)
    toks = rng(10).integers(0, 50000, cfg.n_text_ctx).astype(np.int32)
    ref = dec.state(enc)
    want = [ref.step(toks[:3]).copy()] + [ref.step(toks[i:i + 1]).copy() for i in range(3, cfg.n_text_ctx)]
    st = dec.state(enc)
    with fast():
        for rep in range(2):
            got = [st.step(toks[:3]).copy()] + [st.step(toks[i:i + 1]).copy() for i in range(3, cfg.n_text_ctx)]
            for i, (g, w) in enumerate(zip(got, want)):
                same_bits(g, w, f"rep {rep} step {i}")
            st.reset()
    half = dec.state(enc)
    got = [half.step(toks[:3]).copy()] + [half.step(toks[i:i + 1]).copy() for i in range(3, 30)]
    with fast():
        got += [half.step(toks[i:i + 1]).copy() for i in range(30, cfg.n_text_ctx)]
    for i, (g, w) in enumerate(zip(got, want)):
        same_bits(g, w, f"switched step {i}")
