"""The oracle's f32 self-attention cache (the reference's default: FW_KV_F16
unset, KvCache::new / append nn.rs:5097-5416, attention_decode_step
nn.rs:6340-6400) pinned without restating it:

- closed forms of ref_attention_decode_f32: one cached row gives exactly its v
  (softmax of one score is 1), where the f16 cache gives f16(v); on rows that
  f16 represents exactly the f32 and f16 caches give the same bits (the two
  attentions differ only in where the values come from);
- nn.rs:8559's invariant on rows f16 does not represent: one row at a time
  through the f32 cache equals causal attention over all rows at once (1e-4);
- the decoder with the f32 cache against the float64 textbook decoder with an
  unrounded cache (tests/textbook.py, kv_f16=False): logits within the f16
  arm's bounds step by step, and the same greedy tokens;
- the FAST restatement (transposed scaled keys from the f32 rows, rf_pv_f32)
  bit for bit against the strict one over a whole greedy decode.

CPU only."""
import numpy as np
import pytest

from franken_whisper_amd import abi, synth
from oracle import oracle as O
from tests import textbook as TB
from tests.helpers import rel_maxabs
from tests.test_oracle_composition import DEC_CASES, _dec_case, _logit_run, _max_rel_err, rms


def test_one_cached_row_returns_v_exactly():
    rng = np.random.default_rng(3)
    n_head, d = 4, 256
    q = rng.standard_normal(d).astype(np.float32)
    k = rng.standard_normal((1, d)).astype(np.float32)
    v = rng.standard_normal((1, d)).astype(np.float32)
    out32 = O.attention_decode_f32(q, k, v, n_head)
    assert np.array_equal(out32, v[0])
    out16 = O.attention_decode_f16(q, k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16),
                                   n_head)
    assert np.array_equal(out16, v[0].astype(np.float16).astype(np.float32))
    assert not np.array_equal(out16, out32)


@pytest.mark.parametrize("tk", [1, 7, 64, 130])
def test_f32_and_f16_caches_agree_on_f16_values(tk):
    rng = np.random.default_rng(tk)
    n_head, d = 3, 192
    q = rng.standard_normal(d).astype(np.float32)
    k = TB.f16(rng.standard_normal((tk, d))).astype(np.float32)
    v = TB.f16(rng.standard_normal((tk, d))).astype(np.float32)
    a = O.attention_decode_f32(q, k, v, n_head)
    b = O.attention_decode_f16(q, k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16), n_head)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_f32_cache_incremental_equals_full_recompute():
    """nn.rs:8559 with rows f16 does not represent: the f32 cache keeps them."""
    rng = np.random.default_rng(11)
    n_head, dh, n = 3, 64, 6
    d = n_head * dh
    q = rng.uniform(-1, 1, (n, d)).astype(np.float32)
    k = rng.uniform(-1, 1, (n, d)).astype(np.float32)
    v = rng.uniform(-1, 1, (n, d)).astype(np.float32)
    assert not np.array_equal(TB.f16(k), k)
    full = O.attention(q, k, v, n_head, causal=True)
    inc = np.stack([O.attention_decode_f32(q[t], k[: t + 1], v[: t + 1], n_head) for t in range(n)])
    assert _max_rel_err(inc, full) < 1e-4


@pytest.mark.parametrize("name,seed", DEC_CASES)
@pytest.mark.parametrize("arm", [abi.DEC_F16, abi.DEC_INT8], ids=["f16", "int8"])
def test_decoder_f32_cache_steps_match_textbook(name, seed, arm):
    m, enc, toks = _dec_case(name, seed)
    prompt = m.tokens.sot_sequence()
    od = O.Decoder(m, arm)
    od.set_kv_f16(False)
    want = _logit_run(od.state(enc), prompt, toks)
    got = _logit_run(TB.Decoder(m, TB.Numerics(kv_f16=False)).state(enc), prompt, toks)
    for i, (w, g) in enumerate(zip(want, got)):
        e_max, e_rms = rel_maxabs(w, g), rms(w, g)
        print(f"{name} arm {arm} f32 cache row {i}: max-abs {e_max:.2e} rms {e_rms:.2e}")
        if arm == abi.DEC_F16:
            assert e_max <= 1e-3 and e_rms <= 3e-4, i
            assert int(np.argmax(w)) == int(np.argmax(g)), i
        else:
            assert e_rms <= 6e-2, i
            noise = np.sqrt(np.mean((np.asarray(w, np.float64) - g) ** 2))
            assert g[int(np.argmax(w))] >= np.max(g) - 3 * noise, i


def test_decoder_f32_cache_greedy_tokens_match_textbook():
    m, enc, _ = _dec_case("micro-ml", 5)
    tk, cfg = m.tokens, m.cfg
    n_max = cfg.n_text_ctx // 2 - 4
    od = O.Decoder(m, abi.DEC_F16)
    od.set_kv_f16(False)
    want = od.state(enc).greedy(tk.sot_sequence(), n_max, tk.filter())
    got = TB.Decoder(m, TB.Numerics(kv_f16=False)).state(enc).greedy(tk.sot_sequence(), n_max,
                                                                     TB.NoTimestampsFilter(tk, cfg.n_vocab))
    np.testing.assert_array_equal(want, got)


@pytest.mark.parametrize("arm", [abi.DEC_F16, abi.DEC_INT8], ids=["f16", "int8"])
def test_f32_cache_fast_restatement_bitexact(arm):
    m, enc, _ = _dec_case("micro-ml", 5)
    tk, cfg = m.tokens, m.cfg
    n_max = cfg.n_text_ctx // 2 - 4
    od = O.Decoder(m, arm)
    od.set_kv_f16(False)
    strict = od.state(enc)
    want = _logit_run(strict, tk.sot_sequence(), np.arange(5, 5 + n_max // 2))
    lib = O.lib()
    lib.ref_set_fast(1)
    try:
        fast = od.state(enc)
        got = _logit_run(fast, tk.sot_sequence(), np.arange(5, 5 + n_max // 2))
    finally:
        lib.ref_set_fast(0)
    for i, (w, g) in enumerate(zip(want, got)):
        assert np.array_equal(np.asarray(w).view(np.uint32), np.asarray(g).view(np.uint32)), i
    # and the f16 cache gives other logits on the same tokens
    od16 = O.Decoder(m, arm)
    other = _logit_run(od16.state(enc), tk.sot_sequence(), np.arange(5, 5 + n_max // 2))
    assert any(not np.array_equal(a, b) for a, b in zip(want, other))
