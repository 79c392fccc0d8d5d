"""Pins the ggml restatement (oracle/ggml_ref.py) before it checks the library:

- the reference's own known-answer blocks for every quantized type, its
  byte-length rules and get_scale_min_k4 cases (ggml.rs:2105-2480), and its f16
  bit patterns (ggml.rs:2953-2970);
- the block-loop dequantizers against a per-element restatement from bit
  positions (tests/ggml_elementwise.py) on random blocks;
- the parser on the reference's synthetic-blob cases (ggml.rs:2866-3180) and on
  the seeded-weight model file written by franken_whisper_amd.ggml."""
import io
import struct

import numpy as np
import pytest

from franken_whisper_amd import ggml as W
from franken_whisper_amd import synth
from oracle import ggml_ref as G
from tests import ggml_elementwise as E


def h16(v: float) -> bytes:
    return np.array([v], np.float16).view("<u2").tobytes()


def both(t, raw, n):
    a = G.dequant(t, raw, n)
    b = E.dequant(t, raw, n)
    np.testing.assert_array_equal(a.view(np.uint32), b.view(np.uint32))
    return a


# ---------------------------------------------------------------- known answers

def test_q8_0_known_answer():
    assert G.byte_len(G.Q8_0, 64, "t") == 68
    with pytest.raises(G.InvalidRequest):
        G.byte_len(G.Q8_0, 40, "t")
    qs = np.zeros(32, np.int8)
    qs[:6] = [0, 1, 2, -1, -128, 127]
    out = both(G.Q8_0, h16(0.5) + qs.tobytes(), 32)
    assert list(out[:6]) == [0.0, 0.5, 1.0, -0.5, -64.0, 63.5]
    assert not out[6:].any()


def test_q5_0_known_answer():
    assert G.byte_len(G.Q5_0, 64, "t") == 44
    with pytest.raises(G.InvalidRequest):
        G.byte_len(G.Q5_0, 48, "t")
    qs = bytearray(16)
    qs[0], qs[1] = 0x0F, 0xF0
    raw = h16(1.0) + struct.pack("<I", (1 << 0) | (1 << 16)) + bytes(qs)
    out = both(G.Q5_0, raw, 32)
    assert (out[0], out[16], out[1], out[17], out[2], out[18]) == (15.0, 0.0, -16.0, -1.0, -16.0, -16.0)


def test_q4_0_known_answer():
    assert G.byte_len(G.Q4_0, 64, "t") == 36
    with pytest.raises(G.InvalidRequest):
        G.byte_len(G.Q4_0, 33, "t")
    qs = bytearray(16)
    qs[0], qs[1] = 0xF0, 0x08
    out = both(G.Q4_0, h16(2.0) + bytes(qs), 32)
    assert (out[0], out[16], out[1], out[17], out[2]) == (-16.0, 14.0, 0.0, -16.0, -16.0)


def test_q4_1_and_q5_1_known_answers():
    assert G.byte_len(G.Q4_1, 32, "t") == 20
    qs = bytearray(16)
    qs[0] = 0x30
    out = both(G.Q4_1, h16(2.0) + h16(-1.0) + bytes(qs), 32)
    assert (out[0], out[16]) == (-1.0, 5.0)
    assert G.byte_len(G.Q5_1, 32, "t") == 24
    qs = bytearray(16)
    qs[0] = 0x0F
    out = both(G.Q5_1, h16(1.0) + h16(0.5) + struct.pack("<I", 1) + bytes(qs), 32)
    assert (out[0], out[16]) == (31.5, 0.5)


def test_q6_k_known_answer():
    assert G.byte_len(G.Q6_K, 256, "t") == 210 and G.byte_len(G.Q6_K, 512, "t") == 420
    with pytest.raises(G.InvalidRequest):
        G.byte_len(G.Q6_K, 200, "t")
    raw = bytearray(210)
    raw[0], raw[32], raw[128] = 0x21, 0x53, 0b11_10_01_00
    raw[192], raw[194], raw[196], raw[198] = 1, 2, 0xFF, 4
    raw[208:210] = h16(0.5)
    out = both(G.Q6_K, bytes(raw), 256)
    assert (out[0], out[32], out[64], out[96]) == (-15.5, -13.0, -1.0, 42.0)


SC = bytes([2, 3, 0, 0, 1, 4, 0, 0, 0x25, 0x31, 0, 0])


def test_get_scale_min_k4_known_answers():
    s = np.frombuffer(SC, np.uint8)[None, :]
    got = [tuple(int(v[0]) for v in G.get_scale_min_k4(j, s)) for j in (0, 1, 4, 5)]
    assert got == [(2, 1), (3, 4), (5, 2), (1, 3)]
    assert [E._k4_scale(list(SC), j) for j in (0, 1, 4, 5)] == [(2, 1), (3, 4), (5, 2), (1, 3)]


def test_q4_k_known_answer():
    assert G.byte_len(G.Q4_K, 256, "t") == 144 and G.byte_len(G.Q4_K, 512, "t") == 288
    with pytest.raises(G.InvalidRequest):
        G.byte_len(G.Q4_K, 200, "t")
    raw = bytearray(144)
    raw[0:2], raw[2:4], raw[4:16] = h16(1.0), h16(0.5), SC
    raw[16], raw[80] = 0xA5, 0x24
    out = both(G.Q4_K, bytes(raw), 256)
    assert (out[0], out[32], out[128], out[160]) == (9.5, 28.0, 19.0, 0.5)


def test_q5_k_known_answer():
    assert G.byte_len(G.Q5_K, 256, "t") == 176 and G.byte_len(G.Q5_K, 512, "t") == 352
    with pytest.raises(G.InvalidRequest):
        G.byte_len(G.Q5_K, 200, "t")
    raw = bytearray(176)
    raw[0:2], raw[2:4], raw[4:16] = h16(1.0), h16(0.5), SC
    raw[16], raw[48], raw[48 + 64] = 0x11, 0xA5, 0x24
    out = both(G.Q5_K, bytes(raw), 256)
    assert (out[0], out[32], out[128], out[160]) == (41.5, 28.0, 99.0, 0.5)


def test_q3_k_known_answer():
    assert G.byte_len(G.Q3_K, 256, "t") == 110 and G.byte_len(G.Q3_K, 512, "t") == 220
    with pytest.raises(G.InvalidRequest):
        G.byte_len(G.Q3_K, 200, "t")
    raw = bytearray(110)
    raw[0], raw[1], raw[16] = 1, 0, 1
    raw[32], raw[33], raw[48] = 3, 1, 2
    raw[96], raw[97], raw[98] = 2, 3, 2
    raw[104], raw[105], raw[106] = 2, 1, 2
    raw[108:110] = h16(1.0)
    out = both(G.Q3_K, bytes(raw), 256)
    assert (out[0], out[1], out[16], out[32]) == (6.0, -6.0, -26.0, -8.0)


def test_q2_k_known_answer():
    assert G.byte_len(G.Q2_K, 256, "t") == 84 and G.byte_len(G.Q2_K, 512, "t") == 168
    with pytest.raises(G.InvalidRequest):
        G.byte_len(G.Q2_K, 200, "t")
    raw = bytearray(84)
    raw[0], raw[1], raw[2] = 0x12, 0x43, 0x05
    raw[16], raw[32] = 0x0B, 0x02
    raw[80:82], raw[82:84] = h16(1.0), h16(0.5)
    out = both(G.Q2_K, bytes(raw), 256)
    assert (out[0], out[16], out[32]) == (5.5, 4.0, 10.0)


def test_f16_known_bit_patterns():
    def f(bits):
        return G.dequant(G.F16, struct.pack("<H", bits), 1)[0]
    assert f(0x3C00) == 1.0 and f(0x0000) == 0.0 and f(0xC000) == -2.0
    assert f(0x8000) == 0.0 and np.signbit(f(0x8000))
    assert f(0x0001) == np.float32(2.0 ** -24)
    assert f(0x7C00) == np.inf and f(0xFC00) == -np.inf and np.isnan(f(0x7E00))


# ------------------------------------------------------ two restatements agree

def random_payload(t: int, n: int, seed: int) -> bytes:
    """Random blocks whose f16 fields are finite (so bitwise comparison is
    meaningful); every other byte pattern is a valid block."""
    qk, bb, _ = G.BLOCKS[t]
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, (n // qk, bb), dtype=np.uint8)
    fields = {G.Q4_0: [0], G.Q5_0: [0], G.Q8_0: [0], G.Q4_1: [0, 2], G.Q5_1: [0, 2], G.Q2_K: [80, 82],
              G.Q3_K: [108], G.Q4_K: [0, 2], G.Q5_K: [0, 2], G.Q6_K: [208]}[t]
    for off in fields:
        v = rng.standard_normal(b.shape[0]).astype(np.float16) * np.float16(0.01)
        b[:, off:off + 2] = v.view(np.uint8).reshape(-1, 2)
    return b.tobytes()


QTYPES = [G.Q4_0, G.Q4_1, G.Q5_0, G.Q5_1, G.Q8_0, G.Q2_K, G.Q3_K, G.Q4_K, G.Q5_K, G.Q6_K]


@pytest.mark.parametrize("t", QTYPES, ids=lambda t: G.BLOCKS[t][2])
def test_block_loops_match_elementwise_decode(t):
    n = 8 * G.BLOCKS[t][0]
    both(t, random_payload(t, n, t), n)


# ------------------------------------------------------------------ the parser

def minimal_blob() -> bytes:
    """SyntheticModel::minimal (ggml.rs:2875-2912), byte by byte."""
    b = struct.pack("<I", G.GGML_MAGIC) + struct.pack("<11i", 5, 1500, 384, 6, 4, 448, 384, 6, 4, 80, 1)
    b += struct.pack("<ii", 2, 3) + struct.pack("<6f", 0.0, 0.1, 0.2, 0.3, 0.4, 0.5)
    b += struct.pack("<i", 3)
    for tok in (b"!", b'"', b"ab"):
        b += struct.pack("<I", len(tok)) + tok
    b += struct.pack("<5i", 2, 5, 0, 3, 2) + b"w_f32" + struct.pack("<6f", 1, 2, 3, 4, 5, 6)
    b += struct.pack("<5i", 2, 5, 1, 2, 2) + b"w_f16" + np.array([1.0, 0.0, -2.0, 0.5], "<f2").tobytes()
    return b


def test_minimal_model_structure():
    m = G.parse(minimal_blob())
    assert m.hparams[0] == 5 and m.hparams[2] == 384 and m.hparams[10] == 1
    assert (m.n_mel, m.n_fft) == (2, 3)
    np.testing.assert_array_equal(m.filters, np.float32([0.0, 0.1, 0.2, 0.3, 0.4, 0.5]))
    assert m.vocab == [b"!", b'"', b"ab"]
    assert m.names() == ["w_f16", "w_f32"]
    assert m.tensors["w_f32"][0] == [2, 3] and m.tensors["w_f32"][1] == G.F32
    shape, v = G.tensor_f32(m, "w_f32")
    assert shape == [2, 3] and list(v) == [1, 2, 3, 4, 5, 6]
    shape, v = G.tensor_f32(m, "w_f16")
    assert shape == [2, 2] and list(v) == [1.0, 0.0, -2.0, 0.5]


def bad(blob, cls, *needles):
    with pytest.raises(cls) as e:
        G.parse(blob)
    assert any(s in str(e.value) for s in needles), str(e.value)
    return str(e.value)


def header(ftype=1):
    return struct.pack("<I", G.GGML_MAGIC) + struct.pack("<11i", 5, 1500, 384, 6, 4, 448, 384, 6, 4, 80, ftype)


def test_parser_rejections():
    bad(header() + struct.pack("<ii", 32768, 32768), G.InvalidRequest, "end of file")
    bad(header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 10 ** 9), G.InvalidRequest, "end of file")
    tail = minimal_blob() + struct.pack("<4i", 1, 1, 0, 0) + b"z" + bytes([0xAA, 0xBB, 0xCC])
    bad(tail, G.InvalidRequest, "trailing bytes", "unexpected end of file")
    blob = bytearray(minimal_blob())
    blob[0] = 0
    bad(bytes(blob), G.InvalidRequest, "magic")
    assert "base 15" in bad(header(1015), G.Unsupported, "base 15")
    bad(minimal_blob()[:10], G.InvalidRequest, "end of file")
    base = header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0)
    bad(base + struct.pack("<3i", 0, 1, 0), G.InvalidRequest, "n_dims 0 out of range")
    bad(base + struct.pack("<3i", 5, 1, 0), G.InvalidRequest, "n_dims 5 out of range")
    bad(base + struct.pack("<4i", 1, 1, 4, 1) + b"x", G.Unsupported, "tensor element type 4")
    bad(base + struct.pack("<4i", 1, 1, 0, -3) + b"x", G.InvalidRequest, "tensor dimension is negative (-3)")
    bad(base + struct.pack("<4i", 1, 1, 8, 40) + b"x", G.InvalidRequest, "q8_0 element count 40 is not a multiple of 32")
    bad(base + struct.pack("<4i", 1, 2, 0, 1) + b"\xff\xfe" + bytes(4), G.InvalidRequest, "not valid UTF-8")
    bad(base + struct.pack("<4i", 1, 1, 0, 4) + b"x" + bytes(8), G.InvalidRequest, "needed 16 byte(s)")


def test_quantized_ftypes_with_version_parse():
    # whisper.cpp packs the quantization version: 2007 is q8_0 v2 (ggml.rs:1019-1026)
    blob = header(2007) + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0)
    payload = random_payload(G.Q8_0, 64, 1)
    blob += struct.pack("<5i", 2, 1, G.Q8_0, 32, 2) + b"q" + payload
    m = G.parse(blob)
    assert m.tensors["q"][:2] == ([2, 32], G.Q8_0)
    np.testing.assert_array_equal(G.tensor_f32(m, "q")[1], G.dequant_q8_0(payload, 64))


def test_seeded_model_file_roundtrip():
    m = synth.Model(synth.MICRO, seed=3)
    buf = io.BytesIO()
    fb = synth.mel_filterbank(m.cfg.n_mels)
    W.write(buf, W.hparams11(m.cfg, 1), fb, W.synthetic_vocab(m.tokens.eot), W.model_tensors(m))
    g = G.parse(buf.getvalue())
    assert g.hparams == [51864, 64, 128, 2, 2, 64, 128, 2, 2, 16, 1]
    assert g.names() == sorted(m.t)
    np.testing.assert_array_equal(g.filters.reshape(fb.shape), fb)
    assert len(g.vocab) == m.tokens.eot and g.vocab[65] == b"A"
    for name, a in m.t.items():
        shape, t, _, _ = g.tensors[name]
        assert shape == list(a.shape)
        assert t == (G.F16 if a.dtype == np.uint16 else G.F32)
        want = a.view(np.float16).astype(np.float32) if a.dtype == np.uint16 else a
        np.testing.assert_array_equal(G.tensor_f32(g, name)[1], want.reshape(-1))
