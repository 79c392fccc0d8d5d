"""The library's ggml reader (fwhip_ggml_*: host code, no GPU needed) against
the oracle's restatement of GgmlModel::parse (ggml.rs:982-1136): the same
directory, bytes and errors — class and message — for the reference's
synthetic-blob cases, malformed inputs, and the seeded-weight model file, both
from memory (GgmlModel::from_bytes) and from a file (the pread scan)."""
import struct

import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from franken_whisper_amd import ggml as W
from oracle import ggml_ref as G
from tests.test_oracle_ggml import header, minimal_blob, random_payload

CODE = {G.InvalidRequest: abi.ERR_INVALID, G.Unsupported: abi.ERR_UNSUPPORTED}


def same_as_oracle(g: native.GgmlFile, m: G.Model):
    assert g.hparams == m.hparams
    np.testing.assert_array_equal(g.filters().reshape(-1), m.filters)
    assert g.filters().shape == (m.n_mel, m.n_fft)
    assert g.vocab() == m.vocab
    assert g.names() == m.names()
    for name in m.names():
        shape, t, off, nbytes = m.tensors[name]
        assert g.info(name) == (shape, t, nbytes), name
        assert g.raw(name) == m.raw(name), name


def test_minimal_model_from_bytes():
    blob = minimal_blob()
    g = native.GgmlFile(blob)
    same_as_oracle(g, G.parse(blob))
    with pytest.raises(native.FwhipError) as e:
        g.info("nope")
    assert e.value.code == abi.ERR_INVALID and "unknown tensor 'nope'" in str(e.value)
    g.close()


def test_quantized_tensors_directory(tmp_path):
    blob = header(2008) + struct.pack("<iif", 1, 1, 0.25) + struct.pack("<i", 1) + struct.pack("<I", 2) + b"hi"
    for i, t in enumerate([G.Q4_0, G.Q4_1, G.Q5_0, G.Q5_1, G.Q8_0, G.Q2_K, G.Q3_K, G.Q4_K, G.Q5_K, G.Q6_K]):
        qk = G.BLOCKS[t][0]
        name = f"t{i}.{G.BLOCKS[t][2]}"
        blob += struct.pack("<5i", 2, len(name), t, 2 * qk, 3) + name.encode() + random_payload(t, 6 * qk, i)
    m = G.parse(blob)
    same_as_oracle(native.GgmlFile(blob), m)
    p = tmp_path / "q.bin"
    p.write_bytes(blob)
    same_as_oracle(native.GgmlFile(str(p)), m)


MALFORMED = {
    "absurd filterbank": header() + struct.pack("<ii", 32768, 32768),
    "absurd vocab": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 10 ** 9),
    "trailing junk": minimal_blob() + struct.pack("<4i", 1, 1, 0, 0) + b"z" + bytes([0xAA, 0xBB, 0xCC]),
    "bad magic": b"\x00" + minimal_blob()[1:],
    "ftype base 15": header(1015),
    "truncated header": minimal_blob()[:10],
    "empty": b"",
    "negative n_mel": header() + struct.pack("<ii", -2, 3),
    "n_dims 0": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<3i", 0, 1, 0),
    "n_dims 5": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<3i", 5, 1, 0),
    "ttype 4": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<4i", 1, 1, 4, 1) + b"x",
    "negative dim": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<4i", 1, 1, 0, -3) + b"x",
    "q8_0 count 40": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<4i", 1, 1, 8, 40) + b"x",
    "bad utf-8 name": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<4i", 1, 2, 0, 1)
    + b"\xff\xfe" + bytes(4),
    "surrogate name": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<4i", 1, 3, 0, 1)
    + b"\xed\xa0\x80" + bytes(4),
    "short payload": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<4i", 1, 1, 0, 4)
    + b"x" + bytes(8),
    "short vocab token": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<iI", 1, 9) + b"abc",
    "negative name length": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<3i", 1, -1, 0),
    "huge dims": header() + struct.pack("<iif", 1, 1, 0.0) + struct.pack("<i", 0) + struct.pack("<7i", 4, 1, 0, 2 ** 31 - 1,
                                                                                                 2 ** 31 - 1, 2 ** 31 - 1, 2 ** 31 - 1) + b"x",
}


@pytest.mark.parametrize("name", list(MALFORMED))
def test_malformed_files_fail_like_the_reference(name, tmp_path):
    blob = MALFORMED[name]
    with pytest.raises((G.InvalidRequest, G.Unsupported)) as want:
        G.parse(blob)
    p = tmp_path / "m.bin"
    p.write_bytes(blob)
    for src in (blob, str(p)):
        with pytest.raises(native.FwhipError) as got:
            native.GgmlFile(src)
        assert got.value.code == CODE[type(want.value)], (name, str(got.value))
        assert str(got.value).endswith(str(want.value)), (name, str(got.value), str(want.value))


def test_missing_file_is_an_io_error(tmp_path):
    with pytest.raises(native.FwhipError) as e:
        native.GgmlFile(str(tmp_path / "absent.bin"))
    assert e.value.code == abi.ERR_GENERIC and "io:" in str(e.value)


def test_seeded_model_file(tmp_path):
    m = synth.Model(synth.MICRO, seed=3)
    p = tmp_path / "ggml-micro.bin"
    W.write_model(p, m)
    blob = p.read_bytes()
    o = G.parse(blob)
    g = native.GgmlFile(str(p))
    same_as_oracle(g, o)
    assert g.cfg.n_audio_state == 128 and g.cfg.ftype == 1
    for name, a in m.t.items():
        assert g.raw(name) == np.ascontiguousarray(a).tobytes()
    g.close()


def _mutants(blob, n, seed):
    """Seeded corruptions of a valid file: byte flips, truncations, and 32-bit
    fields overwritten with edge values (0, -1, 1, 2^31 - 1, -2^31, random)."""
    rng = np.random.default_rng(seed)
    edges = [0, -1, 1, 2 ** 31 - 1, -2 ** 31, 3, 1 << 20]
    for i in range(n):
        b = bytearray(blob)
        kind = i % 3
        if kind == 0:
            for _ in range(int(rng.integers(1, 5))):
                b[int(rng.integers(0, len(b)))] ^= int(rng.integers(1, 256))
        elif kind == 1:
            b = b[:int(rng.integers(0, len(b)))]
        else:
            off = int(rng.integers(0, len(b) - 4)) & ~3
            v = edges[int(rng.integers(0, len(edges)))] if rng.random() < 0.7 else int(rng.integers(-2 ** 31, 2 ** 31))
            b[off:off + 4] = struct.pack("<i", v)
        yield bytes(b)


def test_corrupted_files_classify_like_the_reference():
    """Differential robustness of the parser on untrusted input: 1,500 seeded
    corruptions of a valid file with every stored type go through
    fwhip_ggml_open_bytes and the oracle's GgmlModel::parse restatement; both
    accept the same files (then with the same directory and payloads) and
    reject the rest with the same error class.  Built with the host sanitizers
    (build.py asan), this also shows no out-of-bounds access on any of them."""
    blob = header(2008) + struct.pack("<iif", 1, 1, 0.25) + struct.pack("<i", 2) + struct.pack("<I", 2) + b"hi" + \
        struct.pack("<I", 1) + b"!"
    rng = np.random.default_rng(3)
    for i, t in enumerate([G.F32, G.F16, G.Q4_0, G.Q8_0, G.Q4_K, G.Q6_K]):
        qk = G.BLOCKS[t][0] if t in G.BLOCKS else 1
        name = f"t{i}.w"
        if t == G.F32:
            payload = rng.standard_normal(6 * qk).astype(np.float32).tobytes()
        elif t == G.F16:
            payload = rng.standard_normal(6 * qk).astype(np.float16).tobytes()
        else:
            payload = random_payload(t, 6 * qk, i)
        blob += struct.pack("<5i", 2, len(name), t, 2 * qk, 3) + name.encode() + payload
    same_as_oracle(native.GgmlFile(blob), G.parse(blob))
    n_ok = n_nul = 0
    for b in _mutants(blob, 1500, 7):
        try:
            m = G.parse(b)
        except (G.InvalidRequest, G.Unsupported) as e:
            with pytest.raises(native.FwhipError) as got:
                native.GgmlFile(b)
            assert got.value.code == CODE[type(e)], (str(got.value), str(e))
            continue
        if any("\0" in name for name in m.names()):
            # a NUL byte in a name: the reference loads it, the C ABI cannot
            # pass the name and refuses the file (the caller's CPU route)
            with pytest.raises(native.FwhipError) as got:
                native.GgmlFile(b)
            assert got.value.code == abi.ERR_UNSUPPORTED and "nul-in-tensor-name" in str(got.value)
            n_nul += 1
            continue
        g = native.GgmlFile(b)
        same_as_oracle(g, m)
        g.close()
        n_ok += 1
    assert 50 < n_ok < 1450 and n_nul > 0, (n_ok, n_nul)  # every outcome is exercised
