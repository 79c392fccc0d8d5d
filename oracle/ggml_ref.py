"""numpy restatement of the reference's ggml model-file reader and its
dequantizers (src/native_engine/ggml.rs).

TEST INFRASTRUCTURE: imported only by tests/ as the checker of the library's
ggml reader (fwhip_ggml_*) and of its GPU dequantization kernels — never by the
product package.

Every function follows the cited reference code step by step, in float32 with
one rounding per operation as Rust evaluates it (no contraction):

- `parse`            GgmlModel::parse                    ggml.rs:982-1136
- `byte_len`         ggml_byte_len                       ggml.rs:386-474
- `tensor_f32`       GgmlModel::tensor_f32               ggml.rs:1478-1632
- `dequant_q8_0`     dequant_q8_0                        ggml.rs:529-547
- `dequant_q4_0`     dequant_q4_0                        ggml.rs:478-497
- `dequant_q5_0`     dequant_q5_0                        ggml.rs:502-524
- `dequant_q4_1`     dequant_q4_1                        ggml.rs:345-358
- `dequant_q5_1`     dequant_q5_1                        ggml.rs:363-383
- `dequant_q2_k`     dequant_q2_k                        ggml.rs:268-302
- `dequant_q3_k`     dequant_q3_k                        ggml.rs:202-262
- `dequant_q4_k`     dequant_q4_k (get_scale_min_k4)     ggml.rs:117-157
- `dequant_q5_k`     dequant_q5_k                        ggml.rs:165-196
- `dequant_q6_k`     dequant_q6_k                        ggml.rs:307-340

Pins (tests/test_oracle_ggml.py): the reference's own known-answer blocks for
every quantized type (ggml.rs:2105-2480), its f16 bit patterns (ggml.rs:2953)
and synthetic-blob parser cases (ggml.rs:2866-3180), and a second restatement
that decodes each element from its bit position alone (tests/ggml_elementwise.py)
on random blocks.
"""
from __future__ import annotations

import struct

import numpy as np

GGML_MAGIC = 0x67676D6C
MAX_DIMS = 4
QNT_VERSION_FACTOR = 1000

F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 = 0, 1, 2, 3, 6, 7, 8
Q2_K, Q3_K, Q4_K, Q5_K, Q6_K = 10, 11, 12, 13, 14

# ttype -> (values per block, bytes per block, lower-case name)
BLOCKS = {
    F32: (1, 4, "f32"), F16: (1, 2, "f16"),
    Q4_0: (32, 18, "q4_0"), Q4_1: (32, 20, "q4_1"), Q5_0: (32, 22, "q5_0"), Q5_1: (32, 24, "q5_1"),
    Q8_0: (32, 34, "q8_0"),
    Q2_K: (256, 84, "q2_k"), Q3_K: (256, 110, "q3_k"), Q4_K: (256, 144, "q4_k"), Q5_K: (256, 176, "q5_k"),
    Q6_K: (256, 210, "q6_k"),
}
SUPPORTED_BASE_FTYPES = (0, 1, 2, 3, 7, 8, 9, 10, 11, 12, 13, 14)
USIZE_MAX = (1 << 64) - 1


class InvalidRequest(ValueError):
    """FwError::InvalidRequest"""


class Unsupported(ValueError):
    """FwError::Unsupported"""


# --------------------------------------------------------------------------
# dequantization

def _f16(raw: np.ndarray, off) -> np.ndarray:
    """f16_at (ggml.rs:87-92): little-endian binary16 at byte offset `off` of
    each block row, widened exactly to f32."""
    lo = raw[:, off].astype(np.uint16)
    hi = raw[:, off + 1].astype(np.uint16)
    return (lo | (hi << 8)).view(np.float16).astype(np.float32)


def _blocks(raw, n: int, t: int) -> np.ndarray:
    qk, bb, _ = BLOCKS[t]
    a = np.frombuffer(bytes(raw), dtype=np.uint8) if not isinstance(raw, np.ndarray) else raw.view(np.uint8)
    nb = n // qk
    return a[: nb * bb].reshape(nb, bb)


def dequant_q8_0(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q8_0)
    d = _f16(b, 0)[:, None]
    q = b[:, 2:34].view(np.int8).astype(np.float32)
    return (q * d).reshape(-1)


def dequant_q4_0(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q4_0)
    d = _f16(b, 0)[:, None]
    qs = b[:, 2:18].astype(np.int32)
    x0 = ((qs & 0x0F) - 8).astype(np.float32)
    x1 = ((qs >> 4) - 8).astype(np.float32)
    return np.concatenate([x0 * d, x1 * d], axis=1).reshape(-1)


def _qh_u32(b: np.ndarray, off: int) -> np.ndarray:
    return (b[:, off].astype(np.uint32) | (b[:, off + 1].astype(np.uint32) << 8) |
            (b[:, off + 2].astype(np.uint32) << 16) | (b[:, off + 3].astype(np.uint32) << 24))


def _q5_values(b: np.ndarray, qh_off: int, qs_off: int):
    qh = _qh_u32(b, qh_off)[:, None]
    j = np.arange(16, dtype=np.uint32)[None, :]
    qs = b[:, qs_off:qs_off + 16].astype(np.uint32)
    xh0 = ((qh >> j) << 4) & 0x10
    xh1 = (qh >> (j + 12)) & 0x10
    return (qs & 0x0F) | xh0, (qs >> 4) | xh1


def dequant_q5_0(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q5_0)
    d = _f16(b, 0)[:, None]
    x0, x1 = _q5_values(b, 2, 6)
    x0 = (x0.astype(np.int32) - 16).astype(np.float32)
    x1 = (x1.astype(np.int32) - 16).astype(np.float32)
    return np.concatenate([x0 * d, x1 * d], axis=1).reshape(-1)


def dequant_q4_1(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q4_1)
    d = _f16(b, 0)[:, None]
    m = _f16(b, 2)[:, None]
    qs = b[:, 4:20]
    x0 = (qs & 0x0F).astype(np.float32)
    x1 = (qs >> 4).astype(np.float32)
    return np.concatenate([x0 * d + m, x1 * d + m], axis=1).reshape(-1)


def dequant_q5_1(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q5_1)
    d = _f16(b, 0)[:, None]
    m = _f16(b, 2)[:, None]
    x0, x1 = _q5_values(b, 4, 8)
    return np.concatenate([x0.astype(np.float32) * d + m, x1.astype(np.float32) * d + m], axis=1).reshape(-1)


def dequant_q2_k(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q2_K)
    scales = b[:, 0:16]
    qs = b[:, 16:80]
    d = _f16(b, 80)[:, None]
    dmin = _f16(b, 82)[:, None]
    out = np.empty((b.shape[0], 256), np.float32)
    y = 0
    is_ = 0
    for nblk in range(2):
        qoff = nblk * 32
        for j in range(4):
            shift = 2 * j
            for half in range(2):
                sc = scales[:, is_:is_ + 1]
                is_ += 1
                dl = d * (sc & 0x0F).astype(np.float32)
                ml = dmin * (sc >> 4).astype(np.float32)
                q = ((qs[:, qoff + 16 * half: qoff + 16 * half + 16] >> shift) & 3).astype(np.float32)
                out[:, y:y + 16] = dl * q - ml
                y += 16
    return out.reshape(-1)


def dequant_q3_k(raw, n: int) -> np.ndarray:
    KMASK1, KMASK2 = np.uint32(0x03030303), np.uint32(0x0F0F0F0F)
    b = _blocks(raw, n, Q3_K)
    hmask = b[:, 0:32]
    qs = b[:, 32:96]
    sc = b[:, 96:108]
    d_all = _f16(b, 108)[:, None]
    a0 = _qh_u32(sc, 0)
    a1 = _qh_u32(sc, 4)
    tmp = _qh_u32(sc, 8)
    aux = [
        (a0 & KMASK2) | ((tmp & KMASK1) << 4),
        (a1 & KMASK2) | (((tmp >> 2) & KMASK1) << 4),
        ((a0 >> 4) & KMASK2) | (((tmp >> 4) & KMASK1) << 4),
        ((a1 >> 4) & KMASK2) | (((tmp >> 6) & KMASK1) << 4),
    ]
    scales = np.stack([((w >> (8 * k)) & 0xFF).astype(np.uint8).view(np.int8) for w in aux for k in range(4)],
                      axis=1).astype(np.int32)
    out = np.empty((b.shape[0], 256), np.float32)
    y = 0
    is_ = 0
    for nblk in range(2):
        qoff = nblk * 32
        for j in range(4):
            shift = 2 * j
            m = 1 << (nblk * 4 + j)
            for half in range(2):
                dl = (scales[:, is_:is_ + 1] - 32).astype(np.float32) * d_all
                is_ += 1
                q2 = ((qs[:, qoff + 16 * half: qoff + 16 * half + 16] >> shift) & 3).astype(np.int32)
                sub = np.where(hmask[:, 16 * half: 16 * half + 16] & m, 0, 4)
                out[:, y:y + 16] = dl * (q2 - sub).astype(np.float32)
                y += 16
    return out.reshape(-1)


def get_scale_min_k4(j: int, scales: np.ndarray):
    """get_scale_min_k4 (ggml.rs:117-126) over a [blocks, 12] byte array."""
    s = scales.astype(np.uint8)
    if j < 4:
        return s[:, j] & 63, s[:, j + 4] & 63
    d = (s[:, j + 4] & 0x0F) | ((s[:, j - 4] >> 6) << 4)
    m = (s[:, j + 4] >> 4) | ((s[:, j] >> 6) << 4)
    return d, m


def _k4_group(d, dmin, scales, is_):
    sc, m = get_scale_min_k4(is_, scales)
    return d * sc.astype(np.float32)[:, None], dmin * m.astype(np.float32)[:, None]


def dequant_q4_k(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q4_K)
    d = _f16(b, 0)[:, None]
    dmin = _f16(b, 2)[:, None]
    scales = b[:, 4:16]
    qs = b[:, 16:144]
    out = np.empty((b.shape[0], 256), np.float32)
    for g in range(4):
        d1, m1 = _k4_group(d, dmin, scales, 2 * g)
        d2, m2 = _k4_group(d, dmin, scales, 2 * g + 1)
        q = qs[:, 32 * g: 32 * g + 32]
        out[:, 64 * g: 64 * g + 32] = d1 * (q & 0x0F).astype(np.float32) - m1
        out[:, 64 * g + 32: 64 * g + 64] = d2 * (q >> 4).astype(np.float32) - m2
    return out.reshape(-1)


def dequant_q5_k(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q5_K)
    d = _f16(b, 0)[:, None]
    dmin = _f16(b, 2)[:, None]
    scales = b[:, 4:16]
    qh = b[:, 16:48]
    ql = b[:, 48:176]
    out = np.empty((b.shape[0], 256), np.float32)
    for g in range(4):
        u1, u2 = 1 << (2 * g), 1 << (2 * g + 1)
        d1, m1 = _k4_group(d, dmin, scales, 2 * g)
        d2, m2 = _k4_group(d, dmin, scales, 2 * g + 1)
        q = ql[:, 32 * g: 32 * g + 32]
        hi1 = np.where(qh & u1, 16, 0)
        hi2 = np.where(qh & u2, 16, 0)
        out[:, 64 * g: 64 * g + 32] = d1 * ((q & 0x0F) + hi1).astype(np.float32) - m1
        out[:, 64 * g + 32: 64 * g + 64] = d2 * ((q >> 4) + hi2).astype(np.float32) - m2
    return out.reshape(-1)


def dequant_q6_k(raw, n: int) -> np.ndarray:
    b = _blocks(raw, n, Q6_K)
    ql = b[:, 0:128].astype(np.int32)
    qh = b[:, 128:192].astype(np.int32)
    scales = b[:, 192:208].view(np.int8).astype(np.float32)
    d = _f16(b, 208)[:, None]
    out = np.empty((b.shape[0], 256), np.float32)
    for chunk in range(2):
        qlo, qho, sco, yo = chunk * 64, chunk * 32, chunk * 8, chunk * 128
        l = np.arange(32)
        is_ = l // 16
        a = ql[:, qlo + l]
        c = ql[:, qlo + l + 32]
        h = qh[:, qho + l]
        q1 = ((a & 0x0F) | ((h & 3) << 4)) - 32
        q2 = ((c & 0x0F) | (((h >> 2) & 3) << 4)) - 32
        q3 = ((a >> 4) | (((h >> 4) & 3) << 4)) - 32
        q4 = ((c >> 4) | (((h >> 6) & 3) << 4)) - 32
        for k, q in enumerate((q1, q2, q3, q4)):
            sc = scales[:, sco + is_ + 2 * k]
            out[:, yo + 32 * k: yo + 32 * k + 32] = (d * sc) * q.astype(np.float32)
    return out.reshape(-1)


DEQUANT = {
    Q8_0: dequant_q8_0, Q4_0: dequant_q4_0, Q5_0: dequant_q5_0, Q4_1: dequant_q4_1, Q5_1: dequant_q5_1,
    Q2_K: dequant_q2_k, Q3_K: dequant_q3_k, Q4_K: dequant_q4_k, Q5_K: dequant_q5_k, Q6_K: dequant_q6_k,
}


def dequant(t: int, raw, n: int) -> np.ndarray:
    """The per-type decode of tensor_f32 (ggml.rs:1478-1632) on a payload of
    byte_len(t, n) bytes."""
    if t == F32:
        return np.frombuffer(bytes(raw), dtype="<f4", count=n).astype(np.float32)
    if t == F16:
        return np.frombuffer(bytes(raw), dtype="<u2", count=n).view(np.float16).astype(np.float32)
    return DEQUANT[t](raw, n)


def byte_len(t: int, n: int, name: str) -> int:
    """ggml_byte_len (ggml.rs:386-474)."""
    qk, bb, tn = BLOCKS[t]
    if qk > 1 and n % qk:
        raise InvalidRequest(f"tensor '{name}' {tn} element count {n} is not a multiple of {qk}")
    v = (n // qk) * bb
    if v > USIZE_MAX:
        raise InvalidRequest(f"tensor '{name}' byte length overflow")
    return v


# --------------------------------------------------------------------------
# file structure

class _Cursor:
    """Cursor (ggml.rs:1947-2018): bounds-checked little-endian reads."""

    def __init__(self, buf: bytes):
        self.buf, self.pos = buf, 0

    def at_end(self) -> bool:
        return self.pos >= len(self.buf)

    def read_bytes(self, n: int) -> bytes:
        end = self.pos + n
        if end > len(self.buf):
            raise InvalidRequest(f"unexpected end of file: needed {n} byte(s) at offset {self.pos}, have {len(self.buf)}")
        out = self.buf[self.pos:end]
        self.pos = end
        return out

    def u32(self) -> int:
        return struct.unpack("<I", self.read_bytes(4))[0]

    def i32(self) -> int:
        return struct.unpack("<i", self.read_bytes(4))[0]

    def f32(self) -> float:
        return struct.unpack("<f", self.read_bytes(4))[0]


def _usize(v: int, what: str) -> int:
    if v < 0:
        raise InvalidRequest(f"{what} is negative ({v})")
    return v


class Model:
    def __init__(self, blob: bytes, hparams, filters, n_mel, n_fft, vocab, tensors):
        self.blob, self.hparams, self.filters = blob, hparams, filters
        self.n_mel, self.n_fft, self.vocab, self.tensors = n_mel, n_fft, vocab, tensors

    def names(self):
        return sorted(self.tensors)

    def raw(self, name: str) -> bytes:
        shape, t, off, nbytes = self.tensors[name]
        return self.blob[off:off + nbytes]


HPARAM_NAMES = ("n_vocab", "n_audio_ctx", "n_audio_state", "n_audio_head", "n_audio_layer", "n_text_ctx",
                "n_text_state", "n_text_head", "n_text_layer", "n_mels", "ftype")


def parse(blob: bytes) -> Model:
    """GgmlModel::parse (ggml.rs:982-1136)."""
    cur = _Cursor(bytes(blob))
    magic = cur.u32()
    if magic != GGML_MAGIC:
        raise InvalidRequest(f"bad ggml magic: got {magic:#010x}, expected {GGML_MAGIC:#010x}")
    hp = [cur.i32() for _ in range(11)]
    base = hp[10] % QNT_VERSION_FACTOR  # rem_euclid: Python's % is already non-negative here
    if base not in SUPPORTED_BASE_FTYPES:
        raise Unsupported(f"quantized ggml ftype {hp[10]} (base {base}) is not supported (only base 0=f32, 1=f16, "
                          "2=q4_0, 3=q4_1, 7=q8_0, 8=q5_0, 9=q5_1, 10=q2_k, 11=q3_k, 12=q4_k, 13=q5_k, 14=q6_k)")
    n_mel = _usize(cur.i32(), "filters.n_mel")
    n_fft = _usize(cur.i32(), "filters.n_fft")
    filters = [cur.f32() for _ in range(n_mel * n_fft)]
    n_vocab = _usize(cur.i32(), "file vocab count")
    vocab = []
    for _ in range(n_vocab):
        ln = cur.u32()
        vocab.append(cur.read_bytes(ln))
    tensors = {}
    while not cur.at_end():
        n_dims = cur.i32()
        name_len = cur.i32()
        ttype = cur.i32()
        n_dims = _usize(n_dims, "tensor n_dims")
        if n_dims == 0 or n_dims > MAX_DIMS:
            raise InvalidRequest(f"tensor n_dims {n_dims} out of range 1..={MAX_DIMS}")
        name_len = _usize(name_len, "tensor name length")
        if ttype not in BLOCKS:
            raise Unsupported(f"tensor element type {ttype} is not supported (only 0=f32, 1=f16, 2=q4_0, 3=q4_1, "
                              "6=q5_0, 7=q5_1, 8=q8_0, 10=q2_k, 11=q3_k, 12=q4_k, 13=q5_k, 14=q6_k)")
        ne = [_usize(cur.i32(), "tensor dimension") for _ in range(n_dims)]
        try:
            name = cur.read_bytes(name_len).decode("utf-8")
        except UnicodeDecodeError:
            raise InvalidRequest("tensor name is not valid UTF-8") from None
        shape = ne[::-1]
        n = 1
        for dim in shape:
            n *= dim
            if n > USIZE_MAX:
                raise InvalidRequest(f"tensor '{name}' element count overflow")
        nbytes = byte_len(ttype, n, name)
        off = cur.pos
        cur.read_bytes(nbytes)
        tensors[name] = (shape, ttype, off, nbytes)
    return Model(cur.buf, hp, np.array(filters, np.float32), n_mel, n_fft, vocab, tensors)


def tensor_f32(m: Model, name: str):
    """GgmlModel::tensor_f32 (ggml.rs:1478-1632): (logical shape, f32 values)."""
    if name not in m.tensors:
        raise InvalidRequest(f"unknown tensor '{name}'")
    shape, t, _, _ = m.tensors[name]
    n = 1
    for dim in shape:
        n *= dim
    return shape, dequant(t, m.raw(name), n)
