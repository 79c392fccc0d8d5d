"""A second restatement of the ggml dequantizers, written per output element:
element i of a block is decoded from the byte and bit positions the published
block layouts give for it (whisper.cpp / ggml block formats: `block_q4_0` ...
`block_q6_K`), with scalar float32 arithmetic, instead of the block loops of
oracle/ggml_ref.py. The two agreeing on random blocks pins the index algebra of
both (a swapped half, a wrong shift or scale index fails one of them)."""
from __future__ import annotations

import numpy as np

f32 = np.float32


def _h(b, off):
    return f32(np.array([b[off] | (b[off + 1] << 8)], np.uint16).view(np.float16)[0])


def _u32(b, off):
    return b[off] | (b[off + 1] << 8) | (b[off + 2] << 16) | (b[off + 3] << 24)


def q8_0(b, i):
    q = b[2 + i]
    return f32(q - 256 if q > 127 else q) * _h(b, 0)


def q4_0(b, i):
    nib = (b[2 + i % 16] >> (4 * (i // 16))) & 15
    return f32(nib - 8) * _h(b, 0)


def _q5(b, i, qh_off, qs_off):
    qh = _u32(b, qh_off)
    nib = (b[qs_off + i % 16] >> (4 * (i // 16))) & 15
    return nib | (((qh >> i) & 1) << 4)  # bit i of qh is the 5th bit of element i


def q5_0(b, i):
    return f32(_q5(b, i, 2, 6) - 16) * _h(b, 0)


def q4_1(b, i):
    nib = (b[4 + i % 16] >> (4 * (i // 16))) & 15
    return f32(nib) * _h(b, 0) + _h(b, 2)


def q5_1(b, i):
    return f32(_q5(b, i, 4, 8)) * _h(b, 0) + _h(b, 2)


def q2_k(b, i):
    half, r = divmod(i, 128)  # 128-value halves share 32 quant bytes
    j, t = divmod(r, 32)      # 2-bit plane j, element t of the 32
    sc = b[half * 8 + 2 * j + t // 16]
    q = (b[16 + half * 32 + t] >> (2 * j)) & 3
    return _h(b, 80) * f32(sc & 15) * f32(q) - _h(b, 82) * f32(sc >> 4)


def _q3_scale(sc, k):
    """6-bit scale k of 16: low 4 bits from byte k % 8 (low nibble for k < 8,
    high nibble after), high 2 bits from byte 8 + k % 4, bit pair k // 4."""
    lo = (sc[k % 8] >> (4 * (k // 8))) & 15
    hi = (sc[8 + k % 4] >> (2 * (k // 4))) & 3
    return lo | (hi << 4)


def q3_k(b, i):
    half, r = divmod(i, 128)
    j, t = divmod(r, 32)
    k = half * 8 + 2 * j + t // 16
    dl = f32(_q3_scale(b[96:108], k) - 32) * _h(b, 108)
    q = (b[32 + half * 32 + t] >> (2 * j)) & 3
    high = (b[t] >> (half * 4 + j)) & 1
    return dl * f32(q - (0 if high else 4))


def _k4_scale(sc, k):
    """6-bit (scale, min) pair k of 8 (k < 4: low 6 bits of bytes k, k+4;
    k >= 4: a nibble of byte k+4 with the top 2 bits of bytes k-4, k)."""
    if k < 4:
        return sc[k] & 63, sc[k + 4] & 63
    return (sc[k + 4] & 15) | ((sc[k - 4] >> 6) << 4), (sc[k + 4] >> 4) | ((sc[k] >> 6) << 4)


def q4_k(b, i):
    g, r = divmod(i, 64)
    h, t = divmod(r, 32)
    s, m = _k4_scale(b[4:16], 2 * g + h)
    q = (b[16 + 32 * g + t] >> (4 * h)) & 15
    return (_h(b, 0) * f32(s)) * f32(q) - _h(b, 2) * f32(m)


def q5_k(b, i):
    g, r = divmod(i, 64)
    h, t = divmod(r, 32)
    s, m = _k4_scale(b[4:16], 2 * g + h)
    q = ((b[48 + 32 * g + t] >> (4 * h)) & 15) + 16 * ((b[16 + t] >> (2 * g + h)) & 1)
    return (_h(b, 0) * f32(s)) * f32(q) - _h(b, 2) * f32(m)


def q6_k(b, i):
    c, r = divmod(i, 128)
    k, t = divmod(r, 32)  # quarter k: low/high nibble of ql[t] or ql[t + 32]
    lo = (b[c * 64 + t + 32 * (k & 1)] >> (4 * (k >> 1))) & 15
    hi = (b[128 + c * 32 + t] >> (2 * k)) & 3
    sc = b[192 + c * 8 + t // 16 + 2 * k]
    sc = sc - 256 if sc > 127 else sc
    return (_h(b, 208) * f32(sc)) * f32((lo | (hi << 4)) - 32)


FUNCS = {2: (q4_0, 32, 18), 3: (q4_1, 32, 20), 6: (q5_0, 32, 22), 7: (q5_1, 32, 24), 8: (q8_0, 32, 34),
         10: (q2_k, 256, 84), 11: (q3_k, 256, 110), 12: (q4_k, 256, 144), 13: (q5_k, 256, 176),
         14: (q6_k, 256, 210)}


def dequant(t: int, raw: bytes, n: int) -> np.ndarray:
    fn, qk, bb = FUNCS[t]
    raw = [int(x) for x in raw]
    out = np.empty(n, np.float32)
    for blk in range(n // qk):
        b = raw[blk * bb:(blk + 1) * bb]
        for i in range(qk):
            out[blk * qk + i] = fn(b, i)
    return out
