"""Writer of whisper.cpp ggml model files (the layout GgmlModel::load reads,
src/native_engine/ggml.rs:1-47), and the seeded-weight model file.

File order, all little-endian, no padding: the magic 0x67676d6c; eleven i32
hparams (n_vocab, n_audio_ctx, n_audio_state, n_audio_head, n_audio_layer,
n_text_ctx, n_text_state, n_text_head, n_text_layer, n_mels, ftype); the mel
filterbank (n_mel, n_fft as i32, then n_mel * n_fft f32); the vocab (count as
i32, then per token a u32 length and its bytes); then per tensor n_dims,
name_len and ttype as i32, the dims in ggml order (fastest axis first: the
logical row-major shape reversed), the name bytes and the payload.

`write_model` writes a synth.Model (seeded random-init weights) in this
format, the tensor names and shapes of the loaders (encoder.rs:764-1029,
decoder.rs:752-932) — the seeded-weight file a Rust engine run can load
through GgmlModel::load as well as through fwhip_ggml_open.  The test-model
writer of the reference follows the same pattern (mod.rs:2872-3078).
"""
from __future__ import annotations

import struct
from typing import BinaryIO, Iterable, Sequence

import numpy as np

MAGIC = 0x67676D6C
F32, F16 = 0, 1


def tensor_record(name: str, ttype: int, shape: Sequence[int], payload: bytes) -> bytes:
    """One directory entry: header, ggml-order dims, name, payload."""
    nb = name.encode()
    head = struct.pack("<iii", len(shape), len(nb), ttype) + struct.pack(f"<{len(shape)}i", *reversed(shape))
    return head + nb + payload


def write(f: BinaryIO, hparams: Sequence[int], filters: np.ndarray, vocab: Iterable[bytes],
          tensors: Iterable[tuple]) -> None:
    """Write a model file to the binary stream `f`; `tensors` yields
    (name, ttype, logical shape, payload bytes)."""
    if len(hparams) != 11:
        raise ValueError("hparams: eleven i32 values (the last is ftype)")
    fb = np.ascontiguousarray(filters, dtype="<f4")
    f.write(struct.pack("<I", MAGIC) + struct.pack("<11i", *hparams))
    f.write(struct.pack("<ii", fb.shape[0], fb.shape[1]) + fb.tobytes())
    vocab = list(vocab)
    f.write(struct.pack("<i", len(vocab)))
    for tok in vocab:
        f.write(struct.pack("<I", len(tok)) + bytes(tok))
    for name, ttype, shape, payload in tensors:
        f.write(tensor_record(name, ttype, shape, payload))


def synthetic_vocab(n_tokens: int) -> list:
    """A byte-level vocab of n_tokens entries: the 256 single bytes, then
    placeholder tokens (the seeded model has no trained merges)."""
    return [bytes([i]) for i in range(min(n_tokens, 256))] + [f"<{i}>".encode() for i in range(256, n_tokens)]


def model_tensors(model, linear_ttype: int = F16):
    """(name, ttype, shape, payload) of every tensor of a synth.Model: its f16
    tensors (binary16 bits, uint16) as f16 — or as f32 values when
    linear_ttype is F32 — and its f32 tensors as f32."""
    for name in sorted(model.t):
        a = model.t[name]
        if a.dtype == np.uint16:
            if linear_ttype == F16:
                yield name, F16, a.shape, np.ascontiguousarray(a, dtype="<u2").tobytes()
            else:
                yield name, F32, a.shape, a.view(np.float16).astype("<f4").tobytes()
        else:
            yield name, F32, a.shape, np.ascontiguousarray(a, dtype="<f4").tobytes()


def hparams11(cfg, ftype: int) -> list:
    """The header's eleven i32 values for a model shape (WhisperHParams order)."""
    return [cfg.n_vocab, cfg.n_audio_ctx, cfg.n_audio_state, cfg.n_audio_head, cfg.n_audio_layer, cfg.n_text_ctx,
            cfg.n_text_state, cfg.n_text_head, cfg.n_text_layer, cfg.n_mels, ftype]


def write_model(path, model, filters: np.ndarray | None = None, vocab: Sequence[bytes] | None = None,
                linear_ttype: int = F16) -> None:
    """The seeded-weight ggml file of a synth.Model (ftype 1 when the linears
    are f16, 0 when they are written as f32)."""
    from . import synth

    c = model.cfg
    if filters is None:
        filters = synth.mel_filterbank(c.n_mels)
    if vocab is None:
        vocab = synthetic_vocab(model.tokens.eot)
    hp = hparams11(c, 1 if linear_ttype == F16 else 0)
    with open(path, "wb") as f:
        write(f, hp, filters, vocab, model_tensors(model, linear_ttype))
