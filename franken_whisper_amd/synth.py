"""Seeded synthetic Whisper models and inputs.

Weights follow the ggml tensor names and layouts the reference loads
(src/native_engine/encoder.rs:772-1029, decoder.rs:752-932): every >=2-D tensor
is N(0, 0.02) drawn in double, rounded to f32 and then RNE to f16 (positional
embeddings stay f32), LayerNorm gains are 1 and biases 0, linear/conv biases are
N(0, 0.02) f32.  Generation is counter-based (SplitMix64 + Box-Muller keyed by
seed and tensor name, csrc/synth.c) so any tensor can be regenerated alone.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

from . import abi

_HERE = os.path.dirname(os.path.abspath(__file__))
_SYNTH_SO = os.path.join(_HERE, "lib", "libfwsynth.so")
_lib = None


def _synth():
    global _lib
    if _lib is None:
        if not os.path.exists(_SYNTH_SO):
            raise RuntimeError(f"{_SYNTH_SO} missing: run __graft_entry__.build()")
        lib = C.CDLL(_SYNTH_SO)
        lib.fws_normal_f32.argtypes = [C.c_uint64, C.c_char_p, C.c_double, C.c_int64, abi.f32p]
        lib.fws_normal_f16.argtypes = [C.c_uint64, C.c_char_p, C.c_double, C.c_int64, abi.u16p]
        lib.fws_uniform_i32.argtypes = [C.c_uint64, C.c_char_p, C.c_int32, C.c_int32, C.c_int64,
                                        C.POINTER(C.c_int32)]
        lib.fws_audio.argtypes = [C.c_uint64, C.c_int64, C.c_int, abi.f32p]
        _lib = lib
    return _lib


def normal_f16(seed: int, name: str, shape, std: float = 0.02) -> np.ndarray:
    out = np.empty(shape, dtype=np.uint16)
    _synth().fws_normal_f16(seed, name.encode(), std, out.size, abi.ptr(out, C.c_uint16))
    return out


def normal_f32(seed: int, name: str, shape, std: float = 0.02) -> np.ndarray:
    out = np.empty(shape, dtype=np.float32)
    _synth().fws_normal_f32(seed, name.encode(), std, out.size, abi.ptr(out, C.c_float))
    return out


def uniform_i32(seed: int, name: str, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    _synth().fws_uniform_i32(seed, name.encode(), lo, hi, n, abi.ptr(out, C.c_int32))
    return out


def audio(seed: int, seconds: float, gaps: bool = False) -> np.ndarray:
    n = int(round(seconds * 16000))
    out = np.empty(n, dtype=np.float32)
    _synth().fws_audio(seed, n, 1 if gaps else 0, abi.ptr(out, C.c_float))
    return out


@dataclass(frozen=True)
class Config:
    name: str
    n_vocab: int
    n_audio_ctx: int
    n_audio_state: int
    n_audio_head: int
    n_audio_layer: int
    n_text_ctx: int
    n_text_state: int
    n_text_head: int
    n_text_layer: int
    n_mels: int

    def hparams(self) -> abi.HParams:
        return abi.HParams(self.n_vocab, self.n_audio_ctx, self.n_audio_state, self.n_audio_head,
                           self.n_audio_layer, self.n_text_ctx, self.n_text_state,
                           self.n_text_head, self.n_text_layer, self.n_mels)

    @property
    def multilingual(self) -> bool:  # WhisperHParams::is_multilingual, mod.rs:74-76
        return self.n_vocab >= 51865


# Model shapes (mod.rs:703-728).
TINY_EN = Config("tiny.en", 51864, 1500, 384, 6, 4, 448, 384, 6, 4, 80)
TURBO = Config("large-v3-turbo", 51866, 1500, 1280, 20, 32, 448, 1280, 20, 4, 128)
# A small shape for fast parity tests: real vocabulary (so the special ids are
# the real ones), d_head 64, short audio context.
MICRO = Config("micro", 51864, 64, 128, 2, 2, 64, 128, 2, 2, 16)
MICRO_ML = Config("micro-ml", 51866, 64, 128, 2, 2, 64, 128, 2, 2, 16)
CONFIGS = {c.name: c for c in (TINY_EN, TURBO, MICRO, MICRO_ML)}


class Tokens:
    """Special token ids, Tokenizer::from_vocab (tokenizer.rs:230-300)."""

    def __init__(self, cfg: Config):
        ml = cfg.multilingual
        n_langs = cfg.n_vocab - 51765 - (1 if ml else 0)
        self.eot, self.sot = 50256, 50257
        self.translate, self.transcribe, self.solm = 50357, 50358, 50359
        self.sot_prev, self.no_speech, self.no_timestamps, self.timestamp_begin = 50360, 50361, 50362, 50363
        if ml:
            dt = n_langs - 98
            self.eot += 1
            self.sot += 1
            self.translate += dt
            self.transcribe += dt
            self.solm += dt
            self.sot_prev += dt
            self.no_speech += dt
            self.no_timestamps += dt
            self.timestamp_begin += dt
        self.multilingual = ml
        self.space = 220  # b" " in the whisper byte-level BPE vocabulary

    def sot_sequence(self, language_id: int = 0, translate: bool = False,
                     timestamps: bool = False):
        """Tokenizer::sot_sequence, tokenizer.rs:477-510."""
        seq = [self.sot]
        if self.multilingual:
            seq.append(self.sot + 1 + language_id)
            seq.append(self.translate if translate else self.transcribe)
        if not timestamps:
            seq.append(self.no_timestamps)
        return seq

    def filter(self) -> abi.Filter:
        return abi.Filter(self.eot, self.sot, self.sot_prev, self.solm, self.no_speech,
                          self.no_timestamps, self.translate, self.transcribe,
                          self.timestamp_begin, self.space, 100)


class Model:
    """Seeded random-init weights for `cfg`, plus the ctypes descriptors that
    point into them (kept alive by this object)."""

    def __init__(self, cfg: Config, seed: int = 0, encoder: bool = True, decoder: bool = True):
        self.cfg, self.seed = cfg, seed
        self.t = {}
        self.tokens = Tokens(cfg)
        if encoder:
            self._make_encoder()
        if decoder:
            self._make_decoder()

    # -- tensors --
    def _w16(self, name, shape):
        self.t[name] = normal_f16(self.seed, name, shape)

    def _w32(self, name, shape):
        self.t[name] = normal_f32(self.seed, name, shape)

    def _ln(self, prefix, n):
        self.t[prefix + ".weight"] = np.ones(n, np.float32)
        self.t[prefix + ".bias"] = np.zeros(n, np.float32)

    def _make_encoder(self):
        c = self.cfg
        d, nm = c.n_audio_state, c.n_mels
        self._w16("encoder.conv1.weight", (d, nm, 3))
        self._w32("encoder.conv1.bias", (d,))
        self._w16("encoder.conv2.weight", (d, d, 3))
        self._w32("encoder.conv2.bias", (d,))
        self._w32("encoder.positional_embedding", (c.n_audio_ctx, d))
        for i in range(c.n_audio_layer):
            p = f"encoder.blocks.{i}"
            self._ln(p + ".attn_ln", d)
            for nm_, bias in (("query", True), ("key", False), ("value", True), ("out", True)):
                self._w16(f"{p}.attn.{nm_}.weight", (d, d))
                if bias:
                    self._w32(f"{p}.attn.{nm_}.bias", (d,))
            self._ln(p + ".mlp_ln", d)
            self._w16(p + ".mlp.0.weight", (4 * d, d))
            self._w32(p + ".mlp.0.bias", (4 * d,))
            self._w16(p + ".mlp.2.weight", (d, 4 * d))
            self._w32(p + ".mlp.2.bias", (d,))
        self._ln("encoder.ln_post", d)

    def _make_decoder(self):
        c = self.cfg
        d = c.n_text_state
        self._w16("decoder.token_embedding.weight", (c.n_vocab, d))
        self._w32("decoder.positional_embedding", (c.n_text_ctx, d))
        for i in range(c.n_text_layer):
            p = f"decoder.blocks.{i}"
            for att in ("attn", "cross_attn"):
                self._ln(f"{p}.{att}_ln", d)
                for nm_, bias in (("query", True), ("key", False), ("value", True), ("out", True)):
                    self._w16(f"{p}.{att}.{nm_}.weight", (d, d))
                    if bias:
                        self._w32(f"{p}.{att}.{nm_}.bias", (d,))
            self._ln(p + ".mlp_ln", d)
            self._w16(p + ".mlp.0.weight", (4 * d, d))
            self._w32(p + ".mlp.0.bias", (4 * d,))
            self._w16(p + ".mlp.2.weight", (d, 4 * d))
            self._w32(p + ".mlp.2.bias", (d,))
        self._ln("decoder.ln", d)

    # -- descriptors --
    def _p16(self, n):
        return abi.ptr(self.t[n], C.c_uint16)

    def _p32(self, n):
        return abi.ptr(self.t[n], C.c_float)

    def encoder_weights(self) -> abi.EncoderWeights:
        c = self.cfg
        layers = (abi.EncLayer * c.n_audio_layer)()
        for i in range(c.n_audio_layer):
            p = f"encoder.blocks.{i}"
            a = p + ".attn"
            layers[i] = abi.EncLayer(
                self._p32(p + ".attn_ln.weight"), self._p32(p + ".attn_ln.bias"),
                self._p16(a + ".query.weight"), self._p32(a + ".query.bias"),
                self._p16(a + ".key.weight"),
                self._p16(a + ".value.weight"), self._p32(a + ".value.bias"),
                self._p16(a + ".out.weight"), self._p32(a + ".out.bias"),
                self._p32(p + ".mlp_ln.weight"), self._p32(p + ".mlp_ln.bias"),
                self._p16(p + ".mlp.0.weight"), self._p32(p + ".mlp.0.bias"),
                self._p16(p + ".mlp.2.weight"), self._p32(p + ".mlp.2.bias"))
        self._enc_layers = layers
        return abi.EncoderWeights(
            c.hparams(), self._p16("encoder.conv1.weight"), self._p32("encoder.conv1.bias"),
            self._p16("encoder.conv2.weight"), self._p32("encoder.conv2.bias"),
            self._p32("encoder.positional_embedding"), layers,
            self._p32("encoder.ln_post.weight"), self._p32("encoder.ln_post.bias"))

    def decoder_weights(self) -> abi.DecoderWeights:
        c = self.cfg
        layers = (abi.DecLayer * c.n_text_layer)()
        for i in range(c.n_text_layer):
            p = f"decoder.blocks.{i}"
            a, x = p + ".attn", p + ".cross_attn"
            layers[i] = abi.DecLayer(
                self._p32(p + ".attn_ln.weight"), self._p32(p + ".attn_ln.bias"),
                self._p16(a + ".query.weight"), self._p32(a + ".query.bias"),
                self._p16(a + ".key.weight"),
                self._p16(a + ".value.weight"), self._p32(a + ".value.bias"),
                self._p16(a + ".out.weight"), self._p32(a + ".out.bias"),
                self._p32(p + ".cross_attn_ln.weight"), self._p32(p + ".cross_attn_ln.bias"),
                self._p16(x + ".query.weight"), self._p32(x + ".query.bias"),
                self._p16(x + ".key.weight"),
                self._p16(x + ".value.weight"), self._p32(x + ".value.bias"),
                self._p16(x + ".out.weight"), self._p32(x + ".out.bias"),
                self._p32(p + ".mlp_ln.weight"), self._p32(p + ".mlp_ln.bias"),
                self._p16(p + ".mlp.0.weight"), self._p32(p + ".mlp.0.bias"),
                self._p16(p + ".mlp.2.weight"), self._p32(p + ".mlp.2.bias"))
        self._dec_layers = layers
        return abi.DecoderWeights(
            c.hparams(), self._p16("decoder.token_embedding.weight"),
            self._p32("decoder.positional_embedding"), layers,
            self._p32("decoder.ln.weight"), self._p32("decoder.ln.bias"))


def encoder_states(seed: int, n_streams: int, frames: int, d: int) -> np.ndarray:
    """Seeded N(0,1) f32 encoder states [n_streams, frames, d] (a decoder-step
    input isolated from the encoder)."""
    return normal_f32(seed, "encoder_states", (n_streams, frames, d), std=1.0)


def mel_input(seed: int, n_windows: int, n_frames: int, n_mels: int) -> np.ndarray:
    """Seeded N(0,1) time-major log-mel windows [n_windows, n_frames, n_mels]
    (an encoder input isolated from the log-mel frontend)."""
    return normal_f32(seed, "mel", (n_windows, n_frames, n_mels), std=1.0)


def mel_filterbank(n_mel: int = 128, sample_rate: int = 16000, n_fft: int = 400) -> np.ndarray:
    """Slaney-style triangular mel filterbank [n_mel, n_fft/2 + 1] f32 (the
    construction of Whisper's mel_filters asset: Slaney mel scale, area
    normalization), computed in f64 from the published formulas so the frontend
    runs on a realistic sparse bank without the model file."""
    n_bins = n_fft // 2 + 1
    f_sp, min_log_hz = 200.0 / 3.0, 1000.0
    min_log_mel = min_log_hz / f_sp
    logstep = np.log(6.4) / 27.0

    def hz_to_mel(f):
        f = np.asarray(f, dtype=np.float64)
        return np.where(f >= min_log_hz, min_log_mel + np.log(np.maximum(f, 1e-12) / min_log_hz) / logstep,
                        f / f_sp)

    def mel_to_hz(m):
        m = np.asarray(m, dtype=np.float64)
        return np.where(m >= min_log_mel, min_log_hz * np.exp(logstep * (m - min_log_mel)), f_sp * m)

    fft_hz = np.linspace(0.0, sample_rate / 2.0, n_bins)
    mel_hz = mel_to_hz(np.linspace(hz_to_mel(0.0), hz_to_mel(sample_rate / 2.0), n_mel + 2))
    fdiff = np.diff(mel_hz)
    ramps = mel_hz[:, None] - fft_hz[None, :]
    lower = -ramps[:-2] / fdiff[:-1, None]
    upper = ramps[2:] / fdiff[1:, None]
    w = np.maximum(0.0, np.minimum(lower, upper))
    w *= (2.0 / (mel_hz[2:] - mel_hz[:-2]))[:, None]
    return w.astype(np.float32)
