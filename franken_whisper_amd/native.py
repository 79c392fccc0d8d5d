"""ctypes binding of lib/libfwhip.so (include/fwhip.h).

The product path: every call here runs HIP kernels through the C ABI.  There
is no CPU fallback — a missing or unloadable library raises, and a machine
without a gfx950 GPU gets FWHIP_ERR_UNSUPPORTED from fwhip_init.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

from . import abi

_HERE = os.path.dirname(os.path.abspath(__file__))
# FWHIP_LIB selects another build of the same sources (the host-sanitizer
# build of build.py's "asan" target, for CPU-only tests)
LIB_PATH = os.environ.get("FWHIP_LIB") or os.path.join(_HERE, "lib", "libfwhip.so")

_vp = C.c_void_p
_i32p = C.POINTER(C.c_int32)
_i64p = C.POINTER(C.c_int64)

# name -> (restype, argtypes); every symbol include/fwhip.h declares
SIGNATURES = {
    "fwhip_init": (C.c_int32, [C.c_int32, C.POINTER(_vp)]),
    "fwhip_destroy": (None, [_vp]),
    "fwhip_last_error": (C.c_char_p, []),
    "fwhip_abi_version": (C.c_int32, []),
    "fwhip_malloc": (C.c_int32, [_vp, C.c_size_t, C.POINTER(_vp)]),
    "fwhip_free": (C.c_int32, [_vp, _vp]),
    "fwhip_upload": (C.c_int32, [_vp, _vp, _vp, C.c_size_t]),
    "fwhip_download": (C.c_int32, [_vp, _vp, _vp, C.c_size_t]),
    "fwhip_synchronize": (C.c_int32, [_vp]),
    "fwhip_request_cancel": (C.c_int32, [_vp]),
    "fwhip_kernel_timing": (C.c_int32, [_vp, C.c_int32]),
    "fwhip_kernel_stats": (C.c_int32, [_vp, C.c_int32, _i64p, C.POINTER(C.c_double),
                                       C.POINTER(C.c_double)]),
    "fwhip_encoder_load": (C.c_int32, [_vp, C.POINTER(abi.EncoderWeights), C.c_int32, C.POINTER(_vp)]),
    "fwhip_encoder_free": (None, [_vp]),
    "fwhip_encoder_forward": (C.c_int32, [_vp, _vp, C.c_int64, _i64p, C.c_int32, C.c_int32, _vp,
                                          C.POINTER(abi.ExecRecord)]),
    "fwhip_encoder_forward_time_major": (C.c_int32, [_vp, _vp, C.c_int32, C.c_int32, _vp,
                                                     C.POINTER(abi.ExecRecord)]),
    "fwhip_encoder_set_exact": (C.c_int32, [_vp, C.c_int32]),
    "fwhip_encoder_set_tome": (C.c_int32, [_vp, C.c_int32, C.c_int32]),
    "fwhip_encoder_set_tome_schedule": (C.c_int32, [_vp, C.c_int32, C.c_int32]),
    "fwhip_decoder_set_kv_f16": (C.c_int32, [_vp, C.c_int32]),
    "fwhip_decoder_set_cross_v_block": (C.c_int32, [_vp, C.c_int32]),
    "fwhip_tome_merge": (C.c_int32, [_vp, _vp, C.c_int32, C.c_int32, C.c_int32, C.c_int32, _vp, _vp, _i32p]),
    "fwhip_encoder_gemm_i8": (C.c_int32, [_vp, C.c_int32, C.c_int32, _vp, C.c_int32, _vp, _vp]),
    "fwhip_encoder_gemm_i8_fused": (C.c_int32, [_vp, C.c_int32, C.c_int32, _vp, C.c_int32, C.c_int32, _vp, _vp]),
    "fwhip_decoder_load": (C.c_int32, [_vp, C.POINTER(abi.DecoderWeights), C.c_int32, C.POINTER(_vp)]),
    "fwhip_decoder_free": (None, [_vp]),
    "fwhip_decoder_set_exact": (C.c_int32, [_vp, C.c_int32]),
    "fwhip_dstate_new": (C.c_int32, [_vp, C.c_int32, C.c_int32, C.POINTER(_vp)]),
    "fwhip_dstate_free": (None, [_vp]),
    "fwhip_dstate_set_cross": (C.c_int32, [_vp, _vp]),
    "fwhip_dstate_reset": (C.c_int32, [_vp]),
    "fwhip_dstate_len": (C.c_int32, [_vp, C.c_int32]),
    "fwhip_decoder_step": (C.c_int32, [_vp, _i32p, C.c_int32, _vp, _i32p, C.POINTER(abi.Filter),
                                       C.c_int32]),
    "fwhip_dstate_read": (C.c_int32, [_vp, C.c_int32, C.c_int32, _vp, C.c_size_t]),
    "fwhip_decode_greedy": (C.c_int32, [_vp, _i32p, C.c_int32, C.c_int32, C.POINTER(abi.Filter), _i32p,
                                        _i32p]),
    "fwhip_decode_window": (C.c_int32, [_vp, _i32p, C.c_int32, C.POINTER(abi.Filter), C.POINTER(abi.WindowCfg),
                                        C.POINTER(abi.WindowStream), _i32p, C.POINTER(C.c_float)]),
    "fwhip_transcribe": (C.c_int32, [_vp, _vp, _vp, _vp, C.c_int64, _vp, C.c_int32, C.POINTER(abi.Filter),
                                     C.POINTER(abi.Vocab), C.POINTER(abi.TranscribeParams), C.POINTER(_vp)]),
    "fwhip_transcript_n_segments": (C.c_int32, [_vp]),
    "fwhip_transcript_segment": (C.c_int32, [_vp, C.c_int32, C.POINTER(abi.SegmentInfo)]),
    "fwhip_transcript_n_windows": (C.c_int32, [_vp]),
    "fwhip_transcript_window": (C.c_int32, [_vp, C.c_int32, C.POINTER(abi.WindowInfo)]),
    "fwhip_transcript_free": (None, [_vp]),
    "fwhip_argmax_logits": (C.c_int32, [_vp, _vp, C.c_int32, C.c_int32, C.POINTER(abi.Filter), C.c_int32, _i32p]),
    "fwhip_layer_norm": (C.c_int32, [_vp, _vp, _vp, _vp, C.c_int64, C.c_int32, _vp, C.c_int32]),
    "fwhip_gemm_precision_str": (C.c_char_p, [C.c_int32]),
    "fwhip_mel_frames": (C.c_int64, [C.c_int64]),
    "fwhip_log_mel": (C.c_int32, [_vp, _vp, C.c_int64, _vp, C.c_int32, C.c_int32, _vp]),
    "fwhip_log_mel_noalloc": (C.c_int32, [_vp, _vp, C.c_int64, _vp, C.c_int32, C.c_int32, _vp]),
    "fwhip_ggml_open": (C.c_int32, [C.c_char_p, C.POINTER(_vp)]),
    "fwhip_ggml_open_bytes": (C.c_int32, [C.c_char_p, C.c_uint64, C.POINTER(_vp)]),
    "fwhip_ggml_close": (None, [_vp]),
    "fwhip_ggml_header": (C.c_int32, [_vp, _i32p]),
    "fwhip_ggml_filters": (C.c_int32, [_vp, _i32p, _i32p, C.POINTER(C.POINTER(C.c_float))]),
    "fwhip_ggml_vocab_count": (C.c_int32, [_vp]),
    "fwhip_ggml_vocab_token": (C.c_int32, [_vp, C.c_int32, C.POINTER(C.POINTER(C.c_uint8)),
                                           C.POINTER(C.c_uint32)]),
    "fwhip_ggml_tensor_count": (C.c_int32, [_vp]),
    "fwhip_ggml_tensor_name": (C.c_char_p, [_vp, C.c_int32]),
    "fwhip_ggml_tensor_info": (C.c_int32, [_vp, C.c_char_p, _i32p, _i32p, _i64p, C.POINTER(C.c_uint64)]),
    "fwhip_ggml_tensor_raw": (C.c_int32, [_vp, C.c_char_p, _vp, C.c_uint64]),
    "fwhip_ggml_tensor_f32": (C.c_int32, [_vp, _vp, C.c_char_p, _vp, C.c_int64]),
    "fwhip_dequant": (C.c_int32, [_vp, C.c_int32, _vp, C.c_uint64, C.c_int64, _vp]),
    "fwhip_encoder_load_ggml": (C.c_int32, [_vp, _vp, C.c_int32, C.POINTER(_vp)]),
    "fwhip_decoder_load_ggml": (C.c_int32, [_vp, _vp, C.c_int32, C.POINTER(_vp)]),
}

_lib = None


class FwhipError(RuntimeError):
    def __init__(self, code, msg):
        super().__init__(f"fwhip error {code}: {msg}")
        self.code = code


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def check(code):
    if code != abi.OK:
        msg = lib().fwhip_last_error()
        raise FwhipError(code, msg.decode() if msg else "")


class DeviceArray:
    """A device allocation with a numpy dtype/shape (freed with the context)."""

    def __init__(self, ctx: "Context", shape, dtype):
        self.ctx, self.shape, self.dtype = ctx, tuple(shape), np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        p = _vp()
        check(lib().fwhip_malloc(ctx.h, self.nbytes, C.byref(p)))
        self.ptr = p

    def upload(self, a: np.ndarray):
        a = np.ascontiguousarray(a, dtype=self.dtype)
        assert a.nbytes == self.nbytes, (a.shape, self.shape)
        check(lib().fwhip_upload(self.ctx.h, self.ptr, a.ctypes.data_as(_vp), self.nbytes))
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, self.dtype)
        check(lib().fwhip_download(self.ctx.h, out.ctypes.data_as(_vp), self.ptr, self.nbytes))
        return out

    def free(self):
        if self.ptr:
            lib().fwhip_free(self.ctx.h, self.ptr)
            self.ptr = None


def mel_frames(n_samples: int) -> int:
    """n_frames_for (src/native_engine/mel.rs:1127)."""
    return int(lib().fwhip_mel_frames(n_samples))


class Context:
    def __init__(self, device: int = 0):
        h = _vp()
        check(lib().fwhip_init(device, C.byref(h)))
        self.h = h

    def array(self, a: np.ndarray) -> DeviceArray:
        return DeviceArray(self, a.shape, a.dtype).upload(a)

    def empty(self, shape, dtype) -> DeviceArray:
        return DeviceArray(self, shape, dtype)

    def synchronize(self):
        check(lib().fwhip_synchronize(self.h))

    def timing(self, enable: bool):
        check(lib().fwhip_kernel_timing(self.h, 1 if enable else 0))

    def kernel_stats(self, kclass: int):
        n = C.c_int64()
        ms = C.c_double()
        units = C.c_double()
        check(lib().fwhip_kernel_stats(self.h, kclass, C.byref(n), C.byref(ms), C.byref(units)))
        return n.value, ms.value, units.value

    def cancel(self):
        check(lib().fwhip_request_cancel(self.h))

    def log_mel(self, samples_dev: DeviceArray, n_samples: int, filters_dev: DeviceArray, n_mel: int,
                out_dev: DeviceArray, n_fft_bins: int = 201):
        """log_mel (src/native_engine/mel.rs:1476): [n_mel, mel_frames(n)] into out_dev."""
        check(lib().fwhip_log_mel(self.h, samples_dev.ptr if n_samples else None, n_samples,
                                  filters_dev.ptr, n_mel, n_fft_bins, out_dev.ptr))

    def argmax_logits(self, logits_dev: DeviceArray, filt=None, initial=False):
        """process_logits + argmax (decode.rs:702-867, 1708-1790) of each row of
        logits_dev [n_rows, n_vocab]."""
        n_rows, n_vocab = logits_dev.shape
        out = np.zeros(n_rows, np.int32)
        check(lib().fwhip_argmax_logits(self.h, logits_dev.ptr, n_rows, n_vocab,
                                        C.byref(filt) if filt is not None else None, 1 if initial else 0,
                                        out.ctypes.data_as(_i32p)))
        return out

    def layer_norm(self, x_dev: DeviceArray, w_dev: DeviceArray, b_dev: DeviceArray, y_dev: DeviceArray,
                   exact: bool):
        """layer_norm (nn.rs:4351-4545) of every row of x_dev [rows, d] into y_dev
        with the decoder's kernel; exact: the reference's sequential sums."""
        rows, d = x_dev.shape
        check(lib().fwhip_layer_norm(self.h, x_dev.ptr, w_dev.ptr, b_dev.ptr, rows, d, y_dev.ptr,
                                     1 if exact else 0))

    def tome_merge(self, x_dev: DeviceArray, r: int):
        """tome_merge (encoder.rs:1403-1506) of every window of x_dev [n_windows,
        T, d]: returns (merged [n_windows, T - r', d], umap [n_windows, T])."""
        nw, T, d = x_dev.shape
        merged = self.empty((nw, T, d), np.float32)
        umap = self.empty((nw, T), np.int32)
        rows = C.c_int32(0)
        check(lib().fwhip_tome_merge(self.h, x_dev.ptr, nw, T, d, r, merged.ptr, umap.ptr, C.byref(rows)))
        m = merged.download().reshape(nw, T, d)
        # the device rows are packed [n_windows, T - r', d]
        flat = m.reshape(-1)[: nw * rows.value * d].reshape(nw, rows.value, d)
        out = (flat.copy(), umap.download().reshape(nw, T))
        merged.free()
        umap.free()
        return out

    def log_mel_noalloc(self, samples_dev: DeviceArray, n_samples: int, filters_dev: DeviceArray, n_mel: int,
                        out_dev: DeviceArray, n_fft_bins: int = 201):
        """fwhip_log_mel with the library's static device scratch: no allocation."""
        check(lib().fwhip_log_mel_noalloc(self.h, samples_dev.ptr if n_samples else None, n_samples,
                                          filters_dev.ptr, n_mel, n_fft_bins, out_dev.ptr))

    def close(self):
        if self.h:
            lib().fwhip_destroy(self.h)
            self.h = None


class GgmlFile:
    """A ggml model file (GgmlModel, ggml.rs:582-600): the directory is scanned
    on open, payloads are read on demand.  `source` is a path, or bytes for
    GgmlModel::from_bytes."""

    def __init__(self, source):
        h = _vp()
        if isinstance(source, (bytes, bytearray, memoryview)):
            data = bytes(source)
            check(lib().fwhip_ggml_open_bytes(data, len(data), C.byref(h)))
        else:
            check(lib().fwhip_ggml_open(os.fsencode(source), C.byref(h)))
        self.h = h

    @property
    def hparams(self) -> list:
        hp = (C.c_int32 * 11)()
        check(lib().fwhip_ggml_header(self.h, hp))
        return list(hp)

    @property
    def cfg(self):
        """The model shape as the attribute names of WhisperHParams."""
        from types import SimpleNamespace
        keys = ("n_vocab", "n_audio_ctx", "n_audio_state", "n_audio_head", "n_audio_layer", "n_text_ctx",
                "n_text_state", "n_text_head", "n_text_layer", "n_mels", "ftype")
        return SimpleNamespace(name="ggml", **dict(zip(keys, self.hparams)))

    def filters(self) -> np.ndarray:
        nm, nf, p = C.c_int32(), C.c_int32(), C.POINTER(C.c_float)()
        check(lib().fwhip_ggml_filters(self.h, C.byref(nm), C.byref(nf), C.byref(p)))
        n = nm.value * nf.value
        out = np.empty((nm.value, nf.value), np.float32)
        if n:
            C.memmove(out.ctypes.data, p, 4 * n)
        return out

    def vocab(self) -> list:
        out = []
        for i in range(lib().fwhip_ggml_vocab_count(self.h)):
            p, n = C.POINTER(C.c_uint8)(), C.c_uint32()
            check(lib().fwhip_ggml_vocab_token(self.h, i, C.byref(p), C.byref(n)))
            out.append(C.string_at(p, n.value) if n.value else b"")
        return out

    def names(self) -> list:
        return [lib().fwhip_ggml_tensor_name(self.h, i).decode() for i in range(lib().fwhip_ggml_tensor_count(self.h))]

    def info(self, name: str):
        """(logical shape, element type, payload bytes)"""
        t, nd, n = C.c_int32(), C.c_int32(), C.c_uint64()
        shape = (C.c_int64 * 4)()
        check(lib().fwhip_ggml_tensor_info(self.h, name.encode(), C.byref(t), C.byref(nd), shape, C.byref(n)))
        return [int(shape[i]) for i in range(nd.value)], t.value, n.value

    def raw(self, name: str) -> bytes:
        _, _, n = self.info(name)
        buf = C.create_string_buffer(max(n, 1))
        check(lib().fwhip_ggml_tensor_raw(self.h, name.encode(), buf, n))
        return buf.raw[:n]

    def tensor_f32(self, ctx: "Context", name: str) -> "DeviceArray":
        shape, _, _ = self.info(name)
        out = ctx.empty(tuple(shape), np.float32)
        check(lib().fwhip_ggml_tensor_f32(ctx.h, self.h, name.encode(), out.ptr, int(np.prod(shape))))
        return out

    def close(self):
        if self.h:
            lib().fwhip_ggml_close(self.h)
            self.h = None


def dequant(ctx: "Context", dtype: int, raw_dev: "DeviceArray", raw_bytes: int, n: int, out_dev: "DeviceArray"):
    """fwhip_dequant: decode a payload already on the device."""
    check(lib().fwhip_dequant(ctx.h, dtype, raw_dev.ptr, raw_bytes, n, out_dev.ptr))


class Encoder:
    """EncoderWeights + forward (encoder.rs:764, 1224) on the GPU."""

    def __init__(self, ctx: Context, model, precision: int):
        self.ctx, self.cfg = ctx, model.cfg
        self.precision = precision
        h = _vp()
        if isinstance(model, GgmlFile):
            self.cfg = model.cfg
            check(lib().fwhip_encoder_load_ggml(ctx.h, model.h, precision, C.byref(h)))
        else:
            self._desc = model.encoder_weights()
            check(lib().fwhip_encoder_load(ctx.h, C.byref(self._desc), precision, C.byref(h)))
        self.h = h

    def forward_time_major(self, x_dev: DeviceArray, n_windows: int, n_frames: int, out_dev: DeviceArray):
        rec = abi.ExecRecord()
        check(lib().fwhip_encoder_forward_time_major(self.h, x_dev.ptr, n_windows, n_frames, out_dev.ptr,
                                                     C.byref(rec)))
        return rec

    def forward_mel(self, mel_dev: DeviceArray, mel_frames: int, offsets, n_frames: int, out_dev: DeviceArray):
        offs = np.ascontiguousarray(offsets, dtype=np.int64)
        rec = abi.ExecRecord()
        check(lib().fwhip_encoder_forward(self.h, mel_dev.ptr, mel_frames, offs.ctypes.data_as(_i64p),
                                          offs.size, n_frames, out_dev.ptr, C.byref(rec)))
        return rec

    def set_exact(self, exact: bool):
        check(lib().fwhip_encoder_set_exact(self.h, 1 if exact else 0))

    def set_tome(self, r: int, after: int = 3):
        """FW_TOME_R / FW_TOME_LAYER; r < 0 takes the reference's default rule."""
        check(lib().fwhip_encoder_set_tome(self.h, r, after))

    def set_tome_schedule(self, every: int = 0, floor: int = 128):
        """FW_TOME_EVERY / FW_TOME_FLOOR: every > 0 merges again after every
        `every` blocks; no merge leaves fewer than `floor` rows."""
        check(lib().fwhip_encoder_set_tome_schedule(self.h, every, floor))

    def gemm_i8(self, layer: int, which: int, x_dev: DeviceArray, acc_dev: DeviceArray, y_dev: DeviceArray):
        check(lib().fwhip_encoder_gemm_i8(self.h, layer, which, x_dev.ptr, x_dev.shape[0], acc_dev.ptr,
                                          y_dev.ptr))

    def gemm_i8_fused(self, layer: int, which: int, x_dev: DeviceArray, n_windows: int, n_tokens: int,
                      out16_dev: DeviceArray, side_dev: DeviceArray | None = None):
        check(lib().fwhip_encoder_gemm_i8_fused(self.h, layer, which, x_dev.ptr, n_windows, n_tokens, out16_dev.ptr,
                                                side_dev.ptr if side_dev is not None else None))

    def close(self):
        if self.h:
            lib().fwhip_encoder_free(self.h)
            self.h = None


class Decoder:
    """DecoderWeights (decoder.rs:752-932) resident on the GPU."""

    def __init__(self, ctx: Context, model, arm: int):
        self.arm = arm
        h = _vp()
        if isinstance(model, GgmlFile):
            self.cfg = model.cfg
            check(lib().fwhip_decoder_load_ggml(ctx.h, model.h, arm, C.byref(h)))
        else:
            self.ctx, self.cfg = ctx, model.cfg
            self._desc = model.decoder_weights()
            check(lib().fwhip_decoder_load(ctx.h, C.byref(self._desc), arm, C.byref(h)))
        self.ctx = ctx
        self.h = h

    def set_exact(self, exact: bool):
        """Strict sequential-k cross K/V precompute (bit-exact logits) or the fast
        f16-pair MFMA one (the default)."""
        check(lib().fwhip_decoder_set_exact(self.h, 1 if exact else 0))

    def set_kv_f16(self, on: bool):
        """FW_KV_F16: the self-attention cache of states made afterwards, f16
        (True, the initial setting) or f32 (False, the reference's default)."""
        check(lib().fwhip_decoder_set_kv_f16(self.h, 1 if on else 0))
        self.kv_f16 = bool(on)

    def set_cross_v_block(self, on: bool):
        """FW_CROSS_V_BLOCK: block-int8 cross V with f32 softmax weights in the
        value pass, for int8-arm states made afterwards."""
        check(lib().fwhip_decoder_set_cross_v_block(self.h, 1 if on else 0))

    def state(self, n_streams: int, enc_frames: int) -> "DecoderState":
        return DecoderState(self, n_streams, enc_frames)

    def close(self):
        if self.h:
            lib().fwhip_decoder_free(self.h)
            self.h = None


class DecoderState:
    """A cohort of DecoderStates (decoder.rs:980-1285) sharing one weight read."""

    def __init__(self, dec: Decoder, n_streams: int, enc_frames: int):
        self.dec, self.S, self.T = dec, n_streams, enc_frames
        self.kv_f16 = getattr(dec, "kv_f16", True)
        h = _vp()
        check(lib().fwhip_dstate_new(dec.h, n_streams, enc_frames, C.byref(h)))
        self.h = h

    def set_cross(self, enc_dev: DeviceArray):
        check(lib().fwhip_dstate_set_cross(self.h, enc_dev.ptr))

    def reset(self):
        check(lib().fwhip_dstate_reset(self.h))

    @property
    def len(self):
        return lib().fwhip_dstate_len(self.h, 0)

    def step(self, tokens, logits_dev: DeviceArray | None = None, filt=None, initial=False):
        """forward_step for every stream; tokens [S, tq].  Returns argmax [S]."""
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).reshape(self.S, -1))
        am = np.zeros(self.S, np.int32)
        check(lib().fwhip_decoder_step(self.h, t.ctypes.data_as(_i32p), t.shape[1],
                                       logits_dev.ptr if logits_dev is not None else None,
                                       am.ctypes.data_as(_i32p), C.byref(filt) if filt is not None else None,
                                       1 if initial else 0))
        return am

    def read(self, what: int, stream: int = 0) -> np.ndarray:
        c = self.dec.cfg
        if what in (abi.DS_CROSS_K_F16, abi.DS_CROSS_VT_F16):
            n = c.n_text_layer * self.T * c.n_text_state
        else:
            n = c.n_text_layer * c.n_text_ctx * c.n_text_state
        out = np.empty(n, np.uint16 if what in (abi.DS_CROSS_K_F16, abi.DS_CROSS_VT_F16) or self.kv_f16 else np.float32)
        check(lib().fwhip_dstate_read(self.h, what, stream, out.ctypes.data_as(_vp), out.nbytes))
        return out

    def window(self, prompt, filt, cfg, streams):
        """fwhip_decode_window: the window loop of every stream.  `streams`:
        (seek_cs, seek_end_cs, has_prior_segments) per stream; returns one dict
        per stream (tokens, plogs, result_len, has_ts, seek_delta_cs,
        no_speech_lp, n_exact)."""
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        ws = (abi.WindowStream * self.S)()
        for s, (sk, se, hp) in enumerate(streams):
            ws[s].seek_cs, ws[s].seek_end_cs, ws[s].has_prior_segments = sk, se, 1 if hp else 0
        n = cfg.n_max
        toks = np.zeros((self.S, n), np.int32)
        plogs = np.zeros((self.S, n), np.float32)
        check(lib().fwhip_decode_window(self.h, p.ctypes.data_as(_i32p), p.size, C.byref(filt), C.byref(cfg), ws,
                                        toks.ctypes.data_as(_i32p), plogs.ctypes.data_as(C.POINTER(C.c_float))))
        out = []
        for s in range(self.S):
            k = ws[s].n_tokens
            out.append({"tokens": toks[s, :k].tolist(), "plogs": plogs[s, :k].copy(), "result_len": ws[s].result_len,
                        "has_ts": bool(ws[s].has_ts), "seek_delta_cs": ws[s].seek_delta_cs,
                        "no_speech_lp": np.float32(ws[s].no_speech_logprob), "n_exact": ws[s].n_exact})
        return out

    def greedy(self, prompt, n_max: int, filt):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        toks = np.zeros((self.S, n_max), np.int32)
        lens = np.zeros(self.S, np.int32)
        check(lib().fwhip_decode_greedy(self.h, p.ctypes.data_as(_i32p), p.size, n_max, C.byref(filt),
                                        toks.ctypes.data_as(_i32p), lens.ctypes.data_as(_i32p)))
        return [toks[s, : lens[s]].copy() for s in range(self.S)]

    def close(self):
        if self.h:
            lib().fwhip_dstate_free(self.h)
            self.h = None


def transcribe(ctx: Context, enc: Encoder, dec: Decoder, samples_dev: DeviceArray, n_samples: int,
               filters_dev: DeviceArray, n_mel: int, filt, vocab, sot_sequence, timestamps: bool = False,
               max_context: int | None = None, max_tokens: int | None = None, no_context: bool = False,
               retry_failed_window: bool = True, tiny_en_ts_context: bool = False, carry_initial_prompt: bool = False,
               initial_prompt=(), no_speech_threshold: float = 0.6, logprob_threshold: float = -1.0,
               exact_forcing: bool = False):
    """fwhip_transcribe (transcribe_samples, decode.rs:2880-3960, greedy path):
    returns {"segments": [(start_cs, end_cs, text, confidence | None)],
    "windows": [dict]}.  `vocab` is the list of token byte strings."""
    blob = b"".join(vocab)
    offs = np.zeros(len(vocab) + 1, np.uint64)
    offs[1:] = np.cumsum([len(v) for v in vocab], dtype=np.uint64)
    buf = np.frombuffer(blob, np.uint8).copy() if blob else np.zeros(1, np.uint8)
    voc = abi.Vocab(len(vocab), buf.ctypes.data_as(C.POINTER(C.c_uint8)), offs.ctypes.data_as(C.POINTER(C.c_uint64)))
    sot = np.ascontiguousarray(sot_sequence, dtype=np.int32)
    ip = np.ascontiguousarray(list(initial_prompt) or [0], dtype=np.int32)
    p = abi.TranscribeParams(1 if timestamps else 0, max_context if max_context is not None else -1,
                             0 if max_context is None else 1, max_tokens or 0, 1 if no_context else 0,
                             1 if retry_failed_window else 0, 1 if tiny_en_ts_context else 0,
                             1 if carry_initial_prompt else 0, ip.ctypes.data_as(_i32p), len(initial_prompt),
                             sot.ctypes.data_as(_i32p), sot.size, no_speech_threshold, logprob_threshold,
                             1 if exact_forcing else 0)
    h = _vp()
    check(lib().fwhip_transcribe(ctx.h, enc.h, dec.h, samples_dev.ptr, n_samples, filters_dev.ptr, n_mel,
                                 C.byref(filt), C.byref(voc), C.byref(p), C.byref(h)))
    try:
        segs = []
        for i in range(lib().fwhip_transcript_n_segments(h)):
            si = abi.SegmentInfo()
            check(lib().fwhip_transcript_segment(h, i, C.byref(si)))
            conf = None if si.confidence != si.confidence else si.confidence
            segs.append((si.start_cs, si.end_cs, si.text.decode("utf-8"), conf))
        wins = []
        for i in range(lib().fwhip_transcript_n_windows(h)):
            wi = abi.WindowInfo()
            check(lib().fwhip_transcript_window(h, i, C.byref(wi)))
            n = wi.n_tokens
            wins.append({"seek_cs": wi.seek_cs, "avg_logprob": wi.avg_logprob, "no_speech_prob": wi.no_speech_prob,
                         "result_len": wi.result_len, "has_ts": bool(wi.has_ts), "seek_delta_cs": wi.seek_delta_cs,
                         "no_speech": bool(wi.no_speech), "dropped": bool(wi.dropped), "retried": bool(wi.retried),
                         "tokens": [wi.tokens[k] for k in range(n)],
                         "plogs": np.array([wi.plogs[k] for k in range(n)], np.float32)})
    finally:
        lib().fwhip_transcript_free(h)
    return {"segments": segs, "windows": wins}
