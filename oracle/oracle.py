"""ctypes binding of the CPU restatement (refcpu.c).

TEST INFRASTRUCTURE: imported only by tests/, __graft_entry__.smoke() and the
bench's cpu_baseline leg, as the checker or the CPU baseline — never by the
product package.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

from franken_whisper_amd import abi

HERE = os.path.dirname(os.path.abspath(__file__))
# FWHIP_REFCPU_SO selects another build of the same sources (the sanitizer
# build of `make -C oracle asan`)
SO = os.environ.get("FWHIP_REFCPU_SO") or os.path.join(HERE, "build", "librefcpu.so")

_lib = None


class RefFilterCfg(C.Structure):
    """FilterConfig (decode.rs:671-693); -1 is None for the optional fields."""
    _fields_ = [("suppress_blank", C.c_int), ("no_timestamps", C.c_int), ("max_initial_tid", C.c_int),
                ("max_tokens", C.c_int)]


i8p = C.POINTER(C.c_int8)
u8p = C.POINTER(C.c_uint8)
i32p = C.POINTER(C.c_int32)
f32p = abi.f32p
u16p = abi.u16p


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return SO


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(SO):
        build()
    L = C.CDLL(SO)
    sig = {
        "ref_f16_to_f32": (C.c_float, [C.c_uint16]),
        "ref_f32_to_f16": (C.c_uint16, [C.c_float]),
        "ref_f16_to_f32_n": (None, [u16p, f32p, C.c_int64]),
        "ref_f32_to_f16_n": (None, [f32p, u16p, C.c_int64]),
        "ref_gelu_scalar": (C.c_float, [C.c_float]),
        "ref_gelu_table": (f32p, []),
        "ref_quantize_act_i8": (None, [f32p, C.c_int, C.c_float, i8p]),
        "ref_quantize_row_i7_u8": (None, [f32p, C.c_int, C.c_float, u8p]),
        "ref_quant_row_i8_exact": (None, [f32p, C.c_int, C.c_float, i8p]),
        "ref_quantize_f16_row_to_i8": (C.c_float, [u16p, C.c_int, i8p]),
        "ref_quantize_f16_to_i8": (None, [u16p, C.c_int64, C.c_int, i8p, f32p]),
        "ref_quantize_f16_to_i8_blocked": (None, [u16p, C.c_int64, C.c_int, C.c_int, i8p, f32p]),
        "ref_quantize_rows_to_i7": (None, [u16p, C.c_int64, C.c_int, C.c_int, i8p, f32p, i32p]),
        "ref_quantize_enc_i8_rows": (None, [u16p, C.c_int64, C.c_int, i8p, f32p]),
        "ref_act_scale": (C.c_float, [f32p, C.c_int]),
        "ref_dot_i8": (C.c_int32, [i8p, i8p, C.c_int]),
        "ref_dot_f16c": (C.c_float, [u16p, f32p, C.c_int]),
        "ref_dot_i8w_f32": (C.c_float, [i8p, f32p, C.c_int]),
        "ref_gemv_i8": (None, [i8p, f32p, C.c_int64, C.c_int, f32p, f32p, f32p]),
        "ref_gemv_f16": (None, [u16p, C.c_int64, C.c_int, f32p, f32p, f32p]),
        "ref_gemv_i8w_f32a_blocked": (None, [i8p, f32p, C.c_int64, C.c_int, C.c_int, f32p, f32p, f32p]),
        "ref_layer_norm": (None, [f32p, f32p, C.c_int64, C.c_int, f32p, f32p, C.c_float]),
        "ref_gelu_inplace": (None, [f32p, C.c_int64]),
        "ref_softmax_rows": (None, [f32p, C.c_int64, C.c_int]),
        "ref_matmul_strict": (None, [f32p, f32p, f32p, C.c_int64, C.c_int, C.c_int]),
        "ref_argmax_first": (C.c_int, [f32p, C.c_int]),
        "ref_attention": (None, [f32p, C.c_int, f32p, f32p, C.c_int, C.c_int, C.c_int, C.c_int, C.c_int,
                                 f32p]),
        "ref_attention_decode_f16": (None, [f32p, u16p, u16p, C.c_int, C.c_int, C.c_int, f32p]),
        "ref_attention_decode_f32": (None, [f32p, f32p, f32p, C.c_int, C.c_int, C.c_int, f32p]),
        "ref_decoder_set_kv_f16": (None, [C.c_void_p, C.c_int]),
        "ref_decoder_set_cross_v_block": (None, [C.c_void_p, C.c_int]),
        "ref_encoder_new": (C.c_void_p, [C.POINTER(abi.EncoderWeights), C.c_int]),
        "ref_encoder_free": (None, [C.c_void_p]),
        "ref_encoder_forward": (C.c_int, [C.c_void_p, f32p, C.c_int, f32p, C.c_int]),
        "ref_encoder_forward_tome": (C.c_int, [C.c_void_p, f32p, C.c_int, f32p, C.c_int, C.c_int, C.c_int]),
        "ref_encoder_forward_tome2": (C.c_int, [C.c_void_p, f32p, C.c_int, f32p, C.c_int, C.c_int, C.c_int,
                                                C.c_int, C.c_int]),
        "ref_tome_merge": (C.c_int, [f32p, C.c_int, C.c_int, C.c_int, f32p, i32p]),
        "ref_tome_unmerge": (None, [f32p, i32p, C.c_int, C.c_int, f32p]),
        "ref_mel_window": (None, [f32p, C.c_int, C.c_int64, C.c_int64, C.c_int, f32p]),
        "ref_enc_i7_gemm": (None, [C.c_void_p, C.c_int, C.c_int, f32p, C.c_int64, i32p, f32p]),
        "ref_decoder_new": (C.c_void_p, [C.POINTER(abi.DecoderWeights), C.c_int]),
        "ref_decoder_free": (None, [C.c_void_p]),
        "ref_dstate_new": (C.c_void_p, [C.c_void_p, f32p, C.c_int]),
        "ref_dstate_free": (None, [C.c_void_p]),
        "ref_dstate_reset": (None, [C.c_void_p]),
        "ref_dstate_len": (C.c_int, [C.c_void_p]),
        "ref_dstate_cross_k_f16": (u16p, [C.c_void_p]),
        "ref_dstate_cross_vt_f16": (u16p, [C.c_void_p]),
        "ref_decoder_step": (C.c_int, [C.c_void_p, C.c_void_p, i32p, C.c_int, f32p]),
        "ref_process_argmax": (C.c_int, [C.POINTER(abi.Filter), f32p, C.c_int, C.c_int]),
        "ref_decode_greedy": (C.c_int, [C.c_void_p, C.c_void_p, i32p, C.c_int, C.c_int,
                                        C.POINTER(abi.Filter), i32p, i32p]),
        "ref_compute_logprobs": (None, [f32p, C.c_int, f32p]),
        "ref_process_logits": (C.c_int, [C.POINTER(abi.Filter), C.POINTER(RefFilterCfg), f32p, f32p, C.c_int, i32p,
                                         C.c_int, C.c_int, C.c_int64, C.c_int]),
        "ref_mel_frames": (C.c_int64, [C.c_int64]),
        "ref_log_mel": (None, [f32p, C.c_int64, f32p, C.c_int, f32p]),
        "ref_mel_fft400": (None, [f32p, f32p]),
        "ref_log10_floor_approx": (C.c_float, [C.c_double]),
        "ref_mel_hann": (None, [f32p]),
        "ref_num_threads": (C.c_int, []),
        "ref_set_num_threads": (None, [C.c_int]),
        "ref_set_fast": (None, [C.c_int]),
        "ref_get_fast": (C.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def _p(a, t):
    return abi.ptr(a, t)


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


# ---- primitive wrappers -------------------------------------------------------
def f16_to_f32(h):
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().ref_f16_to_f32_n(_p(h, C.c_uint16), _p(out, C.c_float), h.size)
    return out


def f32_to_f16(f):
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().ref_f32_to_f16_n(_p(f, C.c_float), _p(out, C.c_uint16), f.size)
    return out


def gelu_table():
    t = lib().ref_gelu_table()
    return np.ctypeslib.as_array(t, shape=(1 << 16,)).copy()


def gelu(x):
    x = _c(x, np.float32).copy()
    lib().ref_gelu_inplace(_p(x, C.c_float), x.size)
    return x


def quantize_act_i8(x, xinv):
    x = _c(x, np.float32)
    out = np.empty(x.size, np.int8)
    lib().ref_quantize_act_i8(_p(x, C.c_float), x.size, C.c_float(xinv), _p(out, C.c_int8))
    return out


def quantize_row_i7_u8(x, inv):
    x = _c(x, np.float32)
    out = np.empty(x.size, np.uint8)
    lib().ref_quantize_row_i7_u8(_p(x, C.c_float), x.size, C.c_float(inv), _p(out, C.c_uint8))
    return out


def quant_row_i8_exact(x, inv):
    x = _c(x, np.float32)
    out = np.empty(x.size, np.int8)
    lib().ref_quant_row_i8_exact(_p(x, C.c_float), x.size, C.c_float(inv), _p(out, C.c_int8))
    return out


def act_scale(x):
    x = _c(x, np.float32)
    return np.float32(lib().ref_act_scale(_p(x, C.c_float), x.size))


def quantize_f16_to_i8(w):
    w = _c(w, np.uint16)
    out, inp = w.shape
    q = np.empty((out, inp), np.int8)
    s = np.empty(out, np.float32)
    lib().ref_quantize_f16_to_i8(_p(w, C.c_uint16), out, inp, _p(q, C.c_int8), _p(s, C.c_float))
    return q, s


def quantize_f16_to_i8_blocked(w, block=32):
    w = _c(w, np.uint16)
    out, inp = w.shape
    nb = (inp + block - 1) // block
    q = np.empty((out, inp), np.int8)
    s = np.empty((out, nb), np.float32)
    lib().ref_quantize_f16_to_i8_blocked(_p(w, C.c_uint16), out, inp, block, _p(q, C.c_int8),
                                         _p(s, C.c_float))
    return q, s


def quantize_rows_to_i7(w, ef=True):
    w = _c(w, np.uint16)
    out, inp = w.shape
    q = np.empty((out, inp), np.int8)
    s = np.empty(out, np.float32)
    cs = np.empty(out, np.int32)
    lib().ref_quantize_rows_to_i7(_p(w, C.c_uint16), out, inp, 1 if ef else 0, _p(q, C.c_int8),
                                  _p(s, C.c_float), _p(cs, C.c_int32))
    return q, s, cs


def quantize_enc_i8_rows(w):
    w = _c(w, np.uint16)
    out, inp = w.shape
    q = np.empty((out, inp), np.int8)
    s = np.empty(out, np.float32)
    lib().ref_quantize_enc_i8_rows(_p(w, C.c_uint16), out, inp, _p(q, C.c_int8), _p(s, C.c_float))
    return q, s


def dot_f16c(w, x):
    w, x = _c(w, np.uint16), _c(x, np.float32)
    return np.float32(lib().ref_dot_f16c(_p(w, C.c_uint16), _p(x, C.c_float), w.size))


def dot_i8w_f32(w, x):
    w, x = _c(w, np.int8), _c(x, np.float32)
    return np.float32(lib().ref_dot_i8w_f32(_p(w, C.c_int8), _p(x, C.c_float), w.size))


def gemv_i8(q, s, x, bias=None):
    q, s, x = _c(q, np.int8), _c(s, np.float32), _c(x, np.float32)
    out, inp = q.shape
    y = np.empty(out, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().ref_gemv_i8(_p(q, C.c_int8), _p(s, C.c_float), out, inp, _p(x, C.c_float),
                      _p(b, C.c_float), _p(y, C.c_float))
    return y


def gemv_f16(w, x, bias=None):
    w, x = _c(w, np.uint16), _c(x, np.float32)
    out, inp = w.shape
    y = np.empty(out, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().ref_gemv_f16(_p(w, C.c_uint16), out, inp, _p(x, C.c_float), _p(b, C.c_float),
                       _p(y, C.c_float))
    return y


def gemv_i8w_f32a_blocked(q, s, x, bias=None, block=32):
    q, s, x = _c(q, np.int8), _c(s, np.float32), _c(x, np.float32)
    out, inp = q.shape
    y = np.empty(out, np.float32)
    b = None if bias is None else _c(bias, np.float32)
    lib().ref_gemv_i8w_f32a_blocked(_p(q, C.c_int8), _p(s, C.c_float), out, inp, block,
                                    _p(x, C.c_float), _p(b, C.c_float), _p(y, C.c_float))
    return y


def layer_norm(x, w, b, eps=1e-5):
    x = _c(x, np.float32)
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    w, b = _c(w, np.float32), _c(b, np.float32)
    lib().ref_layer_norm(_p(x, C.c_float), _p(y, C.c_float), rows, cols, _p(w, C.c_float),
                         _p(b, C.c_float), C.c_float(eps))
    return y


def softmax_rows(x):
    x = _c(x, np.float32).copy()
    rows, cols = x.reshape(-1, x.shape[-1]).shape
    lib().ref_softmax_rows(_p(x, C.c_float), rows, cols)
    return x


def matmul_strict(a, b):
    a, b = _c(a, np.float32), _c(b, np.float32)
    m, k = a.shape
    k2, n = b.shape
    assert k == k2
    c = np.empty((m, n), np.float32)
    lib().ref_matmul_strict(_p(a, C.c_float), _p(b, C.c_float), _p(c, C.c_float), m, k, n)
    return c


def mel_frames(n_samples):
    """n_frames_for, mel.rs:1127."""
    return int(lib().ref_mel_frames(int(n_samples)))


def log_mel(samples, filters):
    """log_mel, mel.rs:1476-1660: mel-major [n_mel, mel_frames(n)], clamped and
    normalized; filters [n_mel, 201] f32."""
    x = _c(samples, np.float32)
    f = _c(filters, np.float32)
    n_mel = f.shape[0]
    out = np.empty((n_mel, mel_frames(x.size)), dtype=np.float32)
    lib().ref_log_mel(_p(x, C.c_float), x.size, _p(f, C.c_float), n_mel, _p(out, C.c_float))
    return out


def mel_window(mel, frame_offset, n_frames):
    """time_major_mel_window_from_full_mel (encoder.rs:684-737): [n_frames,
    n_mel] from the mel-major full mel, -1.5 past its end."""
    m = _c(mel, np.float32)
    out = np.empty((n_frames, m.shape[0]), np.float32)
    lib().ref_mel_window(_p(m, C.c_float), m.shape[0], m.shape[1], frame_offset, n_frames, _p(out, C.c_float))
    return out


def mel_fft400(frame):
    """fft_twoforone, mel.rs:648-695, of one 400-sample frame: 400 complex bins."""
    x = _c(frame, np.float32)
    assert x.size == 400
    out = np.empty(800, dtype=np.float32)
    lib().ref_mel_fft400(_p(x, C.c_float), _p(out, C.c_float))
    return out[0::2] + 1j * out[1::2].astype(np.float64)


def log10_floor_approx(x):
    """log10_floor_approx, mel.rs:1239-1249."""
    return np.float32(lib().ref_log10_floor_approx(float(x)))


def mel_hann():
    out = np.empty(400, dtype=np.float32)
    lib().ref_mel_hann(_p(out, C.c_float))
    return out


def attention(q, k, v, n_head, causal=False, cache_len=0):
    """attention_raw's per-head path (nn.rs:6035-6131) on [tq, d] x [tk, d]."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    tq, d = q.shape
    tk = k.shape[0]
    out = np.empty((tq, d), np.float32)
    lib().ref_attention(_p(q, C.c_float), tq, _p(k, C.c_float), _p(v, C.c_float), tk, d, n_head,
                        1 if causal else 0, cache_len, _p(out, C.c_float))
    return out


def attention_decode_f16(q, kc16, vc16, n_head):
    """attention_decode_step_f16 (nn.rs:6466-6540): one row over an f16 cache."""
    q = _c(q, np.float32).ravel()
    kc16, vc16 = _c(kc16, np.uint16), _c(vc16, np.uint16)
    tk, d = kc16.shape
    out = np.empty(d, np.float32)
    lib().ref_attention_decode_f16(_p(q, C.c_float), _p(kc16, C.c_uint16), _p(vc16, C.c_uint16), tk, d, n_head,
                                   _p(out, C.c_float))
    return out


def attention_decode_f32(q, kc, vc, n_head):
    """attention_decode_step (nn.rs:6340-6400): one row over an f32 cache."""
    q = _c(q, np.float32).ravel()
    kc, vc = _c(kc, np.float32), _c(vc, np.float32)
    tk, d = kc.shape
    out = np.empty(d, np.float32)
    lib().ref_attention_decode_f32(_p(q, C.c_float), _p(kc, C.c_float), _p(vc, C.c_float), tk, d, n_head,
                                   _p(out, C.c_float))
    return out


def argmax_first(x):
    x = _c(x, np.float32)
    return int(lib().ref_argmax_first(_p(x, C.c_float), x.size))


# ---- model wrappers -----------------------------------------------------------
class Encoder:
    def __init__(self, model, precision):
        self.model = model
        self.desc = model.encoder_weights()
        self.h = lib().ref_encoder_new(C.byref(self.desc), precision)
        self.cfg = model.cfg

    def forward(self, x_time_major, n_layers=-1, tome_r=0, tome_after=3, tome_every=0, tome_floor=128):
        """forward_time_major; tome_r > 0 merges tome_r rows after block
        tome_after (0-based), as FW_TOME_R / FW_TOME_LAYER do, and with
        tome_every > 0 again after every tome_every blocks (FW_TOME_EVERY) while
        the merged length stays >= tome_floor (FW_TOME_FLOOR)."""
        x = _c(x_time_major, np.float32)
        n_frames = x.shape[0]
        out = np.empty((n_frames // 2, self.cfg.n_audio_state), np.float32)
        rc = lib().ref_encoder_forward_tome2(self.h, _p(x, C.c_float), n_frames, _p(out, C.c_float),
                                             n_layers, tome_r, tome_after, tome_every, tome_floor)
        if rc != 0:
            raise ValueError(f"ref_encoder_forward rc={rc}")
        return out

    def gemm(self, layer, which, x):
        x = _c(x, np.float32)
        m = x.shape[0]
        d = self.cfg.n_audio_state
        out = 4 * d if which == 4 else d
        acc = np.empty((m, out), np.int32)
        y = np.empty((m, out), np.float32)
        lib().ref_enc_i7_gemm(self.h, layer, which, _p(x, C.c_float), m, _p(acc, C.c_int32),
                              _p(y, C.c_float))
        return acc, y

    def __del__(self):
        try:
            lib().ref_encoder_free(self.h)
        except Exception:
            pass


def tome_merge(x, r):
    """tome_merge (encoder.rs:1403-1506) of the rows x [seq, d]: returns the
    merged rows [seq - r', d] and the unmerge map [seq]."""
    x = _c(x, np.float32)
    seq, d = x.shape
    merged = np.zeros((seq, d), np.float32)
    umap = np.zeros(seq, np.int32)
    n = lib().ref_tome_merge(_p(x, C.c_float), seq, d, r, _p(merged, C.c_float), _p(umap, C.c_int32))
    return merged[:n].copy(), umap


def tome_unmerge(merged, umap):
    merged = _c(merged, np.float32)
    umap = _c(umap, np.int32)
    out = np.empty((umap.size, merged.shape[1]), np.float32)
    lib().ref_tome_unmerge(_p(merged, C.c_float), _p(umap, C.c_int32), umap.size, merged.shape[1],
                           _p(out, C.c_float))
    return out


class Decoder:
    def __init__(self, model, arm):
        self.model = model
        self.desc = model.decoder_weights()
        self.h = lib().ref_decoder_new(C.byref(self.desc), arm)
        self.cfg = model.cfg

    def set_kv_f16(self, on):
        """FW_KV_F16 for the states made next (True: f16 cache; False: f32)."""
        lib().ref_decoder_set_kv_f16(self.h, 1 if on else 0)

    def set_cross_v_block(self, on):
        """FW_CROSS_V_BLOCK for the states made next (the int8 arm)."""
        lib().ref_decoder_set_cross_v_block(self.h, 1 if on else 0)

    def state(self, enc):
        return DState(self, enc)

    def __del__(self):
        try:
            lib().ref_decoder_free(self.h)
        except Exception:
            pass


class DState:
    def __init__(self, dec, enc):
        self.dec = dec
        enc = _c(enc, np.float32)
        self.T = enc.shape[0]
        self.h = lib().ref_dstate_new(dec.h, _p(enc, C.c_float), self.T)

    def step(self, tokens):
        t = _c(tokens, np.int32)
        logits = np.empty(self.dec.cfg.n_vocab, np.float32)
        rc = lib().ref_decoder_step(self.dec.h, self.h, _p(t, C.c_int32), t.size,
                                    _p(logits, C.c_float))
        if rc != 0:
            raise ValueError(f"ref_decoder_step rc={rc}")
        return logits

    def reset(self):
        lib().ref_dstate_reset(self.h)

    @property
    def len(self):
        return lib().ref_dstate_len(self.h)

    def cross_k_f16(self):
        c = self.dec.cfg
        n = c.n_text_layer * self.T * c.n_text_state
        return np.ctypeslib.as_array(lib().ref_dstate_cross_k_f16(self.h), shape=(n,)).copy()

    def cross_vt_f16(self):
        c = self.dec.cfg
        n = c.n_text_layer * self.T * c.n_text_state
        return np.ctypeslib.as_array(lib().ref_dstate_cross_vt_f16(self.h), shape=(n,)).copy()

    def greedy(self, prompt, n_max, filt):
        p = _c(prompt, np.int32)
        toks = np.zeros(n_max, np.int32)
        n = C.c_int32(0)
        rc = lib().ref_decode_greedy(self.dec.h, self.h, _p(p, C.c_int32), p.size, n_max,
                                     C.byref(filt), _p(toks, C.c_int32), C.byref(n))
        if rc != 0:
            raise ValueError(f"ref_decode_greedy rc={rc}")
        return toks[: n.value]

    def __del__(self):
        try:
            lib().ref_dstate_free(self.h)
        except Exception:
            pass


def process_argmax(filt, logits, initial):
    lg = _c(logits, np.float32)
    return int(lib().ref_process_argmax(C.byref(filt), _p(lg, C.c_float), lg.size,
                                        1 if initial else 0))


def compute_logprobs(logits):
    """compute_logprobs (decode.rs:1666-1701)."""
    lg = _c(logits, np.float32)
    out = np.empty_like(lg)
    lib().ref_compute_logprobs(_p(lg, C.c_float), lg.size, _p(out, C.c_float))
    return out


def process_logits(filt, cfg, logits, prev, has_ts, seek_delta_cs, tokens_in_window):
    """process_logits (decode.rs:702-867): (filtered logits, logprobs, forced)."""
    lg = _c(logits, np.float32).copy()
    lp = np.empty_like(lg)
    pv = _c(prev if len(prev) else [0], np.int32)
    forced = lib().ref_process_logits(C.byref(filt), C.byref(cfg), _p(lg, C.c_float), _p(lp, C.c_float), lg.size,
                                      _p(pv, C.c_int32), len(prev), 1 if has_ts else 0, int(seek_delta_cs),
                                      int(tokens_in_window))
    return lg, lp, bool(forced)
