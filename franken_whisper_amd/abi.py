"""ctypes mirror of include/fwhip.h: status codes, hyper-parameters and the
weight descriptor structs (the ggml tensor layout of the reference's
EncoderWeights / DecoderWeights, src/native_engine/encoder.rs:129-161 and
decoder.rs:514-545)."""
from __future__ import annotations

import ctypes as C

OK = 0
ERR_GENERIC = 1
ERR_INVALID = 2
ERR_UNSUPPORTED = 5
ERR_CANCELLED = 6

ENC_F32 = 0
ENC_INT8 = 1
DEC_INT8 = 0
DEC_F16 = 1

K_ENC_GEMM_I8 = 1
K_ENC_GEMM_F32 = 2
K_ENC_ATTN = 3
K_DEC_GEMV = 4
K_DEC_LOGITS = 5
K_DEC_CROSS = 6
K_DEC_STEP = 7
K_DEQUANT = 8
K_DEC_XATTN = 9

DS_CROSS_K_F16 = 1
DS_CROSS_VT_F16 = 2
DS_KV_K = 3
DS_KV_V = 4

f32p = C.POINTER(C.c_float)
u16p = C.POINTER(C.c_uint16)


class HParams(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "n_vocab", "n_audio_ctx", "n_audio_state", "n_audio_head", "n_audio_layer",
        "n_text_ctx", "n_text_state", "n_text_head", "n_text_layer", "n_mels")]


class EncLayer(C.Structure):
    _fields_ = [
        ("attn_ln_w", f32p), ("attn_ln_b", f32p),
        ("q_w", u16p), ("q_b", f32p), ("k_w", u16p), ("v_w", u16p), ("v_b", f32p),
        ("o_w", u16p), ("o_b", f32p),
        ("mlp_ln_w", f32p), ("mlp_ln_b", f32p),
        ("fc1_w", u16p), ("fc1_b", f32p), ("fc2_w", u16p), ("fc2_b", f32p),
    ]


class EncoderWeights(C.Structure):
    _fields_ = [
        ("hp", HParams),
        ("conv1_w", u16p), ("conv1_b", f32p), ("conv2_w", u16p), ("conv2_b", f32p),
        ("pos_emb", f32p), ("layers", C.POINTER(EncLayer)),
        ("ln_post_w", f32p), ("ln_post_b", f32p),
    ]


class DecLayer(C.Structure):
    _fields_ = [
        ("attn_ln_w", f32p), ("attn_ln_b", f32p),
        ("q_w", u16p), ("q_b", f32p), ("k_w", u16p), ("v_w", u16p), ("v_b", f32p),
        ("o_w", u16p), ("o_b", f32p),
        ("cross_ln_w", f32p), ("cross_ln_b", f32p),
        ("cq_w", u16p), ("cq_b", f32p), ("ck_w", u16p), ("cv_w", u16p), ("cv_b", f32p),
        ("co_w", u16p), ("co_b", f32p),
        ("mlp_ln_w", f32p), ("mlp_ln_b", f32p),
        ("fc1_w", u16p), ("fc1_b", f32p), ("fc2_w", u16p), ("fc2_b", f32p),
    ]


class DecoderWeights(C.Structure):
    _fields_ = [
        ("hp", HParams),
        ("tok_emb", u16p), ("pos_emb", f32p), ("layers", C.POINTER(DecLayer)),
        ("ln_w", f32p), ("ln_b", f32p),
    ]


class Filter(C.Structure):
    _fields_ = [(n, C.c_int32) for n in (
        "eot", "sot", "sot_prev", "solm", "no_speech", "no_timestamps",
        "translate", "transcribe", "timestamp_begin", "space_token", "n_languages")]


class WindowCfg(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("timestamps", "max_initial_tid", "max_tokens", "n_max", "exact")]


class WindowStream(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("seek_cs", "seek_end_cs", "has_prior_segments", "n_tokens", "result_len",
                                         "has_ts", "seek_delta_cs", "n_exact")] + [("no_speech_logprob", C.c_float)]


class Vocab(C.Structure):
    _fields_ = [("n_tokens", C.c_int32), ("bytes", C.POINTER(C.c_uint8)), ("offsets", C.POINTER(C.c_uint64))]


class TranscribeParams(C.Structure):
    _fields_ = [("timestamps", C.c_int32), ("max_context", C.c_int32), ("max_context_set", C.c_int32),
                ("max_tokens", C.c_int32), ("no_context", C.c_int32), ("retry_failed_window", C.c_int32),
                ("tiny_en_ts_context", C.c_int32), ("carry_initial_prompt", C.c_int32),
                ("initial_prompt", C.POINTER(C.c_int32)), ("n_initial_prompt", C.c_int32),
                ("sot_sequence", C.POINTER(C.c_int32)), ("n_sot", C.c_int32),
                ("no_speech_threshold", C.c_double), ("logprob_threshold", C.c_double), ("exact_forcing", C.c_int32)]


class SegmentInfo(C.Structure):
    _fields_ = [("start_cs", C.c_int64), ("end_cs", C.c_int64), ("text", C.c_char_p), ("confidence", C.c_double)]


class WindowInfo(C.Structure):
    _fields_ = [("seek_cs", C.c_int64), ("avg_logprob", C.c_double), ("no_speech_prob", C.c_double)] + [
        (n, C.c_int32) for n in ("result_len", "n_tokens", "has_ts", "seek_delta_cs", "no_speech", "dropped",
                                 "retried")] + [("tokens", C.POINTER(C.c_int32)), ("plogs", C.POINTER(C.c_float))]


# GemmPrecision (encoder.rs:1885-1927) values and GEMM families (fwhip.h)
PREC_F32, PREC_I7, PREC_I8, PREC_F16, PREC_F16_WEIGHTS, PREC_Q8_0_WEIGHTS, PREC_F16_KV, PREC_MIXED, PREC_F16_PAIR = \
    range(9)
FAMILIES = ("conv_stem", "attn_qkv", "attention", "attn_out", "mlp_fc1", "mlp_fc2")


class ExecRecord(C.Structure):
    """EncoderExecution (encoder.rs:1987-2003): route, the precision of each
    GEMM family and what chose it."""
    _fields_ = [("route", C.c_char * 48), ("precision", C.c_int32), ("n_windows", C.c_int32),
                ("device_ms", C.c_double), ("family", C.c_int32 * 6), ("precision_source", C.c_char * 32)]


def ptr(arr, ctype):
    """Pointer to a contiguous numpy array's buffer (caller keeps `arr` alive)."""
    if arr is None:
        return C.cast(None, C.POINTER(ctype))
    assert arr.flags["C_CONTIGUOUS"], "array must be C-contiguous"
    return arr.ctypes.data_as(C.POINTER(ctype))
