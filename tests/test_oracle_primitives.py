"""Pins the oracle's primitives (CPU).  Each check is chosen so a plausible
restatement mistake (wrong rounding mode, dropped term, swapped lane order,
transposed operand) fails it:
  - the reference's own known-answer vectors (nn.rs:7454-7458, 7491-7500,
    8180-8256, 8258-8297);
  - exhaustive comparisons (every f32 -> f16, every f16 -> f32, every float
    of the softmax domain through the device expf restatement vs glibc);
  - exact-integer and constructed-association cases whose answer follows
    from the mathematics."""
import ctypes as C
import os
import subprocess
import struct

import numpy as np
import pytest

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
F16_HARNESS = r"""
#include <immintrin.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include "refcpu.h"
int main(void) {
    long bad = 0;
    #pragma omp parallel for reduction(+:bad) schedule(static)
    for (int64_t u = 0; u <= 0xffffffffLL; u++) {
        uint32_t v = (uint32_t)u; float f; memcpy(&f, &v, 4);
        uint16_t want = _cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT);
        uint16_t got = ref_f32_to_f16(f);
        if (want != got) bad++;
    }
    for (int h = 0; h < 65536; h++) {
        float want = _cvtsh_ss((uint16_t)h), got = ref_f16_to_f32((uint16_t)h);
        if (memcmp(&want, &got, 4) != 0) bad++;
    }
    printf("%ld\n", bad);
    return bad != 0;
}
"""

EXP_HARNESS = r"""
#include <math.h>
#include <stdio.h>
#include "fw_math.h"
int main(void) {
    long bad = 0, n = 0;
    #pragma omp parallel for reduction(+:bad,n) schedule(static)
    for (int64_t u = 0; u <= 0xffffffffLL; u++) {
        uint32_t v = (uint32_t)u; float x; memcpy(&x, &v, 4);
        if (!(x >= -110.0f && x <= 90.0f)) continue;
        n++;
        float a = expf(x), b = fw_expf_host(x);
        if (fw_f2u(a) != fw_f2u(b)) bad++;
    }
    float sp[] = {-INFINITY, 0.0f, -0.0f, -104.0f, 89.0f};
    for (int i = 0; i < 5; i++) if (fw_f2u(expf(sp[i])) != fw_f2u(fw_expf_host(sp[i]))) bad++;
    if (!isnan(fw_expf_host(NAN))) bad++;
    printf("%ld %ld\n", n, bad);
    return bad != 0;
}
"""


FAST_EXP_HARNESS = r"""
#include <math.h>
#include <stdio.h>
#include <stdint.h>
#include <string.h>
#include "refcpu_fast.h"
static uint32_t bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
int main(void) {
    long bad = 0, n = 0;
    #pragma omp parallel for reduction(+:bad,n) schedule(static)
    for (int64_t blk = 0; blk < (1LL << 32); blk += 4096) {
        float x[4096], y[4096];
        int m = 0;
        for (int64_t u = blk; u < blk + 4096; u++) {
            uint32_t v = (uint32_t)u; float f; memcpy(&f, &v, 4);
            if (f >= -110.0f && f <= 90.0f) x[m++] = f;
        }
        rf_expf_n(x, y, m);
        for (int i = 0; i < m; i++) if (bits(expf(x[i])) != bits(y[i])) bad++;
        n += m;
    }
    float sp[] = {-INFINITY, INFINITY, 0.0f, -0.0f, -104.0f, -103.9f, 88.7f, 89.0f, 1e30f, -1e30f};
    float y[10];
    rf_expf_n(sp, y, 10);
    for (int i = 0; i < 10; i++) if (bits(expf(sp[i])) != bits(y[i])) bad++;
    float q = NAN;
    rf_expf_n(&q, y, 1);
    if (!isnan(y[0])) bad++;
    printf("%ld %ld\n", n, bad);
    return bad != 0;
}
"""


LOG_HARNESS = r"""
#include <math.h>
#include <stdio.h>
#include "fw_math.h"
int main(void) {
    long bad = 0, n = 0;
    #pragma omp parallel for reduction(+:bad,n) schedule(static)
    for (int64_t u = 0; u <= 0x7f800000LL; u++) {
        uint32_t v = (uint32_t)u; float x; memcpy(&x, &v, 4);
        n++;
        if (fw_f2u(logf(x)) != fw_f2u(fw_logf_host(x))) bad++;
    }
    if (!isnan(fw_logf_host(-1.0f)) || !isnan(fw_logf_host(NAN)) || fw_logf_host(-0.0f) != -INFINITY) bad++;
    printf("%ld %ld\n", n, bad);
    return bad != 0;
}
"""


def _compile_run(tmp_path, src, name, extra):
    c = tmp_path / f"{name}.c"
    c.write_text(src)
    exe = tmp_path / name
    subprocess.run(["gcc", "-O2", "-fopenmp", "-mf16c", "-mavx2", "-mfma", "-ffp-contract=off", str(c), "-o",
                    str(exe)] + extra + ["-lm"], check=True)
    env = dict(os.environ, OMP_NUM_THREADS=str(min(16, os.cpu_count() or 1)))
    r = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    return r


def test_f16_conversions_exhaustive_vs_f16c(tmp_path):
    O.build()
    r = _compile_run(tmp_path, F16_HARNESS, "f16x", ["-I", os.path.join(ROOT, "oracle"), os.path.join(
        ROOT, "oracle", "refcpu.c"), os.path.join(ROOT, "oracle", "refcpu_fast.c")])
    assert r.returncode == 0 and r.stdout.strip() == "0", r.stdout + r.stderr


def test_device_expf_restatement_matches_glibc_exhaustive(tmp_path):
    r = _compile_run(tmp_path, EXP_HARNESS, "expx", ["-I", os.path.join(ROOT, "franken_whisper_amd", "csrc")])
    n, bad = map(int, r.stdout.split())
    assert bad == 0 and n > 2_000_000_000, r.stdout


def test_fast_softmax_expf_matches_glibc_exhaustive(tmp_path):
    """The 8-lane expf of the FAST restatement's softmax (oracle/refcpu_fast.c)
    against the host's expf over every float of [-110, 90] plus the specials."""
    r = _compile_run(tmp_path, FAST_EXP_HARNESS, "fexpx", ["-I", os.path.join(ROOT, "oracle"),
                                                           os.path.join(ROOT, "oracle", "refcpu_fast.c")])
    n, bad = map(int, r.stdout.split())
    assert bad == 0 and n > 2_000_000_000, r.stdout


def test_device_logf_restatement_matches_glibc_exhaustive(tmp_path):
    r = _compile_run(tmp_path, LOG_HARNESS, "logx", ["-I", os.path.join(ROOT, "franken_whisper_amd", "csrc")])
    n, bad = map(int, r.stdout.split())
    assert bad == 0 and n == 0x7f800001, r.stdout


def _f(bits):
    return struct.unpack("<f", struct.pack("<I", bits))[0]


def test_quantize_act_i8_known_answers():
    # nn.rs:7454-7458: half-away on exact .5, clamp at +-127
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float32)
    np.testing.assert_array_equal(O.quantize_act_i8(x, 1.0), [1, 2, 3, -1, -2, -3, 127, -127])
    # 0x3EFFFFFF (0.49999997): the 8-wide add-trunc body rounds it to 1, the
    # scalar tail (f32::round) to 0 (nn.rs:3036-3038 vs 3050-3053)
    v = _f(0x3EFFFFFF)
    x = np.array([v] * 9, np.float32)
    got = O.quantize_act_i8(x, 1.0)
    assert list(got[:8]) == [1] * 8 and got[8] == 0
    got = O.quantize_act_i8(-x, 1.0)
    assert list(got[:8]) == [-1] * 8 and got[8] == 0


def test_quantize_row_i7_u8_known_answers():
    # nn.rs:7491-7500
    x = np.array([0.5, 1.5, 2.5, -0.5, -1.5, -2.5, 126.5, -126.5], np.float32)
    np.testing.assert_array_equal(O.quantize_row_i7_u8(x, 1.0), [129, 130, 131, 127, 126, 125, 255, 1])


def test_quant_row_i8_exact_is_round_half_away():
    # encoder.rs:2468-2508: exact rounding even in the 8-wide body
    x = np.array([_f(0x3EFFFFFF), 0.5, -0.5, 2.5, -2.5, 1e9, -1e9, 0.0, 3.4999998], np.float32)
    np.testing.assert_array_equal(O.quant_row_i8_exact(x, 1.0), [0, 1, -1, 3, -3, 127, -127, 0, 3])


def test_act_scale_floor():
    assert O.act_scale(np.zeros(16, np.float32)) == np.float32(np.float32(1e-9) / np.float32(127.0))
    assert O.act_scale(np.array([-254.0, 1.0], np.float32)) == np.float32(2.0)


def test_weight_quantizers_properties():
    rng = np.random.default_rng(0)
    w = (rng.standard_normal((37, 300)) * 0.02).astype(np.float16).view(np.uint16)
    wf = w.view(np.float16).astype(np.float32)
    q, s = O.quantize_f16_to_i8(w)
    # per-row: the amax element maps to +-127 and every element is within half a step
    assert np.all(np.abs(q).max(axis=1) == 127)
    wd = wf.astype(np.float64)
    assert np.all(np.abs(wd - q * s[:, None].astype(np.float64)) <= 0.5 * s[:, None] * 1.00001)
    np.testing.assert_allclose(s, np.abs(wf).max(axis=1) / 127, rtol=1e-6)
    # blocked: the same per 32-wide block
    qb, sb = O.quantize_f16_to_i8_blocked(w, 32)
    assert sb.shape == (37, 10)
    for b in range(10):
        blk = wf[:, 32 * b: 32 * b + 32]
        np.testing.assert_allclose(sb[:, b], np.maximum(np.abs(blk).max(axis=1), 1e-9) / 127, rtol=1e-6)
        deq = qb[:, 32 * b: 32 * b + 32].astype(np.float64) * sb[:, b: b + 1].astype(np.float64)
        assert np.all(np.abs(blk.astype(np.float64) - deq) <= 0.5 * sb[:, b: b + 1] * 1.00001)
    # encoder i8 (attn.out): exact rounding, amax/127
    q8, s8 = O.quantize_enc_i8_rows(w)
    assert np.all(np.abs(wd - q8 * s8[:, None].astype(np.float64)) <= 0.5 * s8[:, None] * 1.00001)


def test_i7_error_feedback_invariants():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((23, 512)) * 0.02).astype(np.float16).view(np.uint16)
    wf = w.view(np.float16).astype(np.float64)
    q, s, cs = O.quantize_rows_to_i7(w, ef=True)
    np.testing.assert_array_equal(cs, q.astype(np.int64).sum(axis=1))
    assert np.abs(q).max() <= 63
    # error diffusion keeps every running sum of (target - q) within half a step
    t = wf / s[:, None].astype(np.float64)
    run = np.cumsum(t - q, axis=1)
    assert np.abs(run).max() < 0.5 + 1e-3
    qn, sn, csn = O.quantize_rows_to_i7(w, ef=False)
    assert np.all(np.abs(t - qn) <= 0.5 + 1e-5)
    assert not np.array_equal(q, qn)  # the two schemes genuinely differ


def test_dot_f16c_lane_tree_known_answer():
    # n = 32: accumulator lane (j, l) holds element 8j + l.  Elements 0 and 16
    # (lanes (0,0) and (2,0)) are +-2^24 and element 1 (lane (0,1)) is 1: the
    # reference tree adds (a0+a1)+(a2+a3) lane-wise first, so 2^24 and -2^24
    # cancel exactly and the 1 survives; a sequential sum would lose it.
    w = np.zeros(32, np.float16)
    x = np.zeros(32, np.float32)
    w[0], x[0] = 1.0, 2.0 ** 24
    w[16], x[16] = 1.0, -(2.0 ** 24)
    w[1], x[1] = 1.0, 1.0
    assert O.dot_f16c(w.view(np.uint16), x) == 1.0
    assert np.float32(np.float32(2 ** 24) + np.float32(1)) - np.float32(2 ** 24) == 0.0
    # the 8-wide tail is reduced as its own tree then added: n = 40
    w = np.zeros(40, np.float16)
    x = np.zeros(40, np.float32)
    w[32], x[32] = 1.0, 2.0 ** 24
    w[36], x[36] = 1.0, -(2.0 ** 24)
    w[33], x[33] = 1.0, 1.0
    # tail tree: ((t0+t1)+(t2+t3)) + ((t4+t5)+(t6+t7)) = (2^24+1) + (-2^24) = 0
    assert O.dot_f16c(w.view(np.uint16), x) == 0.0


def test_dot_i8w_f32_matches_exact_integer_sum():
    rng = np.random.default_rng(2)
    for n in (32, 64, 40, 77):
        w = rng.integers(-127, 128, n).astype(np.int8)
        x = rng.integers(-50, 50, n).astype(np.float32)
        assert O.dot_i8w_f32(w, x) == float(np.dot(w.astype(np.int64), x.astype(np.int64)))


def test_gemv_i8_accumulator_and_epilogue():
    rng = np.random.default_rng(3)
    out, inp = 33, 1280
    w = (rng.standard_normal((out, inp)) * 0.02).astype(np.float16).view(np.uint16)
    q, s = O.quantize_f16_to_i8(w)
    x = rng.standard_normal(inp).astype(np.float32)
    b = rng.standard_normal(out).astype(np.float32)
    y = O.gemv_i8(q, s, x, b)
    xs = O.act_scale(x)
    xq = O.quantize_act_i8(x, np.float32(1.0) / xs)
    acc = q.astype(np.int64) @ xq.astype(np.int64)
    want = (acc.astype(np.float32) * s) * xs + b
    np.testing.assert_array_equal(y, want)
    # and it approximates the float product to int8 accuracy
    wf = w.view(np.float16).astype(np.float64)
    assert np.max(np.abs(y - (wf @ x + b))) < 0.05


def test_gemv_f16_and_blocked_vs_float64():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((19, 5120)) * 0.02).astype(np.float16)
    x = rng.standard_normal(5120).astype(np.float32)
    ref = w.astype(np.float64) @ x.astype(np.float64)
    np.testing.assert_allclose(O.gemv_f16(w.view(np.uint16), x), ref, rtol=0, atol=1e-5)
    qb, sb = O.quantize_f16_to_i8_blocked(w.view(np.uint16), 32)
    deq = (qb.reshape(19, 160, 32) * sb[:, :, None]).reshape(19, 5120).astype(np.float64)
    np.testing.assert_allclose(O.gemv_i8w_f32a_blocked(qb, sb, x), deq @ x, rtol=0, atol=1e-5)


def test_layer_norm_known_case_and_properties():
    # nn.rs:8180: [1,2,3,4], eps 0
    y = O.layer_norm(np.array([[1, 2, 3, 4]], np.float32), np.ones(4, np.float32), np.zeros(4, np.float32), 0.0)
    sd = np.sqrt(1.25)
    np.testing.assert_allclose(y[0], (np.array([1, 2, 3, 4]) - 2.5) / sd, atol=1e-6)
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((7, 1280)) * 3 + 1).astype(np.float32)
    w = rng.standard_normal(1280).astype(np.float32)
    b = rng.standard_normal(1280).astype(np.float32)
    y = O.layer_norm(x, w, b)
    xd = x.astype(np.float64)
    m = xd.mean(axis=1, keepdims=True)
    v = ((xd - m) ** 2).mean(axis=1, keepdims=True)
    want = (xd - m) / np.sqrt(v + np.float64(np.float32(1e-5))) * w + b
    np.testing.assert_allclose(y, want, rtol=0, atol=2e-6)


def _gelu_def(x):
    """The table's definition: tanh GELU of the f16-rounded input, re-rounded
    to f16 (whisper.cpp GGML_GELU_FP16), clamped at +-10."""
    x = np.asarray(x, np.float32)
    f = x.astype(np.float16).astype(np.float64)
    g = 0.5 * f * (1 + np.tanh(np.sqrt(2 / np.pi) * f * (1 + 0.044715 * f * f)))
    out = g.astype(np.float16).astype(np.float32)
    out = np.where(x <= -10, 0.0, np.where(x >= 10, x, out))
    return out.astype(np.float32)


def test_gelu_known_values_and_definition():
    g = O.gelu(np.array([0.0, 1.0, -1.0], np.float32))
    assert g[0] == 0.0 and abs(g[1] - 0.8412) < 1e-3 and abs(g[2] + 0.1588) < 1e-3  # nn.rs:8230-8256
    rng = np.random.default_rng(6)
    x = np.concatenate([rng.standard_normal(20000) * 4, [-10, 10, -10.001, 10.001, 9.99, -9.99]]).astype(np.float32)
    got = O.gelu(x)
    want = _gelu_def(x)
    # The reference evaluates the formula in f32 (glibc tanhf): near f16 rounding
    # boundaries that moves the result by one f16 ulp, and in the negative tail
    # the f32 cancellation in 1 + tanh(.) leaves a few 1e-7 of absolute error.
    diff = np.abs(got - want)
    assert np.all(diff <= np.abs(want) * 2 ** -10 + 5e-7)
    assert np.mean(diff == 0) > 0.9
    core = np.abs(x) < 1.5
    assert np.mean(diff[core] == 0) > 0.99


def test_softmax_properties():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((6, 11)).astype(np.float32)
    y = O.softmax_rows(x)
    np.testing.assert_allclose(y.sum(axis=1), 1, atol=1e-6)
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    np.testing.assert_allclose(y, e / e.sum(axis=1, keepdims=True), rtol=1e-6)
    y = O.softmax_rows(np.array([[1e30, 1e30 + 1, 0.0]], np.float32))  # nn.rs:8280
    assert np.all(np.isfinite(y)) and abs(y.sum() - 1) < 1e-5
    y = O.softmax_rows(np.array([[np.nan, 1.0, 0.0]], np.float32))  # nn.rs:8288
    assert y[0, 0] == 0.0 and abs(y.sum() - 1) < 1e-5
    y = O.softmax_rows(np.array([[-np.inf, -np.inf]], np.float32))  # all masked: left as-is
    assert np.all(y == -np.inf)


def test_matmul_strict_exact_integers_and_float():
    rng = np.random.default_rng(8)
    a = rng.integers(-8, 8, (13, 70)).astype(np.float32)
    b = rng.integers(-8, 8, (70, 21)).astype(np.float32)
    np.testing.assert_array_equal(O.matmul_strict(a, b), (a.astype(np.int64) @ b.astype(np.int64)).astype(np.float32))
    a = rng.standard_normal((9, 300)).astype(np.float32)
    b = rng.standard_normal((300, 17)).astype(np.float32)
    np.testing.assert_allclose(O.matmul_strict(a, b), a.astype(np.float64) @ b, rtol=0, atol=1e-4)


def test_argmax_first_semantics():
    assert O.argmax_first(np.array([1, 3, 3, 2], np.float32)) == 1
    assert O.argmax_first(np.array([np.nan, 1, 1], np.float32)) == 1
    assert O.argmax_first(np.array([-np.inf, -np.inf], np.float32)) == 0


def test_process_logits_masks_no_timestamps():
    from franken_whisper_amd import synth
    for cfg in (synth.TINY_EN, synth.TURBO):
        tk = synth.Tokens(cfg)
        f = tk.filter()
        V = cfg.n_vocab
        lg = np.zeros(V, np.float32)
        specials = [tk.eot, tk.sot, tk.sot_prev, tk.solm, tk.no_speech, tk.no_timestamps, tk.translate,
                    tk.transcribe, tk.timestamp_begin, V - 1, tk.sot + 1, tk.sot + 100, tk.space]
        for i, s in enumerate(specials):
            lg[s] = 100.0 - i
        lg[1234] = 50.0
        # first step: eot and the space token are suppressed too
        assert O.process_argmax(f, lg, True) == 1234
        # later steps: eot and the space token are allowed
        assert O.process_argmax(f, lg, False) == tk.eot
        lg[tk.eot] = 0.0
        assert O.process_argmax(f, lg, False) == tk.space



def _f16_weight_rows(amaxes, width):
    """Rows [amax, w...] covering every non-negative f16 w <= amax with both
    signs (zero padded to whole rows)."""
    allw = np.arange(0, 0x7C00, dtype=np.uint16)
    allf = allw.view(np.float16).astype(np.float64)
    rows = []
    for a in amaxes:
        af = float(np.uint16(a).view(np.float16))
        ws = allw[allf <= af]
        ws = np.concatenate([ws, ws | np.uint16(0x8000)])  # both signs
        n = width - 1
        pad = (-ws.size) % n
        ws = np.concatenate([ws, np.zeros(pad, np.uint16)]).reshape(-1, n)
        rows.append(np.concatenate([np.full((ws.shape[0], 1), a, np.uint16), ws], axis=1))
    return np.concatenate(rows)


def _half_away_of_f32_product(rows, amax_col):
    """The quantizer written from its definition: v = f32(w) * inv with
    scale = f32(amax / 127), inv = f32(1 / scale) (nn.rs:2540-2552), then
    round-half-away of v taken exactly in float64 (|v| + 1/2 is exact for an
    f32 v) and clamped to 127."""
    wf = rows.view(np.float16).astype(np.float32)
    af = amax_col.view(np.float16).astype(np.float32)
    scale = (af / np.float32(127.0)).astype(np.float32)
    inv = (np.float32(1.0) / scale).astype(np.float32)
    v = (wf * inv[:, None]).astype(np.float32).astype(np.float64)
    return (np.sign(v) * np.minimum(127.0, np.floor(np.abs(v) + 0.5))).astype(np.int8), wf, af


def _tie_amaxes():
    # amax whose f16 mantissa is a multiple of 127 (for them 127 w / amax can
    # be k + 1/2 for any k; for every other amax only w = amax / 2 gives a
    # tie, 63.5), plus a seeded sample of others
    out = set()
    for a in range(1, 0x7C00):
        m = a & 0x3FF
        mant = (m | 0x400) if (a >> 10) else m
        if mant % 127 == 0:
            out.add(a)
    rng = np.random.default_rng(5)
    out.update(int(x) for x in rng.integers(1, 0x7C00, size=120))
    return sorted(out)


def test_decoder_weight_quantizer_on_every_f16_row():
    """quantize_f16_row_to_i8_into (nn.rs:2490-2555): the 8-wide body rounds by
    add-0.5-then-truncate in f32, the n % 8 tail by round-half-away.  The two
    differ only where f32(w) * inv is +-0x3EFFFFFF (0.49999997 + 0.5 rounds to
    1.0), and no f16 row lands there, so both equal round-half-away of the
    product.  Checked for every f16 w against every tie-capable amax, once
    entirely in the body (rows of 16) and once entirely in the tail (rows of
    7).  Against the exact rational round(127 w / amax) the quantizer differs
    only on the exact ties 63.5 (w = amax / 2) where f32(1 / scale) rounds
    down: the reference gives 63 there, and so must the oracle."""
    amaxes = _tie_amaxes()
    n_ties = n_low = 0
    for width in (16, 7):
        rows = _f16_weight_rows(amaxes, width)
        want, wf, af = _half_away_of_f32_product(rows, rows[:, 0])
        q, s = O.quantize_f16_to_i8(rows)
        np.testing.assert_array_equal(q, want)
        np.testing.assert_array_equal(s.view(np.uint32), (af / np.float32(127.0)).astype(np.float32).view(np.uint32))
        t = 127.0 * np.abs(wf.astype(np.float64)) / af[:, None].astype(np.float64)
        exact = (np.sign(wf) * np.minimum(127.0, np.floor(t + 0.5))).astype(np.int8)
        ties = (t % 1.0 == 0.5) & (t < 127)
        n_ties += int(ties.sum())
        diff = q != exact
        n_low += int(diff.sum())
        assert np.all(t[diff] == 63.5), "only the w = amax / 2 ties may round below the rational value"
        # planted mistake: ties to even (rint) disagrees on exact ties of even k
        even = (np.sign(wf) * np.minimum(127.0, np.rint(t))).astype(np.int8)
        assert np.any(even[ties] != q[ties])
    assert n_ties > 10_000 and n_low > 0


def test_blocked_weight_quantizer_on_f16_rows():
    """quantize_f16_row_blocked_to_int_into (nn.rs:3619-3693, max_level 127,
    block 32): the same per 32-wide block, with the body/tail split at each
    block's multiple of 8.  Rows of 39 = a block of 32 (all body) and a
    block of 7 (all tail), each [amax, w...]."""
    amaxes = [a for a in _tie_amaxes() if a % 3 == 0][:60]
    r32 = _f16_weight_rows(amaxes, 32)
    r7 = _f16_weight_rows(amaxes, 7)
    n = min(r32.shape[0], r7.shape[0])
    rows = np.concatenate([r32[:n], r7[:n]], axis=1)
    w32, _, a0 = _half_away_of_f32_product(rows[:, :32], rows[:, 0])
    w7, _, a1 = _half_away_of_f32_product(rows[:, 32:], rows[:, 32])
    q, s = O.quantize_f16_to_i8_blocked(rows, 32)
    np.testing.assert_array_equal(q, np.concatenate([w32, w7], axis=1))
    np.testing.assert_array_equal(s[:, 0], a0 / np.float32(127.0))
    np.testing.assert_array_equal(s[:, 1], a1 / np.float32(127.0))


def test_weight_quantizer_known_answers():
    # amax 127 (scale 1, inv 1): exact halves round away from zero in the body
    # and in the tail; 126.5 -> 127, -126.5 -> -127
    row = np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, 126.5, -126.5,
                    2.5, -2.5, 0.5, -0.5, 1.5, 126.5, -126.5], np.float16).view(np.uint16)
    q, s = O.quantize_f16_to_i8(row[None, :])
    np.testing.assert_array_equal(q[0], [127, 3, -3, 1, -1, 2, 127, -127, 3, -3, 1, -1, 2, 127, -127])
    assert s[0] == np.float32(1.0)
    # amax 1143 = 127 * 9: scale 9, f32(1/9) rounds up, so 22.5 -> 2.5 -> 3
    row = np.array([1143.0, 22.5, -22.5, 4.5, 31.5, 0.0, 0.0, 0.0, 22.5, 4.5], np.float16).view(np.uint16)
    q, s = O.quantize_f16_to_i8(row[None, :])
    np.testing.assert_array_equal(q[0], [127, 3, -3, 1, 4, 0, 0, 0, 3, 1])
    assert s[0] == np.float32(9.0)
    # w = amax / 2 with f32(1 / scale) rounding down: 63.499996 -> 63 (the
    # rational value 63.5 would give 64), in the body and in the tail
    row = np.array([0x24C, 0x126, 0x8126, 0, 0, 0, 0, 0, 0x126], np.uint16)
    q, s = O.quantize_f16_to_i8(row[None, :])
    np.testing.assert_array_equal(q[0], [127, 63, -63, 0, 0, 0, 0, 0, 63])
    # the 1e-9 floor on an all-zero row
    q, s = O.quantize_f16_to_i8(np.zeros((1, 12), np.uint16))
    assert not q.any() and s[0] == np.float32(np.float32(1e-9) / np.float32(127.0))


def test_no_f16_row_reaches_the_add_trunc_split():
    """Exhaustive: for every positive f16 amax and every f16 w with |w| <= amax,
    f32(|w|) * f32(1 / f32(amax / 127)) is never 0x3EFFFFFF, the one product on
    which add-0.5-then-truncate (1) and round-half-away (0) disagree; so the
    weight quantizers' body and tail give the same values on every f16 row."""
    h = np.arange(1, 0x7C00, dtype=np.uint16)
    hf = h.view(np.float16).astype(np.float32)
    hits = 0
    for amax in hf:
        inv = np.float32(1.0) / (np.float32(amax) / np.float32(127.0))
        prod = (hf[hf <= amax] * inv).astype(np.float32)
        hits += int(np.count_nonzero(prod.view(np.uint32) == np.uint32(0x3EFFFFFF)))
    assert hits == 0
    # the split itself (planted): 0.49999997 + 0.5 rounds to 1.0 in f32
    v = np.uint32(0x3EFFFFFF).view(np.float32)
    assert np.trunc(np.float32(v + np.float32(0.5))) == 1.0 and np.floor(np.float64(v) + 0.5) == 0.0
