"""Benchmark of the hot path on one MI355X.

Default workload (the whole job the headline metric is quoted on): large-v3-turbo
architecture with seeded random-init weights, 300 s of seeded synthetic 16 kHz
audio with silent gaps -> GPU log-mel (128 bins, Slaney filterbank; 33,000
frames) -> 10 windows x 30 s (3000 frames each, offsets 0, 3000, ...), int8 encoder plan
(FW_ENC_ATTN_OUT_I8I32: i7 q/k/v/fc1/fc2, i8 attn.out), cross K/V precompute,
then greedy no-timestamps decode of every window as one cohort with the f16
decoder arm (--dec-arm int8 for the int8 arm) and the f16 KV cache: 4-token
prompt + 220 sampled tokens.  One step = that whole job.  After the timed
region the job runs once more in exact mode (bit-identical to the oracle) and
the timed run's tokens are compared with it window by window; the int8 decoder
arm is timed on the same job and reported beside the headline with its own
token comparison.  Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload job|enc-f32|enc-int8|decode|step|tiny|...]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
PEAK_TFLOPS = {"int8": 5000.0, "f16": 2500.0, "f32": 157.3}
# dense algorithmic work, large-v3-turbo, per 30 s window (no ToMe)
ENC_GOP_PER_WINDOW = 2273.8  # all GEMMs + SDPA
ENC_GEMM_GOP_PER_WINDOW = 1887.4


def _classes():
    from franken_whisper_amd import abi

    # kernel class -> (name, roofline bound, MFMA operand type, traffic record)
    return {
        abi.K_ENC_GEMM_I8: ("encoder int8 GEMM (k_gemm_pi8, persistent int8 tiles)", "mfma", "int8", "enc_gemm_i8"),
        abi.K_ENC_GEMM_F32: ("encoder f16-pair GEMM (k_gemm2, conv stem)", "mfma", "f16", None),
        abi.K_ENC_ATTN: ("encoder attention (k_attention2, f16 pairs)", "mfma", "f16", None),
        abi.K_DEC_CROSS: ("decoder cross K/V precompute (k_gemm2 f16 pairs, all layers)", "mfma", "f16", None),
        abi.K_DEC_STEP: ("decoder step (graph replay of one sampled step: weights + cross K/V + KV cache)",
                         "hbm", None, "dec_step"),
        abi.K_DEC_LOGITS: ("decoder logits GEMV of the prompt row (k_gemv_i8m)", "hbm", None, None),
    }


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--workload", default="job",
                   choices=["job", "enc-f32", "enc-int8", "decode", "step", "tiny", "copy", "load", "transcribe"])
    p.add_argument("--kv", default="f16", choices=["f16", "f32"],
                   help="decoder self-attention cache: f16 (FW_KV_F16) or f32 (the reference's default)")
    p.add_argument("--depths", default="0,64,224,447",
                   help="step workload: KV-cache depths at which one token per stream is stepped")
    p.add_argument("--windows", type=int, default=None)
    p.add_argument("--tokens", type=int, default=220)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "16")))
    p.add_argument("--cpu-runs", type=int, default=5, help="end-to-end runs of one window for the CPU baseline")
    p.add_argument("--copy-mb", type=int, default=512)
    p.add_argument("--exact", action="store_true", help="exact mode: bit-identical to the reference's strict mode")
    p.add_argument("--dec-arm", default="f16", choices=["int8", "f16"],
                   help="decoder arm (f16: the tied f16 logits head, token-stable; int8: the reference default)")
    p.add_argument("--no-verify", action="store_true", help="skip the exact-mode token check of the job")
    p.add_argument("--tome", type=int, default=0,
                   help="ToMe rows merged after encoder block 3 (FW_TOME_R; -1: the reference's default rule, "
                        "500 for large-v3-turbo); 0 = the un-merged encoder")
    p.add_argument("--no-tome-run", action="store_true",
                   help="skip the job's second timed run with the reference's default ToMe")
    return p.parse_args()


def host_topology():
    """CPUs this process may use, and the host's sockets / cores / SMT (lscpu)."""
    import subprocess

    topo = {"nproc": len(os.sched_getaffinity(0))}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        keys = {"Socket(s)": "sockets", "Core(s) per socket": "cores_per_socket",
                "Thread(s) per core": "threads_per_core", "Model name": "model"}
        for line in out.splitlines():
            k, _, v = line.partition(":")
            if k.strip() in keys:
                v = v.strip()
                topo[keys[k.strip()]] = int(v) if v.isdigit() else v
    except (OSError, subprocess.SubprocessError):
        pass
    return topo


def cpu_baseline(model, n_windows, n_tokens, threads, runs, arm):
    """The oracle (C restatement of the reference CPU path, OpenMP) on a bounded
    sample of the same job: window 0 of the job run end to end (int8-plan
    encoder over all layers, cross K/V precompute, prompt prefill and greedy
    decode of n_tokens) plus its share of the whole job's log-mel, scaled to
    audio-seconds per second.  The timed leg is the FAST restatement
    (register-blocked AVX2 / F16C kernels, oracle/refcpu_fast.c, which give the
    strict restatement's bits): the median of `runs` runs, alternating between
    two halves whose medians give an A/A spread (the noise of the
    measurement).  One run of the strict scalar restatement is reported beside
    it, and both must decode the same tokens.  Returns the baseline record and
    the sampled window's tokens."""
    from franken_whisper_amd import abi, synth
    from oracle import oracle as O

    lib = O.lib()
    lib.ref_set_num_threads(threads)
    cfg = model.cfg
    e = O.Encoder(model, abi.ENC_INT8)
    d = O.Decoder(model, arm)
    tk = model.tokens
    filt = tk.filter()
    prompt = tk.sot_sequence(language_id=0)
    nf = 2 * cfg.n_audio_ctx
    samples = synth.audio(AUDIO_SEED, 30.0 * n_windows, gaps=True)
    filters = synth.mel_filterbank(cfg.n_mels)
    t0 = time.perf_counter()
    full = O.log_mel(samples, filters)
    t_mel = (time.perf_counter() - t0) / n_windows
    win = np.ascontiguousarray(full[:, :nf].T)

    def one():
        t0 = time.perf_counter()
        y = e.forward(win)
        t1 = time.perf_counter()
        toks = d.state(y).greedy(prompt, n_tokens, filt)
        t2 = time.perf_counter()
        return t_mel + t2 - t0, t1 - t0, t2 - t1, toks

    try:
        lib.ref_set_fast(1)
        runs_ = [one() for _ in range(runs)]
    finally:
        lib.ref_set_fast(0)
    strict = one()
    times = [r[0] for r in runs_]
    toks = runs_[-1][3]
    same = all(np.array_equal(np.asarray(r[3]), np.asarray(strict[3])) for r in runs_)
    med = float(np.median(times))
    a, b = float(np.median(times[0::2])), float(np.median(times[1::2]))
    topo = host_topology()
    dec_txt = "int8" if arm == abi.DEC_INT8 else "f16"
    rec = {
        "value": round(30.0 / med, 4),
        "unit": "audio-s/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle FAST restatement (register-blocked AVX2/F16C kernels giving the strict restatement's bits, "
                   f"-O3 -march=x86-64-v3, {threads} OpenMP threads = this GPU's share of the host) on window 0 of "
                   f"the job end to end, {runs} runs: median {med:.2f} s per 30 s window (log-mel share "
                   f"{t_mel:.3f} s, int8-plan encoder {np.median([r[1] for r in runs_]):.2f} s, cross K/V + prefill "
                   f"+ greedy decode of {len(toks)} tokens on the {dec_txt} decoder arm "
                   f"{np.median([r[2] for r in runs_]):.2f} s); A/A spread {abs(a - b) / med * 100:.1f}%; the "
                   f"strict scalar restatement takes {strict[0]:.2f} s on the same window; the reference's own "
                   f"engine publishes ~1.44 s per turbo encoder window (docs/PERF_FRONTIER.md:48-59)"),
        "runs_s": [round(t, 3) for t in times],
        "aa_spread": round(abs(a - b) / med, 4),
        "strict": {"value": round(30.0 / strict[0], 4), "s_per_window": round(strict[0], 3),
                   "encoder_s": round(strict[1], 3), "decode_s": round(strict[2], 3),
                   "tokens_identical_to_fast": bool(same)},
        "host": topo,
    }
    return rec, toks


AUDIO_SEED = 1234


# rocprofv3 counter measurements of the job's kernels, per class: file and the
# key of its "key: bytes" line (the counters cannot be read inside a timed run)
TRAFFIC = {"enc_gemm_i8": ("profiles/k_gemm_pi8_int8_encoder_job.md", "traffic_bytes_per_launch"),
           "dec_step_int8": ("profiles/decode_step_int8_10_streams.md", "traffic_bytes_per_step"),
           "dec_step_f16": ("profiles/decode_step_f16_10_streams.md", "traffic_bytes_per_step")}


def measured_traffic(which):
    """HBM bytes per launch (or per decoder step) of a kernel class on this
    job's shapes, as recorded from rocprofv3 FETCH_SIZE / WRITE_SIZE runs."""
    import re

    path, key = TRAFFIC[which]
    try:
        with open(os.path.join(ROOT, path)) as f:
            m = re.search(r"^" + key + r":\s*(\d+)", f.read(), re.M)
        return (int(m.group(1)), path) if m else (None, path)
    except OSError:
        return None, path


def verify_tokens(ctx, model, mel_dev, mel_frames, offsets, nf, W, prompt, n_tokens, filt, got, tome=0, kv_f16=True):
    """The job once more in exact mode (encoder and cross K/V in the reference's
    strict-parity arithmetic, bit-identical to it; tome and kv_f16: the same ToMe
    setting and self-attention cache as the timed job), decoded on each arm;
    returns per arm the exact tokens, and how many of the timed job's windows
    (got: arm -> tokens) match them."""
    from franken_whisper_amd import abi, native

    cfg = model.cfg
    enc = native.Encoder(ctx, model, abi.ENC_INT8)
    enc.set_exact(True)
    enc.set_tome(tome, 3)
    states = ctx.empty((W, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    enc.forward_mel(mel_dev, mel_frames, offsets, nf, states)
    enc.close()
    out = {}
    for arm, toks in got.items():
        dec = native.Decoder(ctx, model, arm)
        dec.set_exact(True)
        dec.set_kv_f16(kv_f16)
        st = dec.state(W, cfg.n_audio_ctx)
        st.set_cross(states)
        ref = st.greedy(prompt, n_tokens, filt)
        st.close()
        dec.close()
        same = sum(int(np.array_equal(a, b)) for a, b in zip(toks, ref))
        out[arm] = (ref, same)
    states.free()
    return out


def copy_calibration(mb, reps):
    """A plain device-to-device copy of known size (torch's elementwise copy
    kernel): the reference reading for the FETCH_SIZE / WRITE_SIZE counters."""
    import torch

    n = mb * (1 << 20) // 4
    a = torch.randn(n, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(reps):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"workload": "copy", "bytes_per_copy": 4 * n, "reps": reps}))


def load_workload(a):
    """Model load from a ggml file, the one-time cost the reference reports as
    model_parse + model_weights (docs/PERF_FRONTIER.md:48-74): the seeded
    large-v3-turbo weights are written once as a ggml f16 file (the layout of
    whisper.cpp's ggml-large-v3-turbo.bin), then each step opens it
    (directory scan), loads the int8-plan encoder and the decoder arm from it
    (pread, upload, load-time quantization and packing on the GPU) and frees
    them.  The file is read from the page cache after the first pass.  Beside
    it, the GPU decode of a q8_0 payload the size of the token embedding
    (51866 x 1280) gives the dequantization kernel's HBM roofline."""
    import shutil
    import tempfile

    from franken_whisper_amd import abi, native, synth
    from franken_whisper_amd import ggml as gg

    cfg = synth.TURBO
    tdir = tempfile.mkdtemp(prefix="fwhip-ggml-")
    path = os.path.join(tdir, "ggml-large-v3-turbo-seeded.bin")
    t = time.perf_counter()
    gg.write_model(path, synth.Model(cfg, seed=0))
    write_s = time.perf_counter() - t
    fsize = os.path.getsize(path)
    ctx = native.Context(0)
    arm = abi.DEC_F16 if a.dec_arm == "f16" else abi.DEC_INT8

    def one():
        t0 = time.perf_counter()
        g = native.GgmlFile(path)
        t1 = time.perf_counter()
        enc = native.Encoder(ctx, g, abi.ENC_INT8)
        ctx.synchronize()
        t2 = time.perf_counter()
        dec = native.Decoder(ctx, g, arm)
        ctx.synchronize()
        t3 = time.perf_counter()
        enc.close()
        dec.close()
        g.close()
        return (t1 - t0) * 1e3, (t2 - t1) * 1e3, (t3 - t2) * 1e3

    for _ in range(a.warmup):
        one()
    runs = [one() for _ in range(a.steps)]
    parse_ms, enc_ms, dec_ms = (float(np.median([r[i] for r in runs])) for i in range(3))
    total = [sum(r) for r in runs]

    # dequantization kernel roofline: q8_0, 51866 x 1280 elements
    n = 51866 * 1280
    rng = np.random.default_rng(5)
    blocks = rng.integers(0, 256, (n // 32, 34), dtype=np.uint8)
    blocks[:, 0:2] = (rng.standard_normal(n // 32).astype(np.float16) * np.float16(0.01)).view(np.uint8).reshape(-1, 2)
    raw = ctx.array(blocks.reshape(-1))
    out = ctx.empty((n,), np.float32)
    for _ in range(3):
        native.dequant(ctx, 8, raw, blocks.size, n, out)
    ctx.synchronize()
    ctx.timing(True)
    reps = 20
    for _ in range(reps):
        native.dequant(ctx, 8, raw, blocks.size, n, out)
    ctx.synchronize()
    launches, ms, units = ctx.kernel_stats(abi.K_DEQUANT)
    ctx.timing(False)
    ach = units / (ms * 1e-3) / 1e9
    ctx.close()
    shutil.rmtree(tdir, ignore_errors=True)
    print(json.dumps({
        "metric": "large-v3-turbo model load from a ggml f16 file (directory scan + int8-plan encoder + decoder arm "
                  "resident on the GPU)",
        "value": round(float(np.median(total)), 1), "unit": "ms", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "higher_is_better": False, "dtype": "f16 file -> int8 encoder, " + a.dec_arm + " decoder",
        "data": "synthetic (seeded random-init large-v3-turbo weights written as a ggml f16 file)",
        "config": {"workload": "model load", "file_bytes": fsize,
                   "decoder_arm": a.dec_arm},
        "parts_ms": {"parse": round(parse_ms, 1), "encoder_weights": round(enc_ms, 1),
                     "decoder_weights": round(dec_ms, 1)},
        "runs_ms": [round(x, 1) for x in total],
        "write_file_s": round(write_s, 1),
        "reference_published": {"model_parse_ms": 182, "model_weights_ms": 745, "source": "docs/PERF_FRONTIER.md:48-59",
                                "note": "the reference's CPU load of large-v3-turbo (int8 encoder plan), measured on "
                                        "its own hardware"},
        "roofline": {"kernel": "k_dequant<q8_0> (51866 x 1280 elements)", "bound": "hbm", "launches": launches,
                     "avg_launch_ms": round(ms / launches, 4), "achieved": round(ach, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(ach / HBM_PEAK_GBS, 4), "traffic": None,
                     "algorithmic_bytes": round(units / launches)},
    }))


def xattn_roofline(ctx, st, S, cfg, filt, depth=114, n=5):
    """Roofline entry of the fused cross-attention sublayer kernel
    (k_cross_attn_f16p / k_cross_attn_i8v2: LayerNorm, q projection, attention
    over the cohort's cross K/V), measured outside the timed region: the
    cohort's caches are refilled to `depth` rows (the job's mean cache depth:
    4 prompt rows + half of 220 steps) with seeded tokens, then `n` one-token
    steps run with direct launches, each kernel bracketed by HIP events on the
    library's stream.  Bytes per launch: the layer's cross K/V of every stream
    and the q weights.  The state is reset afterwards."""
    from franken_whisper_amd import abi, synth

    toks = synth.uniform_i32(6, "xattn_tokens", 0, cfg.n_vocab, S * (depth + n)).reshape(S, depth + n)
    st.reset()
    st.step(toks[:, :depth])
    ctx.synchronize()
    ctx.timing(True)
    for i in range(n):
        st.step(toks[:, depth + i:depth + i + 1], filt=filt)
    k, ms, units = ctx.kernel_stats(abi.K_DEC_XATTN)
    ctx.timing(False)
    st.reset()
    if not k:
        return None
    gbs = units / (ms * 1e-3) / 1e9
    return {"kernel": "decoder cross-attention sublayer (k_cross_attn_f16p / k_cross_attn_i8v2: LayerNorm, q, "
                      f"attention over the cross K/V; one-token steps at cache depth {depth}-{depth + n - 1}, "
                      "direct launches, outside the timed region)",
            "bound": "hbm", "launches": k, "avg_launch_ms": round(ms / k, 4), "total_ms": round(ms, 3),
            "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(gbs / HBM_PEAK_GBS, 4),
            "traffic": None, "algorithmic_bytes": round(units / k), "in_timed_region": False}


def step_workload(a):
    """The large-v3-turbo decoder step in isolation (forward_step + logits_last
    + argmax for every stream of a cohort, decoder.rs:1754-1906, 2048-2147) at
    fixed cache depths: for each depth L the cohort's caches are filled by a
    prefill of L seeded tokens (uniform in [0, 51866)) over seeded N(0,1)
    encoder states (one per stream), then one token per stream is stepped at
    position L (it attends L cached rows and its own).  Each repetition resets
    the state, refills it (untimed) and times the step with HIP events on the
    library's stream (kernel class FWHIP_K_DEC_STEP: direct launches, no graph).
    Reported per depth: device time, tokens/s and algorithmic HBM bytes / time."""
    from franken_whisper_amd import abi, native, synth

    cfg = synth.TURBO
    S = a.windows or 1
    depths = [int(x) for x in a.depths.split(",")]
    if any(not 0 <= L < cfg.n_text_ctx for L in depths):
        raise SystemExit(f"--depths must lie in [0, {cfg.n_text_ctx - 1}]")
    model = synth.Model(cfg, seed=0, encoder=False, decoder=True)
    ctx = native.Context(0)
    arm = abi.DEC_F16 if a.dec_arm == "f16" else abi.DEC_INT8
    dec = native.Decoder(ctx, model, arm)
    if a.exact:
        dec.set_exact(True)
    dec.set_kv_f16(a.kv == "f16")
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(ctx.array(synth.encoder_states(77, S, cfg.n_audio_ctx, cfg.n_audio_state)))
    toks = synth.uniform_i32(5, "step_tokens", 0, cfg.n_vocab, S * cfg.n_text_ctx).reshape(S, cfg.n_text_ctx)
    filt = model.tokens.filter()
    rows = []
    for L in depths:
        def once():
            st.reset()
            if L:
                st.step(toks[:, :L])
            return st.step(toks[:, L:L + 1], filt=filt, initial=L == 0)
        for _ in range(a.warmup):
            once()
        ctx.synchronize()
        ctx.timing(True)
        t0 = time.perf_counter()
        host = 0.0
        for _ in range(a.steps):
            st.reset()
            if L:
                st.step(toks[:, :L])
            t = time.perf_counter()
            st.step(toks[:, L:L + 1], filt=filt, initial=L == 0)
            host += time.perf_counter() - t
        n, ms, units = ctx.kernel_stats(abi.K_DEC_STEP)
        xk, xms, xunits = ctx.kernel_stats(abi.K_DEC_XATTN)
        ctx.timing(False)
        wall = time.perf_counter() - t0
        if n != a.steps:
            raise SystemExit(f"expected {a.steps} timed steps at depth {L}, the library recorded {n}")
        us = ms * 1e3 / n
        gbs = units / (ms * 1e-3) / 1e9
        rows.append({"depth": L, "device_us_per_step": round(us, 1), "tok_s": round(S / (us * 1e-6), 1),
                     "host_us_per_step": round(host * 1e6 / a.steps, 1),
                     "algorithmic_bytes": round(units / n), "achieved_GBs": round(gbs, 1),
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "wall_s": round(wall, 2)})
        if xk:  # the fused cross-attention sublayer kernel, when the cohort takes it
            rows[-1]["xattn_us"] = round(xms * 1e3 / xk, 2)
            rows[-1]["xattn_GBs"] = round(xunits / (xms * 1e-3) / 1e9, 1)
    mean_us = sum(r["device_us_per_step"] for r in rows) / len(rows)
    top = max(rows, key=lambda r: r["device_us_per_step"])
    out = {"metric": "decode tok/s, large-v3-turbo decoder step in isolation", "value": round(S / (mean_us * 1e-6), 1),
           "unit": "tok/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
           "ms_per_step": round(mean_us * 1e-3, 4), "higher_is_better": True, "scaling": "weak",
           "vs_baseline": None, "dtype": "f16" if a.dec_arm == "f16" else "int8+f32",
           "data": "synthetic (seeded random-init weights N(0,0.02), seeded N(0,1) encoder states, seeded tokens)",
           "config": {"workload": f"large-v3-turbo decoder step, {S} stream(s), {a.dec_arm} arm, {a.kv} KV cache "
                                  f"filled to depth L in {depths}, logits + argmax", "streams": S, "depths": depths,
                      "mode": "exact" if a.exact else "fast"},
           "roofline": {"kernel": f"decoder step at depth {top['depth']} (forward, logits, argmax; direct launches)",
                        "bound": "hbm", "achieved": top["achieved_GBs"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": top["frac"], "traffic": None},
           "per_depth": rows}
    st.close()
    dec.close()
    ctx.close()
    print(json.dumps(out))


def tiny_workload(a):
    """Whisper tiny.en end to end on one window: 30 s of seeded synthetic
    16 kHz audio -> GPU log-mel (80 bins) -> f32-plan encoder (4 layers,
    d 384) -> cross K/V -> greedy no-timestamps decode of up to `--tokens`
    tokens from the SOT prefix (the reference loop's end-of-text stop).
    Reported: audio-s/s of the whole window and the decoder's tokens/s."""
    from franken_whisper_amd import abi, native, synth

    cfg = synth.TINY_EN
    W = a.windows or 1
    nf = 2 * cfg.n_audio_ctx
    model = synth.Model(cfg, seed=0)
    ctx = native.Context(0)
    samples = synth.audio(AUDIO_SEED, 30.0 * W)
    sd = ctx.array(samples)
    fd = ctx.array(synth.mel_filterbank(cfg.n_mels))
    mel_frames = native.mel_frames(samples.size)
    mel_dev = ctx.empty((cfg.n_mels, mel_frames), np.float32)
    offsets = np.arange(W, dtype=np.int64) * nf
    enc = native.Encoder(ctx, model, abi.ENC_F32)
    dec = native.Decoder(ctx, model, abi.DEC_F16 if a.dec_arm == "f16" else abi.DEC_INT8)
    if a.exact:
        enc.set_exact(True)
        dec.set_exact(True)
    st = dec.state(W, cfg.n_audio_ctx)
    enc_out = ctx.empty((W, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    tk = model.tokens
    filt = tk.filter()
    prompt = tk.sot_sequence()
    n_tok = [0]

    def one():
        ctx.log_mel(sd, samples.size, fd, cfg.n_mels, mel_dev)
        enc.forward_mel(mel_dev, mel_frames, offsets, nf, enc_out)
        st.set_cross(enc_out)
        out = st.greedy(prompt, a.tokens, filt)
        n_tok[0] = sum(len(t) for t in out)

    for _ in range(a.warmup):
        one()
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        one()
    ctx.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / a.steps
    # the decode alone (cross K/V in place), for the decoder's tokens/s
    t0 = time.perf_counter()
    for _ in range(a.steps):
        st.reset()
        st.greedy(prompt, a.tokens, filt)
    ctx.synchronize()
    dms = (time.perf_counter() - t0) * 1e3 / a.steps
    out = {"metric": "audio-s/sec whisper tiny.en encode+greedy decode", "value": round(30.0 * W / (ms * 1e-3), 2),
           "unit": "audio-s/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup, "ms_per_step": round(ms, 3),
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f32 (f16-pair MFMA)+" + ("f16" if a.dec_arm == "f16" else "int8"),
           "data": "synthetic (seeded random-init weights N(0,0.02), seeded synthetic 16 kHz audio)",
           "config": {"workload": f"whisper tiny.en: {W} x 30 s window(s), log-mel (80 bins), f32 encoder, "
                                  f"greedy decode of up to {a.tokens} tokens, {a.dec_arm} decoder arm",
                      "windows": W, "max_tokens": a.tokens, "mode": "exact" if a.exact else "fast"},
           "tokens": n_tok[0], "decode_ms": round(dms, 3), "decode_tok_s": round(n_tok[0] / (dms * 1e-3), 1)}
    st.close()
    dec.close()
    enc.close()
    ctx.close()
    print(json.dumps(out))


def transcribe_workload(a):
    """The window driver end to end (fwhip_transcribe: log-mel of the whole
    audio, encoder windows at the seeks, the device window loop, the rules
    between windows) on the job's audio (300 s of seeded synthetic 16 kHz
    audio with silent gaps) and the large-v3-turbo architecture (seeded
    random-init weights, int8 encoder, f16 decoder arm), in two settings:
    no timestamps without a carried prompt (independent windows, batched as
    cohorts: the job's own decode semantics), and the reference's timestamp
    mode with its default prompt carry (windows in sequence, one stream)."""
    from franken_whisper_amd import abi, native, synth
    from franken_whisper_amd import ggml as gg

    cfg = synth.TURBO
    W = a.windows or 10
    model = synth.Model(cfg, seed=0)
    ctx = native.Context(0)
    enc = native.Encoder(ctx, model, abi.ENC_INT8)
    dec = native.Decoder(ctx, model, abi.DEC_F16 if a.dec_arm == "f16" else abi.DEC_INT8)
    samples = synth.audio(AUDIO_SEED, 30.0 * W, gaps=True)
    sd = ctx.array(samples)
    fd = ctx.array(synth.mel_filterbank(cfg.n_mels))
    tk = model.tokens
    vocab = gg.synthetic_vocab(tk.eot)
    res = {}
    for name, kw in (("independent_no_timestamps", dict(timestamps=False, max_context=0)),
                     ("timestamps_prompt_carry", dict(timestamps=True))):
        sot = tk.sot_sequence(language_id=0, timestamps=kw["timestamps"])
        out = None
        for _ in range(a.warmup):
            native.transcribe(ctx, enc, dec, sd, samples.size, fd, cfg.n_mels, tk.filter(), vocab, sot, **kw)
        ctx.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            out = native.transcribe(ctx, enc, dec, sd, samples.size, fd, cfg.n_mels, tk.filter(), vocab, sot, **kw)
        ctx.synchronize()
        ms = (time.perf_counter() - t0) * 1e3 / a.steps
        wins = out["windows"]
        res[name] = {"value": round(30.0 * W / (ms * 1e-3), 2), "ms_per_run": round(ms, 2), "windows": len(wins),
                     "sampled_tokens": int(sum(len(w["tokens"]) for w in wins)), "segments": len(out["segments"])}
    enc.close()
    dec.close()
    ctx.close()
    first = res["independent_no_timestamps"]
    print(json.dumps({
        "metric": "audio-s/sec large-v3-turbo transcribe_samples (fwhip_transcribe, from audio)",
        "value": first["value"], "unit": "audio-s/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": first["ms_per_run"], "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "int8+f16" if a.dec_arm == "f16" else "int8+f32",
        "data": "synthetic (seeded random-init weights, seeded synthetic 16 kHz audio with gaps)",
        "config": {"workload": f"fwhip_transcribe over {30 * W} s of audio, greedy, {a.dec_arm} decoder arm",
                   "audio_s": 30.0 * W}, "modes": res}))


def main():
    a = _args()
    if a.gpus != 1:
        print(json.dumps({"error": "bench.py measures one GPU; multi-GPU runs shard windows/streams "
                                   "(data parallel, no exchange) and are not part of this benchmark",
                          "n_gpus": a.gpus}))
        sys.exit(2)
    if a.workload == "copy":
        copy_calibration(a.copy_mb, a.steps)
        return
    if a.workload == "load":
        load_workload(a)
        return
    if a.workload == "transcribe":
        transcribe_workload(a)
        return
    if a.workload == "step":
        step_workload(a)
        return
    if a.workload == "tiny":
        tiny_workload(a)
        return
    from franken_whisper_amd import abi, native, synth

    cfg = synth.TURBO
    W = a.windows or (8 if a.workload == "enc-f32" else 16 if a.workload == "enc-int8" else 10)
    nf = 2 * cfg.n_audio_ctx
    t_setup = time.perf_counter()
    model = synth.Model(cfg, seed=0, encoder=a.workload != "decode", decoder=a.workload in ("job", "decode"))
    ctx = native.Context(0)
    enc = dec = st = None
    frontend = a.workload == "job"
    if frontend:
        # the job starts from audio: W x 30 s of seeded synthetic 16 kHz speech-like
        # audio with silent gaps -> log-mel (128 bins) -> the encoder's 30 s windows
        samples = synth.audio(AUDIO_SEED, 30.0 * W, gaps=True)
        n_samples = samples.size
        samples_dev = ctx.array(samples)
        filters_dev = ctx.array(synth.mel_filterbank(cfg.n_mels))
        mel_frames = native.mel_frames(n_samples)
        mel_dev = ctx.empty((cfg.n_mels, mel_frames), np.float32)
        offsets = np.arange(W, dtype=np.int64) * nf
    else:
        mel = synth.mel_input(1234, W, nf, cfg.n_mels) * np.float32(0.5)
        mel_dev = ctx.array(mel)

    def encode():
        if frontend:
            ctx.log_mel(samples_dev, n_samples, filters_dev, cfg.n_mels, mel_dev)
            enc.forward_mel(mel_dev, mel_frames, offsets, nf, enc_out)
        else:
            enc.forward_time_major(mel_dev, W, nf, enc_out)
    enc_out = ctx.empty((W, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    if a.workload in ("job", "enc-int8"):
        enc = native.Encoder(ctx, model, abi.ENC_INT8)
    elif a.workload == "enc-f32":
        enc = native.Encoder(ctx, model, abi.ENC_F32)
    if enc is not None and a.exact:
        enc.set_exact(True)
    if enc is not None:
        enc.set_tome(a.tome, 3)
    tk = model.tokens
    filt = tk.filter()
    prompt = tk.sot_sequence(language_id=0)
    if a.workload in ("job", "decode"):
        dec = native.Decoder(ctx, model, abi.DEC_INT8 if a.dec_arm == "int8" else abi.DEC_F16)
        if a.exact:
            dec.set_exact(True)
        dec.set_kv_f16(a.kv == "f16")
        st = dec.state(W, cfg.n_audio_ctx)
        if a.workload == "decode":
            enc_out.upload(synth.encoder_states(77, W, cfg.n_audio_ctx, cfg.n_audio_state))
            st.set_cross(enc_out)
    ctx.synchronize()
    t_setup = time.perf_counter() - t_setup

    tokens_out = [0]
    last_tokens = [None]

    def step():
        if enc is not None:
            encode()
        if st is not None:
            if a.workload == "job":
                st.set_cross(enc_out)
            else:
                st.reset()
            toks = st.greedy(prompt, a.tokens, filt)
            tokens_out[0] = sum(len(t) for t in toks)
            last_tokens[0] = toks

    for _ in range(a.warmup):
        step()
    ctx.synchronize()
    # per-component wall times (untimed diagnostic pass)
    comp = {}
    if enc is not None:
        if frontend:
            t = time.perf_counter()
            ctx.log_mel(samples_dev, n_samples, filters_dev, cfg.n_mels, mel_dev)
            ctx.synchronize()
            comp["log_mel_ms"] = (time.perf_counter() - t) * 1e3
            t = time.perf_counter()
            enc.forward_mel(mel_dev, mel_frames, offsets, nf, enc_out)
        else:
            t = time.perf_counter()
            enc.forward_time_major(mel_dev, W, nf, enc_out)
        ctx.synchronize()
        comp["encoder_ms"] = (time.perf_counter() - t) * 1e3
    if st is not None:
        if a.workload == "job":
            t = time.perf_counter()
            st.set_cross(enc_out)
            ctx.synchronize()
            comp["cross_kv_ms"] = (time.perf_counter() - t) * 1e3
        else:
            st.reset()
        t = time.perf_counter()
        toks = st.greedy(prompt, a.tokens, filt)
        ctx.synchronize()
        comp["decode_ms"] = (time.perf_counter() - t) * 1e3
        comp["decode_tokens"] = int(sum(len(x) for x in toks))

    ctx.timing(True)
    ctx.synchronize()
    t0 = time.perf_counter()
    for _ in range(a.steps):
        step()
    ctx.synchronize()
    elapsed = time.perf_counter() - t0
    CLASSES = _classes()
    stats = {k: ctx.kernel_stats(k) for k in CLASSES}
    ctx.timing(False)
    ms_per_step = elapsed * 1e3 / a.steps
    last_tokens_main = last_tokens[0]

    rooflines = []
    for k, (n, ms, units) in stats.items():
        if not n:
            continue
        name, bound, op, tkey = CLASSES[k]
        r = {"kernel": name, "bound": bound, "launches": n, "avg_launch_ms": round(ms / n, 4),
             "total_ms": round(ms, 3)}
        if bound == "mfma":
            ach = units / (ms * 1e-3) / 1e12
            r.update(achieved=round(ach, 2), peak=PEAK_TFLOPS[op], unit="TFLOP/s", op_dtype=op,
                     frac=round(ach / PEAK_TFLOPS[op], 4), traffic=None)
        else:
            ach = units / (ms * 1e-3) / 1e9
            r.update(achieved=round(ach, 1), peak=HBM_PEAK_GBS, unit="GB/s", frac=round(ach / HBM_PEAK_GBS, 4),
                     traffic=None, algorithmic_bytes=round(units / n))
        if tkey == "dec_step":
            tkey = "dec_step_f16" if a.dec_arm == "f16" else "dec_step_int8"
        if tkey and a.workload in ("job", "decode") and W == 10:
            tb, path = measured_traffic(tkey)
            if tb:
                r["traffic"] = tb
                r["traffic_source"] = path + " (rocprofv3 --pmc FETCH_SIZE x2.0 + WRITE_SIZE x1.0)"
        rooflines.append(r)
    rooflines.sort(key=lambda r: -r["total_ms"])
    roof = dict(rooflines[0]) if rooflines else None
    if st is not None:
        xr = xattn_roofline(ctx, st, W, cfg, filt)
        if xr:
            rooflines.append(xr)

    # the int8 decoder arm (the reference's default arm) on the same job:
    # timed the same way, reported beside the headline with its token check
    int8_arm = None
    if a.workload == "job" and a.dec_arm == "f16" and not a.no_verify:
        dec8 = native.Decoder(ctx, model, abi.DEC_INT8)
        st8 = dec8.state(W, cfg.n_audio_ctx)
        toks8 = None
        for i in range(a.warmup + a.steps):
            if i == a.warmup:
                ctx.synchronize()
                t8 = time.perf_counter()
            encode()
            st8.set_cross(enc_out)
            toks8 = st8.greedy(prompt, a.tokens, filt)
        ctx.synchronize()
        ms8 = (time.perf_counter() - t8) * 1e3 / a.steps
        int8_arm = {"value": round(30.0 * W / (ms8 * 1e-3), 2), "ms_per_step": round(ms8, 3), "tokens": toks8}
        st8.close()
        dec8.close()
    # the same job with the reference's shipped large-v3-turbo encoder (ToMe on
    # by default: 500 of 1500 rows merged after block 3, encoder.rs:1264-1337),
    # timed the same way, with its own exact-mode token check
    tome_run = None
    if a.workload == "job" and a.tome == 0 and not a.no_tome_run and not a.no_verify:
        enc.set_tome(-1, 3)
        for i in range(a.warmup + a.steps):
            if i == a.warmup:
                ctx.synchronize()
                tt = time.perf_counter()
            step()
        ctx.synchronize()
        mst = (time.perf_counter() - tt) * 1e3 / a.steps
        tome_run = {"value": round(30.0 * W / (mst * 1e-3), 2), "ms_per_step": round(mst, 3),
                    "tokens": last_tokens[0]}
        t = time.perf_counter()
        encode()
        ctx.synchronize()
        tome_run["encoder_ms"] = round((time.perf_counter() - t) * 1e3, 2)
        enc.set_tome(0, 3)
    # the reference's defaults together: the ToMe encoder above, the int8
    # decoder arm and the f32 self-attention cache (FW_KV_F16 unset), timed the
    # same way, with its own exact-mode token check
    ref_default = None
    if a.workload == "job" and a.tome == 0 and not a.no_tome_run and not a.no_verify:
        enc.set_tome(-1, 3)
        decd = native.Decoder(ctx, model, abi.DEC_INT8)
        decd.set_kv_f16(False)
        std = decd.state(W, cfg.n_audio_ctx)
        toksd = None
        for i in range(a.warmup + a.steps):
            if i == a.warmup:
                ctx.synchronize()
                td = time.perf_counter()
            encode()
            std.set_cross(enc_out)
            toksd = std.greedy(prompt, a.tokens, filt)
        ctx.synchronize()
        msd = (time.perf_counter() - td) * 1e3 / a.steps
        ref_default = {"value": round(30.0 * W / (msd * 1e-3), 2), "ms_per_step": round(msd, 3), "tokens": toksd}
        # the same job in exact mode (bit-identical to the reference's strict
        # mode): one untimed pass for its buffers, one timed
        enc.set_exact(True)
        decd.set_exact(True)
        for i in range(2):
            if i == 1:
                ctx.synchronize()
                td = time.perf_counter()
            encode()
            std.set_cross(enc_out)
            std.greedy(prompt, a.tokens, filt)
        ctx.synchronize()
        mse = (time.perf_counter() - td) * 1e3
        ref_default["exact_mode"] = {"value": round(30.0 * W / (mse * 1e-3), 2), "ms_per_step": round(mse, 3)}
        enc.set_exact(a.exact)
        std.close()
        decd.close()
        enc.set_tome(0, 3)
    verify = None
    if a.workload == "job" and not a.no_verify:
        got = {abi.DEC_F16 if a.dec_arm == "f16" else abi.DEC_INT8: last_tokens_main}
        if int8_arm:
            got[abi.DEC_INT8] = int8_arm.pop("tokens")
        verify = verify_tokens(ctx, model, mel_dev, mel_frames, offsets, nf, W, prompt, a.tokens, filt, got,
                               tome=a.tome)
        if tome_run:
            arm_m = abi.DEC_F16 if a.dec_arm == "f16" else abi.DEC_INT8
            vt = verify_tokens(ctx, model, mel_dev, mel_frames, offsets, nf, W, prompt, a.tokens, filt,
                               {arm_m: tome_run.pop("tokens")}, tome=-1)
            tome_run["tokens_identical_to_exact"] = f"{vt[arm_m][1]}/{W} windows"
            tome_run["note"] = ("the reference's default large-v3-turbo encoder: ToMe merges 500 of 1500 rows per "
                                "window after block 3 (tome_r_for, encoder.rs:1264-1337; not byte-exact against "
                                "the un-merged encoder, WER-certified there); tokens checked against exact mode "
                                "with the same ToMe")
        if ref_default:
            vd = verify_tokens(ctx, model, mel_dev, mel_frames, offsets, nf, W, prompt, a.tokens, filt,
                               {abi.DEC_INT8: ref_default.pop("tokens")}, tome=-1, kv_f16=False)
            ref_default["tokens_identical_to_exact"] = f"{vd[abi.DEC_INT8][1]}/{W} windows"
            ref_default["note"] = ("the reference's default configuration in one job: ToMe (500 of 1500 rows after "
                                   "block 3), the int8 decoder arm and the f32 self-attention cache (FW_KV_F16 "
                                   "unset); fast-mode tokens checked against exact mode with the same settings "
                                   "(the int8 arm re-quantizes every linear's input, so fast mode's sub-ulp "
                                   "differences move tokens); exact_mode: the same job in exact mode, bit-identical "
                                   "to the reference's strict mode")

    audio_s = 30.0 * W
    out = {
        "metric": "audio-s/sec large-v3-turbo encode+greedy decode; enc TFLOP/s; decode tok/s",
        "value": None,
        "unit": "audio-s/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8+f32",
        "data": ("synthetic (seeded random-init weights N(0,0.02), seeded synthetic 16 kHz audio with gaps, "
                 "Slaney mel filterbank)" if frontend else
                 "synthetic (seeded random-init weights N(0,0.02), seeded synthetic log-mel input)"),
        "config": {},
        "roofline": roof,
        "rooflines": rooflines,
    }
    if a.workload == "job":
        out["value"] = round(audio_s / (ms_per_step * 1e-3), 2)
        arm_txt = ("f16 decoder arm (every GEMV f16 in dot_f16c order, f16 cross K/V, tied f16 logits head)"
                   if a.dec_arm == "f16" else "int8 decoder arm")
        out["config"] = {"workload": f"large-v3-turbo whole job: {W} x 30 s windows, int8 encoder "
                                     f"(FW_ENC_ATTN_OUT_I8I32 plan, dense, no ToMe), cross K/V, greedy no-timestamps "
                                     f"decode of {a.tokens} tokens/window (cohort of {W} streams), {arm_txt}, "
                                     f"f16 KV cache; log-mel (128 bins) of {30 * W} s of seeded synthetic 16 kHz audio with "
                                     f"silent gaps computed inside the step", "windows": W, "audio_s": audio_s,
                         "n_frames": nf, "prompt_tokens": len(prompt), "max_tokens": a.tokens,
                         "mode": "exact" if a.exact else "fast"}
        out["dtype"] = "int8+f16" if a.dec_arm == "f16" else "int8+f32"
    elif a.workload.startswith("enc"):
        out["value"] = round(audio_s / (ms_per_step * 1e-3), 2)
        out["dtype"] = "int8+f32" if a.workload == "enc-int8" else "f32 (f16-pair MFMA)"
        out["config"] = {"workload": f"large-v3-turbo encoder only ({a.workload[4:]} plan), {W} x 30 s windows",
                         "windows": W}
    else:
        out["unit"] = "tok/s"
        out["value"] = round(tokens_out[0] / (ms_per_step * 1e-3), 1)
        out["config"] = {"workload": f"large-v3-turbo decoder: {W} streams, prompt + {a.tokens} greedy steps, "
                                     f"{a.dec_arm} arm, {a.kv} KV cache", "streams": W}
    enc_ms = comp.get("encoder_ms")
    out["enc_tflops"] = round(ENC_GOP_PER_WINDOW * W / enc_ms, 1) if enc_ms else None
    if "decode_ms" in comp:
        out["decode_tok_s"] = round(comp["decode_tokens"] / (comp["decode_ms"] * 1e-3), 1)
    out["components_ms"] = {k: round(v, 2) if isinstance(v, float) else v for k, v in comp.items()}
    arm_main = abi.DEC_F16 if a.dec_arm == "f16" else abi.DEC_INT8
    if verify:
        out["tokens_identical_to_exact"] = f"{verify[arm_main][1]}/{W} windows"
        out["tokens_match"] = verify[arm_main][1] == W
    if int8_arm:
        int8_arm["tokens_identical_to_exact"] = f"{verify[abi.DEC_INT8][1]}/{W} windows"
        int8_arm["note"] = ("int8 decoder arm (the reference's default): every linear re-quantizes its input to int8, "
                            "so the sub-ulp f32 reordering of fast mode moves tokens; exact mode is bit-identical")
        out["int8_decoder_arm"] = int8_arm
    if tome_run:
        out["tome_default_job"] = tome_run
    if ref_default:
        out["reference_default_job"] = ref_default
    out["setup_s"] = round(t_setup, 1)
    if a.workload == "job" and not a.no_cpu_baseline:
        cb, cpu_toks = cpu_baseline(model, W, a.tokens, a.cpu_threads, a.cpu_runs, arm_main)
        out["cpu_baseline"] = cb
        out["gpu_over_cpu"] = round(out["value"] / cb["value"], 1)
        g0 = last_tokens_main[0] if last_tokens_main else None
        out["tokens_match_cpu_oracle"] = {
            "window": 0, "identical": bool(g0 is not None and np.array_equal(np.asarray(g0), np.asarray(cpu_toks))),
            "gpu_tokens": int(len(g0)) if g0 is not None else 0, "cpu_tokens": int(len(cpu_toks))}
    for x in (st, dec, enc):
        if x is not None:
            x.close()
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
