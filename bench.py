"""Benchmark of the hot path on one MI355X.

Default workload (the whole job the headline metric is quoted on): large-v3-turbo
architecture with seeded random-init weights, 300 s of seeded synthetic 16 kHz
audio with silent gaps -> GPU log-mel (128 bins, Slaney filterbank; 33,000
frames) -> 10 windows x 30 s (3000 frames each, offsets 0, 3000, ...), int8 encoder plan
(FW_ENC_ATTN_OUT_I8I32: i7 q/k/v/fc1/fc2, i8 attn.out), cross K/V precompute,
then greedy no-timestamps decode of every window as one cohort with the int8
decoder arm and the f16 KV cache: 4-token prompt + 220 sampled tokens.
One step = that whole job.  Prints one JSON line.

  python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload job|enc-f32|enc-int8|decode]
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


def _args():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=3)
    p.add_argument("--warmup", type=int, default=1)
    p.add_argument("--workload", default="job", choices=["job", "enc-f32", "enc-int8", "decode", "copy"])
    p.add_argument("--windows", type=int, default=None)
    p.add_argument("--tokens", type=int, default=220)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "16")))
    p.add_argument("--cpu-windows", type=int, default=2, help="windows of the job the CPU baseline runs")
    p.add_argument("--copy-mb", type=int, default=512)
    return p.parse_args()


def cpu_baseline(model, n_windows, n_tokens, threads, sample_windows):
    """The oracle (C restatement of the reference CPU path, OpenMP) on a bounded
    sample of the same job: `sample_windows` of the job's windows run end to end
    (int8-plan encoder over all layers, cross K/V precompute, prompt prefill and
    greedy decode of n_tokens), timed, and scaled to audio-seconds per second."""
    from franken_whisper_amd import abi, synth
    from oracle import oracle as O

    O.lib().ref_set_num_threads(threads)
    cfg = model.cfg
    e = O.Encoder(model, abi.ENC_INT8)
    d = O.Decoder(model, abi.DEC_INT8)
    tk = model.tokens
    filt = tk.filter()
    prompt = tk.sot_sequence(language_id=0)
    nf = 2 * cfg.n_audio_ctx
    samples = synth.audio(AUDIO_SEED, 30.0 * n_windows, gaps=True)
    filters = synth.mel_filterbank(cfg.n_mels)
    t0 = time.perf_counter()
    full = O.log_mel(samples, filters)
    t_mel = (time.perf_counter() - t0) * sample_windows / n_windows
    t_enc = t_dec = 0.0
    n_tok = 0
    for w in range(sample_windows):
        t0 = time.perf_counter()
        y = e.forward(np.ascontiguousarray(full[:, w * nf:(w + 1) * nf].T))
        t1 = time.perf_counter()
        toks = d.state(y).greedy(prompt, n_tokens, filt)
        t2 = time.perf_counter()
        t_enc += t1 - t0
        t_dec += t2 - t1
        n_tok += len(toks)
    total = t_mel + t_enc + t_dec
    return {
        "value": round(sample_windows * 30.0 / total, 4),
        "unit": "audio-s/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"oracle (C restatement of the reference CPU path, -O3 -march=x86-64-v3, {threads} OpenMP "
                   f"threads) on {sample_windows} of the job's {n_windows} windows end to end: log-mel "
                   f"{t_mel / sample_windows:.3f} s/window (share of the whole job's log-mel), int8-plan encoder "
                   f"{t_enc / sample_windows:.2f} s/window, cross K/V + prefill + greedy decode "
                   f"{t_dec / sample_windows:.2f} s/window ({n_tok} tokens); {total:.1f} s of CPU work"),
    }


AUDIO_SEED = 1234


TRAFFIC_FILE = "profiles/k_gemm_pi8_int8_encoder_job.md"


def measured_traffic():
    """HBM bytes per int8 encoder GEMM dispatch on this job's shapes, as measured
    with rocprofv3 counters and recorded in TRAFFIC_FILE (the counters cannot be
    read from inside a timed run)."""
    import re

    try:
        with open(os.path.join(ROOT, TRAFFIC_FILE)) as f:
            m = re.search(r"^traffic_bytes_per_launch:\s*(\d+)", f.read(), re.M)
        return int(m.group(1)) if m else None
    except OSError:
        return None


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


def main():
    a = _args()
    if a.gpus != 1:
        print(json.dumps({"error": "this build runs on one GPU; multi-GPU runs shard windows/streams "
                                   "(data parallel, no exchange) and are not part of this benchmark",
                          "n_gpus": a.gpus}))
        sys.exit(2)
    if a.workload == "copy":
        copy_calibration(a.copy_mb, a.steps)
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
    tk = model.tokens
    filt = tk.filter()
    prompt = tk.sot_sequence(language_id=0)
    if a.workload in ("job", "decode"):
        dec = native.Decoder(ctx, model, abi.DEC_INT8)
        st = dec.state(W, cfg.n_audio_ctx)
        if a.workload == "decode":
            enc_out.upload(synth.encoder_states(77, W, cfg.n_audio_ctx, cfg.n_audio_state))
            st.set_cross(enc_out)
    ctx.synchronize()
    t_setup = time.perf_counter() - t_setup

    tokens_out = [0]

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
    stats = {k: ctx.kernel_stats(k) for k in (abi.K_ENC_GEMM_I8, abi.K_ENC_GEMM_F32, abi.K_ENC_ATTN,
                                              abi.K_DEC_LOGITS)}
    ctx.timing(False)
    ms_per_step = elapsed * 1e3 / a.steps

    names = {abi.K_ENC_GEMM_I8: ("encoder int8 GEMM (k_gemm_pi8, persistent int8 tiles)", "mfma", "int8"),
             abi.K_ENC_GEMM_F32: ("encoder f16-pair GEMM (k_gemm2, f16-pair tiles)", "mfma", "f16"),
             abi.K_ENC_ATTN: ("encoder attention (k_attention2, f16 pairs)", "mfma", "f16"),
             abi.K_DEC_LOGITS: ("decoder logits GEMV (k_gemv_i8m)", "hbm", None)}
    kclass = max(stats, key=lambda k: stats[k][1])
    n, ms, units = stats[kclass]
    name, bound, op = names[kclass]
    if bound == "mfma":
        achieved = units / (ms * 1e-3) / 1e12
        roof = {"kernel": name, "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_TFLOPS[op],
                "unit": "TFLOP/s", "op_dtype": op, "frac": round(achieved / PEAK_TFLOPS[op], 4), "traffic": None,
                "launches": n, "avg_launch_ms": round(ms / max(n, 1), 4)}
    else:
        achieved = units / (ms * 1e-3) / 1e9
        roof = {"kernel": name, "bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None, "launches": n,
                "avg_launch_ms": round(ms / max(n, 1), 4)}
    kernel_classes = {names[k][0]: {"launches": v[0], "total_ms": round(v[1], 3)} for k, v in stats.items() if v[0]}
    if kclass == abi.K_ENC_GEMM_I8 and a.workload == "job" and W == 10:
        tb = measured_traffic()
        if tb:
            roof["traffic"] = tb
            roof["traffic_source"] = TRAFFIC_FILE + " (rocprofv3 --pmc FETCH_SIZE x2.0 + WRITE_SIZE x1.0, per dispatch)"

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
    }
    if a.workload == "job":
        out["value"] = round(audio_s / (ms_per_step * 1e-3), 2)
        out["config"] = {"workload": f"large-v3-turbo whole job: {W} x 30 s windows, int8 encoder "
                                     f"(FW_ENC_ATTN_OUT_I8I32 plan, dense, no ToMe), cross K/V, greedy no-timestamps "
                                     f"decode of {a.tokens} tokens/window (cohort of {W} streams), int8 decoder arm, "
                                     f"f16 KV cache; log-mel (128 bins) of {30 * W} s of seeded synthetic 16 kHz audio with "
                                     f"silent gaps computed inside the step", "windows": W, "audio_s": audio_s,
                         "n_frames": nf, "prompt_tokens": len(prompt), "max_tokens": a.tokens}
    elif a.workload.startswith("enc"):
        out["value"] = round(audio_s / (ms_per_step * 1e-3), 2)
        out["dtype"] = "int8+f32" if a.workload == "enc-int8" else "f32 (f16-pair MFMA)"
        out["config"] = {"workload": f"large-v3-turbo encoder only ({a.workload[4:]} plan), {W} x 30 s windows",
                         "windows": W}
    else:
        out["unit"] = "tok/s"
        out["value"] = round(tokens_out[0] / (ms_per_step * 1e-3), 1)
        out["config"] = {"workload": f"large-v3-turbo decoder: {W} streams, prompt + {a.tokens} greedy steps, "
                                     f"int8 arm, f16 KV cache", "streams": W}
    enc_ms = comp.get("encoder_ms")
    out["enc_tflops"] = round(ENC_GOP_PER_WINDOW * W / enc_ms, 1) if enc_ms else None
    if "decode_ms" in comp:
        out["decode_tok_s"] = round(comp["decode_tokens"] / (comp["decode_ms"] * 1e-3), 1)
    out["components_ms"] = {k: round(v, 2) if isinstance(v, float) else v for k, v in comp.items()}
    out["kernel_classes"] = kernel_classes
    out["setup_s"] = round(t_setup, 1)
    if a.workload == "job" and not a.no_cpu_baseline:
        cb = cpu_baseline(model, W, a.tokens, a.cpu_threads, a.cpu_windows)
        out["cpu_baseline"] = cb
        out["gpu_over_cpu"] = round(out["value"] / cb["value"], 1)
    for x in (st, dec, enc):
        if x is not None:
            x.close()
    ctx.close()
    print(json.dumps(out))


if __name__ == "__main__":
    main()
