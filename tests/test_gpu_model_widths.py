"""The reference's other model widths (mod.rs:703-728: base d 512 with 8 heads,
small 768 / 12, medium 1024 / 16), here with two encoder and two decoder
layers each and the full 1,500-frame audio context, seeded random-init
weights. The kernels dispatch on d (row groups per lane, fused-kernel
eligibility, GEMV lanes per row), so each width takes shapes the tiny and
turbo tests do not.

Checks, per width:
  - exact mode, int8 encoder plan and int8 decoder arm: encoder states bit
    for bit, and the greedy tokens of a 3-stream cohort (each stream with its
    own encoder state) equal the oracle's, stream by stream;
  - exact mode, f32 plan and f16 arm: the same;
  - fast mode, f32 plan: the encoder within 1e-3 relative max-abs of the
    oracle, and the f16 arm's greedy tokens equal the oracle's."""
import os

import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from oracle import oracle as O
from tests.helpers import assert_bitexact, rel_maxabs

pytestmark = pytest.mark.gpu

WIDTHS = [
    synth.Config("base-2L", 51865, 1500, 512, 8, 2, 448, 512, 8, 2, 80),
    synth.Config("small-2L", 51865, 1500, 768, 12, 2, 448, 768, 12, 2, 80),
    synth.Config("medium-2L", 51865, 1500, 1024, 16, 2, 448, 1024, 16, 2, 80),
]
S = 3
N_TOKENS = 24


def _run(ctx, cfg, precision, arm, exact, seed):
    m = synth.Model(cfg, seed=seed)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(seed + 1, S, nf, cfg.n_mels) * np.float32(0.5)
    enc = native.Encoder(ctx, m, precision)
    enc.set_exact(exact)
    out = ctx.empty((S, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
    enc.forward_time_major(ctx.array(x), S, nf, out)
    states = out.download()
    enc.close()
    tk = m.tokens
    dec = native.Decoder(ctx, m, arm)
    dec.set_exact(exact)
    st = dec.state(S, cfg.n_audio_ctx)
    st.set_cross(out)
    toks = st.greedy(tk.sot_sequence(), N_TOKENS, tk.filter())
    st.close()
    dec.close()
    out.free()
    lib = O.lib()
    lib.ref_set_num_threads(min(os.cpu_count() or 1, 16))
    try:
        lib.ref_set_fast(1)
        oenc = O.Encoder(m, precision)
        odec = O.Decoder(m, arm)
        want_states = [oenc.forward(x[s]) for s in range(S)]
        want_toks = [odec.state(want_states[s]).greedy(tk.sot_sequence(), N_TOKENS, tk.filter()) for s in range(S)]
    finally:
        lib.ref_set_fast(0)
    return states, want_states, toks, want_toks


@pytest.mark.parametrize("cfg", WIDTHS, ids=[c.name for c in WIDTHS])
@pytest.mark.parametrize("precision,arm", [(abi.ENC_INT8, abi.DEC_INT8), (abi.ENC_F32, abi.DEC_F16)],
                         ids=["int8", "f32-f16"])
def test_exact_mode_matches_oracle(ctx, cfg, precision, arm):
    print(f"{cfg.name} exact", flush=True)
    states, want_states, toks, want_toks = _run(ctx, cfg, precision, arm, True, seed=21)
    for s in range(S):
        assert_bitexact(states[s], want_states[s], f"{cfg.name} encoder states, stream {s}")
        np.testing.assert_array_equal(toks[s], np.asarray(want_toks[s]), err_msg=f"{cfg.name} stream {s}")
    print(f"{cfg.name}: token counts {[len(t) for t in toks]}", flush=True)


@pytest.mark.parametrize("cfg", WIDTHS, ids=[c.name for c in WIDTHS])
def test_fast_mode_f32_plan_within_tolerance(ctx, cfg):
    print(f"{cfg.name} fast", flush=True)
    states, want_states, toks, want_toks = _run(ctx, cfg, abi.ENC_F32, abi.DEC_F16, False, seed=22)
    for s in range(S):
        err = rel_maxabs(states[s], want_states[s])
        print(f"{cfg.name} stream {s}: encoder rel max-abs {err:.2e}", flush=True)
        assert err < 1e-3
        np.testing.assert_array_equal(toks[s], np.asarray(want_toks[s]), err_msg=f"{cfg.name} stream {s}")
