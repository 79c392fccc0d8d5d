"""Child process of test_gpu_encoder_paths: runs the int8 fast-mode encoder on
seeded synthetic inputs and saves the outputs (.npy) to the directory given.
The GEMM route is whatever FWHIP_GEMM_I8P in the environment selects."""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

from franken_whisper_amd import abi, native, synth  # noqa: E402

TURBO2 = synth.Config("turbo-2L", 51866, 1500, 1280, 20, 2, 448, 1280, 20, 4, 128)
TINY2 = synth.Config("tiny-2L", 51864, 1500, 384, 6, 2, 448, 384, 6, 4, 80)


def main(out_dir):
    ctx = native.Context(0)
    cases = ((synth.MICRO, 3, 1.0), (TINY2, 3, 1.0), (TURBO2, 3, 1.0), (TURBO2, 2, 15.0))
    for cfg, nw, gain in cases:
        m = synth.Model(cfg, seed=2, decoder=False)
        # a large MLP LayerNorm gain puts many fc1 values beyond +-10
        for i in range(cfg.n_audio_layer):
            m.t[f"encoder.blocks.{i}.mlp_ln.weight"][:] = gain
        nf = 2 * cfg.n_audio_ctx
        x = synth.mel_input(3, nw, nf, cfg.n_mels)
        enc = native.Encoder(ctx, m, abi.ENC_INT8)
        out = ctx.empty((nw, cfg.n_audio_ctx, cfg.n_audio_state), np.float32)
        enc.forward_time_major(ctx.array(x), nw, nf, out)
        np.save(os.path.join(out_dir, f"{cfg.name}_g{int(gain)}.npy"), out.download())
        print(cfg.name, gain, "done", flush=True)
        enc.close()
    ctx.close()


if __name__ == "__main__":
    main(sys.argv[1])
