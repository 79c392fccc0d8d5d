"""Writes tests/golden/ln_order_rows.npz: rows on which the decoder
LayerNorm's fast-mode wave-tree sums give a different f32 output than the
reference's sequential sums (layer_norm, nn.rs:4425-4438), found by the CPU
replay tests/ln_order_replay.c over seeded Gaussian, offset and adversarial
rows of width 1280.  Arrays: x, w, b [n, 1280] f32, y_tree (the output in the
kernels' tree order) [n, 1280] f32, kind [n].  The reference-order output is
the oracle's (ref_layer_norm), computed where the fixture is used.

    python tests/golden/make_ln_order_rows.py
"""
from __future__ import annotations

import os
import subprocess
import sys
import tempfile

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
D = 1280


def main() -> None:
    with tempfile.TemporaryDirectory() as tmp:
        exe = os.path.join(tmp, "lnr")
        subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-fno-fast-math", "-o", exe,
                        os.path.join(HERE, "..", "ln_order_replay.c"), "-lm"], check=True)
        jobs = [(0, 400_000, 11 + i) for i in range(4)] + [(1, 400_000, 21 + i) for i in range(2)] + \
               [(2, 200_000, 31 + i) for i in range(2)]
        procs, dumps, kinds = [], [], []
        for i, (kind, rows, seed) in enumerate(jobs):
            path = os.path.join(tmp, f"dump{i}.bin")
            procs.append(subprocess.Popen([exe, str(kind), str(rows), str(D), str(seed), "0", path],
                                          stdout=subprocess.PIPE, text=True))
            dumps.append(path)
            kinds.append(kind)
        parts, kind_col = [], []
        for p, path, kind in zip(procs, dumps, kinds):
            out, _ = p.communicate()
            assert p.returncode == 0, out
            print(out.strip())
            if os.path.exists(path):
                a = np.fromfile(path, np.float32).reshape(-1, 5, D)
                parts.append(a)
                kind_col += [kind] * a.shape[0]
        a = np.concatenate(parts)
    np.savez_compressed(os.path.join(HERE, "ln_order_rows.npz"), x=a[:, 0], w=a[:, 1], b=a[:, 2],
                        y_tree=a[:, 4], kind=np.array(kind_col, np.int32))
    print(f"{a.shape[0]} rows written", file=sys.stderr)


if __name__ == "__main__":
    main()
