"""The int8 encoder's two GEMM routes agree bit for bit: the persistent
kernels (default; fc1 written as f16 GELU-table indices with exact side values
for |v| >= 9.98, then the index-form GELU quantizer) and the one-tile-per-block
kernels with f32 fc1 rows (FWHIP_GEMM_I8P=0).  Every epilogue (QKV split with
V^T, residual, f32, index form) computes the same f32 values, so the encoder
outputs must be identical; one case uses a large MLP LayerNorm gain so that the
side-value path runs.  Each route runs in its own process (the route is read
once per process)."""
import os
import subprocess
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


def _run(route, out_dir):
    env = dict(os.environ)
    env["FWHIP_GEMM_I8P"] = route
    r = subprocess.run([sys.executable, "-u", os.path.join(HERE, "enc_path_child.py"), out_dir], env=env,
                       capture_output=True, text=True, timeout=300)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stderr


def test_int8_encoder_gemm_routes_bitexact(tmp_path):
    a, b = tmp_path / "persistent", tmp_path / "tiles"
    a.mkdir()
    b.mkdir()
    _run("1", str(a))
    _run("0", str(b))
    names = sorted(os.listdir(a))
    assert len(names) == 4
    for n in names:
        x, y = np.load(a / n), np.load(b / n)
        diff = int((x.view(np.uint32) != y.view(np.uint32)).sum())
        print(n, "differing elements", diff, flush=True)
        assert diff == 0, n
