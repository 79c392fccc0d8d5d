"""The C-ABI library loads without a GPU and exports every entry point
include/fwhip.h declares, and the Python binding declares a signature for each
(no compute calls here)."""
import ctypes as C
import os
import re

from franken_whisper_amd import native

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    src = open(os.path.join(ROOT, "include", "fwhip.h")).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(fwhip_[a-z0-9_]+)\s*\(", src)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("fwhip_init", "fwhip_encoder_load", "fwhip_encoder_forward", "fwhip_decoder_load",
                 "fwhip_dstate_set_cross", "fwhip_decoder_step", "fwhip_decode_greedy"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(native.LIB_PATH)
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_covers_every_declared_symbol():
    assert set(declared_functions()) <= set(native.SIGNATURES), set(declared_functions()) - set(native.SIGNATURES)
    native.lib()  # signatures apply cleanly


def test_abi_version():
    assert native.lib().fwhip_abi_version() == 2


def test_init_without_gpu_names_the_cpu_route():
    """No gfx950 device: fwhip_init returns FWHIP_ERR_UNSUPPORTED with a
    `cpu:<reason>` message, so the caller falls back to its CPU route and records
    why (the pattern of encoder.rs:1700-1725)."""
    import pytest

    from franken_whisper_amd import abi

    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU driver is present; this checks the no-device route")
    h = C.c_void_p()
    rc = native.lib().fwhip_init(0, C.byref(h))
    assert rc == abi.ERR_UNSUPPORTED
    assert not h.value
    assert native.lib().fwhip_last_error().decode().startswith("cpu:")
    with __import__("pytest").raises(native.FwhipError) as e:
        native.Context(0)
    assert e.value.code == abi.ERR_UNSUPPORTED


def test_missing_library_fails_loudly(tmp_path):
    """Without the built HIP library the binding raises at its first use and
    names the build step; nothing falls back to another route."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    env = dict(os.environ)
    env["FWHIP_LIB"] = str(tmp_path / "libfwhip.so")  # does not exist
    code = ("from franken_whisper_amd import native\n"
            "try:\n"
            "    native.Context(0)\n"
            "except RuntimeError as e:\n"
            "    print('RAISED', e)\n")
    r = subprocess.run([sys.executable, "-c", code], cwd=root, env=env, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    assert "RAISED" in r.stdout and "missing" in r.stdout and "build" in r.stdout, r.stdout
