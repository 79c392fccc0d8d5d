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
    assert native.lib().fwhip_abi_version() == 1
