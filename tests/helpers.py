"""Shared fixtures-by-function for the parity tests (seeded models cached per
process)."""
from __future__ import annotations

import functools

import numpy as np

from franken_whisper_amd import synth


@functools.lru_cache(maxsize=None)
def model(name: str, seed: int = 0, encoder: bool = True, decoder: bool = True):
    return synth.Model(synth.CONFIGS[name], seed=seed, encoder=encoder, decoder=decoder)


def enc_states(seed, n_streams, frames, d):
    return synth.encoder_states(seed, n_streams, frames, d)


def bits(a):
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


def assert_bitexact(got, want, what=""):
    g, w = bits(got), bits(want)
    if not np.array_equal(g, w):
        bad = np.flatnonzero(g.ravel() != w.ravel())
        i = bad[0]
        raise AssertionError(
            f"{what}: {bad.size}/{g.size} elements differ; first at {i}: got {np.float32(got.ravel()[i])!r} "
            f"want {np.float32(want.ravel()[i])!r}; max|d|={np.max(np.abs(got.astype(np.float64) - want)):.3e}")


def rel_maxabs(got, want):
    """max|got-want| / max|want| (the 'max-abs relative' tolerance measure)."""
    want = np.asarray(want, np.float64)
    return float(np.max(np.abs(np.asarray(got, np.float64) - want)) / max(np.max(np.abs(want)), 1e-30))
