"""fwhip_log_mel_noalloc (the log-mel with the library's static device
scratch, no allocation) against fwhip_log_mel, bit for bit, on two calls in a
row, the second smaller than the first; inputs past the scratch's limit are
rejected before anything is launched."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth

pytestmark = pytest.mark.gpu


def test_log_mel_noalloc_matches_log_mel(ctx):
    fb = ctx.array(synth.mel_filterbank(128))
    for seed, seconds in ((3, 300.0), (4, 7.3)):
        pcm = synth.audio(seed, seconds, gaps=True)
        nf = native.mel_frames(pcm.size)
        print(f"log-mel noalloc, {seconds} s ({nf} frames)", flush=True)
        dev = ctx.array(pcm)
        a, b = ctx.empty((128, nf), np.float32), ctx.empty((128, nf), np.float32)
        ctx.log_mel(dev, pcm.size, fb, 128, a)
        ctx.log_mel_noalloc(dev, pcm.size, fb, 128, b)
        ctx.synchronize()
        assert np.array_equal(a.download().view(np.uint32), b.download().view(np.uint32))
        for x in (a, b, dev):
            x.free()
    # 80 bins and no samples at all (a window of pure padding)
    fb80 = ctx.array(synth.mel_filterbank(80))
    nf = native.mel_frames(0)
    a, b = ctx.empty((80, nf), np.float32), ctx.empty((80, nf), np.float32)
    ctx.log_mel(None, 0, fb80, 80, a)
    ctx.log_mel_noalloc(None, 0, fb80, 80, b)
    ctx.synchronize()
    assert np.array_equal(a.download().view(np.uint32), b.download().view(np.uint32))


def test_log_mel_noalloc_rejects_inputs_past_its_scratch(ctx):
    fb = ctx.array(synth.mel_filterbank(128))
    tiny = ctx.array(np.zeros(16, np.float32))
    out = ctx.empty((128, 1), np.float32)
    with pytest.raises(native.FwhipError) as e:
        ctx.log_mel_noalloc(tiny, 200_000_000, fb, 128, out)
    assert e.value.code == abi.ERR_INVALID
    assert "scratch" in str(e.value)
