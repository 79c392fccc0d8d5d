"""GPU parity of ToMe token merging (tome_merge / tome_unmerge and the
single-shot schedule, encoder.rs:1264-1632) against the oracle:

- the merge step alone (fwhip_tome_merge) bit for bit — merged rows and the
  unmerge map — from tiny shapes with tie-heavy rows up to large-v3-turbo's
  1500 x 1280 windows with the reference's default r = 500, two windows at once;
- the encoder with ToMe in exact mode bit-identical to the oracle's forward
  with the same FW_TOME_R / FW_TOME_LAYER: a 3-block micro model, tiny-2L and
  all 32 large-v3-turbo blocks on the int8 plan with the reference's default
  rule (fwhip_encoder_set_tome(-1): 500 rows after block 3);
- fast mode with ToMe (MFMA attention feeding the merge): every row the
  oracle's within the fast mode's tolerance except where a near-tie merge
  decision flips, which the test reports;
- the progressive schedule (FW_TOME_EVERY / FW_TOME_FLOOR, encoder.rs:1379-1402):
  two and three merges (the merged rows alternate between two buffers, so both
  parities of the final unmerge's source are covered), a floor that stops a
  merge, both plans, exact mode bit-identical to the oracle; on large-v3-turbo
  the reference's default rule with a 4-block cadence (the full-window test
  looks at the window before its first merge, so the second merge runs)."""
import numpy as np
import pytest

from franken_whisper_amd import abi, native, synth
from oracle import oracle as O
from tests.helpers import assert_bitexact, rel_maxabs

pytestmark = pytest.mark.gpu

TOME_MICRO = synth.Config("tome-micro", 51864, 400, 128, 2, 3, 64, 128, 2, 2, 16)
TINY2 = synth.Config("tiny-2L", 51864, 1500, 384, 6, 2, 448, 384, 6, 4, 80)

MERGE_CASES = [(1, 9, 32, 3), (3, 31, 64, 7), (2, 400, 128, 150), (1, 1501, 64, 600), (2, 1500, 1280, 500)]


@pytest.mark.parametrize("nw,T,d,r", MERGE_CASES)
def test_tome_merge_bitexact(ctx, nw, T, d, r):
    rng = np.random.default_rng(T + d)
    x = rng.standard_normal((nw, T, d)).astype(np.float32)
    print(f"tome_merge windows {nw} T {T} d {d} r {r}", flush=True)
    merged, umap = ctx.tome_merge(ctx.array(x), r)
    for w in range(nw):
        want, wmap = O.tome_merge(x[w], r)
        np.testing.assert_array_equal(umap[w], wmap, err_msg=f"window {w} umap")
        assert_bitexact(merged[w], want, f"window {w} merged rows")


def test_tome_merge_ties_bitexact(ctx):
    """Rows drawn from 4 vectors: exactly equal similarities everywhere, so the
    first-index edge and the stable ranking decide every merge."""
    rng = np.random.default_rng(3)
    basis = rng.standard_normal((4, 64)).astype(np.float32)
    x = basis[rng.integers(0, 4, (2, 300))]
    merged, umap = ctx.tome_merge(ctx.array(x), 120)
    for w in range(2):
        want, wmap = O.tome_merge(x[w], 120)
        np.testing.assert_array_equal(umap[w], wmap)
        assert_bitexact(merged[w], want, f"window {w}")


def _encode(ctx, m, precision, x, r, after, exact, every=0, floor=128):
    cfg = m.cfg
    nw, nf = x.shape[0], x.shape[1]
    enc = native.Encoder(ctx, m, precision)
    enc.set_exact(exact)
    enc.set_tome(r, after)
    enc.set_tome_schedule(every, floor)
    out = ctx.empty((nw, nf // 2, cfg.n_audio_state), np.float32)
    enc.forward_time_major(ctx.array(x), nw, nf, out)
    got = out.download()
    enc.close()
    return got


EXACT_CASES = [(TOME_MICRO, abi.ENC_F32, 150, 1), (TOME_MICRO, abi.ENC_INT8, 150, 1), (TINY2, abi.ENC_F32, 500, 0),
               (TINY2, abi.ENC_INT8, 500, 0)]


@pytest.mark.parametrize("cfg,prec,r,after", EXACT_CASES,
                         ids=[f"{c.name}-{'int8' if p == abi.ENC_INT8 else 'f32'}" for c, p, _, _ in EXACT_CASES])
def test_encoder_tome_exact_bitexact(ctx, cfg, prec, r, after):
    m = synth.Model(cfg, seed=4, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(5, 2, nf, cfg.n_mels)
    print(f"{cfg.name} ToMe r={r} after {after} exact", flush=True)
    got = _encode(ctx, m, prec, x, r, after, True)
    oe = O.Encoder(m, prec)
    for w in range(2):
        assert_bitexact(got[w], oe.forward(x[w], tome_r=r, tome_after=after), f"{cfg.name} window {w}")


def test_turbo_int8_encoder_tome_default_exact_bitexact(ctx):
    """The reference's shipped large-v3-turbo encoder (ToMe on by default: 500
    rows merged after block 3), all 32 blocks, exact mode, one window."""
    cfg = synth.TURBO
    m = synth.Model(cfg, seed=6, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(7, 1, nf, cfg.n_mels) * np.float32(0.5)
    print("turbo int8 exact, 32 layers, ToMe default", flush=True)
    got = _encode(ctx, m, abi.ENC_INT8, x, -1, 3, True)
    assert_bitexact(got[0], O.Encoder(m, abi.ENC_INT8).forward(x[0], tome_r=500, tome_after=3),
                    "turbo int8 exact + ToMe")


def test_tome_default_rule_skips_small_models(ctx):
    """tome_r_for: the default merges only on the 20-head large class; a small
    model with r < 0 is the un-merged encoder bit for bit."""
    cfg = TOME_MICRO
    m = synth.Model(cfg, seed=4, decoder=False)
    x = synth.mel_input(5, 1, 2 * cfg.n_audio_ctx, cfg.n_mels)
    a = _encode(ctx, m, abi.ENC_F32, x, -1, 3, True)
    assert_bitexact(a[0], O.Encoder(m, abi.ENC_F32).forward(x[0]), "default rule, 2-head model")


@pytest.mark.parametrize("cfg,r,after", [(TOME_MICRO, 150, 1), (TINY2, 500, 0)], ids=lambda v: getattr(v, "name", str(v)))
def test_encoder_tome_fast_mode(ctx, cfg, r, after):
    m = synth.Model(cfg, seed=4, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(5, 1, nf, cfg.n_mels)
    got = _encode(ctx, m, abi.ENC_F32, x, r, after, False)[0]
    want = O.Encoder(m, abi.ENC_F32).forward(x[0], tome_r=r, tome_after=after)
    scale = np.max(np.abs(want))
    row_err = np.max(np.abs(got.astype(np.float64) - want), axis=1) / scale
    bad = int(np.sum(row_err > 1e-3))
    print(f"{cfg.name} fast ToMe: max-abs {rel_maxabs(got, want):.2e}, rows beyond 1e-3: {bad}/{row_err.size}",
          flush=True)
    # a flipped near-tie decision moves a handful of rows (a merged pair and
    # its partner), never the rest
    assert bad <= max(4, row_err.size // 100)


# (cfg, precision, r, after, every, floor, merges), seed-5 inputs
PROG_CASES = [(TOME_MICRO, abi.ENC_F32, 50, 0, 1, 128, 3), (TOME_MICRO, abi.ENC_INT8, 50, 0, 1, 128, 3),
              (TOME_MICRO, abi.ENC_F32, 60, 0, 1, 250, 2), (TOME_MICRO, abi.ENC_INT8, 60, 0, 2, 128, 2),
              (TINY2, abi.ENC_INT8, 300, 0, 1, 128, 2)]


@pytest.mark.parametrize("cfg,prec,r,after,every,floor,merges", PROG_CASES,
                         ids=[f"{c.name}-{'int8' if p == abi.ENC_INT8 else 'f32'}-r{r}-e{e}-f{f}"
                              for c, p, r, _, e, f, _ in PROG_CASES])
def test_encoder_tome_progressive_exact_bitexact(ctx, cfg, prec, r, after, every, floor, merges):
    m = synth.Model(cfg, seed=4, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(5, 2, nf, cfg.n_mels)
    print(f"{cfg.name} progressive ToMe r={r} every={every} floor={floor} exact", flush=True)
    got = _encode(ctx, m, prec, x, r, after, True, every, floor)
    oe = O.Encoder(m, prec)
    for w in range(2):
        want = oe.forward(x[w], tome_r=r, tome_after=after, tome_every=every, tome_floor=floor)
        assert np.unique(want, axis=0).shape[0] == cfg.n_audio_ctx - merges * r
        assert_bitexact(got[w], want, f"{cfg.name} window {w}")


def test_turbo_int8_encoder_tome_progressive_default_rule_exact(ctx):
    """large-v3-turbo, int8 plan, exact mode, all 32 blocks: the default rule
    (500 rows after block 3) with a 4-block cadence merges after blocks 3 and 7
    (1500 -> 1000 -> 500; a third merge would leave 0 < 128 rows)."""
    cfg = synth.TURBO
    m = synth.Model(cfg, seed=6, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(7, 1, nf, cfg.n_mels) * np.float32(0.5)
    print("turbo int8 exact, 32 layers, ToMe default rule every 4", flush=True)
    got = _encode(ctx, m, abi.ENC_INT8, x, -1, 3, True, 4, 128)
    lib = O.lib()
    lib.ref_set_fast(1)
    try:
        want = O.Encoder(m, abi.ENC_INT8).forward(x[0], tome_r=500, tome_after=3, tome_every=4, tome_floor=128)
    finally:
        lib.ref_set_fast(0)
    assert np.unique(want, axis=0).shape[0] == 500
    assert_bitexact(got[0], want, "turbo int8 exact + progressive ToMe")


def test_encoder_tome_progressive_fast_mode(ctx):
    cfg, r = TOME_MICRO, 50
    m = synth.Model(cfg, seed=4, decoder=False)
    nf = 2 * cfg.n_audio_ctx
    x = synth.mel_input(5, 1, nf, cfg.n_mels)
    got = _encode(ctx, m, abi.ENC_F32, x, r, 0, False, 1, 128)[0]
    want = O.Encoder(m, abi.ENC_F32).forward(x[0], tome_r=r, tome_after=0, tome_every=1, tome_floor=128)
    scale = np.max(np.abs(want))
    row_err = np.max(np.abs(got.astype(np.float64) - want), axis=1) / scale
    bad = int(np.sum(row_err > 1e-3))
    print(f"{cfg.name} fast progressive ToMe: max-abs {rel_maxabs(got, want):.2e}, rows beyond 1e-3: "
          f"{bad}/{row_err.size}", flush=True)
    assert bad <= max(4, row_err.size // 100)


def test_tome_schedule_rejects_negative_values(ctx):
    m = synth.Model(TOME_MICRO, seed=4, decoder=False)
    enc = native.Encoder(ctx, m, abi.ENC_F32)
    for every, floor in ((-1, 128), (0, -1)):
        with pytest.raises(native.FwhipError) as e:
            enc.set_tome_schedule(every, floor)
        assert e.value.code == abi.ERR_INVALID
    enc.close()
