"""The oracle's ToMe token merge (ref_tome_merge / ref_encoder_forward_tome,
restating tome_merge / tome_unmerge / the single-shot schedule of
forward_time_major, encoder.rs:1403-1517 and 1590-1632) pinned three ways:

- bit for bit against a float32 loop restatement written here from the
  algorithm (strict ascending-k dot products, sequential sums of squares, the
  first strict maximum, a stable descending sort), on small shapes including
  tie-heavy inputs where the tie rules decide the result;
- by closed forms: r = 0 is a pure reordering whose unmerge is the identity;
  identical rows all merge into B row 0 in ascending A order;
- the encoder with ToMe against the independent float64 textbook Whisper
  (tests/textbook.py), with the merge decisions required to be the same and
  planted mistakes (no averaging, merging the least similar rows, ranking by
  the raw dot product) shown to fail the comparison.

CPU only."""
import numpy as np
import pytest

from franken_whisper_amd import abi, synth
from oracle import oracle as O
from tests import textbook as TB
from tests.helpers import rel_maxabs

F = np.float32


def tome_f32(x, r):
    """tome_merge in float32 with the reference's order of operations."""
    x = np.asarray(x, F)
    seq, d = x.shape
    n_a, n_b = (seq + 1) // 2, seq // 2
    r = min(r, n_a, max(seq - 1, 0))
    A, B = x[0::2], x[1::2]

    def dot(u, v):
        acc = F(0.0)
        for k in range(d):
            acc = F(acc + F(u[k] * v[k]))
        return acc

    def norm(u):
        s = F(0.0)
        for k in range(d):
            s = F(s + F(u[k] * u[k]))
        s = np.sqrt(s, dtype=F)
        return s if s > F(1e-9) else F(1e-9)

    na = [norm(A[a]) for a in range(n_a)]
    nb = [norm(B[b]) for b in range(n_b)]
    best_b, best = [], []
    for a in range(n_a):
        bb, bs = 0, F(-np.inf)
        for b in range(n_b):
            c = F(dot(A[a], B[b]) / F(na[a] * nb[b]))
            if c > bs:
                bb, bs = b, c
        best_b.append(bb)
        best.append(bs)
    order = sorted(range(n_a), key=lambda a: -best[a])  # stable: ties keep ascending a
    chosen = set(order[:r])
    merged = [B[b].copy() for b in range(n_b)]
    count = [1] * n_b
    for a in range(n_a):
        if a in chosen:
            merged[best_b[a]] = (merged[best_b[a]] + A[a]).astype(F)
            count[best_b[a]] += 1
    for b in range(n_b):
        if count[b] > 1:
            merged[b] = (merged[b] / F(count[b])).astype(F)
    umap = np.zeros(seq, np.int32)
    umap[1::2] = np.arange(n_b)
    kept = []
    for a in range(n_a):
        if a in chosen:
            umap[2 * a] = best_b[a]
        else:
            umap[2 * a] = n_b + len(kept)
            kept.append(A[a])
    out = np.array(merged + kept, F).reshape(seq - r, d)
    return out, umap


def _same(a, b):
    return a.shape == b.shape and np.array_equal(np.asarray(a, F).view(np.uint32), np.asarray(b, F).view(np.uint32))


CASES = [(2, 4, 1), (3, 4, 1), (9, 8, 3), (10, 16, 5), (31, 16, 7), (32, 64, 16), (40, 8, 19), (17, 32, 100)]


@pytest.mark.parametrize("seq,d,r", CASES)
def test_tome_merge_bitexact_against_f32_restatement(seq, d, r):
    rng = np.random.default_rng(seq * 131 + d)
    x = rng.standard_normal((seq, d)).astype(F)
    got, gmap = O.tome_merge(x, r)
    want, wmap = tome_f32(x, r)
    assert _same(got, want)
    assert np.array_equal(gmap, wmap)
    np.testing.assert_array_equal(O.tome_unmerge(got, gmap), got[gmap])


def test_tome_ties_take_the_first_edge_and_the_lower_a():
    """Rows drawn from 3 distinct vectors: many exactly equal similarities, so
    both the first-index argmax and the stable sort decide the merge."""
    rng = np.random.default_rng(7)
    basis = rng.standard_normal((3, 16)).astype(F)
    x = basis[rng.integers(0, 3, 24)]
    for r in (1, 5, 12):
        got, gmap = O.tome_merge(x, r)
        want, wmap = tome_f32(x, r)
        assert _same(got, want) and np.array_equal(gmap, wmap), r


def test_tome_identical_rows_merge_into_b0_in_order():
    x = np.tile(np.linspace(-1.0, 2.0, 8, dtype=F), (12, 1))
    r = 4
    merged, umap = O.tome_merge(x, r)
    # every A row ties every B row and every other A row: the first four A rows
    # merge, each into B row 0, and B row 0 becomes (x + x + x + x + x) / 5
    assert merged.shape == (12 - r, 8)
    assert list(umap[0:8:2]) == [0, 0, 0, 0] and list(umap[8::2]) == [6, 7]
    acc = x[1].copy()
    for _ in range(r):
        acc = (acc + x[0]).astype(F)
    np.testing.assert_array_equal(merged[0], (acc / F(r + 1)).astype(F))
    np.testing.assert_array_equal(merged[1:6], x[1:6])


@pytest.mark.parametrize("seq", [2, 9, 50])
def test_tome_r0_is_a_reordering_and_unmerge_restores(seq):
    x = np.random.default_rng(seq).standard_normal((seq, 12)).astype(F)
    merged, umap = O.tome_merge(x, 0)
    assert merged.shape == x.shape
    np.testing.assert_array_equal(merged[: seq // 2], x[1::2])
    np.testing.assert_array_equal(merged[seq // 2:], x[0::2])
    np.testing.assert_array_equal(O.tome_unmerge(merged, umap), x)


# ---- the encoder with ToMe against the float64 textbook -------------------------
TOME_MICRO = synth.Config("tome-micro", 51864, 400, 128, 2, 3, 64, 128, 2, 2, 16)
TINY2 = synth.Config("tiny-2L", 51864, 1500, 384, 6, 2, 448, 384, 6, 4, 80)
TOME_CASES = [(TOME_MICRO, 150, 1), (TINY2, 500, 0)]
_cache = {}


def _case(cfg, r, after):
    key = (cfg.name, r, after)
    if key not in _cache:
        m = synth.Model(cfg, seed=4, decoder=False)
        x = synth.mel_input(5, 1, 2 * cfg.n_audio_ctx, cfg.n_mels)[0]
        want = O.Encoder(m, abi.ENC_F32).forward(x, tome_r=r, tome_after=after)
        _cache[key] = (m, x, want)
    return _cache[key]


@pytest.mark.parametrize("cfg,r,after", TOME_CASES, ids=lambda v: getattr(v, "name", str(v)))
def test_encoder_tome_matches_textbook(cfg, r, after):
    m, x, want = _case(cfg, r, after)
    info = {}
    tb = TB.Encoder(m).forward(x, tome_r=r, tome_after=after, info=info)
    # the float32 oracle can only make the float64 model's decisions when no
    # decision sits on a near-tie
    print(f"{cfg.name}: rank margin {info['rank_margin']:.3e}, edge margin {info['edge_margin']:.3e}")
    assert info["rank_margin"] > 1e-5 and info["edge_margin"] > 1e-5
    e = rel_maxabs(want, tb)
    print(f"{cfg.name} ToMe r={r} after block {after}: max-abs {e:.2e}")
    assert e <= 1e-3
    # without the merge the outputs differ well beyond that bound
    dense = O.Encoder(m, abi.ENC_F32).forward(x)
    assert rel_maxabs(dense, want) > 1e-2


@pytest.mark.parametrize("mutation", ["tome_no_average", "tome_merge_lowest", "tome_dot_not_cos"])
def test_tome_planted_mistakes_are_detected(mutation):
    cfg, r, after = TOME_CASES[0]
    m, x, want = _case(cfg, r, after)
    bad = TB.Encoder(m, TB.Numerics(mutate=mutation)).forward(x, tome_r=r, tome_after=after)
    e = rel_maxabs(want, bad)
    print(f"{mutation}: max-abs {e:.2e}")
    assert e > 1e-2


# ---- the progressive schedule (FW_TOME_EVERY / FW_TOME_FLOOR, encoder.rs:1379-1402, 1590-1632)
# (cfg, r, after, every, floor, merges): TOME_MICRO has 400 rows and 3 blocks
# (seed-5 input: every merge decision at least 1e-5 from a tie)
PROG_CASES = [(TOME_MICRO, 50, 0, 1, 128, 3),   # after blocks 0, 1, 2: 400 -> 350 -> 300 -> 250
              (TOME_MICRO, 60, 0, 1, 250, 2),   # the floor stops the third merge (220 < 250)
              (TOME_MICRO, 60, 0, 2, 128, 2),   # after blocks 0 and 2
              (TINY2, 300, 0, 1, 128, 2)]       # 1500 -> 1200 -> 900
_pcache = {}


def _prog(cfg, r, after, every, floor):
    key = (cfg.name, r, after, every, floor)
    if key not in _pcache:
        m = synth.Model(cfg, seed=4, decoder=False)
        x = synth.mel_input(5, 1, 2 * cfg.n_audio_ctx, cfg.n_mels)[0]
        want = O.Encoder(m, abi.ENC_F32).forward(x, tome_r=r, tome_after=after, tome_every=every, tome_floor=floor)
        _pcache[key] = (m, x, want)
    return _pcache[key]


@pytest.mark.parametrize("cfg,r,after,every,floor,merges", PROG_CASES,
                         ids=lambda v: getattr(v, "name", str(v)))
def test_encoder_tome_progressive_matches_textbook(cfg, r, after, every, floor, merges):
    """The oracle's progressive schedule (each merge's map composed into the
    original-row map, one unmerge) against the float64 textbook encoder, which
    composes the maps with numpy indexing: the same merges, within 1e-3."""
    m, x, want = _prog(cfg, r, after, every, floor)
    info = {}
    tb = TB.Encoder(m).forward(x, tome_r=r, tome_after=after, tome_every=every, tome_floor=floor, info=info)
    print(f"{cfg.name} r={r} every={every} floor={floor}: {info['merges']} merges, rank margin "
          f"{info['rank_margin']:.3e}, edge margin {info['edge_margin']:.3e}")
    assert info["merges"] == merges
    assert info["rank_margin"] > 1e-5 and info["edge_margin"] > 1e-5
    e = rel_maxabs(want, tb)
    print(f"  max-abs {e:.2e}")
    assert e <= 1e-3
    # the unmerged rows repeat each final row once per original row merged into
    # it: T - merges * r distinct rows
    assert np.unique(want, axis=0).shape[0] == cfg.n_audio_ctx - merges * r


@pytest.mark.parametrize("mutation,case", [("tome_every_off_by_one", 2), ("tome_ignore_floor", 1)])
def test_tome_progressive_planted_mistakes_are_detected(mutation, case):
    cfg, r, after, every, floor, _ = PROG_CASES[case]
    m, x, want = _prog(cfg, r, after, every, floor)
    bad = TB.Encoder(m, TB.Numerics(mutate=mutation)).forward(x, tome_r=r, tome_after=after, tome_every=every,
                                                               tome_floor=floor)
    e = rel_maxabs(want, bad)
    print(f"{mutation}: max-abs {e:.2e}")
    assert e > 1e-2


def test_tome_schedule_special_cases_are_exact():
    """Closed cases of the schedule, bit for bit in the oracle: a progressive
    cadence with no second due block is the single-shot schedule; a floor at
    the full length never merges (the dense encoder); r = 0 never merges."""
    cfg = TOME_MICRO
    m = synth.Model(cfg, seed=4, decoder=False)
    x = synth.mel_input(5, 1, 2 * cfg.n_audio_ctx, cfg.n_mels)[0]
    enc = O.Encoder(m, abi.ENC_F32)
    single = enc.forward(x, tome_r=60, tome_after=1)
    assert np.array_equal(enc.forward(x, tome_r=60, tome_after=1, tome_every=5), single)
    assert np.array_equal(enc.forward(x, tome_r=60, tome_after=1, tome_every=0, tome_floor=128), single)
    dense = enc.forward(x)
    assert np.array_equal(enc.forward(x, tome_r=60, tome_after=0, tome_every=1, tome_floor=cfg.n_audio_ctx), dense)
    assert np.array_equal(enc.forward(x, tome_r=0, tome_after=0, tome_every=1), dense)
    assert not np.array_equal(single, dense)
