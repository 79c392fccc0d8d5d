"""CPU model of the cross-attention kernel's wave-parallel softmax sum.

`fw_seq_sum_wave` (franken_whisper_amd/csrc/dec_fast.hip) forms the
sequential f32 sum ((0 + v[0]) + v[1]) + ... of softmax_rows (reference
nn.rs:4880-4963) with one 64-lane wave instead of one thread.  This file
restates its four steps in numpy, lane by lane:

1. lane chunks of c values and a rough prefix;
2. per-lane (D0, D1) maps from the two lowest starts of the guessed binade;
3. a segmented composition over runs of lanes of one binade;
4. the exact walk.

The test checks the restatement against np.cumsum in float32 (a sequential
left-to-right sum) on adversarial inputs: ties at half-ulps, values around
powers of two, tiny and zero values, and every length up to 1536.  Bit-identity
of the HIP kernel itself is covered by the GPU decoder parity tests, which
compare whole greedy decodes with the oracle.
"""
import numpy as np
import pytest

W = 64
MAXC = 24


def f2u(x):
    return np.float32(x).view(np.uint32)


def u2f(u):
    return np.uint32(u).view(np.float32)


def seq_sum(v):
    if len(v) == 0:
        return np.float32(0.0)
    return np.cumsum(np.asarray(v, dtype=np.float32), dtype=np.float32)[-1]


def wave_sum(v):
    """Mirror of fw_seq_sum_wave, n <= 64 * MAXC."""
    v = np.asarray(v, dtype=np.float32)
    n = len(v)
    c = max(((n + 63) // 64 + 3) & ~3, 4)
    assert c <= MAXC
    e = np.zeros((W, c), dtype=np.float32)
    for l in range(W):
        lo_i, hi_i = l * c, min((l + 1) * c, n)
        if lo_i < hi_i:
            e[l, : hi_i - lo_i] = v[lo_i:hi_i]
    # 1. rough chunk sums and exclusive prefix (any order is fine here)
    t = np.array([np.float32(np.sum(e[l], dtype=np.float32)) for l in range(W)], dtype=np.float32)
    P = np.zeros(W, dtype=np.float32)
    acc = np.float32(0)
    for l in range(W):
        P[l] = acc
        acc = np.float32(acc + t[l])
    # 2. lane maps
    ok = np.zeros(W, dtype=bool)
    lo = np.zeros(W, dtype=np.uint32)
    d0 = np.zeros(W, dtype=np.int64)
    d1 = np.zeros(W, dtype=np.int64)
    for l in range(W):
        ex = int(f2u(P[l])) >> 23
        lo[l] = np.uint32(ex << 23)
        hi = np.uint32((ex + 1) << 23)
        good = 1 <= ex <= 253
        if good:
            good = (P[l] >= np.float32(u2f(lo[l]) * np.float32(1.0009765625))) and (
                np.float32(P[l] + t[l]) <= np.float32(u2f(hi) * np.float32(0.9990234375)))
        s0, s1 = u2f(lo[l]), u2f(lo[l] + 1)
        for x in e[l]:
            s0 = np.float32(s0 + x)
            s1 = np.float32(s1 + x)
        good = good and f2u(s0) <= hi and f2u(s1) <= hi
        ok[l] = good
        d0[l] = int(f2u(s0)) - int(lo[l])
        d1[l] = int(f2u(s1)) - int(lo[l]) - 1
    # 3. runs of ok lanes with one binade compose their parity maps in order
    key = [int(lo[l]) if ok[l] else (0x80000000 | l) for l in range(W)]
    heads = [l for l in range(W) if l == 0 or key[l] != key[l - 1]]
    # 4. walk
    s = np.float32(0.0)
    for hi_idx, a in enumerate(heads):
        b = heads[hi_idx + 1] - 1 if hi_idx + 1 < len(heads) else W - 1
        done = False
        if ok[b]:
            D0, D1 = d0[a], d1[a]
            for q in range(a + 1, b + 1):
                D0, D1 = D0 + (d1[q] if D0 & 1 else d0[q]), D1 + (d1[q] if (1 + D1) & 1 else d0[q])
            sb = int(f2u(s))
            rlo = int(lo[b])
            rhi = rlo + (1 << 23)
            D = D1 if sb & 1 else D0
            if rlo <= sb < rhi and sb + D <= rhi:
                s = u2f(sb + D)
                done = True
        if not done:
            for q in range(a, b + 1):
                for x in e[q]:
                    s = np.float32(s + x)
    return s


def _vectors(rng):
    out = []
    for n in (1, 2, 3, 5, 63, 64, 65, 100, 255, 256, 257, 777, 1023, 1024, 1499, 1500, 1501, 1535, 1536):
        out.append(rng.random(n).astype(np.float32))
    for kind in range(6):
        for _ in range(8):
            n = 1500 if rng.random() < 0.5 else int(rng.integers(1, 1537))
            if kind == 0:   # softmax-like exps of several spreads, with the max at 1
                sig = float(rng.choice([0.3, 1.0, 3.0, 8.0]))
                x = np.exp(rng.uniform(-8 * sig, 0, n)).astype(np.float32)
                x[rng.integers(n)] = 1.0
            elif kind == 1:  # dyadic values: many exact ties at half-ulps
                x = (rng.integers(0, 64, n) * np.exp2(-rng.integers(0, 12, n).astype(np.float64))).astype(np.float32)
            elif kind == 2:  # values around powers of two
                x = np.ldexp(1.0 + 0.5 * rng.integers(0, 3, n), rng.integers(-12, -2, n)).astype(np.float32)
            elif kind == 3:  # tiny values, subnormals and zeros
                x = np.ldexp(rng.random(n), -rng.integers(0, 140, n)).astype(np.float32)
                x[rng.random(n) < 0.25] = 0.0
            elif kind == 4:  # powers of two and zeros
                x = np.exp2(-rng.integers(0, 30, n).astype(np.float64)).astype(np.float32)
                x[rng.random(n) < 0.3] = 0.0
            else:            # all equal
                x = np.full(n, np.float32(rng.random()), dtype=np.float32)
            out.append(np.minimum(x, np.float32(1.0)).astype(np.float32))
    return out


def test_wave_sum_model_matches_sequential_sum():
    rng = np.random.default_rng(20261201)
    for v in _vectors(rng):
        a, b = seq_sum(v), wave_sum(v)
        assert f2u(a) == f2u(b), (len(v), float(a), float(b))


def test_wave_sum_model_catches_a_wrong_parity_rule():
    """A planted mistake (ties resolved without the running parity) must fail."""
    # 2^0 + 2^-24 ties to even at 1.0; a second tie from an odd start rounds up
    v = np.array([1.0] + [2.0 ** -24] * 40 + [2.0 ** -23] + [2.0 ** -24] * 40, dtype=np.float32)
    exact = seq_sum(v)
    s = np.float32(0.0)
    for x in v:   # a naive model that always rounds ties up
        r = np.float64(s) + np.float64(x)
        ulp = np.float64(np.spacing(s)) if s > 0 else 0.0
        s = np.float32(r) if ulp == 0 or (r / ulp) % 1 != 0.5 else np.float32(r + ulp / 2)
    assert f2u(s) != f2u(exact)
    assert f2u(wave_sum(v)) == f2u(exact)


@pytest.mark.parametrize("n", [1500])
def test_wave_sum_model_uses_the_fast_path(n):
    """On softmax-like data most lanes are applied as composed runs."""
    rng = np.random.default_rng(7)
    x = np.exp(rng.uniform(-3, 0, n)).astype(np.float32)
    assert f2u(wave_sum(x)) == f2u(seq_sum(x))
