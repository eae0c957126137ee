"""Pin the oracle's seeded top-k / top-p sampler (no GPU).

Closed forms (top-1 and tiny nucleus are the argmax; equal logits draw the
lowest top_k indices uniformly; NaN is never drawn), the draw's stream and
index (a two-candidate row of equal weight picks index 1 exactly when bit 63
of the SplitMix64 draw is set), and the distribution itself: the
frequencies of 200k seeded draws against an independent float64 numpy
statement of top-k + nucleus sampling."""
import numpy as np
import pytest

M64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15


def _mix(z):
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M64
    return z ^ (z >> 31)


def _draw(seed, stream, pos):
    base = _mix((seed + GAMMA) & M64) ^ _mix(((stream + 1) * 0xD1B54A32D192ED03) & M64)
    return _mix((base + (pos + 1) * GAMMA) & M64)


def _expected(logits, top_k, top_p, temperature):
    """float64: candidates by value desc / index asc, weights exp((l-l0)/T),
    smallest prefix holding top_p of the mass, renormalised."""
    idx = sorted(range(len(logits)), key=lambda i: (-logits[i], i))[:top_k]
    w = np.exp((np.array([logits[i] for i in idx], np.float64) - logits[idx[0]]) / temperature)
    c = np.cumsum(w)
    J = int(np.argmax(c >= top_p * c[-1]))
    p = np.zeros(len(logits))
    p[idx[:J + 1]] = w[:J + 1] / c[J]
    return p


def test_top1_and_tiny_nucleus_are_argmax(orc):
    rng = np.random.default_rng(0)
    x = rng.standard_normal((64, 3000)).astype(np.float32) * 3
    want = np.array([orc.argmax(r) for r in x])
    for k, p in ((1, 1.0), (64, 1e-7), (5, 1e-7)):
        got = orc.sample(x, k, p, 0.8, 7, np.arange(64), np.arange(64) * 11)
        assert np.array_equal(got, want), (k, p)


def test_equal_logits_lowest_indices_uniform(orc):
    x = np.full((30000, 10), 0.5, np.float32)
    got = orc.sample(x, 3, 1.0, 1.0, 3, 0, np.arange(30000))
    assert set(np.unique(got)) == {0, 1, 2}
    freq = np.bincount(got, minlength=3) / 30000
    assert np.all(np.abs(freq - 1 / 3) < 0.015)


def test_nan_never_drawn_and_all_nan_row(orc):
    x = np.zeros((2000, 6), np.float32)
    x[:, 2] = np.nan
    x[:, 4] = -0.0
    got = orc.sample(x, 6, 1.0, 1.0, 1, 0, np.arange(2000))
    assert 2 not in set(got.tolist()) and set(got.tolist()) == {0, 1, 3, 4, 5}
    assert orc.sample(np.full((1, 5), np.nan, np.float32), 4, 1.0, 1.0, 1, 0, 0)[0] == 0


def test_stream_and_position_indexing(orc):
    """Two equal candidates: c = (1, 2), r = 2u, index 1 iff u >= 1/2, i.e.
    iff bit 63 of the draw is set."""
    x = np.zeros((1, 2), np.float32)
    for seed, stream, pos in ((0, 0, 0), (5, 3, 17), (123456789, 40, 2047), (2**63 + 5, 1, 99)):
        got = orc.sample(x, 2, 1.0, 1.0, seed, stream, pos)[0]
        assert got == _draw(seed, stream, pos) >> 63, (seed, stream, pos)
    picks = orc.sample(np.zeros((512, 2), np.float32), 2, 1.0, 1.0, 9, 7, np.arange(512))
    assert np.array_equal(picks, [_draw(9, 7, p) >> 63 for p in range(512)])


@pytest.mark.parametrize("top_k,top_p,temp", [(8, 1.0, 1.0), (5, 1.0, 0.7), (8, 0.8, 1.3),
                                              (3, 0.5, 0.9), (6, 0.93, 2.0)])
def test_frequencies_match_float64_distribution(orc, top_k, top_p, temp):
    logits = np.array([0.3, 1.7, -0.4, 1.1, 0.9, 2.2, -1.5, 0.0], np.float32)
    n = 200_000
    got = orc.sample(np.broadcast_to(logits, (n, 8)), top_k, top_p, temp, 2026, 5, np.arange(n))
    freq = np.bincount(got, minlength=8) / n
    p = _expected(logits.astype(np.float64).tolist(), top_k, top_p, temp)
    tol = 5 * np.sqrt(p * (1 - p) / n) + 1e-9
    assert np.all(np.abs(freq - p) <= tol), (freq, p)
