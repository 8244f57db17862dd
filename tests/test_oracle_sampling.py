"""Pins of the token-choice oracle (oracle/sampling.py): Philox4x32-10 against the known-answer vectors published
with it, the Gumbel transform against the distribution's closed-form moments, the packed key against a sort, and
the choice rules against brute force and sampling frequencies. CPU only; none retypes the oracle's formula."""

import math

import numpy as np
import pytest

from oracle import sampling as S


@pytest.mark.parametrize("ctr, key, want", [
    # Random123's known-answer vectors for philox4x32 with 10 rounds (Salmon et al., SC '11)
    ((0, 0, 0, 0), (0, 0), (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff,) * 4, (0xffffffff,) * 2, (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
])
def test_philox_known_answers(ctr, key, want):
    got = tuple(int(x) for x in S.philox4x32_10(ctr, key))
    assert got == want, [hex(x) for x in got]


def test_philox_is_a_bijection_of_the_counter_on_a_sample():
    """Distinct counters under one key give distinct outputs (no collision among 2^16 consecutive rows)."""
    rows = np.arange(1 << 16, dtype=np.uint32)
    z = np.zeros_like(rows)
    x = S.philox4x32_10((rows, z, z, z), (np.uint32(7), np.uint32(9)))
    packed = (x[0].astype(np.uint64) << np.uint64(32)) | x[1].astype(np.uint64)
    assert len(np.unique(packed)) == len(rows)


def test_gumbel_moments():
    """Gumbel(0, 1): mean = Euler-Mascheroni, variance = pi^2 / 6; 400K draws over rows and indices."""
    g = np.concatenate([S.gumbel(12345, i, np.arange(100_000)) for i in range(4)]).astype(np.float64)
    assert np.isfinite(g).all()
    assert abs(g.mean() - 0.5772156649) < 0.01
    assert abs(g.var() - math.pi ** 2 / 6) < 0.03


def test_gumbel_depends_on_seed_index_and_row():
    rows = np.arange(1000)
    a = S.gumbel(1, 0, rows)
    assert not np.array_equal(a, S.gumbel(2, 0, rows))
    assert not np.array_equal(a, S.gumbel(1, 1, rows))
    assert not np.array_equal(a, S.gumbel(1 << 40, 0, rows))  # the seed's high word is part of the key
    assert np.array_equal(a, S.gumbel(1, 0, rows))
    assert len(np.unique(a)) > 990


def test_choice_key_orders_by_score_then_lowest_row():
    """Brute force: the largest key is the largest score, the lowest row among ties; negatives and zero included."""
    rng = np.random.default_rng(0)
    for _ in range(200):
        n = int(rng.integers(1, 40))
        s = rng.choice(np.array([-3.5, -1.0, -0.25, 0.0, 0.5, 2.0, 7.0], np.float32), size=n)
        keys = S.choice_key(s, np.arange(n))
        best = int(np.argmax(keys))
        want = min(range(n), key=lambda r: (-float(s[r]), r))
        assert best == want
        assert S.key_row(int(keys.max())) == want
    assert S.key_row(0) == -1


def _logits(B, V, seed, scale=3.0):
    return (np.random.default_rng(seed).standard_normal((B, V)) * scale).astype(np.float32)


def test_greedy_is_the_first_argmax_over_allowed_rows():
    B, V = 16, 300
    x = _logits(B, V, 1)
    x[3, 10] = x[3, 20] = x[3].max() + 1  # a tie: the lower row wins
    allow = np.random.default_rng(2).random((B, V)) < 0.3
    allow[3, [10, 20]] = True
    masked = np.arange(B) % 2 == 1
    from nanochat_amd.sampling import allow_rows
    zeros = np.zeros(B)
    tok, alt, pos = S.choose(x, temperature=np.zeros(B, np.float32), top_p=np.ones(B, np.float32),
                             seed=zeros.astype(np.uint64), pos=np.arange(B, dtype=np.int32),
                             first=zeros.astype(np.int32), masked=masked, allow=allow_rows(allow).view(np.uint32),
                             lazy=5)
    for b in range(B):
        ok = allow[b] if masked[b] else np.ones(V, bool)
        cand = np.where(ok, x[b], -np.inf)
        assert tok[b] == int(np.argmax(cand))
        alt_cand = cand.copy()
        alt_cand[5] = -np.inf
        assert alt[b] == int(np.argmax(alt_cand))
    assert tok[3] == 10
    assert np.array_equal(pos, np.arange(B) + 1)


def _frequencies(x, T, top_p, n, softcap):
    V = len(x)
    counts = np.zeros(V)
    for s in range(n):
        tok, _, _ = S.choose(x[None], temperature=np.array([T], np.float32), top_p=np.array([top_p], np.float32),
                             seed=np.array([s * 7919 + 13], np.uint64), pos=np.array([5], np.int32),
                             first=np.array([2], np.int32), softcap=softcap)
        counts[tok[0]] += 1
    return counts / n


def test_temperature_sampling_follows_the_softmax():
    """Gumbel-max over z / T samples softmax(z / T), z the capped logit: 8000 seeds against the closed form."""
    x = np.array([2.0, 1.0, 0.5, 0.0, -1.0, 30.0, 29.0, -40.0], np.float32)
    T, c = 1.3, 15.0
    z = c * np.tanh(x.astype(np.float64) / c)
    p = np.exp(z / T - (z / T).max())
    p /= p.sum()
    f = _frequencies(x, T, 1.0, 8000, c)
    assert np.abs(f - p).max() < 0.02, (f, p)


def test_nucleus_keep_matches_the_sorted_cumulative_definition():
    """transformers' TopPLogitsWarper: sort ascending, drop the prefix whose cumulative mass is <= 1 - top_p, but
    keep at least the largest (min_tokens_to_keep = 1)."""
    rng = np.random.default_rng(3)
    for _ in range(300):
        V = int(rng.integers(2, 60))
        e = rng.random(V).astype(np.float32)
        e[int(rng.integers(V))] = 1.0
        top_p = float(rng.choice([0.1, 0.5, 0.8, 0.95, 0.0]))
        order = np.argsort(e, kind="stable")
        cum = np.cumsum(e[order].astype(np.float64))
        drop = float(np.float32(np.float32(1 - np.float32(top_p)) * np.float32(e.astype(np.float64).sum())))
        removed = np.zeros(V, bool)
        removed[order[cum <= drop]] = True
        removed[order[-1]] = False
        assert np.array_equal(S.nucleus_keep(e, top_p), ~removed), (e, top_p)


def test_nucleus_sampling_follows_the_renormalised_nucleus():
    x = np.array([3.0, 2.5, 2.0, 1.0, 0.0, -1.0, -2.0, -5.0], np.float32)
    T, top_p = 1.0, 0.8
    p = np.exp(x.astype(np.float64) - x.max())
    p /= p.sum()
    keep = S.nucleus_keep(np.exp(x - x.max()).astype(np.float32), top_p)
    q = np.where(keep, p, 0)
    q /= q.sum()
    f = _frequencies(x, T, top_p, 6000, 0.0)
    assert (f[~keep] == 0).all()
    assert np.abs(f - q).max() < 0.025, (f, q)


def test_masks_inactive_slots_and_the_empty_mask():
    B, V = 6, 64
    x = _logits(B, V, 4)
    allow = np.zeros((B, V), bool)
    allow[0, [3, 9]] = True
    allow[1, :] = False  # nothing allowed: -1
    allow[2, 5] = True
    from nanochat_amd.sampling import allow_rows
    active = np.array([1, 1, 1, 0, 1, 1], bool)
    masked = np.array([1, 1, 1, 1, 0, 0], bool)
    T = np.array([0.8, 0.8, 0.0, 1.0, 0.0, 0.7], np.float32)
    tok, alt, pos = S.choose(x, temperature=T, top_p=np.array([1, 1, 1, 1, 1, 0.5], np.float32),
                             seed=np.arange(B, dtype=np.uint64), pos=np.full(B, 10, np.int32),
                             first=np.zeros(B, np.int32), active=active, masked=masked,
                             allow=allow_rows(allow).view(np.uint32), lazy=9)
    assert tok[0] in (3, 9) and alt[0] == 3
    assert tok[1] == -1 and alt[1] == -1
    assert tok[2] == 5
    assert tok[3] == -2 and pos[3] == 10  # inactive: untouched
    assert tok[4] == int(np.argmax(x[4]))
    assert alt[5] == -1  # a nucleus slot has no alternative
    assert np.array_equal(pos, [11, 11, 11, 10, 11, 11])
