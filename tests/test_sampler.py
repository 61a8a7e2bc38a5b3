"""The temperature sampler's pieces on the CPU: the oracle's restatement of
TemperatureSampler.Sample (src/ChatNet.Core/Samplers/TemperatureSampler.cs:33-112)
and of the seeded System.Random it draws from, pinned by published outputs of
.NET's Random and by what the sampling rule fixes; and the library's own
generator (chatnet_net_random, used by chatnet_generate_sampled) against it."""
import numpy as np
import pytest

import oracle
from chatnet_amd import net_random


def test_net_random_published_values():
    # new Random(0).Next() == 1559595546, NextDouble() == 0.7262432699679598;
    # new Random(42).Next() == 1434747710 (values printed by .NET's Random).
    assert oracle.NetRandom(0).sample() == 1559595546
    assert oracle.NetRandom(0).next_double() == 0.7262432699679598
    assert oracle.NetRandom(42).sample() == 1434747710
    # |seed| is used, and int.MinValue maps to int.MaxValue (Random(int) ctor)
    a, b = oracle.NetRandom(-42), oracle.NetRandom(42)
    assert [a.sample() for _ in range(10)] == [b.sample() for _ in range(10)]
    a, b = oracle.NetRandom(-2**31), oracle.NetRandom(2**31 - 1)
    assert [a.sample() for _ in range(10)] == [b.sample() for _ in range(10)]
    r = oracle.NetRandom(7)
    vals = [r.next_double() for _ in range(10000)]
    assert 0.0 <= min(vals) and max(vals) < 1.0 and abs(np.mean(vals) - 0.5) < 0.02


@pytest.mark.parametrize("seed", [0, 1, 42, 12345, -7, 2**31 - 1, -2**31])
def test_library_generator_matches_oracle(seed):
    r = oracle.NetRandom(seed)
    assert np.array_equal(net_random(seed, 500), [r.next_double() for _ in range(500)])


def _ref_sample(logits, t, k, p, draw):
    """Independent float64 statement of the rule (ties excluded by construction)."""
    z = np.asarray(logits, np.float64) / t
    q = np.exp(z - z.max())
    q /= q.sum()
    order = np.argsort(-q, kind="stable")[:k]
    c = np.cumsum(q[order])
    hit = np.nonzero(c >= p)[0]
    cut = int(hit[0]) + 1 if hit.size else k
    w = q[order[:cut]] / q[order[:cut]].sum()
    j = np.nonzero(draw < np.cumsum(w))[0]
    return int(order[j[0]] if j.size else order[cut - 1])


def test_oracle_sampler_follows_the_rule():
    rng = np.random.default_rng(3)
    checked = 0
    for trial in range(300):
        n = int(rng.integers(2, 3000))
        logits = (rng.standard_normal(n) * rng.uniform(0.5, 6)).astype(np.float32)
        t = float(rng.choice([0.2, 0.7, 1.0, 1.8]))
        k = int(rng.choice([1, 2, 7, 40, 1000]))
        p = float(rng.choice([0.05, 0.5, 0.9, 1.0, 1.5]))
        draw = float(np.float32(rng.random()))
        tok, margin = oracle.temperature_sample(logits, t, k, p, draw)
        if margin < 1e-5:
            continue
        assert tok == _ref_sample(logits, t, min(k, n), p, draw), trial
        checked += 1
    assert checked > 250


def test_oracle_sampler_special_cases():
    logits = np.array([0.1, 2.0, -1.0, 1.9, 0.5], np.float32)
    assert oracle.temperature_sample(logits, 0.0, 40, 0.9, 0.99)[0] == 1   # greedy fallback
    assert oracle.temperature_sample(logits, -1.0, 40, 0.9, 0.99)[0] == 1
    for draw in (0.0, 0.5, 0.999):
        assert oracle.temperature_sample(logits, 1.0, 1, 0.9, draw)[0] == 1  # top-1
        assert oracle.temperature_sample(logits, 1.0, 40, 1e-9, draw)[0] == 1  # nucleus of one
    # top-2 renormalised: p(1) = e^2 / (e^2 + e^1.9)
    split = np.exp(2.0) / (np.exp(2.0) + np.exp(1.9))
    assert oracle.temperature_sample(logits, 1.0, 2, 1.0, split - 1e-3)[0] == 1
    assert oracle.temperature_sample(logits, 1.0, 2, 1.0, split + 1e-3)[0] == 3
    # a draw at or past the last running sum returns the last kept token (:108)
    assert oracle.temperature_sample(logits, 1.0, 2, 1.0, 1.0)[0] == 3
    assert oracle.temperature_sample(logits, 1.0, 0, 0.9, 0.5)[0] == -1      # the reference throws here


def test_oracle_sampler_frequencies():
    logits = np.array([1.0, 0.0, 2.0, 0.5, -3.0, 1.5], np.float32)
    t, k, p = 0.9, 4, 0.95
    draws = net_random(99, 20000).astype(np.float32)
    counts = np.bincount([oracle.temperature_sample(logits, t, k, p, float(d))[0] for d in draws], minlength=6)
    z = logits / t
    q = np.exp(z - z.max())
    q /= q.sum()
    order = np.argsort(-q)[:k]
    c = np.cumsum(q[order])
    cut = int(np.nonzero(c >= p)[0][0]) + 1 if (c >= p).any() else k
    expect = np.zeros(6)
    expect[order[:cut]] = q[order[:cut]] / q[order[:cut]].sum()
    assert np.all(counts[expect == 0] == 0)
    assert np.max(np.abs(counts / len(draws) - expect)) < 0.015
