"""Device temperature sampler (chatnet_sample / chatnet_generate_sampled)
against the oracle's TemperatureSampler.Sample
(src/ChatNet.Core/Samplers/TemperatureSampler.cs:33-112) on the same logits
and draws.  Bar: identical tokens; a differing token is accepted only where the
oracle reports a decision within 1e-5 of its threshold (the device softmax sums
in a different order)."""
import numpy as np
import pytest

import oracle
from chatnet_amd import (TINY_TEST, TINYLLAMA_1B, HipLlamaModel, TemperatureSampler, _native, generate, net_random,
                         synth)
from gpu_util import announce

pytestmark = pytest.mark.gpu

MARGIN = 1e-5


def _check(tok, logits, t, k, p, draw, where):
    ref, margin = oracle.temperature_sample(logits, t, k, p, draw)
    if tok != ref:
        assert margin < MARGIN, f"{where}: device {tok} vs oracle {ref} (margin {margin:.3g})"
        return False
    return True


@pytest.mark.parametrize("cfg_name", ["tinyllama-vocab", "tiny", "vocab-40000"])
def test_sample_matches_oracle(cfg_name):
    """Vocabularies up to 32768 keep the probabilities in registers, larger
    ones (40000 here) in a scratch array."""
    cfg = {"tinyllama-vocab": TINYLLAMA_1B.replace(n_layers=1, context_length=64), "tiny": TINY_TEST,
           "vocab-40000": TINY_TEST.replace(vocab_size=40000)}[cfg_name]
    ck = synth.llama_checkpoint(cfg, seed=41, mix="q4_0")
    toks = synth.tokens(41, "prompt", 12, cfg.vocab_size)
    draws = net_random(41, 400).astype(np.float32)
    announce(f"device sampler vs oracle, vocab {cfg.vocab_size}")
    agree = total = 0
    with HipLlamaModel(cfg, ck) as m:
        for pos, tok in enumerate(toks):
            m.forward([tok], pos)
            logits = m.get_logits()
            # the raw logits of a random-weight model are nearly flat; scale
            # the temperature so the distributions range from peaked to flat
            spread = float(np.std(logits))
            # k = 64 and 65: the largest top-k sorted across one wave's lanes and
            # the smallest sorted in LDS
            for j, (t, k, p) in enumerate([(0.05, 40, 0.9), (0.3, 40, 0.9), (1.0, 40, 0.95), (1.0, 1, 0.9),
                                           (0.5, 1024, 1.0), (2.0, 7, 0.5), (0.2, 300, 0.99), (1.0, 64, 1.0),
                                           (1.0, 65, 1.0)]):
                t = t * spread
                draw = float(draws[(pos * 9 + j) % draws.size])
                got = m.sample(t, k, p, draw)
                agree += _check(got, logits, t, k, p, draw, f"pos {pos} T {t:.3g} k {k} p {p}")
                total += 1
            assert m.sample(0.0, 40, 0.9, 0.5) == m.argmax() == oracle.argmax(logits)
    print(f"{agree}/{total} identical (the rest within the decision margin)", flush=True)
    assert agree >= total - 2


def test_sample_argument_errors():
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=42, mix="q4_0")
    with HipLlamaModel(cfg, ck) as m:
        with pytest.raises(_native.ChatnetArgumentError):
            m.sample(1.0, 40, 0.9, 0.5)  # no logits yet
        m.forward([1, 2, 3], 0)
        with pytest.raises(_native.ChatnetArgumentError):
            m.sample(1.0, 0, 0.9, 0.5)
        with pytest.raises(_native.ChatnetArgumentError):
            m.sample(1.0, 1025, 0.9, 0.5)
        assert 0 <= m.sample(1.0, 40, 0.9, 0.5) < cfg.vocab_size


def test_generate_sampled_matches_host_loop_and_oracle():
    """chatnet_generate_sampled (device loop, graphs) == the host loop of
    InferenceEngine.Generate with the device sampler == the oracle's forward +
    sampler with the same draws (teacher-forced past a near-boundary draw)."""
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=43, mix="q4_0")
    prompt = synth.tokens(43, "prompt", 5, cfg.vocab_size)  # < 8: token by token in both loops
    n = 40
    with HipLlamaModel(cfg, ck) as m:
        spread = float(np.std(m.forward(prompt, 0)))
    t, k, p, seed = 0.6 * spread, 40, 0.9, 1234
    announce("generate_sampled vs host loop vs oracle")
    with HipLlamaModel(cfg, ck) as m:
        dev = list(m.generate_sampled(prompt, n, t, k, p, seed))
    with HipLlamaModel(cfg, ck) as m:
        host = generate(m, prompt, n, TemperatureSampler(m, t, k, p, seed))
    assert dev == host
    assert len(dev) == n
    draws = net_random(seed, n + 2).astype(np.float32)
    ora = oracle.OracleLlama(cfg, ck)
    logits = ora.forward(list(prompt), 0)
    for i in range(n):
        ref, margin = oracle.temperature_sample(logits, t, k, p, float(draws[i]))
        if ref != dev[i]:
            assert margin < 1e-3, f"step {i}: device {dev[i]} vs oracle {ref} (margin {margin:.3g})"
            print(f"near-boundary draw at step {i}; stopping comparison", flush=True)
            break
        logits = ora.forward([dev[i]], len(prompt) + i)


def test_generate_sampled_greedy_fallback_and_eos():
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=44, mix="q4_0")
    prompt = [5, 6, 7, 8]
    with HipLlamaModel(cfg, ck) as m:
        g = list(m.generate_greedy(prompt, 12))
        s = list(m.generate_sampled(prompt, 12, 0.0, 40, 0.9, 3))
        assert s == g
        a = list(m.generate_sampled(prompt, 12, 1.0, 40, 0.95, 5))
        b = list(m.generate_sampled(prompt, 12, 1.0, 40, 0.95, 5))
        assert a == b  # same seed, same tokens
        cut = list(m.generate_sampled(prompt, 12, 1.0, 40, 0.95, 5, eos_token=a[4]))
        assert cut == a[: a.index(a[4])]
