"""Committed golden fixtures (tests/golden/, written by make_golden.py):
the oracle and the synthetic generator must keep reproducing them, and the
GPU path must match them."""
import os

import numpy as np
import pytest

import npref
import oracle
from chatnet_amd import TINY_TEST, synth

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
TAGS = ["q4_0", "q4_k", "q6_k", "q8_0", "q5_k", "q4_1", "q5_0", "q5_1", "q2_k", "q3_k", "q8_k", "iq2_xxs", "iq2_xs",
        "iq3_xxs", "iq1_s", "iq4_nl", "iq3_s", "iq2_s", "iq4_xs", "iq1_m"]


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


@pytest.mark.parametrize("tag", TAGS)
def test_block_fixtures_reproduce(tag):
    g = load(f"blocks_{tag}.npz")
    qtype, rows, K = int(g["ggml_type"]), int(g["rows"]), int(g["K"])
    # the generator still produces the same bytes
    t = synth.tensor(qtype, 2024, f"golden-{tag}", rows, K)
    assert np.array_equal(t.data, g["raw"])
    # the oracle still produces the same numbers, bit for bit
    assert np.array_equal(oracle.dequant(qtype, g["raw"], rows * K).reshape(rows, K), g["dequant"])
    assert np.array_equal(oracle.matvec(qtype, g["raw"], g["x"], rows, K), g["dots"])
    # and they agree with the float64 restatement
    ref = npref.DEQUANT[qtype](g["raw"], rows * K).reshape(rows, K) @ g["x"].astype(np.float64)
    assert np.max(np.abs(g["dots"] - ref)) / np.max(np.abs(ref)) < 1e-5


def test_tiny_model_fixture_reproduces():
    import hashlib

    def checkpoint_digest(ck):  # same digest as tests/golden/make_golden.py
        h = hashlib.sha256()
        for name in sorted(ck):
            h.update(name.encode())
            h.update(np.ascontiguousarray(ck[name].data).tobytes())
        return h.hexdigest()

    g = load("tiny_llama_q4_0.npz")
    ck = synth.llama_checkpoint(TINY_TEST, seed=int(g["seed"]), mix="q4_0")
    assert checkpoint_digest(ck) == str(g["digest"])
    ora = oracle.OracleLlama(TINY_TEST, ck)
    assert np.array_equal(ora.forward(g["prompt"], 0), g["logits"])
    toks, _ = oracle.OracleLlama(TINY_TEST, ck).generate_greedy(list(g["prompt"]), 16)
    assert toks == [int(t) for t in g["tokens"]]


@pytest.mark.gpu
@pytest.mark.parametrize("tag", TAGS)
def test_gpu_matches_block_fixtures(tag):
    from gpu_util import announce, gpu_matmul, normwise

    g = load(f"blocks_{tag}.npz")
    announce(f"golden blocks {tag}")
    y = gpu_matmul(int(g["ggml_type"]), g["raw"], g["x"], int(g["rows"]), int(g["K"]))[0]
    assert normwise(y, g["dots"]) <= 1e-3


@pytest.mark.gpu
def test_gpu_matches_tiny_model_fixture():
    from chatnet_amd import HipLlamaModel
    from gpu_util import announce

    g = load("tiny_llama_q4_0.npz")
    ck = synth.llama_checkpoint(TINY_TEST, seed=int(g["seed"]), mix="q4_0")
    announce("golden tiny model")
    with HipLlamaModel(TINY_TEST, ck) as m:
        logits = m.forward(g["prompt"], 0)
        assert np.max(np.abs(logits - g["logits"])) <= 1e-2
        toks = m.generate_greedy(g["prompt"], 16)
    margins = g["margins"]
    for i, (a, b) in enumerate(zip(toks, g["tokens"])):
        if a != b:
            assert margins[i] < 1e-3, f"step {i}"
            break
