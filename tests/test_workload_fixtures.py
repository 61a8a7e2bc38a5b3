"""The committed workload fixtures (tests/golden/workload_<name>.npz) against
the CPU oracle and the generator: every named workload has one, its arrays
are consistent, the short TinyLlama workload's checkpoint regenerates with
the recorded digest, and the oracle reproduces its prompt logits and first
greedy tokens bit for bit."""
import os

import numpy as np
import pytest

import oracle
from chatnet_amd.workloads import WORKLOADS, checkpoint_digest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLDEN, f"workload_{name}.npz"))


@pytest.mark.parametrize("name", list(WORKLOADS))
def test_fixture_is_consistent(name):
    w = WORKLOADS[name]
    fx = load(name)
    assert int(fx["n_prompt"]) == w.n_prompt and int(fx["n_decode"]) == w.n_decode and int(fx["seed"]) == w.seed
    assert str(fx["mix"]) == w.mix
    assert fx["prompt"].shape == (w.n_prompt,) and np.array_equal(fx["prompt"], w.prompt())
    assert fx["tokens"].shape == (w.n_decode,) and fx["margins"].shape == (w.n_decode,)
    assert np.all((fx["tokens"] >= 0) & (fx["tokens"] < w.config.vocab_size))
    assert np.all(fx["margins"] >= 0)
    for k in ("logits_prompt", "logits_final"):
        assert fx[k].shape == (w.config.vocab_size,) and np.all(np.isfinite(fx[k]))
    # the first token is the argmax of the prompt logits (GreedySampler, first maximum)
    assert int(fx["tokens"][0]) == oracle.argmax(fx["logits_prompt"])


def test_oracle_reproduces_tinyllama_decode_fixture():
    w = WORKLOADS["tinyllama_q4_0_decode"]
    fx = load(w.name)
    ck = w.checkpoint()
    assert checkpoint_digest(ck) == str(fx["digest"])
    oracle.set_threads(os.cpu_count() or 1)
    try:
        ora = oracle.OracleLlama(w.config, ck)
        logits = ora.forward(w.prompt(), 0)
        assert np.array_equal(logits, fx["logits_prompt"])
        pos = w.n_prompt
        for i in range(4):
            tok = oracle.argmax(logits)
            assert tok == int(fx["tokens"][i])
            logits = ora.forward([tok], pos)
            pos += 1
        ora.close()
    finally:
        oracle.set_threads(1)
