"""The named end-to-end workloads: model shape, seeded weights, seeded prompt.

Each workload fixes everything a run depends on, so a GPU run, the CPU
oracle and the committed expected-output fixtures (tests/golden/) all see the
same bytes: the checkpoint is a pure function of (config, seed, mix) through
chatnet_amd.synth, and the prompt of (seed, prompt_stream, n_prompt).

    tinyllama_q4_0_decode   TinyLlama-1.1B shape, Q4_0, 16-token prompt, 32
                            greedy tokens, context 64
    tinyllama_q4_0_prefill  TinyLlama-1.1B shape, Q4_0, 512-token prompt as one
                            span, 128 greedy tokens (cache to 640 positions)
    llama2_7b_q4_0_decode   Llama-2-7B shape, Q4_0, 128-token prompt as one
                            span, 256 greedy tokens, context 2048
    llama2_7b_q4_k_m_decode Llama-2-7B shape, Q4_K attention + gate/up, Q6_K
                            down + output, 16-token prompt, 64 greedy tokens
    llama2_7b_q3_k_m_decode Llama-2-7B shape, Q3_K attention + gate/up, Q4_K
                            down, Q6_K output, 16-token prompt, 64 greedy tokens
"""
from __future__ import annotations

import dataclasses

import numpy as np

from . import synth
from .config import LLAMA2_7B, TINYLLAMA_1B, LlamaConfig


@dataclasses.dataclass(frozen=True)
class Workload:
    name: str
    config: LlamaConfig
    seed: int
    mix: str
    prompt_stream: str
    n_prompt: int
    n_decode: int

    def checkpoint(self) -> dict:
        return synth.llama_checkpoint(self.config, seed=self.seed, mix=self.mix)

    def prompt(self) -> np.ndarray:
        return synth.tokens(self.seed, self.prompt_stream, self.n_prompt, self.config.vocab_size)


WORKLOADS = {w.name: w for w in (
    Workload("tinyllama_q4_0_decode", TINYLLAMA_1B.replace(context_length=64), 1234, "q4_0", "prompt", 16, 32),
    Workload("tinyllama_q4_0_prefill", TINYLLAMA_1B.replace(context_length=2048), 77, "q4_0", "prefill", 512, 128),
    Workload("llama2_7b_q4_0_decode", LLAMA2_7B.replace(context_length=2048), 7, "q4_0", "prompt", 128, 256),
    Workload("llama2_7b_q4_k_m_decode", LLAMA2_7B.replace(context_length=2048), 11, "q4_k_m", "prompt", 16, 64),
    Workload("llama2_7b_q3_k_m_decode", LLAMA2_7B.replace(context_length=2048), 13, "q3_k_m", "prompt", 16, 64),
)}


def checkpoint_digest(ck: dict) -> str:
    """XXH3-128 over every tensor's name, byte count and every byte, in name
    order: tells whether a machine regenerates exactly the same checkpoint
    (about 0.1 s per GB)."""
    import xxhash

    h = xxhash.xxh3_128()
    for name in sorted(ck):
        data = np.ascontiguousarray(ck[name].data).view(np.uint8).ravel()
        h.update(name.encode())
        h.update(str(data.size).encode())
        h.update(memoryview(data))
    return h.hexdigest()
