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

and, at the same 7B shape with a 16-token prompt and 16 greedy tokens, one
workload per mix of the types the device reads as packed units (the
reference's MatVecMulGeneric branches, LlamaModel.cs:488-562), so that each
of them is checked at full depth and width:

    llama2_7b_legacy_blocks_decode  Q4_1 attention and output, Q5_0 gate and
                                    down, Q5_1 up
    llama2_7b_q2_k_decode           Q2_K attention + gate/up, Q3_K down, Q8_K
                                    output
    llama2_7b_iq_a_decode           IQ4_XS attention, IQ3_XXS gate, IQ2_XS up,
                                    IQ4_NL down, IQ1_M output
    llama2_7b_iq_b_decode           IQ3_S attention, IQ2_S gate/up, IQ2_XXS
                                    down, IQ1_S output
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
    Workload("llama2_7b_legacy_blocks_decode", LLAMA2_7B.replace(context_length=2048), 21, "legacy_blocks", "prompt",
             16, 16),
    Workload("llama2_7b_q2_k_decode", LLAMA2_7B.replace(context_length=2048), 22, "q2_k", "prompt", 16, 16),
    Workload("llama2_7b_iq_a_decode", LLAMA2_7B.replace(context_length=2048), 23, "iq_a", "prompt", 16, 16),
    Workload("llama2_7b_iq_b_decode", LLAMA2_7B.replace(context_length=2048), 24, "iq_b", "prompt", 16, 16),
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
