"""Host-side mirrors of ChatNet's samplers and generation loop.

GreedySampler       src/ChatNet.Core/Samplers/GreedySampler.cs:13-26
TemperatureSampler  src/ChatNet.Core/Samplers/TemperatureSampler.cs:19-112 (runs
                    on the device through HipLlamaModel.sample)
generate            InferenceEngine.Generate's token loop, InferenceEngine.cs:234-307,
                    with token ids in and out (no tokenizer, no stop strings).
"""
from __future__ import annotations

import os
from typing import Callable, List, Optional

import numpy as np


class GreedySampler:
    """ISampler.Sample: index of the first maximum (strict '>')."""

    def sample(self, logits) -> int:
        # Vectorised equivalent of the strict '>' scan from index 0: the first
        # index of the maximum over the non-NaN values, except that a NaN at
        # index 0 never loses a comparison, so the answer is then 0.
        arr = np.asarray(logits, dtype=np.float32)
        if np.isnan(arr[0]):
            return 0
        return int(np.argmax(np.where(np.isnan(arr), -np.inf, arr)))


def net_random(seed: int, n: int) -> np.ndarray:
    """The first n values of System.Random(seed).NextDouble(), the .NET BCL's
    seeded generator TemperatureSampler draws from (TemperatureSampler.cs:29)."""
    from . import _native

    out = np.empty(max(n, 1), dtype=np.float64)
    _native.check(_native.hip_lib().chatnet_net_random(int(seed), int(n), out.ctypes.data))
    return out[:n]


class TemperatureSampler:
    """TemperatureSampler (TemperatureSampler.cs:19-112) for a HipLlamaModel:
    Sample runs on the device over the model's last logits, with the draws of
    System.Random(seed) taken in order, one per Sample when temperature > 0
    (TemperatureSampler.cs:97); temperature <= 0 is the greedy fallback.  A
    negative seed stands for the reference's unseeded Random."""

    def __init__(self, model, temperature: float, top_k: int = 40, top_p: float = 0.9, seed: int = -1):
        self.model = model
        self.temperature = float(temperature)
        self.top_k = int(top_k)
        self.top_p = float(top_p)
        self.seed = int(seed) if seed >= 0 else int.from_bytes(os.urandom(4), "little") & 0x7FFFFFFF
        self._draws = net_random(self.seed, 256)
        self._next = 0

    def sample(self, logits=None) -> int:
        """ISampler.Sample; the logits are those the model last produced (a host
        copy passed here is not read)."""
        if self.temperature <= 0.0:
            return self.model.argmax()
        if self._next >= len(self._draws):
            self._draws = net_random(self.seed, 2 * len(self._draws))
        draw = float(np.float32(self._draws[self._next]))
        self._next += 1
        return self.model.sample(self.temperature, self.top_k, self.top_p, draw)


def generate(model, prompt_ids, max_tokens: int, sampler=None, eos_token: Optional[int] = None,
             on_token: Optional[Callable[[int], None]] = None) -> List[int]:
    """Token loop of InferenceEngine.Generate (InferenceEngine.cs:234-307).

    The prompt is forwarded one token at a time (:235-239), then each sampled
    token is emitted, checked against EOS (:258-261) and the context limit
    (:295-298), forwarded at the next position (:302-303) and sampled (:306).
    """
    sampler = sampler or GreedySampler()
    cfg = model.config
    logits = np.empty(cfg.vocab_size, dtype=np.float32)
    prompt = [int(t) for t in prompt_ids]
    for i, tok in enumerate(prompt):
        model.forward([tok], i, logits)
    next_token = sampler.sample(logits)
    generated: List[int] = []
    pos = len(prompt)
    while len(generated) < max_tokens:
        if eos_token is not None and next_token == eos_token:
            break
        generated.append(next_token)
        if on_token:
            on_token(next_token)
        if pos >= cfg.context_length - 1:
            break
        model.forward([next_token], pos, logits)
        pos += 1
        next_token = sampler.sample(logits)
    return generated
