"""Host-side mirrors of ChatNet's sampler and generation loop.

GreedySampler   src/ChatNet.Core/Samplers/GreedySampler.cs:13-26
generate        InferenceEngine.Generate's token loop, InferenceEngine.cs:234-307,
                with token ids in and out (no tokenizer, no stop strings).
"""
from __future__ import annotations

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
