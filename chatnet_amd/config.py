"""Model hyper-parameters and the named workloads.

LlamaConfig mirrors src/ChatNet.Core/Models/Llama/LlamaConfig.cs:8-38 (itself
derived from ModelConfig, src/ChatNet.Core/Abstractions/ModelConfig.cs:6-27).
"""
from __future__ import annotations

import dataclasses

from . import _native


@dataclasses.dataclass(frozen=True)
class LlamaConfig:
    dim: int                 # Dim (embedding_length)
    hidden_dim: int          # HiddenDim (feed_forward_length)
    n_layers: int            # LayerCount
    n_heads: int             # HeadCount
    n_kv_heads: int          # KvHeadCount
    head_dim: int            # HeadDim
    vocab_size: int          # VocabSize
    context_length: int      # ContextLength (KV-cache capacity)
    rope_freq_base: float = 10000.0
    rms_norm_eps: float = 1e-5
    kv_dtype: int = _native.KV_F32
    arch: int = _native.ARCH_LLAMA  # ARCH_QWEN2: QwenModel's biases and NeoX RoPE

    @property
    def kv_dim(self) -> int:  # LlamaConfig.cs:34
        return self.n_kv_heads * self.head_dim

    @property
    def kv_mul(self) -> int:  # LlamaConfig.cs:37
        return self.n_heads // self.n_kv_heads

    def replace(self, **kw) -> "LlamaConfig":
        return dataclasses.replace(self, **kw)

    def to_c(self) -> _native.ChatnetConfig:
        return _native.ChatnetConfig(
            self.dim, self.hidden_dim, self.n_layers, self.n_heads, self.n_kv_heads, self.head_dim,
            self.vocab_size, self.context_length, self.rope_freq_base, self.rms_norm_eps, self.kv_dtype, self.arch,
        )


# TinyLlama-1.1B architecture (GgufReader.cs:80-182 defaults are TinyLlama's).
TINYLLAMA_1B = LlamaConfig(dim=2048, hidden_dim=5632, n_layers=22, n_heads=32, n_kv_heads=4, head_dim=64,
                           vocab_size=32000, context_length=2048)
# Llama-2-7B architecture.
LLAMA2_7B = LlamaConfig(dim=4096, hidden_dim=11008, n_layers=32, n_heads=32, n_kv_heads=32, head_dim=128,
                        vocab_size=32000, context_length=2048)
# A small Llama for tests (GQA, both block sizes usable).
TINY_TEST = LlamaConfig(dim=256, hidden_dim=512, n_layers=2, n_heads=8, n_kv_heads=2, head_dim=32,
                        vocab_size=512, context_length=64)
# Qwen2-0.5B architecture (QwenConfig.cs; rope base 1e6, eps 1e-6, tied embeddings).
QWEN2_0_5B = LlamaConfig(dim=896, hidden_dim=4864, n_layers=24, n_heads=14, n_kv_heads=2, head_dim=64,
                         vocab_size=151936, context_length=2048, rope_freq_base=1000000.0, rms_norm_eps=1e-6,
                         arch=_native.ARCH_QWEN2)
