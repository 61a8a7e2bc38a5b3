"""chatnet_amd — MI355X-native quantized Llama forward pass for ChatNet.

The hot path of ChatNet (LlamaModel.Forward with the dequant-matvecs of every
weight type it dispatches, F32, F16, Q4_0, Q4_1, Q5_0, Q5_1, Q8_0 and Q2_K ..
Q8_K, and the Mistral and Qwen2 variants of it) as hand-written gfx950 HIP
kernels behind a C ABI
(libchatnet_hip.so, include/chatnet_hip.h).  Python here is a thin host:
ctypes bindings, the IModel-shaped wrapper and the synthetic-weight tools.
"""
from . import _native
from .config import LLAMA2_7B, QWEN2_0_5B, TINY_TEST, TINYLLAMA_1B, LlamaConfig
from .engine import GreedySampler, TemperatureSampler, generate, net_random
from .model import HipLlamaModel

__all__ = [
    "_native",
    "LlamaConfig",
    "TINYLLAMA_1B",
    "LLAMA2_7B",
    "TINY_TEST",
    "QWEN2_0_5B",
    "HipLlamaModel",
    "GreedySampler",
    "TemperatureSampler",
    "generate",
    "net_random",
]
