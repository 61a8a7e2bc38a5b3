"""chatnet_amd — MI355X-native quantized Llama forward pass for ChatNet.

The hot path of ChatNet (LlamaModel.Forward with the Q4_0 / Q4_K / Q6_K
dequant-matvecs) as hand-written gfx950 HIP kernels behind a C ABI
(libchatnet_hip.so, include/chatnet_hip.h).  Python here is a thin host:
ctypes bindings, the IModel-shaped wrapper and the synthetic-weight tools.
"""
from . import _native
from .config import LLAMA2_7B, TINY_TEST, TINYLLAMA_1B, LlamaConfig
from .engine import GreedySampler, TemperatureSampler, generate, net_random
from .model import HipLlamaModel

__all__ = [
    "_native",
    "LlamaConfig",
    "TINYLLAMA_1B",
    "LLAMA2_7B",
    "TINY_TEST",
    "HipLlamaModel",
    "GreedySampler",
    "TemperatureSampler",
    "generate",
    "net_random",
]
