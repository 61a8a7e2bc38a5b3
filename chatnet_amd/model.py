"""HipLlamaModel — the IModel of ChatNet backed by libchatnet_hip.

Mirrors the reference's interface (src/ChatNet.Core/Abstractions/IModel.cs:8-19):
    config                                   IModel.Config
    forward(token_ids, position, logits)     IModel.Forward(ReadOnlySpan<int>, int, Span<float>)
    close() / context manager                IDisposable.Dispose
Every call goes through the C ABI of include/chatnet_hip.h; the weights live
in HBM in their raw GGUF block layout (uploaded once, never dequantized on the
host).  Like the reference (TensorMath.cs:30-37), a model is not thread-safe.
"""
from __future__ import annotations

import ctypes
from typing import Mapping, Optional

import numpy as np

from . import _native
from .config import LlamaConfig


class HipLlamaModel:
    def __init__(self, config: LlamaConfig, weights: Optional[Mapping] = None, device: int = 0):
        self._lib = _native.hip_lib()
        self._cfg = config
        self._h = ctypes.c_void_p()
        c = config.to_c()
        _native.check(self._lib.chatnet_create(ctypes.byref(c), device, ctypes.byref(self._h)))
        if weights is not None:
            for name, t in weights.items():
                self.upload_tensor(name, t.type, t.dims, t.data)

    @classmethod
    def from_gguf(cls, path: str, kv_dtype: int = _native.KV_F32, context_length: Optional[int] = None,
                  device: int = 0) -> "HipLlamaModel":
        """InferenceEngine.LoadFromGguf (InferenceEngine.cs:57-110) for the Llama,
        Mistral and Qwen2 paths: the config from the file's metadata
        (GgufReader.ExtractModelConfig, the variant by ModelFactory's
        architecture rule), then the tensors LlamaWeights.ResolveAll resolves
        (LlamaWeights.cs:78-145; for Qwen2 also the q/k/v biases of a layer that
        has attn_q.bias, QwenWeights.cs:158-170) uploaded straight from the
        read-only mapping of the file; any other tensors in the file are left
        alone, as the reference leaves them."""
        from .gguf import GgufFile

        g = GgufFile(path)
        cfg = g.config(kv_dtype=kv_dtype, context_length=context_length)
        names = ["token_embd.weight", "output_norm.weight", "output.weight"]
        for l in range(cfg.n_layers):
            names += [f"blk.{l}.{n}.weight" for n in ("attn_norm", "ffn_norm", "attn_q", "attn_k", "attn_v",
                                                     "attn_output", "ffn_gate", "ffn_up", "ffn_down")]
            if cfg.arch == _native.ARCH_QWEN2 and g.has_tensor(f"blk.{l}.attn_q.bias"):
                names += [f"blk.{l}.{n}.bias" for n in ("attn_q", "attn_k", "attn_v")]
        m = cls(cfg, device=device)
        try:
            for name in names:
                if name == "output.weight" and not g.has_tensor(name):
                    continue  # the tied-embedding fallback is decided at the first forward
                t = g.tensor_info(name)
                m.upload_tensor(name, t.type, t.dims, g.tensor_bytes(name))
        except BaseException:
            m.close()
            raise
        return m

    # -- IModel -----------------------------------------------------------
    @property
    def config(self) -> LlamaConfig:
        return self._cfg

    def forward(self, token_ids, position: int, logits: Optional[np.ndarray] = None) -> np.ndarray:
        """LlamaModel.Forward (LlamaModel.cs:93-238): runs every token of the span,
        fills `logits` (vocab floats) with the last token's logits and returns it."""
        toks = np.ascontiguousarray(np.asarray(token_ids, dtype=np.int32).ravel())
        if logits is None:
            logits = np.empty(self._cfg.vocab_size, dtype=np.float32)
        if logits.dtype != np.float32 or logits.size < self._cfg.vocab_size or not logits.flags.c_contiguous:
            raise ValueError("logits must be a contiguous float32 array of at least vocab_size elements")
        _native.check(self._lib.chatnet_forward(
            self._h, toks.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), int(toks.size), int(position),
            logits.ctypes.data))
        return logits

    # -- extras over the reference interface -----------------------------
    def upload_tensor(self, name: str, ggml_type: int, dims, data: np.ndarray) -> None:
        arr = np.ascontiguousarray(data).view(np.uint8).ravel()
        d = (ctypes.c_uint64 * len(dims))(*[int(x) for x in dims])
        _native.check(self._lib.chatnet_upload_tensor(
            self._h, name.encode(), int(ggml_type), d, len(dims), arr.ctypes.data, int(arr.nbytes)))

    def argmax(self) -> int:
        """Device-side GreedySampler.Sample over the last logits."""
        out = ctypes.c_int32()
        _native.check(self._lib.chatnet_argmax(self._h, ctypes.byref(out)))
        return int(out.value)

    def sample(self, temperature: float, top_k: int, top_p: float, draw: float) -> int:
        """Device-side TemperatureSampler.Sample (TemperatureSampler.cs:33-112)
        over the last logits with the draw (float)Random.NextDouble()."""
        out = ctypes.c_int32()
        _native.check(self._lib.chatnet_sample(self._h, float(temperature), int(top_k), float(top_p), float(draw),
                                               ctypes.byref(out)))
        return int(out.value)

    def generate_sampled(self, prompt, max_tokens: int, temperature: float, top_k: int = 40, top_p: float = 0.9,
                         seed: int = -1, eos_token: int = -1) -> np.ndarray:
        """InferenceEngine.Generate with TemperatureSampler(temperature, top_k,
        top_p, seed) on the device (draw i = i-th NextDouble of Random(seed))."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32).ravel())
        out = np.empty(max(max_tokens, 1), dtype=np.int32)
        n = ctypes.c_int()
        _native.check(self._lib.chatnet_generate_sampled(
            self._h, p.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), int(p.size), int(max_tokens),
            float(temperature), int(top_k), float(top_p), int(seed), int(eos_token),
            out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), ctypes.byref(n)))
        return out[: n.value].copy()

    def get_logits(self) -> np.ndarray:
        out = np.empty(self._cfg.vocab_size, dtype=np.float32)
        _native.check(self._lib.chatnet_get_logits(self._h, out.ctypes.data))
        return out

    def generate_greedy(self, prompt, max_tokens: int, eos_token: int = -1) -> np.ndarray:
        """InferenceEngine.Generate's greedy loop (InferenceEngine.cs:234-307) on the device."""
        p = np.ascontiguousarray(np.asarray(prompt, dtype=np.int32).ravel())
        out = np.empty(max(max_tokens, 1), dtype=np.int32)
        n = ctypes.c_int()
        _native.check(self._lib.chatnet_generate_greedy(
            self._h, p.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), int(p.size), int(max_tokens),
            int(eos_token), out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)), ctypes.byref(n)))
        return out[: n.value].copy()

    def decode_greedy(self, max_tokens: int, eos_token: int = -1) -> np.ndarray:
        """Greedy continuation after forward() (InferenceEngine.cs:241-307) on the device."""
        out = np.empty(max(max_tokens, 1), dtype=np.int32)
        n = ctypes.c_int()
        _native.check(self._lib.chatnet_decode_greedy(
            self._h, int(max_tokens), int(eos_token), out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32)),
            ctypes.byref(n)))
        return out[: n.value].copy()

    def close(self) -> None:
        if self._h:
            self._lib.chatnet_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
