"""Seeded synthetic Llama checkpoints in GGUF block layouts.

A checkpoint is a dict: GGUF tensor name -> SynthTensor(type, dims, data),
with dims in GGUF order (ne0 = inner dimension) and data the raw bytes the
reference would mmap (MemoryMappedWeights.GetTensorPointer,
MemoryMappedWeights.cs:76-84).  Weights are N(0, 0.02) quantized by
libchatnet_synth; embeddings are F32 N(0, 0.02); norm weights are 1.0.
"""
from __future__ import annotations

import ctypes
import dataclasses
from typing import Optional

import numpy as np

from . import _native
from .config import LlamaConfig

SIGMA = 0.02

# Quantization mixes.  "q4_0": every matrix Q4_0.  "q4_k_m": Q4_K for the
# attention and ffn_gate/up matrices, Q6_K for ffn_down and output; "q5_k_m"
# likewise with Q5_K; "q4_k", "q6_k", "q8_0": every matrix of that type.
MIXES = {
    "q4_0": {"attn": _native.GGML_Q4_0, "gate_up": _native.GGML_Q4_0, "down": _native.GGML_Q4_0,
             "output": _native.GGML_Q4_0},
    "q4_k_m": {"attn": _native.GGML_Q4_K, "gate_up": _native.GGML_Q4_K, "down": _native.GGML_Q6_K,
               "output": _native.GGML_Q6_K},
    "q4_k": {"attn": _native.GGML_Q4_K, "gate_up": _native.GGML_Q4_K, "down": _native.GGML_Q4_K,
             "output": _native.GGML_Q4_K},
    "q6_k": {"attn": _native.GGML_Q6_K, "gate_up": _native.GGML_Q6_K, "down": _native.GGML_Q6_K,
             "output": _native.GGML_Q6_K},
    "q8_0": {"attn": _native.GGML_Q8_0, "gate_up": _native.GGML_Q8_0, "down": _native.GGML_Q8_0,
             "output": _native.GGML_Q8_0},
    # Q5_K_M-style: Q5_K attention and ffn_gate/up, Q6_K ffn_down and output
    "q5_k_m": {"attn": _native.GGML_Q5_K, "gate_up": _native.GGML_Q5_K, "down": _native.GGML_Q6_K,
               "output": _native.GGML_Q6_K},
    # unquantized matrices (TensorMath.MatVecMul / LlamaModel.MatVecMulF16)
    "f32": {"attn": _native.GGML_F32, "gate_up": _native.GGML_F32, "down": _native.GGML_F32,
            "output": _native.GGML_F32},
    "f16": {"attn": _native.GGML_F16, "gate_up": _native.GGML_F16, "down": _native.GGML_F16,
            "output": _native.GGML_F16},
    # every matrix dispatched on its own type, ffn_gate and ffn_up differing
    "mixed": {"attn": _native.GGML_Q8_0, "gate": _native.GGML_Q4_0, "up": _native.GGML_F16,
              "down": _native.GGML_Q4_K, "output": _native.GGML_F32},
    # block types only, each matrix on its own type and ffn_gate/up differing
    "mixed_blocks": {"attn": _native.GGML_Q8_0, "gate": _native.GGML_Q4_0, "up": _native.GGML_Q5_K,
                     "down": _native.GGML_Q6_K, "output": _native.GGML_Q4_K},
    # the types served through packed units (LlamaModel.MatVecMulByType's
    # generic branches): legacy 32-blocks, then the small K-quants
    "legacy_blocks": {"attn": _native.GGML_Q4_1, "gate": _native.GGML_Q5_0, "up": _native.GGML_Q5_1,
                      "down": _native.GGML_Q5_0, "output": _native.GGML_Q4_1},
    "q3_k_m": {"attn": _native.GGML_Q3_K, "gate_up": _native.GGML_Q3_K, "down": _native.GGML_Q4_K,
               "output": _native.GGML_Q6_K},
    "q2_k": {"attn": _native.GGML_Q2_K, "gate_up": _native.GGML_Q2_K, "down": _native.GGML_Q3_K,
             "output": _native.GGML_Q8_K},
    # float and block projections side by side: F16 attention, Q4_0 gate/up,
    # F32 down (each GEMM of a span on its own weight format)
    "float_mix": {"attn": _native.GGML_F16, "gate_up": _native.GGML_Q4_0, "down": _native.GGML_F32,
                  "output": _native.GGML_Q4_K},
    # the IQ family as DequantIQ.cs decodes it, every type in one of two mixes
    "iq_a": {"attn": _native.GGML_IQ4_XS, "gate": _native.GGML_IQ3_XXS, "up": _native.GGML_IQ2_XS,
             "down": _native.GGML_IQ4_NL, "output": _native.GGML_IQ1_M},
    "iq_b": {"attn": _native.GGML_IQ3_S, "gate_up": _native.GGML_IQ2_S, "down": _native.GGML_IQ2_XXS,
             "output": _native.GGML_IQ1_S},
}


@dataclasses.dataclass
class SynthTensor:
    type: int
    dims: tuple  # GGUF order: (ne0, ne1)
    data: np.ndarray  # uint8 raw bytes (float32 view for F32)

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n


def stream_id(name: str) -> int:
    return int(_native.synth_lib().chatnet_synth_stream_id(name.encode()))


def normal(seed: int, name: str, n: int, sigma: float = SIGMA, start: int = 0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    _native.synth_lib().chatnet_synth_normal(seed, stream_id(name), start, n, sigma, out.ctypes.data)
    return out


def quantize(ggml_type: int, w: np.ndarray) -> np.ndarray:
    """Quantizes a float32 array (length a multiple of the block) to raw bytes."""
    w = np.ascontiguousarray(w, dtype=np.float32).ravel()
    nbytes = _native.tensor_nbytes(ggml_type, w.size) if ggml_type != _native.GGML_F32 else w.size * 4
    out = np.empty(nbytes, dtype=np.uint8)
    wrote = _native.synth_lib().chatnet_synth_quantize(ggml_type, w.ctypes.data, w.size, out.ctypes.data)
    if wrote != nbytes:
        raise ValueError(f"quantize: type {ggml_type} cannot hold {w.size} elements")
    return out


def float_to_half(f: float) -> int:
    return int(_native.synth_lib().chatnet_float_to_half(ctypes.c_float(f)))


def tensor(ggml_type: int, seed: int, name: str, rows: int, cols: int, sigma: float = SIGMA) -> SynthTensor:
    """rows x cols matrix (GGUF dims (cols, rows)) of N(0, sigma) weights in `ggml_type`."""
    n = rows * cols
    if ggml_type == _native.GGML_F32:
        data = normal(seed, name, n, sigma).view(np.uint8)
    elif ggml_type == _native.GGML_F16:  # round to nearest even, as System.Half's conversion
        data = normal(seed, name, n, sigma).astype(np.float16).view(np.uint8)
    else:
        nbytes = _native.tensor_nbytes(ggml_type, n)
        data = np.empty(nbytes, dtype=np.uint8)
        wrote = _native.synth_lib().chatnet_synth_tensor(ggml_type, seed, stream_id(name), sigma, n,
                                                         data.ctypes.data)
        if wrote != nbytes:
            raise ValueError(f"synth_tensor failed for {name}")
    return SynthTensor(ggml_type, (cols, rows), data)


def tokens(seed: int, name: str, n: int, vocab: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    _native.synth_lib().chatnet_synth_tokens(seed, stream_id(name), n, vocab, out.ctypes.data)
    return out


BIAS_SIGMA = 0.25  # N(0, 0.25) QKV biases: comparable to the projections of a normalised x


def llama_checkpoint(cfg: LlamaConfig, seed: int = 1234, mix: str = "q4_0",
                     with_output: bool = True, embedding: int = _native.GGML_F32,
                     qkv_bias: Optional[bool] = None) -> dict:
    """All tensors LlamaWeights.ResolveAll (LlamaWeights.cs:78-145) looks up;
    for an ARCH_QWEN2 config also the F32 q/k/v biases QwenWeights resolves
    (QwenWeights.cs:158-170) unless qkv_bias is False.  with_output=False leaves
    out output.weight (the tied-embedding fallback); `embedding` is the type of
    token_embd.weight."""
    q = MIXES[mix]
    if qkv_bias is None:
        qkv_bias = cfg.arch == _native.ARCH_QWEN2
    ck = {}
    ck["token_embd.weight"] = tensor(embedding, seed, "token_embd.weight", cfg.vocab_size, cfg.dim)
    ones = np.ones(cfg.dim, dtype=np.float32)
    ck["output_norm.weight"] = SynthTensor(_native.GGML_F32, (cfg.dim,), ones.view(np.uint8).copy())
    if with_output:
        ck["output.weight"] = tensor(q["output"], seed, "output.weight", cfg.vocab_size, cfg.dim)
    kvd = cfg.kv_dim
    for l in range(cfg.n_layers):
        p = f"blk.{l}."
        ck[p + "attn_norm.weight"] = SynthTensor(_native.GGML_F32, (cfg.dim,), ones.view(np.uint8).copy())
        ck[p + "ffn_norm.weight"] = SynthTensor(_native.GGML_F32, (cfg.dim,), ones.view(np.uint8).copy())
        ck[p + "attn_q.weight"] = tensor(q["attn"], seed, p + "attn_q.weight", cfg.dim, cfg.dim)
        ck[p + "attn_k.weight"] = tensor(q["attn"], seed, p + "attn_k.weight", kvd, cfg.dim)
        ck[p + "attn_v.weight"] = tensor(q["attn"], seed, p + "attn_v.weight", kvd, cfg.dim)
        ck[p + "attn_output.weight"] = tensor(q["attn"], seed, p + "attn_output.weight", cfg.dim, cfg.dim)
        ck[p + "ffn_gate.weight"] = tensor(q.get("gate", q.get("gate_up")), seed, p + "ffn_gate.weight",
                                           cfg.hidden_dim, cfg.dim)
        ck[p + "ffn_up.weight"] = tensor(q.get("up", q.get("gate_up")), seed, p + "ffn_up.weight",
                                         cfg.hidden_dim, cfg.dim)
        ck[p + "ffn_down.weight"] = tensor(q["down"], seed, p + "ffn_down.weight", cfg.dim, cfg.hidden_dim)
        if qkv_bias:
            for nm, n in (("attn_q.bias", cfg.dim), ("attn_k.bias", kvd), ("attn_v.bias", kvd)):
                ck[p + nm] = SynthTensor(_native.GGML_F32, (n,),
                                         normal(seed, p + nm, n, BIAS_SIGMA).view(np.uint8).copy())
    return ck


def checkpoint_bytes(ck: dict) -> int:
    return sum(int(t.data.nbytes) for t in ck.values())
