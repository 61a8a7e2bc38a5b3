"""ctypes bindings of the in-tree native libraries.

libchatnet_hip.so is the product: every compute call goes through it, and a
missing or stale library raises instead of falling back to anything else.
"""
from __future__ import annotations

import ctypes
import os

LIBDIR = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib")

# chatnet_status (include/chatnet_hip.h)
OK = 0
ERR_INVALID_ARG = -1
ERR_NOT_FOUND = -2
ERR_UNSUPPORTED_TYPE = -3
ERR_SIZE_MISMATCH = -4
ERR_OUT_OF_RANGE = -5
ERR_NO_DEVICE = -6
ERR_HIP = -7
ERR_OUT_OF_MEMORY = -8

GGML_F32 = 0
GGML_F16 = 1
GGML_Q4_0 = 2
GGML_Q8_0 = 8
GGML_Q4_K = 12
GGML_Q5_K = 13
GGML_Q6_K = 14
GGML_Q4_1 = 3
GGML_Q5_0 = 6
GGML_Q5_1 = 7
GGML_Q2_K = 10
GGML_Q3_K = 11
GGML_Q8_K = 15
GGML_IQ2_XXS = 16
GGML_IQ2_XS = 17
GGML_IQ3_XXS = 18
GGML_IQ1_S = 19
GGML_IQ4_NL = 20
GGML_IQ3_S = 21
GGML_IQ2_S = 22
GGML_IQ4_XS = 23
GGML_IQ1_M = 29

KV_F32 = 0
KV_F16 = 1

# forward-pass variant (chatnet_config.arch)
ARCH_LLAMA = 0   # LlamaModel; MistralModel computes the same
ARCH_QWEN2 = 1   # QwenModel: optional QKV biases, split-half (NeoX) RoPE


class ChatnetError(RuntimeError):
    """Base class of errors raised from libchatnet_hip status codes."""

    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


class ChatnetArgumentError(ChatnetError, ValueError):
    """ArgumentException."""


class ChatnetKeyNotFound(ChatnetError, KeyError):
    """KeyNotFoundException (missing tensor)."""


class ChatnetNotSupported(ChatnetError, NotImplementedError):
    """NotSupportedException (unsupported ggml type)."""


class ChatnetSizeMismatch(ChatnetError, ValueError):
    """Tensor byte size differs from GgufTensorInfo.ByteSize."""


class ChatnetOutOfRange(ChatnetError, IndexError):
    """IndexOutOfRangeException (position / token id)."""


class ChatnetNoDevice(ChatnetError):
    """No usable HIP device."""


class ChatnetHipError(ChatnetError):
    """A HIP runtime call failed."""


class ChatnetOutOfMemory(ChatnetError, MemoryError):
    """Device allocation failed."""


_ERRORS = {
    ERR_INVALID_ARG: ChatnetArgumentError,
    ERR_NOT_FOUND: ChatnetKeyNotFound,
    ERR_UNSUPPORTED_TYPE: ChatnetNotSupported,
    ERR_SIZE_MISMATCH: ChatnetSizeMismatch,
    ERR_OUT_OF_RANGE: ChatnetOutOfRange,
    ERR_NO_DEVICE: ChatnetNoDevice,
    ERR_HIP: ChatnetHipError,
    ERR_OUT_OF_MEMORY: ChatnetOutOfMemory,
}


class ChatnetConfig(ctypes.Structure):
    """chatnet_config (mirrors LlamaConfig, LlamaConfig.cs:8-38)."""

    _fields_ = [
        ("dim", ctypes.c_int32),
        ("hidden_dim", ctypes.c_int32),
        ("n_layers", ctypes.c_int32),
        ("n_heads", ctypes.c_int32),
        ("n_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("vocab_size", ctypes.c_int32),
        ("context_length", ctypes.c_int32),
        ("rope_freq_base", ctypes.c_float),
        ("rms_norm_eps", ctypes.c_float),
        ("kv_dtype", ctypes.c_int32),
        ("arch", ctypes.c_int32),
    ]


# name -> (restype, argtypes); must match include/chatnet_hip.h
_P = ctypes.c_void_p
_SIGNATURES = {
    "chatnet_create": (ctypes.c_int, [ctypes.POINTER(ChatnetConfig), ctypes.c_int, ctypes.POINTER(_P)]),
    "chatnet_upload_tensor": (
        ctypes.c_int,
        [_P, ctypes.c_char_p, ctypes.c_uint32, ctypes.POINTER(ctypes.c_uint64), ctypes.c_int, _P, ctypes.c_uint64],
    ),
    "chatnet_forward": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int32), ctypes.c_int, ctypes.c_int, _P]),
    "chatnet_argmax": (ctypes.c_int, [_P, ctypes.POINTER(ctypes.c_int32)]),
    "chatnet_generate_greedy": (
        ctypes.c_int,
        [_P, ctypes.POINTER(ctypes.c_int32), ctypes.c_int, ctypes.c_int, ctypes.c_int32,
         ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int)],
    ),
    "chatnet_decode_greedy": (
        ctypes.c_int,
        [_P, ctypes.c_int, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int)],
    ),
    "chatnet_sample": (
        ctypes.c_int, [_P, ctypes.c_float, ctypes.c_int, ctypes.c_float, ctypes.c_float, ctypes.POINTER(ctypes.c_int32)],
    ),
    "chatnet_generate_sampled": (
        ctypes.c_int,
        [_P, ctypes.POINTER(ctypes.c_int32), ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_float,
         ctypes.c_int32, ctypes.c_int32, ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int)],
    ),
    "chatnet_net_random": (ctypes.c_int, [ctypes.c_int32, ctypes.c_int, _P]),
    "chatnet_get_logits": (ctypes.c_int, [_P, _P]),
    "chatnet_matmul": (
        ctypes.c_int,
        [ctypes.c_uint32, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P],
    ),
    "chatnet_matmul_noalloc": (
        ctypes.c_int,
        [ctypes.c_uint32, _P, _P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P],
    ),
    "chatnet_tensor_nbytes": (ctypes.c_uint64, [ctypes.c_uint32, ctypes.c_uint64]),
    "chatnet_destroy": (None, [_P]),
    "chatnet_last_error": (ctypes.c_char_p, []),
}

_hip = None
_synth = None


def lib_path(name: str = "libchatnet_hip.so") -> str:
    return os.path.join(LIBDIR, name)


def hip_lib() -> ctypes.CDLL:
    """Loads libchatnet_hip.so (built by chatnet_amd.build_lib); raises if absent."""
    global _hip
    if _hip is None:
        path = lib_path("libchatnet_hip.so")
        if not os.path.exists(path):
            raise ImportError(
                f"{path} is missing: build it with `python -m chatnet_amd.build_lib` "
                "(there is no fallback path)"
            )
        lib = ctypes.CDLL(path)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _hip = lib
    return _hip


def synth_lib() -> ctypes.CDLL:
    global _synth
    if _synth is None:
        path = lib_path("libchatnet_synth.so")
        if not os.path.exists(path):
            raise ImportError(f"{path} is missing: build it with `python -m chatnet_amd.build_lib`")
        lib = ctypes.CDLL(path)
        lib.chatnet_synth_stream_id.restype = ctypes.c_uint64
        lib.chatnet_synth_stream_id.argtypes = [ctypes.c_char_p]
        lib.chatnet_synth_normal.restype = None
        lib.chatnet_synth_normal.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_uint64,
                                             ctypes.c_uint64, ctypes.c_float, _P]
        lib.chatnet_synth_tokens.restype = None
        lib.chatnet_synth_tokens.argtypes = [ctypes.c_uint64, ctypes.c_uint64, ctypes.c_int, ctypes.c_int, _P]
        lib.chatnet_float_to_half.restype = ctypes.c_uint16
        lib.chatnet_float_to_half.argtypes = [ctypes.c_float]
        lib.chatnet_synth_quantize.restype = ctypes.c_uint64
        lib.chatnet_synth_quantize.argtypes = [ctypes.c_uint32, _P, ctypes.c_uint64, _P]
        lib.chatnet_synth_tensor.restype = ctypes.c_uint64
        lib.chatnet_synth_tensor.argtypes = [ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                             ctypes.c_uint64, _P]
        _synth = lib
    return _synth


def check(status: int) -> None:
    """Raises the ChatnetError subclass for a non-zero status."""
    if status == OK:
        return
    msg = hip_lib().chatnet_last_error()
    text = msg.decode("utf-8", "replace") if msg else ""
    raise _ERRORS.get(status, ChatnetError)(status, text)


def tensor_nbytes(ggml_type: int, n_elements: int) -> int:
    """GgufTensorInfo.ByteSize (GgufTensorInfo.cs:30-113)."""
    return int(hip_lib().chatnet_tensor_nbytes(ggml_type, n_elements))
