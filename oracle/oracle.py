"""ctypes wrapper of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: loaded by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker.  The product (chatnet_amd/)
never imports this module.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "liboracle.so")

F32, F16, Q4_0, Q8_0, Q4_K, Q5_K, Q6_K = 0, 1, 2, 8, 12, 13, 14
Q4_1, Q5_0, Q5_1, Q2_K, Q3_K, Q8_K = 3, 6, 7, 10, 11, 15
IQ2_XXS, IQ2_XS, IQ3_XXS, IQ1_S, IQ4_NL, IQ3_S, IQ2_S, IQ4_XS, IQ1_M = 16, 17, 18, 19, 20, 21, 22, 23, 29
_NAMES = {Q4_0: "q4_0", Q8_0: "q8_0", Q4_K: "q4_k", Q5_K: "q5_k", Q6_K: "q6_k", Q4_1: "q4_1", Q5_0: "q5_0",
          Q5_1: "q5_1", Q2_K: "q2_k", Q3_K: "q3_k", Q8_K: "q8_k", IQ2_XXS: "iq2_xxs", IQ2_XS: "iq2_xs",
          IQ3_XXS: "iq3_xxs", IQ1_S: "iq1_s", IQ4_NL: "iq4_nl", IQ3_S: "iq3_s", IQ2_S: "iq2_s", IQ4_XS: "iq4_xs",
          IQ1_M: "iq1_m"}
# IQ3_S reads 28 bytes past a tensor's last block (DequantIQ.cs:255-283): its
# buffers get this many zero bytes appended, as the device copy's tail holds.
IQ3_S_TAIL = 32


def _padded(qtype: int, data: np.ndarray) -> np.ndarray:
    d = np.ascontiguousarray(data).view(np.uint8).ravel()
    if qtype == IQ3_S:
        d = np.concatenate([d, np.zeros(IQ3_S_TAIL, np.uint8)])
    return d
_P = ctypes.c_void_p
_lib = None


class OracleConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in
                ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "head_dim", "vocab_size",
                 "context_length")] + [("rope_freq_base", ctypes.c_float), ("rms_norm_eps", ctypes.c_float),
                                       ("arch", ctypes.c_int32)]


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        L = ctypes.CDLL(LIB)
        L.oracle_set_threads.argtypes = [ctypes.c_int]
        L.oracle_get_threads.restype = ctypes.c_int
        L.oracle_half_to_float.restype = ctypes.c_float
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        for q in _NAMES.values():
            getattr(L, f"oracle_dequant_{q}").argtypes = [_P, _P, ctypes.c_int]
            getattr(L, f"oracle_dequant_{q}").restype = None
            getattr(L, f"oracle_dot_{q}").argtypes = [_P, _P, ctypes.c_int]
            getattr(L, f"oracle_dot_{q}").restype = ctypes.c_float
        L.oracle_dot_f32.argtypes = [_P, _P, ctypes.c_int]
        L.oracle_dot_f32.restype = ctypes.c_float
        L.oracle_matvec.argtypes = [ctypes.c_uint32, _P, _P, _P, ctypes.c_int, ctypes.c_int]
        L.oracle_rmsnorm.argtypes = [_P, _P, _P, ctypes.c_int, ctypes.c_float]
        L.oracle_softmax.argtypes = [_P, ctypes.c_int]
        L.oracle_silu_mul.argtypes = [_P, _P, ctypes.c_int]
        L.oracle_add.argtypes = [_P, _P, ctypes.c_int]
        L.oracle_rope.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.oracle_rope_neox.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float]
        L.oracle_argmax.argtypes = [_P, ctypes.c_int]
        L.oracle_argmax.restype = ctypes.c_int
        L.oracle_net_random_init.argtypes = [_P, ctypes.c_int32]
        L.oracle_net_random_sample.argtypes = [_P]
        L.oracle_net_random_sample.restype = ctypes.c_int32
        L.oracle_net_random_next_double.argtypes = [_P]
        L.oracle_net_random_next_double.restype = ctypes.c_double
        L.oracle_temperature_sample.argtypes = [_P, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_float,
                                                ctypes.c_float, _P]
        L.oracle_temperature_sample.restype = ctypes.c_int
        L.oracle_llama_create.argtypes = [ctypes.POINTER(OracleConfig)]
        L.oracle_llama_create.restype = _P
        L.oracle_llama_set_tensor.argtypes = [_P, ctypes.c_char_p, ctypes.c_uint32, _P]
        L.oracle_llama_forward.argtypes = [_P, _P, ctypes.c_int, ctypes.c_int, _P]
        L.oracle_llama_kv.argtypes = [_P, ctypes.c_int, ctypes.c_int, ctypes.c_int, _P]
        L.oracle_llama_destroy.argtypes = [_P]
        _lib = L
    return _lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def set_threads(n: int) -> None:
    lib().oracle_set_threads(int(n))


def half_to_float(h: int) -> float:
    return float(lib().oracle_half_to_float(h))


def dequant(qtype: int, data: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    name = _NAMES[qtype]
    d = _padded(qtype, np.ascontiguousarray(data, dtype=np.uint8))
    getattr(lib(), f"oracle_dequant_{name}")(d.ctypes.data, out.ctypes.data, n)
    return out


def dot(qtype: int, row: np.ndarray, x: np.ndarray) -> float:
    name = _NAMES[qtype]
    r = _padded(qtype, np.ascontiguousarray(row, dtype=np.uint8))
    xx = _f32(x)
    return float(getattr(lib(), f"oracle_dot_{name}")(r.ctypes.data, xx.ctypes.data, xx.size))


def matvec(qtype: int, w: np.ndarray, x: np.ndarray, M: int, K: int) -> np.ndarray:
    y = np.empty(M, dtype=np.float32)
    ww = _padded(qtype, w) if qtype == IQ3_S else np.ascontiguousarray(w)
    xx = _f32(x)
    rc = lib().oracle_matvec(qtype, ww.ctypes.data, xx.ctypes.data, y.ctypes.data, M, K)
    if rc:
        raise ValueError(f"oracle_matvec: unsupported type {qtype}")
    return y


def rmsnorm(x, w, eps):
    x, w = _f32(x), _f32(w)
    out = np.empty_like(x)
    lib().oracle_rmsnorm(x.ctypes.data, w.ctypes.data, out.ctypes.data, x.size, eps)
    return out


def softmax(x):
    x = _f32(x).copy()
    lib().oracle_softmax(x.ctypes.data, x.size)
    return x


def silu_mul(g, u):
    g, u = _f32(g).copy(), _f32(u)
    lib().oracle_silu_mul(g.ctypes.data, u.ctypes.data, g.size)
    return g


def rope(q, k, pos, head_dim, n_heads, n_kv_heads, base):
    q, k = _f32(q).copy(), _f32(k).copy()
    lib().oracle_rope(q.ctypes.data, k.ctypes.data, pos, head_dim, n_heads, n_kv_heads, base)
    return q, k


def rope_neox(q, k, pos, head_dim, n_heads, n_kv_heads, base):
    q, k = _f32(q).copy(), _f32(k).copy()
    lib().oracle_rope_neox(q.ctypes.data, k.ctypes.data, pos, head_dim, n_heads, n_kv_heads, base)
    return q, k


def argmax(logits) -> int:
    l = _f32(logits)
    return int(lib().oracle_argmax(l.ctypes.data, l.size))


class NetRandom(ctypes.Structure):
    """System.Random(seed) of the .NET BCL (the seeded compat generator)."""
    _fields_ = [("seed_array", ctypes.c_int32 * 56), ("inext", ctypes.c_int32), ("inextp", ctypes.c_int32)]

    def __init__(self, seed: int):
        super().__init__()
        lib().oracle_net_random_init(ctypes.addressof(self), int(seed))

    def sample(self) -> int:
        return int(lib().oracle_net_random_sample(ctypes.addressof(self)))

    def next_double(self) -> float:
        return float(lib().oracle_net_random_next_double(ctypes.addressof(self)))


def temperature_sample(logits, temperature: float, top_k: int, top_p: float, draw: float):
    """TemperatureSampler.Sample with the draw given: (token, margin)."""
    l = _f32(logits)
    m = ctypes.c_float()
    tok = lib().oracle_temperature_sample(l.ctypes.data, l.size, temperature, top_k, top_p, draw,
                                          ctypes.addressof(m))
    return int(tok), float(m.value)


class OracleLlama:
    """LlamaModel (LlamaModel.cs; MistralModel computes the same) or, for an
    ARCH_QWEN2 config, QwenModel (QwenModel.cs) on the CPU over borrowed host
    tensors."""

    def __init__(self, cfg, checkpoint: dict):
        c = OracleConfig(cfg.dim, cfg.hidden_dim, cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                         cfg.vocab_size, cfg.context_length, cfg.rope_freq_base, cfg.rms_norm_eps,
                         getattr(cfg, "arch", 0))
        self.cfg = cfg
        self._h = lib().oracle_llama_create(ctypes.byref(c))
        if not self._h:
            raise MemoryError("oracle_llama_create failed")
        self._keep = []
        for name, t in checkpoint.items():
            arr = _padded(t.type, t.data) if t.type == IQ3_S else np.ascontiguousarray(t.data)
            self._keep.append(arr)
            rc = lib().oracle_llama_set_tensor(self._h, name.encode(), t.type, arr.ctypes.data)
            if rc:
                raise KeyError(name)

    def forward(self, tokens, position: int) -> np.ndarray:
        t = np.ascontiguousarray(np.asarray(tokens, dtype=np.int32).ravel())
        logits = np.empty(self.cfg.vocab_size, dtype=np.float32)
        rc = lib().oracle_llama_forward(self._h, t.ctypes.data, t.size, position, logits.ctypes.data)
        if rc:
            raise RuntimeError(f"oracle forward failed: {rc}")
        return logits

    def kv(self, layer: int, position: int, which: int) -> np.ndarray:
        out = np.empty(self.cfg.kv_dim, dtype=np.float32)
        if lib().oracle_llama_kv(self._h, layer, position, which, out.ctypes.data):
            raise IndexError("kv out of range")
        return out

    def generate_greedy(self, prompt, max_tokens: int):
        """InferenceEngine.cs:234-307 with a greedy sampler and no EOS stop.
        Returns (tokens, per-step top1-top2 margins)."""
        cfg = self.cfg
        logits = None
        for i, tok in enumerate(prompt):
            logits = self.forward([tok], i)
        out, margins = [], []
        nxt = argmax(logits)
        margins.append(_margin(logits))
        pos = len(prompt)
        while len(out) < max_tokens:
            out.append(nxt)
            if pos >= cfg.context_length - 1:
                break
            logits = self.forward([nxt], pos)
            pos += 1
            nxt = argmax(logits)
            margins.append(_margin(logits))
        return out, margins

    def close(self):
        if self._h:
            lib().oracle_llama_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def _margin(logits) -> float:
    top2 = np.partition(np.asarray(logits), -2)[-2:]
    return float(abs(top2[1] - top2[0]))
