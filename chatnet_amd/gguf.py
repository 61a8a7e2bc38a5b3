"""GGUF v3 files for Llama checkpoints.

Reader — the rules of src/ChatNet.Core/Gguf/GgufReader.cs:
  Load (:34-75)              magic 0x46554747, version 2..3, u64 tensor and KV
                             counts, KV pairs, `general.alignment` (default 32,
                             GgufConstants.cs:9-15), tensor infos, data at the
                             aligned end of the header (AlignOffset :308-312)
  ReadMetadataValue (:194-212), ReadArray (:214-296)
                             value types of GgufConstants.cs:20-35; arrays are
                             u32 element type + u64 length
  ReadTensorInfo (:298-306)  name, u32 n_dims, u64 dims[n_dims], u32 type,
                             u64 offset relative to the data start
  ReadString (:364-377)      u64 length + UTF-8, at most 1 000 000 bytes
  ExtractModelConfig (:80-182) the <architecture>.* keys with bare-key fallbacks and the
                             defaults below; vocabulary size from the
                             tokenizer.ggml.tokens array when present
  GgufMetadata.GetInt32 (GgufMetadata.cs:53-63) accepts int32, uint32, int64
                             and uint64 values only; GetArchFloat
                             (GgufReader.cs:95-112) float32, float64, uint32,
                             int32 in that order.
Tensor bytes are GgufTensorInfo.ByteSize (GgufTensorInfo.cs:30-113) at
data_offset + offset (MemoryMappedWeights.GetTensorData,
MemoryMappedWeights.cs:48-57), mapped read-only, never copied on the host.

Writer — the metadata the reference needs to load the file unchanged through
InferenceEngine.LoadFromGguf (InferenceEngine.cs:57-110): general.architecture
("llama", "mistral" or "qwen2"), the shape keys under that prefix, and a tokenizer vocabulary
(BpeTokenizer.cs:96-117: tokens, scores, token types, BOS/EOS ids, model
"llama"); tensors in the order given, each at an offset aligned to the file's
alignment.

    python -m chatnet_amd.gguf write OUT.gguf --model tinyllama --mix q4_0 --seed 1234
    python -m chatnet_amd.gguf write OUT.gguf --model qwen2-0.5b --mix q8_0 --tied
    python -m chatnet_amd.gguf info FILE.gguf
"""
from __future__ import annotations

import argparse
import dataclasses
import struct
import sys
from typing import Dict, List, Mapping, Optional, Tuple

import numpy as np

from . import _native
from .config import LLAMA2_7B, QWEN2_0_5B, TINY_TEST, TINYLLAMA_1B, LlamaConfig

MAGIC = 0x46554747
VERSION = 3
DEFAULT_ALIGNMENT = 32
MAX_STRING = 1_000_000

# GgufMetadataValueType (GgufConstants.cs:20-35)
UINT8, INT8, UINT16, INT16, UINT32, INT32, FLOAT32, BOOL, STRING, ARRAY, UINT64, INT64, FLOAT64 = range(13)

_SCALAR = {UINT8: "<B", INT8: "<b", UINT16: "<H", INT16: "<h", UINT32: "<I", INT32: "<i", FLOAT32: "<f",
           BOOL: "<B", UINT64: "<Q", INT64: "<q", FLOAT64: "<d"}


class GgufError(ValueError):
    """InvalidDataException / EndOfStreamException of GgufReader."""


@dataclasses.dataclass(frozen=True)
class Value:
    """A metadata value with its GGUF type (arrays: `elem` is the element type)."""
    type: int
    value: object
    elem: Optional[int] = None


@dataclasses.dataclass(frozen=True)
class TensorInfo:
    name: str
    dims: Tuple[int, ...]   # GGUF order, ne0 first
    type: int
    offset: int             # relative to the data start

    @property
    def n_elements(self) -> int:
        n = 1
        for d in self.dims:
            n *= int(d)
        return n

    @property
    def nbytes(self) -> int:
        return _native.tensor_nbytes(self.type, self.n_elements)


@dataclasses.dataclass
class GgufTensor:
    """Raw tensor bytes as the model uploads them (the shape of synth.SynthTensor)."""
    type: int
    dims: tuple
    data: np.ndarray


def _align(offset: int, alignment: int) -> int:
    return (offset + alignment - 1) // alignment * alignment


# --------------------------------------------------------------------------
# reading

class _Cursor:
    def __init__(self, buf):
        self.buf = buf
        self.pos = 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.buf):
            raise GgufError("unexpected end of GGUF header")
        b = bytes(self.buf[self.pos:self.pos + n])
        self.pos += n
        return b

    def scalar(self, t: int):
        fmt = _SCALAR[t]
        v = struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]
        return bool(v) if t == BOOL else v

    def string(self) -> str:
        n = self.scalar(UINT64)
        if n > MAX_STRING:
            raise GgufError(f"GGUF string length too large: {n}")
        return self.take(n).decode("utf-8")

    def value(self, t: int) -> Value:
        if t == STRING:
            return Value(t, self.string())
        if t == ARRAY:
            et = self.scalar(UINT32)
            n = self.scalar(UINT64)
            if et == STRING:
                return Value(t, [self.string() for _ in range(n)], et)
            if et == ARRAY:
                return Value(t, [self.value(ARRAY) for _ in range(n)], et)
            if et not in _SCALAR:
                raise GgufError(f"Unknown GGUF metadata value type: {et}")
            fmt = _SCALAR[et]
            size = struct.calcsize(fmt)
            vals = np.frombuffer(self.take(size * n), dtype=np.dtype(fmt)).copy()
            return Value(t, vals, et)
        if t not in _SCALAR:
            raise GgufError(f"Unknown GGUF metadata value type: {t}")
        return Value(t, self.scalar(t))


class GgufFile:
    """A parsed GGUF file: metadata, tensor infos and read-only tensor bytes."""

    def __init__(self, path: str):
        self.path = path
        raw = np.memmap(path, dtype=np.uint8, mode="r")
        c = _Cursor(raw)
        magic = c.scalar(UINT32)
        if magic != MAGIC:
            raise GgufError(f"Invalid GGUF magic: 0x{magic:08X}, expected 0x{MAGIC:08X}")
        self.version = c.scalar(UINT32)
        if self.version < 2 or self.version > 3:
            raise GgufError(f"Unsupported GGUF version: {self.version}")
        n_tensors = c.scalar(UINT64)
        n_kv = c.scalar(UINT64)
        self.metadata: Dict[str, Value] = {}
        for _ in range(n_kv):
            key = c.string()
            t = c.scalar(UINT32)
            self.metadata[key] = c.value(t)
        self.alignment = self.get_int("general.alignment", DEFAULT_ALIGNMENT)
        if self.alignment <= 0 or self.alignment & (self.alignment - 1):
            raise GgufError(f"GGUF alignment must be a power of two, got {self.alignment}")
        self.tensors: List[TensorInfo] = []
        for _ in range(n_tensors):
            name = c.string()
            nd = c.scalar(UINT32)
            dims = tuple(c.scalar(UINT64) for _ in range(nd))
            t = c.scalar(UINT32)
            off = c.scalar(UINT64)
            self.tensors.append(TensorInfo(name, dims, t, off))
        self.data_offset = _align(c.pos, self.alignment)
        self._by_name = {t.name: t for t in self.tensors}
        self._raw = raw
        for t in self.tensors:
            if self.data_offset + t.offset + t.nbytes > raw.size:
                raise GgufError(f"tensor {t.name} extends past the end of the file")

    # -- GgufMetadata accessors ------------------------------------------
    def get_int(self, key: str, default: int) -> int:
        """GgufMetadata.GetInt32: int32/uint32/int64/uint64 values, cast to int32."""
        v = self.metadata.get(key)
        if v is None or v.type not in (INT32, UINT32, INT64, UINT64):
            return default
        x = int(v.value) & 0xFFFFFFFF
        return x - (1 << 32) if x >= 1 << 31 else x

    def _try_float(self, key: str) -> Optional[float]:
        v = self.metadata.get(key)
        if v is None or v.type not in (FLOAT32, FLOAT64, UINT32, INT32):
            return None
        return float(np.float32(v.value))

    def get_string(self, key: str, default: str = "") -> str:
        v = self.metadata.get(key)
        return v.value if v is not None and v.type == STRING else default

    def get_string_array(self, key: str) -> Optional[List[str]]:
        v = self.metadata.get(key)
        return v.value if v is not None and v.type == ARRAY and v.elem == STRING else None

    # -- GgufReader.ExtractModelConfig -------------------------------------
    def config(self, kv_dtype: int = _native.KV_F32, context_length: Optional[int] = None) -> LlamaConfig:
        arch = self.get_string("general.architecture", "llama")
        variant = architecture_variant(arch)

        def arch_int(suffix: str, default: int) -> int:
            val = self.get_int(f"{arch}.{suffix}", -1)
            return val if val >= 0 else self.get_int(suffix, default)

        def arch_float(suffix: str, default: float) -> float:
            for key in (f"{arch}.{suffix}", suffix):
                f = self._try_float(key)
                if f is not None:
                    return f
            return default

        n_heads = arch_int("attention.head_count", 32)
        n_kv = arch_int("attention.head_count_kv", n_heads)
        dim = arch_int("embedding_length", 2048)
        key_len = arch_int("attention.key_length", -1)
        head_dim = key_len if key_len > 0 else dim // n_heads
        rope_dims = arch_int("rope.dimension_count", -1)
        partial = arch_float("rope.partial_rotary_factor", 0.0)
        if (0.0 < partial < 1.0) or (0 < rope_dims < head_dim):
            raise _native.ChatnetNotSupported(_native.ERR_UNSUPPORTED_TYPE,
                                              "partial rotary embeddings are not on this path")
        tokens = self.get_string_array("tokenizer.ggml.tokens")
        vocab = len(tokens) if tokens is not None else arch_int("vocab_size", 32000)
        ctx = arch_int("context_length", 2048)
        return LlamaConfig(dim=dim, hidden_dim=arch_int("feed_forward_length", 5632),
                           n_layers=arch_int("block_count", 22), n_heads=n_heads, n_kv_heads=n_kv,
                           head_dim=head_dim, vocab_size=vocab,
                           context_length=ctx if context_length is None else int(context_length),
                           rope_freq_base=arch_float("rope.freq_base", 10000.0),
                           rms_norm_eps=arch_float("attention.layer_norm_rms_epsilon", 1e-5),
                           kv_dtype=kv_dtype, arch=variant)

    # -- tensor data ---------------------------------------------------------
    def has_tensor(self, name: str) -> bool:
        """IWeightLoader.HasTensor (IWeightLoader.cs:14)."""
        return name in self._by_name

    def tensor_info(self, name: str) -> TensorInfo:
        try:
            return self._by_name[name]
        except KeyError:
            raise _native.ChatnetKeyNotFound(_native.ERR_NOT_FOUND, f"tensor not in GGUF: {name}") from None

    def tensor_bytes(self, name: str) -> np.ndarray:
        t = self.tensor_info(name)
        start = self.data_offset + t.offset
        return self._raw[start:start + t.nbytes]

    def checkpoint(self) -> Dict[str, GgufTensor]:
        return {t.name: GgufTensor(t.type, t.dims, self.tensor_bytes(t.name)) for t in self.tensors}


# --------------------------------------------------------------------------
# writing

def _pack_string(s: str) -> bytes:
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def _pack_value(v: Value) -> bytes:
    if v.type == STRING:
        return _pack_string(v.value)
    if v.type == ARRAY:
        out = [struct.pack("<IQ", v.elem, len(v.value))]
        if v.elem == STRING:
            out += [_pack_string(s) for s in v.value]
        else:
            out.append(np.asarray(v.value, dtype=np.dtype(_SCALAR[v.elem])).tobytes())
        return b"".join(out)
    return struct.pack(_SCALAR[v.type], v.value)


def vocabulary(n: int) -> Tuple[List[str], np.ndarray, np.ndarray]:
    """A SentencePiece-shaped vocabulary of n entries: <unk>, <s>, </s>, the 256
    byte tokens <0xXX> (BpeTokenizer's byte fallback), then placeholder pieces;
    scores -i, token types unknown 2 / control 3 / byte 6 / normal 1."""
    tokens, types = [], []
    for i in range(n):
        if i == 0:
            tok, typ = "<unk>", 2
        elif i in (1, 2):
            tok, typ = ("<s>" if i == 1 else "</s>"), 3
        elif i < 259:
            tok, typ = f"<0x{i - 3:02X}>", 6
        else:
            tok, typ = f"▁t{i}", 1
        tokens.append(tok)
        types.append(typ)
    return tokens, -np.arange(n, dtype=np.float32), np.asarray(types, dtype=np.int32)


def architecture_variant(arch: str) -> int:
    """ModelFactory.DetectArchitecture (ModelFactory.cs:23-39) narrowed to the
    variants that run here: llama and mistral take LlamaModel's forward
    (MistralModel computes the same), qwen2 / qwen QwenModel's; gemma and phi
    are refused; any other name falls back to llama with the reference's
    warning."""
    a = arch.lower()
    if a in ("llama", "mistral"):
        return _native.ARCH_LLAMA
    if a in ("qwen2", "qwen"):
        return _native.ARCH_QWEN2
    if a in ("gemma", "gemma2", "phi2", "phi3", "phi"):
        raise _native.ChatnetNotSupported(_native.ERR_UNSUPPORTED_TYPE,
                                          f"architecture '{arch}': Gemma and Phi do not run on this path")
    print(f"[WARN] Unknown architecture '{arch}', defaulting to Llama.", file=sys.stderr)
    return _native.ARCH_LLAMA


def llama_metadata(cfg: LlamaConfig, name: str = "chatnet-synthetic",
                   alignment: int = DEFAULT_ALIGNMENT, architecture: Optional[str] = None) -> Dict[str, Value]:
    """Metadata of a checkpoint of `cfg`; the keys carry the architecture
    prefix ("llama" or, for ARCH_QWEN2, "qwen2" unless `architecture` names
    another, e.g. "mistral")."""
    arch = architecture or ("qwen2" if cfg.arch == _native.ARCH_QWEN2 else "llama")
    if architecture_variant(arch) != cfg.arch:
        raise ValueError(f"architecture '{arch}' does not match the config's variant {cfg.arch}")
    tokens, scores, types = vocabulary(cfg.vocab_size)
    md = {
        "general.architecture": Value(STRING, arch),
        "general.name": Value(STRING, name),
        "general.alignment": Value(UINT32, alignment),
        f"{arch}.context_length": Value(UINT32, cfg.context_length),
        f"{arch}.embedding_length": Value(UINT32, cfg.dim),
        f"{arch}.block_count": Value(UINT32, cfg.n_layers),
        f"{arch}.feed_forward_length": Value(UINT32, cfg.hidden_dim),
        f"{arch}.attention.head_count": Value(UINT32, cfg.n_heads),
        f"{arch}.attention.head_count_kv": Value(UINT32, cfg.n_kv_heads),
        f"{arch}.attention.key_length": Value(UINT32, cfg.head_dim),
        f"{arch}.attention.value_length": Value(UINT32, cfg.head_dim),
        f"{arch}.rope.dimension_count": Value(UINT32, cfg.head_dim),
        f"{arch}.rope.freq_base": Value(FLOAT32, float(cfg.rope_freq_base)),
        f"{arch}.attention.layer_norm_rms_epsilon": Value(FLOAT32, float(cfg.rms_norm_eps)),
        f"{arch}.vocab_size": Value(UINT32, cfg.vocab_size),
        "tokenizer.ggml.model": Value(STRING, "llama"),
        "tokenizer.ggml.tokens": Value(ARRAY, tokens, STRING),
        "tokenizer.ggml.scores": Value(ARRAY, scores, FLOAT32),
        "tokenizer.ggml.token_type": Value(ARRAY, types, INT32),
        "tokenizer.ggml.bos_token_id": Value(UINT32, 1),
        "tokenizer.ggml.eos_token_id": Value(UINT32, 2),
    }
    return md


def write(path: str, tensors: Mapping, metadata: Mapping[str, Value],
          alignment: int = DEFAULT_ALIGNMENT) -> None:
    """Writes a GGUF v3 file: `tensors` maps name -> object with .type, .dims
    (GGUF order) and .data (raw bytes of exactly ByteSize)."""
    if alignment <= 0 or alignment & (alignment - 1):
        raise ValueError("alignment must be a power of two")
    infos, blobs, off = [], [], 0
    for name, t in tensors.items():
        data = np.ascontiguousarray(t.data).view(np.uint8).ravel()
        info = TensorInfo(name, tuple(int(d) for d in t.dims), int(t.type), off)
        if data.nbytes != info.nbytes:
            raise ValueError(f"{name}: {data.nbytes} bytes, ByteSize says {info.nbytes}")
        infos.append(info)
        blobs.append(data)
        off = _align(off + data.nbytes, alignment)
    head = [struct.pack("<IIQQ", MAGIC, VERSION, len(infos), len(metadata))]
    for key, v in metadata.items():
        head += [_pack_string(key), struct.pack("<I", v.type), _pack_value(v)]
    for info in infos:
        head += [_pack_string(info.name), struct.pack("<I", len(info.dims)),
                 struct.pack(f"<{len(info.dims)}Q", *info.dims), struct.pack("<IQ", info.type, info.offset)]
    header = b"".join(head)
    data_start = _align(len(header), alignment)
    with open(path, "wb") as f:
        f.write(header)
        f.write(b"\0" * (data_start - len(header)))
        pos = 0
        for info, data in zip(infos, blobs):
            f.write(b"\0" * (info.offset - pos))
            f.write(data.tobytes())
            pos = info.offset + data.nbytes


def write_llama(path: str, cfg: LlamaConfig, checkpoint: Mapping, name: str = "chatnet-synthetic",
                alignment: int = DEFAULT_ALIGNMENT, architecture: Optional[str] = None) -> None:
    """A Llama / Mistral / Qwen2 checkpoint (name -> tensor, e.g.
    synth.llama_checkpoint) as GGUF."""
    write(path, checkpoint, llama_metadata(cfg, name, alignment, architecture), alignment)


# --------------------------------------------------------------------------

_MODELS = {"tinyllama": TINYLLAMA_1B, "llama2-7b": LLAMA2_7B, "tiny-test": TINY_TEST,
           "qwen2-0.5b": QWEN2_0_5B, "tiny-qwen2": TINY_TEST.replace(arch=_native.ARCH_QWEN2)}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m chatnet_amd.gguf")
    sub = ap.add_subparsers(dest="cmd", required=True)
    w = sub.add_parser("write", help="write a seeded synthetic Llama checkpoint as GGUF")
    w.add_argument("out")
    w.add_argument("--model", choices=sorted(_MODELS), default="tinyllama")
    w.add_argument("--mix", default="q4_0", help="q4_0, q8_0, q4_k_m, q5_k_m, q4_k or q6_k")
    w.add_argument("--architecture", default=None, help="general.architecture (e.g. mistral); "
                   "default llama, or qwen2 for the Qwen2 models")
    w.add_argument("--tied", action="store_true",
                   help="no output.weight: Q8_0 token embeddings double as the LM head")
    w.add_argument("--seed", type=int, default=1234)
    w.add_argument("--layers", type=int, default=None, help="override the layer count")
    i = sub.add_parser("info", help="print the config and tensor table of a GGUF file")
    i.add_argument("path")
    a = ap.parse_args(argv)
    if a.cmd == "write":
        from . import synth
        cfg = _MODELS[a.model]
        if a.layers is not None:
            cfg = cfg.replace(n_layers=a.layers)
        emb = _native.GGML_Q8_0 if a.tied else _native.GGML_F32
        ck = synth.llama_checkpoint(cfg, seed=a.seed, mix=a.mix, with_output=not a.tied, embedding=emb)
        write_llama(a.out, cfg, ck, name=f"{a.model}-{a.mix}-seed{a.seed}", architecture=a.architecture)
        print(f"wrote {a.out}: {len(ck)} tensors")
    else:
        g = GgufFile(a.path)
        print(g.config())
        print(f"version {g.version}, alignment {g.alignment}, data at {g.data_offset}")
        for t in g.tensors:
            print(f"{t.name:40s} type {t.type:2d} dims {t.dims} offset {t.offset} bytes {t.nbytes}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
