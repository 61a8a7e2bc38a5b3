"""GGUF writer and reader (chatnet_amd.gguf) against the rules of the
reference's GgufReader (src/ChatNet.Core/Gguf/GgufReader.cs).

The hand-packed file below is built with struct, not with the writer, and its
expected config follows ExtractModelConfig (GgufReader.cs:80-182) read as
text: arch keys first, bare keys as fallback, GetInt32 accepting only
int32/uint32/int64/uint64 (GgufMetadata.cs:53-63), GetArchFloat trying
float32, float64, uint32, int32 (GgufReader.cs:95-112)."""
import os
import struct
import subprocess
import sys

import numpy as np
import pytest

from chatnet_amd import TINY_TEST, _native, gguf, synth

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _s(x: str) -> bytes:
    b = x.encode()
    return struct.pack("<Q", len(b)) + b


def _kv(key, t, payload: bytes) -> bytes:
    return _s(key) + struct.pack("<I", t) + payload


def _handmade(version=2, magic=0x46554747, alignment=64, extra_kv=()):
    kvs = [
        _kv("general.architecture", 8, _s("llama")),
        _kv("llama.embedding_length", 10, struct.pack("<Q", 128)),       # uint64: accepted
        _kv("llama.attention.head_count", 5, struct.pack("<i", 4)),       # int32
        _kv("llama.block_count", 2, struct.pack("<H", 3)),                # uint16: not an int32 source
        _kv("block_count", 4, struct.pack("<I", 5)),                      # bare-key fallback
        _kv("llama.rope.freq_base", 4, struct.pack("<I", 500000)),        # uint32 as float
        _kv("llama.attention.layer_norm_rms_epsilon", 12, struct.pack("<d", 1e-6)),  # float64
        _kv("llama.vocab_size", 4, struct.pack("<I", 300)),
        _kv("general.alignment", 4, struct.pack("<I", alignment)),
        _kv("x.u8s", 9, struct.pack("<IQ", 0, 3) + bytes([1, 2, 255])),
        _kv("x.flag", 7, b"\x01"),
        _kv("x.i64", 11, struct.pack("<q", -7)),
        _kv("x.nested", 9, struct.pack("<IQ", 9, 2) + struct.pack("<IQ", 6, 1) + struct.pack("<f", 1.5)
            + struct.pack("<IQ", 8, 1) + _s("ab")),
        *extra_kv,
    ]
    f32 = np.arange(8, dtype=np.float32)
    q8 = np.arange(68, dtype=np.uint8)          # Q8_0, 64 elements: 2 blocks x 34 B
    tinfo = (_s("a.f32") + struct.pack("<I", 2) + struct.pack("<QQ", 4, 2) + struct.pack("<IQ", 0, 0)
             + _s("b.q8_0") + struct.pack("<I", 1) + struct.pack("<Q", 64) + struct.pack("<IQ", 8, alignment))
    head = struct.pack("<IIQQ", magic, version, 2, len(kvs)) + b"".join(kvs) + tinfo
    start = (len(head) + alignment - 1) // alignment * alignment
    body = head + b"\0" * (start - len(head)) + f32.tobytes() + b"\0" * (alignment - 32) + q8.tobytes()
    return body, f32, q8, start


def test_handmade_file_follows_extract_model_config(tmp_path):
    body, f32, q8, start = _handmade()
    p = tmp_path / "h.gguf"
    p.write_bytes(body)
    g = gguf.GgufFile(str(p))
    assert g.version == 2 and g.alignment == 64 and g.data_offset == start
    c = g.config()
    assert (c.dim, c.n_heads, c.n_kv_heads, c.head_dim) == (128, 4, 4, 32)   # kv heads default to heads
    assert c.n_layers == 5                                                   # uint16 skipped, bare key used
    assert (c.hidden_dim, c.context_length) == (5632, 2048)                  # defaults
    assert c.vocab_size == 300                                               # no token array
    assert c.rope_freq_base == 500000.0
    assert c.rms_norm_eps == float(np.float32(1e-6))
    assert list(g.metadata["x.u8s"].value) == [1, 2, 255]
    assert g.metadata["x.flag"].value is True and g.metadata["x.i64"].value == -7
    nested = g.metadata["x.nested"].value
    assert float(nested[0].value[0]) == 1.5 and nested[1].value == ["ab"]
    assert np.array_equal(g.tensor_bytes("a.f32").view(np.float32), f32)
    assert g.tensor_info("b.q8_0").nbytes == 68                              # ByteSize: 2 blocks x 34
    assert np.array_equal(g.tensor_bytes("b.q8_0"), q8)
    assert g.has_tensor("a.f32") and not g.has_tensor("c")
    with pytest.raises(_native.ChatnetKeyNotFound):
        g.tensor_info("c")


@pytest.mark.parametrize("kw,msg", [
    (dict(magic=0x46554746), "magic"),
    (dict(version=1), "version"),
    (dict(version=4), "version"),
])
def test_header_errors(tmp_path, kw, msg):
    body = _handmade(**kw)[0]
    p = tmp_path / "bad.gguf"
    p.write_bytes(body)
    with pytest.raises(gguf.GgufError, match=msg):
        gguf.GgufFile(str(p))


def test_truncated_and_oversized_strings(tmp_path):
    body = _handmade()[0]
    p = tmp_path / "t.gguf"
    p.write_bytes(body[:40])
    with pytest.raises(gguf.GgufError):
        gguf.GgufFile(str(p))
    p.write_bytes(struct.pack("<IIQQ", 0x46554747, 3, 0, 1) + struct.pack("<Q", 1_000_001))
    with pytest.raises(gguf.GgufError, match="too large"):
        gguf.GgufFile(str(p))
    body = _handmade()[0]
    p.write_bytes(body[:-10])   # tensor data cut short
    with pytest.raises(gguf.GgufError, match="past the end"):
        gguf.GgufFile(str(p))


def test_unsupported_models_are_refused(tmp_path):
    body = _handmade(extra_kv=[_kv("llama.rope.dimension_count", 4, struct.pack("<I", 16))])[0]
    p = tmp_path / "partial.gguf"
    p.write_bytes(body)
    with pytest.raises(_native.ChatnetNotSupported):
        gguf.GgufFile(str(p)).config()
    body = _handmade(extra_kv=[_kv("general.architecture", 8, _s("phi3"))])[0]   # a later key wins
    p.write_bytes(body)
    with pytest.raises(_native.ChatnetNotSupported):
        gguf.GgufFile(str(p)).config()


@pytest.mark.parametrize("mix,alignment", [("q4_0", 32), ("q4_k_m", 64)])
def test_round_trip(tmp_path, mix, alignment):
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=7, mix=mix)
    p = str(tmp_path / "m.gguf")
    gguf.write_llama(p, cfg, ck, alignment=alignment)
    with open(p, "rb") as f:
        assert struct.unpack("<IIQQ", f.read(24)) == (0x46554747, 3, len(ck), len(gguf.llama_metadata(cfg)))
    g = gguf.GgufFile(p)
    assert g.config() == cfg.replace(rms_norm_eps=float(np.float32(cfg.rms_norm_eps)))
    assert g.alignment == alignment and g.data_offset % alignment == 0
    assert [t.name for t in g.tensors] == list(ck)
    for t in g.tensors:
        assert t.offset % alignment == 0
        src = ck[t.name]
        assert t.type == src.type and t.dims == tuple(src.dims)
        assert np.array_equal(g.tensor_bytes(t.name), np.asarray(src.data).view(np.uint8).ravel())
    toks = g.get_string_array("tokenizer.ggml.tokens")
    assert len(toks) == cfg.vocab_size and toks[:3] == ["<unk>", "<s>", "</s>"] and toks[3] == "<0x00>"
    assert g.get_int("tokenizer.ggml.eos_token_id", 0) == 2


@pytest.mark.parametrize("architecture,variant", [("mistral", _native.ARCH_LLAMA), ("qwen2", _native.ARCH_QWEN2),
                                                  ("Qwen", _native.ARCH_QWEN2)])
def test_variants_round_trip(tmp_path, architecture, variant):
    # ModelFactory.DetectArchitecture (ModelFactory.cs:23-39) lower-cases the name;
    # ExtractModelConfig reads the keys under the name as written (GgufReader.cs:82-110)
    cfg = TINY_TEST.replace(arch=variant, rope_freq_base=1e6)
    ck = synth.llama_checkpoint(cfg, seed=8, mix="q8_0", with_output=False, embedding=_native.GGML_Q8_0)
    assert ("blk.0.attn_q.bias" in ck) == (variant == _native.ARCH_QWEN2)
    p = str(tmp_path / "v.gguf")
    gguf.write_llama(p, cfg, ck, architecture=architecture)
    g = gguf.GgufFile(p)
    assert g.get_string("general.architecture") == architecture
    assert g.get_int(f"{architecture}.block_count", -1) == cfg.n_layers
    assert g.config() == cfg.replace(rms_norm_eps=float(np.float32(cfg.rms_norm_eps)))
    assert not g.has_tensor("output.weight")
    for t in g.tensors:
        assert np.array_equal(g.tensor_bytes(t.name), np.asarray(ck[t.name].data).view(np.uint8).ravel())
    with pytest.raises(ValueError):   # a Qwen2 config under a Llama name, or the reverse
        gguf.llama_metadata(cfg, architecture="llama" if variant == _native.ARCH_QWEN2 else "qwen2")


def test_unknown_architecture_defaults_to_llama(tmp_path, capsys):
    # ModelFactory.cs:36-37: an unknown name runs LlamaModel after a warning
    body = _handmade(extra_kv=[_kv("general.architecture", 8, _s("yi"))])[0]
    p = tmp_path / "yi.gguf"
    p.write_bytes(body)
    cfg = gguf.GgufFile(str(p)).config()
    assert cfg.arch == _native.ARCH_LLAMA
    assert "Unknown architecture 'yi', defaulting to Llama" in capsys.readouterr().err


def test_writer_rejects_wrong_sizes(tmp_path):
    t = synth.SynthTensor(_native.GGML_Q4_0, (64, 2), np.zeros(35, np.uint8))   # ByteSize is 72
    with pytest.raises(ValueError):
        gguf.write(str(tmp_path / "x.gguf"), {"w": t}, {})


def test_cli_write_and_info(tmp_path):
    out = str(tmp_path / "cli.gguf")
    env = dict(os.environ, PYTHONPATH=REPO)
    subprocess.run([sys.executable, "-m", "chatnet_amd.gguf", "write", out, "--model", "tiny-test", "--mix",
                    "q4_k_m", "--seed", "3"], check=True, cwd=REPO, env=env, capture_output=True)
    r = subprocess.run([sys.executable, "-m", "chatnet_amd.gguf", "info", out], check=True, cwd=REPO, env=env,
                       capture_output=True, text=True)
    assert "blk.1.ffn_down.weight" in r.stdout and "n_layers=2" in r.stdout
