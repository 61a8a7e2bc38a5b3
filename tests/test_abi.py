"""CPU-side checks of the C ABI: the library loads, exports every symbol the
header declares, sizes follow GgufTensorInfo.ByteSize, and host-side errors
are reported without touching a GPU."""
import ctypes
import os
import re

import numpy as np
import pytest

from chatnet_amd import TINY_TEST, _native, synth
from chatnet_amd.engine import GreedySampler

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def header_functions():
    with open(os.path.join(ROOT, "include", "chatnet_hip.h")) as f:
        text = f.read()
    return re.findall(r"CHATNET_API\s+[\w\s\*]+?\b(chatnet_\w+)\s*\(", text)


def test_library_exports_every_declared_symbol():
    lib = _native.hip_lib()
    names = header_functions()
    assert len(names) >= 10
    for n in names:
        assert hasattr(lib, n), n
    assert set(names) == set(_native._SIGNATURES), "ctypes signatures out of sync with the header"


def test_exported_symbols_are_only_the_abi():
    import subprocess

    out = subprocess.run(["nm", "-D", "--defined-only", _native.lib_path()], capture_output=True, text=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    chatnet = {s for s in exported if s.startswith("chatnet_")}
    assert chatnet == set(header_functions())


def test_byte_size_table():  # QuantizationTests.cs:642-698
    cases = [(0, 1, 4), (1, 1, 2), (2, 32, 18), (3, 32, 20), (6, 32, 22), (7, 32, 24), (8, 32, 34),
             (10, 256, 84), (11, 256, 110), (12, 256, 144), (13, 256, 176), (14, 256, 210), (15, 256, 292),
             (20, 32, 18), (23, 256, 136), (21, 256, 110), (18, 256, 98), (17, 256, 74), (16, 256, 66),
             (22, 256, 82), (19, 256, 50), (29, 256, 56)]
    for t, blk, bpb in cases:
        elements = 1024 if blk == 1 else blk * 4
        want = elements * bpb if blk == 1 else ((elements + blk - 1) // blk) * bpb
        assert _native.tensor_nbytes(t, elements) == want, t
    assert _native.tensor_nbytes(2, 33) == 36  # partial block rounds up
    assert _native.tensor_nbytes(999, 32) == 0


def test_create_without_device_reports_no_device():
    from chatnet_amd import hiprt

    if hiprt.device_count() > 0:
        pytest.skip("a GPU is visible")
    with pytest.raises(_native.ChatnetNoDevice):
        from chatnet_amd import HipLlamaModel
        HipLlamaModel(TINY_TEST)


def test_create_rejects_bad_config():
    lib = _native.hip_lib()
    h = ctypes.c_void_p()
    c = TINY_TEST.replace(n_kv_heads=3).to_c()
    assert lib.chatnet_create(ctypes.byref(c), 0, ctypes.byref(h)) == _native.ERR_INVALID_ARG
    assert b"multiple" in lib.chatnet_last_error()
    c = TINY_TEST.replace(head_dim=48, dim=48 * 8).to_c()
    assert lib.chatnet_create(ctypes.byref(c), 0, ctypes.byref(h)) == _native.ERR_INVALID_ARG
    assert lib.chatnet_create(None, 0, ctypes.byref(h)) == _native.ERR_INVALID_ARG


def test_matmul_rejects_bad_arguments_before_launch():
    lib = _native.hip_lib()
    assert lib.chatnet_matmul(2, None, None, None, 4, 64, 1, None) == _native.ERR_INVALID_ARG
    fake = ctypes.c_void_p(16)
    # Q8_1 (9) is not a weight type MatVecMulByType dispatches (LlamaModel.cs:474-566)
    assert lib.chatnet_matmul(9, fake, fake, fake, 4, 64, 1, None) == _native.ERR_UNSUPPORTED_TYPE
    assert lib.chatnet_matmul(2, fake, fake, fake, 4, 48, 1, None) == _native.ERR_INVALID_ARG
    assert lib.chatnet_matmul(12, fake, fake, fake, 4, 128, 1, None) == _native.ERR_INVALID_ARG
    # block multiples of the types read as packed units: 64 for Q4_1/Q5_0/Q5_1, 256 for Q2_K/Q3_K/Q8_K
    assert lib.chatnet_matmul(3, fake, fake, fake, 4, 96, 1, None) == _native.ERR_INVALID_ARG
    assert lib.chatnet_matmul(10, fake, fake, fake, 4, 128, 1, None) == _native.ERR_INVALID_ARG
    assert lib.chatnet_matmul(15, fake, fake, fake, 4, 16640, 1, None) == _native.ERR_INVALID_ARG


def test_greedy_sampler_host_mirror():
    s = GreedySampler()
    assert s.sample(np.array([1, 5, 5, 2], np.float32)) == 1
    assert s.sample(np.array([np.nan, 5, 9], np.float32)) == 0
    assert s.sample(np.array([1, np.nan, 9, 9], np.float32)) == 2
    assert s.sample(np.array([-np.inf, -np.inf], np.float32)) == 0
    assert s.sample(np.array([3, 1, 2], np.float32)) == 0


def test_synth_is_deterministic_and_quantizers_round_trip():
    import npref

    a = synth.tensor(2, 5, "det", 8, 256)
    b = synth.tensor(2, 5, "det", 8, 256)
    assert np.array_equal(a.data, b.data)
    assert not np.array_equal(a.data, synth.tensor(2, 6, "det", 8, 256).data)
    w = synth.normal(5, "det", 8 * 256, synth.SIGMA).astype(np.float64)
    for q, tol in ((2, 0.6), (12, 1.1), (14, 0.6)):
        t = synth.tensor(q, 5, "det", 8, 256)
        err = np.abs(npref.matrix(t).ravel() - w)
        # each element is within about one quantization step of the truth
        assert np.max(err) < tol * np.max(np.abs(w)) / 4, q
    # normal() and tensor() draw the same stream
    assert np.allclose(npref.matrix(synth.tensor(0, 5, "det", 8, 256)).ravel(), w)


def test_float_to_half_matches_numpy():
    vals = np.concatenate([synth.normal(9, "h", 5000, 1.0) * s for s in (1e-7, 1e-5, 1e-3, 1.0, 1e3, 6e4)])
    vals = np.concatenate([vals, np.array([65504, 65519.99, 65520, 1e9, -0.0, 2.0 ** -25, 2.0 ** -24], np.float32)])
    with np.errstate(over="ignore"):  # values past 65520 round to inf, on purpose
        for v in vals.astype(np.float32):
            assert synth.float_to_half(float(v)) == int(np.float16(v).view(np.uint16)), v
