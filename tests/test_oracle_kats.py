"""Pins the CPU oracle before it is trusted as the parity checker.

Known-answer vectors come from the reference's own tests
(tests/ChatNet.Tests/QuantizationTests.cs), closed forms and hand-derived
byte-position cases; random blocks are checked against the independent
float64 restatement in npref.py.
"""
import numpy as np
import pytest

import npref
import oracle
from chatnet_amd import synth


def h16(f: float) -> bytes:
    """QuantizationTests.WriteHalf (:768-773): fp32 -> System.Half -> LE bytes."""
    return np.array([f], dtype=np.float16).view(np.uint16).astype("<u2").tobytes()


# ---------------------------------------------------------------- half -> float
def test_half_to_float_all_65536_inputs():
    bits = np.arange(65536, dtype=np.uint32)
    want = bits.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([oracle.half_to_float(int(b)) for b in bits], dtype=np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
    # subnormal KATs: smallest subnormal and largest subnormal
    assert oracle.half_to_float(0x0001) == 2.0 ** -24
    assert oracle.half_to_float(0x03FF) == 1023 * 2.0 ** -24
    assert oracle.half_to_float(0x8001) == -(2.0 ** -24)


# ---------------------------------------------------------------- Q4_0
def test_q4_0_dequantize_all_zero_is_minus_8():  # QuantizationTests.cs:23-41
    blk = np.frombuffer(h16(1.0) + bytes(16), dtype=np.uint8)
    assert np.all(oracle.dequant(oracle.Q4_0, blk, 32) == -8.0)


def test_q4_0_dequantize_midpoint_is_zero():  # QuantizationTests.cs:43-60
    blk = np.frombuffer(h16(0.5) + bytes([0x88] * 16), dtype=np.uint8)
    assert np.all(oracle.dequant(oracle.Q4_0, blk, 32) == 0.0)


def test_q4_0_dot_closed_form():  # QuantizationTests.cs:62-87
    blk = np.frombuffer(h16(2.0) + bytes([0x37] * 16), dtype=np.uint8)
    # 16 * (7 - 8) * 2 + 16 * (3 - 8) * 2 = -192
    assert oracle.dot(oracle.Q4_0, blk, np.ones(32, np.float32)) == -192.0
    deq = oracle.dequant(oracle.Q4_0, blk, 32)
    assert np.all(deq[:16] == -2.0) and np.all(deq[16:] == -10.0)


def test_q4_0_multiblock_dequantize():  # QuantizationTests.cs:704-726
    data = np.frombuffer(h16(1.0) + bytes([0x88] * 16) + h16(2.0) + bytes([0x88] * 16), dtype=np.uint8)
    assert np.all(oracle.dequant(oracle.Q4_0, data, 64) == 0.0)


def test_q4_0_nibble_positions():
    # low nibble of qs[j] -> element j, high nibble -> element 16+j (DequantQ4_0.cs:12-14)
    qs = bytearray([0x88] * 16)
    qs[5] = 0x8B   # low nibble 11 -> element 5 = +3
    qs[9] = 0x18   # high nibble 1 -> element 25 = -7
    blk = np.frombuffer(h16(1.0) + bytes(qs), dtype=np.uint8)
    deq = oracle.dequant(oracle.Q4_0, blk, 32)
    want = np.zeros(32, np.float32)
    want[5], want[25] = 3.0, -7.0
    assert np.array_equal(deq, want)


def test_q4_0_partial_final_block():
    # DequantQ4_0.Dequantize handles elementCount not a multiple of 32 (:39-56)
    blk = np.frombuffer(h16(1.0) + bytes([0x9A] * 16), dtype=np.uint8)
    deq = oracle.dequant(oracle.Q4_0, blk, 20)
    assert np.array_equal(deq, np.array([2.0] * 16 + [1.0] * 4, np.float32))


# ---------------------------------------------------------------- Q4_K
def q4k_block(d, dmin, scale_byte, qs_byte):
    return np.frombuffer(h16(d) + h16(dmin) + bytes([scale_byte] * 12) + bytes([qs_byte] * 128), np.uint8)


def test_q4_k_dot_closed_form():  # QuantizationTests.cs:464-489
    blk = q4k_block(0.5, 0.25, 0x11, 0x33)
    # sc/m = 17 for s<4 and 1 for s>=4: values 21.25 and 1.25; dot = 2880
    deq = oracle.dequant(oracle.Q4_K, blk, 256)
    assert np.all(deq[:128] == 21.25) and np.all(deq[128:] == 1.25)
    assert oracle.dot(oracle.Q4_K, blk, np.ones(256, np.float32)) == 2880.0


def test_q4_k_two_block_dot():  # QuantizationTests.cs:728-759
    blk = np.concatenate([q4k_block(0.5, 0.25, 0x11, 0x55)] * 2)
    assert oracle.dot(oracle.Q4_K, blk, np.full(512, 0.5, np.float32)) == 5184.0


def test_q4_k_finite():  # QuantizationTests.cs:445-462
    blk = np.frombuffer(h16(1.0) + h16(0.5) + bytes([0x11] * 12) + bytes(128), np.uint8)
    assert np.all(np.isfinite(oracle.dequant(oracle.Q4_K, blk, 256)))


def test_q4_k_reference_nibble_order():
    # ChatNet's own order (DequantQ4K.cs:59-72): sub-block s owns qs[16s..16s+15];
    # byte 3 of sub-block 2 carries element 67 (low) and element 83 (high).
    # llama.cpp's order would put these bytes at elements 3 / 35 of sub-blocks 0/1.
    scales = bytes([1, 1, 1, 1, 0, 0, 0, 0, 1, 1, 1, 1])  # sc = 1, m = 0 for all 8
    qs = bytearray(128)
    qs[16 * 2 + 3] = 0x5A
    blk = np.frombuffer(h16(1.0) + h16(0.0) + scales + bytes(qs), np.uint8)
    deq = oracle.dequant(oracle.Q4_K, blk, 256)
    want = np.zeros(256, np.float32)
    want[67], want[83] = 10.0, 5.0
    assert np.array_equal(deq, want)


def test_q4_k_scale_decode_high_bits():
    # get_scale_min_k4 (DequantQ4K.cs:218-241): 6-bit sc/m for s>=4 take their
    # top two bits from bytes 0..7.
    s = bytearray(12)
    s[0] = 0xC0 | 5      # sc[0] = 5, top bits of sc[4] = 3
    s[4] = 0x40 | 7      # m[0] = 7, top bits of m[4] = 1
    s[8] = 0x92          # sc[4] low = 2, m[4] low = 9
    sc, m = npref.q4k_scales(np.frombuffer(bytes(s), np.uint8))
    assert sc[0, 0] == 5 and m[0, 0] == 7 and sc[0, 4] == 2 + (3 << 4) and m[0, 4] == 9 + (1 << 4)
    qs = bytes([0x11] * 128)
    blk = np.frombuffer(h16(1.0) + h16(1.0) + bytes(s) + qs, np.uint8)
    deq = oracle.dequant(oracle.Q4_K, blk, 256)
    assert deq[0] == 5 * 1 - 7 and deq[32 * 4] == (2 + 48) * 1 - (9 + 16)


# ---------------------------------------------------------------- Q6_K
def test_q6_k_dot_closed_form():  # QuantizationTests.cs:321-345
    raw = bytearray(210)
    raw[0:128] = bytes([0x22] * 128)
    raw[192:208] = bytes([2] * 16)
    raw[208:210] = h16(0.1)
    blk = np.frombuffer(bytes(raw), np.uint8)
    d = float(np.float16(0.1))
    assert d == 0.0999755859375
    deq = oracle.dequant(oracle.Q6_K, blk, 256)
    assert np.all(deq == np.float32(d * 2 * -30))
    assert oracle.dot(oracle.Q6_K, blk, np.ones(256, np.float32)) == 256 * 2 * -30 * d  # -1535.625


def test_q6_k_finite():  # QuantizationTests.cs:302-319
    raw = bytearray(210)
    raw[192:208] = bytes([1] * 16)
    raw[208:210] = h16(1.0)
    assert np.all(np.isfinite(oracle.dequant(oracle.Q6_K, np.frombuffer(bytes(raw), np.uint8), 256)))


def test_q6_k_element_positions_and_signed_scales():
    # Background: ql nibbles 0 and qh bit-pairs 2 -> q = 32 -> value 0.
    raw = bytearray(210)
    raw[128:192] = bytes([0xAA] * 64)
    sc = np.arange(1, 17, dtype=np.int8)
    sc[4] = -3
    raw[192:208] = sc.tobytes()
    raw[208:210] = h16(1.0)
    raw[64 + 32 + 5] = 0x71   # h=1, l=5: q2 low nibble 1 -> elem 165; q4 high nibble 7 -> elem 229
    raw[128 + 7] = 0xBA       # h=0, l=7: q3 high bits 3 -> elem 71 = (48 - 32) * sc[4]
    deq = oracle.dequant(oracle.Q6_K, np.frombuffer(bytes(raw), np.uint8), 256)
    want = np.zeros(256, np.float32)
    want[165] = 1 * sc[10]   # scale index 8h + l/16 + 2
    want[229] = 7 * sc[14]   # 8h + l/16 + 6
    want[71] = 16 * sc[4]    # 8h + l/16 + 4, a negative int8 scale
    assert np.array_equal(deq, want)


# ---------------------------------------------------------------- Q8_0
def test_q8_0_dequantize():  # QuantizationTests.cs:237-270
    blk = np.frombuffer(h16(0.5) + bytes([10] * 32), np.uint8)
    assert np.all(oracle.dequant(oracle.Q8_0, blk, 32) == 5.0)
    blk = np.frombuffer(h16(1.0) + bytes([0xF6] * 32), np.uint8)
    assert np.all(oracle.dequant(oracle.Q8_0, blk, 32) == -10.0)


def test_q8_0_dot():  # QuantizationTests.cs:273-295: 0.25 * (0 + 1 + ... + 31)
    blk = np.frombuffer(h16(0.25) + bytes(range(32)), np.uint8)
    assert oracle.dot(oracle.Q8_0, blk, np.ones(32, np.float32)) == 124.0


def test_q8_0_element_positions_and_partial_block():
    q = bytes([0] * 32)
    blk = bytearray(h16(2.0) + q + h16(-1.0) + q)
    blk[2 + 5] = 0x81        # block 0 element 5 = -127 * 2
    blk[34 + 2 + 31] = 3     # block 1 element 31 = 3 * -1
    deq = oracle.dequant(oracle.Q8_0, np.frombuffer(bytes(blk), np.uint8), 64)
    want = np.zeros(64, np.float32)
    want[5], want[63] = -254.0, -3.0
    assert np.array_equal(deq, want)
    assert np.array_equal(oracle.dequant(oracle.Q8_0, np.frombuffer(bytes(blk), np.uint8), 40), want[:40])


# ---------------------------------------------------------------- Q5_K
def q5k_block(d, dmin, scale_byte, qs_byte, qh=bytes(32)):
    return np.frombuffer(h16(d) + h16(dmin) + bytes([scale_byte] * 12) + qh + bytes([qs_byte] * 128), np.uint8)


def test_q5_k_dot_closed_form():  # QuantizationTests.cs:513-537
    # sc = m = 17 for sub-blocks 0..3 and 1 for 4..7, q5 = 5:
    # 4*32*(0.5*17*5 - 0.25*17) + 4*32*(0.5*1*5 - 0.25*1) = 5184
    blk = q5k_block(0.5, 0.25, 0x11, 0x55)
    assert oracle.dot(oracle.Q5_K, blk, np.ones(256, np.float32)) == 5184.0


def test_q5_k_finite():  # QuantizationTests.cs:495-511
    raw = bytearray(176)
    raw[0:2], raw[2:4], raw[4:16] = h16(1.0), h16(0.5), bytes([0x11] * 12)
    assert np.all(np.isfinite(oracle.dequant(oracle.Q5_K, np.frombuffer(bytes(raw), np.uint8), 256)))


def test_q5_k_high_bit_positions():
    """Bit e%8 of qh[e/8] adds 16 to element e only (DequantQ5K.cs:67-80), in the
    reference's nibble order (qs[16s+j] low -> 32s+j, high -> 32s+16+j)."""
    base = oracle.dequant(oracle.Q5_K, q5k_block(1.0, 0.0, 0x01, 0x00), 256)  # sc = 1, m = 0 -> q5
    assert np.all(base == 0.0)
    for e in (0, 7, 8, 31, 32, 47, 100, 255):
        qh = bytearray(32)
        qh[e // 8] |= 1 << (e % 8)
        deq = oracle.dequant(oracle.Q5_K, q5k_block(1.0, 0.0, 0x01, 0x00, bytes(qh)), 256)
        want = np.zeros(256, np.float32)
        want[e] = 16.0
        assert np.array_equal(deq, want), e
    raw = bytearray(q5k_block(1.0, 0.0, 0x01, 0x00).tobytes())
    raw[48 + 16 * 3 + 5] = 0x9A  # sub-block 3: element 96+5 gets 0xA, element 96+16+5 gets 0x9
    deq = oracle.dequant(oracle.Q5_K, np.frombuffer(bytes(raw), np.uint8), 256)
    want = np.zeros(256, np.float32)
    want[101], want[117] = 10.0, 9.0
    assert np.array_equal(deq, want)


# ---------------------------------------------------------------- brute force
@pytest.mark.parametrize("qtype", [oracle.Q4_0, oracle.Q4_K, oracle.Q6_K, oracle.Q8_0, oracle.Q5_K])
def test_dequant_and_dot_match_float64_restatement(qtype):
    rows, K = 48, 512
    t = synth.tensor(qtype, 7, f"bf{qtype}", rows, K)
    x = synth.normal(8, "bf-x", K, 1.0)
    W64 = npref.matrix(t)
    got_deq = oracle.dequant(qtype, t.data, rows * K).reshape(rows, K)
    np.testing.assert_allclose(got_deq, W64, rtol=1e-6, atol=1e-12)
    y = oracle.matvec(qtype, t.data, x, rows, K)
    ref = W64 @ x.astype(np.float64)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-5


def test_matvec_threads_do_not_change_results():
    M, K = 1024, 512  # above ParallelRowThreshold (TensorMath.cs:28)
    t = synth.tensor(oracle.Q4_0, 3, "thr", M, K)
    x = synth.normal(3, "thr-x", K, 1.0)
    oracle.set_threads(1)
    a = oracle.matvec(oracle.Q4_0, t.data, x, M, K)
    oracle.set_threads(4)
    b = oracle.matvec(oracle.Q4_0, t.data, x, M, K)
    oracle.set_threads(1)
    assert np.array_equal(a, b)


def test_dot_f32_matches_float64():
    a = synth.normal(1, "fa", 1000, 1.0)
    b = synth.normal(1, "fb", 1000, 1.0)
    r = float(np.dot(a.astype(np.float64), b.astype(np.float64)))
    assert abs(float(oracle.lib().oracle_dot_f32(a.ctypes.data, b.ctypes.data, 1000)) - r) < 1e-4


# ---------------------------------------------------------------- fp32 ops
def test_rmsnorm_closed_form():
    n, c, eps = 2048, 0.75, 1e-5
    w = synth.normal(2, "rw", n, 1.0)
    out = oracle.rmsnorm(np.full(n, c, np.float32), w, eps)
    np.testing.assert_allclose(out, w * c / np.sqrt(c * c + eps), rtol=2e-6)
    x = synth.normal(2, "rx", 1000, 1.0)  # 1000: exercises the 8-lane remainder and scalar tail
    np.testing.assert_allclose(oracle.rmsnorm(x, w[:1000], eps), npref.rmsnorm(x.astype(np.float64), w[:1000], eps),
                               rtol=2e-6, atol=1e-7)


def test_rope_identity_at_zero_and_norm_preserving():
    hd, nh, nkv = 64, 4, 2
    q = synth.normal(4, "rq", nh * hd, 1.0)
    k = synth.normal(4, "rk", nkv * hd, 1.0)
    q0, k0 = oracle.rope(q, k, 0, hd, nh, nkv, 10000.0)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    q5, k5 = oracle.rope(q, k, 517, hd, nh, nkv, 10000.0)
    pn = lambda v: np.hypot(v[0::2], v[1::2])
    np.testing.assert_allclose(pn(q5), pn(q), rtol=1e-5)
    np.testing.assert_allclose(q5, npref.rope(q.astype(np.float64), 517, hd, 10000.0), atol=5e-4)
    np.testing.assert_allclose(k5, npref.rope(k.astype(np.float64), 517, hd, 10000.0), atol=5e-4)


def _split_half_to_pairs(v, hd):
    # per head: element j -> 2j and element j + hd/2 -> 2j + 1
    h = v.reshape(-1, 2, hd // 2)
    return np.stack([h[:, 0], h[:, 1]], axis=-1).reshape(-1)


def test_rope_neox_closed_form_and_invariants():
    # TensorMath.ApplyRoPENeox (TensorMath.cs:475-520), hd 4: pairs (0, 2) and (1, 3)
    # with angles pos * base^0 and pos * base^(-1/2)
    q = np.array([1.0, 2.0, 3.0, 4.0], dtype=np.float32)
    k = np.array([0.5, -1.0, 0.25, 2.0], dtype=np.float32)
    pos, base = 3, 100.0
    t0, t1 = pos * 1.0, pos * base ** -0.5
    want = np.array([1 * np.cos(t0) - 3 * np.sin(t0), 2 * np.cos(t1) - 4 * np.sin(t1),
                     3 * np.cos(t0) + 1 * np.sin(t0), 4 * np.cos(t1) + 2 * np.sin(t1)])
    qn, kn = oracle.rope_neox(q, k, pos, 4, 1, 1, base)
    np.testing.assert_allclose(qn, want, atol=2e-6)
    np.testing.assert_allclose(kn[0], 0.5 * np.cos(t0) - 0.25 * np.sin(t0), atol=2e-6)
    # identity at position 0, pair norms kept, float64 restatement
    hd, nh, nkv = 64, 4, 2
    q = synth.normal(4, "nq", nh * hd, 1.0)
    k = synth.normal(4, "nk", nkv * hd, 1.0)
    q0, k0 = oracle.rope_neox(q, k, 0, hd, nh, nkv, 1e6)
    assert np.array_equal(q0, q) and np.array_equal(k0, k)
    q5, k5 = oracle.rope_neox(q, k, 517, hd, nh, nkv, 1e6)
    pn = lambda v: np.hypot(v.reshape(-1, 2, hd // 2)[:, 0], v.reshape(-1, 2, hd // 2)[:, 1])
    np.testing.assert_allclose(pn(q5), pn(q), rtol=1e-5)
    np.testing.assert_allclose(q5, npref.rope_neox(q.astype(np.float64), 517, hd, 1e6), atol=5e-4)
    np.testing.assert_allclose(k5, npref.rope_neox(k.astype(np.float64), 517, hd, 1e6), atol=5e-4)


def test_rope_neox_is_interleaved_rope_of_the_permuted_head():
    # Exact in float32: ApplyRoPENeox's angle for element j equals ApplyRoPE's for
    # the pair at 2j (j*(2/hd) and 2j*(1/hd) differ by an exact factor 2), and
    # x1*c + x0*s is x0*s + x1*c.  This is the identity the device path relies on
    # when it stores q/k rows of a split-half model in pair order.
    hd, nh, nkv = 64, 14, 2
    q = synth.normal(9, "pq", nh * hd, 1.0)
    k = synth.normal(9, "pk", nkv * hd, 1.0)
    for pos in (1, 7, 1000, 4095):
        qn, kn = oracle.rope_neox(q, k, pos, hd, nh, nkv, 1e6)
        qi, ki = oracle.rope(_split_half_to_pairs(q, hd), _split_half_to_pairs(k, hd), pos, hd, nh, nkv, 1e6)
        assert np.array_equal(_split_half_to_pairs(qn, hd), qi)
        assert np.array_equal(_split_half_to_pairs(kn, hd), ki)


def test_softmax_sums_to_one_and_is_shift_invariant():
    x = synth.normal(5, "sm", 300, 3.0)
    p = oracle.softmax(x)
    assert abs(float(p.astype(np.float64).sum()) - 1.0) < 1e-5
    np.testing.assert_allclose(oracle.softmax(x + 7.0), p, rtol=1e-4, atol=1e-7)
    e = np.exp(x.astype(np.float64) - x.max())
    np.testing.assert_allclose(p, e / e.sum(), rtol=1e-5, atol=1e-9)


def test_silu_mul():
    g = synth.normal(6, "sg", 999, 2.0)
    u = synth.normal(6, "su", 999, 1.0)
    g64 = g.astype(np.float64)
    np.testing.assert_allclose(oracle.silu_mul(g, u), g64 / (1 + np.exp(-g64)) * u, rtol=1e-5, atol=1e-7)
    assert oracle.silu_mul(np.zeros(4, np.float32), np.ones(4, np.float32)).tolist() == [0.0] * 4


def test_argmax_tie_rule():  # GreedySampler.cs:13-26
    assert oracle.argmax(np.array([1, 5, 5, 2], np.float32)) == 1
    assert oracle.argmax(np.array([np.nan, 5, 9], np.float32)) == 0
    assert oracle.argmax(np.array([1, np.nan, 9, 9], np.float32)) == 2
    assert oracle.argmax(np.array([-np.inf, -np.inf], np.float32)) == 0


# ---------------------------------------------------------------- Q4_1 / Q5_0 / Q5_1
def test_q4_1_dequantize_and_dot():  # QuantizationTests.cs:93-135
    blk = np.frombuffer(h16(2.0) + h16(1.0) + bytes(16), np.uint8)
    assert np.all(oracle.dequant(oracle.Q4_1, blk, 32) == 1.0)  # 0 * 2 + 1
    blk = np.frombuffer(h16(1.0) + h16(0.5) + bytes([0x55] * 16), np.uint8)
    assert oracle.dot(oracle.Q4_1, blk, np.ones(32, np.float32)) == 32 * 5.5


def test_q4_1_nibble_positions():
    qs = bytearray(16)
    qs[3] = 0xA7  # element 3 gets 7, element 19 gets 10
    deq = oracle.dequant(oracle.Q4_1, np.frombuffer(h16(1.0) + h16(-1.0) + bytes(qs), np.uint8), 32)
    want = np.full(32, -1.0, np.float32)
    want[3], want[19] = 6.0, 9.0
    assert np.array_equal(deq, want)


def test_q5_0_dequantize_and_dot():  # QuantizationTests.cs:140-184
    blk = np.frombuffer(h16(1.0) + bytes(20), np.uint8)
    assert np.all(oracle.dequant(oracle.Q5_0, blk, 32) == -16.0)
    # qh = 0x0000FFFF: elements 0..15 get the fifth bit; qs nibbles 0xA
    blk = np.frombuffer(h16(0.5) + bytes([0xFF, 0xFF, 0, 0]) + bytes([0xAA] * 16), np.uint8)
    deq = oracle.dequant(oracle.Q5_0, blk, 32)
    assert np.all(deq[:16] == 5.0) and np.all(deq[16:] == -3.0)  # (26 - 16) / 2, (10 - 16) / 2
    assert oracle.dot(oracle.Q5_0, blk, np.full(32, 0.5, np.float32)) == 16.0


def test_q5_1_dequantize_and_dot():  # QuantizationTests.cs:189-232
    blk = np.frombuffer(h16(1.0) + h16(2.0) + bytes(20), np.uint8)
    assert np.all(oracle.dequant(oracle.Q5_1, blk, 32) == 2.0)
    blk = np.frombuffer(h16(0.25) + h16(0.5) + bytes(4) + bytes([0x33] * 16), np.uint8)
    assert oracle.dot(oracle.Q5_1, blk, np.ones(32, np.float32)) == 32 * 1.25


@pytest.mark.parametrize("qtype,head", [(6, 2), (7, 4)])
def test_q5_high_bit_positions(qtype, head):
    # bit j of the little-endian qh word is element j's fifth bit (DequantQ5_0.cs:36-62)
    raw = bytearray(h16(1.0) + (h16(0.0) if qtype == 7 else b"") + bytes(20))
    qh = (1 << 5) | (1 << 20)
    raw[head:head + 4] = qh.to_bytes(4, "little")
    deq = oracle.dequant(qtype, np.frombuffer(bytes(raw), np.uint8), 32)
    base = -16.0 if qtype == 6 else 0.0
    want = np.full(32, base, np.float32)
    want[5] += 16.0
    want[20] += 16.0
    assert np.array_equal(deq, want)


# ---------------------------------------------------------------- Q2_K / Q3_K / Q8_K
def q2k_block(d, dmin, scale_byte, qs_byte):
    return np.frombuffer(bytes([scale_byte] * 16) + bytes([qs_byte] * 64) + h16(d) + h16(dmin), np.uint8)


def test_q2_k_closed_forms():  # QuantizationTests.cs:351-394
    assert np.all(oracle.dequant(oracle.Q2_K, q2k_block(1.0, 0.5, 0x21, 0), 256) == -1.0)  # 0 - 0.5 * 2
    # q = 1 everywhere (0x55), scale 1, min 1: 0.5 * 1 - 0.25 = 0.25 per element
    assert oracle.dot(oracle.Q2_K, q2k_block(0.5, 0.25, 0x11, 0x55), np.ones(256, np.float32)) == 64.0


def test_q2_k_element_positions():
    # element 128g + 32t + 16h + l = bits 2t.. of qs[32g + 16h + l], scale byte 8g + 2t + h
    raw = bytearray(q2k_block(1.0, 1.0, 0x00, 0).tobytes())
    raw[16 + 32 * 1 + 16 * 1 + 7] = 0b11 << 4  # g=1, h=1, l=7, t=2 -> element 128+64+16+7 = 215
    raw[8 + 2 * 2 + 1] = 0x35  # its scale byte: scale 5, min 3
    deq = oracle.dequant(oracle.Q2_K, np.frombuffer(bytes(raw), np.uint8), 256)
    want = np.zeros(256, np.float32)
    want[208:224] = -3.0  # the sub-block's min applies to all 16 of its elements
    want[215] = 5.0 * 3 - 3.0
    assert np.array_equal(deq, want)


def test_q3_k_closed_forms():  # QuantizationTests.cs:399-438
    zero = np.frombuffer(bytes(108) + h16(1.0), np.uint8)  # scales 0 - 32, q3 0: 1 * -32 * -4
    assert np.all(oracle.dequant(oracle.Q3_K, zero, 256) == 128.0)
    blk = np.frombuffer(bytes(32) + bytes([0x55] * 64) + bytes(12) + h16(0.1), np.uint8)
    d = float(np.float16(0.1))
    deq = oracle.dequant(oracle.Q3_K, blk, 256)
    assert np.all(deq == np.float32(np.float32(d) * np.float32(-32.0)) * np.float32(-3.0))
    y = oracle.dot(oracle.Q3_K, blk, np.ones(256, np.float32))
    assert abs(y - 256 * 96 * d) < 1e-3  # sum of sc * (q3 - 4) = 256 * 96, times d


def test_q3_k_scale_decode_and_positions():
    s = bytearray(12)
    s[2] = 0x9C  # sc[2] low nibble 0xC, sc[10] low nibble 0x9
    s[8 + 2] = 0b11_01_10_01  # sc[2] += 1 << 4, sc[6] += 2 << 4, sc[10] += 1 << 4, sc[14] += 3 << 4
    sc = npref.q3k_scales(np.frombuffer(bytes(s), np.uint8))[0]
    assert sc[2] == 0x1C - 32 and sc[6] == 0x20 - 32 and sc[10] == 0x19 - 32 and sc[14] == 0x30 - 32
    raw = bytearray(bytes(32) + bytes(64) + bytes(s) + h16(1.0))
    raw[32 + 170 // 4] = 0b10 << (2 * (170 % 4))  # element 170: q2 = 2
    raw[170 // 8] = 1 << (170 % 8)  # its high bit: q3 = 6
    deq = oracle.dequant(oracle.Q3_K, np.frombuffer(bytes(raw), np.uint8), 256)
    assert deq[170] == (0x19 - 32) * (6 - 4)  # sub-block 10
    assert deq[169] == (0x19 - 32) * (0 - 4) and deq[32] == (0x1C - 32) * -4


def test_q8_k_closed_forms():  # QuantizationTests.cs:544-586
    blk = np.frombuffer(np.float32(0.5).tobytes() + bytes([10] * 256) + bytes(32), np.uint8)
    assert np.all(oracle.dequant(oracle.Q8_K, blk, 256) == 5.0)
    q = bytes([(i % 20) for i in range(4, 260)])
    blk = np.frombuffer(np.float32(0.25).tobytes() + q + bytes(32), np.uint8)
    assert oracle.dot(oracle.Q8_K, blk, np.ones(256, np.float32)) == 0.25 * sum(q)
    neg = np.frombuffer(np.float32(2.0).tobytes() + bytes([0xFF] + [0] * 255) + bytes(32), np.uint8)
    assert oracle.dequant(oracle.Q8_K, neg, 256)[0] == -2.0  # sbyte


@pytest.mark.parametrize("qtype", [3, 6, 7, 10, 11, 15])
def test_packed_types_match_float64_restatement(qtype):
    rows, K = 48, 512
    t = synth.tensor(qtype, 11, f"pk{qtype}", rows, K)
    x = synth.normal(12, "pk-x", K, 1.0)
    W64 = npref.matrix(t)
    np.testing.assert_allclose(oracle.dequant(qtype, t.data, rows * K).reshape(rows, K), W64, rtol=1e-6,
                               atol=1e-12)
    y = oracle.matvec(qtype, t.data, x, rows, K)
    ref = W64 @ x.astype(np.float64)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-5


# ---------------------------------------------------------------- IQ family
# DequantIQ.cs: the reference's own bit-field decoders (no codebooks).
IQ4NL = [-127, -104, -83, -65, -49, -35, -22, -10, 1, 13, 25, 38, 53, 69, 89, 113]


def test_iq4_nl_reference_kats():  # QuantizationTests.cs:594-635
    blk = bytearray(h16(1.0) + bytes(16))
    blk[2] = 0x80  # element 0: index 0, element 16: index 8
    deq = oracle.dequant(oracle.IQ4_NL, np.frombuffer(bytes(blk), np.uint8), 32)
    assert deq[0] == -127.0 and deq[16] == 1.0
    q = np.frombuffer(h16(0.01) + bytes([0x88] * 16), np.uint8)
    d = float(np.float16(0.01))
    dq = oracle.dequant(oracle.IQ4_NL, q, 32)
    assert np.all(dq == np.float32(d))
    assert abs(oracle.dot(oracle.IQ4_NL, q, np.ones(32, np.float32)) - float(np.sum(dq))) < 1e-5


def test_iq4_nl_table_positions():
    raw = bytearray(h16(2.0) + bytes(16))
    for j in range(16):
        raw[2 + j] = j | ((15 - j) << 4)
    deq = oracle.dequant(oracle.IQ4_NL, np.frombuffer(bytes(raw), np.uint8), 32)
    assert list(deq[:16]) == [2.0 * v for v in IQ4NL]
    assert list(deq[16:]) == [2.0 * v for v in IQ4NL[::-1]]


def test_iq4_xs_scale_bytes_and_positions():
    # all-zero fields: every scale (0 | 0 << 6) - 32, every index 0 (-127)
    zero = np.frombuffer(h16(1.0) + bytes(134), np.uint8)
    assert np.all(oracle.dequant(oracle.IQ4_XS, zero, 256) == 4064.0)
    raw = bytearray(h16(0.5) + bytes(134))
    raw[4 + 5] = 0xFF                      # low scale of sub-block 5: 0x3F (bits 6, 7 dropped)
    raw[2] = 0b10 << (2 * 1)               # scales_h bits for sub-block 1 -> (0 | 2 << 6) - 32 = 96
    raw[3] = 0b01 << (2 * (5 - 4))         # scales_h bits for sub-block 5 -> (63 | 1 << 6) - 32 = 95
    raw[8 + 16 * 5 + 3] = 0x0F             # sub-block 5: element 3 -> index 15, element 19 -> index 0
    raw[8 + 16 * 1 + 9] = 0xA0             # sub-block 1: element 9 -> index 0, element 25 -> index 10
    deq = oracle.dequant(oracle.IQ4_XS, np.frombuffer(bytes(raw), np.uint8), 256)
    assert deq[32 * 5 + 3] == np.float32(0.5 * 95) * 113 and deq[32 * 5 + 19] == np.float32(0.5 * 95) * -127
    assert deq[32 * 1 + 9] == np.float32(0.5 * 96) * -127 and deq[32 * 1 + 25] == np.float32(0.5 * 96) * 25
    # the scale of sub-block 4 is byte 8: sub-block 0's first quant byte
    raw2 = bytearray(h16(1.0) + bytes(134))
    raw2[8] = 0x25                         # sub-block 0: element 0 index 5, element 16 index 2
    deq = oracle.dequant(oracle.IQ4_XS, np.frombuffer(bytes(raw2), np.uint8), 256)
    assert deq[0] == -32.0 * IQ4NL[5] and deq[16] == -32.0 * IQ4NL[2]
    assert np.all(deq[128:160] == (0x25 - 32) * -127.0)   # sub-block 4: scale 0x25 - 32 = 5, index 0


def test_iq3_s_reads_signs_and_scales_from_the_next_block():
    # one block: signs of sub-blocks 12..31 and every scale come from the
    # (zero) tail: scale 1, positive
    blk = bytearray(h16(1.0) + bytes(108))
    blk[2 + 5 // 4] = 0b11 << (2 * (5 % 4))  # element 5: q2 = 3
    blk[66 + 0] = 1 << 5                      # element 5: high bit -> q3 = 7
    blk[98 + 0] = 1 << 5                      # sub-block 0 sign byte: element 5 negated
    blk[2 + 200 // 4] = 0b10 << (2 * (200 % 4))  # element 200 (sub-block 25): q3 = 2, sign from the tail
    deq = oracle.dequant(oracle.IQ3_S, np.frombuffer(bytes(blk), np.uint8), 256)
    want = np.zeros(256, np.float32)
    want[5], want[200] = -7.0, 2.0
    assert np.array_equal(deq, want)
    # two blocks: block 0's sub-block 25 takes sign byte 98 + 25 = 123 = block 1's byte 13 and
    # scale byte 130 + 25 // 4 = 136 = block 1's byte 26
    nxt = bytearray(h16(1.0) + bytes(108))
    nxt[13] = 1 << 0                                  # element 200 = sub-block 25, j = 0: negated
    nxt[26] = 0b10 << (2 * (25 % 4))                  # sub-block 25 scale 2 + 1 = 3
    two = np.frombuffer(bytes(blk) + bytes(nxt), np.uint8)
    deq = oracle.dequant(oracle.IQ3_S, two, 512)
    assert deq[200] == -6.0 and deq[5] == -7.0
    np.testing.assert_array_equal(npref.dequant_iq3_s(two, 512), deq)
    x = np.zeros(512, np.float32)
    x[200], x[5] = 1.0, 2.0
    assert oracle.dot(oracle.IQ3_S, two, x) == -20.0


def test_iq3_xxs_fields():
    zero = np.frombuffer(h16(0.5) + bytes(96), np.uint8)
    assert np.all(oracle.dequant(oracle.IQ3_XXS, zero, 256) == -2.0)  # 0.5 * (0 - 4)
    raw = bytearray(zero.tobytes())
    word = 6 << (3 * 5)  # element 77 = sub-block 9, j = 5: q3 = 6
    for k in range(3):
        raw[2 + 3 * 9 + k] = (word >> (8 * k)) & 0xFF
    deq = oracle.dequant(oracle.IQ3_XXS, np.frombuffer(bytes(raw), np.uint8), 256)
    assert deq[77] == 1.0 and np.sum(deq != -2.0) == 1
    assert oracle.dot(oracle.IQ3_XXS, np.frombuffer(bytes(raw), np.uint8), np.ones(256, np.float32)) == 0.5 * (
        255 * -4 + 2)


def test_iq2_xs_scale_nibbles_and_fields():
    raw = bytearray(h16(1.0) + bytes(72))
    raw[66 + 5 // 2] = 0xB0            # sub-block 5 (odd: high nibble of a negative sbyte): 11 - 8 = 3
    raw[2 + 4 * 5 + 6 // 4] = 0b11 << (2 * (6 % 4))  # sub-block 5, element 6: q = 3
    deq = oracle.dequant(oracle.IQ2_XS, np.frombuffer(bytes(raw), np.uint8), 256)
    assert deq[16 * 5 + 6] == 6.0                       # 3 * (3 - 1)
    assert np.all(np.delete(deq[80:96], 6) == -3.0)     # 3 * (0 - 1)
    assert deq[16 * 4] == 8.0                           # sub-block 4: low nibble 0 - 8 = -8, q = 0
    np.testing.assert_array_equal(npref.dequant_iq2_xs(np.frombuffer(bytes(raw), np.uint8), 256), deq)


def test_iq2_xxs_fields():
    raw = bytearray(h16(0.25) + bytes(64))
    raw[2 + 4 * 7 + 13 // 4] = 0b10 << (2 * (13 % 4))  # element 7 * 16 + 13: q = 2
    deq = oracle.dequant(oracle.IQ2_XXS, np.frombuffer(bytes(raw), np.uint8), 256)
    assert deq[125] == 0.25 and np.all(np.delete(deq, 125) == -0.25)


def test_iq2_s_signs_only_on_the_first_four_elements():
    raw = bytearray(h16(1.0) + bytes(80))
    for j in range(4):
        raw[2 + 4 * 3 + j] = 0xFF          # sub-block 3: every q = 3
    raw[66 + 3] = 0b1011_0101              # scale 5 + 1 = 6, sign nibble 0b1011
    deq = oracle.dequant(oracle.IQ2_S, np.frombuffer(bytes(raw), np.uint8), 256)
    assert list(deq[48:52]) == [-18.0, -18.0, 18.0, -18.0]
    assert np.all(deq[52:64] == 18.0)
    assert np.all(deq[:48] == 0.0) and np.all(deq[64:] == 0.0)


@pytest.mark.parametrize("qtype,size", [(19, 50), (29, 56)])
def test_iq1_ternary_fields(qtype, size):
    raw = bytearray(h16(2.0) + bytes(size - 2))
    raw[2 + 5] = 1 << 3                    # sub-block 5, element 3: +1
    raw[34 + 5 // 2] = 1 << ((5 % 2) * 4 + 6 // 2)  # sub-block 5, elements 6 and 7: -1
    raw[2 + 5] |= 1 << 7                   # ... but element 7's qs bit wins: +1
    deq = oracle.dequant(qtype, np.frombuffer(bytes(raw), np.uint8), 256)
    sc = 1.0 if qtype == 19 else 0.5       # IQ1_M: scale bit 5 of byte 50 clear -> 0.5
    want = np.zeros(256, np.float32)
    want[43], want[46], want[47] = 2.0 * sc, -2.0 * sc, 2.0 * sc
    assert np.array_equal(deq, want)
    if qtype == 29:
        raw[50] = 1 << 5                   # sub-block 5 full scale
        deq = oracle.dequant(qtype, np.frombuffer(bytes(raw), np.uint8), 256)
        assert deq[43] == 2.0 and deq[46] == -2.0


def test_iq1_s_dot_closed_form():
    blk = np.frombuffer(h16(0.5) + bytes([0xFF] * 32) + bytes(16), np.uint8)
    assert oracle.dot(oracle.IQ1_S, blk, np.ones(256, np.float32)) == 128.0


@pytest.mark.parametrize("qtype", [16, 17, 18, 19, 20, 21, 22, 23, 29])
def test_iq_types_match_float64_restatement(qtype):
    rows, K = 24, 512
    t = synth.tensor(qtype, 13, f"iq{qtype}", rows, K)
    x = synth.normal(14, "iq-x", K, 1.0)
    W64 = npref.matrix(t)
    np.testing.assert_allclose(oracle.dequant(qtype, t.data, rows * K).reshape(rows, K), W64, rtol=1e-6,
                               atol=1e-12)
    y = oracle.matvec(qtype, t.data, x, rows, K)
    ref = W64 @ x.astype(np.float64)
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) < 1e-5
