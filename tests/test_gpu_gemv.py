"""GPU parity of the fused dequant-GEMV (chatnet_matmul, N=1) against the
oracle's MatVecMulByType on identical seeded blocks.  Bar: normwise error
max|y-r|/max|r| <= 1e-3 (fp32 accumulate)."""
import numpy as np
import pytest

import oracle
from chatnet_amd import synth
from gpu_util import announce, gpu_matmul, normwise

pytestmark = pytest.mark.gpu

TOL = 1e-3

# Isolated Q4_0 sweep shapes (out x in) and the K-quant shapes of the
# Q4_K_M-style mix.
Q4_0_SHAPES = [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632), (32000, 2048), (4096, 4096),
               (11008, 4096)]
KQ_SHAPES = [(12, 4096, 4096), (12, 11008, 4096), (14, 4096, 11008), (14, 32000, 4096)]
# Q8_0 and Q5_K (MatVecMulGeneric types, LlamaModel.cs:501-519) on the 7B shapes.
GENERIC_SHAPES = [(8, 4096, 4096), (8, 11008, 4096), (8, 4096, 11008), (8, 32000, 4096),
                  (13, 4096, 4096), (13, 11008, 4096), (13, 4096, 11008)]


@pytest.fixture(scope="module", autouse=True)
def _threads():
    oracle.set_threads(16)
    yield
    oracle.set_threads(1)


def run_case(qtype, M, K, seed=1):
    announce(f"gemv type={qtype} M={M} K={K} seed={seed}")
    t = synth.tensor(qtype, seed, f"w{qtype}_{M}_{K}", M, K)
    x = synth.normal(seed, f"x{K}", K, 1.0)
    y = gpu_matmul(qtype, t.data, x, M, K)[0]
    r = oracle.matvec(qtype, t.data, x, M, K)
    assert np.all(np.isfinite(y))
    err = normwise(y, r)
    assert err <= TOL, (qtype, M, K, err)
    return err


@pytest.mark.parametrize("qtype", [0, 1, 2, 8, 11, 12, 13, 14, 3, 23])
def test_growing_k_past_64kb_of_lds_in_one_process(qtype):
    """Rows of K > 15872 stage x in more than 64 KB of LDS, which a kernel may
    use only once its maximum was raised.  The same type and epilogue at
    K = 16128 and then K = 16384 (a larger staging area for the same kernel
    instance) must both run and match the oracle.  Placed first in this file so
    the K = 16128 launch is the instance's first above 64 KB in the process."""
    for K in (16128, 16384):
        run_case(qtype, 5, K, seed=23)


@pytest.mark.parametrize("M,K", Q4_0_SHAPES)
def test_q4_0_gemv_sweep_shapes(M, K):
    run_case(2, M, K)


@pytest.mark.parametrize("qtype,M,K", KQ_SHAPES)
def test_kquant_gemv_shapes(qtype, M, K):
    run_case(qtype, M, K)


@pytest.mark.parametrize("qtype,M,K", GENERIC_SHAPES)
def test_generic_type_gemv_shapes(qtype, M, K):
    run_case(qtype, M, K)


@pytest.mark.parametrize("qtype,M,K", [
    (2, 1, 64), (2, 3, 64), (2, 17, 192), (2, 33, 2048), (2, 130, 5632), (2, 7, 11008),
    (8, 1, 64), (8, 3, 128), (8, 17, 192), (8, 33, 2048), (8, 5, 16384),   # 1..4 units per lane
    (13, 1, 256), (13, 9, 768), (13, 40, 2816),
    (12, 1, 256), (12, 5, 768), (12, 31, 11008),
    (14, 1, 256), (14, 9, 768), (14, 18, 1280),   # 768/1280: rows start 2 bytes off a dword
    # half super-blocks per lane: 44 per row (one per lane, base-256 digits for
    # Q4_K too) and 128 per row (K = 16384, two per lane)
    (12, 7, 5632), (13, 7, 5632), (14, 7, 5632),
    # Q4_0 rows of 65..128 units: K split over two waves (65: the second wave
    # holds one unit; 128: both full)
    (2, 5, 4160), (2, 3, 8192), (2, 1, 8192),
    # Q4_0 rows of 129..192 units: one row per lane, three units each
    (2, 1, 8256), (2, 5, 12288), (2, 4097, 11008),
    (12, 3, 16384), (13, 3, 16384), (14, 3, 16384), (8, 9, 16320),
    # Q5_K rows of 65..96 half super-blocks: one row per lane, 32 lanes x 3 units
    (13, 5, 8448), (13, 7, 12288), (13, 66, 11008),
    # Q6_K rows of 65..96 half super-blocks: quarter super-blocks, 64 lanes x 3
    # (rows start 2 bytes off a dword on every other row)
    (14, 5, 8448), (14, 7, 12288), (14, 131, 11008), (14, 1, 11008),
])
def test_ragged_and_misaligned_shapes(qtype, M, K):
    run_case(qtype, M, K, seed=5)


def test_q6_k_rows_off_dword_alignment_are_exact_per_row():
    # K=768 gives a 630-byte row stride: odd rows start at 2 mod 4.
    M, K = 64, 768
    t = synth.tensor(14, 9, "q6mis", M, K)
    x = synth.normal(9, "q6mis-x", K, 1.0)
    announce("q6_k misaligned rows")
    y = gpu_matmul(14, t.data, x, M, K)[0]
    r = oracle.matvec(14, t.data, x, M, K)
    # A misread row is off by about its own size.  The floor (1 % of the largest
    # row) keeps rows that cancel to near zero from failing on the digit path's
    # rounding of x, ~2^-19 of each 16-element group's maximum.
    rel = np.abs(y - r) / np.maximum(np.abs(r), 1e-2 * np.max(np.abs(r)))
    assert np.max(rel[1::2]) < 1e-3 and np.max(rel[0::2]) < 1e-3


def test_subnormal_fp16_scales_are_not_flushed():
    # K-quant and Q4_0 scales of N(0, 0.02) weights sit near fp16's min normal;
    # the kernel must convert subnormal halves exactly (DequantQ4_0.cs:190-194).
    M, K = 4, 64
    blk = bytearray()
    for r in range(M):
        for b in range(K // 32):
            blk += np.uint16(0x0001 + 0x0100 * r + b).tobytes()  # subnormal d (< 0x0400)
            blk += bytes([(0x1F * (r + 3 * b + j)) & 0xFF for j in range(16)])
    w = np.frombuffer(bytes(blk), np.uint8)
    x = synth.normal(4, "sub-x", K, 1.0)
    announce("q4_0 subnormal scales")
    y = gpu_matmul(2, w, x, M, K)[0]
    r = oracle.matvec(2, w, x, M, K)
    assert np.all(r != 0)
    assert normwise(y, r) < 1e-5


@pytest.mark.parametrize("N", [8, 64])
def test_batched_columns_match_per_column_gemv(N):
    M, K = 2048, 2048
    t = synth.tensor(2, 2, "batch", M, K)
    x = synth.normal(2, "batch-x", N * K, 1.0).reshape(N, K)
    announce(f"q4_0 matmul N={N}")
    y = gpu_matmul(2, t.data, x, M, K)
    for n in range(0, N, max(1, N // 4)):
        r = oracle.matvec(2, t.data, x[n], M, K)
        assert normwise(y[n], r) <= 1e-2



# F32 and F16 weight matrices (TensorMath.MatVecMul, TensorMath.cs:527-540, and
# LlamaModel.MatVecMulF16, LlamaModel.cs:570-598), including ragged row counts,
# the longest rows (K = 16384: 64 KB of staged x) and the LM-head shape.
@pytest.mark.parametrize("qtype,M,K", [
    (0, 2048, 2048), (0, 256, 2048), (0, 4096, 4096), (0, 2048, 5632), (0, 32000, 2048),
    (1, 2048, 2048), (1, 256, 2048), (1, 4096, 11008), (1, 11008, 4096), (1, 32000, 4096),
    (0, 1, 64), (0, 7, 192), (0, 33, 16384), (1, 1, 64), (1, 5, 320), (1, 9, 16384),
])
def test_float_weight_gemv_shapes(qtype, M, K):
    run_case(qtype, M, K, seed=7)


# The MatVecMulGeneric branches of LlamaModel.MatVecMulByType (LlamaModel.cs:488-528):
# Q4_1, Q5_0, Q5_1, Q2_K and Q8_K the GEMV reads as packed units (re-encoded on
# the device first: u8 codes with an fp32 scale and offset per 16 weights, each
# weight equal to the type's dequantized value); Q3_K it reads from the stored
# 110-byte blocks (rows of an odd number of blocks start 2 bytes off a dword).
PACKED_ONLY = {3: "q4_1", 6: "q5_0", 7: "q5_1", 10: "q2_k", 11: "q3_k", 15: "q8_k"}
# The IQ family (DequantIQ.cs), read the same way.
IQ = {16: "iq2_xxs", 17: "iq2_xs", 18: "iq3_xxs", 19: "iq1_s", 20: "iq4_nl", 21: "iq3_s", 22: "iq2_s",
      23: "iq4_xs", 29: "iq1_m"}


@pytest.mark.parametrize("M,K", [(4096, 4096), (11008, 4096), (4096, 11008), (32000, 2048)])
@pytest.mark.parametrize("qtype", sorted(PACKED_ONLY))
def test_packed_unit_types_gemv_shapes(qtype, M, K):
    run_case(qtype, M, K, seed=11)


@pytest.mark.parametrize("qtype,M,K", [
    (3, 1, 64), (6, 3, 128), (7, 17, 192), (3, 33, 2048), (6, 5, 16384), (7, 130, 5632),
    (10, 1, 256), (11, 9, 768), (15, 40, 2816), (10, 7, 5632), (11, 3, 16384), (15, 5, 16384),
    (11, 1, 256), (11, 7, 256), (11, 65, 1280), (11, 130, 5632), (11, 257, 4352),
])
def test_packed_unit_types_ragged_shapes(qtype, M, K):
    run_case(qtype, M, K, seed=13)


@pytest.mark.parametrize("M,K", [(4096, 4096), (4096, 11008)])
@pytest.mark.parametrize("qtype", sorted(IQ))
def test_iq_types_gemv_shapes(qtype, M, K):
    run_case(qtype, M, K, seed=17)


@pytest.mark.parametrize("qtype,M,K", [
    (20, 1, 64), (20, 17, 192), (20, 5, 16384), (21, 1, 256), (21, 9, 768), (21, 3, 16384),
    (16, 7, 5632), (17, 40, 2816), (18, 1, 256), (19, 5, 768), (22, 33, 2048), (23, 9, 16384), (29, 130, 1280),
])
def test_iq_types_ragged_shapes(qtype, M, K):
    run_case(qtype, M, K, seed=19)


@pytest.mark.parametrize("N", [1, 16])
def test_iq3_s_ignores_bytes_after_the_matrix(N):
    # IQ3_S's last block of a row reads 28 bytes past it (DequantIQ.cs:255-283);
    # past the matrix's end the library reads zeros whatever memory follows
    M, K = 9, 512
    t = synth.tensor(21, 23, "iq3s-tail", M, K)
    x = synth.normal(23, "iq3s-tail-x", N * K, 1.0).reshape(N, K)
    announce(f"iq3_s tail N={N}")
    garbage = np.concatenate([t.data, np.full(256, 0xFF, np.uint8)])
    y = gpu_matmul(21, garbage, x, M, K)
    for n in range(N):
        r = oracle.matvec(21, t.data, x[n], M, K)  # the oracle appends zeros
        assert normwise(y[n], r) <= (TOL if N == 1 else 1e-2)
