"""chatnet_matmul_noalloc (the allocation-free variant of chatnet_matmul: its
scratch is the library's fixed per-device array) against chatnet_matmul on
the same inputs, through the C ABI: two calls in a row, the second smaller,
so the second runs on scratch the first left behind.  Bar: the batched MFMA
GEMM's 1e-2 normwise, and the GEMV path's 1e-3.  The outputs are identical
where both run the same launch; for 11008 x 4096 at N = 512 chatnet_matmul
shares the tiles past one per CU between workgroups (stream-K, summed in
another order) and the no-allocation variant, which keeps no tile counters,
runs the plain tile grid."""
import numpy as np
import pytest

from chatnet_amd import _native, hiprt, synth
from gpu_util import announce, normwise

pytestmark = pytest.mark.gpu


def _call(fn_name, qtype, w_d, x_d, M, K, N, stream):
    lib = _native.hip_lib()
    y = hiprt.DeviceBuffer(4 * M * N)
    y.fill(0xFF)  # NaN pattern: anything left unwritten stays NaN
    _native.check(getattr(lib, fn_name)(qtype, w_d.ptr, x_d.ptr, y.ptr, M, K, N, stream))
    hiprt.synchronize()
    out = y.to_numpy(np.float32, M * N).reshape(N, M)
    y.free()
    return out


@pytest.mark.parametrize("first,second", [
    ((11008, 4096, 512), (4096, 4096, 64)),   # K-split partials, then a smaller split
    ((2048, 5632, 512), (256, 2048, 8)),
    ((4096, 4096, 64), (2048, 2048, 3)),       # then the GEMV path (no scratch)
])
def test_noalloc_matches_matmul_on_two_calls(first, second):
    stream = hiprt.Stream()
    for (M, K, N) in (first, second):
        announce(f"noalloc M={M} K={K} N={N}")
        t = synth.tensor(2, 3, f"na{M}x{K}", M, K)
        x = synth.normal(3, f"nax{N}x{K}", N * K, 1.0)
        w_d = hiprt.DeviceBuffer.from_numpy(t.data, pad=256)
        x_d = hiprt.DeviceBuffer.from_numpy(x)
        ref = _call("chatnet_matmul", 2, w_d, x_d, M, K, N, stream.h)
        got = _call("chatnet_matmul_noalloc", 2, w_d, x_d, M, K, N, stream.h)
        w_d.free()
        x_d.free()
        assert np.all(np.isfinite(got))
        err = normwise(got, ref)
        print(f"noalloc M={M} K={K} N={N}: normwise {err:.3g}, identical {bool(np.array_equal(got, ref))}",
              flush=True)
        assert err <= (1e-2 if N >= 8 else 1e-3)
    stream.synchronize()


def test_noalloc_refuses_more_scratch_than_it_has():
    # N*K*2 = 128 MiB of bf16 x alone: refused before anything is launched
    M, K, N = 256, 16384, 4096
    lib = _native.hip_lib()
    with pytest.raises(_native.ChatnetArgumentError):
        _native.check(lib.chatnet_matmul_noalloc(2, 16, 16, 16, M, K, N, None))


@pytest.mark.parametrize("qtype,first,second", [
    (10, (2048, 2048, 64), (1024, 1024, 2)),   # Q2_K: packed W in the scratch, GEMM then GEMV
    (11, (2048, 2048, 64), (1024, 1024, 2)),   # Q3_K: GEMV over the stored blocks per column
    (3, (4096, 4096, 1), (512, 2048, 16)),     # Q4_1: GEMV then GEMM
])
def test_noalloc_packed_unit_types_match_matmul(qtype, first, second):
    stream = hiprt.Stream()
    for (M, K, N) in (first, second):
        announce(f"noalloc type={qtype} M={M} K={K} N={N}")
        t = synth.tensor(qtype, 5, f"nap{qtype}-{M}x{K}", M, K)
        x = synth.normal(5, f"napx{N}x{K}", N * K, 1.0)
        w_d = hiprt.DeviceBuffer.from_numpy(t.data, pad=256)
        x_d = hiprt.DeviceBuffer.from_numpy(x)
        ref = _call("chatnet_matmul", qtype, w_d, x_d, M, K, N, stream.h)
        got = _call("chatnet_matmul_noalloc", qtype, w_d, x_d, M, K, N, stream.h)
        w_d.free()
        x_d.free()
        assert np.all(np.isfinite(got))
        err = normwise(got, ref)
        print(f"noalloc type={qtype} M={M} K={K} N={N}: normwise {err:.3g}", flush=True)
        assert err <= (1e-2 if N >= 8 else 1e-3)
    stream.synchronize()


def test_noalloc_refuses_a_packed_copy_larger_than_its_scratch():
    # Q2_K 11008 x 4096 packs into 11008 * 64 * 96 bytes (64.5 MiB)
    lib = _native.hip_lib()
    with pytest.raises(_native.ChatnetArgumentError):
        _native.check(lib.chatnet_matmul_noalloc(10, 16, 16, 16, 11008, 4096, 1, None))
