"""Stand-alone quantized matrix products on caller-owned device memory.

matmul_ptr() is chatnet_matmul of include/chatnet_hip.h, the batched form of
TensorMath.MatVecMulQ4_0 / MatVecMulQ6K / MatVecMulGeneric (TensorMath.cs:548-656).
"""
from __future__ import annotations

from . import _native


def matmul_ptr(ggml_type: int, w_ptr: int, x_ptr: int, y_ptr: int, M: int, K: int, N: int,
               stream: int = 0) -> None:
    """y[N][M] = x[N][K] . W[M][K]^T with W in raw GGUF blocks (device pointers)."""
    lib = _native.hip_lib()
    _native.check(lib.chatnet_matmul(int(ggml_type), w_ptr, x_ptr, y_ptr, int(M), int(K), int(N),
                                     stream or None))


def matmul(ggml_type: int, w, x, y, M: int, K: int, N: int = 1, stream: int = 0) -> None:
    """Same on hiprt.DeviceBuffer objects (w: raw blocks, x: N*K fp32, y: N*M fp32)."""
    need_w = _native.tensor_nbytes(ggml_type, M * K)
    if w.nbytes < need_w or x.nbytes < 4 * N * K or y.nbytes < 4 * N * M:
        raise ValueError("device buffers are smaller than the M x K x N problem")
    matmul_ptr(ggml_type, w.ptr, x.ptr, y.ptr, M, K, N, stream)
