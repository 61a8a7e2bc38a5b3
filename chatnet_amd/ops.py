"""Stand-alone quantized matrix products on caller-owned device memory.

matmul() is chatnet_matmul of include/chatnet_hip.h, the batched form of
TensorMath.MatVecMulQ4_0 / MatVecMulQ6K / MatVecMulGeneric (TensorMath.cs:548-656).
Torch tensors are accepted only as carriers of device pointers and streams.
"""
from __future__ import annotations

from . import _native


def matmul_ptr(ggml_type: int, w_ptr: int, x_ptr: int, y_ptr: int, M: int, K: int, N: int,
               stream: int = 0) -> None:
    """y[N][M] = x[N][K] . W[M][K]^T with W in raw GGUF blocks (device pointers)."""
    lib = _native.hip_lib()
    _native.check(lib.chatnet_matmul(int(ggml_type), w_ptr, x_ptr, y_ptr, int(M), int(K), int(N),
                                     stream or None))


def matmul(ggml_type: int, w, x, y, M: int, K: int) -> None:
    """Torch-tensor convenience: w uint8 (raw blocks), x float32 [N, K], y float32 [N, M], all on the GPU."""
    import torch

    if not (w.is_cuda and x.is_cuda and y.is_cuda):
        raise ValueError("w, x and y must be device tensors")
    if x.dtype != torch.float32 or y.dtype != torch.float32 or w.dtype != torch.uint8:
        raise ValueError("w must be uint8, x and y float32")
    if not (w.is_contiguous() and x.is_contiguous() and y.is_contiguous()):
        raise ValueError("tensors must be contiguous")
    N = x.numel() // K
    if x.numel() != N * K or y.numel() != N * M:
        raise ValueError("x must hold N*K and y N*M elements")
    if w.numel() < _native.tensor_nbytes(ggml_type, M * K):
        raise ValueError("w is smaller than the M x K tensor")
    stream = torch.cuda.current_stream(x.device).cuda_stream
    matmul_ptr(ggml_type, w.data_ptr(), x.data_ptr(), y.data_ptr(), M, K, N, stream)
