"""Shared helpers of the GPU tests (device buffers through chatnet_amd.hiprt)."""
import sys

import numpy as np


def announce(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def normwise(y: np.ndarray, r: np.ndarray) -> float:
    """max|y - r| / max|r| (the sweep's error metric)."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(y - r)) / max(np.max(np.abs(r)), 1e-30))


def gpu_matmul(qtype: int, w_bytes: np.ndarray, x: np.ndarray, M: int, K: int) -> np.ndarray:
    """Runs chatnet_matmul on device copies and returns y as [N, M]."""
    from chatnet_amd import hiprt, ops

    x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
    N = x.shape[0]
    # 256 bytes of slack behind the weights, as the model's own uploads have
    w_d = hiprt.DeviceBuffer.from_numpy(np.ascontiguousarray(w_bytes, np.uint8), pad=256)
    x_d = hiprt.DeviceBuffer.from_numpy(x)
    y_d = hiprt.DeviceBuffer(4 * N * M)
    y_d.fill(0xFF)  # NaN pattern: rows the kernel fails to write stay NaN
    ops.matmul(qtype, w_d, x_d, y_d, M, K, N)
    hiprt.synchronize()
    y = y_d.to_numpy(np.float32, N * M).reshape(N, M)
    for b in (w_d, x_d, y_d):
        b.free()
    return y
