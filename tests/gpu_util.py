"""Shared helpers of the GPU tests (torch is used only for device buffers)."""
import sys

import numpy as np


def announce(msg: str) -> None:
    print(f"[gpu-case] {msg}", flush=True)
    sys.stdout.flush()


def device_tensor(arr: np.ndarray):
    import torch

    return torch.from_numpy(np.ascontiguousarray(arr)).to("cuda:0")


def normwise(y: np.ndarray, r: np.ndarray) -> float:
    """max|y - r| / max|r| (the sweep's error metric)."""
    y = np.asarray(y, np.float64)
    r = np.asarray(r, np.float64)
    return float(np.max(np.abs(y - r)) / max(np.max(np.abs(r)), 1e-30))


def gpu_matmul(qtype: int, w_bytes: np.ndarray, x: np.ndarray, M: int, K: int) -> np.ndarray:
    """Runs chatnet_matmul on device copies and returns y as [N, M]."""
    import torch

    from chatnet_amd import ops

    x = np.ascontiguousarray(x, np.float32).reshape(-1, K)
    N = x.shape[0]
    # 256 bytes of slack behind the weights, as the model's own uploads have
    padded = np.zeros(w_bytes.size + 256, np.uint8)
    padded[: w_bytes.size] = w_bytes
    w_d = device_tensor(padded)
    x_d = device_tensor(x)
    y_d = torch.full((N, M), float("nan"), dtype=torch.float32, device="cuda:0")
    ops.matmul(qtype, w_d, x_d, y_d, M, K)
    torch.cuda.synchronize()
    return y_d.cpu().numpy()
