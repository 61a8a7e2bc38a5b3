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


# Greedy-identity results of the GPU tests, printed in pytest's terminal
# summary (visible under -q): (case, identical steps, steps, near-tie steps
# teacher-forced, smallest oracle top-1/top-2 margin).
GREEDY_RECORDS = []
NEAR_TIE = 1e-3  # a step whose oracle margin is below this may pick either token


def record_greedy(case: str, same: int, steps: int, forced: int = 0, min_margin: float = float("nan")) -> None:
    GREEDY_RECORDS.append((case, same, steps, forced, min_margin))


def greedy_against_expected(model, expected, margins, p0: int, case: str):
    """Runs the device greedy loop (chatnet_decode_greedy) after a forward of
    positions < p0 and compares every token with `expected` (the oracle's).
    A step that differs fails the test unless the oracle's top-1/top-2 margin
    there is below NEAR_TIE; the model is then teacher-forced: the expected
    token is forwarded at that position (chatnet_forward) and the device loop
    continues from it, so all steps and the final logits are compared against
    the same sequence.  Returns the number of teacher-forced steps."""
    n = len(expected)
    done, forced = 0, 0
    while done < n:
        got = [int(t) for t in model.decode_greedy(n - done)]
        k = next((i for i, (g, e) in enumerate(zip(got, expected[done:])) if g != int(e)), None)
        if k is None:
            assert len(got) == n - done, (case, len(got), n - done)
            break
        step = done + k
        if not margins[step] < NEAR_TIE:
            record_greedy(case, step, n, forced, float(np.min(margins)))
            raise AssertionError(f"{case}: {step}/{n} greedy tokens identical; step {step}: gpu {got[k]} vs "
                                 f"oracle {int(expected[step])}, oracle margin {margins[step]:.3g}")
        forced += 1
        print(f"[greedy] {case}: near-tie at step {step} (margin {margins[step]:.3g}), teacher-forced", flush=True)
        model.forward([int(expected[step])], p0 + step)
        done = step + 1
    record_greedy(case, n - forced, n, forced, float(np.min(margins)))
    return forced
