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


def _continue(resume, prefix, k):
    """The oracle's k greedy tokens (and margins) after the prompt + prefix."""
    if callable(resume):
        return resume(prefix, k)
    import oracle

    cfg, ck, prompt = resume
    return oracle.OracleLlama(cfg, ck).generate_greedy(list(prompt) + list(prefix), k)


def compare_greedy(gpu_tokens, ora_tokens, margins, case="greedy", resume=None):
    """Compares the GPU's greedy tokens with the oracle's, every step.  A
    difference fails unless the oracle's top-1/top-2 margin at that step is
    below NEAR_TIE (either token is then a valid pick); the oracle is then
    teacher-forced onto the GPU's pick: `resume` = (cfg, checkpoint, prompt)
    regenerates the oracle's greedy continuation after the prompt and the
    GPU's tokens so far (or a callable (prefix, k) -> (tokens, margins) does),
    and the remaining steps are compared against it.
    Returns the number of leading steps identical without forcing (callers
    compare final logits only when that is every step).  The result is
    recorded for the terminal summary either way."""
    gpu = [int(t) for t in gpu_tokens]
    exp = [int(t) for t in ora_tokens]
    mar = [float(m) for m in margins[:len(exp)]]
    first, forced, i = len(exp), 0, 0
    while i < len(exp):
        if i >= len(gpu):
            break
        if gpu[i] != exp[i]:
            if not mar[i] < NEAR_TIE:
                record_greedy(case, i, len(exp), forced, float(np.min(mar)))
                raise AssertionError(f"{case}: {i}/{len(exp)} greedy tokens identical; step {i}: gpu {gpu[i]} vs "
                                     f"oracle {exp[i]}, margin {mar[i]:.3g}")
            assert resume is not None, f"{case}: near-tie at step {i} but no oracle continuation given"
            print(f"[greedy] {case}: near-tie at step {i} (margin {mar[i]:.3g}), oracle teacher-forced", flush=True)
            forced += 1
            first = min(first, i)
            rest, rm = [], []
            if i + 1 < len(exp):
                rest, rm = _continue(resume, gpu[:i + 1], len(exp) - i - 1)
            exp = exp[:i] + [gpu[i]] + [int(t) for t in rest]
            mar = mar[:i + 1] + [float(m) for m in rm[:len(rest)]]
        i += 1
    assert len(gpu) == len(exp), f"{case}: {len(gpu)} tokens, oracle {len(exp)}"
    record_greedy(case, len(exp) - forced, len(exp), forced, float(np.min(mar)) if mar else float("nan"))
    return first


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
