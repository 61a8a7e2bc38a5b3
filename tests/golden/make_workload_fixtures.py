"""Writes tests/golden/workload_<name>.npz: the oracle's expected output for
each named end-to-end workload of chatnet_amd.workloads (run from the
repository root; the 7B workloads take a few minutes of CPU each).

A fixture is data only: the workload's prompt, a digest of every byte of the
regenerated checkpoint (the weights themselves are a pure function of the
seed and are never stored), the logits after the prompt, the greedy tokens of
InferenceEngine.Generate's loop (InferenceEngine.cs:234-307, no EOS stop) with
each step's top-1/top-2 logit margin, and the logits after the last decode
token was forwarded.

    python tests/golden/make_workload_fixtures.py [--threads N] [--digest-only] [name ...]

--digest-only regenerates each named checkpoint and rewrites only the digest
field of its existing fixture (the expected outputs are left as they are).
"""
import argparse
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle")]

import oracle  # noqa: E402
from chatnet_amd.workloads import WORKLOADS, checkpoint_digest  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def margin(logits: np.ndarray) -> float:
    top2 = np.partition(np.asarray(logits, np.float32), -2)[-2:]
    return float(abs(top2[1] - top2[0]))


def make(name: str) -> str:
    w = WORKLOADS[name]
    t0 = time.time()
    ck = w.checkpoint()
    prompt = w.prompt()
    digest = checkpoint_digest(ck)
    ora = oracle.OracleLlama(w.config, ck)
    logits_prompt = ora.forward(prompt, 0).copy()
    logits = logits_prompt
    toks, margins = [], []
    pos = w.n_prompt
    for _ in range(w.n_decode):
        nxt = oracle.argmax(logits)
        margins.append(margin(logits))
        toks.append(nxt)
        if pos >= w.config.context_length - 1:
            break
        logits = ora.forward([nxt], pos)
        pos += 1
    ora.close()
    path = os.path.join(OUT, f"workload_{name}.npz")
    np.savez_compressed(path, prompt=prompt.astype(np.int32), tokens=np.array(toks, np.int32),
                        margins=np.array(margins, np.float32), logits_prompt=logits_prompt.astype(np.float32),
                        logits_final=np.asarray(logits, np.float32), digest=digest, seed=w.seed, mix=w.mix,
                        n_prompt=w.n_prompt, n_decode=w.n_decode)
    print(f"{name}: {len(toks)} tokens, min margin {min(margins):.3g}, {time.time() - t0:.0f} s -> {path}",
          flush=True)
    return path


def redigest(name: str) -> str:
    path = os.path.join(OUT, f"workload_{name}.npz")
    with np.load(path, allow_pickle=False) as z:
        fields = {k: z[k] for k in z.files}
    fields["digest"] = checkpoint_digest(WORKLOADS[name].checkpoint())
    np.savez_compressed(path, **fields)
    print(f"{name}: digest {fields['digest']} -> {path}", flush=True)
    return path


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--threads", type=int, default=os.cpu_count() or 1)
    ap.add_argument("--digest-only", action="store_true")
    ap.add_argument("names", nargs="*")
    args = ap.parse_args()
    oracle.set_threads(args.threads)
    for name in args.names or list(WORKLOADS):
        (redigest if args.digest_only else make)(name)


if __name__ == "__main__":
    main()
