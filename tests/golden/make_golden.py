"""Writes the golden fixtures of tests/golden/ (run from the repository root).

Fixtures are data only: seeded inputs and the CPU oracle's outputs for them.
  blocks_{q4_0,q4_1,q5_0,q5_1,q8_0,q2_k,q3_k,q4_k,q5_k,q6_k,q8_k}.npz and
  blocks_{iq2_xxs,iq2_xs,iq3_xxs,iq1_s,iq4_nl,iq3_s,iq2_s,iq4_xs,iq1_m}.npz
      raw blocks of 16 rows x 512 weights, an x vector, and the oracle's
      dequantized rows and row dots (DequantQ*.Dequantize / DotProduct).
  tiny_llama_q4_0.npz
      a 2-layer dim-256 Llama (TINY_TEST shape) regenerated from its seed: the
      prompt, the logits after the prompt and 16 greedy tokens.
The weights of the tiny model are not stored: they are a pure function of the
seed (chatnet_amd.synth), and the test regenerates and checksums them.
Existing fixtures are kept (their bytes would only differ in zip timestamps);
pass --force to rewrite them.
"""
import hashlib
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "oracle")]

import oracle  # noqa: E402
from chatnet_amd import TINY_TEST, synth  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))


def checkpoint_digest(ck) -> str:
    h = hashlib.sha256()
    for name in sorted(ck):
        h.update(name.encode())
        h.update(np.ascontiguousarray(ck[name].data).tobytes())
    return h.hexdigest()


def main():
    force = "--force" in sys.argv[1:]
    for qtype, tag in ((oracle.Q4_0, "q4_0"), (oracle.Q4_K, "q4_k"), (oracle.Q6_K, "q6_k"), (oracle.Q8_0, "q8_0"),
                       (oracle.Q5_K, "q5_k"), (oracle.Q4_1, "q4_1"), (oracle.Q5_0, "q5_0"), (oracle.Q5_1, "q5_1"),
                       (oracle.Q2_K, "q2_k"), (oracle.Q3_K, "q3_k"), (oracle.Q8_K, "q8_k"),
                       (oracle.IQ2_XXS, "iq2_xxs"), (oracle.IQ2_XS, "iq2_xs"), (oracle.IQ3_XXS, "iq3_xxs"),
                       (oracle.IQ1_S, "iq1_s"), (oracle.IQ4_NL, "iq4_nl"), (oracle.IQ3_S, "iq3_s"),
                       (oracle.IQ2_S, "iq2_s"), (oracle.IQ4_XS, "iq4_xs"), (oracle.IQ1_M, "iq1_m")):
        if os.path.exists(os.path.join(OUT, f"blocks_{tag}.npz")) and not force:
            continue
        rows, K = 16, 512
        t = synth.tensor(qtype, 2024, f"golden-{tag}", rows, K)
        x = synth.normal(2024, f"golden-x-{tag}", K, 1.0)
        deq = oracle.dequant(qtype, t.data, rows * K).reshape(rows, K)
        dots = oracle.matvec(qtype, t.data, x, rows, K)
        np.savez_compressed(os.path.join(OUT, f"blocks_{tag}.npz"), raw=t.data, x=x, dequant=deq, dots=dots,
                            rows=rows, K=K, ggml_type=qtype)
    if os.path.exists(os.path.join(OUT, "tiny_llama_q4_0.npz")) and not force:
        print("fixtures written to", OUT)
        return
    cfg = TINY_TEST
    ck = synth.llama_checkpoint(cfg, seed=77, mix="q4_0")
    prompt = synth.tokens(77, "golden-prompt", 8, cfg.vocab_size)
    ora = oracle.OracleLlama(cfg, ck)
    logits = ora.forward(prompt, 0)
    ora2 = oracle.OracleLlama(cfg, ck)
    toks, margins = ora2.generate_greedy(list(prompt), 16)
    np.savez_compressed(os.path.join(OUT, "tiny_llama_q4_0.npz"), prompt=prompt, logits=logits,
                        tokens=np.array(toks, np.int32), margins=np.array(margins, np.float32),
                        seed=77, digest=checkpoint_digest(ck))
    print("fixtures written to", OUT)


if __name__ == "__main__":
    main()
