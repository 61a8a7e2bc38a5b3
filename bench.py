#!/usr/bin/env python3
"""Benchmark of the quantized Llama decode path on one MI355X.

Headline (`value`): Llama-2-7B-shaped Q4_0 batch-1 greedy decode, tok/s
(workload llama2_7b_q4_0_decode of chatnet_amd.workloads).  A step is one
decode token (embedding, 32 layers of fused GEMVs + attention, LM head,
device argmax) replayed as one HIP graph; the 128-token prompt is forwarded as
one span before the timed region, then exactly --steps decode tokens are
timed (KV cache grows 128 -> 128+steps).  Weights are seeded random N(0, 0.02)
quantized to Q4_0 in HBM; inputs are resident before timing starts.

Every timed run's tokens (and the logits after its prompt) are checked
against the oracle's expected outputs committed under tests/golden/
(`parity`).  Extra legs: the TinyLlama-1.1B workloads (16-token prompt + 32
tokens at context 64; 512-token span + 128 tokens), the 7B Q4_K_M-style
decode, the isolated GEMV and GEMM sweeps (cold: every launch of a timed
graph reads its own copy of the weights and each shape cycles at least 1 GiB,
so the 256 MB MALL cannot serve them), the roofline object of the dominant
kernel (the Q4_0 GEMV at the 11008 x 4096 ffn shape) and the CPU baseline
(the oracle's restatement of the reference's C# path on the host cores,
bounded samples).
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0  # dense bf16
METRIC = "decode tok/s bs1 (1.1B & 7B Q4_0); Q4_0 GEMV achieved HBM GB/s vs peak"
SWEEP = [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632), (32000, 2048), (4096, 4096), (11008, 4096)]
ROOF_SHAPE = (11008, 4096)
# legs --only can select
LEGS = ("gemv_sweep", "roofline", "kquant", "gemm_sweep", "gemm_counters", "gemv_counters", "llama7b_decode",
        "tinyllama_decode", "prefill", "sampled")
# one N = 1 chatnet_matmul per (type, M, K) for counter runs: the 7B shapes of
# the Q4_0 and K-quant decodes
COUNTER_GEMVS = [(2, 11008, 4096), (2, 4096, 11008), (12, 4096, 4096), (12, 11008, 4096), (14, 4096, 11008),
                 (14, 32000, 4096), (11, 4096, 4096), (11, 11008, 4096), (11, 4096, 11008), (13, 11008, 4096),
                 (8, 11008, 4096)]
# Q4_K_M-style mix on Llama-2-7B shapes: Q4_K attention + gate/up, Q6_K down + output
KQ4_SHAPES = [(4096, 4096), (11008, 4096)]
KQ6_SHAPES = [(4096, 11008), (32000, 4096)]
# MatVecMulGeneric types on the 7B projection shapes
GENERIC_SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008)]
ROTATE_BYTES = 1 << 30  # weight bytes each cold sweep shape cycles through
NEAR_TIE = 1e-3


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


BLOCK = {0: (1, 4), 1: (1, 2), 2: (32, 18), 8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176),
         14: (256, 210)}  # ggml type -> (weights, bytes) per block


def weight_bytes(M: int, K: int, qtype: int = 2) -> int:
    w, b = BLOCK[qtype]
    return M * K // w * b


def gemv_algorithmic_bytes(M: int, K: int, qtype: int = 2) -> int:
    # weights + x (fp32) + y (fp32)
    return weight_bytes(M, K, qtype) + 4 * K + 4 * M


def decode_gemv_bytes(cfg, mix_types) -> int:
    """Algorithmic bytes of one decode step's GEMVs (weights + fp32 x + fp32 y
    per launch): QKV, O, gate/up and down per layer, then the LM head."""
    attn, gate_up, down, out = mix_types
    kvd = cfg.kv_dim
    per_layer = (gemv_algorithmic_bytes(cfg.dim + 2 * kvd, cfg.dim, attn)
                 + gemv_algorithmic_bytes(cfg.dim, cfg.dim, attn)
                 + gemv_algorithmic_bytes(2 * cfg.hidden_dim, cfg.dim, gate_up)
                 + gemv_algorithmic_bytes(cfg.dim, cfg.hidden_dim, down))
    return cfg.n_layers * per_layer + gemv_algorithmic_bytes(cfg.vocab_size, cfg.dim, out)


# -- parity of the timed runs against the oracle's committed expected outputs --
def fixture(name: str):
    path = os.path.join(ROOT, "tests", "golden", f"workload_{name}.npz")
    return np.load(path) if os.path.exists(path) else None


def parity(name: str, tokens, prompt_logits=None):
    """Leading tokens identical to the oracle's; a first difference is
    acceptable only at a step whose oracle top-1/top-2 margin is < 1e-3."""
    fx = fixture(name)
    if fx is None:
        return {"fixture": None}
    exp = [int(t) for t in fx["tokens"]]
    got = [int(t) for t in tokens]
    n = min(len(got), len(exp))
    same = 0
    while same < n and got[same] == exp[same]:
        same += 1
    res = {"checked": n, "identical_prefix": same}
    if same < n:
        res["first_difference_oracle_margin"] = round(float(fx["margins"][same]), 6)
    res["ok"] = same == n or float(fx["margins"][same]) < NEAR_TIE
    if prompt_logits is not None:
        err = float(np.max(np.abs(np.asarray(prompt_logits) - fx["logits_prompt"])))
        res["prompt_logits_max_abs_err"] = float(f"{err:.3g}")
        res["ok"] = bool(res["ok"] and err <= 1e-2)
    return res


def decode_run(cfg, ck, prompt, steps, warmup):
    """Forward the prompt, warm up (graph capture), forward the prompt again
    and time `steps` greedy decode tokens on the device."""
    from chatnet_amd import HipLlamaModel, hiprt

    with HipLlamaModel(cfg, ck) as m:
        lp = m.forward(prompt, 0).copy()
        m.decode_greedy(max(warmup, 1))             # warm-up (also captures the graph)
        m.forward(prompt, 0)                         # reset to the prompt
        hiprt.synchronize()
        t0 = time.perf_counter()
        toks = m.decode_greedy(steps)                # synchronizes before returning
        hiprt.synchronize()
        dt = time.perf_counter() - t0
    assert len(toks) == steps, (len(toks), steps)
    return dt, toks, lp


def short_decode_run(cfg, ck, prompt, steps, repeats):
    """A short workload timed `repeats` times (forward the prompt, then
    `steps` greedy tokens timed): median decode tok/s and the last tokens."""
    from chatnet_amd import HipLlamaModel, hiprt

    rates = []
    with HipLlamaModel(cfg, ck) as m:
        lp = m.forward(prompt, 0).copy()
        m.decode_greedy(steps)                       # graph capture
        for _ in range(repeats):
            m.forward(prompt, 0)
            hiprt.synchronize()
            t0 = time.perf_counter()
            toks = m.decode_greedy(steps)
            rates.append(steps / (time.perf_counter() - t0))
    return statistics.median(rates), toks, lp


def _cold_pool(qtype, M, K, rotate_bytes):
    """Distinct copies of one seeded weight matrix, at least rotate_bytes in all."""
    from chatnet_amd import hiprt, synth

    nb = weight_bytes(M, K, qtype)
    stride = (nb + 256 + 4095) // 4096 * 4096
    copies = max(4, -(-rotate_bytes // stride))
    t = synth.tensor(qtype, 99, f"sweep{M}x{K}", M, K)
    base = hiprt.DeviceBuffer.from_numpy(t.data)
    pool = hiprt.DeviceBuffer(copies * stride)
    pool.fill(0)
    for c in range(copies):
        pool.copy_from(base, nb, dst_offset=c * stride)
    base.free()
    return pool, stride, copies


def gemv_sweep(shapes, replays=2, rotate_bytes=ROTATE_BYTES, qtype=2):
    """Cold per-launch GEMV time: one launch per weight copy (at least
    rotate_bytes of copies, so no launch finds its weights in the 256 MB MALL)
    captured into one HIP graph, so the device runs them back to back; HIP
    events on that stream time `replays` replays."""
    from chatnet_amd import hiprt, ops, synth

    res = {}
    for (M, K) in shapes:
        pool, stride, copies = _cold_pool(qtype, M, K, rotate_bytes)
        x = hiprt.DeviceBuffer.from_numpy(synth.normal(99, f"sweepx{K}", K, 1.0))
        y = hiprt.DeviceBuffer(4 * M)
        hiprt.synchronize()
        stream = hiprt.Stream()

        def issue():
            for c in range(copies):
                ops.matmul_ptr(qtype, pool.ptr + c * stride, x.ptr, y.ptr, M, K, 1, stream.h)

        graph = hiprt.Graph(stream, issue)
        graph.launch()  # warm-up
        stream.synchronize()
        e0, e1 = hiprt.Event(), hiprt.Event()
        e0.record(stream.h)
        for _ in range(replays):
            graph.launch()
        e1.record(stream.h)
        us = e0.elapsed_ms(e1) * 1000.0 / (copies * replays)
        del graph
        stream.synchronize()
        alg = gemv_algorithmic_bytes(M, K, qtype)
        res[f"{M}x{K}"] = {"us": round(us, 3), "GB/s": round(alg / us / 1e3, 1),
                           "frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 4), "alg_bytes": alg,
                           "launches": copies, "rotated_MB": round(copies * stride / 1e6, 1)}
        log(f"  gemv type {qtype} {M}x{K}: {res[f'{M}x{K}']['us']} us")
        for b in (pool, x, y):
            b.free()
    return res


def gemm_sweep(shapes, ns, rotate_bytes=ROTATE_BYTES):
    """Batched chatnet_matmul per call: the multi-column GEMV for few columns
    of smaller matrices, else x fp32 -> bf16, the MFMA GEMM and the split-K
    reduce when used; cold
    weights as in gemv_sweep (one call per weight copy); HIP events on the
    stream the calls are captured on."""
    from chatnet_amd import hiprt, ops, synth

    res = {}
    for (M, K) in shapes:
        pool, stride, copies = _cold_pool(2, M, K, rotate_bytes)
        nb = weight_bytes(M, K, 2)
        per = {}
        for N in ns:
            x = hiprt.DeviceBuffer.from_numpy(synth.normal(99, f"gemmx{N}x{K}", N * K, 1.0))
            y = hiprt.DeviceBuffer(4 * M * N)
            stream = hiprt.Stream()
            ops.matmul_ptr(2, pool.ptr, x.ptr, y.ptr, M, K, N, stream.h)  # sizes the workspace
            stream.synchronize()

            def issue():
                for c in range(copies):
                    ops.matmul_ptr(2, pool.ptr + c * stride, x.ptr, y.ptr, M, K, N, stream.h)

            graph = hiprt.Graph(stream, issue)
            graph.launch()
            stream.synchronize()
            e0, e1 = hiprt.Event(), hiprt.Event()
            replays = 2
            e0.record(stream.h)
            for _ in range(replays):
                graph.launch()
            e1.record(stream.h)
            us = e0.elapsed_ms(e1) * 1000.0 / (copies * replays)
            del graph
            stream.synchronize()
            alg = nb + 4 * K * N + 4 * M * N
            tflops = 2.0 * M * N * K / us / 1e6
            gemv = N < 8 or (N <= 16 and M * K * N <= 8 * 4096 * 4096)  # the library's choice
            per[str(N)] = {"path": "multi-column GEMV" if gemv else "MFMA GEMM", "us": round(us, 2),
                           "GB/s": round(alg / us / 1e3, 1), "hbm_frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 4),
                           "TFLOP/s": round(tflops, 1),
                           "mfma_frac": None if gemv else round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                           "launches": copies}
            x.free()
            y.free()
        res[f"{M}x{K}"] = per
        log(f"  gemm {M}x{K}: {json.dumps(per)}")
        pool.free()
    return res


def gemm_counters(shapes, ns=(64, 512)):
    """One chatnet_matmul call per shape and N (warm weights), for counter
    collection, where every dispatch is serialized by the profiler."""
    from chatnet_amd import hiprt, ops, synth

    for (M, K) in shapes:
        w = hiprt.DeviceBuffer.from_numpy(synth.tensor(2, 7, f"ctr{M}x{K}", M, K).data, pad=256)
        for N in ns:
            x = hiprt.DeviceBuffer.from_numpy(synth.normal(99, f"gemmx{N}x{K}", N * K, 1.0))
            y = hiprt.DeviceBuffer(4 * M * N)
            ops.matmul_ptr(2, w.ptr, x.ptr, y.ptr, M, K, N, 0)
            hiprt.synchronize()
            x.free()
            y.free()
            log(f"  counters: {M}x{K} N={N} done")
        w.free()


def gemv_counters(cases=COUNTER_GEMVS):
    """One N = 1 chatnet_matmul per (type, M, K), direct launches, each on its
    own freshly uploaded weights, for counter collection."""
    from chatnet_amd import hiprt, ops, synth

    for (qt, M, K) in cases:
        w = hiprt.DeviceBuffer.from_numpy(synth.tensor(qt, 7, f"gctr{qt}-{M}x{K}", M, K).data, pad=256)
        x = hiprt.DeviceBuffer.from_numpy(synth.normal(99, f"gctrx{K}", K, 1.0))
        y = hiprt.DeviceBuffer(4 * M)
        ops.matmul_ptr(qt, w.ptr, x.ptr, y.ptr, M, K, 1, 0)
        hiprt.synchronize()
        for b in (w, x, y):
            b.free()
        log(f"  counters: type {qt} {M}x{K} done")


def copy_rate(nbytes=512 << 20, reps=5):
    """The box's measured streaming rate: a device-to-device copy of nbytes
    (read + write bytes per second), HIP events on the null stream."""
    from chatnet_amd import hiprt

    a, b = hiprt.DeviceBuffer(nbytes), hiprt.DeviceBuffer(nbytes)
    a.fill(1)
    b.copy_from(a, nbytes)
    hiprt.synchronize()
    e0, e1 = hiprt.Event(), hiprt.Event()
    e0.record(0)
    for _ in range(reps):
        b.copy_from(a, nbytes)
    e1.record(0)
    ms = e0.elapsed_ms(e1)
    a.free()
    b.free()
    return round(2 * nbytes * reps / (ms * 1e-3) / 1e9, 1)


def sampled_run(cfg, ck, prompt, steps):
    """Decode tok/s with the device temperature sampler (T 0.8, top-k 40,
    top-p 0.9, seed 1) in place of the argmax, prompt included in the call."""
    from chatnet_amd import HipLlamaModel

    with HipLlamaModel(cfg, ck) as m:
        m.generate_sampled(prompt, 8, 0.8, 40, 0.9, 1)  # warm-up, graph capture
        t0 = time.perf_counter()
        m.forward(prompt, 0)
        t1 = time.perf_counter()
        toks = m.generate_sampled(prompt, steps, 0.8, 40, 0.9, 1)
        t2 = time.perf_counter()
    assert len(toks) == steps
    return round(steps / ((t2 - t1) - (t1 - t0)), 1)


def prefill_run(w, ck):
    """Time to first token of the workload's prompt forwarded as one span,
    then its greedy decode tokens; both checked against the fixture."""
    from chatnet_amd import HipLlamaModel, hiprt

    prompt = w.prompt()
    with HipLlamaModel(w.config, ck) as m:
        m.forward(prompt, 0)  # warm-up: span buffers, kernel attributes
        m.decode_greedy(4)
        hiprt.synchronize()
        t0 = time.perf_counter()
        lp = m.forward(prompt, 0).copy()  # returns after the logits are on the host
        t1 = time.perf_counter()
        toks = m.decode_greedy(w.n_decode)
        t2 = time.perf_counter()
    assert len(toks) == w.n_decode
    return {"prompt_tokens": w.n_prompt, "ttft_ms": round((t1 - t0) * 1e3, 3),
            "prefill_tok_s": round(w.n_prompt / (t1 - t0), 1), "decode_tokens": w.n_decode,
            "decode_tok_s": round(w.n_decode / (t2 - t1), 1), "parity": parity(w.name, toks, lp)}


def profile_value(path: str, key: str):
    """The text after `key:` on its line in a committed profiles/ summary."""
    try:
        with open(os.path.join(ROOT, "profiles", path)) as f:
            for line in f:
                if line.startswith(key + ":"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def profile_figure(path: str, key: str):
    """A number recorded as `key: value` in a committed profiles/ summary."""
    v = profile_value(path, key)
    try:
        return float(v.split()[0]) if v else None
    except ValueError:
        return None


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg7, ck7, w1, ck1):
    """The oracle (C restatement of the reference's CPU path) on the host
    cores, bounded samples: the 7B decode (headline unit), the TinyLlama
    workload (its 16-token prompt and 32 greedy tokens) at all threads and a
    shorter sample at one thread, and the isolated Q4_0 GEMV at the seven
    sweep shapes (N = 1; the reference has no batched product)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle
    from chatnet_amd import synth

    cores = int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))

    def decode_rate(cfg, ck, prompt_len, decode, threads):
        oracle.set_threads(threads)
        ora = oracle.OracleLlama(cfg, ck)
        logits = ora.forward(list(range(1, prompt_len + 1)), 0)
        tok = oracle.argmax(logits)
        t0 = time.perf_counter()
        for j in range(decode):
            logits = ora.forward([tok], prompt_len + j)
            tok = oracle.argmax(logits)
        dt = time.perf_counter() - t0
        ora.close()
        return decode / dt

    def workload_rate(w, ck, threads):
        """The workload's prompt token by token, then its greedy decode
        (InferenceEngine.Generate's loop); decode tok/s and the tokens."""
        oracle.set_threads(threads)
        ora = oracle.OracleLlama(w.config, ck)
        logits = None
        for i, tk in enumerate(w.prompt()):
            logits = ora.forward([int(tk)], i)
        toks = []
        t0 = time.perf_counter()
        pos = w.n_prompt
        for _ in range(w.n_decode):
            tok = oracle.argmax(logits)
            toks.append(tok)
            logits = ora.forward([tok], pos)
            pos += 1
        dt = time.perf_counter() - t0
        ora.close()
        return w.n_decode / dt, toks

    v7 = decode_rate(cfg7, ck7, 4, 8, cores)
    legs = {"cpu_model": cpu_model(), "host_threads_visible": os.cpu_count(), "threads_used": cores}
    if w1 is not None:
        r1, toks1 = workload_rate(w1, ck1, cores)
        legs["tinyllama_q4_0_decode_tok_s"] = round(r1, 3)
        legs["tinyllama_q4_0_decode_workload"] = f"{w1.n_prompt}-token prompt, {w1.n_decode} greedy tokens timed"
        fx = fixture(w1.name)
        legs["tinyllama_q4_0_decode_tokens_match_fixture"] = (
            None if fx is None else [int(t) for t in fx["tokens"]] == [int(t) for t in toks1])
        legs["tinyllama_q4_0_decode_tok_s_1_thread"] = round(decode_rate(w1.config, ck1, 2, 4, 1), 3)
    oracle.set_threads(cores)
    reps = 5
    gbs = {}
    for (M, K) in SWEEP:
        t = synth.tensor(2, 99, f"sweep{M}x{K}", M, K)
        x = synth.normal(99, f"sweepx{K}", K, 1.0)
        oracle.matvec(2, t.data, x, M, K)
        t0 = time.perf_counter()
        for _ in range(reps):
            oracle.matvec(2, t.data, x, M, K)
        dt = (time.perf_counter() - t0) / reps
        gbs[f"{M}x{K}"] = round(gemv_algorithmic_bytes(M, K) / dt / 1e9, 2)
    legs["gemv_q4_0_n1_GBs"] = gbs
    oracle.set_threads(1)
    return {"value": round(v7, 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"oracle LlamaModel.Forward restatement, {cfg7.n_layers}-layer {cfg7.dim}-dim Q4_0, "
                      f"4-token prompt then 8 greedy decode tokens timed, row-parallel over {cores} threads; "
                      f"legs: the TinyLlama-shaped 16+32 workload at {cores} threads (4 tokens at 1 thread) "
                      f"and {reps} isolated Q4_0 GEMVs per sweep shape",
            "legs": legs}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-tinyllama", action="store_true")
    ap.add_argument("--no-gemm", action="store_true", help="skip the batched GEMM sweep")
    ap.add_argument("--no-kquant", action="store_true", help="skip the Q4_K / Q6_K / Q8_0 / Q5_K legs")
    ap.add_argument("--roofline-only", action="store_true", help="only the isolated GEMV legs")
    ap.add_argument("--only", choices=LEGS, help="run this one leg (for profiling); the line carries what it measured")
    args = ap.parse_args()

    def want(leg: str) -> bool:
        return args.only is None or args.only == leg
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)

    from chatnet_amd import QWEN2_0_5B, _native, hiprt, synth
    from chatnet_amd.workloads import WORKLOADS

    if hiprt.device_count() < 1:
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    copy_gbs = sweep = None
    roof = {}
    if args.only == "roofline":  # the roofline shape alone (counter runs)
        sweep = gemv_sweep([ROOF_SHAPE])
        roof = sweep[f"{ROOF_SHAPE[0]}x{ROOF_SHAPE[1]}"]
    if want("gemv_sweep"):
        copy_gbs = copy_rate()
        log(f"device-to-device copy: {copy_gbs} GB/s (read + write)")
        log("gemv sweep (cold: one launch per weight copy, >= 1 GiB of copies per shape)")
        sweep = gemv_sweep(SWEEP)
        roof = sweep[f"{ROOF_SHAPE[0]}x{ROOF_SHAPE[1]}"]
        log(f"sweep: {json.dumps(sweep)}")

    value = ms = None
    cpu = None
    tiny = None
    tiny_sampled = None
    gsweep = None
    prefill = None
    kq = None
    qwen = None
    fp16kv = None
    par = {}
    if not args.roofline_only and not args.no_kquant and want("kquant"):
        log("Q4_K / Q6_K / Q8_0 / Q5_K / Q3_K / F16 gemv (cold), 7B Q4_K_M- and Q3_K_M-style 64-token decodes")
        kq = {"gemv_q4_k_cold": gemv_sweep(KQ4_SHAPES, qtype=12),
              "gemv_q6_k_cold": gemv_sweep(KQ6_SHAPES, qtype=14),
              "gemv_q8_0_cold": gemv_sweep(GENERIC_SHAPES, qtype=8),
              "gemv_q5_k_cold": gemv_sweep(GENERIC_SHAPES, qtype=13),
              "gemv_q3_k_cold": gemv_sweep(GENERIC_SHAPES, qtype=11),
              "gemv_f16_cold": gemv_sweep(GENERIC_SHAPES[:2], qtype=1)}
        wk = WORKLOADS["llama2_7b_q4_k_m_decode"]
        ckk = wk.checkpoint()
        dtk, tk, lpk = decode_run(wk.config, ckk, wk.prompt(), wk.n_decode, 4)
        kq["llama2_7b_q4_k_m_decode_tok_s"] = round(wk.n_decode / dtk, 1)
        kq["weights_GB"] = round(synth.checkpoint_bytes(ckk) / 1e9, 3)
        par[wk.name] = parity(wk.name, tk, lpk)
        del ckk
        # the same shape in a Q3_K_M-style mix, every matrix read from its
        # stored blocks: Q3_K attention and gate/up, Q4_K down, Q6_K head
        w3 = WORKLOADS["llama2_7b_q3_k_m_decode"]
        ck3 = w3.checkpoint()
        dt3, t3, lp3 = decode_run(w3.config, ck3, w3.prompt(), w3.n_decode, 4)
        kq["llama2_7b_q3_k_m_decode_tok_s"] = round(w3.n_decode / dt3, 1)
        kq["q3_k_m_weights_GB"] = round(synth.checkpoint_bytes(ck3) / 1e9, 3)
        par[w3.name] = parity(w3.name, t3, lp3)
        del ck3
        log(f"  {json.dumps(kq)}")
    if args.only == "gemm_counters":
        log("gemm counter leg: one call per shape, N = 64 and 512")
        gemm_counters(SWEEP)
    if args.only == "gemv_counters":
        log("gemv counter leg: one N = 1 call per type and shape")
        gemv_counters()
    if not args.roofline_only and not args.no_gemm and want("gemm_sweep"):
        log("gemm sweep N = 8, 64, 512 (cold)")
        gsweep = gemm_sweep(SWEEP, (8, 64, 512))
        log(f"gemm sweep: {json.dumps(gsweep)}")
    if not args.roofline_only and want("llama7b_decode"):
        w7 = WORKLOADS["llama2_7b_q4_0_decode"]
        cfg7 = w7.config
        log("generating Llama-2-7B-shaped Q4_0 checkpoint")
        t0 = time.perf_counter()
        ck7 = w7.checkpoint()
        log(f"  {synth.checkpoint_bytes(ck7) / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")
        prompt = w7.prompt()
        log(f"7B decode: prompt {w7.n_prompt} (one span), warmup {args.warmup}, timed {args.steps}")
        dt, toks7, lp7 = decode_run(cfg7, ck7, prompt, args.steps, args.warmup)
        value = args.steps / dt
        ms = dt * 1000.0 / args.steps
        par[w7.name] = parity(w7.name, toks7, lp7)
        log(f"  {value:.1f} tok/s ({ms:.3f} ms/token); parity {json.dumps(par[w7.name])}")
        dt16, toks16, _ = decode_run(cfg7.replace(kv_dtype=_native.KV_F16), ck7, prompt, args.steps, args.warmup)
        fp16kv = round(args.steps / dt16, 1)
        log(f"  fp16 KV cache: {fp16kv} tok/s")
        w1 = WORKLOADS["tinyllama_q4_0_decode"]
        if not args.no_cpu and args.only is None:
            log("cpu baseline (oracle on host cores)")
            cpu = cpu_baseline(cfg7, ck7, w1, w1.checkpoint())
            log(f"  {cpu['value']} tok/s on {cpu['cores']} threads; {json.dumps(cpu['legs'])}")
        del ck7
    if not args.roofline_only and not args.no_tinyllama:
        if want("tinyllama_decode"):
            w1 = WORKLOADS["tinyllama_q4_0_decode"]
            ck1 = w1.checkpoint()
            rate1, toks1, lp1 = short_decode_run(w1.config, ck1, w1.prompt(), w1.n_decode, 20)
            tiny = round(rate1, 1)
            par[w1.name] = parity(w1.name, toks1, lp1)
            log(f"TinyLlama decode ({w1.n_prompt}-token prompt, {w1.n_decode} tokens, context "
                f"{w1.config.context_length}): {tiny} tok/s; parity {json.dumps(par[w1.name])}")
            if args.only is None:
                tiny_sampled = sampled_run(w1.config.replace(context_length=2048), ck1, w1.prompt(), 128)
                log(f"TinyLlama decode, temperature sampler on the device: {tiny_sampled} tok/s")
            del ck1
        if args.only == "sampled":  # the sampled decode alone (for profiling)
            w1 = WORKLOADS["tinyllama_q4_0_decode"]
            tiny_sampled = sampled_run(w1.config.replace(context_length=2048), w1.checkpoint(), w1.prompt(), 128)
            log(f"TinyLlama decode, temperature sampler on the device: {tiny_sampled} tok/s")
        if want("prefill"):
            w2 = WORKLOADS["tinyllama_q4_0_prefill"]
            log(f"TinyLlama {w2.n_prompt}-token prefill + {w2.n_decode} decode")
            prefill = prefill_run(w2, w2.checkpoint())
            log(f"  {json.dumps(prefill)}")
        if args.only is None:
            cfgq = QWEN2_0_5B.replace(context_length=2048)
            ckq = synth.llama_checkpoint(cfgq, seed=5, mix="q8_0", with_output=False, embedding=_native.GGML_Q8_0)
            pq = synth.tokens(5, "prompt", 16, cfgq.vocab_size)
            dtq, _, _ = decode_run(cfgq, ckq, pq, 128, 8)
            qwen = {"qwen2_0_5b_q8_0_decode_tok_s": round(128 / dtq, 1),
                    "weights_GB": round(synth.checkpoint_bytes(ckq) / 1e9, 3)}
            log(f"Qwen2-0.5B-shaped Q8_0 (tied embeddings, QKV biases) decode: {json.dumps(qwen)}")
            del ckq

    tiny_gemv_bytes = decode_gemv_bytes(WORKLOADS["tinyllama_q4_0_decode"].config, (2, 2, 2, 2))
    tiny_gemv_us = profile_figure("tinyllama_q4_0_decode_kernels.md", "gemv_us_per_token")
    res = {
        "metric": METRIC,
        "value": round(value, 2) if value else None,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4) if ms else None,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded N(0,0.02) weights quantized to Q4_0, seeded prompt ids)",
        "config": {"workload": "llama2-7b-q4_0-decode-bs1", "prompt_tokens": 128, "prompt_as": "one span",
                   "decode_tokens": args.steps, "kv_cache": "f32", "context_length": 2048,
                   "weights": "Q4_0 (all matrices)",
                   "llama2_7b_q4_0_fp16_kv_decode_tok_s": fp16kv,
                   "tinyllama_1b_q4_0_decode_tok_s": tiny,
                   "tinyllama_1b_q4_0_decode_workload": "16-token prompt, 32 greedy tokens, context 64, "
                                                       "median of 20 timed runs",
                   "tinyllama_1b_q4_0_sampled_decode_tok_s": tiny_sampled},
        "parity": par,
        "tinyllama_decode": {
            "step_frac_of_hbm_roofline": (round(tiny * decode_gemv_bytes(
                WORKLOADS["tinyllama_q4_0_decode"].config, (2, 2, 2, 2)) / 1e9 / HBM_PEAK_GBS, 4) if tiny else None),
            "gemv_alg_bytes_per_token": tiny_gemv_bytes,
            "gemv_us_per_token": tiny_gemv_us,
            "gemv_frac_of_hbm_peak": (round(tiny_gemv_bytes / (tiny_gemv_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
                                      if tiny_gemv_us else None),
            "gemv_source": "profiles/tinyllama_q4_0_decode_kernels.md (rocprofv3 kernel trace of the workload, "
                           "read from the committed summary, not measured by this run)",
            "gemv_source_commit": profile_value("tinyllama_q4_0_decode_kernels.md", "commit")},
        "gemv_sweep_q4_0_n1_cold": sweep,
        "gemm_sweep_q4_0_cold": gsweep,
        "tinyllama_q4_0_prefill": prefill,
        "llama2_7b_q4_k_m": kq,
        "qwen2_0_5b_q8_0": qwen,
        "roofline": {"bound": "hbm", "achieved": roof.get("GB/s"), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": roof.get("frac"),
                     "traffic": profile_figure("gemv_q4_0_sweep_roofline.md",
                                               f"traffic_bytes_per_launch {ROOF_SHAPE[0]}x{ROOF_SHAPE[1]}"),
                     "traffic_source": "profiles/gemv_q4_0_sweep_roofline.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)",
                     "traffic_source_commit": profile_value("gemv_q4_0_sweep_roofline.md", "commit"),
                     "kernel": "gemv_kernel<Q4_0> (chatnet_matmul N=1) at 11008x4096, cold",
                     "alg_bytes_per_launch": roof.get("alg_bytes"), "avg_launch_us": roof.get("us"),
                     "measured_copy_GBs": copy_gbs,
                     "measured_copy_note": "512 MiB device-to-device copy, read + write bytes per second"},
        "cpu_baseline": cpu,
    }
    if res["tinyllama_decode"]["gemv_us_per_token"] is not None:
        res["tinyllama_decode"]["gemv_us_per_token"] = round(tiny_gemv_us, 2)
    if res["roofline"]["traffic"] is not None:
        res["roofline"]["traffic"] = int(res["roofline"]["traffic"])
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
