#!/usr/bin/env python3
"""Benchmark of the quantized Llama decode path on one MI355X.

Headline (`value`): Llama-2-7B-shaped Q4_0 batch-1 greedy decode, tok/s.
A step is one decode token (embedding, 32 layers of fused GEMVs + attention,
LM head, device argmax) replayed as one HIP graph; the 128-token prompt is
forwarded before the timed region, then exactly --steps decode tokens are
timed (KV cache grows 128 -> 128+steps).  Weights are seeded random N(0, 0.02)
quantized to Q4_0 in HBM; inputs are resident before timing starts.

Extra fields: TinyLlama-1.1B decode tok/s, the isolated Q4_0 GEMV sweep
(achieved HBM GB/s per shape, cold: every launch reads a different copy of the
weights, >= 1 GiB in rotation so the 256 MB MALL cannot serve them), the
roofline object of the dominant kernel (the Q4_0 GEMV at the 11008 x 4096
ffn shape) and the CPU baseline (the oracle's restatement of the reference's
C# path on the host cores, bounded sample).
"""
from __future__ import annotations

import argparse
import json
import os
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
# Q4_K_M-style mix on Llama-2-7B shapes: Q4_K attention + gate/up, Q6_K down + output
KQ4_SHAPES = [(4096, 4096), (11008, 4096)]
KQ6_SHAPES = [(4096, 11008), (32000, 4096)]
# MatVecMulGeneric types on the 7B projection shapes
GENERIC_SHAPES = [(4096, 4096), (11008, 4096), (4096, 11008)]


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


BLOCK = {2: (32, 18), 8: (32, 34), 12: (256, 144), 13: (256, 176), 14: (256, 210)}  # ggml type -> (weights, bytes) per block


def weight_bytes(M: int, K: int, qtype: int = 2) -> int:
    w, b = BLOCK[qtype]
    return M * K // w * b


def q4_0_bytes(M: int, K: int) -> int:
    return weight_bytes(M, K, 2)


def gemv_algorithmic_bytes(M: int, K: int, qtype: int = 2) -> int:
    # weights + x (fp32) + y (fp32)
    return weight_bytes(M, K, qtype) + 4 * K + 4 * M


def decode_run(cfg, ck, prompt, steps, warmup):
    from chatnet_amd import HipLlamaModel, hiprt

    with HipLlamaModel(cfg, ck) as m:
        m.forward(prompt, 0)
        m.decode_greedy(max(warmup, 1))             # warm-up (also captures the graph)
        m.forward(prompt, 0)                         # reset to the prompt
        hiprt.synchronize()
        t0 = time.perf_counter()
        toks = m.decode_greedy(steps)                # synchronizes before returning
        hiprt.synchronize()
        dt = time.perf_counter() - t0
    assert len(toks) == steps, (len(toks), steps)
    return dt, toks


def gemv_sweep(shapes, launches_per_shape=64, replays=5, rotate_bytes=1 << 30, qtype=2):
    """Cold per-launch GEMV time: `launches_per_shape` launches over distinct
    weight copies are captured into one HIP graph, so the device runs them
    back to back, and HIP events on that stream time `replays` replays."""
    from chatnet_amd import hiprt, ops, synth

    res = {}
    for (M, K) in shapes:
        nb = weight_bytes(M, K, qtype)
        stride = (nb + 256 + 4095) // 4096 * 4096
        copies = max(4, min(256, -(-rotate_bytes // stride)))
        t = synth.tensor(qtype, 99, f"sweep{M}x{K}", M, K)
        base = hiprt.DeviceBuffer.from_numpy(t.data)
        pool = hiprt.DeviceBuffer(copies * stride)
        pool.fill(0)
        for c in range(copies):
            pool.copy_from(base, nb, dst_offset=c * stride)
        x = hiprt.DeviceBuffer.from_numpy(synth.normal(99, f"sweepx{K}", K, 1.0))
        y = hiprt.DeviceBuffer(4 * M)
        hiprt.synchronize()
        stream = hiprt.Stream()

        def issue():
            for i in range(launches_per_shape):
                c = i % copies
                ops.matmul_ptr(qtype, pool.ptr + c * stride, x.ptr, y.ptr, M, K, 1, stream.h)

        graph = hiprt.Graph(stream, issue)
        graph.launch()  # warm-up
        stream.synchronize()
        e0, e1 = hiprt.Event(), hiprt.Event()
        e0.record(stream.h)
        for _ in range(replays):
            graph.launch()
        e1.record(stream.h)
        us = e0.elapsed_ms(e1) * 1000.0 / (launches_per_shape * replays)
        del graph
        stream.synchronize()
        alg = gemv_algorithmic_bytes(M, K, qtype)
        res[f"{M}x{K}"] = {"us": round(us, 3), "GB/s": round(alg / us / 1e3, 1),
                           "frac": round(alg / us / 1e3 / HBM_PEAK_GBS, 4), "alg_bytes": alg}
        for b in (pool, base, x, y):
            b.free()
    return res


def gemm_sweep(shapes, ns, rotate_bytes=1 << 30):
    """Batched chatnet_matmul (x fp32 -> bf16, MFMA GEMM, split-K reduce when
    used) per call, cold weights as in gemv_sweep; HIP events on the stream the
    calls are captured on."""
    from chatnet_amd import hiprt, ops, synth

    res = {}
    for (M, K) in shapes:
        nb = q4_0_bytes(M, K)
        stride = (nb + 256 + 4095) // 4096 * 4096
        copies = max(4, min(64, -(-rotate_bytes // stride)))
        t = synth.tensor(2, 99, f"sweep{M}x{K}", M, K)
        base = hiprt.DeviceBuffer.from_numpy(t.data)
        pool = hiprt.DeviceBuffer(copies * stride)
        pool.fill(0)
        for c in range(copies):
            pool.copy_from(base, nb, dst_offset=c * stride)
        per = {}
        for N in ns:
            x = hiprt.DeviceBuffer.from_numpy(synth.normal(99, f"gemmx{N}x{K}", N * K, 1.0))
            y = hiprt.DeviceBuffer(4 * M * N)
            stream = hiprt.Stream()
            launches = 32 if N <= 64 else 8
            ops.matmul_ptr(2, pool.ptr, x.ptr, y.ptr, M, K, N, stream.h)  # sizes the workspace
            stream.synchronize()

            def issue():
                for i in range(launches):
                    ops.matmul_ptr(2, pool.ptr + (i % copies) * stride, x.ptr, y.ptr, M, K, N, stream.h)

            graph = hiprt.Graph(stream, issue)
            graph.launch()
            stream.synchronize()
            e0, e1 = hiprt.Event(), hiprt.Event()
            replays = 3
            e0.record(stream.h)
            for _ in range(replays):
                graph.launch()
            e1.record(stream.h)
            us = e0.elapsed_ms(e1) * 1000.0 / (launches * replays)
            del graph
            stream.synchronize()
            alg = nb + 4 * K * N + 4 * M * N
            tflops = 2.0 * M * N * K / us / 1e6
            per[str(N)] = {"us": round(us, 2), "GB/s": round(alg / us / 1e3, 1), "TFLOP/s": round(tflops, 1),
                           "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)}
            x.free()
            y.free()
        res[f"{M}x{K}"] = per
        pool.free()
        base.free()
    return res


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


def prefill_run(cfg, ck, n_prompt, n_decode):
    """Time to first token of an n_prompt-token prompt forwarded as one span,
    then n_decode greedy decode tokens."""
    from chatnet_amd import HipLlamaModel, hiprt, synth

    prompt = synth.tokens(77, "prefill", n_prompt, cfg.vocab_size)
    with HipLlamaModel(cfg, ck) as m:
        m.forward(prompt, 0)  # warm-up: span buffers, kernel attributes
        m.decode_greedy(4)
        hiprt.synchronize()
        t0 = time.perf_counter()
        m.forward(prompt, 0)  # returns after the logits are on the host
        t1 = time.perf_counter()
        toks = m.decode_greedy(n_decode)
        t2 = time.perf_counter()
    assert len(toks) == n_decode
    return {"prompt_tokens": n_prompt, "ttft_ms": round((t1 - t0) * 1e3, 3),
            "prefill_tok_s": round(n_prompt / (t1 - t0), 1), "decode_tokens": n_decode,
            "decode_tok_s": round(n_decode / (t2 - t1), 1)}


def measured_traffic(shape):
    """HBM bytes per launch of the roofline GEMV, from the committed
    rocprofv3 FETCH_SIZE + WRITE_SIZE summary (counters scaled by the same
    counters read on a copy kernel of known size), or None if absent."""
    path = os.path.join(ROOT, "profiles", "gemv_q4_0_sweep_roofline.md")
    key = f"traffic_bytes_per_launch {shape[0]}x{shape[1]}:"
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(key):
                    return int(line[len(key):].strip())
    except OSError:
        pass
    return None


def cpu_baseline(cfg, ck, prompt_len=4, decode=8):
    """The oracle (C restatement of the reference's CPU path) on the host cores."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle

    cores = int(os.environ.get("OMP_NUM_THREADS") or len(os.sched_getaffinity(0)))
    oracle.set_threads(cores)
    ora = oracle.OracleLlama(cfg, ck)
    prompt = list(range(1, prompt_len + 1))
    t0 = time.perf_counter()
    for i, tk in enumerate(prompt):
        logits = ora.forward([tk], i)
    t1 = time.perf_counter()
    tok = oracle.argmax(logits)
    for j in range(decode):
        logits = ora.forward([tok], prompt_len + j)
        tok = oracle.argmax(logits)
    t2 = time.perf_counter()
    ora.close()
    oracle.set_threads(1)
    return {"value": round(decode / (t2 - t1), 3), "unit": "tok/s", "cores": cores, "kind": "port",
            "sample": f"oracle LlamaModel.Forward restatement, {cfg.n_layers}-layer {cfg.dim}-dim Q4_0, "
                      f"{prompt_len}-token prompt then {decode} greedy decode tokens timed "
                      f"(positions {prompt_len}..{prompt_len + decode - 1}), row-parallel over {cores} threads"}


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
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {args.gpus}); "
              "multi-GPU sharding is design-only", file=sys.stderr)
        sys.exit(2)

    from chatnet_amd import LLAMA2_7B, QWEN2_0_5B, TINYLLAMA_1B, _native, hiprt, synth

    if hiprt.device_count() < 1:
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    copy_gbs = copy_rate()
    log(f"device-to-device copy: {copy_gbs} GB/s (read + write)")
    log("gemv sweep (cold, rotating >= 1 GiB)")
    sweep = gemv_sweep(SWEEP)
    roof = sweep[f"{ROOF_SHAPE[0]}x{ROOF_SHAPE[1]}"]
    log(f"sweep: {json.dumps(sweep)}")

    value = ms = None
    toks7 = None
    cpu = None
    tiny = None
    tiny_sampled = None
    gsweep = None
    prefill = None
    kq = None
    qwen = None
    fp16kv = None
    if not args.roofline_only and not args.no_kquant:
        log("Q4_K / Q6_K / Q8_0 / Q5_K gemv (cold) and 7B Q4_K_M-style 64-token decode")
        kq = {"gemv_q4_k_cold": gemv_sweep(KQ4_SHAPES, qtype=12),
              "gemv_q6_k_cold": gemv_sweep(KQ6_SHAPES, qtype=14),
              "gemv_q8_0_cold": gemv_sweep(GENERIC_SHAPES, qtype=8),
              "gemv_q5_k_cold": gemv_sweep(GENERIC_SHAPES, qtype=13)}
        cfgk = LLAMA2_7B.replace(context_length=2048)
        ckk = synth.llama_checkpoint(cfgk, seed=11, mix="q4_k_m")
        pk = synth.tokens(11, "prompt", 16, cfgk.vocab_size)
        dtk, _ = decode_run(cfgk, ckk, pk, 64, 4)
        kq["llama2_7b_q4_k_m_decode_tok_s"] = round(64 / dtk, 1)
        kq["weights_GB"] = round(synth.checkpoint_bytes(ckk) / 1e9, 3)
        del ckk
        log(f"  {json.dumps(kq)}")
    if not args.roofline_only and not args.no_gemm:
        log("gemm sweep N = 8, 64, 512 (cold)")
        gsweep = gemm_sweep(SWEEP, (8, 64, 512))
        log(f"gemm sweep: {json.dumps(gsweep)}")
    if not args.roofline_only:
        cfg7 = LLAMA2_7B.replace(context_length=2048)
        log("generating Llama-2-7B-shaped Q4_0 checkpoint")
        t0 = time.perf_counter()
        ck7 = synth.llama_checkpoint(cfg7, seed=7, mix="q4_0")
        log(f"  {synth.checkpoint_bytes(ck7) / 1e9:.2f} GB in {time.perf_counter() - t0:.1f} s")
        prompt = synth.tokens(7, "prompt", 128, cfg7.vocab_size)
        log(f"7B decode: prompt 128, warmup {args.warmup}, timed {args.steps}")
        dt, toks7 = decode_run(cfg7, ck7, prompt, args.steps, args.warmup)
        value = args.steps / dt
        ms = dt * 1000.0 / args.steps
        log(f"  {value:.1f} tok/s ({ms:.3f} ms/token)")
        dt16, _ = decode_run(cfg7.replace(kv_dtype=_native.KV_F16), ck7, prompt, args.steps, args.warmup)
        fp16kv = round(args.steps / dt16, 1)
        log(f"  fp16 KV cache: {fp16kv} tok/s")
        if not args.no_cpu:
            log("cpu baseline (oracle on host cores)")
            cpu = cpu_baseline(cfg7, ck7)
            log(f"  {cpu['value']} tok/s on {cpu['cores']} threads")
        del ck7
        if not args.no_tinyllama:
            cfg1 = TINYLLAMA_1B.replace(context_length=2048)
            ck1 = synth.llama_checkpoint(cfg1, seed=1234, mix="q4_0")
            p1 = synth.tokens(1234, "prompt", 16, cfg1.vocab_size)
            dt1, _ = decode_run(cfg1, ck1, p1, 128, 8)
            tiny = round(128 / dt1, 1)
            log(f"TinyLlama decode: {tiny} tok/s")
            tiny_sampled = sampled_run(cfg1, ck1, p1, 128)
            log(f"TinyLlama decode, temperature sampler on the device: {tiny_sampled} tok/s")
            log("TinyLlama 512-token prefill + 128 decode")
            prefill = prefill_run(cfg1, ck1, 512, 128)
            log(f"  {json.dumps(prefill)}")
            del ck1
            cfgq = QWEN2_0_5B.replace(context_length=2048)
            ckq = synth.llama_checkpoint(cfgq, seed=5, mix="q8_0", with_output=False, embedding=_native.GGML_Q8_0)
            pq = synth.tokens(5, "prompt", 16, cfgq.vocab_size)
            dtq, _ = decode_run(cfgq, ckq, pq, 128, 8)
            qwen = {"qwen2_0_5b_q8_0_decode_tok_s": round(128 / dtq, 1),
                    "weights_GB": round(synth.checkpoint_bytes(ckq) / 1e9, 3)}
            log(f"Qwen2-0.5B-shaped Q8_0 (tied embeddings, QKV biases) decode: {json.dumps(qwen)}")
            del ckq

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
        "config": {"workload": "llama2-7b-q4_0-decode-bs1", "prompt_tokens": 128, "decode_tokens": args.steps,
                   "kv_cache": "f32", "context_length": 2048, "weights": "Q4_0 (all matrices)",
                   "llama2_7b_q4_0_fp16_kv_decode_tok_s": fp16kv,
                   "tinyllama_1b_q4_0_decode_tok_s": tiny,
                   "tinyllama_1b_q4_0_sampled_decode_tok_s": tiny_sampled},
        "gemv_sweep_q4_0_n1_cold": sweep,
        "gemm_sweep_q4_0_cold": gsweep,
        "tinyllama_q4_0_prefill": prefill,
        "llama2_7b_q4_k_m": kq,
        "qwen2_0_5b_q8_0": qwen,
        "roofline": {"bound": "hbm", "achieved": roof["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": roof["frac"], "traffic": measured_traffic(ROOF_SHAPE),
                     "traffic_source": "profiles/gemv_q4_0_sweep_roofline.md (rocprofv3 --pmc FETCH_SIZE, WRITE_SIZE)",
                     "kernel": "gemv_kernel<Q4_0> (chatnet_matmul N=1) at 11008x4096, cold",
                     "alg_bytes_per_launch": roof["alg_bytes"], "avg_launch_us": roof["us"],
                     "measured_copy_GBs": copy_gbs,
                     "measured_copy_note": "512 MiB device-to-device copy, read + write bytes per second"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
