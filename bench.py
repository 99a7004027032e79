#!/usr/bin/env python3
"""HipLLM benchmark: quantized decode GEMV bandwidth + end-to-end decode.

Headline (``value``): Q4_K decode-GEMV throughput in GB/s of algorithmic
bytes at Qwen2.5-7B shapes, batch 1. One step = the four weight GEMVs of one
decoder layer (fused QKV 3584->4608, gate 3584->18944, up 3584->18944, down
18944->3584), FP32 activations N(0, 1), weights N(0, 0.02) quantized to
Q4_K. Steps rotate over enough weight copies (> 2x the 256 MB Infinity Cache)
that every GEMV streams its weights from HBM. Algorithmic bytes per GEMV =
N * row_bytes + 4 K + 4 N. Inputs are resident in HBM before timing; the
timed steps replay a HIP graph of the launches.

Also reported: the same for Q6_K; per-launch kernel durations from HIP events
(the roofline entry uses the gate/up GEMV, the dominant kernel); end-to-end
greedy decode and prefill tok/s of synthetic Qwen2.5-0.5B- and 7B-shaped
Q4_K_M models through the HipLLM backend; and a bounded CPU baseline.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-e2e] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import os
import pathlib
import sys
import tempfile
import time

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "decode tok/s + Q4_K GEMV HBM GB/s (% peak); prefill tok/s; 1 GPU"
PEAK_HBM_GBPS = 8000.0
SHAPES = [("qkv", 4608, 3584), ("gate", 18944, 3584), ("up", 18944, 3584), ("down", 3584, 18944)]
MALL_BYTES = 256 << 20


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(n, k, row_bytes):
    return n * row_bytes + 4 * k + 4 * n


def bench_gemv(qtype, steps, warmup, torch, cuda):
    from myllm_amd import synth
    from myllm_amd.hipllm import kernels

    host = {}
    for name, n, k in SHAPES:
        if (n, k) not in host:
            host[(n, k)] = synth.random_quantized(n, k, qtype, seed=n * 7 + k)
    per_step = sum(host[(n, k)].nbytes for _, n, k in SHAPES)
    copies = max(4, int(np.ceil(3 * MALL_BYTES / per_step)))
    weights = []
    for c in range(copies):
        layer = {}
        for name, n, k in SHAPES:
            src = host[(n, k)]
            buf = torch.empty(src.nbytes + 256, dtype=torch.uint8, device=cuda)
            buf[: src.nbytes].copy_(torch.from_numpy(src.reshape(-1)))
            layer[name] = (buf, src.shape[1])
        weights.append(layer)
    xs = {k: torch.from_numpy(synth.normal(k, seed=k)).to(cuda) for k in (3584, 18944)}
    sums = {}
    for k, x in xs.items():
        sums[k] = torch.empty(k // 16, dtype=torch.float32, device=cuda)
        kernels.prep_sums(x, sums[k], k)
    ys = {name: torch.empty(n, dtype=torch.float32, device=cuda) for name, n, _ in SHAPES}

    def launch(c, name, n, k):
        buf, rb = weights[c][name]
        kernels.gemv_prepped(qtype, buf, rb, xs[k], sums[k], None, None, ys[name], n, k)

    def step(c):
        for name, n, k in SHAPES:
            launch(c, name, n, k)

    # Warm up eagerly, then capture `copies` steps into one graph.
    for i in range(warmup):
        step(i % copies)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for c in range(copies):
                step(c)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    replays = max(1, int(np.ceil(steps / copies)))
    t0 = time.perf_counter()
    for _ in range(replays):
        graph.replay()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timed_steps = replays * copies
    step_bytes = sum(gemv_bytes(n, k, host[(n, k)].shape[1]) for _, n, k in SHAPES)
    gbps = step_bytes * timed_steps / elapsed / 1e9

    # Per-launch kernel durations (HIP events on the launch stream).
    durations = {name: [] for name, _, _ in SHAPES}
    events = []
    for i in range(timed_steps):
        c = i % copies
        for name, n, k in SHAPES:
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            launch(c, name, n, k)
            e1.record()
            events.append((name, e0, e1))
    torch.cuda.synchronize()
    for name, e0, e1 in events:
        durations[name].append(e0.elapsed_time(e1) * 1e-3)
    kernels_out = {}
    for name, n, k in SHAPES:
        d = float(np.mean(durations[name]))
        b = gemv_bytes(n, k, host[(n, k)].shape[1])
        kernels_out[name] = {"n": n, "k": k, "bytes": b, "avg_us": d * 1e6, "gbps": b / d / 1e9}
    return {"gbps": gbps, "ms_per_step": elapsed / timed_steps * 1e3, "steps": timed_steps,
            "copies": copies, "step_bytes": step_bytes, "kernels": kernels_out}


def bench_e2e(shape_name, prompt_len, decode_steps, workdir, max_sequence=0):
    from myllm_amd import synth
    from myllm_amd.hipllm import HipLLM

    shape = synth.SHAPES[shape_name]
    t0 = time.perf_counter()
    path = synth.write_qwen2(pathlib.Path(workdir) / f"{shape_name}.gguf", shape, seed=0)
    gen_s = time.perf_counter() - t0
    prompt = synth.uniform_ids(prompt_len, shape.vocab, seed=0).tolist()
    t0 = time.perf_counter()
    model = HipLLM(path, max_sequence or prompt_len + decode_steps + 1)
    load_s = time.perf_counter() - t0
    try:
        model.reset()
        model.prefill(prompt)  # warm-up turn
        model.decode(1)
        model.reset()
        t0 = time.perf_counter()
        nxt = model.prefill(prompt)
        prefill_s = time.perf_counter() - t0
        dec = 0.0
        for _ in range(decode_steps):
            t0 = time.perf_counter()
            nxt = model.decode(nxt)
            dec += time.perf_counter() - t0
        stats = model.memory_stats()
    finally:
        model.close()
        os.unlink(path)
    return {"model": shape_name, "prompt_tokens": prompt_len, "decode_steps": decode_steps,
            "prefill_tok_s": prompt_len / prefill_s, "decode_tok_s": decode_steps / dec,
            "decode_ms_per_token": dec / decode_steps * 1e3, "weight_bytes": stats["weight_bytes"],
            "gguf_gen_s": gen_s, "load_s": load_s}


def cpu_baseline(budget_s: float = 12.0):
    """CPULLM's FP32 GEMV (gevmt, cpu_llm.cpp:512-526) over the same shapes,
    one thread, on FP32 weights dequantized from the same Q4_K bytes."""
    import oracle
    from myllm_amd import synth

    mats = {}
    for name, n, k in SHAPES:
        if (n, k) not in mats:
            q = synth.random_quantized(n, k, synth.Q4_K, seed=n * 7 + k)
            mats[(n, k)] = (oracle.dequant_rows(synth.Q4_K, q, k), q.shape[1])
    xs = {k: synth.normal(k, seed=k) for k in (3584, 18944)}
    done_bytes, t0 = 0, time.perf_counter()
    steps = 0
    while time.perf_counter() - t0 < budget_s or steps == 0:
        for name, n, k in SHAPES:
            w, rb = mats[(n, k)]
            oracle.gevmt(w, xs[k])
            done_bytes += gemv_bytes(n, k, rb)
        steps += 1
    el = time.perf_counter() - t0
    out = {"value": done_bytes / el / 1e9, "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"{steps} step(s) of the same four GEMVs (QKV, gate, up, down at Qwen2.5-7B shapes) "
                     f"with the oracle's CPULLM gevmt on FP32-dequantized Q4_K weights, 1 thread of "
                     f"{os.cpu_count()} host cores, {el:.1f} s"}
    if oracle.REF_BIN.exists():
        # The reference's own CPULLM on the 0.5B-shaped model: 4-token prompt,
        # 8 greedy tokens (7 decode steps).
        with tempfile.TemporaryDirectory(dir="/dev/shm" if os.path.isdir("/dev/shm") else None) as tmp:
            path = synth.write_qwen2(pathlib.Path(tmp) / "c0.gguf", synth.SHAPES["qwen2.5-0.5b"], seed=0)
            prompt = synth.uniform_ids(4, synth.SHAPES["qwen2.5-0.5b"].vocab, seed=0)
            r = oracle.run_reference(path, prompt, 8, max_sequence=64, timeout=600)
        out["reference_cpullm_qwen05b"] = {
            "decode_tok_s": r["decode_steps"] / (r["decode_ms"] / 1e3),
            "prefill_tok_s": r["prompt_tokens"] / (r["prefill_ms"] / 1e3),
            "sample": "reference CPULLM (oracle/_ref) on the Qwen2.5-0.5B-shaped Q4_K_M model, "
                      "4-token prompt, 7 decode steps, 1 thread"}
    return out


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=96)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-7b", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU; the multi-GPU layout is "
                                   "described in DESIGN.md and not built", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    cuda = torch.device("cuda:0")
    from myllm_amd import synth

    log("[bench] Q4_K GEMV")
    q4 = bench_gemv(synth.Q4_K, args.steps, args.warmup, torch, cuda)
    log(f"[bench] Q4_K {q4['gbps']:.1f} GB/s; kernels " +
        ", ".join(f"{k}={v['gbps']:.0f}GB/s/{v['avg_us']:.1f}us" for k, v in q4["kernels"].items()))
    log("[bench] Q6_K GEMV")
    q6 = bench_gemv(synth.Q6_K, args.steps, args.warmup, torch, cuda)
    log(f"[bench] Q6_K {q6['gbps']:.1f} GB/s")

    e2e = {}
    if not args.no_e2e:
        with tempfile.TemporaryDirectory(dir="/dev/shm" if os.path.isdir("/dev/shm") else None) as tmp:
            log("[bench] e2e qwen2.5-0.5b")
            e2e["qwen2.5-0.5b"] = bench_e2e("qwen2.5-0.5b", 16, 32, tmp)
            log(f"[bench] {e2e['qwen2.5-0.5b']}")
            if not args.no_7b:
                log("[bench] e2e qwen2.5-7b")
                e2e["qwen2.5-7b"] = bench_e2e("qwen2.5-7b", 16, 32, tmp)
                log(f"[bench] {e2e['qwen2.5-7b']}")

    cpu = None
    if not args.no_cpu:
        log("[bench] CPU baseline")
        cpu = cpu_baseline()
        log(f"[bench] CPU {cpu}")

    dom = q4["kernels"]["gate"]
    out = {
        "metric": METRIC,
        "value": round(q4["gbps"], 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": q4["steps"],
        "warmup": args.warmup,
        "ms_per_step": round(q4["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {"workload": "Q4_K decode GEMV at Qwen2.5-7B shapes, batch 1: one step = fused QKV "
                               "3584->4608 + gate 3584->18944 + up 3584->18944 + down 18944->3584",
                   "weights": "Q4_K (GGML layout, N(0,0.02))", "activations": "f32 N(0,1)",
                   "weight_copies_rotated": q4["copies"], "step_bytes": q4["step_bytes"]},
        "roofline": {"bound": "hbm", "achieved": round(dom["gbps"], 2), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(dom["gbps"] / PEAK_HBM_GBPS, 4), "traffic": None,
                     "kernel": "gemv_kernel<Q4_K> 3584->18944", "bytes_per_launch": dom["bytes"],
                     "avg_launch_us": round(dom["avg_us"], 3)},
        "gemv": {"q4_k": {"step_gbps": round(q4["gbps"], 2),
                          "kernels": {k: {"gbps": round(v["gbps"], 1), "avg_us": round(v["avg_us"], 2)}
                                      for k, v in q4["kernels"].items()}},
                 "q6_k": {"step_gbps": round(q6["gbps"], 2),
                          "kernels": {k: {"gbps": round(v["gbps"], 1), "avg_us": round(v["avg_us"], 2)}
                                      for k, v in q6["kernels"].items()}}},
        "e2e": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                for k, v in e2e.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
