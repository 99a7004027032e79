#!/usr/bin/env python3
"""HipLLM benchmark: quantized decode GEMV bandwidth, prefill matmul, end-to-end.

Headline (``value``): Q4_K decode-GEMV throughput in GB/s of algorithmic bytes
at Qwen2.5-7B shapes, batch 1. One step = the four weight GEMVs of one decoder
layer (fused QKV 3584->4608, gate 3584->18944, up 3584->18944, down
18944->3584) with FP32 activations N(0, 1) and N(0, 0.02) weights quantized to
Q4_K, held in the x16 tile-packed form the int8-MFMA GEMV reads (the same
bytes as the GGUF rows, regrouped into 16-row tiles; the vector GEMV on the
GGUF rows is timed beside it). Steps rotate over at least 16 weight copies
(and 3x the 256 MB Infinity Cache) so that every GEMV, also when timed alone,
streams its weights from HBM; inputs are resident in HBM before timing and
the timed steps replay a HIP graph of the launches. Algorithmic bytes per
GEMV = N * row_bytes + 4 K + 4 N.

The same JSON line carries:
* ``roofline``: the dominant kernel (the 3584->18944 gate GEMV) timed alone
  with HIP events on its launch stream, against MI355X's 8 TB/s; ``traffic``
  is read from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary when
  present (see --profile-kernel);
* ``gemv``: per-shape results for Q4_K and Q6_K;
* ``prefill_gemm``: the fp16-MFMA prefill matmul, M in {64, 512, 2048} x
  K 3584 x N 18944, Q4_K weights, TFLOP/s against the 2.5 PFLOP/s dense
  fp16/bf16 MFMA peak;
* ``e2e``: greedy prefill and decode tok/s of synthetic Qwen2.5-0.5B-, 7B- and
  14B-shaped Q4_K_M models and a Qwen3.5-35B-A3B-shaped qwen35moe model (all
  256 experts resident) through the HipLLM handle API;
* ``cpu_baseline``: a bounded sample of the same GEMV step on the host (the
  oracle's restatement of CPULLM's gevmt, one thread), plus the restated
  CPULLM's decode rate on the same 7B-shaped model (a bounded sample) and the
  GPU/CPU decode ratio.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-e2e] [--no-cpu]
                       [--no-14b] [--no-moe] [--profile-kernel gate|prefill64|prefill512|prefill2048]
                       [--profile-reps N]
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
PEAK_F16_TFLOPS = 2500.0
SHAPES = [("qkv", 4608, 3584), ("gate", 18944, 3584), ("up", 18944, 3584), ("down", 3584, 18944)]
MALL_BYTES = 256 << 20
TRAFFIC_SUMMARY = ROOT / "profiles" / "gemv_q4k_gate_3584x18944_traffic.txt"


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(n, k, row_bytes):
    return n * row_bytes + 4 * k + 4 * n


def scratch_dir():
    return "/dev/shm" if os.path.isdir("/dev/shm") else None


class Rotation:
    """Device copies of one layer's four weight matrices, rotated per step:
    at least 16 copies and 3x the 256 MB Infinity Cache, so that a matrix
    timed alone is also read from HBM every time (its 15 other copies, over
    570 MB for the gate, pass through the cache between two reads of it).
    packed: also hold each Q4_K / Q6_K copy in the x16 tile-packed form that
    the MFMA GEMV reads (same byte count)."""

    def __init__(self, qtype, torch, cuda, min_bytes=3 * MALL_BYTES, packed=False):
        from myllm_amd import synth
        from myllm_amd.hipllm import kernels
        self.host = {}
        for _, n, k in SHAPES:
            if (n, k) not in self.host:
                self.host[(n, k)] = synth.random_quantized(n, k, qtype, seed=n * 7 + k)
        per_step = sum(self.host[(n, k)].nbytes for _, n, k in SHAPES)
        self.copies = max(16, int(np.ceil(min_bytes / per_step)))
        self.layers, self.packed = [], []
        for _ in range(self.copies):
            layer, player = {}, {}
            for name, n, k in SHAPES:
                src = self.host[(n, k)]
                buf = torch.empty(src.nbytes + 256, dtype=torch.uint8, device=cuda)
                buf[: src.nbytes].copy_(torch.from_numpy(src.reshape(-1)))
                layer[name] = buf
                if packed:
                    pk = torch.empty(kernels.x16_bytes(qtype, n, k), dtype=torch.uint8, device=cuda)
                    kernels.pack_x16(qtype, buf, src.shape[1], n, k, pk)
                    player[name] = pk
            self.layers.append(layer)
            self.packed.append(player)
        self.step_bytes = sum(gemv_bytes(n, k, self.host[(n, k)].shape[1]) for _, n, k in SHAPES)

    def row_bytes(self, n, k):
        return self.host[(n, k)].shape[1]


def gemv_setup(qtype, torch, cuda, packed=False):
    """packed (Q4_K / Q6_K): launch the MFMA GEMV on the x16-packed copies
    instead of the vector GEMV on the GGUF rows."""
    from myllm_amd import synth
    from myllm_amd.hipllm import kernels
    rot = Rotation(qtype, torch, cuda, packed=packed)
    xs = {k: torch.from_numpy(synth.normal(k, seed=k)).to(cuda) for k in (3584, 18944)}
    xq = {}  # XGroup form of each input (k / 16 groups of 64 bytes)
    for k, x in xs.items():
        xq[k] = torch.empty(k, dtype=torch.float32, device=cuda)
        kernels.prep_x(x, xq[k], k)
    ys = {name: torch.empty(n, dtype=torch.float32, device=cuda) for name, n, _ in SHAPES}

    def launch(c, name, n, k, stream=None):
        if packed:
            kernels.gemv_x16(qtype, rot.packed[c][name], xq[k], None, None, ys[name], n, k, 0, stream=stream)
        else:
            kernels.gemv_prepped(qtype, rot.layers[c][name], rot.row_bytes(n, k), xs[k], xq[k], None, None,
                                 ys[name], n, k, 0, stream=stream)

    return rot, launch


def time_kernel(torch, fn, count, replays=5):
    """Average launch duration of fn(i, stream) over `count` launches recorded
    in one HIP graph and replayed `replays` times, timed with HIP events on the
    stream the replays run on (torch's current stream), so host launch cost
    is excluded and back-to-back launches are measured as the decode step runs
    them."""
    side = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        fn(0, side)
        torch.cuda.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for i in range(count):
                fn(i, side)
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(replays):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    del graph
    return e0.elapsed_time(e1) * 1e-3 / (count * replays)


def bench_gemv(qtype, steps, warmup, torch, cuda, packed=False):
    rot, launch = gemv_setup(qtype, torch, cuda, packed=packed)
    copies = rot.copies

    def step(c, stream=None):
        for name, n, k in SHAPES:
            launch(c, name, n, k, stream)

    for i in range(warmup):
        step(i % copies)
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph, stream=stream):
            for c in range(copies):
                step(c, stream)
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
    gbps = rot.step_bytes * timed_steps / elapsed / 1e9

    kernels_out = {}
    for name, n, k in SHAPES:
        reps = copies * 8
        d = time_kernel(torch, lambda i, st: launch(i % copies, name, n, k, st), reps)
        b = gemv_bytes(n, k, rot.row_bytes(n, k))
        kernels_out[name] = {"n": n, "k": k, "bytes": b, "avg_us": d * 1e6, "gbps": b / d / 1e9, "launches": reps}
    del graph, rot
    torch.cuda.empty_cache()
    return {"gbps": gbps, "ms_per_step": elapsed / timed_steps * 1e3, "steps": timed_steps,
            "copies": copies, "kernels": kernels_out}


def bench_copy(torch, cuda, nbytes):
    """A plain device copy of nbytes (read + write), rotated past the MALL:
    the reference point for the HBM counters and for what a trivial
    streaming kernel reaches at this size."""
    n = nbytes // 4
    bufs = [torch.empty(n, dtype=torch.float32, device=cuda) for _ in range(12)]
    dst = torch.empty(n, dtype=torch.float32, device=cuda)
    for b in bufs:
        b.fill_(1.0)
    d = time_kernel(torch, lambda i, st: dst.copy_(bufs[i % 12]), 96)
    return {"bytes_read": n * 4, "bytes_written": n * 4, "avg_us": d * 1e6, "gbps_read_plus_write": 2 * n * 4 / d / 1e9}


def bench_prefill_gemm(torch, cuda):
    from myllm_amd import synth
    from myllm_amd.hipllm import kernels, lib
    K, N = 3584, 18944
    src = synth.random_quantized(N, K, synth.Q4_K, seed=N * 7 + K)
    copies = 8
    ws = []
    for _ in range(copies):
        w = torch.empty(src.nbytes + 256, dtype=torch.uint8, device=cuda)
        w[: src.nbytes].copy_(torch.from_numpy(src.reshape(-1)))
        ws.append(w)
    out = {}
    for M in (64, 512, 2048):
        x = torch.randn(M, K, device=cuda)
        xh = torch.empty(M, K, device=cuda, dtype=torch.float16)
        xs = torch.empty(M, device=cuda)
        kernels.to_f16(x, K, xh, xs, M, K)
        y = torch.empty(M, N, device=cuda)
        split_ws = torch.empty(max(16, lib().hipllm_gemm_mfma_workspace_bytes(M, N, K, -1, 0)), dtype=torch.uint8,
                               device=cuda)
        fn = lambda i, st=None: kernels.gemm_mfma(synth.Q4_K, ws[i % copies], src.shape[1], xh, xs, None, None, y, M, N,
                                                  K, stream=st, workspace=split_ws)
        for i in range(3):
            fn(i)
        d = time_kernel(torch, fn, 24)
        flops = 2.0 * M * N * K
        tf = flops / d / 1e12
        wbytes = N * src.shape[1] + M * K * 2 + M * N * 4
        out[str(M)] = {"avg_us": round(d * 1e6, 2), "tflops": round(tf, 1), "frac_f16_peak": round(tf / PEAK_F16_TFLOPS, 4),
                       "gbps": round(wbytes / d / 1e9, 1)}
    del ws
    torch.cuda.empty_cache()
    # Context, not a comparison of like with like: the same product through
    # torch.matmul (hipBLASLt) on plain bf16 weights (3.5x the bytes of Q4_K,
    # no dequant), 4 rotated copies.
    wb = [torch.randn(K, N, device=cuda).to(torch.bfloat16) for _ in range(4)]  # [K, N], no transposed view
    for M in (64, 512, 2048):
        xb = torch.randn(M, K, device=cuda).to(torch.bfloat16)
        y = torch.empty(M, N, device=cuda, dtype=torch.bfloat16)
        fn = lambda i, st=None: torch.matmul(xb, wb[i % 4], out=y)
        d = time_kernel(torch, fn, 16)
        tf = 2.0 * M * N * K / d / 1e12
        out[str(M)]["hipblaslt_bf16_weights"] = {"avg_us": round(d * 1e6, 2), "tflops": round(tf, 1)}
    del wb
    torch.cuda.empty_cache()
    return out


def bench_e2e(shape_name, prompt_len, decode_steps, workdir, max_sequence=0, keep_file=False):
    """Greedy prefill + decode through the handle API; keep_file leaves the
    synthetic GGUF in workdir (its path is in the result) for the CPU leg."""
    from myllm_amd import synth
    from myllm_amd.hipllm import HipLLM

    shape = synth.SHAPES[shape_name]
    t0 = time.perf_counter()
    path = synth.write_qwen2(pathlib.Path(workdir) / f"{shape_name}.gguf", shape, seed=0)
    gen_s = time.perf_counter() - t0
    prompt = synth.uniform_ids(prompt_len, shape.vocab, seed=0).tolist()
    try:
        t0 = time.perf_counter()
        model = HipLLM(path, max_sequence or prompt_len + decode_steps + 1)
        load_s = time.perf_counter() - t0
        try:
            model.reset()  # warm-up turn (first-launch costs)
            nxt = model.prefill(prompt)
            for _ in range(2):
                nxt = model.decode(nxt)
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
            cfg = model.config
        finally:
            model.close()
    finally:
        if not keep_file:
            os.unlink(path)
    return {"model": shape_name, "path": str(path) if keep_file else None, "prompt_tokens": prompt_len, "decode_steps": decode_steps,
            "max_sequence": max_sequence or prompt_len + decode_steps + 1,
            "prefill_tok_s": prompt_len / prefill_s, "decode_tok_s": decode_steps / dec,
            "decode_ms_per_token": dec / decode_steps * 1e3,
            "weight_bytes": stats["weight_bytes"], "kv_cache_bytes": stats["kv_cache_bytes"],
            "layers": cfg["layer_count"], "gguf_gen_s": gen_s, "load_s": load_s}


def bench_e2e_moe(shape_name, prompt_len, decode_steps, workdir):
    """qwen35moe greedy prefill + decode through the HipLLM handle API (the
    backend is picked from the file's architecture, as the CLI's --gpu does)."""
    from myllm_amd import synth
    from myllm_amd.hipllm import HipLLM

    shape = synth.MOE_SHAPES[shape_name]
    t0 = time.perf_counter()
    path = synth.write_qwen35moe(pathlib.Path(workdir) / f"{shape_name}.gguf", shape, seed=0)
    gen_s = time.perf_counter() - t0
    prompt = synth.uniform_ids(prompt_len, shape.vocab, seed=0).tolist()
    cap = prompt_len + decode_steps + 1
    try:
        t0 = time.perf_counter()
        model = HipLLM(path, cap)
        load_s = time.perf_counter() - t0
        try:
            model.reset()
            nxt = model.prefill(prompt)
            for _ in range(2):
                nxt = model.decode(nxt)
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
        # A longer prompt on the same weights: from about four routed vectors
        # per expert the expert products run as gathered matmuls.
        long_len = 512
        long_prompt = synth.uniform_ids(long_len, shape.vocab, seed=1).tolist()
        model = HipLLM(path, long_len + 1)
        try:
            model.prefill(long_prompt)
            model.reset()
            t0 = time.perf_counter()
            model.prefill(long_prompt)
            long_s = time.perf_counter() - t0
        finally:
            model.close()
    finally:
        os.unlink(path)
    return {"model": shape_name, "prompt_tokens": prompt_len, "decode_steps": decode_steps, "max_sequence": cap,
            "prefill_tok_s": prompt_len / prefill_s, "decode_tok_s": decode_steps / dec,
            "decode_ms_per_token": dec / decode_steps * 1e3, "weight_bytes": stats["weight_bytes"],
            "recurrent_state_bytes": stats["recurrent_state_bytes"], "kv_cache_bytes": stats["kv_cache_bytes"],
            "layers": shape.layers, "experts_resident": shape.experts, "gguf_gen_s": gen_s, "load_s": load_s,
            "prefill_512": {"prompt_tokens": long_len, "prefill_tok_s": long_len / long_s}}


def cpu_model_name() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return ""


def cpu_baseline(budget_s: float = 12.0, qwen7b_path=None):
    """The CPU baseline, timed on this host with one thread, as CPULLM runs
    (it has no threads), from the oracle: the repository's own C++
    restatement of CPULLM (cpu_llm.cpp, model.cpp), built like the reference
    (C++17, -O2, no -march, no FP contraction).

    * value: CPULLM's FP32 GEMV (gevmt, cpu_llm.cpp:512-526) over the same
      four Q4_K GEMV shapes as the headline, on FP32 weights dequantized
      from the same Q4_K bytes, a budget_s sample, in GB/s of the same
      algorithmic bytes.
    * qwen2.5-7b: the restated CPULLM end to end on the same
      Qwen2.5-7B-shaped Q4_K_M file the GPU decodes (a bounded sample: a
      4-token prompt and 3 greedy decode steps, generate()'s timing,
      chat.cpp:851-871)."""
    import oracle
    from myllm_amd import synth

    mats = {}
    for _, n, k in SHAPES:
        if (n, k) not in mats:
            q = synth.random_quantized(n, k, synth.Q4_K, seed=n * 7 + k)
            mats[(n, k)] = (oracle.dequant_rows(synth.Q4_K, q, k), q.shape[1])
    xs = {k: synth.normal(k, seed=k) for k in (3584, 18944)}
    done_bytes, steps = 0, 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s or steps == 0:
        for _, n, k in SHAPES:
            w, rb = mats[(n, k)]
            oracle.gevmt(w, xs[k])
            done_bytes += gemv_bytes(n, k, rb)
        steps += 1
    el = time.perf_counter() - t0
    del mats
    cpu_model = cpu_model_name()
    out = {"value": round(done_bytes / el / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
           "sample": f"{steps} step(s) of the same four GEMVs (QKV, gate, up, down at Qwen2.5-7B shapes), "
                     f"the oracle's restatement of CPULLM gevmt on FP32 weights dequantized from the same Q4_K "
                     f"bytes, 1 thread of {os.cpu_count()} host cores ({cpu_model}), {el:.1f} s",
           "host_cores": os.cpu_count(), "cpu_model": cpu_model}
    if qwen7b_path:
        shape = synth.SHAPES["qwen2.5-7b"]
        prompt = synth.uniform_ids(4, shape.vocab, seed=0).tolist()
        t0 = time.perf_counter()
        cpu = oracle.CpuOracle(qwen7b_path, 16)
        load_s = time.perf_counter() - t0
        try:
            cpu.reset()
            t0 = time.perf_counter()
            nxt = cpu.prefill(prompt)
            prefill_s = time.perf_counter() - t0
            dec, steps = 0.0, 3
            for _ in range(steps):
                t0 = time.perf_counter()
                nxt = cpu.decode(nxt)
                dec += time.perf_counter() - t0
        finally:
            cpu.close()
        out["qwen2.5-7b"] = {
            "decode_tok_s": round(steps / dec, 4), "prefill_tok_s": round(len(prompt) / prefill_s, 4),
            "load_s": round(load_s, 1), "cores": 1,
            "sample": f"the oracle's restated CPULLM on the Qwen2.5-7B-shaped Q4_K_M model the GPU decodes: "
                      f"{len(prompt)}-token prompt, {steps} greedy decode steps, 1 thread of {os.cpu_count()} "
                      f"host cores ({cpu_model})"}
    return out


def read_traffic():
    """Per-launch HBM bytes of the gate GEMV from the committed rocprofv3
    summary (FETCH_SIZE + WRITE_SIZE, copy-kernel calibrated), or None."""
    if not TRAFFIC_SUMMARY.exists():
        return None
    for line in TRAFFIC_SUMMARY.read_text().splitlines():
        if line.startswith("hbm_bytes_per_launch:"):
            return float(line.split(":", 1)[1])
    return None


def profile_kernel(name, reps, torch, cuda):
    """Runs one GEMV shape `reps` times plus a plain copy of the same byte
    count, for rocprofv3 counter collection (--pmc FETCH_SIZE / WRITE_SIZE)."""
    from myllm_amd import synth
    rot, launch = gemv_setup(synth.Q4_K, torch, cuda, packed=True)
    _, n, k = next(s for s in SHAPES if s[0] == name)
    for i in range(reps):
        launch(i % rot.copies, name, n, k)
    torch.cuda.synchronize()
    copy = bench_copy(torch, cuda, gemv_bytes(n, k, rot.row_bytes(n, k)) // 256 * 256)
    print(json.dumps({"profiled": name, "launches": reps, "bytes_per_launch": gemv_bytes(n, k, rot.row_bytes(n, k)),
                      "copy": copy}), flush=True)


def profile_prefill(m, reps, torch, cuda):
    """Runs the Q4_K prefill matmul (K = 3584, N = 18944, m rows, fp16
    operands, the default tile and K split) `reps` times over 8 rotated
    weight copies plus a plain copy of the weight bytes, for rocprofv3
    counter collection."""
    from myllm_amd import synth
    from myllm_amd.hipllm import kernels, lib
    K, N = 3584, 18944
    src = synth.random_quantized(N, K, synth.Q4_K, seed=N * 7 + K)
    ws = []
    for _ in range(8):
        w = torch.empty(src.nbytes + 256, dtype=torch.uint8, device=cuda)
        w[: src.nbytes].copy_(torch.from_numpy(src.reshape(-1)))
        ws.append(w)
    x = torch.randn(m, K, device=cuda)
    xh = torch.empty(m, K, device=cuda, dtype=torch.float16)
    xs = torch.empty(m, device=cuda)
    kernels.to_f16(x, K, xh, xs, m, K)
    y = torch.empty(m, N, device=cuda)
    split_ws = torch.empty(max(16, lib().hipllm_gemm_mfma_workspace_bytes(m, N, K, -1, 0)), dtype=torch.uint8,
                           device=cuda)
    for i in range(reps):
        kernels.gemm_mfma(synth.Q4_K, ws[i % 8], src.shape[1], xh, xs, None, None, y, m, N, K, workspace=split_ws)
    torch.cuda.synchronize()
    copy = bench_copy(torch, cuda, src.nbytes // 256 * 256)
    print(json.dumps({"profiled": f"prefill matmul M={m}", "launches": reps, "weight_bytes": int(src.nbytes),
                      "flops": 2 * m * N * K, "copy": copy}), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=96)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-14b", action="store_true")
    ap.add_argument("--no-moe", action="store_true")
    ap.add_argument("--profile-kernel", choices=[s[0] for s in SHAPES] + ["prefill64", "prefill512", "prefill2048"])
    ap.add_argument("--e2e-only", choices=["qwen2.5-0.5b", "qwen2.5-7b", "qwen2.5-14b", "qwen3.5-35b-a3b"],
                    help="run one end-to-end model only (for profiling) and print its result")
    ap.add_argument("--profile-reps", type=int, default=200)
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "this benchmark runs on exactly one GPU: the backend is single-GPU and its "
                                   "multi-GPU layout is a design, not built", "n_gpus": args.gpus}))
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        raise SystemExit("bench.py needs a GPU")
    cuda = torch.device("cuda:0")
    from myllm_amd import synth

    if args.profile_kernel and args.profile_kernel.startswith("prefill"):
        profile_prefill(int(args.profile_kernel[len("prefill"):]), min(args.profile_reps, 50), torch, cuda)
        return
    if args.profile_kernel:
        profile_kernel(args.profile_kernel, args.profile_reps, torch, cuda)
        return
    if args.e2e_only:
        with tempfile.TemporaryDirectory(dir=scratch_dir()) as tmp:
            if args.e2e_only == "qwen3.5-35b-a3b":
                r = bench_e2e_moe(args.e2e_only, 64, 64, tmp)
            else:
                p, d, cap = {"qwen2.5-0.5b": (16, 32, 0), "qwen2.5-7b": (128, 64, 0),
                             "qwen2.5-14b": (128, 128, 4096)}[args.e2e_only]
                r = bench_e2e(args.e2e_only, p, d, tmp, cap)
        print(json.dumps(r), flush=True)
        return

    log("[bench] Q4_K GEMV (x16-packed weights, int8 MFMA)")
    q4 = bench_gemv(synth.Q4_K, args.steps, args.warmup, torch, cuda, packed=True)
    log(f"[bench] Q4_K {q4['gbps']:.1f} GB/s; kernels " +
        ", ".join(f"{k}={v['gbps']:.0f}GB/s/{v['avg_us']:.1f}us" for k, v in q4["kernels"].items()))
    log("[bench] Q4_K GEMV (GGUF rows, vector ALU)")
    q4n = bench_gemv(synth.Q4_K, args.steps, args.warmup, torch, cuda)
    log(f"[bench] Q4_K GGUF rows {q4n['gbps']:.1f} GB/s")
    log("[bench] Q6_K GEMV (x16-packed weights, int8 MFMA)")
    q6 = bench_gemv(synth.Q6_K, args.steps, args.warmup, torch, cuda, packed=True)
    log(f"[bench] Q6_K x16 {q6['gbps']:.1f} GB/s")
    log("[bench] Q6_K GEMV (GGUF rows, vector ALU)")
    q6n = bench_gemv(synth.Q6_K, args.steps, args.warmup, torch, cuda)
    log(f"[bench] Q6_K GGUF rows {q6n['gbps']:.1f} GB/s")
    copy = bench_copy(torch, cuda, q4["kernels"]["gate"]["bytes"] // 256 * 256)
    log(f"[bench] plain copy of the gate GEMV's bytes: {copy['avg_us']:.2f} us")
    log("[bench] prefill GEMM")
    gemm = bench_prefill_gemm(torch, cuda)
    log(f"[bench] prefill GEMM {gemm}")

    e2e = {}
    cpu = None
    with tempfile.TemporaryDirectory(dir=scratch_dir()) as tmp:
        if not args.no_e2e:
            runs = [("qwen2.5-0.5b", 16, 32, 0), ("qwen2.5-7b", 128, 64, 0)]
            if not args.no_14b:
                runs.append(("qwen2.5-14b", 128, 128, 4096))
            for name, p, d, cap in runs:
                log(f"[bench] e2e {name}")
                e2e[name] = bench_e2e(name, p, d, tmp, cap, keep_file=(name == "qwen2.5-7b" and not args.no_cpu))
                log(f"[bench] {e2e[name]}")
            if not args.no_moe:
                log("[bench] e2e qwen3.5-35b-a3b (all 256 experts resident)")
                e2e["qwen3.5-35b-a3b"] = bench_e2e_moe("qwen3.5-35b-a3b", 64, 64, tmp)
                log(f"[bench] {e2e['qwen3.5-35b-a3b']}")
        if not args.no_cpu:
            log("[bench] CPU baseline")
            q7 = e2e.get("qwen2.5-7b", {}).pop("path", None)
            cpu = cpu_baseline(qwen7b_path=q7)
            if q7 and "qwen2.5-7b" in cpu:
                cpu["qwen2.5-7b"]["gpu_over_cpu_decode"] = round(
                    e2e["qwen2.5-7b"]["decode_tok_s"] / cpu["qwen2.5-7b"]["decode_tok_s"], 1)
            log(f"[bench] CPU {cpu}")
    for v in e2e.values():
        v.pop("path", None)

    dom = q4["kernels"]["gate"]
    traffic = read_traffic()
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
                   "weights": "Q4_K (N(0,0.02) quantized), held in the x16 tile-packed form (same bytes as the "
                              "GGML rows)", "activations": "f32 N(0,1)",
                   "weight_copies_rotated": q4["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(dom["gbps"], 2), "peak": PEAK_HBM_GBPS, "unit": "GB/s",
                     "frac": round(dom["gbps"] / PEAK_HBM_GBPS, 4), "traffic": traffic,
                     "kernel": "gemv Q4_K x16 MFMA 3584->18944 (gate)", "bytes_per_launch": dom["bytes"],
                     "avg_launch_us": round(dom["avg_us"], 3), "launches_timed": dom["launches"],
                     "plain_copy_same_bytes_us": round(copy["avg_us"], 3)},
        "gemv": {"q4_k": {"step_gbps": round(q4["gbps"], 2), "weights": "x16 tile-packed, int8 MFMA",
                          "kernels": {k: {"gbps": round(v["gbps"], 1), "avg_us": round(v["avg_us"], 2)}
                                      for k, v in q4["kernels"].items()}},
                 "q4_k_gguf_rows": {"step_gbps": round(q4n["gbps"], 2), "weights": "GGUF rows, vector ALU",
                                    "kernels": {k: {"gbps": round(v["gbps"], 1), "avg_us": round(v["avg_us"], 2)}
                                                for k, v in q4n["kernels"].items()}},
                 "q6_k": {"step_gbps": round(q6["gbps"], 2), "weights": "x16 tile-packed, int8 MFMA",
                          "kernels": {k: {"gbps": round(v["gbps"], 1), "avg_us": round(v["avg_us"], 2)}
                                      for k, v in q6["kernels"].items()}},
                 "q6_k_gguf_rows": {"step_gbps": round(q6n["gbps"], 2), "weights": "GGUF rows, vector ALU",
                                    "kernels": {k: {"gbps": round(v["gbps"], 1), "avg_us": round(v["avg_us"], 2)}
                                                for k, v in q6n["kernels"].items()}}},
        "prefill_gemm": {"weights": "Q4_K", "k": 3584, "n": 18944, "by_m": gemm},
        "e2e": {k: {kk: (round(vv, 3) if isinstance(vv, float) else vv) for kk, vv in v.items()}
                for k, v in e2e.items()},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
