"""Benchmark of the attention hot path on one MI355X.

Default workload: decode attention for one token
over 43 layers, each layer with its own 32768-row FP8 E4M3FN KV cache (1% of
rows scaled x8), 64 query heads sharing one 512-dim latent KV head, bf16 Q,
fp32 output. One step = one decode-attention call over all 43 layers (the
split-K partial kernel + the merge kernel). Inputs are resident in HBM before
the timed region.

Prints one JSON line. `value` is the algorithmic KV-read GB/s of the whole
step (bytes per step / step time). `roofline` reports the dominant kernel
(the split partial kernel), timed alone with HIP events on the stream it
runs on. `cpu_baseline` times the oracle's scalar C++ decode attention (the
same math) on a bounded sample on this host.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

import numpy as np


def log(*a):
    print(*a, file=sys.stderr, flush=True)


N_LAYERS, N_KV, N_HEAD, HEAD_DIM = 43, 32768, 64, 512
ROW_BYTES = 584                                   # FP8 cache row: 448 codes + 8 exps + 128 tail
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFLOPS = 2500.0                          # dense f16 / bf16


def bytes_per_layer():
    # KV rows + Q (bf16) + out (fp32) + sinks
    return N_KV * ROW_BYTES + N_HEAD * HEAD_DIM * 2 + N_HEAD * HEAD_DIM * 4 + N_HEAD * 4


def cpu_baseline(seed=0):
    """Oracle (scalar C++, same math) on one layer of the workload; 1 thread
    and all host threads. Returns the threaded figure plus both timings."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests"))
    import oracle as O
    from ds4cuda_amd import synth
    n_kv = N_KV
    x = synth.kv_rows(seed, 1, n_kv, outlier_frac=0.01)
    codes, sexp, tail, _ = O.fp8_quant_rows(x)
    q = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(seed, 2, N_HEAD * HEAD_DIM)))
    q = q.reshape(N_HEAD, HEAD_DIM)
    sinks = synth.normal(seed, 3, N_HEAD)
    rows = np.arange(n_kv)
    threads = os.cpu_count() or 1
    t0 = time.perf_counter()
    O.attn_decode_fp8(q, codes, sexp, tail, rows, sinks, n_threads=1)
    t1 = time.perf_counter() - t0
    t0 = time.perf_counter()
    O.attn_decode_fp8(q, codes, sexp, tail, rows, sinks, n_threads=threads)
    tn = time.perf_counter() - t0
    b = bytes_per_layer()
    return {"value": round(b / tn / 1e9, 3), "unit": "GB/s", "cores": threads,
            "kind": "port",
            "sample": f"one layer of the workload ({n_kv} FP8 rows, 64 heads), oracle scalar C++; "
                      f"{threads} threads {tn*1e3:.1f} ms/layer, 1 thread {t1*1e3:.1f} ms/layer "
                      f"({b / t1 / 1e9:.3f} GB/s)"}


def time_ms(fn, steps, warmup, stream):
    import torch
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(steps):
        fn()
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def bench_prefill(dev, stream, steps):
    """2048 new queries over 8192 cached rows + causal
    self, 64 heads, head_dim 512, bf16 Q, FP8 KV."""
    import torch
    from ds4cuda_amd import ops
    n_cached, n_q = 8192, 2048
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    cache = ops.Fp8KVCache.empty(n_cached + n_q, device=dev)
    cache.append(torch.randn((n_cached + n_q, HEAD_DIM), generator=g, device=dev))
    q = torch.randn((n_q, N_HEAD, HEAD_DIM), generator=g, device=dev).to(torch.bfloat16)
    sinks = torch.randn((N_HEAD,), generator=g, device=dev)
    out = torch.empty((n_q, N_HEAD, HEAD_DIM), device=dev)
    ws = ops.flash_attn_prefill_fp8(q, sinks, out, cache, n_q, n_cached, stream=stream)
    ms = time_ms(lambda: ops.flash_attn_prefill_fp8(q, sinks, out, cache, n_q, n_cached,
                                                    workspace=ws, stream=stream),
                 steps, 2, stream)
    causal = 4 * N_HEAD * HEAD_DIM * sum(n_cached + i + 1 for i in range(n_q))
    full = 4 * N_HEAD * HEAD_DIM * n_q * (n_cached + n_q)
    tf = causal / (ms * 1e-3) / 1e12
    return {"workload": "chunked prefill: 2048 queries over 8192 cached + causal self, 64 heads, "
                        "head_dim 512, bf16 Q, FP8 KV (BASELINE configs[3])",
            "ms": round(ms, 4), "tflops_causal": round(tf, 1),
            "tflops_nomask_credit": round(full / (ms * 1e-3) / 1e12, 1),
            "flops_causal": causal, "peak_tflops": MFMA_PEAK_TFLOPS,
            "frac": round(tf / MFMA_PEAK_TFLOPS, 4)}


def bench_sparse(dev, stream, steps):
    """indexer over 131072 bf16 index keys (64 heads x
    128), top-2048 incl. the last 128, then decode over the 2048 gathered FP8
    rows of a 131072-row cache."""
    import torch
    from ds4cuda_amd import ops
    n, top_k, recent = 131072, 2048, 128
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    keys = torch.randn((n, 128), generator=g, device=dev).to(torch.bfloat16)
    qi = torch.randn((N_HEAD, 128), generator=g, device=dev).to(torch.bfloat16).float()
    w = torch.randn((N_HEAD,), generator=g, device=dev) / float(np.sqrt(128 * N_HEAD))
    cache = ops.Fp8KVCache.empty(n, device=dev)
    for r0 in range(0, n, 32768):
        cache.append(torch.randn((32768, HEAD_DIM), generator=g, device=dev), row0=r0)
    q = torch.randn((1, N_HEAD, HEAD_DIM), generator=g, device=dev).to(torch.bfloat16)
    sinks = torch.randn((1, N_HEAD), generator=g, device=dev)
    out = torch.empty((1, N_HEAD, HEAD_DIM), device=dev)
    from ds4cuda_amd._lib import lib
    scores = torch.empty(n, device=dev)
    select = torch.empty(lib().ds4hip_indexer_select_scratch_bytes(n), dtype=torch.uint8,
                         device=dev)
    pos = torch.empty((1, top_k), dtype=torch.int32, device=dev)
    ws = torch.empty(ops.decode_fp8_workspace_bytes([top_k]), dtype=torch.uint8, device=dev)

    def step():
        ops.indexer_topk_positions(qi, w, keys, top_k, recent, scores=scores, select=select,
                                   positions=pos[0], stream=stream)
        ops.flash_attn_decode_fp8(q, sinks, out, cache, [top_k], row_idx=pos, workspace=ws,
                                  stream=stream)

    def sel_only():
        ops.indexer_topk_positions(qi, w, keys, top_k, recent, scores=scores, select=select,
                                   positions=pos[0], stream=stream)

    ms = time_ms(step, steps, 3, stream)
    ms_idx = time_ms(sel_only, steps, 3, stream)
    b = n * 128 * 2 + N_HEAD * 128 * 4 + N_HEAD * 4 + 2 * n * 4 + top_k * (ROW_BYTES + 4) \
        + N_HEAD * HEAD_DIM * 6 + N_HEAD * 4
    return {"workload": "sparse decode: indexer over 131072 bf16 keys (64 heads x 128), top-2048 "
                        "incl. last 128, decode over the gathered FP8 rows (BASELINE configs[2])",
            "us": round(ms * 1e3, 2), "us_indexer": round(ms_idx * 1e3, 2),
            "bytes": b, "gbs": round(b / (ms * 1e-3) / 1e9, 1),
            "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the prefill / sparse-decode / batched-block figures")
    args = ap.parse_args()
    if args.gpus != 1:
        log("bench.py measures the single-GPU path only: the attention path has no "
            "cross-GPU component in this build (run with --gpus 1).")
        sys.exit(2)

    import torch
    from ds4cuda_amd import ops

    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    total_rows = N_LAYERS * N_KV
    log(f"building {N_LAYERS} x {N_KV} FP8 cache ({total_rows * ROW_BYTES / 1e6:.0f} MB)")
    cache = ops.Fp8KVCache.empty(total_rows, device=dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    for l in range(N_LAYERS):
        x = torch.randn((N_KV, HEAD_DIM), generator=g, device=dev, dtype=torch.float32)
        sel = torch.rand((N_KV,), generator=g, device=dev) < 0.01
        x[sel] *= 8.0
        cache.append(x, row0=l * N_KV)
    del x
    q = torch.randn((N_LAYERS, N_HEAD, HEAD_DIM), generator=g, device=dev).to(torch.bfloat16)
    sinks = torch.randn((N_LAYERS, N_HEAD), generator=g, device=dev)
    out = torch.zeros((N_LAYERS, N_HEAD, HEAD_DIM), device=dev)
    counts = [N_KV] * N_LAYERS
    ws = torch.empty(ops.decode_fp8_workspace_bytes(counts), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()

    def step(phases=3):
        ops.flash_attn_decode_fp8(q, sinks, out, cache, counts, row_base_stride=N_KV,
                                  workspace=ws, phases=phases, stream=stream)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K whole steps
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps

    # dominant kernel alone (split partial kernel), events on the same stream
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps)]
    for i in range(args.steps):
        starts[i].record(stream)
        step(phases=1)
        ends[i].record(stream)
        step(phases=2)
    torch.cuda.synchronize()
    k_ms = float(np.mean([s.elapsed_time(e) for s, e in zip(starts, ends)]))

    step_bytes = N_LAYERS * bytes_per_layer()
    value = step_bytes / (ms * 1e-3) / 1e9
    achieved = step_bytes / (k_ms * 1e-3) / 1e9
    res = {
        "metric": "decode attn KV-read GB/s (% of 8 TB/s)",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (torch.randn KV ~N(0,1) with 1% of rows x8, FP8 E4M3FN per-64-block "
                "pow2 scales; bf16 Q ~N(0,1); sinks ~N(0,1))",
        "config": {"workload": "decode attention, 43 layers x 32768-row FP8 KV cache, batch 1, "
                               "64 q-heads / 1 latent KV head, head_dim 512 (BASELINE configs[1])",
                   "layers": N_LAYERS, "n_kv": N_KV, "n_head": N_HEAD, "head_dim": HEAD_DIM,
                   "kv_bytes_per_row": ROW_BYTES, "us_per_layer": round(ms * 1e3 / N_LAYERS, 3),
                   "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2)},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "decode_fp8_kernel<bf16 q>",
                     "kernel_ms": round(k_ms, 4), "bytes_per_launch": step_bytes},
    }
    if not args.no_secondary:
        log("secondary configs: chunked prefill, sparse decode")
        res["secondary"] = {"prefill": bench_prefill(dev, stream, max(3, args.steps // 10)),
                            "sparse_decode": bench_sparse(dev, stream, args.steps)}
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (oracle) on one layer")
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
