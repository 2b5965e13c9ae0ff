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
COPY_BYTES = 1 << 30                               # --copy-calibration: 1 GiB read + 1 GiB written
# HBM bytes per launch of the cfg-2 partial kernel, measured with rocprofv3
# (FETCH_SIZE + WRITE_SIZE, each scaled by what the counter reads for
# `--copy-calibration`); the counter summaries and their commands are in
# profiles/decode_flat_kernel_cfg2_traffic.md (flat kernel) and
# profiles/decode_ws_kernel_cfg2_traffic.md (register-load kernel).
# Re-measure after a kernel change.
TRAFFIC_BYTES_PER_LAUNCH = {"ws": 882340981, "flat": 882271833}
TRAFFIC_MEASURED_AT = {"ws": "22db79c", "flat": "36157d5"}   # commit whose partial kernel was counted
DECODE_KERNEL = "flat"
KERNEL_LABEL = {"ws": "decode_ws_kernel<0, false> (direct rows, register loads, one f16 P)",
                "flat": "decode_flat_kernel<false, true, 0, 0> (direct rows, DMA-fed flat LDS stages, one f16 P)"}


def bytes_per_layer():
    # KV rows + Q (bf16) + out (fp32) + sinks
    return N_KV * ROW_BYTES + N_HEAD * HEAD_DIM * 2 + N_HEAD * HEAD_DIM * 4 + N_HEAD * 4


def cpu_baseline():
    """Oracle (scalar C++, same math) on one layer of the workload; 1 thread
    and all host threads. Returns the threaded figure plus both timings."""
    sys.path.insert(0, os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests"))
    import oracle as O
    from ds4cuda_amd import synth
    n_kv = N_KV
    # layer 0 of the GPU workload (the same seeded streams, see decode_inputs)
    x = synth.kv_rows(1, 0, n_kv, outlier_frac=0.01)
    codes, sexp, tail, _ = O.fp8_quant_rows(x)
    q = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(2, 0, N_HEAD * HEAD_DIM)))
    q = q.reshape(N_HEAD, HEAD_DIM)
    sinks = synth.normal(3, 0, N_HEAD)
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
                      f"({b / t1 / 1e9:.3f} GB/s)",
            "other_configs": cpu_other_configs(threads)}


def cpu_other_configs(threads):
    """The oracle on the other configs, bounded samples: cfg 1 in full, cfg 3
    (indexer over 131072 keys, single thread, + decode of 2048 rows), cfg 4
    (4 of the 2048 prefill queries, scaled to the chunk)."""
    import ctypes as C
    tests = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tests")
    if tests not in sys.path:
        sys.path.insert(0, tests)
    import oracle as O
    from ds4cuda_amd import synth
    res = {}
    # cfg 1: 4096-row decode, one layer
    x = synth.kv_rows(10, 1, 4096)
    codes, sexp, tail, _ = O.fp8_quant_rows(x)
    q = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(10, 2, N_HEAD * HEAD_DIM)))
    q = q.reshape(N_HEAD, HEAD_DIM)
    sinks = synth.normal(10, 3, N_HEAD)
    t0 = time.perf_counter()
    O.attn_decode_fp8(q, codes, sexp, tail, np.arange(4096), sinks, n_threads=1)
    res["cfg1_decode_4096_ms_1thread"] = round((time.perf_counter() - t0) * 1e3, 2)
    # cfg 3: indexer scores + top-k (one thread), decode over the 2048 rows
    n = 131072
    keys = synth.to_bf16_bits(synth.normal(11, 1, n * 128))
    qi = synth.bf16_bits_to_f32(synth.to_bf16_bits(synth.normal(11, 2, N_HEAD * 128)))
    w = synth.normal(11, 3, N_HEAD).astype(np.float32)
    scores = np.empty(n, np.float32)
    pos = np.empty(2048, np.int32)
    t0 = time.perf_counter()
    O.lib().orc_indexer_scores(O.P(qi), O.P(w), O.P(keys), C.c_int(2), C.c_int(n), C.c_int(N_HEAD),
                               C.c_int(128), O.P(scores))
    O.lib().orc_topk_positions(O.P(scores), C.c_int(n), C.c_int(2048), C.c_int(128), O.P(pos))
    t_idx = time.perf_counter() - t0
    x = synth.kv_rows(12, 1, 2048)
    codes, sexp, tail, _ = O.fp8_quant_rows(x)
    t0 = time.perf_counter()
    O.attn_decode_fp8(q, codes, sexp, tail, np.arange(2048), sinks, n_threads=threads)
    t_dec = time.perf_counter() - t0
    res["cfg3_indexer_ms_1thread"] = round(t_idx * 1e3, 1)
    res["cfg3_decode_2048_ms"] = round(t_dec * 1e3, 2)
    # cfg 4: 4 sampled queries of the 2048 (each over 8192 cached rows + its own prefix)
    x = synth.kv_rows(13, 1, 8192 + 2048)
    codes, sexp, tail, _ = O.fp8_quant_rows(x)
    t0 = time.perf_counter()
    for t in (0, 682, 1365, 2047):
        O.attn_decode_fp8(q, codes, sexp, tail, np.arange(8192 + t + 1), sinks, n_threads=threads)
    per_q = (time.perf_counter() - t0) / 4
    res["cfg4_prefill_ms_est"] = round(per_q * 2048 * 1e3, 0)
    res["cfg4_prefill_tflops_est"] = round(2.474035380224e12 / (per_q * 2048) / 1e12, 4)
    return res


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
    from ds4cuda_amd import ops, synth
    n_cached, n_q = 8192, 2048
    cache = ops.Fp8KVCache.empty(n_cached + n_q, device=dev)
    cache.append(synth.kv_rows_device(13, 1, n_cached + n_q, dev))
    q = synth.normal_device(13, 2, n_q * N_HEAD * HEAD_DIM, dev).reshape(n_q, N_HEAD, HEAD_DIM)
    q = q.to(torch.bfloat16)
    sinks = synth.normal_device(13, 3, N_HEAD, dev)
    out = torch.empty((n_q, N_HEAD, HEAD_DIM), device=dev)
    ws = ops.flash_attn_prefill_fp8(q, sinks, out, cache, n_q, n_cached, stream=stream)
    ms = time_ms(lambda: ops.flash_attn_prefill_fp8(q, sinks, out, cache, n_q, n_cached,
                                                    workspace=ws, stream=stream),
                 steps, 2, stream)
    ms_exact = time_ms(lambda: ops.flash_attn_prefill_fp8(q, sinks, out, cache, n_q, n_cached,
                                                          workspace=ws, exact_p=True, stream=stream),
                       steps, 2, stream)
    causal = 4 * N_HEAD * HEAD_DIM * sum(n_cached + i + 1 for i in range(n_q))
    full = 4 * N_HEAD * HEAD_DIM * n_q * (n_cached + n_q)
    tf = causal / (ms * 1e-3) / 1e12
    return {"workload": "chunked prefill: 2048 queries over 8192 cached + causal self, 64 heads, "
                        "head_dim 512, bf16 Q, FP8 KV (BASELINE configs[3])",
            "ms": round(ms, 4), "tflops_causal": round(tf, 1),
            "tflops_nomask_credit": round(full / (ms * 1e-3) / 1e12, 1),
            "flops_causal": causal, "peak_tflops": MFMA_PEAK_TFLOPS,
            "frac": round(tf / MFMA_PEAK_TFLOPS, 4),
            "p_precision": "one f16 P (default); hi + lo P figure under exact_p",
            "exact_p": {"ms": round(ms_exact, 4),
                        "tflops_causal": round(causal / (ms_exact * 1e-3) / 1e12, 1),
                        "frac": round(causal / (ms_exact * 1e-3) / 1e12 / MFMA_PEAK_TFLOPS, 4)}}


def bench_sparse(dev, stream, steps):
    """indexer over 131072 bf16 index keys (64 heads x
    128), top-2048 incl. the last 128, then decode over the 2048 gathered FP8
    rows of a 131072-row cache."""
    import torch
    from ds4cuda_amd import ops, synth
    n, top_k, recent = 131072, 2048, 128
    keys = synth.normal_device(11, 1, n * 128, dev).reshape(n, 128).to(torch.bfloat16)
    qi = synth.normal_device(11, 2, N_HEAD * 128, dev).reshape(N_HEAD, 128)
    qi = qi.to(torch.bfloat16).float()
    w = synth.normal_device(11, 3, N_HEAD, dev) / float(np.sqrt(128 * N_HEAD))
    cache = ops.Fp8KVCache.empty(n, device=dev)
    cache.append(synth.kv_rows_device(11, 4, n, dev, outlier_frac=0.01))
    q = synth.normal_device(11, 5, N_HEAD * HEAD_DIM, dev).reshape(1, N_HEAD, HEAD_DIM)
    q = q.to(torch.bfloat16)
    sinks = synth.normal_device(11, 6, N_HEAD, dev).reshape(1, N_HEAD)
    out = torch.empty((1, N_HEAD, HEAD_DIM), device=dev)
    from ds4cuda_amd._lib import lib
    scores = torch.empty(n, device=dev)
    select = torch.empty(lib().ds4hip_indexer_select_scratch_bytes(n), dtype=torch.uint8,
                         device=dev)
    pos = torch.empty((1, top_k), dtype=torch.int32, device=dev)
    ws = torch.empty(ops.decode_fp8_workspace_bytes([top_k]), dtype=torch.uint8, device=dev)

    def step(st=stream):
        sel_only(st)
        ops.flash_attn_decode_fp8(q, sinks, out, cache, [top_k], row_idx=pos, workspace=ws,
                                  stream=st)

    def sel_only(st=stream):
        ops.indexer_topk_positions(qi, w, keys, top_k, recent, scores=scores, select=select,
                                   positions=pos[0], stream=st)

    ms = time_ms(step, steps, 3, stream)
    ms_idx = time_ms(sel_only, steps, 3, stream)
    b = n * 128 * 2 + N_HEAD * 128 * 4 + N_HEAD * 4 + 2 * n * 4 + top_k * (ROW_BYTES + 4) \
        + N_HEAD * HEAD_DIM * 6 + N_HEAD * 4
    return {"workload": "sparse decode: indexer over 131072 bf16 keys (64 heads x 128), top-2048 "
                        "incl. last 128, decode over the gathered FP8 rows (BASELINE configs[2])",
            "us": round(ms * 1e3, 2), "us_indexer": round(ms_idx * 1e3, 2),
            "bytes": b, "gbs": round(b / (ms * 1e-3) / 1e9, 1),
            "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)}


def batch_weights(dev, seed=70):
    """Random-init weights of the batched block (fp32 compressor projections
    ~N(0, 0.02), bf16 output projection ~N(0, 0.02)), from the shared generator."""
    import torch
    from ds4cuda_amd import synth
    n = lambda s, shape, std: synth.normal_device(seed, s, int(np.prod(shape)), dev,
                                                  std).reshape(shape)
    return {
        "w_kv": n(1, (1024, 4096), 0.02), "w_gate": n(2, (1024, 4096), 0.02),
        "wi_kv": n(3, (256, 4096), 0.02), "wi_gate": n(4, (256, 4096), 0.02),
        "ape": n(5, (4, 1024), 0.02).half().view(torch.int16).contiguous(),
        "ape_i": n(6, (4, 256), 0.02).half().view(torch.int16).contiguous(),
        "wn": (1.0 + n(7, (512,), 0.1)).contiguous(),
        "wn_i": (1.0 + n(8, (128,), 0.1)).contiguous(),
        "w_out": n(9, (4096, N_HEAD * HEAD_DIM), 0.02).to(torch.bfloat16).contiguous(),
    }


def bench_token(dev, stream, steps, ctx=4096):
    """The attention slice (Steps 11-16) of all 43 layers for one token at
    context `ctx` over the FP8 session (ds4cuda_amd.token), model top-k 512:
    eager launches from Python against one HIP graph of the whole token
    (cuda/forward_token.cu:368-378 runs the layers one launch at a time)."""
    import torch
    from ds4cuda_amd import session, token
    w = token.synthetic_weights(dev)
    s = session.Session(ctx + 64)
    try:
        token.fill_history(s, ctx)
        ts = token.TokenSlice(s, w, top_k=512)
        g = torch.Generator(device=dev)
        g.manual_seed(7)
        x = [torch.randn(shape, generator=g, device=dev) for shape in ((43, 512), (43, 4096),
                                                                      (43, 64, 512), (43, 1024))]
        out = torch.empty((43, 4096), device=dev)
        n_eager = max(3, steps // 10)
        torch.cuda.synchronize()
        ts.step(ctx, *x, out, stream=stream)          # warm
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(n_eager):
            ts.step(ctx + 1 + i, *x, out, stream=stream)
        e1.record(stream)
        torch.cuda.synchronize()
        us_eager = e0.elapsed_time(e1) * 1e3 / n_eager
        graph = ts.capture(ctx + 1 + n_eager, *x, out)
        us_graph = time_ms(graph.replay, steps, 3, torch.cuda.current_stream()) * 1e3
    finally:
        s.close()
    # weight bytes a token streams: the Q8_0 output projections (8192 x 4096 and
    # 4096 x 8192, 34 B per 32) and the f16 compressor / indexer projections
    q8 = 2 * 8192 * 4096 // 32 * 34
    f16c = sum((2 * 2 * 512 * 4096 * 2 + 2 * 2 * 128 * 4096 * 2 + 8192 * 1024 * 2 + 64 * 4096 * 2)
               if token.layer_ratio(il) == 4 else (2 * 512 * 4096 * 2 if token.layer_ratio(il) else 0)
               for il in range(43))
    b = 43 * q8 + f16c
    return {"workload": f"attention slice (Steps 11-16) of all 43 layers for one token at context {ctx}, "
                        "FP8 session, fp32 Q, indexer top-512, Q8_0 attn_out",
            "us_per_token_graph": round(us_graph, 1), "us_per_token_eager": round(us_eager, 1),
            "us_per_layer_graph": round(us_graph / 43, 2),
            "weight_bytes": b, "gbs_graph": round(b / (us_graph * 1e-6) / 1e9, 1),
            "frac": round(b / (us_graph * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}


def bench_batch(dev, stream, steps):
    """the attention block of one layer for 16 sequences
    in batched decode (contexts ~U[1024, 16384], seeded): compressor (ratio
    4, fp32 weights) for the attention and the indexer keys, FP8 quantize +
    append into a 256-row paged cache, sparse top-2048 selection, decode
    attention, inverse tail RoPE and the bf16 attn_out projection
    32768 -> 4096 (ds4cuda_amd.batch_block.BatchedAttentionBlock, the code
    tests/test_gpu_block.py checks against the oracle)."""
    from ds4cuda_amd import synth
    from ds4cuda_amd.batch_block import BatchedAttentionBlock
    B, IN, TOPK, SWA = 16, 4096, 2048, 128
    ctx = np.random.default_rng(5).integers(1024, 16385, size=B)
    pos = (ctx - 1).astype(np.int64)
    w = batch_weights(dev)
    blk = BatchedAttentionBlock(w, B, int(pos.max()) + 1, device=dev)
    for b in range(B):
        n = int(pos[b]) // 4
        blk.load_history(b, synth.kv_rows_device(71, b, n, dev, outlier_frac=0.01),
                         synth.kv_rows_device(72, b, SWA, dev),
                         np.arange(pos[b] - SWA + 1, pos[b] + 1),
                         synth.normal_device(73, b, n * 128, dev).reshape(n, 128), stream=stream)
    g = lambda s, shape: synth.normal_device(75, s, int(np.prod(shape)), dev).reshape(shape)
    x, kv_cur = g(1, (B, IN)), g(2, (B, 512))
    import torch
    q = g(3, (B, N_HEAD, HEAD_DIM)).to(torch.bfloat16)
    q_idx = g(4, (B, N_HEAD, 128))
    w_idx = g(5, (B, N_HEAD)) / float(np.sqrt(128 * N_HEAD))
    sinks = g(6, (B, N_HEAD))
    blk.plan(pos)

    def step():
        blk.step(pos, x, kv_cur, q, q_idx, w_idx, sinks, stream=stream)

    ms_eager = time_ms(step, steps, 3, stream)
    # the same step captured once in a HIP graph (13 kernels, one graph launch)
    torch.cuda.synchronize()
    graph_error = None
    try:
        graph = blk.capture(pos, x, kv_cur, q, q_idx, w_idx, sinks)
        ms = time_ms(graph.replay, steps, 3, stream)
    except Exception as e:   # noqa: BLE001
        graph_error = f"{type(e).__name__}: {e}"
        log(f"graph capture of the batched block failed ({graph_error}); reporting the eager step")
        ms = ms_eager
    n_comp = blk.plan(pos)["n_comp"]
    sel = [min(int(n), TOPK) for n in n_comp]
    b = (w["w_out"].numel() * 2 + sum(w[k].numel() for k in ("w_kv", "w_gate", "wi_kv", "wi_gate")) * 4
         + int(sum(n * 512 for n in n_comp if n > TOPK))
         + sum((SWA + s_) * ROW_BYTES for s_ in sel) + B * (IN * 4 + N_HEAD * HEAD_DIM * (2 + 4 + 4)
                                                          + 4096 * 4))
    return {"workload": "batched-decode attention block, one layer: 16 sequences, ctx ~U[1024,16384] "
                        "(seed 5), compressor ratio 4 (fp32 W), FP8 append into 256-row pages, "
                        "top-2048 selection, decode, inverse RoPE, bf16 attn_out 32768->4096 "
                        "(BASELINE configs[4])",
            "us_per_step_layer": round(ms * 1e3, 2), "us_per_step_layer_eager": round(ms_eager * 1e3, 2),
            "timing": ("HIP graph replay of the step (us_per_step_layer_eager: the same launches from Python)"
                       if graph_error is None else f"eager step (graph capture failed: {graph_error})"),
            "bytes": b,
            "gbs": round(b / (ms * 1e-3) / 1e9, 1),
            "frac": round(b / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "contexts": [int(c) for c in ctx]}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-secondary", action="store_true",
                    help="skip the prefill / sparse-decode / batched-block figures")
    ap.add_argument("--kernel", choices=("flat", "ws"), default=None,
                    help="decode kernel for direct rows: the flat-stage kernel (default) or the "
                         "register-load kernel")
    ap.add_argument("--only", choices=("prefill", "sparse", "batch", "token"),
                    help="run one secondary config alone and print its figures as one JSON "
                         "line (for profiling it without the cfg 2 cache)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of known size (the reference kernel "
                         "that scales the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        log("bench.py measures the single-GPU path only: the attention path has no "
            "cross-GPU component in this build (run with --gpus 1).")
        sys.exit(2)

    global DECODE_KERNEL
    if args.kernel:
        DECODE_KERNEL = args.kernel
    import torch
    from ds4cuda_amd import ops

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        n = COPY_BYTES // 4
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration": {"bytes_read": COPY_BYTES, "bytes_written": COPY_BYTES,
                                               "launches": 5}}), flush=True)
        return
    if args.only:
        stream = torch.cuda.current_stream()
        fn = {"prefill": lambda: bench_prefill(dev, stream, max(3, args.steps // 10)),
              "sparse": lambda: bench_sparse(dev, stream, args.steps),
              "batch": lambda: bench_batch(dev, stream, args.steps),
              "token": lambda: bench_token(dev, stream, args.steps)}[args.only]
        log(f"secondary config {args.only} alone")
        print(json.dumps({"only": args.only, "figures": fn()}), flush=True)
        return
    from ds4cuda_amd import synth
    total_rows = N_LAYERS * N_KV
    log(f"building {N_LAYERS} x {N_KV} FP8 cache ({total_rows * ROW_BYTES / 1e6:.0f} MB)")
    cache = ops.Fp8KVCache.empty(total_rows, device=dev)
    # layer l: kv_rows(seed 1, stream l) with 1% of rows x8; Q, sinks: seeds 2, 3
    for l in range(N_LAYERS):
        cache.append(synth.kv_rows_device(1, l, N_KV, dev, outlier_frac=0.01), row0=l * N_KV)
    q_f32 = synth.normal_device(2, 0, N_LAYERS * N_HEAD * HEAD_DIM, dev)
    q_f32 = q_f32.reshape(N_LAYERS, N_HEAD, HEAD_DIM)
    q = q_f32.to(torch.bfloat16)
    sinks = synth.normal_device(3, 0, N_LAYERS * N_HEAD, dev).reshape(N_LAYERS, N_HEAD)
    out = torch.zeros((N_LAYERS, N_HEAD, HEAD_DIM), device=dev)
    counts = [N_KV] * N_LAYERS
    ws = torch.empty(ops.decode_fp8_workspace_bytes(counts), dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream()

    kern = "regload" if DECODE_KERNEL == "ws" else "auto"

    def step(phases=3, exact_p=False, st=stream, qq=q):
        ops.flash_attn_decode_fp8(qq, sinks, out, cache, counts, row_base_stride=N_KV,
                                  workspace=ws, phases=phases, exact_p=exact_p, kernel=kern,
                                  stream=st)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    ref_out = out.clone()

    # the K steps recorded as one HIP graph (2K kernel nodes), as a serving
    # loop records its decode; a replay of a one-step graph costs more than
    # the step's own launches, so the graph holds all K
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            for _ in range(args.steps):
                step(st=side)
    stream.wait_stream(side)
    graph.replay()   # warm
    out.zero_()
    torch.cuda.synchronize()

    # timed region: K whole steps (one replay)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    graph.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / args.steps
    graph_ok = bool(torch.equal(out, ref_out))
    # the same K steps launched from Python, two launches per step
    ms_eager = time_ms(step, args.steps, 2, stream)

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

    # the same step with P passed to P.V as f16 hi + lo halves (~22 bits)
    ms_exact = time_ms(lambda: step(exact_p=True), args.steps, 2, stream)
    # the same step with the fp32 Q a model layer's Q producer hands the decode
    ms_f32 = time_ms(lambda: step(qq=q_f32), args.steps, 2, stream)

    step_bytes = N_LAYERS * bytes_per_layer()
    fp32_bytes = step_bytes + N_LAYERS * N_HEAD * HEAD_DIM * 2   # Q read as fp32
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
        "data": "synthetic, splitmix64 + Box-Muller (ds4cuda_amd.synth, generated on the device): "
                "KV ~N(0,1) with 1% of rows x8, FP8 E4M3FN per-64-block pow2 scales; bf16 Q "
                "~N(0,1); sinks ~N(0,1)",
        "config": {"workload": "decode attention, 43 layers x 32768-row FP8 KV cache, batch 1, "
                               "64 q-heads / 1 latent KV head, head_dim 512 (BASELINE configs[1])",
                   "layers": N_LAYERS, "n_kv": N_KV, "n_head": N_HEAD, "head_dim": HEAD_DIM,
                   "kv_bytes_per_row": ROW_BYTES, "us_per_layer": round(ms * 1e3 / N_LAYERS, 3),
                   "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
                   "timing": "one HIP graph of the K steps (2K launches), replayed once inside the "
                             "timed region; ms_per_step_eager: the same steps launched from Python",
                   "ms_per_step_eager": round(ms_eager, 4), "graph_matches_eager": graph_ok,
                   "p_precision": "one f16 P (default); hi + lo P figure under exact_p",
                   "exact_p": {"ms_per_step": round(ms_exact, 4),
                               "value": round(step_bytes / (ms_exact * 1e-3) / 1e9, 2)},
                   "fp32_q": {"ms_per_step": round(ms_f32, 4),
                              "value": round(fp32_bytes / (ms_f32 * 1e-3) / 1e9, 2),
                              "note": "the same step with fp32 Q (three FP8 parts of Q in the flat kernel); "
                                      "bytes count Q at 4 B per element"}},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": TRAFFIC_BYTES_PER_LAUNCH.get(DECODE_KERNEL),
                     "traffic_measured_at": TRAFFIC_MEASURED_AT.get(DECODE_KERNEL),
                     "kernel": KERNEL_LABEL[DECODE_KERNEL],
                     "kernel_ms": round(k_ms, 4), "bytes_per_launch": step_bytes},
    }
    if not args.no_secondary:
        log("secondary configs: chunked prefill, sparse decode, batched block")
        # a failing secondary config is reported in its entry; it does not
        # take the headline line down with it
        def guarded(fn):
            try:
                return fn()
            except Exception as e:   # noqa: BLE001
                log(f"secondary config failed: {type(e).__name__}: {e}")
                return {"error": f"{type(e).__name__}: {e}"}
        res["secondary"] = {"prefill": guarded(lambda: bench_prefill(dev, stream, max(3, args.steps // 10))),
                            "sparse_decode": guarded(lambda: bench_sparse(dev, stream, args.steps)),
                            "batched_block": guarded(lambda: bench_batch(dev, stream, args.steps)),
                            "token_slice": guarded(lambda: bench_token(dev, stream, args.steps))}
    if not args.no_cpu_baseline:
        log("timing the CPU baseline (oracle) on one layer")
        res["cpu_baseline"] = cpu_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
