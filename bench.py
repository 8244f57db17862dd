"""Benchmark of the fp8-KV decode hot path on one MI355X (BASELINE.json metric: decode-attn HBM GB/s (% of peak) +
decode tokens/s, bs64 ctx8K).

Workload (config 3): batch 64, 16 query / 4 kv heads, head dim 128, prior context per sequence U[512, 8192]
(seeded), fp8 e4m3 K/V in 16-token pages under a random block permutation, values N(0,1) with 1 % outliers at
8σ. A step appends one token to every sequence (QK-norm + RoPE + quantise) and runs decode attention over the fp8
cache, new keys included: one nc_decode_step_fp8 call (the append fused into the attention kernel; --unfused: an
nc_kv_append_fp8 call, then nc_decode_attn_fp8). Each step also writes the next positions, pos + 1; two steps
(positions ping-ponging between two tensors) are captured in a HIP graph and replayed.

Output: one JSON line. value = algorithmic attention bytes per step / measured step time (GB/s, inputs resident in
HBM); roofline = the step's attention call (k_decode, then k_merge): the timed steps themselves (one
nc_decode_step_fp8 call each), or with --unfused the attention call alone at the last step's context, timed over
graph replays of 10 back-to-back calls, with HIP events on their stream; attention_only = that attention call
alone in either mode (the decode kernel and the split-K merge without the append, the kernels the metric counts);
cpu_baseline = the numpy oracle over a bounded sample of the same sequences on this host's cores.
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

METRIC = "decode-attn HBM GB/s (% of peak) + decode tokens/sec, bs64 ctx8K"
HBM_PEAK_GBS = 8000.0
MFMA_PEAK_TFS = 2500.0  # dense bf16 / fp16 MFMA, MI355X
ATTN_REPS = 10  # decode-attention calls per timed graph replay: the replay-to-replay gap is not kernel time
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_attn_traffic.json")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bound of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the config 2 decode, config 4 prefill and config 5 end-to-end lines")
    ap.add_argument("--only", choices=["decode2", "prefill4", "e2e5"],
                    help="run one secondary workload alone and print its object (for profiling runs)")
    ap.add_argument("--e2e-steps", type=int, default=None, help="decode steps of the config 5 run (default 512)")
    ap.add_argument("--unfused", action="store_true",
                    help="time the step as two calls (nc_kv_append_fp8, then nc_decode_attn_fp8) instead of the "
                         "fused nc_decode_step_fp8")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the measurement, copy a 1 GiB buffer 3 times (the byte-counter calibration kernel)")
    return ap.parse_args()


def replay_ms(graph, n: int, stream) -> float:
    """Mean GPU time of one replay over n back-to-back replays, HIP events on the replay stream."""
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        start.record(stream)
        for _ in range(n):
            graph.replay()
        end.record(stream)
    end.synchronize()
    return start.elapsed_time(end) / n


def traffic_bytes(call: str):
    """HBM bytes per `call` (nc_decode_step_fp8 or nc_decode_attn_fp8) from the rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes, each scaled by what the counter reads for a plain 1 GiB copy (TRAFFIC_FILE, written from the profiling
    runs); None if absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)[call]["bytes_per_call"]
    except (OSError, KeyError, ValueError):
        return None


def copy_probe(dev) -> None:
    import torch

    src = torch.ones(1 << 28, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()


def time_calls(fn, calls: int, replays: int, stream) -> float:
    """Mean GPU time (ms) of one fn() call: a graph of `calls` back-to-back calls replayed `replays` times, HIP
    events on the replay stream."""
    import torch

    with torch.cuda.stream(stream):
        fn()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(calls):
                fn()
        graph.replay()
    return replay_ms(graph, replays, stream) / calls


def extra_decode_cfg2(dev, stream) -> dict:
    """Config 2 (B 32, 10/10 heads, ctx 4096 contiguous): one decode-attention call after the step's append."""
    from nanochat_amd.attention import decode_attention, decode_workspace
    from nanochat_amd.workloads import CONFIG2, build_decode_case, decode_bytes

    cfg = CONFIG2
    case = build_decode_case(cfg, dev, steps=1)
    pos = case.positions(0)
    q = case.cache.append(case.qkv[0], pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq)
    ctx = pos + 1
    ws = decode_workspace(cfg.batch, cfg.hq, cfg.hkv, case.cache.capacity, dev)
    out = torch_empty_like(q)
    ms = time_calls(lambda: decode_attention(q, case.cache, ctx, max_ctx=case.cache.capacity, out=out, workspace=ws),
                    ATTN_REPS, 20, stream)
    nbytes = decode_bytes(case.ctx + 1, cfg.hkv, cfg.window)
    gbs = nbytes / (ms * 1e-3) / 1e9
    return {"workload": cfg.name, "attn_us": round(ms * 1e3, 3), "bytes": int(nbytes), "GB_s": round(gbs, 2),
            "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}


def extra_prefill_cfg4(dev, stream) -> dict:
    """Config 4 (B 8, 16/4 heads, 3584 cached + 512-token chunk): the chunk's append, then prefill attention; the
    attention call timed alone (MFMA-bound: algorithmic flops over time against the dense bf16 peak)."""
    from nanochat_amd.attention import prefill_attention
    from nanochat_amd.workloads import CONFIG4, build_prefill_case, prefill_flops

    cfg = CONFIG4
    case = build_prefill_case(cfg, dev)
    q = case.cache.append(case.qkv, case.pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq)
    out = torch_empty_like(q)
    ms = time_calls(lambda: prefill_attention(q, case.cache, case.pos, case.seq, out=out), ATTN_REPS, 10, stream)
    append_ms = time_calls(lambda: case.cache.append(case.qkv, case.pos, case.seq, case.q_gain, case.k_gain, case.cos,
                                                     case.sin, cfg.hq), ATTN_REPS, 10, stream)
    flops = prefill_flops(case.pos.cpu().numpy(), cfg.hq, cfg.window)
    tfs = flops / (ms * 1e-3) / 1e12
    return {"workload": cfg.name, "attn_us": round(ms * 1e3, 3), "append_us": round(append_ms * 1e3, 3),
            "flops": flops, "TFLOP_s": round(tfs, 1), "bound": "mfma", "peak_TFLOP_s": MFMA_PEAK_TFS,
            "frac_of_mfma_peak": round(tfs / MFMA_PEAK_TFS, 4)}


def extra_e2e_cfg5(dev, steps: int | None = None) -> dict:
    """Config 5: random-init 26-layer d1664 model, 128 random 2048-token prompts prefilled into the fp8 cache, then
    512 greedy decode steps replayed from one captured graph; tokens/s and the decode steps' algorithmic HBM bytes
    (bf16 weights once + 264 B per cached (token, head, layer))."""
    import torch

    from nanochat_amd.decoder import CONFIG5, generate

    cfg = CONFIG5
    if steps is not None:
        from dataclasses import replace

        cfg = replace(cfg, steps=steps, name=cfg.name.replace(f"steps{cfg.steps}", f"steps{steps}"))
    toks, info, keep = generate(cfg, dev)
    del keep
    torch.cuda.empty_cache()
    m, B, steps = cfg.model, cfg.batch, cfg.steps
    kv = sum((cfg.prompt - 1 + i + 1) * B * m.kv_heads * 264 * m.layers for i in range(steps))
    step_bytes = (kv + steps * info["weight_bytes"]) / steps
    dec_s, pre_s = info["decode_ms"] * 1e-3, info["prefill_ms"] * 1e-3
    gbs = step_bytes / (dec_s / steps) / 1e9
    return {"workload": cfg.name, "prefill_s": round(pre_s, 4), "decode_s": round(dec_s, 4),
            "decode_ms_per_step": round(info["decode_ms_per_step"], 4),
            "decode_tokens_per_s": round(B * steps / dec_s, 1),
            "e2e_tokens_per_s": round(B * steps / (pre_s + dec_s), 1),
            "decode_step_bytes": int(step_bytes), "decode_GB_s": round(gbs, 1),
            "decode_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "check": {"first_tokens": toks[0, :4].tolist(), "distinct_tokens": int(toks.unique().numel())}}


def torch_empty_like(t):
    import torch

    return torch.empty_like(t)


def cpu_baseline(case, final_ctx: np.ndarray, q, budget_s: float) -> dict:
    """The oracle's decode attention (numpy, fp64 over the dequantised cache) on whole sequences of the same cache,
    in order, until budget_s of work; GB/s over the same algorithmic bytes as the GPU figure."""
    import math

    from threadpoolctl import threadpool_limits

    from nanochat_amd.workloads import decode_bytes
    from oracle import golden as G

    cores = len(os.sched_getaffinity(0))
    cache = case.cache
    host = G.PagedCache(cache.num_blocks, cache.hkv)
    host.pages[...] = cache.pages.cpu().numpy()
    table = cache.block_table.cpu().numpy() if cache.block_table is not None else None
    qb = q.contiguous().cpu().view(__import__("torch").int16).numpy().view(np.uint16)
    cfg = case.cfg
    done, t_total = 0, 0.0
    with threadpool_limits(limits=cores):
        while done < cfg.batch and t_total < budget_s:
            b = done
            t0 = time.perf_counter()
            G.decode_attention(qb[b:b + 1], host, table[b:b + 1] if table is not None else None, cache.max_blocks,
                               final_ctx[b:b + 1], cfg.window, cfg.hq, cfg.hkv, 1 / math.sqrt(128))
            t_total += time.perf_counter() - t0
            done += 1
    nbytes = decode_bytes(final_ctx[:done], cfg.hkv, cfg.window)
    return {"value": round(nbytes / t_total / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle decode attention (numpy fp64 over dequantised fp8) of the first {done} of "
                      f"{cfg.batch} sequences ({int(final_ctx[:done].sum())} keys x {cfg.hkv} kv heads), "
                      f"{t_total:.1f} s"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the decode path shards by "
              "(sequence, kv head) with no exchange, see DESIGN.md", file=sys.stderr)
        sys.exit(2)
    import torch

    from nanochat_amd.attention import decode_attention, decode_step, decode_workspace
    from nanochat_amd.workloads import CONFIG3, build_decode_case, decode_bytes

    dev = torch.device("cuda:0")
    if args.only:
        s = torch.cuda.Stream(dev)
        run = {"decode2": lambda: extra_decode_cfg2(dev, s), "prefill4": lambda: extra_prefill_cfg4(dev, s),
               "e2e5": lambda: extra_e2e_cfg5(dev, args.e2e_steps)}[args.only]
        print(json.dumps(run()), flush=True)
        return
    cfg = CONFIG3
    steps, warmup = args.steps, args.warmup
    case = build_decode_case(cfg, dev, steps=steps + warmup + 2)
    B = cfg.batch
    max_ctx = case.cache.capacity
    # positions ping-pong between two tensors: a step appends at pos and writes pos + 1 into the other tensor, the
    # next step's positions (no position-advance kernel)
    p0 = case.positions(0).contiguous()
    p1 = torch.empty_like(p0)
    qkv = case.qkv[0].contiguous()
    ws = decode_workspace(B, cfg.hq, cfg.hkv, max_ctx, dev)
    out = torch.empty((B, cfg.hq, 128), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()

    def fused(pos, nxt):
        decode_step(qkv, case.cache, pos, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq, max_ctx=max_ctx,
                    window=cfg.window, out=out, workspace=ws, pos_out=nxt)

    def unfused(pos, ctx):
        q = case.cache.append(qkv, pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq, ctx_out=ctx)
        decode_attention(q, case.cache, ctx, max_ctx=max_ctx, window=cfg.window, out=out, workspace=ws)

    step = unfused if args.unfused else fused

    stream = torch.cuda.Stream(dev)
    graph_ab, graph_a, attn_graph = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.stream(stream):
        # eager warm-up of every launch path before capture: two steps, positions back in p0
        step(p0, p1)
        step(p1, p0)
        stream.synchronize()
        with torch.cuda.graph(graph_ab, stream=stream):
            step(p0, p1)
            step(p1, p0)
        with torch.cuda.graph(graph_a, stream=stream):
            step(p0, p1)
    done = 2
    for _ in range(warmup // 2):
        graph_ab.replay()
        done += 2
    stream.synchronize()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(steps // 2):
            graph_ab.replay()
        if steps % 2:
            graph_a.replay()
        e1.record(stream)
    e1.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    wall = time.perf_counter() - t0
    torch.cuda.synchronize()
    base = case.ctx + done  # keys before the timed steps (prior context + the appended tokens)
    final_ctx = base + steps  # the keys of the last step
    ctx_len = p1 if steps % 2 else p0  # the last step's context lengths: its positions + 1
    with torch.cuda.stream(stream):
        # the last step's queries (cpu_baseline); appending its tokens again rewrites the same cache bytes
        q = case.cache.append(qkv, ctx_len - 1, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq)
    step_bytes = np.mean([decode_bytes(base + i + 1, cfg.hkv, cfg.window) for i in range(steps)])
    value = step_bytes / (step_ms * 1e-3) / 1e9
    # the attention call alone (the metric's decode kernel + split-K merge, without the append): ATTN_REPS calls at
    # the last step's context in one graph
    with torch.cuda.stream(stream):
        decode_attention(q, case.cache, ctx_len, max_ctx=max_ctx, window=cfg.window, out=out, workspace=ws)
        stream.synchronize()
        with torch.cuda.graph(attn_graph, stream=stream):
            for _ in range(ATTN_REPS):
                decode_attention(q, case.cache, ctx_len, max_ctx=max_ctx, window=cfg.window, out=out, workspace=ws)
    attn_ms = replay_ms(attn_graph, max(steps // ATTN_REPS, 2), stream) / ATTN_REPS
    attn_bytes = decode_bytes(final_ctx, cfg.hkv, cfg.window)
    attn_kernel = (f"nc_decode_attn_fp8 = k_decode<false> + k_merge, a graph of {ATTN_REPS} calls at the last "
                   "step's context, HIP events on their stream")
    if args.unfused:
        call_ms, call_bytes, call_kernel = attn_ms, attn_bytes, attn_kernel
    else:
        # the step is one nc_decode_step_fp8 call: the timed region is the roofline measurement itself
        call_ms, call_bytes = step_ms, step_bytes
        call_kernel = ("nc_decode_step_fp8 = k_decode<true> + k_merge, one call per timed step, HIP events on their "
                       "stream")
    achieved = call_bytes / (call_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3-kv/bf16+f16-mfma/fp32-softmax",
        "data": "synthetic",
        "config": {"workload": cfg.name, "batch": B, "hq": cfg.hq, "hkv": cfg.hkv, "head_dim": 128,
                   "ctx_prior": "U[512,8192] seed 3", "page": 16, "outliers": "1% at 8 sigma",
                   "mean_keys_per_seq": round(float(np.mean(base + steps / 2 + 1)), 1),
                   "step": ("nc_kv_append_fp8 + nc_decode_attn_fp8" if args.unfused else
                            "nc_decode_step_fp8 (append fused into the attention kernel)") +
                           ": append 1 token/seq (qk-norm+rope+fp8 quantise, emitting the next positions) + split-K "
                           "decode attention, one attention layer, graph replays of two steps"},
        "pct_of_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "decode_tokens_per_s_one_layer": round(B / (step_ms * 1e-3), 1),
        "attention_only": {"kernel": attn_kernel, "call_us": round(attn_ms * 1e3, 3),
                           "GB_s": round(attn_bytes / (attn_ms * 1e-3) / 1e9, 2),
                           "frac_of_hbm_peak": round(attn_bytes / (attn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
        "call_us": round(call_ms * 1e3, 3),
        "step_us": round(step_ms * 1e3, 3),
        "wall_s_timed": round(wall, 4),
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic_bytes("nc_decode_attn_fp8" if args.unfused else "nc_decode_step_fp8"),
                     "kernel": call_kernel, "bytes_per_launch": int(call_bytes)},
    }
    if not args.no_extra:
        result["decode_cfg2"] = extra_decode_cfg2(dev, stream)
        result["prefill_cfg4"] = extra_prefill_cfg4(dev, stream)
        result["e2e_cfg5"] = extra_e2e_cfg5(dev, args.e2e_steps)
    if args.copy_probe:
        copy_probe(dev)
    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(case, final_ctx, q, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
