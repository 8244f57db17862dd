"""Benchmark of the fp8-KV decode hot path on one MI355X (BASELINE.json metric: decode-attn HBM GB/s (% of peak) +
decode tokens/s, bs64 ctx8K).

Workload (config 3): batch 64, 16 query / 4 kv heads, head dim 128, prior context per sequence U[512, 8192]
(seeded), fp8 e4m3 K/V in 16-token pages under a random block permutation, values N(0,1) with 1 % outliers at
8σ. A step appends one token to every sequence (QK-norm + RoPE + quantise) and runs decode attention over the fp8
cache, new keys included: one nc_decode_step_fp8 call (the append fused into the attention kernel; --unfused: an
nc_kv_append_fp8 call, then nc_decode_attn_fp8). Each step also writes the next positions, pos + 1; ten steps
(positions ping-ponging between two tensors) are captured in a HIP graph and replayed, as a decoder captures a
whole multi-layer step.

Output: one JSON line. value = algorithmic attention bytes per step / measured step time (GB/s, inputs resident in
HBM); roofline = the step's attention call (k_decode, then k_merge): the timed steps themselves (one
nc_decode_step_fp8 call each), or with --unfused the attention call alone at the last step's context, timed over
graph replays of 10 back-to-back calls, with HIP events on their stream; attention_only = that attention call
alone in either mode (the decode kernel and the split-K merge without the append, the kernels the metric counts);
cpu_baseline = the numpy oracle over a bounded sample of the same sequences on this host's cores; the config 2, 4
and 5 objects carry their own cpu_baseline (config 5's: the oracle's CPU model on one sequence, extrapolated to the
whole run and labelled so), each with the host's CPU model, thread count and torch version.

Profiling helpers (no measurement): --pmc-summary turns rocprofv3 --pmc output into per-kernel bytes and MFMA
figures, --stats-summary prints a rocprofv3 --stats kernel table; profiles/ holds their output.
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
POOLS = 2  # distinct cache pools (layers) the timed steps alternate between, so each step reads its pool cold
STEP_GROUP = 12  # decode steps per timed graph replay: whole cycles of the pools' position ping-pong (2 x POOLS)
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "decode_attn_traffic.json")


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--warm-seconds", type=float, default=1.0,
                    help="before the warm-up steps, replay steps that leave the pools unchanged for this long: the "
                         "GPU's clocks settle over about a second (a cold start measured 7 %% slower)")
    ap.add_argument("--cpu-seconds", type=float, default=15.0, help="bound of the CPU baseline sample")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-extra", action="store_true",
                    help="skip the config 2 decode, config 4 prefill and config 5 end-to-end lines")
    ap.add_argument("--only", choices=["decode1", "decode2", "prefill4", "e2e5", "handle5", "gemm5", "sweep"],
                    help="run one secondary workload alone and print its object (for profiling runs)")
    ap.add_argument("--e2e-steps", type=int, default=None, help="decode steps of the config 5 run (default 512)")
    ap.add_argument("--unfused", action="store_true",
                    help="time the step as two calls (nc_kv_append_fp8, then nc_decode_attn_fp8) instead of the "
                         "fused nc_decode_step_fp8")
    ap.add_argument("--copy-probe", action="store_true",
                    help="after the measurement, copy a 1 GiB buffer 3 times (the byte-counter calibration kernel)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="no measurement: summarise rocprofv3 --pmc output directories (counter_collection.csv) "
                         "per kernel of --kernels, as JSON")
    ap.add_argument("--kernels", default="k_decode<true, true>;k_merge",
                    help="--pmc-summary: the kernels (short names, separated by ;) whose last --last dispatches are averaged")
    ap.add_argument("--last", type=int, default=20, help="--pmc-summary: dispatches per kernel averaged")
    ap.add_argument("--stats-summary", metavar="DIR",
                    help="no measurement: print the kernel table of a rocprofv3 --kernel-trace --stats directory")
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


CALL_KERNELS = {"nc_decode_step_fp8": ("k_decode<true, true>", "k_merge"),  # config 3: paged (block table)
                "nc_decode_attn_fp8": ("k_decode<false, true>", "k_merge")}


def traffic_bytes(call: str):
    """Memory bytes per `call` (nc_decode_step_fp8 or nc_decode_attn_fp8): its kernels' read bytes (TCC_EA0_RDREQ
    by request size) plus write bytes (WRITE_SIZE's expression), per dispatch, from the rocprofv3 --pmc passes
    summarised in TRAFFIC_FILE (bench.py --pmc-summary); None if absent."""
    try:
        with open(TRAFFIC_FILE) as f:
            summary = json.load(f)[call]["summary"]
        return int(sum(summary[k]["read_bytes"] + summary[k]["write_bytes"] for k in CALL_KERNELS[call]))
    except (OSError, KeyError, ValueError):
        return None


def traffic_algorithmic() -> int | None:
    """The algorithmic bytes per call of the profiled run TRAFFIC_FILE summarises (its traffic is compared with
    those, not with this run's)."""
    try:
        with open(TRAFFIC_FILE) as f:
            return int(json.load(f)["algorithmic_bytes_per_call"])
    except (OSError, KeyError, ValueError):
        return None


COPY_PROBE_BYTES = 1 << 30  # read and written by each dispatch of the copy probe


def copy_probe(dev) -> None:
    """Three dispatches of an elementwise kernel that reads 1 GiB and writes 1 GiB (torch.neg, kernel name
    containing "neg"): the byte counters' calibration."""
    import torch

    src = torch.ones(COPY_PROBE_BYTES // 4, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()


def stats_summary(d: str, rows: int = 20) -> str:
    """The rocprofv3 --stats kernel table (kernel_stats.csv under d): calls, average / min / max duration, share."""
    import csv
    import glob

    f = glob.glob(os.path.join(d, "**", "*kernel_stats.csv"), recursive=True)[0]
    lines = [f"{'kernel':60s} {'calls':>6s} {'avg_us':>9s} {'min_us':>9s} {'max_us':>9s} {'pct':>6s}"]
    with open(f) as fh:
        for r in list(csv.DictReader(fh))[:rows]:
            n = r["Name"] if len(r["Name"]) < 60 else r["Name"][:57] + "..."
            lines.append(f"{n:60s} {int(r['Calls']):6d} {float(r['AverageNs']) / 1e3:9.3f} "
                         f"{float(r['MinNs']) / 1e3:9.3f} {float(r['MaxNs']) / 1e3:9.3f} {float(r['Percentage']):6.2f}")
    return "\n".join(lines)


SIMDS = 1024  # MI355X: 256 CUs x 4 SIMDs (SQ_VALU_MFMA_BUSY_CYCLES is summed over SIMDs)
XCDS = 8


def pmc_summary(dirs: list[str], kernels: list[str], last: int) -> dict:
    """Per-dispatch averages of every counter in rocprofv3 --pmc output directories for the named kernels (their
    last `last` dispatches) and for the copy probe, and the figures derived from them:
      read_bytes  = 32 RDREQ_32B + 64 RDREQ_64B + 128 RDREQ_128B   (TCC_EA0_* sums: requests from L2 to memory)
      fetch_bytes = FETCH_SIZE's own expression x 1024 (BUBBLE, RDREQ, RDREQ_32B)
      write_bytes = 32 (WRREQ - WRREQ_64B) + 64 WRREQ_64B            (WRITE_SIZE's expression x 1024)
      mfma_busy   = SQ_VALU_MFMA_BUSY_CYCLES / (GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs)  (GRBM_GUI_ACTIVE as collected
                    is the sum of the 8 XCDs' busy cycles; the busy cycles are summed over every SIMD)
    and for the copy probe each byte figure over the bytes it moves (1 GiB each way: the counters' calibration)."""
    import csv
    import glob
    from collections import defaultdict

    per = defaultdict(list)
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(f) as fh:
                for r in csv.DictReader(fh):
                    name = r["Kernel_Name"].split("(")[0]
                    name = name[5:] if name.startswith("void ") else name
                    if name not in kernels and name.split("<")[0] in kernels:  # a template named by its base name
                        name = name.split("<")[0]
                    if name not in kernels:
                        name = "copy_probe" if "neg" in r["Kernel_Name"] else None
                    if name:
                        per[(name, r["Counter_Name"])].append((int(r["Dispatch_Id"]), float(r["Counter_Value"])))
    out = {}
    for name in list(kernels) + ["copy_probe"]:
        c, n = {}, 0
        for (k, counter), v in per.items():
            if k == name:
                v.sort()
                vals = [x for _, x in v[-(3 if name == "copy_probe" else last):]]
                c[counter], n = sum(vals) / len(vals), len(vals)
        if not c:
            continue
        d = {"dispatches_averaged": n, "counters": c}
        g = lambda n: c.get(n + "_sum", c.get(n))
        if all(g(n) is not None for n in ("TCC_EA0_RDREQ_32B", "TCC_EA0_RDREQ_64B", "TCC_EA0_RDREQ_128B")):
            d["read_bytes"] = 32 * g("TCC_EA0_RDREQ_32B") + 64 * g("TCC_EA0_RDREQ_64B") + 128 * g("TCC_EA0_RDREQ_128B")
        if all(g(n) is not None for n in ("TCC_BUBBLE", "TCC_EA0_RDREQ", "TCC_EA0_RDREQ_32B")):
            d["fetch_bytes"] = (128 * g("TCC_BUBBLE") + 64 * (g("TCC_EA0_RDREQ") - g("TCC_BUBBLE") -
                                                             g("TCC_EA0_RDREQ_32B")) + 32 * g("TCC_EA0_RDREQ_32B"))
        if all(g(n) is not None for n in ("TCC_EA0_WRREQ", "TCC_EA0_WRREQ_64B")):
            d["write_bytes"] = 32 * (g("TCC_EA0_WRREQ") - g("TCC_EA0_WRREQ_64B")) + 64 * g("TCC_EA0_WRREQ_64B")
        if g("SQ_VALU_MFMA_BUSY_CYCLES") is not None and g("GRBM_GUI_ACTIVE"):
            d["mfma_busy"] = g("SQ_VALU_MFMA_BUSY_CYCLES") / (g("GRBM_GUI_ACTIVE") / XCDS * SIMDS)
            d["gpu_cycles"] = g("GRBM_GUI_ACTIVE") / XCDS
        if g("SQ_VALU_MFMA_COEXEC_CYCLES") is not None and g("SQ_VALU_MFMA_BUSY_CYCLES"):
            d["coexec_of_mfma_busy"] = g("SQ_VALU_MFMA_COEXEC_CYCLES") / g("SQ_VALU_MFMA_BUSY_CYCLES")
        if g("SQ_INSTS_VALU") is not None and g("SQ_INSTS_MFMA"):
            d["valu_per_mfma"] = g("SQ_INSTS_VALU") / g("SQ_INSTS_MFMA")
        mops = [g(n) for n in ("SQ_INSTS_VALU_MFMA_MOPS_F16", "SQ_INSTS_VALU_MFMA_MOPS_BF16",
                               "SQ_INSTS_VALU_MFMA_MOPS_F8") if g(n) is not None]
        if mops:
            d["mfma_flops"] = 512 * sum(mops)
        if name == "copy_probe":
            for key in ("read_bytes", "fetch_bytes", "write_bytes"):
                if key in d:
                    d[key.replace("_bytes", "_over_moved")] = d[key] / COPY_PROBE_BYTES
        out[name] = d
    return out


WARM_SECONDS = [1.0]  # set from --warm-seconds: replays before a timed measurement while the clocks settle


def time_calls(fn, calls: int, replays: int, stream) -> float:
    """Mean GPU time (ms) of one fn() call: a graph of `calls` back-to-back calls replayed `replays` times, HIP
    events on the replay stream, after replays for WARM_SECONDS."""
    import torch

    with torch.cuda.stream(stream):
        fn()
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for _ in range(calls):
                fn()
        graph.replay()
        t0 = time.perf_counter()
        while time.perf_counter() - t0 < WARM_SECONDS[0]:
            graph.replay()
            stream.synchronize()
    return replay_ms(graph, replays, stream) / calls


def extra_decode_cfg2(dev, stream, cpu_s: float | None = None) -> dict:
    """Config 2 (B 32, 10/10 heads, ctx 4096 contiguous): the decode-attention call after the step's append, over
    POOLS pools in turn (each read cold, as in a model); with cpu_s, the oracle's CPU leg on a bounded sample of the
    same sequences."""
    from nanochat_amd.attention import decode_attention, decode_workspace
    from nanochat_amd.workloads import CONFIG2, build_decode_case, decode_bytes

    cfg = CONFIG2
    cases = [build_decode_case(cfg, dev, steps=1) for _ in range(POOLS)]
    case = cases[0]
    pos = case.positions(0)
    qs = [c.cache.append(c.qkv[0], pos, c.seq, c.q_gain, c.k_gain, c.cos, c.sin, cfg.hq) for c in cases]
    ctx = pos + 1
    ws = decode_workspace(cfg.batch, cfg.hq, cfg.hkv, case.cache.capacity, dev)
    out = torch_empty_like(qs[0])
    turn = [0]

    def call():
        k = turn[0] % POOLS
        turn[0] += 1
        decode_attention(qs[k], cases[k].cache, ctx, max_ctx=case.cache.capacity, out=out, workspace=ws)

    ms = time_calls(call, ATTN_REPS, 20, stream)
    nbytes = decode_bytes(case.ctx + 1, cfg.hkv, cfg.window)
    gbs = nbytes / (ms * 1e-3) / 1e9
    res = {"workload": cfg.name, "pools": POOLS, "attn_us": round(ms * 1e3, 3), "bytes": int(nbytes),
           "GB_s": round(gbs, 2), "frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4)}
    if cpu_s:
        res["cpu_baseline"] = cpu_decode(case, case.ctx + 1, qs[0], cpu_s, gbs)
    return res


# Shapes of the decode sweep beside the five configs: (name, batch, query heads, kv heads, prior context, paged)
SWEEP_SHAPES = [("b1-16/4-ctx131072", 1, 16, 4, 131072, True),
                ("b8-16/4-ctx32768", 8, 16, 4, 32768, True),
                ("b64-16/4-ctx8192", 64, 16, 4, 8192, True),
                ("b256-8/8-ctx2048", 256, 8, 8, 2048, False),
                ("b128-13/13-ctx2304", 128, 13, 13, 2304, False),
                ("b32-32/8-ctx4096", 32, 32, 8, 4096, True),
                ("b16-64/4-ctx8192", 16, 64, 4, 8192, True)]


def extra_decode_sweep(dev, stream) -> list:
    """The decode path beyond the benchmark configs: for each of SWEEP_SHAPES (uniform contexts, N(0, 1) values),
    POOLS pools read cold in turn: the attention call alone (nc_decode_attn_fp8), the fused step
    (nc_decode_step_fp8, positions fixed so every call appends the same bytes) and the fused step with the
    batch-independent piece plan (16-page pieces), each as ATTN_REPS calls per graph replay."""
    import torch

    from nanochat_amd.attention import decode_attention, decode_step, decode_workspace
    from nanochat_amd.workloads import DecodeConfig, build_decode_case, decode_bytes

    rows = []
    for name, B, hq, hkv, ctx, paged in SWEEP_SHAPES:
        cfg = DecodeConfig(name, B, hq, hkv, ctx=(ctx,), paged=paged, seed=11)
        cases = [build_decode_case(cfg, dev, steps=1) for _ in range(POOLS)]
        case = cases[0]
        max_ctx = case.cache.capacity
        pos = case.positions(0)
        nxt = torch.empty_like(pos)
        qs = [c.cache.append(c.qkv[0], pos, c.seq, c.q_gain, c.k_gain, c.cos, c.sin, hq) for c in cases]
        ctx_len = pos + 1
        qkv = case.qkv[0].contiguous()
        ws = decode_workspace(B, hq, hkv, max_ctx, dev)
        out = torch_empty_like(qs[0])
        turn = [0]

        def attn():
            k = turn[0] % POOLS
            turn[0] += 1
            decode_attention(qs[k], cases[k].cache, ctx_len, max_ctx=max_ctx, out=out, workspace=ws)

        def step(pieces=0):
            k = turn[0] % POOLS
            turn[0] += 1
            c = cases[k]
            decode_step(qkv, c.cache, pos, c.q_gain, c.k_gain, c.cos, c.sin, hq, max_ctx=max_ctx, out=out,
                        workspace=ws, pos_out=nxt, piece_pages=pieces)

        nbytes = decode_bytes(case.ctx + 1, hkv)
        row = {"shape": name, "batch": B, "hq": hq, "hkv": hkv, "ctx": ctx + 1, "paged": paged, "bytes": int(nbytes)}
        for leg, fn in (("attn", attn), ("step", step), ("step_pieces", lambda: step(16))):
            ms = time_calls(fn, ATTN_REPS, 20, stream)
            gbs = nbytes / (ms * 1e-3) / 1e9
            row[leg] = {"us": round(ms * 1e3, 2), "GB_s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
        rows.append(row)
        print(json.dumps(row), flush=True)
        del cases, case, qs, ws, out, qkv
        torch.cuda.empty_cache()
    return rows


def extra_decode_cfg1(dev, stream, cpu_s: float | None = None) -> dict:
    """Config 1 (CPU plumbing: B 1, 6/6 heads, 1024 cached tokens + 1 appended, θ 1e6): the fused step on the GPU (a
    launch-bound figure, reported for completeness) and, with cpu_s, the oracle's append + decode attention on the
    host (1 warm-up, median of the timed calls)."""
    import math

    from nanochat_amd.attention import decode_step, decode_workspace
    from nanochat_amd.workloads import CONFIG1, build_decode_case, decode_bytes
    from oracle import golden as G

    cfg = CONFIG1
    case = build_decode_case(cfg, dev, steps=1)
    host, _ = _host_cache(case.cache)
    pos = case.positions(0)
    max_ctx = int(case.ctx.max()) + 1
    ws = decode_workspace(cfg.batch, cfg.hq, cfg.hkv, max_ctx, dev)
    out = torch_empty_like(case.qkv[0][:, :cfg.hq * 128].reshape(cfg.batch, cfg.hq, 128))
    ms = time_calls(lambda: decode_step(case.qkv[0], case.cache, pos, case.q_gain, case.k_gain, case.cos, case.sin,
                                        cfg.hq, max_ctx=max_ctx, out=out, workspace=ws), ATTN_REPS, 20, stream)
    nbytes = decode_bytes(case.ctx + 1, cfg.hkv, cfg.window)
    res = {"workload": cfg.name, "step_us": round(ms * 1e3, 3), "bytes": int(nbytes),
           "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 2), "note": "1.6 MB per step: launch-bound, not a bandwidth figure"}
    if cpu_s:
        qkv = _q_bits(case.qkv[0])
        p = pos.cpu().numpy()
        args = (case.q_gain.cpu().numpy(), case.k_gain.cpu().numpy(), case.cos.cpu().numpy(), case.sin.cpu().numpy())

        def call():
            c = G.PagedCache(host.pages.shape[0], cfg.hkv)
            c.pages[...] = host.pages
            qr = G.append(c, qkv, p, np.arange(cfg.batch), *args, cfg.hq, cfg.hkv, None, case.cache.max_blocks)
            G.decode_attention(qr, c, None, case.cache.max_blocks, p + 1, cfg.window, cfg.hq, cfg.hkv,
                               1 / math.sqrt(128))

        from threadpoolctl import threadpool_limits

        with threadpool_limits(limits=1):
            med, times = cpu_timed(call, cpu_s)
        res["cpu_baseline"] = {"value": round(nbytes / med / 1e9, 4), "unit": "GB/s", "cores": 1, "kind": "port",
                               "sample": f"the whole config: oracle append (numpy) + decode attention (fp64), 1 "
                                         f"warm-up call, median of {len(times)} timed calls ({med * 1e3:.1f} ms)",
                               "call_ms": round(med * 1e3, 2), "host": host_info()}
    return res


def extra_prefill_cfg4(dev, stream, cpu_s: float | None = None) -> dict:
    """Config 4 (B 8, 16/4 heads, 3584 cached + 512-token chunk): the chunk's append, then prefill attention; the
    attention call timed alone (MFMA-bound: algorithmic flops over time against the dense bf16 peak); with cpu_s,
    the oracle's CPU leg on a bounded sample of the same rows."""
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
    res = {"workload": cfg.name, "attn_us": round(ms * 1e3, 3), "append_us": round(append_ms * 1e3, 3),
           "flops": flops, "TFLOP_s": round(tfs, 1), "bound": "mfma", "peak_TFLOP_s": MFMA_PEAK_TFS,
           "frac_of_mfma_peak": round(tfs / MFMA_PEAK_TFS, 4)}
    if cpu_s:
        res["cpu_baseline"] = cpu_prefill(case, q, cpu_s, tfs)
    return res


def extra_e2e_cfg5(dev, steps: int | None = None, cpu_s: float | None = None) -> dict:
    """Config 5: random-init 26-layer d1664 model, 128 random 2048-token prompts prefilled into the fp8 cache, then
    512 greedy decode steps replayed from one captured graph; tokens/s and the decode steps' algorithmic HBM bytes
    (bf16 weights once + 264 B per cached (token, head, layer)); with cpu_s, the oracle's CPU model on one sequence,
    extrapolated to the whole run."""
    import torch

    from nanochat_amd.decoder import CONFIG5, generate

    cfg = CONFIG5
    if steps is not None:
        from dataclasses import replace

        cfg = replace(cfg, steps=steps, name=cfg.name.replace(f"steps{cfg.steps}", f"steps{steps}"))
    toks, info, (model, dec, prompts) = generate(cfg, dev)
    del dec
    torch.cuda.empty_cache()
    m, B, steps = cfg.model, cfg.batch, cfg.steps
    kv = sum((cfg.prompt - 1 + i + 1) * B * m.kv_heads * 264 * m.layers for i in range(steps))
    step_bytes = (kv + steps * info["weight_bytes"]) / steps
    dec_s, pre_s = info["decode_ms"] * 1e-3, info["prefill_ms"] * 1e-3
    gbs = step_bytes / (dec_s / steps) / 1e9
    import hashlib

    res = {"workload": cfg.name, "prefill_s": round(pre_s, 4), "decode_s": round(dec_s, 4),
           "decode_ms_per_step": round(info["decode_ms_per_step"], 4),
           "decode_tokens_per_s": round(B * steps / dec_s, 1),
           "e2e_tokens_per_s": round(B * steps / (pre_s + dec_s), 1),
           "decode_step_bytes": int(step_bytes), "decode_GB_s": round(gbs, 1),
           "decode_frac_of_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
           "tokens_sha256": hashlib.sha256(toks.cpu().numpy().astype("<i4").tobytes()).hexdigest()[:16]}
    if cpu_s:
        res["cpu_baseline"] = cpu_e2e(model, prompts, cfg, 2 * cpu_s, res)
    return res


def extra_gemm_cfg5(dev, stream) -> dict:
    """Config 5's four decode-step GEMMs at M = 128 (qkv 4992x1664 NORM_STORE, o 1664x1664 RESID, up 6656x1664
    RELU2_NORM, down 1664x6656 RESID): nc_slot_gemm_bf16 against the library's torch.matmul(x, Wᵀ) (plain bf16
    product, no epilogue), each over LAYERS weight copies in turn so that every call reads its W cold, as the
    decode step does; graphs of LAYERS calls, HIP events on their stream."""
    import torch

    from nanochat_amd.decoder import CONFIG5
    from nanochat_amd.slot_gemm import NORM_STORE, RELU2_NORM, RESID, slot_gemm

    d, m, layers = CONFIG5.model.d_model, CONFIG5.batch, CONFIG5.model.layers
    g = torch.Generator(device=dev).manual_seed(5)
    shapes = (("qkv", 3 * d, d, NORM_STORE), ("o", d, d, RESID), ("up", 4 * d, d, RELU2_NORM),
              ("down", d, 4 * d, RESID))
    res = {"workload": "cfg5 decode GEMMs, M 128, bf16 W [n][k]", "weight_copies": layers}
    total = {"slot_gemm": 0.0, "torch_matmul": 0.0}
    for name, n, k, epi in shapes:
        ws = [torch.randn(n, k, generator=g, device=dev).mul_(k ** -0.5).to(torch.bfloat16) for _ in range(layers)]
        x = torch.randn(m, k, generator=g, device=dev).to(torch.bfloat16)
        r = torch.randn(m, n, generator=g, device=dev).to(torch.bfloat16)
        out = torch.empty(m, n, dtype=torch.bfloat16, device=dev)
        turn = [0, 0]

        def ours():
            w = ws[turn[0] % layers]
            turn[0] += 1
            slot_gemm(x, w, epi, res=r if epi == RESID else None, out=out)

        def lib():
            w = ws[turn[1] % layers]
            turn[1] += 1
            torch.matmul(x, w.t(), out=out)

        row = {"n": n, "k": k, "w_bytes": n * k * 2}
        for key, fn in (("slot_gemm", ours), ("torch_matmul", lib)):
            ms = time_calls(fn, layers, 20, stream)
            row[f"{key}_us"] = round(ms * 1e3, 3)
            row[f"{key}_GB_s"] = round(n * k * 2 / (ms * 1e-3) / 1e9, 1)
            total[key] += ms * 1e3
        res[name] = row
        del ws
        torch.cuda.empty_cache()
    res["per_layer_us"] = {key: round(v, 2) for key, v in total.items()}
    return res


def extra_e2e_cfg5_handle(dev, steps: int | None = None) -> dict:
    """Config 5 through the dec_* handle (csrc/decoder.hip, the reference's NativeDecoder protocol,
    inference/decoder.py:194-232): the model and prompts of e2e_cfg5; every prompt admitted (dec_set_prompt, greedy),
    prefilled by dec_prefill in dec_prefill_rows() rows per call, then `steps` steps of dec_launch_body +
    dec_launch_head + dec_tokens, the host waiting for each step's tokens as the reference's loop does. The tokens
    hash the same way as e2e_cfg5's."""
    import hashlib

    import torch

    from nanochat_amd.decoder import CONFIG5, RandomModel
    from nanochat_amd.native_decoder import NativeDecoder
    from nanochat_amd.sampling import slot_masks
    from nanochat_amd.serving import prompt_rows

    cfg = CONFIG5
    steps = cfg.steps if steps is None else steps
    B, P = cfg.batch, cfg.prompt
    model = RandomModel(cfg.model, dev, seed=cfg.seed)
    g = torch.Generator(device=dev).manual_seed(cfg.seed + 1)
    prompts = torch.randint(0, cfg.model.vocab, (B, P), generator=g, device=dev, dtype=torch.int64).to(torch.int32)
    ids = prompts.cpu().numpy()
    nd = NativeDecoder(model, bos=-1, max_length=P - 1 + steps, batch=B)
    lib, h = nd.lib, nd.handle
    for b in range(B):
        lib.dec_set_prompt(h, b, int(ids[b, -1]), P - 1, 0.0, 1.0, 0)
    rows = prompt_rows([(b, ids[b].tolist()) for b in range(B)])
    words = np.ascontiguousarray(slot_masks([True] * B))
    out = np.empty(2 * B, dtype=np.int32)
    toks = np.empty((steps, B), dtype=np.int32)
    nd.stream.synchronize()
    t0 = time.perf_counter()
    for lo in range(0, rows.shape[1], nd.rows_per_call):
        part = np.ascontiguousarray(rows[:, lo:lo + nd.rows_per_call])
        lib.dec_prefill(h, part.shape[1], part.ctypes.data)
    nd.stream.synchronize()
    t1 = time.perf_counter()
    lib.dec_set_active(h, words.ctypes.data)
    for i in range(steps):
        lib.dec_launch_body(h)
        lib.dec_launch_head(h)
        lib.dec_tokens(h, out.ctypes.data)
        toks[i] = out[:B]
    t2 = time.perf_counter()
    pre_s, dec_s = t1 - t0, t2 - t1
    res = {"workload": cfg.name.replace(f"steps{cfg.steps}", f"steps{steps}") + "-dec-handle",
           "prefill_calls": -(-rows.shape[1] // nd.rows_per_call), "prefill_s": round(pre_s, 4),
           "decode_s": round(dec_s, 4), "decode_ms_per_step": round(dec_s / steps * 1e3, 4),
           "decode_tokens_per_s": round(B * steps / dec_s, 1), "e2e_tokens_per_s": round(B * steps / (pre_s + dec_s), 1),
           "timing": "host wall clock (the handle's calls are host-synchronous per step, as the reference's loop)",
           "tokens_sha256": hashlib.sha256(np.ascontiguousarray(toks.T).astype("<i4").tobytes()).hexdigest()[:16]}
    del nd
    torch.cuda.empty_cache()
    return res


def torch_empty_like(t):
    import torch

    return torch.empty_like(t)


def host_info() -> dict:
    """The host the CPU legs run on: CPU model, the threads used, torch and numpy versions."""
    import torch

    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "threads": len(os.sched_getaffinity(0)), "torch": torch.__version__,
            "numpy": np.__version__}


def _q_bits(q) -> np.ndarray:
    import torch

    return q.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def _host_cache(cache):
    from oracle import golden as G

    host = G.PagedCache(cache.num_blocks, cache.hkv)
    host.pages[...] = cache.pages.cpu().numpy()
    table = cache.block_table.cpu().numpy() if cache.block_table is not None else None
    return host, table


CPU_CALLS = 5  # timed calls of every CPU leg after one warm-up call; the median is reported


def cpu_timed(call, budget_s: float) -> tuple[float, list[float]]:
    """One warm-up call, then CPU_CALLS timed calls (more while the budget lasts, up to 9); (median s, times)."""
    call()
    times, t_all = [], time.perf_counter()
    while len(times) < CPU_CALLS or (len(times) < 9 and time.perf_counter() - t_all < budget_s / 2):
        t0 = time.perf_counter()
        call()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), times


def cpu_sample(one_cost: float, n: int, budget_s: float) -> int:
    """How many of n equal units (one measured at one_cost s) fit a call of budget_s / (CPU_CALLS + 1)."""
    return int(max(1, min(n, (budget_s / (CPU_CALLS + 1)) // max(one_cost, 1e-9))))


def cpu_decode(case, final_ctx: np.ndarray, q, budget_s: float, gpu_gbs: float) -> dict:
    """The oracle's decode attention (numpy, fp64 over the dequantised cache) on the first sequences of the same
    cache (as many as let 1 warm-up + CPU_CALLS timed calls fit budget_s); the median call, in GB/s over the same
    algorithmic bytes as the GPU figure."""
    import math

    from threadpoolctl import threadpool_limits

    from nanochat_amd.workloads import decode_bytes
    from oracle import golden as G

    cores = len(os.sched_getaffinity(0))
    cache = case.cache
    host, table = _host_cache(cache)
    qb = _q_bits(q)
    cfg = case.cfg

    def call(n):
        G.decode_attention(qb[:n], host, table[:n] if table is not None else None, cache.max_blocks,
                           final_ctx[:n], cfg.window, cfg.hq, cfg.hkv, 1 / math.sqrt(128))

    with threadpool_limits(limits=cores):
        t0 = time.perf_counter()
        call(1)
        per_key = (time.perf_counter() - t0) / final_ctx[0]
        n, acc = 0, 0.0  # sequences whose keys fit one call's share of the budget
        while n < cfg.batch and (acc + final_ctx[n] * per_key <= budget_s / (CPU_CALLS + 1) or n == 0):
            acc += final_ctx[n] * per_key
            n += 1
        med, times = cpu_timed(lambda: call(n), budget_s)
    nbytes = decode_bytes(final_ctx[:n], cfg.hkv, cfg.window)
    value = nbytes / med / 1e9
    return {"value": round(value, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "sample": f"oracle decode attention (numpy fp64 over dequantised fp8) of the first {n} of {cfg.batch} "
                      f"sequences ({int(final_ctx[:n].sum())} keys x {cfg.hkv} kv heads) per call; 1 warm-up call, "
                      f"median of {len(times)} timed calls ({med:.2f} s, range {min(times):.2f}-{max(times):.2f} s)",
            "speedup_gpu_over_cpu": round(gpu_gbs / value, 1), "host": host_info()}


def cpu_prefill(case, q, budget_s: float, gpu_tfs: float) -> dict:
    """The oracle's prefill attention (numpy fp64 over the dequantised cache) on the chunk rows of the first
    sequences (as many as let 1 warm-up + CPU_CALLS timed calls fit budget_s); the median call, in TFLOP/s over the
    same algorithmic flops as the GPU figure."""
    import math

    from threadpoolctl import threadpool_limits

    from nanochat_amd.workloads import prefill_flops
    from oracle import golden as G

    cores = len(os.sched_getaffinity(0))
    cfg = case.cfg
    host, table = _host_cache(case.cache)
    qb = _q_bits(q)
    pos, seq = case.pos.cpu().numpy(), case.seq.cpu().numpy()

    def call(n):
        rows = np.nonzero(seq < n)[0]
        G.rows_attention(qb[rows], pos[rows], seq[rows], host, table, case.cache.max_blocks, cfg.batch,
                         cfg.window, cfg.hq, cfg.hkv, 1 / math.sqrt(128))
        return rows

    with threadpool_limits(limits=cores):
        t0 = time.perf_counter()
        call(1)
        n = cpu_sample(time.perf_counter() - t0, cfg.batch, budget_s)
        med, times = cpu_timed(lambda: call(n), budget_s)
    rows = np.nonzero(seq < n)[0]
    flops = prefill_flops(pos[rows], cfg.hq, cfg.window)
    value = flops / med / 1e12
    return {"value": round(value, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"oracle prefill attention (numpy fp64 over dequantised fp8) of the chunk rows of the first {n} "
                      f"of {cfg.batch} sequences ({flops:.3e} flop) per call; 1 warm-up call, median of {len(times)} "
                      f"timed calls ({med:.2f} s, range {min(times):.2f}-{max(times):.2f} s)",
            "speedup_gpu_over_cpu": round(gpu_tfs / value, 1), "host": host_info()}


def cpu_e2e(model, prompts, cfg, budget_s: float, gpu: dict) -> dict:
    """The oracle's CPU model (oracle/model.py: torch-CPU bf16 GEMMs, numpy append and fp64 attention) on one
    sequence of the same model and prompts: its prompt prefilled in 256-row chunks until done or 2/3 of budget_s,
    then 8 greedy decode steps at batch 1. The whole workload's time is extrapolated from it (labelled): every
    sequence one after another, prefill scaled by rows, 512 steps at the measured step time."""
    import torch

    from oracle.model import CpuModel

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    n_prompt, steps = cfg.prompt - 1, 8
    cpu = CpuModel(model, 1, cfg.prompt + steps + 1)
    ids = prompts[0].cpu().numpy().astype(np.int64)
    done, t0 = 0, time.perf_counter()
    while done < n_prompt and time.perf_counter() - t0 < budget_s * 2 / 3:
        n = min(256, n_prompt - done)
        cpu.prefill_rows(ids[done:done + n], np.arange(done, done + n), np.zeros(n, np.int64))
        done += n
    prefill_s = time.perf_counter() - t0
    tok = ids[n_prompt:n_prompt + 1] if done == n_prompt else ids[done:done + 1]
    times = []
    for i in range(steps + 1):  # step 0 is the warm-up
        t1 = time.perf_counter()
        tok = cpu.step(tok, done + i).argmax(1)
        if i:
            times.append(time.perf_counter() - t1)
    step_s = float(np.median(times))
    per_seq = prefill_s * n_prompt / done + cfg.steps * step_s
    total_s = cfg.batch * per_seq
    value = cfg.batch * cfg.steps / total_s
    return {"value": round(value, 3), "unit": "tokens/s", "cores": cores, "kind": "port", "extrapolated": True,
            "sample": f"oracle CPU model, sequence 0 only: {done} of its {n_prompt} prompt positions prefilled in "
                      f"{prefill_s:.1f} s (one pass), then 1 warm-up and {steps} timed greedy steps at batch 1 (median "
                      f"{step_s:.2f} s, range {min(times):.2f}-{max(times):.2f} s); the full run "
                      f"extrapolated as {cfg.batch} sequences one after another, prefill scaled to {n_prompt} rows "
                      f"and {cfg.steps} steps each: {total_s:.0f} s",
            "decode_tokens_per_s_batch1": round(1 / step_s, 3),
            "prefill_tokens_per_s": round(done / prefill_s, 2),
            "speedup_gpu_over_cpu": round(gpu["e2e_tokens_per_s"] / value, 1), "host": host_info()}


def main():
    args = parse()
    WARM_SECONDS[0] = args.warm_seconds
    if args.stats_summary:
        print(stats_summary(args.stats_summary))
        return
    if args.pmc_summary:
        print(json.dumps({"dirs": args.pmc_summary, "summary": pmc_summary(args.pmc_summary, args.kernels.split(";"),
                                                                            args.last)}, indent=1))
        return
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); the decode path shards by "
              "(sequence, kv head) with no exchange, so N GPUs would each run this step on their own share",
              file=sys.stderr)
        sys.exit(2)
    import torch

    from nanochat_amd.attention import decode_attention, decode_step, decode_workspace
    from nanochat_amd.workloads import CONFIG3, build_decode_case, decode_bytes

    dev = torch.device("cuda:0")
    if args.only:
        s = torch.cuda.Stream(dev)
        cpu_s = None if args.no_cpu else args.cpu_seconds
        run = {"decode1": lambda: extra_decode_cfg1(dev, s, cpu_s), "decode2": lambda: extra_decode_cfg2(dev, s, cpu_s),
               "prefill4": lambda: extra_prefill_cfg4(dev, s, cpu_s),
               "e2e5": lambda: extra_e2e_cfg5(dev, args.e2e_steps, cpu_s),
               "handle5": lambda: extra_e2e_cfg5_handle(dev, args.e2e_steps),
               "gemm5": lambda: extra_gemm_cfg5(dev, s), "sweep": lambda: extra_decode_sweep(dev, s)}[args.only]
        print(json.dumps(run()), flush=True)
        return
    cfg = CONFIG3
    steps, warmup = args.steps, args.warmup
    B = cfg.batch
    # POOLS layer pools at different addresses (the same seeded contents), stepped in turn: as in a model, where a
    # layer's cache is read again only after the other layers' caches, no step finds its pages in the 256 MB
    # memory-side cache (one pool is ~330 MB; two alternate with a whole pool read between two reads of each)
    per_pool = (steps + warmup + 3 * STEP_GROUP) // POOLS + 4
    cases = [build_decode_case(cfg, dev, steps=per_pool) for _ in range(POOLS)]
    case = cases[0]
    max_ctx = case.cache.capacity
    # each pool's positions ping-pong between two tensors: a step appends at pos and writes pos + 1 into the other
    # tensor, the pool's next positions (no position-advance kernel)
    pos = [[c.positions(0).contiguous(), torch.empty_like(c.positions(0))] for c in cases]
    qkv = case.qkv[0].contiguous()
    ws = decode_workspace(B, cfg.hq, cfg.hkv, max_ctx, dev)
    out = torch.empty((B, cfg.hq, 128), dtype=torch.bfloat16, device=dev)
    torch.cuda.synchronize()

    def fused(c, p_in, p_out):
        decode_step(qkv, c.cache, p_in, c.q_gain, c.k_gain, c.cos, c.sin, cfg.hq, max_ctx=max_ctx,
                    window=cfg.window, out=out, workspace=ws, pos_out=p_out)

    def unfused(c, p_in, p_out):
        q = c.cache.append(qkv, p_in, c.seq, c.q_gain, c.k_gain, c.cos, c.sin, cfg.hq, ctx_out=p_out)
        decode_attention(q, c.cache, p_out, max_ctx=max_ctx, window=cfg.window, out=out, workspace=ws)

    step = unfused if args.unfused else fused

    def phase_step(i: int) -> None:
        """Step i of the cycle of 2 POOLS: pool i % POOLS, its positions forward (0 -> 1) or back (1 -> 0)."""
        k, d = i % POOLS, (i // POOLS) % 2
        step(cases[k], pos[k][d], pos[k][1 - d])

    cycle = 2 * POOLS  # steps after which every pool's positions are back in their first tensor
    stream = torch.cuda.Stream(dev)
    # STEP_GROUP steps per graph, as a decoder captures a whole multi-layer step (the gap between two graph
    # replays is host launch latency, not kernel time); graph_c (one cycle) and the single steps take the rest
    graph_n, graph_c = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    singles = [torch.cuda.CUDAGraph() for _ in range(cycle)]
    with torch.cuda.stream(stream):
        # eager warm-up of every launch path before capture: one cycle, positions back in their first tensors
        for i in range(cycle):
            phase_step(i)
        stream.synchronize()
        with torch.cuda.graph(graph_n, stream=stream):
            for i in range(STEP_GROUP):
                phase_step(i)
        with torch.cuda.graph(graph_c, stream=stream):
            for i in range(cycle):
                phase_step(i)
        for i in range(cycle):
            with torch.cuda.graph(singles[i], stream=stream):
                phase_step(i)
    done = cycle

    def replay(n: int, at: int) -> int:
        """n steps from cycle phase `at` (graph_n whenever the phase is 0); returns the phase after them."""
        while n > 0:
            if at == 0 and n >= STEP_GROUP:
                graph_n.replay()
                n -= STEP_GROUP
            elif at == 0 and n >= cycle:
                graph_c.replay()
                n -= cycle
            else:
                singles[at].replay()
                at, n = (at + 1) % cycle, n - 1
        return at

    # settle the clocks: steps at each pool's current positions, their next positions going to scratch tensors,
    # append the same bytes the next step appends, so the pools and positions are unchanged
    warm_graph = torch.cuda.CUDAGraph()
    warm_next = [torch.empty_like(p[0]) for p in pos]
    with torch.cuda.stream(stream):
        with torch.cuda.graph(warm_graph, stream=stream):
            for i in range(STEP_GROUP):
                step(cases[i % POOLS], pos[i % POOLS][0], warm_next[i % POOLS])
        t_warm = time.perf_counter()
        while time.perf_counter() - t_warm < args.warm_seconds:
            for _ in range(10):
                warm_graph.replay()
            stream.synchronize()
    with torch.cuda.stream(stream):
        # warm-up: graph_n once (its first replay is not timed), then `warmup` steps, ending at phase 0
        graph_n.replay()
        w = warmup + (-warmup) % cycle
        replay(w, 0)
        done += STEP_GROUP + w
    stream.synchronize()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    with torch.cuda.stream(stream):
        e0.record(stream)
        replay(steps, 0)
        e1.record(stream)
    e1.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    wall = time.perf_counter() - t0
    torch.cuda.synchronize()
    # keys before the timed steps per pool (prior context + the tokens each pool appended); timed step i is step
    # i // POOLS of pool i % POOLS
    base = case.ctx + done // POOLS
    step_bytes = np.mean([decode_bytes(base + i // POOLS + 1, cfg.hkv, cfg.window) for i in range(steps)])
    value = step_bytes / (step_ms * 1e-3) / 1e9
    pool_steps = [(done + steps - k + POOLS - 1) // POOLS for k in range(POOLS)]  # steps each pool has taken
    ctx_len = [pos[k][pool_steps[k] % 2] for k in range(POOLS)]  # each pool's last context lengths: positions + 1
    final_ctx = [case.ctx + n for n in pool_steps]
    with torch.cuda.stream(stream):
        # each pool's last queries (attention alone, cpu_baseline); appending them again rewrites the same bytes
        qs = [c.cache.append(qkv, cl - 1, c.seq, c.q_gain, c.k_gain, c.cos, c.sin, cfg.hq)
              for c, cl in zip(cases, ctx_len)]
    q = qs[0]
    # the attention call alone (the metric's decode kernel + split-K merge, without the append): ATTN_REPS calls
    # in one graph, the pools in turn at their last contexts
    turn = [0]

    def attn_call():
        k = turn[0] % POOLS
        turn[0] += 1
        decode_attention(qs[k], cases[k].cache, ctx_len[k], max_ctx=max_ctx, window=cfg.window, out=out,
                         workspace=ws)

    attn_ms = time_calls(attn_call, STEP_GROUP, max(steps // STEP_GROUP, 2), stream)
    attn_bytes = np.mean([decode_bytes(final_ctx[r % POOLS], cfg.hkv, cfg.window) for r in range(POOLS)])
    attn_kernel = (f"nc_decode_attn_fp8 = k_decode<false> + k_merge, a graph of {STEP_GROUP} calls over {POOLS} "
                   "pools in turn at their last contexts, HIP events on their stream")
    if args.unfused:
        call_ms, call_bytes, call_kernel = attn_ms, attn_bytes, attn_kernel
    else:
        # the step is one nc_decode_step_fp8 call: the timed region is the roofline measurement itself
        call_ms, call_bytes = step_ms, step_bytes
        call_kernel = ("nc_decode_step_fp8 = k_decode<true> + k_merge, one call per timed step, HIP events on their "
                       f"stream, {POOLS} pools in turn")
    achieved = call_bytes / (call_ms * 1e-3) / 1e9
    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "warm_seconds": args.warm_seconds,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp8e4m3-kv/bf16+f16-mfma/fp32-softmax",
        "data": "synthetic",
        "config": {"workload": cfg.name, "batch": B, "hq": cfg.hq, "hkv": cfg.hkv, "head_dim": 128,
                   "ctx_prior": "U[512,8192] seed 3", "page": 16, "outliers": "1% at 8 sigma",
                   "pools": POOLS, "mean_keys_per_seq": round(float(np.mean(base + steps / (2 * POOLS) + 1)), 1),
                   "step": ("nc_kv_append_fp8 + nc_decode_attn_fp8" if args.unfused else
                            "nc_decode_step_fp8 (append fused into the attention kernel)") +
                           ": append 1 token/seq (qk-norm+rope+fp8 quantise, emitting the next positions) + split-K "
                           f"decode attention, one attention layer per step, {POOLS} layer pools stepped in turn "
                           f"(cold), graph replays of {STEP_GROUP} steps"},
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
                     "traffic_run_algorithmic_bytes": traffic_algorithmic(),
                     "kernel": call_kernel, "bytes_per_launch": int(call_bytes)},
    }
    cpu_s = None if args.no_cpu else args.cpu_seconds
    if not args.no_extra:
        result["decode_cfg1"] = extra_decode_cfg1(dev, stream, cpu_s)
        result["decode_cfg2"] = extra_decode_cfg2(dev, stream, cpu_s)
        result["prefill_cfg4"] = extra_prefill_cfg4(dev, stream, cpu_s)
        result["e2e_cfg5"] = extra_e2e_cfg5(dev, args.e2e_steps, cpu_s)
        hd = extra_e2e_cfg5_handle(dev, args.e2e_steps)
        hd["same_tokens_as_e2e_cfg5"] = hd["tokens_sha256"] == result["e2e_cfg5"]["tokens_sha256"]
        result["e2e_cfg5_handle"] = hd
    if args.copy_probe:
        copy_probe(dev)
    if cpu_s:
        result["cpu_baseline"] = cpu_decode(case, final_ctx[0], q, cpu_s, value)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
