"""How often greedy tokens differ between the reference's two roundings of one model (TEST INFRASTRUCTURE ONLY, see
oracle/__init__.py: it runs the oracle's two CPU variants and nothing of the product): the torch path's
(inference/modeling_nanochat.py, oracle.model.CpuModel, which this build's decoder follows) and the CUDA engine's
(model/kernels/decode.cu, oracle.model.EngineCpuModel: fp32 x0, the unrounded mix under the qkv norm, the MLP's
rstd from the o-projection's fp32 sum).

Teacher-forced: after a shared random prompt, both variants are fed the torch path's greedy token at every step,
so every step compares two choices made from the same history. Per (step, sequence) it records whether the two
greedy tokens differ, the torch path's top-2 logit margin and the largest logit difference between the variants.

    python -m oracle.engine_rounding [--layers 26 --d-model 1664 --heads 13 --vocab 65536 --batch 8 --prompt 128
                                      --steps 64 --x0-lambda 0.1 --seed 5]
"""

from __future__ import annotations

import argparse
import json
import time

import numpy as np
import torch


def measure(layers: int, d_model: int, heads: int, vocab: int, batch: int, prompt: int, steps: int,
            x0_lambda: float, seed: int) -> dict:
    from nanochat_amd.decoder import ModelConfig, RandomModel
    from oracle.model import CpuModel, EngineCpuModel

    cfg = ModelConfig(layers=layers, d_model=d_model, heads=heads, vocab=vocab)
    model = RandomModel(cfg, "cpu", seed=seed)
    model.x0_lambdas.fill_(x0_lambda)
    rng = np.random.default_rng(seed)
    prompts = rng.integers(0, vocab, (batch, prompt)).astype(np.int64)
    torch_path, engine = CpuModel(model, batch, prompt + steps), EngineCpuModel(model, batch, prompt + steps)
    t0 = time.perf_counter()
    for m in (torch_path, engine):
        m.prefill(prompts)
    tok, flips, margins, deltas, flip_margins = prompts[:, -1], 0, [], [], []
    for s in range(steps):
        a = torch_path.step(tok, prompt - 1 + s)
        b = engine.step(tok, prompt - 1 + s)
        top2 = np.sort(a, axis=1)[:, -2:]
        margin = top2[:, 1] - top2[:, 0]
        delta = np.abs(a - b).max(axis=1)
        diff = a.argmax(1) != b.argmax(1)
        flips += int(diff.sum())
        flip_margins += margin[diff].tolist()
        margins += margin.tolist()
        deltas += delta.tolist()
        tok = a.argmax(1)
    margins, deltas = np.array(margins), np.array(deltas)
    return {"model": f"l{layers}-d{d_model}-h{heads}-v{vocab}", "random_init_std": 0.02, "x0_lambda": x0_lambda,
            "batch": batch, "prompt": prompt, "steps": steps, "tokens": int(margins.size), "flips": flips,
            "flip_rate": flips / margins.size, "flip_margins": sorted(flip_margins),
            "median_top2_margin": float(np.median(margins)), "median_max_logit_delta": float(np.median(deltas)),
            "max_logit_delta": float(deltas.max()),
            "steps_with_margin_below_max_delta": int((margins < deltas).sum()),
            "cpu_seconds": round(time.perf_counter() - t0, 1)}


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--layers", type=int, default=26)
    ap.add_argument("--d-model", type=int, default=1664)
    ap.add_argument("--heads", type=int, default=13)
    ap.add_argument("--vocab", type=int, default=65536)
    ap.add_argument("--batch", type=int, default=8)
    ap.add_argument("--prompt", type=int, default=128)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--x0-lambda", type=float, default=0.1)
    ap.add_argument("--seed", type=int, default=5)
    a = ap.parse_args()
    print(json.dumps(measure(a.layers, a.d_model, a.heads, a.vocab, a.batch, a.prompt, a.steps, a.x0_lambda,
                             a.seed)))


if __name__ == "__main__":
    main()
