"""Rotary tables (reference: CausalLM.init_buffers, model/modeling.py:169-176; rotary,
inference/modeling_nanochat.py:29-34): cos/sin[t][i] = fp32(cos/sin(t θ^(-2i/128))), angles in fp64 and rounded
once, i in [0, 64). θ is a parameter: 1e6 in the reference fork (model/config.py:9), 10000 in upstream nanochat."""

from __future__ import annotations

import torch

HEAD_DIM = 128


def rotary_tables(n: int, theta: float, device: torch.device | str | None = None) -> tuple[torch.Tensor, torch.Tensor]:
    """cos, sin: fp32 [n][64], contiguous."""
    exponent = torch.arange(0, HEAD_DIM, 2, dtype=torch.float64, device=device) / HEAD_DIM
    t = torch.arange(n, dtype=torch.float64, device=device)
    freqs = torch.outer(t, theta ** -exponent)
    return freqs.cos().float().contiguous(), freqs.sin().float().contiguous()
