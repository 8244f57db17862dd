"""Fused q/k prologue: per-head RMS norm with an fp32 per-dim gain, then RoPE (rotation by -θ of the pairs
(i, i + 64)); fp32 math, one bf16 rounding per output. Drop-in for model/ops/qk_prologue.py:13-21 (`qk_forward`):
same arguments, same shapes, same call into a `qkp_forward` entry point with the same C signature
(model/kernels/qk_prologue.cu:111-118), here the HIP library's.

q, k: (B, T, H, 128) bf16 column blocks of the fused projection (token stride 3 H 128); gains (128,) fp32;
cos, sin: fp32 [T][64] (the position of token t of a sequence is t)."""

from __future__ import annotations

import ctypes

import torch
from torch import Tensor

from nanochat_amd.native import hip_library, pointer, stream


def qk_forward(q: Tensor, k: Tensor, q_norm_weight: Tensor, k_norm_weight: Tensor, cos: Tensor,
               sin: Tensor) -> tuple[Tensor, Tensor]:
    """(normed and rotated q, k), contiguous."""
    B, T, H, D = q.shape
    C = H * D
    if D != 128 or k.shape != q.shape:
        raise ValueError(f"q {tuple(q.shape)}, k {tuple(k.shape)}: (B, T, H, 128) each")
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16:
        raise ValueError("q and k must be bf16")
    want = (T * 3 * C, 3 * C, D, 1)
    if q.stride() != want or k.stride() != want or k.data_ptr() - q.data_ptr() != C * q.element_size():
        raise ValueError("q, k must be the first two column blocks of a contiguous (B, T, 3C) projection")
    for t, name in ((q_norm_weight, "q_norm_weight"), (k_norm_weight, "k_norm_weight")):
        if t.dtype != torch.float32 or t.shape != (D,) or not t.is_contiguous():
            raise ValueError(f"{name} must be fp32 (128,) contiguous")
    for t, name in ((cos, "cos"), (sin, "sin")):
        if t.dtype != torch.float32 or t.dim() != 2 or t.shape[0] < T or t.shape[1] != 64 or not t.is_contiguous():
            raise ValueError(f"{name} must be fp32 [>= T][64] contiguous")
    q_out, k_out = q.new_empty(q.shape), k.new_empty(k.shape)
    hip_library().qkp_forward(pointer(q), pointer(k), pointer(q_norm_weight), pointer(k_norm_weight), pointer(q_out),
                              pointer(k_out), pointer(cos), pointer(sin), ctypes.c_longlong(B * T * H), H, T,
                              stream())
    return q_out, k_out
