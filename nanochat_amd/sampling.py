"""The decode step's token choice (nc_choose_tokens): greedy, temperature (Gumbel-max), nucleus and masked slots,
with the commit, as the reference's CHOICE ARGMAX epilogue, k_nucleus and k_commit
(model/kernels/decode.cu:98-105,170-230,360-404,676-689) under inference/decoder.py:28-40's rules:
temperature 0 is the argmax (ties to the lowest id); > 0 a sample of softmax(logits / temperature) drawn from
(seed, generated position) alone; top_p < 1 nucleus sampling; a masked slot chooses among its allowed tokens.
"""

from __future__ import annotations

import numpy as np
import torch
from torch import Tensor

from nanochat_amd.native import check, hip_library, pointer, stream

SOFTCAP = 15.0  # the reference's final logit cap (model/modeling.py:23), applied to sampled logits only


def slot_masks(active, masked=None) -> np.ndarray:
    """Host words [2][ceil(B / 64)] (uint64 viewed as int64 for torch): the active slots' bits, then the masked
    slots'; slot b at bit b % 64 of word b // 64 (dec_set_active's layout, decode.cu:1080-1084)."""
    active = np.asarray(active, dtype=bool)
    masked = np.zeros_like(active) if masked is None else np.asarray(masked, dtype=bool)
    words = (len(active) + 63) // 64
    out = np.zeros((2, words * 64), dtype=bool)
    out[0, :len(active)] = active
    out[1, :len(masked)] = masked
    return np.packbits(out.reshape(2, words, 64), axis=-1, bitorder="little").view("<u8").reshape(2, words).view(
        np.int64)


def allow_rows(allowed) -> np.ndarray:
    """Bool [B][vocab] -> int32 words [B][ceil(vocab / 32)], bit t % 32 of word t // 32 (inference/decoder.py:69-70)."""
    allowed = np.asarray(allowed, dtype=bool)
    B, V = allowed.shape
    pad = np.zeros((B, -(-V // 32) * 32), dtype=bool)
    pad[:, :V] = allowed
    return np.packbits(pad, axis=-1, bitorder="little").view("<u4").view(np.int32)


def choose_workspace(batch: int, vocab: int, device) -> Tensor:
    n = int(hip_library().nc_choose_workspace_bytes(batch, vocab))
    return torch.empty(max(n, 1), dtype=torch.uint8, device=device)


def _req(t: Tensor | None, name: str, dtype: torch.dtype, n: int | None = None) -> None:
    if t is None:
        return
    if not isinstance(t, Tensor) or t.dtype != dtype or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} GPU tensor")
    if n is not None and t.shape[0] != n:
        raise ValueError(f"{name} has {t.shape[0]} rows, expected {n}")


def choose_tokens(logits: Tensor, vocab: int, pos: Tensor, *, temperature: Tensor | None = None,
                  top_p: Tensor | None = None, seed: Tensor | None = None, first: Tensor | None = None,
                  slots: Tensor | None = None, allow: Tensor | None = None, softcap: float = SOFTCAP, lazy: int = -1,
                  tokens: Tensor | None = None, alt_tokens: Tensor | None = None,
                  workspace: Tensor | None = None) -> tuple[Tensor, Tensor]:
    """logits fp32 [B][>= vocab] (row stride free, columns contiguous); pos int32 [B] (advanced by one for every
    active slot); per slot temperature / top_p fp32, seed int64 (the uint64 bits), first int32; slots int64
    [2][ceil(B / 64)] (slot_masks; None: all active, none masked); allow int32 [B][ceil(vocab / 32)] (allow_rows).
    Returns (tokens, alt_tokens) int32 [B]."""
    if logits.dim() != 2 or logits.dtype != torch.float32 or not logits.is_cuda or logits.stride(1) != 1:
        raise ValueError("logits must be a row-major fp32 [B][cols] GPU tensor")
    B = logits.shape[0]
    if not 0 < vocab <= logits.shape[1]:
        raise ValueError(f"vocab {vocab} outside [1, {logits.shape[1]}]")
    _req(pos, "pos", torch.int32, B)
    _req(temperature, "temperature", torch.float32, B)
    _req(top_p, "top_p", torch.float32, B)
    _req(seed, "seed", torch.int64, B)
    _req(first, "first", torch.int32, B)
    _req(slots, "slots", torch.int64)
    _req(allow, "allow", torch.int32, B)
    if slots is not None and tuple(slots.shape) != (2, (B + 63) // 64):
        raise ValueError(f"slots must be [2][{(B + 63) // 64}]")
    if allow is not None and allow.shape[1] != (vocab + 31) // 32:
        raise ValueError(f"allow must be [{B}][{(vocab + 31) // 32}]")
    if tokens is None:
        tokens = torch.empty(B, dtype=torch.int32, device=logits.device)
    if alt_tokens is None:
        alt_tokens = torch.empty(B, dtype=torch.int32, device=logits.device)
    _req(tokens, "tokens", torch.int32, B)
    _req(alt_tokens, "alt_tokens", torch.int32, B)
    if workspace is None:
        workspace = choose_workspace(B, vocab, logits.device)
    check(hip_library().nc_choose_tokens(
        pointer(logits), B, vocab, logits.stride(0), pointer(slots), pointer(allow), pointer(temperature),
        pointer(top_p), pointer(seed), pointer(first), pointer(pos), float(softcap), lazy, pointer(tokens),
        pointer(alt_tokens), pointer(workspace), workspace.numel() * workspace.element_size(), stream()))
    return tokens, alt_tokens
