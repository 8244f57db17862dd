"""Attention over the fp8 cache: single-token decode (split-K flash-decode) and chunked prefill.

decode_attention replaces the reference's k_attn (model/kernels/decode.cu:567-675): query b sits at position
ctx_len[b] - 1 and attends the keys [max(p - window, 0), p] of its sequence in the cache (its own key appended
first), query head h reading kv head h // (Hq / Hkv). Softmax in fp32, output bf16.

prefill_attention replaces dec_prefill's rows (model/kernels/decode.cu:1039-1051, each row a k_attn block): row r
at position pos[r] of sequence seq[r] attends keys [max(pos - window, 0), pos] after the whole chunk was appended
(decode.cu:859-863), on MFMA tiles that share every fp8 page among the rows and heads of a kv head.
"""

from __future__ import annotations

import math

import torch
from torch import Tensor

from nanochat_amd.kv_cache import HEAD_DIM, Fp8KVCache, _require
from nanochat_amd.native import check, hip_library, pointer, stream


def decode_workspace_bytes(batch: int, hq: int, hkv: int, max_ctx: int) -> int:
    return int(hip_library().nc_decode_workspace_bytes(batch, hq, hkv, max_ctx))


def decode_workspace(batch: int, hq: int, hkv: int, max_ctx: int, device) -> Tensor:
    """A workspace for decode_attention: partial results between its two kernels. Calls in one stream (and graph
    replays) may share it; calls that may overlap on two streams need one each."""
    return torch.zeros(max(decode_workspace_bytes(batch, hq, hkv, max_ctx), 1), dtype=torch.uint8, device=device)


def decode_attention(q: Tensor, cache: Fp8KVCache, ctx_len: Tensor, *, max_ctx: int, window: int = -1,
                     sm_scale: float | None = None, out: Tensor | None = None,
                     workspace: Tensor | None = None) -> Tensor:
    """q bf16 [B][Hq][128] (normed and rotated, e.g. Fp8KVCache.append's q_out); ctx_len int32 [B] on the GPU, each
    at most max_ctx (larger values are clamped to it); window: keys before the query, < 0 for all. workspace: from
    decode_workspace, allocated per call if None. Returns bf16 [B][Hq][128]."""
    _require(q, "q", torch.bfloat16, 3)
    B, hq, D = q.shape
    if D != HEAD_DIM:
        raise ValueError(f"head dim {D} != 128")
    _require(ctx_len, "ctx_len", torch.int32, 1)
    if ctx_len.shape[0] != B or B > cache.num_seqs:
        raise ValueError(f"ctx_len has {ctx_len.shape[0]} entries for batch {B} (cache holds {cache.num_seqs})")
    if not 0 < max_ctx <= cache.capacity:
        raise ValueError(f"max_ctx {max_ctx} outside [1, {cache.capacity}]")
    scale = 1.0 / math.sqrt(HEAD_DIM) if sm_scale is None else float(sm_scale)
    if out is None:
        out = torch.empty_like(q)
    else:
        _require(out, "out", torch.bfloat16, 3)
        if out.shape != q.shape:
            raise ValueError("out must have q's shape")
    need = decode_workspace_bytes(B, hq, cache.hkv, max_ctx)
    if workspace is None:
        workspace = decode_workspace(B, hq, cache.hkv, max_ctx, q.device)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace of {workspace.numel() * workspace.element_size()} bytes, {need} needed")
    lib = hip_library()
    check(lib.nc_decode_attn_fp8(pointer(q), pointer(cache.pages), pointer(cache.block_table), cache.max_blocks,
                                 cache.num_blocks, pointer(ctx_len), window, B, hq, cache.hkv, max_ctx, scale,
                                 pointer(out), pointer(workspace), workspace.numel() * workspace.element_size(),
                                 stream()))
    return out


def decode_step(qkv: Tensor, cache: Fp8KVCache, pos: Tensor, q_gain: Tensor, k_gain: Tensor, cos: Tensor,
                sin: Tensor, hq: int, *, max_ctx: int, window: int = -1, sm_scale: float | None = None,
                out: Tensor | None = None, workspace: Tensor | None = None, pos_out: Tensor | None = None,
                piece_pages: int = 0) -> Tensor:
    """Fp8KVCache.append (row b into sequence b at pos[b]) and decode_attention (ctx_len = pos + 1) in one call of
    two launches, with bit-identical cache bytes and output: the reference's decode-body append (decode.cu:550-565)
    and k_attn. qkv bf16 [B][>= (hq + 2 hkv) 128] row-major; pos int32 [B]. A row with pos < 0 gets a zero row, a
    row with pos at or past max_ctx or len(cos) a NaN row; neither writes the cache. pos_out (int32 [B], another
    tensor than pos) receives pos + 1. piece_pages > 0: the sequence-local piece plan (nc_decode_step_fp8_pieces),
    every sequence's output bits independent of the batch. Returns bf16 [B][hq][128]."""
    if qkv.dim() != 2 or qkv.dtype != torch.bfloat16 or not qkv.is_cuda or qkv.stride(1) != 1:
        raise ValueError("qkv must be a row-major bf16 [B][width] GPU tensor")
    B = qkv.shape[0]
    _require(pos, "pos", torch.int32, 1)
    if pos.shape[0] != B or B > cache.num_seqs:
        raise ValueError(f"pos has {pos.shape[0]} entries for batch {B} (cache holds {cache.num_seqs})")
    for t, name in ((q_gain, "q_gain"), (k_gain, "k_gain"), (cos, "cos"), (sin, "sin")):
        _require(t, name, torch.float32)
    if pos_out is not None:
        _require(pos_out, "pos_out", torch.int32, 1)
        if pos_out.shape[0] != B:
            raise ValueError(f"pos_out has {pos_out.shape[0]} entries for batch {B}")
    if not 0 < max_ctx <= cache.capacity:
        raise ValueError(f"max_ctx {max_ctx} outside [1, {cache.capacity}]")
    scale = 1.0 / math.sqrt(HEAD_DIM) if sm_scale is None else float(sm_scale)
    if out is None:
        out = torch.empty((B, hq, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
    else:
        _require(out, "out", torch.bfloat16, 3)
        if tuple(out.shape) != (B, hq, HEAD_DIM):
            raise ValueError(f"out must be [{B}][{hq}][{HEAD_DIM}]")
    need = decode_workspace_bytes(B, hq, cache.hkv, max_ctx)
    if workspace is None:
        workspace = decode_workspace(B, hq, cache.hkv, max_ctx, qkv.device)
    elif workspace.numel() * workspace.element_size() < need:
        raise ValueError(f"workspace of {workspace.numel() * workspace.element_size()} bytes, {need} needed")
    args = (pointer(qkv), qkv.stride(0), pointer(pos), pointer(pos_out), pointer(q_gain), pointer(k_gain), pointer(cos),
            pointer(sin), cos.shape[0], pointer(cache.pages), pointer(cache.block_table), cache.max_blocks,
            cache.num_blocks, window, B, hq, cache.hkv, max_ctx, scale)
    tail = (pointer(out), pointer(workspace), workspace.numel() * workspace.element_size(), stream())
    lib = hip_library()
    if piece_pages > 0:
        check(lib.nc_decode_step_fp8_pieces(*args, piece_pages, *tail))
    else:
        check(lib.nc_decode_step_fp8(*args, *tail))
    return out


def prefill_attention(q: Tensor, cache: Fp8KVCache, pos: Tensor, seq: Tensor, *, window: int = -1,
                      sm_scale: float | None = None, out: Tensor | None = None) -> Tensor:
    """q bf16 [n][Hq][128] (Fp8KVCache.append's q_out for the chunk); pos, seq int32 [n] on the GPU. The chunk's
    keys must already be in the cache. Rows with pos < 0 or seq outside the cache's sequences get zero rows; the
    heads of one kv head of a row whose q is not finite (the append's rows past the rotary table) get NaN rows.
    Fastest when each sequence's rows are consecutive. Returns bf16 [n][Hq][128]."""
    _require(q, "q", torch.bfloat16, 3)
    n, hq, D = q.shape
    if D != HEAD_DIM:
        raise ValueError(f"head dim {D} != 128")
    _require(pos, "pos", torch.int32, 1)
    _require(seq, "seq", torch.int32, 1)
    if pos.shape[0] != n or seq.shape[0] != n:
        raise ValueError(f"pos / seq have {pos.shape[0]} / {seq.shape[0]} entries for {n} rows")
    scale = 1.0 / math.sqrt(HEAD_DIM) if sm_scale is None else float(sm_scale)
    if out is None:
        out = torch.empty_like(q)
    else:
        _require(out, "out", torch.bfloat16, 3)
        if out.shape != q.shape:
            raise ValueError("out must have q's shape")
    lib = hip_library()
    check(lib.nc_prefill_attn_fp8(pointer(q), pointer(pos), pointer(seq), n, pointer(cache.pages),
                                  pointer(cache.block_table), cache.max_blocks, cache.num_blocks, cache.num_seqs,
                                  window, hq, cache.hkv, scale, pointer(out), stream()))
    return out
