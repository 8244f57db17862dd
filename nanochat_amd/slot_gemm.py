"""The decode step's skinny weight GEMM (nc_slot_gemm_bf16): out[b] = epilogue(W x[b]) for the rows of a decode batch,
the reference's slot GEMM and its epilogues (model/kernels/decode.cu:107-123,169-184,292-338,848-877).

    slot_gemm(x, w)                        bf16(x Wᵀ)
    slot_gemm(x, w, NORM_STORE)            bf16(norm(x) Wᵀ) with the RMS norm folded in: (x Wᵀ) r, r per row of x
    slot_gemm(x, w, RESID, res=h, out=h)   h = bf16(h + x Wᵀ), one rounding, in place
    slot_gemm(x, w, RELU2_NORM)            bf16(relu(p) p), p = (x Wᵀ) r
    slot_gemm(x, w, NORM_F32)              fp32 (x Wᵀ) r: logits

r = 1 / sqrt(mean(x²) + FLT_EPSILON) over the row of x (model/modeling.py:47-49, the decoder's norms). Sums are fp32
in a fixed order, so results are deterministic.
"""

from __future__ import annotations

import torch
from torch import Tensor

from nanochat_amd.native import check, hip_library, pointer, stream

STORE, NORM_STORE, RESID, RELU2_NORM, NORM_F32 = range(5)


def slot_gemm(x: Tensor, w: Tensor, epi: int = STORE, *, res: Tensor | None = None, out: Tensor | None = None,
              tile: tuple[int, int] = (0, 0), prefetch: Tensor | None = None) -> Tensor:
    """x bf16 [m][k], w bf16 [n][k] (contiguous): the [m][n] result (bf16, fp32 for NORM_F32), into out if given.
    tile = (rows of w, rows of x) per work unit; (0, 0) picks one from the shape. prefetch: a contiguous GPU tensor
    (the next GEMM's weights) that the launch's idle compute units read into the memory-side cache
    (nc_slot_gemm_bf16_prefetch); the result is the same."""
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16 or x.dim() != 2 or w.dim() != 2:
        raise ValueError("slot_gemm takes bf16 x [m][k] and w [n][k]")
    if not (x.is_contiguous() and w.is_contiguous()):
        raise ValueError("slot_gemm needs contiguous x and w")
    m, k = x.shape
    n = w.shape[0]
    if w.shape[1] != k:
        raise ValueError(f"x {tuple(x.shape)} and w {tuple(w.shape)} disagree on k")
    dtype = torch.float32 if epi == NORM_F32 else torch.bfloat16
    if out is None:
        out = torch.empty((m, n), dtype=dtype, device=x.device)
    elif out.shape != (m, n) or out.dtype != dtype or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous {dtype} [{m}][{n}]")
    if epi == RESID:
        if res is None or res.shape != (m, n) or res.dtype != torch.bfloat16 or not res.is_contiguous():
            raise ValueError(f"RESID needs a contiguous bf16 res [{m}][{n}]")
    if prefetch is None:
        check(hip_library().nc_slot_gemm_bf16(pointer(w), n, k, pointer(x), m, epi, pointer(out), pointer(res),
                                              tile[0], tile[1], stream()))
        return out
    if not (prefetch.is_cuda and prefetch.is_contiguous()):
        raise ValueError("prefetch must be a contiguous GPU tensor")
    check(hip_library().nc_slot_gemm_bf16_prefetch(pointer(w), n, k, pointer(x), m, epi, pointer(out), pointer(res),
                                                   tile[0], tile[1], pointer(prefetch),
                                                   prefetch.numel() * prefetch.element_size(), stream()))
    return out
