"""The fp8 (OCP e4m3fn) KV cache: per-(token, kv head) absmax scales, 16-position pages, contiguous or paged.

The reference caches K and V in bf16, contiguous per slot ([slot][layer][max_len][C], model/kernels/decode.cu:726,
761-762) and appends them in k_prologue (decode.cu:550-565). This cache keeps fp8 codes plus one fp32 scale per
(token, kv head) for K and for V, in 16-position blocks; a block table maps each sequence's pages to blocks, and a
contiguous cache is the special case where sequence s owns blocks [s * max_blocks, (s + 1) * max_blocks).

Device layout (also nanochat_amd/csrc/layout.h): one pool `pages`, uint8 [num_blocks][Hkv][4224], and per
(block, kv head) tile
  K codes  bytes [0, 2048)      key t, dim d at K_BYTES[t][d]
  V codes  bytes [2048, 4096)   key t, dim d at V_BYTES[t][d] (quad-transposed: the 4 keys of a quad in one dword)
  k_scale  fp32 [16]            bytes [4096, 4160)
  v_scale  fp32 [16]            bytes [4160, 4224)
so that one page of one kv head is a single contiguous 4224-byte read. The codes lie in four 1 KiB parts of 64
16-byte fragments, lane f's MFMA fragment at part * 1024 + 16 f, so each load of a wave reads 1 KiB contiguous.
"""

from __future__ import annotations

import torch
from torch import Tensor

from nanochat_amd.native import check, hip_library, pointer, stream

PAGE = 16
HEAD_DIM = 128
TILE_BYTES = 4224
ROW_BYTES = 264  # one position of one kv head as a row: K codes, V codes, K scale, V scale


def _code_bytes() -> tuple[Tensor, Tensor]:
    t, d = torch.arange(PAGE)[:, None], torch.arange(HEAD_DIM)[None, :]
    k = (d // 16 % 2) * 1024 + (t + 16 * (d // 32)) * 16 + d % 16
    v = 2048 + (d // 4 % 2) * 1024 + (d // 8 + 16 * (t // 4)) * 16 + d % 4 * 4 + t % 4
    return k, v


K_BYTES, V_BYTES = _code_bytes()  # byte of key t, dim d within a tile, int64 [16][128] (CPU)


def _require(t: Tensor, name: str, dtype: torch.dtype, dim: int | None = None) -> None:
    if not isinstance(t, Tensor) or t.dtype != dtype or not t.is_cuda or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous {dtype} tensor on the GPU")
    if dim is not None and t.dim() != dim:
        raise ValueError(f"{name} must have {dim} dimensions, has {t.dim()}")


class Fp8KVCache:
    """One layer's cache. num_seqs sequences of at most max_blocks pages each."""

    def __init__(self, num_blocks: int, hkv: int, max_blocks: int, num_seqs: int, block_table: Tensor | None = None,
                 device: torch.device | str = "cuda"):
        if num_blocks <= 0 or hkv <= 0 or max_blocks <= 0 or num_seqs <= 0:
            raise ValueError("num_blocks, hkv, max_blocks and num_seqs must be positive")
        if block_table is None and num_seqs * max_blocks > num_blocks:
            raise ValueError(f"contiguous cache: {num_seqs} x {max_blocks} blocks exceed {num_blocks}")
        if block_table is not None:
            _require(block_table, "block_table", torch.int32, 2)
            if tuple(block_table.shape) != (num_seqs, max_blocks):
                raise ValueError(f"block_table {tuple(block_table.shape)} != ({num_seqs}, {max_blocks})")
        self.num_blocks, self.hkv, self.max_blocks, self.num_seqs = num_blocks, hkv, max_blocks, num_seqs
        self.block_table = block_table
        self.pages = torch.zeros((num_blocks, hkv, TILE_BYTES), dtype=torch.uint8, device=device)

    @property
    def k_scale(self) -> Tensor:
        """K scales, a view fp32 [num_blocks][hkv][16]."""
        return self.pages[..., 4096:4160].view(torch.float32)

    @property
    def v_scale(self) -> Tensor:
        """V scales, a view fp32 [num_blocks][hkv][16]."""
        return self.pages[..., 4160:4224].view(torch.float32)

    @classmethod
    def contiguous(cls, num_seqs: int, max_len: int, hkv: int, device: torch.device | str = "cuda") -> "Fp8KVCache":
        max_blocks = -(-max_len // PAGE)
        return cls(num_seqs * max_blocks, hkv, max_blocks, num_seqs, None, device)

    @classmethod
    def paged(cls, block_table: Tensor, num_blocks: int, hkv: int) -> "Fp8KVCache":
        return cls(num_blocks, hkv, block_table.shape[1], block_table.shape[0], block_table, block_table.device)

    @property
    def capacity(self) -> int:
        """Positions per sequence."""
        return self.max_blocks * PAGE

    def _cache_args(self):
        return (pointer(self.pages), pointer(self.block_table), self.max_blocks, self.num_blocks, self.num_seqs)

    def append(self, qkv: Tensor, pos: Tensor, seq: Tensor, q_gain: Tensor, k_gain: Tensor, cos: Tensor,
               sin: Tensor, hq: int, ctx_out: Tensor | None = None, q_out: Tensor | None = None) -> Tensor:
        """Fused append of n rows of the projection qkv bf16 [n][>= (hq + 2 hkv) 128] (q heads, k heads, v heads):
        q and k normed, gained and rotated at pos[n] (int32), k and v quantised into sequence seq[n]'s page.
        Returns q_out bf16 [n][hq][128]. Rows out of range write nothing and get a NaN q_out row. ctx_out (int32
        [n], another tensor than pos) receives pos + 1: the context lengths for the decode step that follows.
        q_out: where to write q (contiguous bf16 [n][hq][128]), a new tensor if None."""
        if qkv.dim() != 2 or qkv.dtype != torch.bfloat16 or not qkv.is_cuda or qkv.stride(1) != 1:
            raise ValueError("qkv must be a row-major bf16 [n][width] GPU tensor")
        n = qkv.shape[0]
        for t, name in ((pos, "pos"), (seq, "seq")):
            _require(t, name, torch.int32, 1)
            if t.shape[0] != n:
                raise ValueError(f"{name} has {t.shape[0]} rows, qkv {n}")
        for t, name in ((q_gain, "q_gain"), (k_gain, "k_gain"), (cos, "cos"), (sin, "sin")):
            _require(t, name, torch.float32)
        if ctx_out is not None:
            _require(ctx_out, "ctx_out", torch.int32, 1)
            if ctx_out.shape[0] != n:
                raise ValueError(f"ctx_out has {ctx_out.shape[0]} rows, qkv {n}")
        if q_out is None:
            q_out = torch.empty((n, hq, HEAD_DIM), dtype=torch.bfloat16, device=qkv.device)
        elif q_out.shape != (n, hq, HEAD_DIM) or q_out.dtype != torch.bfloat16 or not q_out.is_contiguous():
            raise ValueError(f"q_out must be contiguous bf16 [{n}][{hq}][{HEAD_DIM}]")
        lib = hip_library()
        check(lib.nc_kv_append_fp8(pointer(qkv), qkv.stride(0), n, pointer(pos), pointer(seq), pointer(q_gain),
                                   pointer(k_gain), pointer(cos), pointer(sin), cos.shape[0], hq, self.hkv,
                                   pointer(q_out), *self._cache_args(), pointer(ctx_out), stream()))
        return q_out

    def store(self, k: Tensor, v: Tensor, pos: Tensor, seq: Tensor) -> None:
        """Quantise final K/V rows bf16 [n][hkv * 128] (no norm or rotation) into the pages of (seq, pos)."""
        for t, name in ((k, "k"), (v, "v")):
            if t.dim() != 2 or t.dtype != torch.bfloat16 or not t.is_cuda or t.stride(1) != 1:
                raise ValueError(f"{name} must be a row-major bf16 [n][hkv * 128] GPU tensor")
        if k.shape != v.shape or k.stride(0) != v.stride(0) or k.shape[1] < self.hkv * HEAD_DIM:
            raise ValueError(f"k {tuple(k.shape)}, v {tuple(v.shape)} must match and hold {self.hkv} heads")
        n = k.shape[0]
        for t, name in ((pos, "pos"), (seq, "seq")):
            _require(t, name, torch.int32, 1)
            if t.shape[0] != n:
                raise ValueError(f"{name} has {t.shape[0]} rows, k {n}")
        check(hip_library().nc_kv_store_fp8(pointer(k), pointer(v), k.stride(0), n, pointer(pos), pointer(seq),
                                            self.hkv, *self._cache_args(), stream()))

    def gather(self, ctx_len: Tensor, max_ctx: int) -> tuple[Tensor, Tensor, Tensor, Tensor]:
        """The first ctx_len[b] positions of sequences b < len(ctx_len) in the canonical row-major layout:
        K, V codes uint8 [B][hkv][max_ctx][128], scales fp32 [B][hkv][max_ctx]; later positions zero."""
        _require(ctx_len, "ctx_len", torch.int32, 1)
        B = ctx_len.shape[0]
        if B > self.num_seqs:
            raise ValueError(f"{B} sequences, the cache holds {self.num_seqs}")
        dev = self.pages.device
        k = torch.empty((B, self.hkv, max_ctx, HEAD_DIM), dtype=torch.uint8, device=dev)
        v = torch.empty_like(k)
        ks = torch.empty((B, self.hkv, max_ctx), dtype=torch.float32, device=dev)
        vs = torch.empty_like(ks)
        args = self._cache_args()[:-1]  # gather's sequence count is B
        check(hip_library().nc_kv_gather_fp8(*args, pointer(ctx_len), B, self.hkv, max_ctx, pointer(k), pointer(v),
                                             pointer(ks), pointer(vs), stream()))
        return k, v, ks, vs

    def export_rows(self, seq: int, at: int, n: int, out: Tensor | None = None) -> Tensor:
        """Positions [at, at + n) of sequence seq (any at, any n) as rows uint8 [n][hkv][264]: K codes, V codes in
        dim order, K scale and V scale (fp32 bytes). A position whose block is missing gives a zero row."""
        if out is None:
            out = torch.empty((n, self.hkv, ROW_BYTES), dtype=torch.uint8, device=self.pages.device)
        elif out.shape != (n, self.hkv, ROW_BYTES) or out.dtype != torch.uint8 or not out.is_contiguous():
            raise ValueError(f"out must be contiguous uint8 [{n}][{self.hkv}][{ROW_BYTES}]")
        pages, table, mb, nb, ns = self._cache_args()
        check(hip_library().nc_kv_export_fp8(pages, 0, 1, table, mb, nb, ns, seq, at, n, self.hkv, pointer(out),
                                             stream()))
        return out

    def import_rows(self, rows: Tensor, seq: int, at: int) -> None:
        """export_rows' inverse: rows uint8 [n][hkv][264] into positions [at, at + n) of sequence seq; only those
        positions' bytes change."""
        _require(rows, "rows", torch.uint8, 3)
        if rows.shape[1:] != (self.hkv, ROW_BYTES):
            raise ValueError(f"rows {tuple(rows.shape)} must be [n][{self.hkv}][{ROW_BYTES}]")
        pages, table, mb, nb, ns = self._cache_args()
        check(hip_library().nc_kv_import_fp8(pointer(rows), 1, pages, 0, table, mb, nb, ns, seq, at, rows.shape[0],
                                             self.hkv, stream()))
