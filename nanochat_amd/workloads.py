"""Seeded synthetic inputs of the benchmark configurations (random-init, no datasets or checkpoints).

Values are N(0, 1) drawn in fp32 from a seeded torch generator and rounded to bf16; "outliers" replace a seeded
fraction of elements by ±8 (8σ). A decode case is a cache already holding each sequence's prior context, plus the
next token's fused projection row per sequence; the step appends it and attends.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from nanochat_amd.kv_cache import HEAD_DIM, PAGE, Fp8KVCache
from nanochat_amd.rotary import rotary_tables


@dataclass(frozen=True)
class DecodeConfig:
    """One decode-attention configuration: batch, heads, each sequence's prior context (before the appended
    token), paging, outliers, RoPE base, seed."""
    name: str
    batch: int
    hq: int
    hkv: int
    ctx: tuple[int, ...] | None = None        # fixed prior context per sequence, or
    ctx_range: tuple[int, int] | None = None  # uniform [lo, hi] per sequence (seeded)
    paged: bool = False
    outliers: float = 0.0
    theta: float = 10000.0
    window: int = -1
    seed: int = 0

    def contexts(self) -> np.ndarray:
        if self.ctx is not None:
            c = np.array(self.ctx if len(self.ctx) == self.batch else self.ctx * self.batch, dtype=np.int64)
            return c[:self.batch]
        rng = np.random.default_rng(self.seed + 1)
        return rng.integers(self.ctx_range[0], self.ctx_range[1] + 1, size=self.batch).astype(np.int64)


# BASELINE.json configs 1-3 (decode). Config 1 is the reference fork's d24 head shape (6/6, θ = 1e6).
CONFIG1 = DecodeConfig("cfg1-plumbing-b1-h6-ctx1024", 1, 6, 6, ctx=(1024,), theta=1e6, seed=0)
CONFIG2 = DecodeConfig("cfg2-d20-b32-h10-ctx4096", 32, 10, 10, ctx=(4096,), seed=2)
CONFIG3 = DecodeConfig("cfg3-ragged-gqa-b64-h16/4-ctx512..8192-paged16", 64, 16, 4, ctx_range=(512, 8192),
                       paged=True, outliers=0.01, seed=3)


@dataclass(frozen=True)
class PrefillConfig:
    """One chunked-prefill configuration: every sequence holds `cached` tokens and appends a `chunk`-token chunk
    (QK-norm + RoPE + quantise), then the chunk's rows attend causally over the cache (its own keys included)."""
    name: str
    batch: int
    hq: int
    hkv: int
    cached: tuple[int, ...]
    chunk: tuple[int, ...]
    paged: bool = False
    outliers: float = 0.0
    theta: float = 10000.0
    window: int = -1
    seed: int = 0

    def per_seq(self, v: tuple[int, ...]) -> np.ndarray:
        return np.array(v if len(v) == self.batch else v * self.batch, dtype=np.int64)[:self.batch]


# 8 sequences append a 512-token chunk onto 3584 cached tokens, 16 / 4 heads, θ = 1e4.
CONFIG4 = PrefillConfig("cfg4-prefill-b8-h16/4-cache3584+chunk512", 8, 16, 4, cached=(3584,), chunk=(512,), seed=4)


def seeded_normal(shape, seed: int, device, outliers: float = 0.0) -> torch.Tensor:
    """N(0, 1) fp32 -> bf16 (RNE), with a seeded fraction of elements replaced by ±8."""
    g = torch.Generator(device=device).manual_seed(seed)
    x = torch.randn(shape, generator=g, device=device, dtype=torch.float32)
    if outliers > 0:
        hit = torch.rand(shape, generator=g, device=device) < outliers
        x = torch.where(hit, 8.0 * torch.where(x < 0, -1.0, 1.0), x)
    return x.to(torch.bfloat16)


def block_table_for(ctx_cap: np.ndarray, seed: int, device) -> tuple[torch.Tensor, int]:
    """A block table giving every sequence ceil(cap / 16) pages, all of them a random permutation of the pool;
    unused entries -1. Returns (table int32 [B][max_pages], num_blocks)."""
    pages = (ctx_cap + PAGE - 1) // PAGE
    total, max_pages = int(pages.sum()), int(pages.max())
    perm = torch.randperm(total, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    table = torch.full((len(ctx_cap), max_pages), -1, dtype=torch.int32)
    off = 0
    for b, n in enumerate(pages):
        table[b, :n] = perm[off:off + n]
        off += int(n)
    return table.to(device), total


@dataclass
class DecodeCase:
    cfg: DecodeConfig
    cache: Fp8KVCache
    ctx: np.ndarray                 # prior context per sequence (host)
    qkv: torch.Tensor               # [steps][B][(hq + 2 hkv) 128] bf16: the appended tokens' projections
    q_gain: torch.Tensor
    k_gain: torch.Tensor
    cos: torch.Tensor
    sin: torch.Tensor
    seq: torch.Tensor               # [B] int32
    extra: dict = field(default_factory=dict)

    def positions(self, step: int) -> torch.Tensor:
        """Positions of step `step`'s appended tokens: each sequence's prior context + step."""
        return torch.from_numpy((self.ctx + step).astype(np.int32)).to(self.seq.device)


def build_decode_case(cfg: DecodeConfig, device, steps: int = 1, fill: bool = True) -> DecodeCase:
    """The cache holding each sequence's prior context (K, V ~ N(0,1) bf16, quantised by nc_kv_store_fp8) and
    `steps` next-token projection rows per sequence."""
    ctx = cfg.contexts()
    cap = ctx + steps
    B, hkv, hq = cfg.batch, cfg.hkv, cfg.hq
    if cfg.paged:
        table, num_blocks = block_table_for(cap, cfg.seed + 7, device)
        cache = Fp8KVCache.paged(table, num_blocks, hkv)
    else:
        cache = Fp8KVCache.contiguous(B, int(cap.max()), hkv, device)
    if fill:
        # prior context in slabs of at most 2^20 rows (bounded temporaries)
        seq_all = np.repeat(np.arange(B), ctx)
        pos_all = np.concatenate([np.arange(c) for c in ctx]) if B else np.zeros(0, np.int64)
        slab = 1 << 20
        for i, s0 in enumerate(range(0, len(seq_all), slab)):
            s1 = min(s0 + slab, len(seq_all))
            k = seeded_normal((s1 - s0, hkv * HEAD_DIM), cfg.seed * 1000 + 2 * i, device, cfg.outliers)
            v = seeded_normal((s1 - s0, hkv * HEAD_DIM), cfg.seed * 1000 + 2 * i + 1, device, cfg.outliers)
            cache.store(k, v, torch.from_numpy(pos_all[s0:s1].astype(np.int32)).to(device),
                        torch.from_numpy(seq_all[s0:s1].astype(np.int32)).to(device))
    qkv = seeded_normal((steps, B, (hq + 2 * hkv) * HEAD_DIM), cfg.seed * 1000 + 999, device, cfg.outliers)
    g = torch.Generator().manual_seed(cfg.seed + 5)
    q_gain = (0.5 + torch.rand(HEAD_DIM, generator=g)).to(device)
    k_gain = (0.5 + torch.rand(HEAD_DIM, generator=g)).to(device)
    cos, sin = rotary_tables(int(cap.max()), cfg.theta, device)
    seq = torch.arange(B, dtype=torch.int32, device=device)
    return DecodeCase(cfg, cache, ctx, qkv, q_gain, k_gain, cos, sin, seq)


def decode_step(case: DecodeCase, step: int, max_ctx: int, out: torch.Tensor | None = None,
                workspace: torch.Tensor | None = None):
    """One decode step of the hot path: append every sequence's next token, then attend. Returns (q, out)."""
    from nanochat_amd.attention import decode_attention

    pos = case.positions(step)
    q = case.cache.append(case.qkv[step], pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, case.cfg.hq)
    ctx_len = pos + 1
    o = decode_attention(q, case.cache, ctx_len, max_ctx=max_ctx, window=case.cfg.window, out=out,
                         workspace=workspace)
    return q, o


@dataclass
class PrefillCase:
    cfg: PrefillConfig
    cache: Fp8KVCache
    cached: np.ndarray              # tokens already in the cache per sequence (host)
    chunk: np.ndarray               # chunk length per sequence (host)
    qkv: torch.Tensor               # [rows][(hq + 2 hkv) 128] bf16, the chunk rows sequence by sequence
    pos: torch.Tensor               # [rows] int32
    seq: torch.Tensor               # [rows] int32
    q_gain: torch.Tensor
    k_gain: torch.Tensor
    cos: torch.Tensor
    sin: torch.Tensor


def build_prefill_case(cfg: PrefillConfig, device) -> PrefillCase:
    """The cache holding each sequence's cached tokens and the chunk's projection rows, in sequence order."""
    cached, chunk = cfg.per_seq(cfg.cached), cfg.per_seq(cfg.chunk)
    dcfg = DecodeConfig(cfg.name, cfg.batch, cfg.hq, cfg.hkv, ctx=tuple(int(c) for c in cached), paged=cfg.paged,
                        outliers=cfg.outliers, theta=cfg.theta, window=cfg.window, seed=cfg.seed)
    cap = int((cached + chunk).max())
    base = build_decode_case(dcfg, device, steps=max(cap - int(cached.min()), 1))
    cache = base.cache
    rows = int(chunk.sum())
    qkv = seeded_normal((rows, (cfg.hq + 2 * cfg.hkv) * HEAD_DIM), cfg.seed * 1000 + 555, device, cfg.outliers)
    pos = np.concatenate([np.arange(c, c + k) for c, k in zip(cached, chunk)]).astype(np.int32)
    seq = np.repeat(np.arange(cfg.batch), chunk).astype(np.int32)
    cos, sin = rotary_tables(cap, cfg.theta, device)
    return PrefillCase(cfg, cache, cached, chunk, qkv, torch.from_numpy(pos).to(device),
                       torch.from_numpy(seq).to(device), base.q_gain, base.k_gain, cos, sin)


def prefill_step(case: PrefillCase, out: torch.Tensor | None = None):
    """Append the whole chunk, then every chunk row attends (the reference's order, decode.cu:859-863).
    Returns (q, out)."""
    from nanochat_amd.attention import prefill_attention

    q = case.cache.append(case.qkv, case.pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, case.cfg.hq)
    o = prefill_attention(q, case.cache, case.pos, case.seq, window=case.cfg.window, out=out)
    return q, o


def prefill_flops(pos: np.ndarray, hq: int, window: int = -1) -> int:
    """Algorithmic flops of prefill attention: per (row, query head, attended key) 2 * 128 for QK and 2 * 128
    for PV."""
    keys = pos + 1 if window < 0 else np.minimum(pos + 1, window + 1)
    return int(keys.sum()) * hq * 4 * HEAD_DIM


def decode_bytes(ctx_len: np.ndarray, hkv: int, window: int = -1) -> int:
    """Algorithmic HBM bytes of one decode-attention step: 264 B per attended (token, kv head)
    (128 B K + 128 B V codes + 2 fp32 scales)."""
    keys = ctx_len if window < 0 else np.minimum(ctx_len, window + 1)
    return int(keys.sum()) * hkv * (2 * HEAD_DIM + 8)
