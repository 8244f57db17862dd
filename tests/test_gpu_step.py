"""GPU parity of the fused decode step (nc_decode_step_fp8): the same cache bytes and bit-identical output as the
append followed by decode attention, within the benchmark tolerance of the fp64 oracle, and its edge rows."""

import math

import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits, oracle_cache, table
from nanochat_amd.attention import decode_attention
from nanochat_amd.attention import decode_step as fused_step
from nanochat_amd.kv_cache import Fp8KVCache
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.workloads import (CONFIG1, CONFIG2, CONFIG3, DecodeConfig, block_table_for, build_decode_case,
                                    decode_step, seeded_normal)
from oracle import golden as G

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)

CASES = [
    CONFIG1,
    CONFIG2,
    CONFIG3,
    DecodeConfig("window512-gqa", 8, 16, 4, ctx_range=(100, 3000), paged=True, window=512, seed=71),
    DecodeConfig("window-not-page-aligned", 4, 8, 2, ctx=(1000, 37, 16, 515), window=100, seed=72),
    DecodeConfig("g16-one-kv-head-first-token", 3, 16, 1, ctx=(0, 31, 2047), paged=True, seed=73),
    DecodeConfig("g5-page-multiples", 6, 10, 2, ctx=(15, 16, 31, 32, 63, 64), seed=74),
    DecodeConfig("long-single-seq-many-pieces", 1, 4, 1, ctx=(30000,), paged=True, outliers=0.01, seed=75),
]


@pytest.mark.parametrize("cfg", CASES, ids=[c.name for c in CASES])
def test_step_equals_append_then_decode(gpu, cfg):
    print(f"fused step case {cfg.name}", flush=True)
    case = build_decode_case(cfg, gpu, steps=1)
    max_ctx = int(case.ctx.max()) + 1
    before = case.cache.pages.clone()
    q, want = decode_step(case, 0, max_ctx)  # nc_kv_append_fp8, then nc_decode_attn_fp8
    two_kernel_pages = case.cache.pages.clone()
    case.cache.pages.copy_(before)
    got = fused_step(case.qkv[0], case.cache, case.positions(0), case.q_gain, case.k_gain, case.cos, case.sin,
                     cfg.hq, max_ctx=max_ctx, window=cfg.window)
    torch.cuda.synchronize()
    assert torch.equal(case.cache.pages, two_kernel_pages), "cache bytes differ from the two-kernel path"
    np.testing.assert_array_equal(bits(got), bits(want))
    ref = oracle_cache(case.cache)
    expect = G.decode_attention(bits(q), ref, table(case.cache), case.cache.max_blocks, case.ctx + 1, cfg.window,
                                cfg.hq, cfg.hkv, SCALE)
    assert_attention_close(got, expect, cfg.name)


def _edge_setup(dev, hq=8, hkv=2, cap=64, rope=64):
    tbl, nb = block_table_for(np.full(6, cap), 81, dev)
    cache = Fp8KVCache.paged(tbl, nb + 2, hkv)
    g = torch.Generator().manual_seed(82)
    cache.pages.copy_(torch.randint(0, 0x7E, cache.pages.shape, generator=g, dtype=torch.uint8))
    for t in (cache.k_scale, cache.v_scale):
        t.copy_(torch.rand(t.shape, generator=g) * 0.01)
    qkv = seeded_normal((6, (hq + 2 * hkv) * 128), 83, dev)
    gains = (0.5 + torch.rand(2, 128, generator=g)).to(dev)
    cos, sin = rotary_tables(rope, 1e4, dev)
    return cache, qkv, gains[0].contiguous(), gains[1].contiguous(), cos, sin


def test_step_edge_rows(gpu):
    """pos < 0: zero row; pos >= rope_len: NaN row; neither writes the cache. A page with no block (a hole in the
    table) writes nothing and is masked. Valid rows stay bit-identical to the two-kernel path."""
    dev = gpu
    hq, hkv = 8, 2
    cache, qkv, qg, kg, cos, sin = _edge_setup(dev, hq, hkv)
    cache.block_table[3, 2] = -1
    pos = torch.tensor([-1, 70, 20, 40, 5, 63], dtype=torch.int32, device=dev)
    before = cache.pages.clone()
    q = cache.append(qkv, pos, torch.arange(6, dtype=torch.int32, device=dev), qg, kg, cos, sin, hq)
    ctx = pos + 1
    ctx[1] = 0  # the fused step schedules no work for the NaN row: the same split, so identical valid rows
    want = decode_attention(q, cache, ctx, max_ctx=64)
    two_kernel_pages = cache.pages.clone()
    cache.pages.copy_(before)
    got = fused_step(qkv, cache, pos, qg, kg, cos, sin, hq, max_ctx=64)
    torch.cuda.synchronize()
    assert torch.equal(cache.pages, two_kernel_pages)
    gb = bits(got)
    assert (gb[0] == 0).all()
    assert np.isnan(G.bf16_to_f32(gb[1])).all()
    np.testing.assert_array_equal(gb[2:], bits(want)[2:])


def test_step_position_past_max_ctx_writes_nothing(gpu):
    """A position inside the rotary table but at or past max_ctx: NaN row, cache untouched (the two-kernel path
    would append it and attend only the first max_ctx keys)."""
    dev = gpu
    hq, hkv = 8, 2
    cache, qkv, qg, kg, cos, sin = _edge_setup(dev, hq, hkv)
    pos = torch.tensor([49, 50, 55, 10, 0, 48], dtype=torch.int32, device=dev)
    before = cache.pages.clone()
    got = fused_step(qkv, cache, pos, qg, kg, cos, sin, hq, max_ctx=50)
    torch.cuda.synchronize()
    changed = (cache.pages != before).any(dim=-1).nonzero().cpu().numpy()
    tbl = cache.block_table.cpu().numpy()
    written = {(int(tbl[s, p // 16]), h) for s, p in [(0, 49), (3, 10), (4, 0), (5, 48)] for h in range(hkv)}
    assert {(int(b), int(h)) for b, h in changed} <= written
    gb = bits(got)
    for r in (1, 2):
        assert np.isnan(G.bf16_to_f32(gb[r])).all(), r
    for r in (0, 3, 4, 5):
        assert not np.isnan(G.bf16_to_f32(gb[r])).any(), r


def test_step_repeated_steps_match(gpu):
    """Eight steps in a row through the fused call and through the two-kernel path: same cache, same outputs."""
    cfg = DecodeConfig("ragged-steps", 8, 16, 4, ctx_range=(1, 600), paged=True, seed=91)
    a = build_decode_case(cfg, gpu, steps=8)
    b = build_decode_case(cfg, gpu, steps=8)
    max_ctx = int(a.ctx.max()) + 8
    for s in range(8):
        _, want = decode_step(a, s, max_ctx)
        got = fused_step(b.qkv[s], b.cache, b.positions(s), b.q_gain, b.k_gain, b.cos, b.sin, cfg.hq,
                         max_ctx=max_ctx)
        np.testing.assert_array_equal(bits(got), bits(want), err_msg=f"step {s}")
    assert torch.equal(a.cache.pages, b.cache.pages)
