"""GPU parity of the cache's write side and gather against the oracle: bit-exact q rows, cache bytes and scales."""

import numpy as np
import pytest
import torch

from helpers import assert_same_cache, bits, oracle_cache, table
from nanochat_amd.kv_cache import Fp8KVCache
from nanochat_amd.qk_prologue import qk_forward
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.workloads import block_table_for, seeded_normal
from oracle import golden as G

pytestmark = pytest.mark.gpu


def random_bytes(cache: Fp8KVCache, seed: int) -> None:
    """Fill the cache with seeded garbage so untouched bytes are checked to stay untouched."""
    g = torch.Generator().manual_seed(seed)
    cache.pages.copy_(torch.randint(0, 256, cache.pages.shape, generator=g, dtype=torch.uint8))
    for t in (cache.k_scale, cache.v_scale):
        t.copy_(torch.rand(t.shape, generator=g))


def make_cache(kind: str, n_seq: int, cap: int, hkv: int, dev, seed: int) -> Fp8KVCache:
    if kind == "contiguous":
        return Fp8KVCache.contiguous(n_seq, cap, hkv, dev)
    tbl, nb = block_table_for(np.full(n_seq, cap), seed, dev)
    return Fp8KVCache.paged(tbl, nb + 3, hkv)  # spare blocks nobody owns


APPEND_CASES = [
    # name, B sequences, rows per sequence, first position, hq, hkv, theta, layout
    ("cfg1-decode-b1-h6", 1, 1, 1024, 6, 6, 1e6, "contiguous"),
    ("cfg2-decode-b32-h10", 32, 1, 4096, 10, 10, 1e4, "contiguous"),
    ("cfg3-decode-b64-gqa", 64, 1, 700, 16, 4, 1e4, "paged"),
    ("cfg4-chunk-b8-512", 8, 512, 3584, 16, 4, 1e4, "paged"),
    ("page-edges", 3, 33, 0, 4, 2, 1e4, "paged"),
]


@pytest.mark.parametrize("name, B, rows, start, hq, hkv, theta, layout", APPEND_CASES)
def test_append_bit_exact(gpu, name, B, rows, start, hq, hkv, theta, layout):
    print(f"append case {name}", flush=True)
    dev = gpu
    cap = start + rows
    cache = make_cache(layout, B, cap, hkv, dev, seed=11)
    random_bytes(cache, 12)
    ref = oracle_cache(cache)
    n = B * rows
    qkv = seeded_normal((n, (hq + 2 * hkv) * 128), 13, dev, outliers=0.01)
    # zero heads: a zero k row (after norm it stays zero) and a zero v row give scale 0 and codes 0
    qkv[0, hq * 128:(hq + 1) * 128] = 0
    qkv[-1, (hq + hkv) * 128:(hq + hkv + 1) * 128] = 0
    pos = torch.from_numpy(np.tile(np.arange(start, start + rows), B).astype(np.int32)).to(dev)
    seq = torch.from_numpy(np.repeat(np.arange(B), rows).astype(np.int32)).to(dev)
    g = torch.Generator().manual_seed(14)
    q_gain, k_gain = (0.5 + torch.rand(128, generator=g)).to(dev), (0.5 + torch.rand(128, generator=g)).to(dev)
    cos, sin = rotary_tables(cap, theta, dev)
    q = cache.append(qkv, pos, seq, q_gain, k_gain, cos, sin, hq)
    torch.cuda.synchronize()
    q_ref = G.append(ref, bits(qkv), pos.cpu().numpy(), seq.cpu().numpy(), q_gain.cpu().numpy(),
                     k_gain.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy(), hq, hkv, table(cache),
                     cache.max_blocks)
    np.testing.assert_array_equal(bits(q), q_ref)
    assert_same_cache(cache, ref)


def test_append_rows_in_any_order(gpu):
    """Rows of two sequences in an order that keeps some position quads whole and in order (their V codes are
    written as dwords) and breaks others (reversed, split, or the partial last quad): the cache bytes are the
    oracle's either way."""
    dev = gpu
    hq, hkv, rows = 4, 2, 42
    cache = make_cache("paged", 2, 48, hkv, dev, seed=31)
    random_bytes(cache, 32)
    ref = oracle_cache(cache)
    order = np.arange(2 * rows)
    order[4:8], order[8:12] = np.arange(8, 12), np.arange(4, 8)  # two whole quads swapped
    order[12:16] = order[12:16][::-1]                             # a quad reversed
    order[20:30] = order[20:30][np.random.default_rng(3).permutation(10)]
    pos = torch.from_numpy(np.tile(np.arange(rows), 2)[order].astype(np.int32)).to(dev)
    seq = torch.from_numpy(np.repeat(np.arange(2), rows)[order].astype(np.int32)).to(dev)
    qkv = seeded_normal((2 * rows, (hq + 2 * hkv) * 128), 33, dev)
    g = torch.Generator().manual_seed(34)
    q_gain, k_gain = (0.5 + torch.rand(128, generator=g)).to(dev), (0.5 + torch.rand(128, generator=g)).to(dev)
    cos, sin = rotary_tables(48, 1e4, dev)
    q = cache.append(qkv, pos, seq, q_gain, k_gain, cos, sin, hq)
    torch.cuda.synchronize()
    q_ref = G.append(ref, bits(qkv), pos.cpu().numpy(), seq.cpu().numpy(), q_gain.cpu().numpy(),
                     k_gain.cpu().numpy(), cos.cpu().numpy(), sin.cpu().numpy(), hq, hkv, table(cache),
                     cache.max_blocks)
    np.testing.assert_array_equal(bits(q), q_ref)
    assert_same_cache(cache, ref)


def test_append_rows_out_of_range_write_nothing(gpu):
    dev = gpu
    hq, hkv = 4, 2
    cache = make_cache("paged", 2, 64, hkv, dev, seed=21)
    cache.block_table[1, 2] = -1  # a hole in the table
    random_bytes(cache, 22)
    before = oracle_cache(cache)
    cos, sin = rotary_tables(64, 1e4, dev)
    qkv = seeded_normal((5, (hq + 2 * hkv) * 128), 23, dev)
    # pos < 0, pos >= rope_len, seq >= num_seqs, a page with no block, and one valid row
    pos = torch.tensor([-1, 64, 3, 40, 5], dtype=torch.int32, device=dev)
    seq = torch.tensor([0, 0, 2, 1, 1], dtype=torch.int32, device=dev)
    ones = torch.ones(128, device=dev)
    ctx = torch.full_like(pos, -7)
    q = cache.append(qkv, pos, seq, ones, ones, cos, sin, hq, ctx_out=ctx)
    torch.cuda.synchronize()
    assert torch.isnan(q[:3].float()).all() and not torch.isnan(q[3:].float()).any()
    assert ctx.tolist() == (pos + 1).tolist()  # every row, in range or not, gets pos + 1
    G.append(before, bits(qkv[4:]), np.array([5]), np.array([1]), np.ones(128, np.float32),
             np.ones(128, np.float32), cos.cpu().numpy(), sin.cpu().numpy(), hq, hkv, table(cache),
             cache.max_blocks)
    assert_same_cache(cache, before)


@pytest.mark.parametrize("layout", ["contiguous", "paged"])
def test_store_bit_exact(gpu, layout):
    dev = gpu
    hkv, B, L = 4, 5, 77
    cache = make_cache(layout, B, 80, hkv, dev, seed=31)
    random_bytes(cache, 32)
    ref = oracle_cache(cache)
    n = B * L
    k = seeded_normal((n, hkv * 128), 33, dev, outliers=0.01)
    v = seeded_normal((n, hkv * 128), 34, dev, outliers=0.01)
    k[5] = 0
    v[7, :128] = 0
    pos = torch.from_numpy(np.tile(np.arange(L), B).astype(np.int32)).to(dev)
    seq = torch.from_numpy(np.repeat(np.arange(B), L).astype(np.int32)).to(dev)
    cache.store(k, v, pos, seq)
    torch.cuda.synchronize()
    kc, ks = G.quantize_rows(bits(k).reshape(n, hkv, 128))
    vc, vs = G.quantize_rows(bits(v).reshape(n, hkv, 128))
    blk = G.PagedCache.block_of(seq.cpu().numpy(), pos.cpu().numpy(), table(cache), cache.max_blocks)
    t = pos.cpu().numpy() % 16
    for h in range(hkv):
        ref.write(blk, h, t, kc[:, h], ks[:, h], vc[:, h], vs[:, h])
    assert_same_cache(cache, ref)


def test_store_scale_extremes_bit_exact(gpu):
    """Rows whose absmax puts the scale below the normal range (the per-value division path), just above it and
    near the top of the fp32 range (the reciprocal path, where every quotient must still be x / scale rounded
    once), and rows with exact ties of the e4m3 rounding: the codes and scales are the oracle's bit for bit."""
    dev = gpu
    hkv, B, L = 2, 2, 48
    cache = make_cache("paged", B, 48, hkv, dev, seed=41)
    random_bytes(cache, 42)
    ref = oracle_cache(cache)
    n = B * L
    g = torch.Generator(device=dev).manual_seed(43)
    base = torch.randn((n, hkv * 128), generator=g, device=dev)
    mags = torch.tensor([1e-39, 3e-38, 1e-37, 1.5e-36, 1.8e-36, 2.2e-36, 1e-30, 1.0, 3e20, 1e37, 5e37], device=dev)
    k = (base * mags[torch.arange(n, device=dev) % len(mags)][:, None]).to(torch.bfloat16)
    v = (base.flip(0) * mags.flip(0)[torch.arange(n, device=dev) % len(mags)][:, None]).to(torch.bfloat16)
    # ties: absmax 28 makes scale 1/16 exactly, and x / scale = 16 x lands on e4m3 midpoints (17 between 16 and 18,
    # 34 between 32 and 36, ..., 2^-10 and 3 2^-10 between subnormal steps), each rounded to the even neighbour
    mids = torch.tensor([28.0 * 16, 17, 19, 21, 23, 8.5, 9.5, 34, 38, 68, 76, 136, 152, 272, 304, 2 ** -10,
                         3 * 2 ** -10, 5 * 2 ** -10], device=dev) / 16
    row = mids[torch.arange(128, device=dev) % len(mids)] * (1 - 2 * (torch.arange(128, device=dev) % 2))
    row[0] = 28.0
    k[3, :128] = row.to(torch.bfloat16)
    v[4, 128:] = row.flip(0).to(torch.bfloat16)
    pos = torch.from_numpy(np.tile(np.arange(L), B).astype(np.int32)).to(dev)
    seq = torch.from_numpy(np.repeat(np.arange(B), L).astype(np.int32)).to(dev)
    cache.store(k, v, pos, seq)
    torch.cuda.synchronize()
    kc, ks = G.quantize_rows(bits(k).reshape(n, hkv, 128))
    vc, vs = G.quantize_rows(bits(v).reshape(n, hkv, 128))
    assert (ks[ks > 0] < 2.0 ** -126).any() and (vs > 1e34).any()  # both paths are exercised
    blk = G.PagedCache.block_of(seq.cpu().numpy(), pos.cpu().numpy(), table(cache), cache.max_blocks)
    t = pos.cpu().numpy() % 16
    for h in range(hkv):
        ref.write(blk, h, t, kc[:, h], ks[:, h], vc[:, h], vs[:, h])
    assert_same_cache(cache, ref)


def test_qkp_forward_bit_exact(gpu):
    """The training-layout prologue (model/ops/qk_prologue.py:13-21 surface) against the oracle's row math."""
    dev = gpu
    B, T, H = 2, 96, 6
    C = H * 128
    qkv = seeded_normal((B, T, 3 * C), 41, dev)
    q, k = qkv[..., :C].unflatten(-1, (H, 128)), qkv[..., C:2 * C].unflatten(-1, (H, 128))
    g = torch.Generator().manual_seed(42)
    gq, gk = (0.5 + torch.rand(128, generator=g)).to(dev), (0.5 + torch.rand(128, generator=g)).to(dev)
    cos, sin = rotary_tables(T, 1e6, dev)
    qo, ko = qk_forward(q, k, gq, gk, cos, sin)
    torch.cuda.synchronize()
    c, s = cos.cpu().numpy()[None, :, None, :], sin.cpu().numpy()[None, :, None, :]
    np.testing.assert_array_equal(bits(qo), G.qk_norm_rope(bits(q), gq.cpu().numpy(), c, s))
    np.testing.assert_array_equal(bits(ko), G.qk_norm_rope(bits(k), gk.cpu().numpy(), c, s))


@pytest.mark.parametrize("layout", ["contiguous", "paged"])
def test_gather_bit_exact(gpu, layout):
    dev = gpu
    hkv, B = 3, 4
    cache = make_cache(layout, B, 100, hkv, dev, seed=51)
    random_bytes(cache, 52)
    ctx = torch.tensor([100, 0, 17, 64], dtype=torch.int32, device=dev)
    k, v, ks, vs = cache.gather(ctx, 100)
    torch.cuda.synchronize()
    want = G.gather(oracle_cache(cache), table(cache), cache.max_blocks, ctx.cpu().numpy(), 100)
    for got, w in zip((k, v, ks, vs), want):
        np.testing.assert_array_equal(got.cpu().numpy(), w)


ROW_CASES = [
    # layout, hkv, sequence, at, n: unaligned starts and lengths, whole pages, a single position, none
    ("paged", 4, 2, 37, 50),
    ("contiguous", 13, 1, 0, 2047 % 64),
    ("paged", 2, 0, 16, 32),
    ("contiguous", 3, 3, 99, 1),
    ("paged", 1, 1, 5, 0),
]


@pytest.mark.parametrize("layout, hkv, s, at, n", ROW_CASES)
def test_position_rows_bit_exact(gpu, layout, hkv, s, at, n):
    """nc_kv_export_fp8 equals the oracle's rows; nc_kv_import_fp8 of those rows into another sequence at another
    unaligned start changes exactly the bytes the oracle's import changes (the whole pool compared)."""
    print(f"position rows {layout} hkv {hkv} seq {s} [{at}, {at + n})", flush=True)
    dev = gpu
    cache = make_cache(layout, 4, 160, hkv, dev, seed=61)
    random_bytes(cache, 62)
    ref = oracle_cache(cache)
    rows = cache.export_rows(s, at, n)
    torch.cuda.synchronize()
    want = G.export_rows(ref, table(cache), cache.max_blocks, s, at, n)
    np.testing.assert_array_equal(rows.cpu().numpy(), want)
    dst_seq, dst_at = (s + 1) % 4, 160 - n - 3 if n else 7
    cache.import_rows(rows, dst_seq, dst_at)
    torch.cuda.synchronize()
    G.import_rows(ref, want, table(cache), cache.max_blocks, dst_seq, dst_at)
    assert_same_cache(cache, ref)


def test_position_rows_of_several_layers(gpu):
    """The decoder's form: layers pools spaced pool_bytes apart in one allocation, exported and imported in one
    call each, against the oracle layer by layer."""
    from nanochat_amd.native import check, hip_library, pointer, stream

    dev = gpu
    L, hkv, B, cap = 3, 2, 2, 64
    caches = [make_cache("contiguous", B, cap, hkv, dev, seed=70 + l) for l in range(L)]
    pool = torch.stack([c.pages for c in caches])  # [L][blocks][hkv][4224]
    g = torch.Generator().manual_seed(73)
    pool.copy_(torch.randint(0, 256, pool.shape, generator=g, dtype=torch.uint8))
    refs = []
    for l in range(L):
        r = G.PagedCache(caches[l].num_blocks, hkv)
        r.pages[...] = pool[l].cpu().numpy()
        refs.append(r)
    mb, nb = caches[0].max_blocks, caches[0].num_blocks
    pool_bytes = pool[0].numel()
    rows = torch.empty((L, 21, hkv, 264), dtype=torch.uint8, device=dev)
    lib = hip_library()
    check(lib.nc_kv_export_fp8(pointer(pool), pool_bytes, L, None, mb, nb, B, 1, 11, 21, hkv, pointer(rows),
                               stream()))
    torch.cuda.synchronize()
    want = np.stack([G.export_rows(r, None, mb, 1, 11, 21) for r in refs])
    np.testing.assert_array_equal(rows.cpu().numpy(), want)
    check(lib.nc_kv_import_fp8(pointer(rows), L, pointer(pool), pool_bytes, None, mb, nb, B, 0, 40, 21, hkv,
                               stream()))
    torch.cuda.synchronize()
    for l in range(L):
        G.import_rows(refs[l], want[l], None, mb, 0, 40)
        np.testing.assert_array_equal(pool[l].cpu().numpy(), refs[l].pages)
