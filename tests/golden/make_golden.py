"""Writes the golden fixtures of this directory from the oracle (oracle/golden.py): small, seeded inputs and their
expected outputs, frozen so that a change of the oracle or of the HIP path shows against fixed data.

    python tests/golden/make_golden.py

decode_small.npz   one sequence (2 kv heads, 4 query heads) holding 40 cached tokens in a paged cache, one appended
                   token, then decode attention over the 41 keys: the append's q bits and cache bytes, the
                   attention output (fp64).
prefill_small.npz  two sequences (1 kv head, 3 query heads) with 20 and 5 cached tokens, chunks of 13 and 7 rows
                   appended, then chunked-prefill attention of every chunk row, window 9.

The reference ships no vectors for this path (its only test, eval/test_dry.py, covers DRY sampling), so the
expected outputs here are the oracle's, whose rules are pinned by tests/test_oracle.py.
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import golden as G  # noqa: E402


def bf16(rng, shape, scale=1.0):
    return G.bf16_bits((rng.standard_normal(shape) * scale).astype(np.float32))


def filled_cache(rng, ctx, hkv, max_blocks, table):
    c = G.PagedCache(table.max() + 1 if table is not None else len(ctx) * max_blocks, hkv)
    for b, L in enumerate(ctx):
        if L == 0:
            continue
        t = np.arange(L)
        blk = G.PagedCache.block_of(np.full(L, b), t, table, max_blocks)
        for h in range(hkv):
            kc, ks = G.quantize_rows(bf16(rng, (L, 128)))
            vc, vs = G.quantize_rows(bf16(rng, (L, 128)))
            c.write(blk, h, t % G.PAGE, kc, ks, vc, vs)
    return c


def decode_small():
    rng = np.random.default_rng(1001)
    hq, hkv, ctx, max_blocks, theta = 4, 2, 40, 4, 1e6
    table = np.array([[5, 2, 7, 0]], np.int32)  # 4 pages, a permutation of blocks of an 8-block pool
    cache = filled_cache(rng, [ctx], hkv, max_blocks, table)
    cache_in = cache.pages.copy()
    qkv = bf16(rng, (1, (hq + 2 * hkv) * 128))
    q_gain = (0.5 + rng.random(128)).astype(np.float32)
    k_gain = (0.5 + rng.random(128)).astype(np.float32)
    cos, sin = G.rotary_tables(64, theta)
    pos = np.array([ctx], np.int32)
    q = G.append(cache, qkv, pos, np.array([0]), q_gain, k_gain, cos, sin, hq, hkv, table, max_blocks)
    out = G.decode_attention(q, cache, table, max_blocks, pos + 1, -1, hq, hkv, 128 ** -0.5)
    return dict(hq=hq, hkv=hkv, theta=theta, rope_len=64, max_blocks=max_blocks, table=table, cache_in=cache_in,
                qkv=qkv, q_gain=q_gain, k_gain=k_gain, pos=pos, q_out=q, cache_out=cache.pages, attn=out)


def prefill_small():
    rng = np.random.default_rng(1002)
    hq, hkv, max_blocks, theta, window = 3, 1, 3, 1e4, 9
    cached, chunk = [20, 5], [13, 7]
    cache = filled_cache(rng, cached, hkv, max_blocks, None)
    cache_in = cache.pages.copy()
    n = sum(chunk)
    qkv = bf16(rng, (n, (hq + 2 * hkv) * 128))
    q_gain = np.ones(128, np.float32)
    k_gain = (0.5 + rng.random(128)).astype(np.float32)
    cos, sin = G.rotary_tables(48, theta)
    pos = np.concatenate([np.arange(c, c + k) for c, k in zip(cached, chunk)]).astype(np.int32)
    seq = np.repeat(np.arange(2), chunk).astype(np.int32)
    q = G.append(cache, qkv, pos, seq, q_gain, k_gain, cos, sin, hq, hkv, None, max_blocks)
    out = G.rows_attention(q, pos, seq, cache, None, max_blocks, 2, window, hq, hkv, 128 ** -0.5)
    return dict(hq=hq, hkv=hkv, theta=theta, rope_len=48, max_blocks=max_blocks, window=window, cache_in=cache_in,
                qkv=qkv, q_gain=q_gain, k_gain=k_gain, pos=pos, seq=seq, q_out=q, cache_out=cache.pages, attn=out)


FIXTURES = {"decode_small.npz": decode_small, "prefill_small.npz": prefill_small}

if __name__ == "__main__":
    for name, make in FIXTURES.items():
        np.savez_compressed(os.path.join(HERE, name), **make())
        print("wrote", name)
