"""GPU parity of chunked prefill (append the whole chunk, then MFMA attention of every chunk row over the fp8 cache)
against the oracle: bit-exact q rows and cache bytes for the append, and attention within the benchmark tolerance
(max abs <= 2e-2, mean <= 2e-3) of the fp64 oracle over the same cache bytes."""

import math

import numpy as np
import pytest
import torch

from helpers import assert_attention_close, assert_same_cache, bits, oracle_cache, table
from nanochat_amd.attention import decode_attention, prefill_attention
from nanochat_amd.workloads import CONFIG4, PrefillConfig, build_prefill_case, prefill_step
from oracle import golden as G

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)


def oracle_rows(case, q, pos, seq, window):
    return G.rows_attention(bits(q), pos.cpu().numpy(), seq.cpu().numpy(), oracle_cache(case.cache),
                            table(case.cache), case.cache.max_blocks, case.cache.num_seqs, window, case.cfg.hq,
                            case.cfg.hkv, SCALE)


def run_and_check(cfg: PrefillConfig, dev, check_append: bool = False):
    print(f"prefill case {cfg.name}", flush=True)
    case = build_prefill_case(cfg, dev)
    before = oracle_cache(case.cache) if check_append else None
    q, out = prefill_step(case)
    torch.cuda.synchronize()
    if check_append:
        q_ref = G.append(before, bits(case.qkv), case.pos.cpu().numpy(), case.seq.cpu().numpy(),
                         case.q_gain.cpu().numpy(), case.k_gain.cpu().numpy(), case.cos.cpu().numpy(),
                         case.sin.cpu().numpy(), cfg.hq, cfg.hkv, table(case.cache), case.cache.max_blocks)
        np.testing.assert_array_equal(bits(q), q_ref)
        assert_same_cache(case.cache, before)
    want = oracle_rows(case, q, case.pos, case.seq, cfg.window)
    return assert_attention_close(out, want, cfg.name)


def test_config4_full_size(gpu):
    run_and_check(CONFIG4, gpu, check_append=True)


@pytest.mark.parametrize("cfg", [
    PrefillConfig("mha-g1", 2, 4, 4, cached=(100, 1000), chunk=(300, 45), paged=True, seed=41),
    PrefillConfig("g16-one-kv-head", 2, 16, 1, cached=(0, 700), chunk=(37, 5), seed=42),
    PrefillConfig("g3-window64", 1, 6, 2, cached=(500,), chunk=(77,), window=64, paged=True, seed=43),
    PrefillConfig("g8-window-not-aligned", 3, 8, 1, cached=(900, 17, 250), chunk=(20, 100, 9), window=100, seed=44),
    PrefillConfig("ragged-chunks-cross-tiles", 5, 16, 4, cached=(3, 60, 1, 300, 31), chunk=(7, 13, 3, 29, 1),
                  paged=True, outliers=0.01, seed=45),
    PrefillConfig("long-over-1024-pages", 1, 4, 1, cached=(17000,), chunk=(40,), paged=True, seed=46),
])
def test_prefill_edge_shapes(gpu, cfg):
    run_and_check(cfg, gpu)


@pytest.mark.parametrize("cfg", [
    CONFIG4,
    PrefillConfig("causal-g1", 4, 16, 16, cached=(0,), chunk=(700,), seed=9),
    PrefillConfig("g4-outliers", 4, 16, 4, cached=(300,), chunk=(500,), outliers=0.01, seed=10),
    PrefillConfig("g8-window-paged", 3, 16, 2, cached=(900, 50, 400), chunk=(200, 300, 90), window=250, paged=True,
                  seed=11),
])
def test_a_row_does_not_depend_on_its_neighbours(gpu, cfg):
    """Each column keeps its own softmax state (lazy max, value-scale exponent) and meets its keys in page pairs that
    start at even pages, so a row's output bits do not depend on the rows computed with it: every subset, order and
    alignment gives the bits of the full call (the reference's k_attn attends each row alone)."""
    print(f"prefill grouping case {cfg.name}", flush=True)
    case = build_prefill_case(cfg, gpu)
    q = case.cache.append(case.qkv, case.pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq)
    full = prefill_attention(q, case.cache, case.pos, case.seq, window=cfg.window)
    n = q.shape[0]
    perm = torch.from_numpy(np.random.default_rng(cfg.seed).permutation(n)).to(gpu)
    subsets = {"odd rows": torch.arange(1, n, 2, device=gpu), "shifted by 5": torch.arange(5, n, device=gpu),
               "reversed": torch.arange(n - 1, -1, -1, device=gpu), "permuted": perm,
               "a few alone": perm[:7]}
    for name, idx in subsets.items():
        rows = [idx[i:i + 1] for i in range(idx.numel())] if name == "a few alone" else [idx]
        for r in rows:
            sub = prefill_attention(q[r].contiguous(), case.cache, case.pos[r].contiguous(),
                                    case.seq[r].contiguous(), window=cfg.window)
            torch.cuda.synchronize()
            assert torch.equal(sub.view(torch.int16), full[r].view(torch.int16)), f"{cfg.name}: {name}"


def test_rows_in_any_order_and_invalid_rows(gpu):
    """Shuffled rows (so tiles mix sequences and positions) give the oracle's per-row result; rows with pos < 0 or
    a sequence out of range are zero and disturb no other row."""
    dev = gpu
    cfg = PrefillConfig("shuffled", 3, 8, 2, cached=(200, 40, 513), chunk=(50, 21, 64), paged=True, seed=51)
    case = build_prefill_case(cfg, dev)
    q, _ = prefill_step(case)
    perm = torch.from_numpy(np.random.default_rng(52).permutation(q.shape[0])).to(dev)
    qp, pos, seq = q[perm].contiguous(), case.pos[perm].contiguous(), case.seq[perm].contiguous()
    pos[5], seq[9], seq[10] = -1, 3, -2
    out = prefill_attention(qp, case.cache, pos, seq)
    torch.cuda.synchronize()
    want = oracle_rows(case, qp, pos, seq, -1)
    assert not bits(out[[5, 9, 10]]).any()
    assert_attention_close(out, want, "shuffled")


def test_rows_whose_q_is_not_finite(gpu):
    """Rows past the rotary table get NaN q rows from the append (and write no cache byte); the prefill gives them
    NaN rows, as the decode step does for the same positions, and every other row keeps the bits it has without
    them and the oracle's result. A NaN or an infinity in one head of an otherwise valid row makes the G heads that
    share its kv head NaN; the row's other heads keep their bits. Rows with pos < 0 stay zero whatever their q."""
    dev = gpu
    cfg = PrefillConfig("nonfinite", 2, 8, 2, cached=(120, 300), chunk=(40, 33), paged=True, seed=71)
    case = build_prefill_case(cfg, dev)
    G_ = cfg.hq // cfg.hkv
    rope_len = case.cos.shape[0]
    pos = case.pos.clone()
    past = [3, 17, 50]
    pos[past] = rope_len + torch.tensor([0, 5, 1000], dtype=torch.int32, device=dev)
    before = oracle_cache(case.cache)
    q = case.cache.append(case.qkv, pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq)
    torch.cuda.synchronize()
    assert (bits(q[past]) == 0x7fc0).all()
    keep = [i for i in range(q.shape[0]) if i not in past]
    # the append skipped the rows past the table: the cache equals one written without them
    G.append(before, bits(case.qkv[keep]), case.pos[keep].cpu().numpy(), case.seq[keep].cpu().numpy(),
             case.q_gain.cpu().numpy(), case.k_gain.cpu().numpy(), case.cos.cpu().numpy(), case.sin.cpu().numpy(),
             cfg.hq, cfg.hkv, table(case.cache), case.cache.max_blocks)
    assert_same_cache(case.cache, before)
    q_bad = q.clone()
    q_bad[8, 3, 77] = float("nan")   # kv head 0's group of row 8
    q_bad[9, G_, 0] = float("inf")   # kv head 1's group of row 9
    pos_bad = pos.clone()
    pos_bad[12] = -1
    q_bad[12, 1, 5] = float("nan")   # pos < 0: zero row whatever its q
    out = prefill_attention(q_bad, case.cache, pos_bad, case.seq)
    clean = prefill_attention(q[[8, 9]].contiguous(), case.cache, pos[[8, 9]].contiguous(),
                              case.seq[[8, 9]].contiguous())
    torch.cuda.synchronize()
    assert (bits(out[past]) == 0x7fc0).all()
    assert (bits(out[8, :G_]) == 0x7fc0).all() and (bits(out[9, G_:]) == 0x7fc0).all()
    assert np.array_equal(bits(out[8, G_:]), bits(clean[0, G_:])) and np.array_equal(bits(out[9, :G_]),
                                                                                      bits(clean[1, :G_]))
    assert not bits(out[12]).any()
    rest = torch.tensor([i for i in range(q.shape[0]) if i not in past + [8, 9, 12]], device=dev)
    alone = prefill_attention(q[rest].contiguous(), case.cache, pos[rest].contiguous(), case.seq[rest].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(out[rest].view(torch.int16), alone.view(torch.int16))
    want = oracle_rows(case, q[rest].contiguous(), pos[rest].contiguous(), case.seq[rest].contiguous(), -1)
    assert_attention_close(out[rest], want, "nonfinite neighbours")


def test_missing_blocks_are_skipped(gpu):
    dev = gpu
    cfg = PrefillConfig("holes", 2, 4, 2, cached=(300, 300), chunk=(40, 40), paged=True, seed=61)
    case = build_prefill_case(cfg, dev)
    q, _ = prefill_step(case)
    case.cache.block_table[0, 3] = -1           # keys 48..63 of sequence 0
    case.cache.block_table[1, 5] = 10 ** 6      # beyond the pool
    out = prefill_attention(q, case.cache, case.pos, case.seq)
    torch.cuda.synchronize()
    assert_attention_close(out, oracle_rows(case, q, case.pos, case.seq, -1), "holes")


def test_single_rows_agree_with_decode(gpu):
    """One row per sequence at its last position is a decode step: the two kernels agree closely."""
    dev = gpu
    cfg = PrefillConfig("as-decode", 4, 16, 4, cached=(1000, 2047, 16, 5000), chunk=(1,), paged=True, seed=71)
    case = build_prefill_case(cfg, dev)
    q, out = prefill_step(case)
    ctx = case.pos + 1
    dec = decode_attention(q, case.cache, ctx, max_ctx=case.cache.capacity)
    torch.cuda.synchronize()
    torch.testing.assert_close(out.float(), dec.float(), atol=4e-3, rtol=2e-2)
    assert_attention_close(out, oracle_rows(case, q, case.pos, case.seq, -1), "as-decode")



def test_value_scales_below_the_headroom_cap(gpu):
    """Every value scale below 2^-65, so the kernel's P headroom w = 2^lw sits at its cap (2^64) throughout, and the
    largest v_scale exponent rises once (the first 8 pages at 2^-67 times the ordinary scales, the rest of the cache
    and the chunk's values at 2^-66): o and l must keep one unit across the rise. Outputs are ~2^-66, so both sides
    are compared after a factor 2^66; a wrong rescale of o would shift the first pages' half of every row by 2x."""
    dev = gpu
    cfg = PrefillConfig("values-below-cap", 2, 8, 2, cached=(200, 150), chunk=(40, 30), paged=True, seed=81)
    case = build_prefill_case(cfg, dev)
    c = case.cache
    v0 = (cfg.hq + cfg.hkv) * 128
    case.qkv[:, v0:] = (case.qkv[:, v0:].float() * 2.0 ** -66).to(torch.bfloat16)
    for s in range(cfg.batch):
        for p in range(-(-int(case.cached[s]) // 16)):
            blk = int(c.block_table[s, p]) if c.block_table is not None else s * c.max_blocks + p
            c.v_scale[blk] *= 2.0 ** (-67 if p < 8 else -66)
    q, out = prefill_step(case)
    torch.cuda.synchronize()
    want = oracle_rows(case, q, case.pos, case.seq, -1)
    assert np.abs(want).max() < 2.0 ** -60
    assert_attention_close((out.float() * 2.0 ** 66).to(torch.bfloat16), want * 2.0 ** 66, cfg.name)  # exact scaling
