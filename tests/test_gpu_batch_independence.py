"""A request's bits do not depend on the batch it is decoded with: the reference's promise that "a request's tokens
depend on neither the batch nor the store" (inference/decoder.py:124-125), which its k_attn keeps with one block per
(head, slot) (model/kernels/decode.cu:567-675) and eval/verify.py:401-405 relies on.

Checked at three levels, each for grouped-query (16 / 4) and multi-head attention:
  * nc_decode_step_fp8_pieces: a ragged batch of 64 sequences, then one sequence alone and every other sequence
    (the rest idle, position -1): each active sequence's output bits equal the full batch's; the outputs are within
    the north star's tolerance of the fp64 oracle and the cache bytes equal the oracle's append;
  * the torch-driven decoder (Fp8Decoder): a request's logits, step by step, decoded alone and among 63 others of
    other lengths are bit-identical;
  * the dec_* handle (dec_create_v2): a request's tokens, greedy and sampled, alone and among 63 others.
And the reference's own entry point, dec_create (7 configuration fields, an fp32 embedding table, the slot count
from the free memory), driven with the reference's store protocol, decodes like the CPU model.
"""

import ctypes
import math

import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits, oracle_cache, table
from nanochat_amd.attention import decode_step
from nanochat_amd.decoder import Fp8Decoder, ModelConfig, RandomModel
from nanochat_amd.workloads import DecodeConfig, build_decode_case
from oracle import golden as G

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)
PIECES = 16

KERNEL_CASES = [
    DecodeConfig("gqa-paged-ragged-64", 64, 16, 4, ctx_range=(1, 3000), paged=True, outliers=0.01, seed=301),
    DecodeConfig("mha-contiguous-window-64", 64, 8, 8, ctx_range=(1, 2500), window=700, seed=302),
    # segments of 1875 and 563 pages: 118 and 36 pieces of 16 pages (the cap follows max_ctx), 12 merge groups in
    # 1024-lane workgroups folding the long segment in two rounds, G = 5
    DecodeConfig("long-segments-g5", 3, 5, 1, ctx=(30000, 9000, 700), paged=True, seed=304),
    # one sequence of 131072 keys beside a short one: 256 pieces of 32 pages per segment, so its 4 segments still
    # occupy every wave
    DecodeConfig("long-context-b2", 2, 16, 4, ctx=(131072, 500), paged=True, seed=307),
    # more sequences than the schedule keeps in LDS: context lengths read from memory by every segment walk
    DecodeConfig("batch-past-lds-2100", 2100, 4, 2, ctx_range=(0, 200), seed=305),
]


def _step(case, pos, max_ctx, piece_pages=PIECES):
    cfg = case.cfg
    return decode_step(case.qkv[0], case.cache, pos, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq,
                       max_ctx=max_ctx, window=cfg.window, piece_pages=piece_pages)


@pytest.mark.parametrize("cfg", KERNEL_CASES, ids=[c.name for c in KERNEL_CASES])
def test_pieces_step_bits_do_not_depend_on_the_batch(gpu, cfg):
    print(f"batch independence, kernel: {cfg.name}", flush=True)
    case = build_decode_case(cfg, gpu, steps=1)
    max_ctx = int(case.ctx.max()) + 1
    before = case.cache.pages.clone()
    pos = case.positions(0)
    full = bits(_step(case, pos, max_ctx))
    torch.cuda.synchronize()
    # correctness of the plan: the appended bytes and the attention against the oracle
    host = G.PagedCache(case.cache.num_blocks, cfg.hkv)
    host.pages[...] = before.cpu().numpy()
    q_ref = G.append(host, bits(case.qkv[0]), pos.cpu().numpy(), np.arange(cfg.batch), case.q_gain.cpu().numpy(),
                     case.k_gain.cpu().numpy(), case.cos.cpu().numpy(), case.sin.cpu().numpy(), cfg.hq, cfg.hkv,
                     table(case.cache), case.cache.max_blocks)
    np.testing.assert_array_equal(case.cache.pages.cpu().numpy(), host.pages)
    want = G.decode_attention(q_ref, host, table(case.cache), case.cache.max_blocks, case.ctx + 1, cfg.window, cfg.hq,
                              cfg.hkv, SCALE)
    assert_attention_close(torch.from_numpy(full.view(np.int16)).view(torch.bfloat16), want, cfg.name)
    # the same sequences decoded alone and in other company: the same bits
    for name, active in (("alone 0", [0]), ("alone mid", [min(37, cfg.batch - 1)]), ("alone last", [cfg.batch - 1]),
                         ("odd", list(range(1, cfg.batch, 2)))):
        case.cache.pages.copy_(before)
        p = torch.full_like(pos, -1)
        p[active] = pos[active]
        got = bits(_step(case, p, max_ctx))
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got[active], full[active], err_msg=name)


def test_pieces_step_is_correct_at_every_piece_length(gpu):
    """Pieces of 1 page (every page its own piece, so a segment of up to 8 pages) up to one piece per segment."""
    cfg = DecodeConfig("pieces-lengths", 12, 8, 2, ctx=(1, 15, 16, 17, 127, 128, 129, 700, 1000, 2048, 33, 260),
                       paged=True, seed=303)
    for piece_pages in (1, 3, 16, 64, 65536):
        case = build_decode_case(cfg, gpu, steps=1)
        max_ctx = int(case.ctx.max()) + 1
        pos = case.positions(0)
        q = case.cache.append(case.qkv[0], pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq)
        ref = oracle_cache(case.cache)
        want = G.decode_attention(bits(q), ref, table(case.cache), case.cache.max_blocks, case.ctx + 1, cfg.window,
                                  cfg.hq, cfg.hkv, SCALE)
        got = _step(case, pos, max_ctx, piece_pages)  # rewrites the same appended bytes
        assert_attention_close(got, want, f"piece_pages {piece_pages}")


@pytest.mark.parametrize("hq,hkv", [(4, 4), (16, 4), (16, 2)], ids=["g1", "g4", "g8"])
def test_pieces_step_bits_do_not_depend_on_max_ctx(gpu, hq, hkv):
    """k_merge launches only the lane groups that the longest segment allowed by max_ctx can fill (1 to 4 groups of
    8 pieces). Sequences at the group boundaries (8, 9, 16, 17 and 31 pieces of 16 or 17 pages after the append)
    keep their bits whatever max_ctx the call names, as long as it admits them."""
    print(f"piece plan, max_ctx groups: hq {hq} hkv {hkv}", flush=True)
    cfg = DecodeConfig(f"pieces-max-ctx-{hq}-{hkv}", 7, hq, hkv, ctx=(0, 99, 2047, 2048, 4095, 4096, 8400),
                       paged=True, seed=306)
    case = build_decode_case(cfg, gpu, steps=1)
    pos = case.positions(0)
    ctx_after = case.ctx + 1
    full = bits(_step(case, pos, case.cache.capacity))
    torch.cuda.synchronize()
    ref = oracle_cache(case.cache)
    q = case.cache.append(case.qkv[0], pos, case.seq, case.q_gain, case.k_gain, case.cos, case.sin, cfg.hq)
    want = G.decode_attention(bits(q), ref, table(case.cache), case.cache.max_blocks, ctx_after, cfg.window, cfg.hq,
                              cfg.hkv, SCALE)
    assert_attention_close(torch.from_numpy(full.view(np.int16)).view(torch.bfloat16), want, cfg.name)
    for max_ctx in (4097, 4096, 2048, 100):  # 17, 16, 8 and 1 pieces at most: 3, 2, 1 and 1 groups
        active = np.flatnonzero(ctx_after <= max_ctx)
        p = torch.full_like(pos, -1)
        p[active] = pos[active]
        got = bits(_step(case, p, max_ctx))  # rewrites the same appended bytes
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got[active], full[active], err_msg=f"max_ctx {max_ctx}")


def _ragged_prompts(rng, n, vocab, lo, hi):
    return [rng.integers(0, vocab, int(rng.integers(lo, hi + 1))).astype(np.int32) for _ in range(n)]


def _prefill_ragged(dec, prompts, dev):
    """Each prompt's positions 0..T-2 into its own sequence, all rows in one call."""
    tok = np.concatenate([p[:-1] for p in prompts])
    pos = np.concatenate([np.arange(len(p) - 1) for p in prompts])
    seq = np.concatenate([np.full(len(p) - 1, b) for b, p in enumerate(prompts)])
    as_dev = lambda a: torch.from_numpy(a.astype(np.int32)).to(dev)
    dec._prefill_rows(as_dev(tok), as_dev(pos), as_dev(seq))


@pytest.mark.parametrize("kv_heads", [2, 0], ids=["gqa", "mha"])
def test_decoder_logits_alone_equal_in_a_ragged_batch(gpu, kv_heads):
    print(f"batch independence, decoder: kv heads {kv_heads or 'all'}", flush=True)
    cfg = ModelConfig(layers=2, d_model=512, heads=4, vocab=1000, n_kv_heads=kv_heads)
    model = RandomModel(cfg, gpu, seed=311)
    rng = np.random.default_rng(312)
    prompts = _ragged_prompts(rng, 64, cfg.vocab, 2, 300)
    steps, pick = 6, [0, 21, 63]
    big = Fp8Decoder(model, 64, 310, gpu)
    _prefill_ragged(big, prompts, gpu)
    tok = torch.tensor([int(p[-1]) for p in prompts], dtype=torch.int32, device=gpu)
    pos = torch.tensor([len(p) - 1 for p in prompts], dtype=torch.int32, device=gpu)
    out = torch.empty(64, dtype=torch.int32, device=gpu)
    batch_logits, batch_toks = [], []
    for s in range(steps):
        logits = big._step(tok, pos.clone(), out)
        batch_logits.append(logits.clone())
        batch_toks.append(out.clone())
        tok, pos = out.clone(), pos + 1
    for b in pick:
        alone = Fp8Decoder(model, 1, 310, gpu)
        _prefill_ragged(alone, [prompts[b]], gpu)
        t = torch.tensor([int(prompts[b][-1])], dtype=torch.int32, device=gpu)
        p = torch.tensor([len(prompts[b]) - 1], dtype=torch.int32, device=gpu)
        o = torch.empty(1, dtype=torch.int32, device=gpu)
        for s in range(steps):
            logits = alone._step(t, p.clone(), o)
            assert torch.equal(logits[0], batch_logits[s][b]), (b, s)
            assert int(o[0]) == int(batch_toks[s][b]), (b, s)
            t, p = o.clone(), p + 1


@pytest.mark.parametrize("kv_heads", [2, 0], ids=["gqa", "mha"])
def test_handle_tokens_alone_equal_in_a_ragged_batch(gpu, kv_heads):
    print(f"batch independence, handle: kv heads {kv_heads or 'all'}", flush=True)
    from nanochat_amd.native_decoder import NativeDecoder
    from nanochat_amd.serving import Request

    cfg = ModelConfig(layers=2, d_model=512, heads=4, vocab=1000, n_kv_heads=kv_heads)
    model = RandomModel(cfg, gpu, seed=321)
    rng = np.random.default_rng(322)
    reqs = [Request(input_ids=p.tolist(), max_new_tokens=8, temperature=0.0 if k % 2 else 0.9, seed=900 + k)
            for k, p in enumerate(_ragged_prompts(rng, 64, cfg.vocab, 2, 200))]
    big = NativeDecoder(model, bos=-1, max_length=220, batch=64)
    together = dict(big.generate(reqs))
    assert sorted(together) == list(range(64))
    for k in (0, 1, 30, 63):
        one = NativeDecoder(model, bos=-1, max_length=220, batch=1)
        alone = dict(one.generate([reqs[k]]))
        assert alone[0] == together[k], (k, alone[0], together[k])


def test_reference_dec_create_decodes_like_the_cpu_model(gpu):
    """dec_create as inference/decoder.py:157-185 calls it: 7 configuration fields (no kv head count, slot count or
    embedding dtype: MHA, the slots the free memory holds, an fp32 embed_tokens table), then the reference's protocol
    for two prompts: dec_set_prompt, dec_prefill of the rows [token, position, slot], dec_save_prompt at the store
    offsets the reference hands out (used = 0, then the first prompt's length), greedy steps. Every greedy token
    whose CPU top-two margin clears the tolerance equals the CPU model's, fed the same fp32 table."""
    from nanochat_amd.native import hip_library
    from nanochat_amd.native_decoder import handle_pointers
    from nanochat_amd.rotary import rotary_tables
    from nanochat_amd.sampling import slot_masks
    from oracle.model import CpuModel

    cfg = ModelConfig(layers=2, d_model=256, heads=2, vocab=1000)
    model = RandomModel(cfg, gpu, seed=331)
    wte32 = model.wte.float().contiguous()  # the reference's fp32 embedding table
    max_len, store = 64, 128
    cos, sin = rotary_tables(max_len, cfg.theta, gpu)
    tensors = handle_pointers(model, cos, sin)
    tensors[0] = wte32
    ptrs = np.array([0 if t is None else t.data_ptr() for t in tensors], dtype=np.uint64)
    scal = np.append(np.stack([model.resid_lambdas.cpu().numpy(), model.x0_lambdas.cpu().numpy()], 1).reshape(-1),
                     np.float32(cfg.softcap)).astype(np.float32)
    window = np.full(cfg.layers, -1, dtype=np.int32)
    config = np.array([cfg.layers, cfg.d_model, cfg.mlp_mult * cfg.d_model, cfg.vocab, max_len, store, -1],
                      dtype=np.int32)
    lib = hip_library()
    stream = torch.cuda.Stream(gpu)
    torch.cuda.synchronize()
    h = ctypes.c_void_p(lib.dec_create(config.ctypes.data, ptrs.ctypes.data, scal.ctypes.data, window.ctypes.data,
                                       ctypes.c_void_p(stream.cuda_stream)))
    try:
        B = lib.dec_batch(h)
        assert 2 <= B <= 1024
        rng = np.random.default_rng(332)
        prompts = [rng.integers(0, cfg.vocab, n).astype(np.int32) for n in (23, 9)]
        used = 0
        for b, ids in enumerate(prompts):
            lib.dec_set_prompt(h, b, int(ids[-1]), len(ids) - 1, 0.0, 1.0, 0)
        rows = np.concatenate([np.array([ids[:-1], np.arange(len(ids) - 1), np.full(len(ids) - 1, b)], np.int32)
                               for b, ids in enumerate(prompts)], axis=1)
        rows = np.ascontiguousarray(rows)
        lib.dec_prefill(h, rows.shape[1], rows.ctypes.data)
        for b, ids in enumerate(prompts):  # the reference's save(): back-to-back store offsets
            lib.dec_save_prompt(h, b, 0, used, len(ids) - 1)
            used += len(ids) - 1
        words = np.ascontiguousarray(slot_masks([b < len(prompts) for b in range(B)]))
        lib.dec_set_active(h, words.ctypes.data)
        out = np.empty(2 * B, dtype=np.int32)
        steps = 10
        got = np.empty((steps, len(prompts)), dtype=np.int32)
        for s in range(steps):
            lib.dec_launch_body(h)
            lib.dec_launch_head(h)
            lib.dec_tokens(h, out.ctypes.data)
            got[s] = out[:len(prompts)]
    finally:
        lib.dec_destroy(h)

    class Fp32Table:
        pass

    ref = Fp32Table()
    for k in ("cfg", "layers", "lm_head", "resid_lambdas", "x0_lambdas"):
        setattr(ref, k, getattr(model, k))
    ref.wte = wte32
    checked = 0
    for b, ids in enumerate(prompts):
        cpu = CpuModel(ref, 1, max_len)
        cpu.prefill(ids[None])
        tok, p = ids[-1:], len(ids) - 1
        for s in range(steps):
            logits = cpu.step(tok, p)[0]
            top = np.sort(logits)[-2:]
            if top[1] - top[0] > 2e-2:
                assert got[s, b] == int(np.argmax(logits)), (b, s, got[s, b], int(np.argmax(logits)))
                checked += 1
            tok, p = np.array([got[s, b]], np.int32), p + 1
    assert checked >= 15, checked
