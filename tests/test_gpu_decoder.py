"""GPU end-to-end decoder (prefill + greedy decode over the fp8 cache) against a CPU restatement of the same model:
oracle/model.py's CpuModel, torch bf16 GEMMs on the CPU and the oracle's append and fp64 attention over
bit-identical cache bytes. Logits
within tolerance at every step (the two sides feed the same tokens), the greedy choice equal wherever the CPU
logits' top-two margin exceeds the tolerance, and the captured graph's replays equal to eager steps."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from nanochat_amd.decoder import Fp8Decoder, ModelConfig, RandomModel, argmax_rows
from oracle.model import CpuModel

pytestmark = pytest.mark.gpu

TINY = ModelConfig(layers=2, d_model=256, heads=2, vocab=1000)
LOGIT_ATOL = 2e-2
# 26 layers of bf16 residual roundings move the logits (std 0.82) more than two layers do: at this shape the CPU model
# itself differs from the same model with fp32 activations (only the cache rows rounded to bf16) by max 0.065 and
# mean 0.011, so the GPU is held to about twice that
CFG5_LOGIT_ATOL = 1.5e-1
CFG5_LOGIT_MEAN = 2.5e-2


def test_argmax_lowest_index_on_ties(gpu):
    x = torch.randn((5, 3001), device=gpu)
    x[0, 17] = x[0, 2000] = x[0].max() + 1  # a tie: the lower index wins
    x[1] = -1.0  # all equal: index 0
    x[2, -1] = 100.0  # the last, unaligned column
    got = argmax_rows(x).cpu().numpy()
    want = x.cpu().numpy().argmax(1)  # numpy: first occurrence
    np.testing.assert_array_equal(got, want)
    assert got[0] == 17 and got[1] == 0 and got[2] == 3000


def test_decoder_matches_cpu_model_step_by_step(gpu):
    check_against_cpu(gpu, RandomModel(TINY, gpu, seed=7))


def test_loaded_checkpoint_matches_cpu_model(gpu, tmp_path):
    """A trained-like export (inference/export_hf.py's format): sliding windows, value embeddings, QK-norm gains
    and a non-identity residual / x0 mix, written by save_hf, read back by load_hf, decoded against the CPU model."""
    from nanochat_amd.checkpoint import load_hf, save_hf
    from nanochat_amd.decoder import ModelConfig

    cfg = ModelConfig(layers=4, d_model=256, heads=2, vocab=1000, theta=1e6, windows=(16, 16, 16, -1),
                      ve_layers=(1, 3))
    m = RandomModel(cfg, "cpu", seed=13)
    g = torch.Generator().manual_seed(14)
    m.resid_lambdas = 0.8 + 0.4 * torch.rand(cfg.layers, generator=g)
    m.x0_lambdas = 0.4 * torch.rand(cfg.layers, generator=g) - 0.2
    for lw in m.layers:
        lw["q_gain"] = 0.5 + torch.rand(128, generator=g)
        lw["k_gain"] = 0.5 + torch.rand(128, generator=g)
        if "ve_gate" in lw:
            lw["ve_gate"] = torch.randn(lw["ve_gate"].shape, generator=g) * 0.1
            lw["ve"] = (torch.randn(lw["ve"].shape, generator=g) * 0.5).to(torch.bfloat16)
    save_hf(m, tmp_path, max_positions=128)
    loaded = load_hf(tmp_path, gpu)
    assert loaded.mixes and loaded.cfg.windows == (16, 16, 16, -1)
    check_against_cpu(gpu, loaded)


def check_against_cpu(gpu, model, B=3, T=40, steps=6, atol=LOGIT_ATOL, mean_tol=LOGIT_ATOL / 10, row_chunk=32):
    """Prefill B random prompts of T tokens (in chunks of row_chunk rows: several of them), then `steps` greedy
    steps on the GPU decoder and the CPU model fed the same tokens; returns the largest logit difference."""
    dev = gpu
    prompts = np.random.default_rng(8).integers(0, model.cfg.vocab, (B, T)).astype(np.int32)
    dec = Fp8Decoder(model, B, T - 1 + steps, dev, row_chunk=row_chunk)
    cpu = CpuModel(model, B, T - 1 + steps)
    dec.prefill(torch.from_numpy(prompts).to(dev))
    cpu.prefill(prompts)
    tok = prompts[:, -1].copy()
    out = torch.empty(B, dtype=torch.int32, device=dev)
    worst = 0.0
    for s in range(steps):
        p = T - 1 + s
        logits = dec._step(torch.from_numpy(tok).to(dev), torch.full((B,), p, dtype=torch.int32, device=dev), out)
        want = cpu.step(tok, p)
        got = logits.cpu().numpy()
        diff = np.abs(got - want)
        err = diff.max()
        print(f"step {s}: logit difference max {err:.3e} mean {diff.mean():.3e}, logits std {want.std():.3f}",
              flush=True)
        assert err <= atol and diff.mean() <= mean_tol, (s, err, diff.mean())
        worst = max(worst, err)
        chosen = out.cpu().numpy()
        top2 = np.sort(want, axis=1)[:, -2:]
        sure = top2[:, 1] - top2[:, 0] > 2 * atol
        np.testing.assert_array_equal(chosen[sure], want.argmax(1)[sure])
        tok = chosen  # both sides continue from the GPU's choice
    return worst


def test_graph_replays_equal_eager_steps(gpu):
    dev = gpu
    B, T, steps = 4, 33, 5
    model = RandomModel(TINY, dev, seed=9)
    prompts = torch.from_numpy(np.random.default_rng(10).integers(0, TINY.vocab, (B, T)).astype(np.int32)).to(dev)
    eager = Fp8Decoder(model, B, T - 1 + steps, dev)
    eager.prefill(prompts)
    tok, outs = prompts[:, -1].clone(), []
    for s in range(steps):
        nxt = torch.empty(B, dtype=torch.int32, device=dev)
        eager._step(tok, torch.full((B,), T - 1 + s, dtype=torch.int32, device=dev), nxt)
        outs.append(nxt.clone())
        tok = nxt
    want = torch.stack(outs, 1).cpu()
    graphed = Fp8Decoder(model, B, T - 1 + steps, dev)
    graphed.prefill(prompts)
    graphed.start(prompts[:, -1], T - 1)
    for _ in range(steps):  # one replay at a time, with eager work and a synchronisation in between
        graphed.run(1)
        torch.cuda.synchronize()
        torch.zeros(1 << 20, device=dev).sum()
    torch.testing.assert_close(graphed.tokens(steps).cpu(), want)


def test_sampled_decoding_follows_the_choice_rules(gpu):
    """Per-slot temperature / top_p / seed: every step's tokens are the oracle's choice (oracle/sampling.py) on that
    step's own logits, the positions advance by the commit, and graph replays equal eager steps."""
    from oracle import sampling as S

    dev = gpu
    B, T, steps = 4, 30, 4
    model = RandomModel(TINY, dev, seed=11)
    prompts = torch.from_numpy(np.random.default_rng(12).integers(0, TINY.vocab, (B, T)).astype(np.int32)).to(dev)
    temp = np.array([0.0, 0.7, 1.5, 1.0], np.float32)
    top_p = np.array([1.0, 1.0, 0.9, 0.5], np.float32)
    seeds = np.array([1, 2, 3, (1 << 40) + 5], np.uint64)
    eager = Fp8Decoder(model, B, T - 1 + steps, dev)
    eager.prefill(prompts)
    eager.set_sampling(temp, top_p, seeds, first=T - 1)
    tok, outs = prompts[:, -1].clone(), []
    pos = torch.full((B,), T - 1, dtype=torch.int32, device=dev)
    for s in range(steps):
        nxt = torch.empty(B, dtype=torch.int32, device=dev)
        before = pos.cpu().numpy()
        logits = eager._step(tok, pos, nxt).cpu().numpy()
        want, _, want_pos = S.choose(logits, temperature=temp, top_p=top_p, seed=seeds, pos=before,
                                     first=np.full(B, T - 1, np.int32))
        np.testing.assert_array_equal(nxt.cpu().numpy(), want, err_msg=f"step {s}")
        np.testing.assert_array_equal(pos.cpu().numpy(), want_pos)
        outs.append(nxt.clone())
        tok = nxt
    graphed = Fp8Decoder(model, B, T - 1 + steps, dev)
    graphed.prefill(prompts)
    graphed.set_sampling(temp, top_p, seeds, first=T - 1)
    graphed.start(prompts[:, -1], T - 1)
    for _ in range(steps):
        graphed.run(1)
        torch.cuda.synchronize()
    torch.testing.assert_close(graphed.tokens(steps).cpu(), torch.stack(outs, 1).cpu())


CFG5_SHAPE = ModelConfig(layers=26, d_model=1664, heads=13, vocab=65536)  # BASELINE config 5's architecture


def test_config5_architecture_matches_cpu_model(gpu):
    """The full config-5 model (26 layers, d 1664, 13 heads, vocab 65536, random init) at a size the CPU model covers:
    4 sequences of 256-token prompts, then 4 greedy steps. Every step's logits within CFG5_LOGIT_ATOL (max) and
    CFG5_LOGIT_MEAN (mean) of the CPU model's (torch bf16 GEMMs on the CPU, the oracle's append and fp64 attention),
    greedy tokens equal wherever the CPU logits' top-two margin exceeds twice the tolerance."""
    print("config 5 architecture: 4 x 256-token prompts, 4 steps", flush=True)
    torch.set_num_threads(min(16, torch.get_num_threads()))
    check_against_cpu(gpu, RandomModel(CFG5_SHAPE, gpu, seed=5), B=4, T=256, steps=4, atol=CFG5_LOGIT_ATOL,
                      mean_tol=CFG5_LOGIT_MEAN, row_chunk=1024)


def test_config5_full_batch_anchored_on_two_sequences(gpu):
    """BASELINE config 5 at its own batch and prompt length (B 128, 2048-token prompts; the full architecture, random
    init) for 3 greedy steps; sequences 0 and 127 checked against the CPU model run on those two prompts alone:
    logits within CFG5_LOGIT_ATOL / CFG5_LOGIT_MEAN, greedy tokens equal wherever the CPU logits' top-two margin
    exceeds twice the tolerance. The piece plan makes a sequence's bits independent of the other 126, so the CPU
    model needs only the two."""
    B, T, steps, pick = 128, 2048, 3, [0, 127]
    torch.set_num_threads(min(16, torch.get_num_threads()))
    model = RandomModel(CFG5_SHAPE, gpu, seed=5)
    prompts = np.random.default_rng(18).integers(0, CFG5_SHAPE.vocab, (B, T)).astype(np.int32)
    print("config 5 full batch: GPU prefill of 128 x 2048 tokens", flush=True)
    dec = Fp8Decoder(model, B, T - 1 + steps, gpu)
    dec.prefill(torch.from_numpy(prompts).to(gpu))
    cpu = CpuModel(model, len(pick), T - 1 + steps)
    sub = prompts[pick]
    for r in range(0, T - 1, 512):  # the CPU prefill in 4 chunks of positions, each after the earlier ones
        e = min(r + 512, T - 1)
        print(f"CPU prefill of positions {r}..{e - 1} of sequences {pick}", flush=True)
        cpu.prefill_rows(sub[:, r:e].reshape(-1), np.tile(np.arange(r, e), len(pick)),
                         np.repeat(np.arange(len(pick)), e - r))
    tok = prompts[:, -1].copy()
    out = torch.empty(B, dtype=torch.int32, device=gpu)
    for s in range(steps):
        p = T - 1 + s
        logits = dec._step(torch.from_numpy(tok).to(gpu), torch.full((B,), p, dtype=torch.int32, device=gpu), out)
        want = cpu.step(tok[pick], p)
        got = logits.cpu().numpy()[pick]
        diff = np.abs(got - want)
        print(f"step {s}: logit difference max {diff.max():.3e} mean {diff.mean():.3e}", flush=True)
        assert diff.max() <= CFG5_LOGIT_ATOL and diff.mean() <= CFG5_LOGIT_MEAN, (s, diff.max(), diff.mean())
        chosen = out.cpu().numpy()
        top2 = np.sort(want, axis=1)[:, -2:]
        sure = top2[:, 1] - top2[:, 0] > 2 * CFG5_LOGIT_ATOL
        np.testing.assert_array_equal(chosen[pick][sure], want.argmax(1)[sure])
        tok = chosen


def test_prefill_in_chunks_leaves_the_same_bytes(gpu):
    """A prompt prefilled in two calls (positions 0..99, then 100..174) leaves the bytes of one call in every layer:
    each row attends its own key range with its own arithmetic (whatever rows share its workgroup), and a GEMM row's
    bits do not depend on the rows computed with it. GQA (4 query heads per kv head), a window and a value-embedding
    layer, so every prefill path takes part."""
    cfg = ModelConfig(layers=3, d_model=512, heads=8, vocab=1000, n_kv_heads=2, windows=(64, -1, -1), ve_layers=(1,))
    model = RandomModel(cfg, gpu, seed=19)
    prompts = torch.from_numpy(np.random.default_rng(20).integers(0, 1000, (3, 176)).astype(np.int32)).to(gpu)
    whole = Fp8Decoder(model, 3, 200, gpu)
    whole.prefill(prompts)
    parts = Fp8Decoder(model, 3, 200, gpu)
    for lo, hi in ((0, 100), (100, 175)):
        tok = prompts[:, lo:hi].reshape(-1).contiguous()
        pos = torch.arange(lo, hi, dtype=torch.int32, device=gpu).repeat(3)
        seq = torch.arange(3, dtype=torch.int32, device=gpu).repeat_interleave(hi - lo)
        parts._prefill_rows(tok, pos, seq)
    torch.cuda.synchronize()
    for l in range(cfg.layers):
        assert torch.equal(whole.caches[l].pages, parts.caches[l].pages), f"layer {l}"


def test_prefill_is_deterministic_and_batch_independent(gpu):
    """Every sum of the prefill is in a fixed order: prefilling the same prompts twice gives the same cache bytes,
    and a prompt prefilled alone gives the bytes it gets among others (the prefill's share of the reference's promise
    that a request's tokens depend on neither the batch nor the store, inference/decoder.py:124-125; the decode
    step's attention balances its split over the batch, so only run-to-run repetition is asserted for the tokens).
    700 rows: the GEMMs take the many-rows tile together and the decode tile alone."""
    model = RandomModel(ModelConfig(layers=2, d_model=512, heads=4, vocab=1000), gpu, seed=17)
    prompts = torch.from_numpy(np.random.default_rng(18).integers(0, 1000, (4, 176)).astype(np.int32)).to(gpu)
    a = Fp8Decoder(model, 4, 200, gpu)
    b = Fp8Decoder(model, 4, 200, gpu)
    a.prefill(prompts)
    b.prefill(prompts)
    alone = Fp8Decoder(model, 1, 200, gpu)
    alone.prefill(prompts[2:3])
    torch.cuda.synchronize()
    mb = a.caches[0].max_blocks
    for l in range(2):
        assert torch.equal(a.caches[l].pages, b.caches[l].pages), l
        assert torch.equal(a.caches[l].pages[2 * mb:3 * mb], alone.caches[l].pages[:mb]), l
    # and the generations that follow: the same tokens, run after run (bench.py's config 5 digest, at a small size)
    for d in (a, b):
        d.start(prompts[:, -1], 175)
        d.run(12)
    assert torch.equal(a.tokens(12), b.tokens(12))
