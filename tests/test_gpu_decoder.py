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


def check_against_cpu(gpu, model):
    dev = gpu
    B, T, steps = 3, 40, 6
    prompts = np.random.default_rng(8).integers(0, model.cfg.vocab, (B, T)).astype(np.int32)
    dec = Fp8Decoder(model, B, T - 1 + steps, dev, row_chunk=32)  # several row chunks in the prefill
    cpu = CpuModel(model, B, T - 1 + steps)
    dec.prefill(torch.from_numpy(prompts).to(dev))
    cpu.prefill(prompts)
    tok = prompts[:, -1].copy()
    out = torch.empty(B, dtype=torch.int32, device=dev)
    for s in range(steps):
        p = T - 1 + s
        logits = dec._step(torch.from_numpy(tok).to(dev), torch.full((B,), p, dtype=torch.int32, device=dev), out)
        want = cpu.step(tok, p)
        got = logits.cpu().numpy()
        err = np.abs(got - want).max()
        assert err <= LOGIT_ATOL, (s, err)
        chosen = out.cpu().numpy()
        top2 = np.sort(want, axis=1)[:, -2:]
        sure = top2[:, 1] - top2[:, 0] > 2 * LOGIT_ATOL
        np.testing.assert_array_equal(chosen[sure], want.argmax(1)[sure])
        tok = chosen  # both sides continue from the GPU's choice


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
