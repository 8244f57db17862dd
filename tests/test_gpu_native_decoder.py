"""The decoder handle (dec_*, nanochat_amd/native_decoder.py over csrc/decoder.hip): the reference's NativeDecoder
protocol run natively. Every request's tokens are checked against a CPU run of that request alone (the serving
tests' check_alone), for a random model and for a trained-like export (windows, value embeddings, residual mix);
the prompt store and the narrow graphs are exercised on the way."""

import numpy as np
import pytest
import torch

from nanochat_amd.decoder import Fp8Decoder, ModelConfig, RandomModel
from nanochat_amd.native_decoder import NativeDecoder
from nanochat_amd.sampling import slot_masks
from nanochat_amd.serving import Request, prompt_rows
from test_gpu_decoder import TINY
from test_gpu_serving import BOS, check_alone

pytestmark = pytest.mark.gpu


def mixed_requests(rng, vocab, even):
    lens, news = [6, 12, 25, 9, 30, 4, 17], [5, 3, 6, 8, 2, 7, 4]
    temps = [0.0, 0.0, 0.8, 0.0, 1.2, 0.0, 0.5]
    reqs = []
    for k, (n, m, t) in enumerate(zip(lens, news, temps)):
        ids = [BOS] + rng.integers(8, vocab, n - 1).tolist()
        mask = (lambda out: even) if k == 3 else None
        stop = (lambda out: len(out) >= 2 and out[-1] == out[-2]) if k == 1 else None
        reqs.append(Request(input_ids=ids, max_new_tokens=m, temperature=t, seed=1000 + k, mask=mask,
                            stopping_criteria=stop))
    return reqs


def test_native_decoder_matches_each_request_alone(gpu):
    print("native decoder: random model, 3 slots", flush=True)
    model = RandomModel(TINY, gpu, seed=51)
    even = np.arange(TINY.vocab) % 2 == 0
    reqs = mixed_requests(np.random.default_rng(52), TINY.vocab, even)
    dec = NativeDecoder(model, bos=BOS, max_length=48, batch=3)
    assert dec.batch == 3
    got = dict(dec.generate(reqs))
    assert sorted(got) == list(range(len(reqs)))
    checked = sum(check_alone(model, k, r, got[k], even) for k, r in enumerate(reqs))
    assert checked >= 25, checked


def test_native_decoder_runs_a_trained_like_export(gpu, tmp_path):
    """Grouped-query heads (4 over 2), sliding windows, value embeddings, QK-norm gains and a non-identity residual /
    x0 mix (fp32 lambdas), loaded from the export format: the handle's GQA, mix, value-embedding and window paths
    against the CPU model."""
    print("native decoder: trained-like export", flush=True)
    from nanochat_amd.checkpoint import load_hf, save_hf

    cfg = ModelConfig(layers=4, d_model=512, heads=4, vocab=1000, theta=1e6, windows=(16, 16, 16, -1),
                      ve_layers=(1, 3), n_kv_heads=2)
    m = RandomModel(cfg, "cpu", seed=53)
    g = torch.Generator().manual_seed(54)
    m.resid_lambdas = 0.8 + 0.4 * torch.rand(cfg.layers, generator=g)
    m.x0_lambdas = 0.4 * torch.rand(cfg.layers, generator=g) - 0.2
    for lw in m.layers:
        lw["q_gain"] = 0.5 + torch.rand(128, generator=g)
        lw["k_gain"] = 0.5 + torch.rand(128, generator=g)
        if "ve_gate" in lw:
            lw["ve_gate"] = torch.randn(lw["ve_gate"].shape, generator=g) * 0.1
            lw["ve"] = (torch.randn(lw["ve"].shape, generator=g) * 0.5).to(torch.bfloat16)
    save_hf(m, tmp_path, max_positions=128)
    model = load_hf(tmp_path, gpu)
    assert model.cfg.kv_heads == 2
    rng = np.random.default_rng(55)
    reqs = [Request(input_ids=[BOS] + rng.integers(8, cfg.vocab, n).tolist(), max_new_tokens=6,
                    temperature=0.0 if k % 2 == 0 else 0.9, seed=70 + k) for k, n in enumerate([20, 33, 9, 26])]
    dec = NativeDecoder(model, bos=BOS, max_length=48, batch=2)
    got = dict(dec.generate(reqs))
    checked = sum(check_alone(model, k, r, got[k]) for k, r in enumerate(reqs))
    assert checked >= 12, checked


def test_native_prompt_store_and_narrow_graphs(gpu):
    """300 slots (the narrow graphs cover the first 256): requests in slots past 256 end first, the rest then run on
    the narrow graphs; repeated prompts load their stored pages (and decode as their CPU runs alone)."""
    print("native decoder: 300 slots, prompt store", flush=True)
    model = RandomModel(TINY, gpu, seed=61)
    rng = np.random.default_rng(62)
    base = [BOS] + rng.integers(8, TINY.vocab, 22).tolist()
    reqs = [Request(input_ids=base if k in (0, 299) else [BOS] + rng.integers(8, TINY.vocab, 5 + k % 9).tolist(),
                    max_new_tokens=2 if k >= 256 else 5, temperature=0.0, seed=k) for k in range(300)]
    dec = NativeDecoder(model, bos=BOS, max_length=48, prompt_store=256, batch=300)
    got = dict(dec.generate(reqs))
    assert sorted(got) == list(range(300))
    assert dec.loads == 0  # every prompt was new when its slot started (all 300 start together)
    again = dict(dec.generate([reqs[0], reqs[1]]))
    assert dec.loads == 2  # both prompts come from the store now
    checked = sum(check_alone(model, k, reqs[k], got[k]) for k in (0, 1, 2, 255, 256, 298))
    checked += sum(check_alone(model, k, reqs[k], again[k]) for k in (0, 1))
    assert checked >= 14, checked


def test_native_rejected_bos_takes_the_alternative(gpu):
    """Masks allowing only BOS and one token x, and requests that never accept BOS: every chosen BOS gives way to the
    alternative through dec_take_alt, so each continuation is x repeated (the serving test, on the handle)."""
    model = RandomModel(TINY, gpu, seed=41)
    rng = np.random.default_rng(42)
    reqs = []
    for k in range(6):
        allowed = np.zeros(TINY.vocab, bool)
        allowed[[BOS, 100 + 37 * k]] = True
        reqs.append(Request(input_ids=[BOS] + rng.integers(8, TINY.vocab, 12).tolist(), max_new_tokens=4,
                            mask=lambda out, m=allowed: m, accept_bos=lambda out: False))
    dec = NativeDecoder(model, bos=BOS, max_length=32, batch=3)
    out = dict(dec.generate(reqs))
    for k in range(6):
        assert out[k] == [100 + 37 * k] * 4, (k, out[k])
    assert dec.alts_taken > 0


def test_native_store_at_unaligned_positions_decodes_as_prefilled(gpu):
    """The reference's store protocol (inference/decoder.py:202-232): each new prompt of n cached positions is saved at
    the store position where the previous one ended (0, 5, 23, 55: page boundaries neither at the starts nor the ends
    but the first; the fifth prompt's 20 positions from 66 do not fit the 80), and a repeated prompt is loaded from
    there instead of prefilled. One slot, so every run of a prompt has the same schedule: the loaded runs
    must give exactly the prefilled runs' tokens (greedy and seeded sampling), and the first runs match the CPU
    model."""
    print("native decoder: unaligned prompt store", flush=True)
    model = RandomModel(TINY, gpu, seed=81)
    rng = np.random.default_rng(82)
    prompts = [[BOS] + rng.integers(8, TINY.vocab, n).tolist() for n in (5, 18, 32, 11, 20)]
    reqs = [Request(input_ids=ids, max_new_tokens=6, temperature=0.0 if k % 2 == 0 else 0.9, seed=90 + k)
            for k, ids in enumerate(prompts)]
    dec = NativeDecoder(model, bos=BOS, max_length=48, prompt_store=80, batch=1)
    first = dict(dec.generate(reqs))
    assert dec.loads == 0
    assert dec.stored == {tuple(p): at for p, at in zip(prompts[:4], (0, 5, 23, 55))}  # the fifth does not fit
    again = dict(dec.generate(list(reversed(reqs))))
    assert dec.loads == 4
    for k in range(5):
        assert again[4 - k] == first[k], (k, first[k], again[4 - k])
    checked = sum(check_alone(model, k, r, first[k]) for k, r in enumerate(reqs))
    assert checked >= 12, checked


def test_torch_server_store_at_unaligned_positions(gpu):
    """The torch-driven server's store is position-granular too (the same PromptStore offsets, rows moved by
    nc_kv_export_fp8 / nc_kv_import_fp8): loaded runs equal prefilled runs."""
    from nanochat_amd.serving import Server

    print("torch server: unaligned prompt store", flush=True)
    model = RandomModel(TINY, gpu, seed=83)
    rng = np.random.default_rng(84)
    prompts = [[BOS] + rng.integers(8, TINY.vocab, n).tolist() for n in (9, 26, 3)]
    reqs = [Request(input_ids=ids, max_new_tokens=5) for ids in prompts]
    server = Server(model, batch=1, max_len=48, device=gpu, bos=BOS, prompt_store=40)
    first = dict(server.generate(reqs))
    assert server.stored == {tuple(prompts[0]): 0, tuple(prompts[1]): 9, tuple(prompts[2]): 35}
    again = dict(server.generate(reqs))
    assert server.loads == 3
    assert again == first


def test_handle_tokens_equal_the_torch_decoder(gpu):
    """The handle and the torch-driven decoder (Fp8Decoder) run the same kernels on the same rows in the same order,
    so their greedy tokens are bit-identical: 64 prompts of 260 tokens (16576 prefill rows: two dec_prefill calls of
    at most dec_prefill_rows() rows against one attention call per layer in the torch decoder; the split falls on
    a tile boundary), then 8 steps driven the way the reference's loop drives them."""
    model = RandomModel(ModelConfig(layers=2, d_model=256, heads=2, vocab=1000), gpu, seed=23)
    B, T, steps = 64, 260, 8
    ids = np.random.default_rng(24).integers(0, 1000, (B, T)).astype(np.int32)
    prompts = torch.from_numpy(ids).to(gpu)
    ref = Fp8Decoder(model, B, T - 1 + steps, gpu)
    ref.prefill(prompts)
    ref.start(prompts[:, -1], T - 1)
    ref.run(steps)
    want = ref.tokens(steps).cpu().numpy()
    nd = NativeDecoder(model, bos=-1, max_length=T - 1 + steps, batch=B)
    lib, h = nd.lib, nd.handle
    for b in range(B):
        lib.dec_set_prompt(h, b, int(ids[b, -1]), T - 1, 0.0, 1.0, 0)
    rows = prompt_rows([(b, ids[b].tolist()) for b in range(B)])
    assert rows.shape[1] > nd.rows_per_call
    for lo in range(0, rows.shape[1], nd.rows_per_call):
        part = np.ascontiguousarray(rows[:, lo:lo + nd.rows_per_call])
        lib.dec_prefill(h, part.shape[1], part.ctypes.data)
    words = np.ascontiguousarray(slot_masks([True] * B))
    lib.dec_set_active(h, words.ctypes.data)
    out = np.empty(2 * B, dtype=np.int32)
    got = np.empty((steps, B), dtype=np.int32)
    for i in range(steps):
        lib.dec_launch_body(h)
        lib.dec_launch_head(h)
        lib.dec_tokens(h, out.ctypes.data)
        got[i] = out[:B]
    np.testing.assert_array_equal(got.T, want)
