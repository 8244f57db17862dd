"""Continuous batching (serving.Server, the reference's NativeDecoder.generate protocol): more requests than slots,
mixed prompt lengths, greedy and sampled, a masked request, BOS and stopping criteria. Every request's tokens are
checked against a CPU restatement of the model run on that request alone (the decoder test's CpuModel): at each
generated position the CPU logits' choice (greedy, or Gumbel-max with the request's seed and generated index) must
equal the served token wherever the choice is clear of the logit tolerance."""

import numpy as np
import pytest

from nanochat_amd.decoder import RandomModel
from nanochat_amd.serving import Request, Server
from oracle import sampling as S
from oracle.model import CpuModel
from test_gpu_decoder import LOGIT_ATOL, TINY

pytestmark = pytest.mark.gpu

BOS = 7


def expected_choice(logits, r: Request, i: int, allowed):
    """The oracle's choice on CPU logits, and whether it is clear of the tolerance."""
    x = logits.astype(np.float32)
    if allowed is not None:
        x = np.where(allowed, x, -np.inf).astype(np.float32)
    if r.temperature > 0:
        score = S.capped(x, 15.0) / np.float32(r.temperature) + S.gumbel(r.seed, i, np.arange(len(x)))
        tol = 2 * LOGIT_ATOL / r.temperature
    else:
        score, tol = x, 2 * LOGIT_ATOL
    top2 = np.sort(score)[-2:]
    return int(np.argmax(score)), bool(top2[1] - top2[0] > tol)


def test_continuous_batching_matches_each_request_alone(gpu):
    model = RandomModel(TINY, gpu, seed=21)
    rng = np.random.default_rng(22)
    lens, news = [6, 12, 25, 9, 30, 4, 17], [5, 3, 6, 8, 2, 7, 4]
    temps = [0.0, 0.0, 0.8, 0.0, 1.2, 0.0, 0.5]
    even = np.arange(TINY.vocab) % 2 == 0
    reqs = []
    for k, (n, m, t) in enumerate(zip(lens, news, temps)):
        ids = [BOS] + rng.integers(8, TINY.vocab, n - 1).tolist()
        mask = (lambda out: even) if k == 3 else None
        stop = (lambda out: len(out) >= 2 and out[-1] == out[-2]) if k == 1 else None
        reqs.append(Request(input_ids=ids, max_new_tokens=m, temperature=t, seed=1000 + k, mask=mask,
                            stopping_criteria=stop))
    server = Server(model, batch=3, max_len=48, device=gpu, bos=BOS)
    got = dict(server.generate(reqs))
    assert sorted(got) == list(range(len(reqs)))
    checked = sum(check_alone(model, k, r, got[k], even) for k, r in enumerate(reqs))
    assert checked >= 25, checked


def check_alone(model, k, r: Request, out, allowed=None) -> int:
    """Request k's served tokens against a CPU run of that request alone; returns how many choices were clear of
    the tolerance (and so checked)."""
    assert 1 <= len(out) + (len(out) < r.max_new_tokens) and len(out) <= r.max_new_tokens
    if r.mask is not None:
        assert all(allowed[t] for t in out)
    cpu = CpuModel(model, 1, 48)
    ids = np.array(r.input_ids, np.int32)
    cpu.prefill(ids[None])
    tok, p = ids[-1:], len(ids) - 1
    stopped_early = len(out) < r.max_new_tokens and not (r.stopping_criteria and r.stopping_criteria(out))
    checked = 0
    for i in range(len(out) + stopped_early):
        logits = cpu.step(tok, p)[0]
        want, sure = expected_choice(logits, r, i, allowed if r.mask is not None else None)
        served = out[i] if i < len(out) else BOS
        if sure:
            assert served == want, (k, i, served, want)
            checked += 1
        tok, p = np.array([served], np.int32), p + 1
    return checked


def test_narrow_graph_serves_the_low_slots(gpu):
    """batch 128 with a narrow graph over the first 64 slots (decode.cu:995-1005): while slots 64 and 65 are busy
    the full graph runs, afterwards the narrow one; requests on both sides of the boundary decode as alone."""
    model = RandomModel(TINY, gpu, seed=41)
    rng = np.random.default_rng(42)
    reqs = [Request(input_ids=[BOS] + rng.integers(8, TINY.vocab, 5 + k % 7).tolist(),
                    max_new_tokens=2 if k >= 64 else 6, temperature=0.7 if k % 3 == 0 else 0.0, seed=500 + k)
            for k in range(66)]
    server = Server(model, batch=128, max_len=48, device=gpu, bos=BOS, narrow=64)
    got = dict(server.generate(reqs))
    assert sorted(got) == list(range(len(reqs)))
    assert 0 < server.narrow_steps < server.steps, (server.narrow_steps, server.steps)
    checked = sum(check_alone(model, k, reqs[k], got[k]) for k in (0, 1, 2, 62, 63, 64, 65))
    assert checked >= 20, checked


def test_prompt_store_loads_instead_of_prefilling(gpu):
    """A repeated prompt is loaded from the pinned prompt store (decode.cu:1053-1075) instead of prefilled, and
    decodes exactly as the first time (one slot: the same schedule every step); a prompt past the store's room is
    prefilled each time."""
    model = RandomModel(TINY, gpu, seed=31)
    rng = np.random.default_rng(32)
    a = [BOS] + rng.integers(8, TINY.vocab, 37).tolist()   # 38 tokens: 37 cached prompt positions
    b = [BOS] + rng.integers(8, TINY.vocab, 20).tolist()
    big = [BOS] + rng.integers(8, TINY.vocab, 40).tolist()
    reqs = [Request(input_ids=ids, max_new_tokens=5) for ids in (a, b, a, big, a, big)]
    server = Server(model, batch=1, max_len=48, device=gpu, bos=BOS, prompt_store=5 * 16)
    out = dict(server.generate(reqs))
    assert server.loads == 2          # a twice; b stored too (positions 37..56), big (40) no longer fits in 80
    assert set(server.stored) == {tuple(a), tuple(b)}
    assert out[0] == out[2] == out[4]
    assert out[3] == out[5]
    plain = Server(model, batch=1, max_len=48, device=gpu, bos=BOS)
    assert dict(plain.generate(reqs[:1]))[0] == out[0]


def test_rejected_bos_takes_the_alternative(gpu):
    """Masks allowing only BOS and one token x, and a request that never accepts BOS: every chosen BOS gives way to
    the choice's alternative, so the continuation is x repeated to max_new_tokens."""
    model = RandomModel(TINY, gpu, seed=41)
    rng = np.random.default_rng(42)
    reqs = []
    for k in range(6):
        allowed = np.zeros(TINY.vocab, bool)
        x = 100 + 37 * k
        allowed[[BOS, x]] = True
        reqs.append(Request(input_ids=[BOS] + rng.integers(8, TINY.vocab, 12).tolist(), max_new_tokens=4,
                            mask=lambda out, m=allowed: m, accept_bos=lambda out: False))
    server = Server(model, batch=3, max_len=32, device=gpu, bos=BOS)
    out = dict(server.generate(reqs))
    for k in range(6):
        assert out[k] == [100 + 37 * k] * 4, (k, out[k])
    assert server.alts_taken > 0
