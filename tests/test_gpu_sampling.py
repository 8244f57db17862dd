"""GPU parity of the token choice (nc_choose_tokens) against the oracle (oracle/sampling.py): the same tokens,
alternatives and committed positions for greedy, temperature, nucleus, masked, inactive and empty-mask slots."""

import numpy as np
import pytest
import torch

from nanochat_amd.sampling import allow_rows, choose_tokens, slot_masks
from oracle import sampling as S

pytestmark = pytest.mark.gpu


def make_case(B, V, seed, ld_pad=0):
    rng = np.random.default_rng(seed)
    logits = (rng.standard_normal((B, V + ld_pad)) * 3).astype(np.float32)
    temperature = rng.choice(np.array([0.0, 0.5, 1.0, 2.0], np.float32), size=B)
    top_p = rng.choice(np.array([1.0, 1.0, 0.9, 0.5, 0.0], np.float32), size=B)
    seeds = rng.integers(0, 2 ** 63, size=B, dtype=np.int64).astype(np.uint64) * np.uint64(2) + np.uint64(1)
    first = rng.integers(0, 100, size=B).astype(np.int32)
    pos = (first + rng.integers(0, 500, size=B)).astype(np.int32)
    active = rng.random(B) < 0.85
    masked = rng.random(B) < 0.3
    allowed = rng.random((B, V)) < rng.choice([0.002, 0.3, 0.9], size=(B, 1))
    allowed[0] = False  # slot 0 allows nothing (masked below)
    masked[0] = active[0] = True
    return dict(logits=logits, V=V, temperature=temperature, top_p=top_p, seed=seeds, first=first, pos=pos,
                active=active, masked=masked, allowed=allowed)


def run_both(c, dev, softcap=15.0, lazy=0):
    V = c["V"]
    words = allow_rows(c["allowed"])
    want_tok, want_alt, want_pos = S.choose(
        c["logits"][:, :V], temperature=c["temperature"], top_p=c["top_p"], seed=c["seed"], pos=c["pos"],
        first=c["first"], active=c["active"], masked=c["masked"], allow=words.view(np.uint32), softcap=softcap,
        lazy=lazy)
    t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(dev).to(dt)
    pos = t(c["pos"], torch.int32)
    tokens = torch.full((len(pos),), -2, dtype=torch.int32, device=dev)
    alts = torch.full((len(pos),), -2, dtype=torch.int32, device=dev)
    choose_tokens(t(c["logits"], torch.float32), V, pos, temperature=t(c["temperature"], torch.float32),
                  top_p=t(c["top_p"], torch.float32), seed=t(c["seed"].view(np.int64), torch.int64),
                  first=t(c["first"], torch.int32), slots=t(slot_masks(c["active"], c["masked"]), torch.int64),
                  allow=t(words, torch.int32), softcap=softcap, lazy=lazy, tokens=tokens, alt_tokens=alts)
    torch.cuda.synchronize()
    return (tokens.cpu().numpy(), alts.cpu().numpy(), pos.cpu().numpy()), (want_tok, want_alt, want_pos)


@pytest.mark.parametrize("B, V, seed, pad, softcap", [
    (64, 65536, 1, 0, 15.0),   # config 5's vocabulary
    (7, 1000, 2, 24, 15.0),    # a vocabulary that is not a multiple of 32, padded rows
    (33, 50257, 3, 0, 0.0),    # no logit cap
    (130, 4096, 4, 0, 30.0),   # more slots than one mask word
])
def test_choose_matches_the_oracle(gpu, B, V, seed, pad, softcap):
    print(f"choose case B {B} V {V} seed {seed}", flush=True)
    c = make_case(B, V, seed, pad)
    (tok, alt, pos), (wt, wa, wp) = run_both(c, gpu, softcap=softcap)
    act = c["active"]
    np.testing.assert_array_equal(tok[act], wt[act])
    np.testing.assert_array_equal(alt[act], wa[act])
    np.testing.assert_array_equal(pos, wp)
    assert (tok[~act] == -2).all() and (alt[~act] == -2).all()  # inactive slots untouched
    assert tok[0] == -1  # nothing allowed


def test_greedy_without_masks_or_sampling_arguments(gpu):
    """Defaults: every slot active, temperature 0: the first argmax, as nc_argmax_f32."""
    rng = np.random.default_rng(5)
    x = (rng.standard_normal((9, 3000)) * 2).astype(np.float32)
    x[4, 100] = x[4, 2000] = 50.0
    logits = torch.from_numpy(x).to(gpu)
    pos = torch.arange(9, dtype=torch.int32, device=gpu)
    tok, alt = choose_tokens(logits, 3000, pos, lazy=int(np.argmax(x[2])))
    torch.cuda.synchronize()
    assert np.array_equal(tok.cpu().numpy(), np.argmax(x, axis=1))
    assert tok[4].item() == 100
    x2 = x[2].copy()
    x2[np.argmax(x[2])] = -np.inf
    assert alt[2].item() == int(np.argmax(x2))
    assert np.array_equal(pos.cpu().numpy(), np.arange(9) + 1)


def test_sampling_is_reproducible_and_follows_the_index(gpu):
    """The same (seed, pos - first) gives the same token; a later position draws fresh noise."""
    c = make_case(16, 8192, 6)
    c["active"][:] = True
    c["masked"][:] = False
    c["temperature"][:] = 1.0
    c["top_p"][:] = 1.0
    (t1, _, _), _ = run_both(c, gpu)
    (t2, _, _), _ = run_both(c, gpu)
    assert np.array_equal(t1, t2)
    c["pos"] = c["pos"] + 1
    (t3, _, _), (w3, _, _) = run_both(c, gpu)
    assert np.array_equal(t3, w3)
    assert not np.array_equal(t1, t3)
