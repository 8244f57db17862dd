"""Seeded random sweeps against the same bars as the fixed-shape tests, through their own check functions:

- decode attention, the fused decode step and chunked prefill against the oracle (batch, GQA group, per-sequence
  contexts, paging, windows, outliers): q rows and cache bytes bit-exact, the fused step bit-identical to the append
  followed by decode attention, attention within max abs 2e-2 and mean 2e-3 of fp64;
- the slot GEMM against its fp32 torch restatement (rows, weight rows, K, epilogue): within its bf16 rounding bound,
  and each row's bits the same when the row is computed alone;
- the token choice against oracle/sampling.py (slots, vocabulary, padding, logit cap, lazy token): the same tokens,
  alternatives and positions.

The configurations come from fixed generators; sizes keep each oracle call to a few seconds."""

import numpy as np
import pytest
import torch

import test_gpu_decode as D
import test_gpu_slot_gemm as GM
import test_gpu_prefill as P
import test_gpu_sampling as C
import test_gpu_step as S
from nanochat_amd.slot_gemm import NORM_F32, NORM_STORE, RELU2_NORM, RESID, STORE, slot_gemm
from nanochat_amd.workloads import DecodeConfig, PrefillConfig

pytestmark = pytest.mark.gpu

GROUPS = (1, 2, 3, 4, 5, 8, 16)


def _window(rng, top):
    return -1 if rng.random() < 0.5 else int(rng.integers(1, top))


def decode_cases(n: int, seed: int) -> list[DecodeConfig]:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        hkv = int(rng.choice((1, 2, 3, 4)))
        g = int(rng.choice(GROUPS))
        batch = int(rng.integers(1, 41))
        lo = int(rng.integers(0, 2000))
        hi = lo + int(rng.integers(0, 2500))
        window = _window(rng, 1500)
        paged = bool(rng.integers(0, 2))
        outliers = 0.01 if rng.random() < 0.3 else 0.0
        name = f"s{seed}-{i}-b{batch}-h{g * hkv}/{hkv}-ctx{lo}..{hi}-w{window}{'-paged' if paged else ''}"
        cases.append(DecodeConfig(name, batch, g * hkv, hkv, ctx_range=(lo, hi), paged=paged, outliers=outliers,
                                  window=window, seed=seed * 100 + i))
    return cases


def prefill_cases(n: int, seed: int) -> list[PrefillConfig]:
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        hkv = int(rng.choice((1, 2, 4)))
        g = int(rng.choice(GROUPS))
        batch = int(rng.integers(1, 5))
        cached = tuple(int(rng.integers(0, 1200)) for _ in range(batch))
        chunk = tuple(int(rng.integers(1, 130)) for _ in range(batch))
        window = _window(rng, 600)
        paged = bool(rng.integers(0, 2))
        outliers = 0.01 if rng.random() < 0.3 else 0.0
        name = f"s{seed}-{i}-b{batch}-h{g * hkv}/{hkv}-w{window}{'-paged' if paged else ''}"
        cases.append(PrefillConfig(name, batch, g * hkv, hkv, cached=cached, chunk=chunk, paged=paged,
                                   outliers=outliers, window=window, seed=seed * 100 + i))
    return cases


def gemm_cases(n: int, seed: int) -> list[tuple[int, int, int, int]]:
    """(m, n, k, epilogue): m on both sides of the many-rows switch (512 rows)."""
    rng = np.random.default_rng(seed)
    epis = (STORE, NORM_STORE, RESID, RELU2_NORM, NORM_F32)
    return [(int(rng.integers(1, 800)), 32 * int(rng.integers(1, 81)), 64 * int(rng.integers(1, 41)),
             int(rng.choice(epis))) for _ in range(n)]


def choose_cases(n: int, seed: int) -> list[tuple[int, int, int, int, float, int]]:
    """(slots, vocabulary, case seed, padded columns, logit cap, lazy token or -1)."""
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        V = int(rng.integers(2, 70000))
        cases.append((int(rng.integers(1, 300)), V, seed * 100 + i, int(rng.choice((0, 0, 7, 32))),
                      float(rng.choice((0.0, 15.0, 30.0))), int(rng.integers(0, V)) if rng.random() < 0.5 else -1))
    return cases


DECODE = decode_cases(24, 2024)
STEP = decode_cases(16, 2025)
PREFILL = prefill_cases(16, 2026)
GEMM = gemm_cases(24, 2027)
CHOOSE = choose_cases(12, 2028)


@pytest.mark.parametrize("cfg", DECODE, ids=[c.name for c in DECODE])
def test_decode_sweep(gpu, cfg):
    D.run_and_check(cfg, gpu, check_append_rows=1)


@pytest.mark.parametrize("cfg", STEP, ids=[c.name for c in STEP])
def test_fused_step_sweep(gpu, cfg):
    S.test_step_equals_append_then_decode(gpu, cfg)


@pytest.mark.parametrize("cfg", PREFILL, ids=[c.name for c in PREFILL])
def test_prefill_sweep(gpu, cfg):
    P.run_and_check(cfg, gpu, check_append=True)


@pytest.mark.parametrize("m, n, k, epi", GEMM, ids=[f"m{m}-n{n}-k{k}-e{e}" for m, n, k, e in GEMM])
def test_slot_gemm_sweep(gpu, m, n, k, epi):
    print(f"slot gemm m {m} n {n} k {k} epilogue {epi}", flush=True)
    x, w, res = GM.data(m, n, k, gpu, seed=m * 31 + n * 7 + k)
    got = slot_gemm(x, w, epi, res=res if epi == RESID else None)
    torch.cuda.synchronize()
    GM.check(got, GM.reference(x, w, epi, res), f"m {m} n {n} k {k} epi {epi}")
    rows = min(m, 7)  # the same rows alone: a row's bits do not depend on the rows computed with it
    alone = slot_gemm(x[:rows].contiguous(), w, epi, res=res[:rows].contiguous() if epi == RESID else None)
    torch.cuda.synchronize()
    assert torch.equal(alone, got[:rows]), "a row's result depends on the rows computed with it"


@pytest.mark.parametrize("B, V, seed, pad, softcap, lazy", CHOOSE,
                         ids=[f"b{b}-v{v}-pad{p}-cap{c:g}-lazy{z}" for b, v, _, p, c, z in CHOOSE])
def test_choose_sweep(gpu, B, V, seed, pad, softcap, lazy):
    print(f"choose B {B} V {V} seed {seed} pad {pad} softcap {softcap} lazy {lazy}", flush=True)
    c = C.make_case(B, V, seed, pad)
    (tok, alt, pos), (wt, wa, wp) = C.run_both(c, gpu, softcap=softcap, lazy=lazy)
    act = c["active"]
    np.testing.assert_array_equal(tok[act], wt[act])
    np.testing.assert_array_equal(alt[act], wa[act])
    np.testing.assert_array_equal(pos, wp)
    assert (tok[~act] == -2).all() and (alt[~act] == -2).all()
