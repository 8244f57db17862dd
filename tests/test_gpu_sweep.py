"""Seeded random sweeps of decode attention, the fused decode step and chunked prefill against the oracle, and of
the slot GEMM against its fp32 torch restatement. The configurations come from a fixed generator: batch, GQA group,
per-sequence contexts, paging, windows and outliers; for the GEMM, rows, weight rows, K and the epilogue. Each one is
held to the fixed-shape tests' bars through their own check functions. For the append, q rows and cache
bytes are bit-exact. The fused step is bit-identical to the append followed by decode attention. Attention is within
max abs 2e-2 and mean 2e-3 of fp64. The GEMM is within its bf16 rounding bound, and each row's bits are the same when
the row is computed alone. Sizes keep each oracle call to a few seconds."""

import numpy as np
import pytest
import torch

import test_gpu_decode as D
import test_gpu_slot_gemm as GM
import test_gpu_prefill as P
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


DECODE = decode_cases(24, 2024)
STEP = decode_cases(16, 2025)
PREFILL = prefill_cases(16, 2026)
GEMM = gemm_cases(24, 2027)


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
