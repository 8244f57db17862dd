"""Test helpers: move GPU tensors into the oracle's numpy structures, and the attention tolerance of the
benchmark contract (max abs err <= 2e-2, mean <= 2e-3 against the fp64 oracle)."""

import numpy as np
import torch

from oracle import golden as G

MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 numpy bits."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def oracle_cache(cache) -> G.PagedCache:
    c = G.PagedCache(cache.num_blocks, cache.hkv)
    c.pages[...] = cache.pages.cpu().numpy()
    return c


def table(cache):
    return None if cache.block_table is None else cache.block_table.cpu().numpy()


def assert_same_cache(gpu_cache, ref: G.PagedCache) -> None:
    """Every byte of the pool: codes and the scales' fp32 bit patterns."""
    got = gpu_cache.pages.cpu().numpy()
    regions = {"k codes [block][head][key][dim]": G.K_BYTES, "v codes [block][head][key][dim]": G.V_BYTES,
               "k scales": np.arange(4096, 4160), "v scales": np.arange(4160, 4224)}
    for name, at in regions.items():  # name the region that differs first
        np.testing.assert_array_equal(got[..., at], ref.pages[..., at], name)
    np.testing.assert_array_equal(got, ref.pages)


def attention_error(got: torch.Tensor, want: np.ndarray) -> tuple[float, float]:
    g = G.bf16_to_f32(bits(got)).astype(np.float64)
    assert not np.isnan(g).any(), "NaN in the GPU output"
    err = np.abs(g - want)
    return float(err.max()), float(err.mean())


def assert_attention_close(got: torch.Tensor, want: np.ndarray, label: str = "") -> tuple[float, float]:
    mx, mean = attention_error(got, want)
    print(f"{label} max abs err {mx:.3e} mean {mean:.3e}", flush=True)
    assert mx <= MAX_ABS and mean <= MEAN_ABS, (label, mx, mean)
    return mx, mean
