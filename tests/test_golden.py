"""The frozen fixtures of tests/golden: the oracle still produces them (CPU), and the HIP path reproduces their cache
bytes and q bits exactly and their attention outputs within the benchmark tolerance (GPU, through the C ABI)."""

import os
import sys

import numpy as np
import pytest
import torch

from helpers import assert_attention_close, bits

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, HERE)

import make_golden  # noqa: E402


def load(name):
    with np.load(os.path.join(HERE, name), allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_oracle_reproduces_fixture(name):
    want = load(name)
    got = make_golden.FIXTURES[name]()
    assert set(got) == set(want)
    for k in want:
        np.testing.assert_array_equal(np.asarray(got[k]), want[k], err_msg=k)


def to_dev(a, dev, dtype=None):
    t = torch.from_numpy(np.ascontiguousarray(a))
    return t.to(dev) if dtype is None else t.view(dtype).to(dev)


def gpu_cache(fx, dev, paged):
    from nanochat_amd.kv_cache import Fp8KVCache

    hkv, mb = int(fx["hkv"]), int(fx["max_blocks"])
    if paged:
        cache = Fp8KVCache.paged(to_dev(fx["table"], dev), fx["cache_in"].shape[0], hkv)
    else:
        cache = Fp8KVCache.contiguous(fx["cache_in"].shape[0] // mb, mb * 16, hkv, dev)
    cache.pages.copy_(to_dev(fx["cache_in"], dev))
    return cache


@pytest.mark.gpu
def test_decode_fixture_on_gpu(gpu):
    from nanochat_amd.attention import decode_attention
    from nanochat_amd.rotary import rotary_tables

    fx = load("decode_small.npz")
    dev = gpu
    cache = gpu_cache(fx, dev, paged=True)
    cos, sin = rotary_tables(int(fx["rope_len"]), float(fx["theta"]), dev)
    pos = to_dev(fx["pos"], dev)
    q = cache.append(to_dev(fx["qkv"], dev, torch.bfloat16), pos, torch.zeros(1, dtype=torch.int32, device=dev),
                     to_dev(fx["q_gain"], dev), to_dev(fx["k_gain"], dev), cos, sin, int(fx["hq"]))
    out = decode_attention(q, cache, pos + 1, max_ctx=cache.capacity)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(q), fx["q_out"])
    np.testing.assert_array_equal(cache.pages.cpu().numpy(), fx["cache_out"])
    assert_attention_close(out, fx["attn"], "decode fixture")


@pytest.mark.gpu
def test_prefill_fixture_on_gpu(gpu):
    from nanochat_amd.attention import prefill_attention
    from nanochat_amd.rotary import rotary_tables

    fx = load("prefill_small.npz")
    dev = gpu
    cache = gpu_cache(fx, dev, paged=False)
    cos, sin = rotary_tables(int(fx["rope_len"]), float(fx["theta"]), dev)
    pos, seq = to_dev(fx["pos"], dev), to_dev(fx["seq"], dev)
    q = cache.append(to_dev(fx["qkv"], dev, torch.bfloat16), pos, seq, to_dev(fx["q_gain"], dev),
                     to_dev(fx["k_gain"], dev), cos, sin, int(fx["hq"]))
    out = prefill_attention(q, cache, pos, seq, window=int(fx["window"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(bits(q), fx["q_out"])
    np.testing.assert_array_equal(cache.pages.cpu().numpy(), fx["cache_out"])
    assert_attention_close(out, fx["attn"], "prefill fixture")
