"""GPU parity of the skinny weight GEMM (nc_slot_gemm_bf16) against an fp32 torch restatement of each epilogue:
bf16 outputs within one bf16 rounding of the fp32 result, fp32 logits within fp32 summation-order error; every work
tile; batch rows that do not fill a tile; the in-place residual update; and bitwise-repeatable results."""

import pytest
import torch

from nanochat_amd.slot_gemm import NORM_F32, NORM_STORE, RELU2_NORM, RESID, STORE, slot_gemm

pytestmark = pytest.mark.gpu

EPS = torch.finfo(torch.float32).eps
TILES = [(32, 32), (64, 32), (32, 64), (64, 64), (32, 128), (64, 128), (128, 64), (128, 128)]


def data(m, n, k, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    x = torch.randn((m, k), generator=g, device=dev).to(torch.bfloat16)
    w = (0.02 * torch.randn((n, k), generator=g, device=dev)).to(torch.bfloat16)
    res = torch.randn((m, n), generator=g, device=dev).to(torch.bfloat16)
    return x, w, res


def reference(x, w, epi, res):
    """The epilogue in fp32 over fp32 sums (torch fp32 GEMM on the same bf16 values)."""
    s = torch.mm(x.float(), w.float().t())
    r = torch.rsqrt(x.float().square().mean(1, keepdim=True) + EPS)
    if epi == STORE:
        return s
    if epi == NORM_STORE:
        return s * r
    if epi == RESID:
        return s + res.float()
    if epi == RELU2_NORM:
        p = s * r
        return p.clamp_min(0) * p
    return s * r


def check(got, want, label):
    """bf16 outputs: within one bf16 rounding (2^-8 relative) of the fp32 value, plus a floor for values near 0 where
    summation order decides; fp32 outputs: summation-order error only."""
    scale = want.abs().max().item()
    if got.dtype == torch.bfloat16:
        torch.testing.assert_close(got.float(), want, rtol=2 ** -7, atol=2 ** -12 * scale, msg=label)
    else:
        torch.testing.assert_close(got, want, rtol=1e-4, atol=1e-5 * scale, msg=label)


@pytest.mark.parametrize("m, n, k", [
    (128, 4992, 1664),   # config 5 qkv
    (128, 1664, 1664),   # o
    (128, 6656, 1664),   # up
    (128, 1664, 6656),   # down
    (1, 32, 64),
    (5, 64, 64),
    (9, 96, 128),        # two chunks: fewer than the ring holds
    (37, 224, 192),
    (200, 96, 320),
])
@pytest.mark.parametrize("epi", [STORE, NORM_STORE, RESID, RELU2_NORM, NORM_F32])
def test_epilogues_and_shapes(gpu, m, n, k, epi):
    x, w, res = data(m, n, k, gpu, seed=m * 7 + n + k)
    got = slot_gemm(x, w, epi, res=res if epi == RESID else None)
    torch.cuda.synchronize()
    check(got, reference(x, w, epi, res), f"m {m} n {n} k {k} epi {epi}")


@pytest.mark.parametrize("tile", TILES)
def test_every_tile(gpu, tile):
    m, n, k = 70, 256, 384  # 70 rows: partial slices for every tile height
    x, w, res = data(m, n, k, gpu, seed=11)
    for epi in (STORE, RELU2_NORM, RESID):
        got = slot_gemm(x, w, epi, res=res if epi == RESID else None, tile=tile)
        torch.cuda.synchronize()
        check(got, reference(x, w, epi, res), f"tile {tile} epi {epi}")


def test_lm_head_logits(gpu):
    m, n, k = 128, 65536, 1664
    x, w, _ = data(m, n, k, gpu, seed=5)
    got = slot_gemm(x, w, NORM_F32)
    torch.cuda.synchronize()
    check(got, reference(x, w, NORM_F32, None), "lm_head")


def test_resid_in_place_and_repeatable(gpu):
    m, n, k = 128, 1664, 1664
    x, w, res = data(m, n, k, gpu, seed=3)
    want = reference(x, w, RESID, res)
    h = res.clone()
    slot_gemm(x, w, RESID, res=h, out=h)
    torch.cuda.synchronize()
    check(h, want, "in place")
    again = slot_gemm(x, w, RESID, res=res)
    torch.cuda.synchronize()
    assert torch.equal(again, h)  # same bits, call after call


@pytest.mark.parametrize("m, n, k", [
    (1000, 1664, 1664),   # o / a prefill chunk of the decoder handle: partial x and W tiles
    (600, 4992, 1664),    # qkv
    (2100, 6656, 1664),   # up
    (513, 1664, 6656),    # down, one row past a tile
    (700, 128, 320),      # 5 K chunks (an odd count) and a single partial W tile
])
@pytest.mark.parametrize("epi", [STORE, NORM_STORE, RESID, RELU2_NORM, NORM_F32])
def test_many_rows_equal_the_decode_tiles(gpu, m, n, k, epi):
    """From 512 rows on the automatic tile is the many-rows kernel (256 x 256 tiles): every output bit equals the
    decode kernel's (a forced 64 x 128 tile) for the same rows, so a row's result does not depend on how many rows
    were computed with it; and both are within the epilogue's tolerance of fp32."""
    x, w, res = data(m, n, k, gpu, seed=m + 3 * n + k + epi)
    r = res if epi == RESID else None
    got = slot_gemm(x, w, epi, res=r)
    want = slot_gemm(x, w, epi, res=r, tile=(64, 128))
    torch.cuda.synchronize()
    assert torch.equal(got, want), (got.float() - want.float()).abs().max()
    check(got, reference(x, w, epi, res), f"many rows m {m} n {n} k {k} epi {epi}")


def test_many_rows_in_place_residual(gpu):
    m, n, k = 777, 1664, 1664
    x, w, res = data(m, n, k, gpu, seed=21)
    want = slot_gemm(x, w, RESID, res=res)
    h = res.clone()
    slot_gemm(x, w, RESID, res=h, out=h)
    torch.cuda.synchronize()
    assert torch.equal(h, want)


@pytest.mark.parametrize("m, n, k, pf_bytes", [
    (128, 4992, 1664, 1664 * 1664 * 2),  # config 5 qkv, prefetching W_o
    (128, 6656, 1664, 1664 * 6656 * 2),  # up, prefetching W_down
    (128, 1664, 6656, 4992 * 1664 * 2),  # down, prefetching the next W_qkv
    (37, 224, 192, 65536 * 3 + 4096),    # whole 64 KiB blocks and a remainder that is skipped
    (5, 64, 64, 60000),                  # under one block: nothing read
    (600, 1664, 1664, 1664 * 1664 * 2),  # the many-rows tile: nothing read
])
@pytest.mark.parametrize("epi", [NORM_STORE, RESID, RELU2_NORM])
def test_prefetch_leaves_the_result_bit_identical(gpu, m, n, k, pf_bytes, epi):
    """nc_slot_gemm_bf16_prefetch: the workgroups past the tiles read the prefetch range on the idle compute units;
    the GEMM's outputs equal nc_slot_gemm_bf16's bit for bit, in place (RESID) too."""
    x, w, res = data(m, n, k, gpu, 41)
    pf = torch.randint(0, 1 << 15, (pf_bytes // 2,), dtype=torch.int16, device=gpu)
    if epi == RESID:
        r1, r2 = res.clone(), res.clone()
        plain = slot_gemm(x, w, epi, res=r1, out=r1)
        fetched = slot_gemm(x, w, epi, res=r2, out=r2, prefetch=pf)
    else:
        plain = slot_gemm(x, w, epi)
        fetched = slot_gemm(x, w, epi, prefetch=pf)
    torch.cuda.synchronize()
    assert torch.equal(plain.view(torch.int16), fetched.view(torch.int16))
