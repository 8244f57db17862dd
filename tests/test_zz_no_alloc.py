"""nc_decode_step_fp8_noalloc (the fused decode step over the library's static scratch, for callers that cannot
allocate) against nc_decode_step_fp8 with a workspace: bit-identical outputs, cache bytes and next positions, on
two calls in a row where the second is smaller (the scratch keeps the first call's partial results), called through
the C ABI."""

import math

import numpy as np
import pytest
import torch

from helpers import bits
from nanochat_amd.native import check, hip_library, pointer, stream
from nanochat_amd.attention import decode_workspace
from nanochat_amd.workloads import CONFIG3, DecodeConfig, build_decode_case

pytestmark = pytest.mark.gpu

SCALE = 1 / math.sqrt(128)


def _step(lib, case, cfg, max_ctx, noalloc, ws):
    c = case.cache
    qkv = case.qkv[0]
    pos = case.positions(0)
    out = torch.empty((cfg.batch, cfg.hq, 128), dtype=torch.bfloat16, device=qkv.device)
    pos_out = torch.empty_like(pos)
    args = [pointer(qkv), qkv.stride(0), pointer(pos), pointer(pos_out), pointer(case.q_gain), pointer(case.k_gain),
            pointer(case.cos), pointer(case.sin), case.cos.shape[0], pointer(c.pages), pointer(c.block_table),
            c.max_blocks, c.num_blocks, cfg.window, cfg.batch, cfg.hq, cfg.hkv, max_ctx, SCALE, pointer(out)]
    if noalloc:
        check(lib.nc_decode_step_fp8_noalloc(*args, stream()))
    else:
        check(lib.nc_decode_step_fp8(*args, pointer(ws), ws.numel(), stream()))
    return out, pos_out


SHAPES = [CONFIG3, DecodeConfig("small-after-large", 5, 8, 2, ctx_range=(3, 900), paged=True, window=300, seed=97)]


def test_scratch_is_reserved_by_the_noalloc_entry_alone(gpu):
    """The 64 MiB scratch lives in a code object of its own: the decode entries leave it unloaded, and the first
    no-allocation call on a device loads it (no other test calls that entry, so this one runs first in any run).
    Every tensor exists before the device's free memory is read."""
    lib = hip_library()
    cfg = SHAPES[1]
    case = build_decode_case(cfg, gpu, steps=1)
    max_ctx = int(case.ctx.max()) + 1
    ws = decode_workspace(cfg.batch, cfg.hq, cfg.hkv, max_ctx, gpu)
    out = torch.empty((cfg.batch, cfg.hq, 128), dtype=torch.bfloat16, device=gpu)
    pos = case.positions(0)
    pos_out = torch.empty_like(pos)
    c, qkv = case.cache, case.qkv[0]
    args = [pointer(qkv), qkv.stride(0), pointer(pos), pointer(pos_out), pointer(case.q_gain), pointer(case.k_gain),
            pointer(case.cos), pointer(case.sin), case.cos.shape[0], pointer(c.pages), pointer(c.block_table),
            c.max_blocks, c.num_blocks, cfg.window, cfg.batch, cfg.hq, cfg.hkv, max_ctx, SCALE, pointer(out)]
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    check(lib.nc_decode_step_fp8(*args, pointer(ws), ws.numel(), stream()))
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    check(lib.nc_decode_step_fp8_noalloc(*args, stream()))
    torch.cuda.synchronize()
    free2 = torch.cuda.mem_get_info()[0]
    mib = 1 << 20
    print(f"first decode call {(free0 - free1) / mib:.1f} MiB, first no-alloc call {(free1 - free2) / mib:.1f} MiB",
          flush=True)
    assert free0 - free1 < 16 * mib
    assert free1 - free2 >= 64 * mib


def test_noalloc_step_equals_workspace_step(gpu):
    lib = hip_library()
    for cfg in SHAPES:  # the larger call first, then the smaller one over the same scratch
        print(f"no-alloc step {cfg.name}", flush=True)
        a = build_decode_case(cfg, gpu, steps=1)
        b = build_decode_case(cfg, gpu, steps=1)
        max_ctx = int(a.ctx.max()) + 1
        ws = decode_workspace(cfg.batch, cfg.hq, cfg.hkv, max_ctx, gpu)
        want, want_pos = _step(lib, a, cfg, max_ctx, False, ws)
        got, got_pos = _step(lib, b, cfg, max_ctx, True, None)
        torch.cuda.synchronize()
        np.testing.assert_array_equal(bits(got), bits(want), err_msg=cfg.name)
        assert torch.equal(got_pos, want_pos), cfg.name
        assert torch.equal(a.cache.pages, b.cache.pages), cfg.name


def test_noalloc_rejects_a_shape_past_the_scratch(gpu):
    """4096 sequences of 16 MHA heads need more partial-result room than the 64 MiB scratch: a clear error, no
    launch."""
    lib = hip_library()
    need = lib.nc_decode_workspace_bytes(4096, 16, 16, 1024)
    assert need > 64 << 20
    fake = torch.empty(16, dtype=torch.uint8, device=gpu)
    p = pointer(fake)
    rc = lib.nc_decode_step_fp8_noalloc(p, 48 * 128, p, None, p, p, p, p, 1024, p, None, 64, 4096 * 64, -1, 4096, 16,
                                        16, 1024, SCALE, p, stream())
    assert rc < 0
    assert "static scratch" in lib.nc_last_error().decode()
