"""GPU row kernels of the decoder against torch fp32 references of the same ops: the fused residual add + RMS norm
(nc_add_rms_norm_bf16), relu^2 (nc_relu2_bf16), the value-embedding mix (nc_value_embed_bf16), the embedding norm
(nc_embed_rms_norm) and the residual mix (nc_mix_bf16). Rounded results agree within one bf16 step; the cases where
the math is exact in fp32 agree bit for bit."""

import pytest
import torch
import torch.nn.functional as F

from nanochat_amd.decoder import EPS, add_rms_norm, relu2, value_embed

pytestmark = pytest.mark.gpu


def ulps(a: torch.Tensor, b: torch.Tensor) -> int:
    """The largest distance in bf16 steps between two bf16 tensors of one sign pattern (0 when equal)."""
    ia = a.view(torch.int16).to(torch.int32)
    ib = b.view(torch.int16).to(torch.int32)
    ia = torch.where(ia < 0, -(ia & 0x7FFF), ia)  # sign-magnitude -> an ordered integer line
    ib = torch.where(ib < 0, -(ib & 0x7FFF), ib)
    return int((ia - ib).abs().max().item()) if a.numel() else 0


@pytest.mark.parametrize("n, d", [(1, 256), (7, 1280), (64, 2048), (3, 8192)])
def test_add_rms_norm_matches_torch(gpu, n, d):
    print(f"add_rms_norm case n {n} d {d}", flush=True)
    g = torch.Generator().manual_seed(n * d)
    x = (torch.randn((n, d), generator=g) * 3).to(torch.bfloat16)
    delta = torch.randn((n, d), generator=g).to(torch.bfloat16)
    xs, ds = x.to(gpu), delta.to(gpu)
    out = torch.empty_like(xs)
    y = add_rms_norm(xs, ds, out)
    torch.cuda.synchronize()
    s = (x.float() + delta.float()).to(torch.bfloat16)
    assert torch.equal(out.cpu(), s)  # the sum of two bf16 values rounded once
    want = F.rms_norm(s.double(), (d,), eps=EPS).to(torch.bfloat16)
    assert ulps(y.cpu(), want) <= 1
    y2 = add_rms_norm(xs, None)  # no delta: the norm of x itself
    torch.cuda.synchronize()
    assert ulps(y2.cpu(), F.rms_norm(x.double(), (d,), eps=EPS).to(torch.bfloat16)) <= 1


def test_relu2_matches_torch(gpu):
    x = (torch.randn(3 * 4096 + 8) * 4).to(torch.bfloat16)
    x[:4] = torch.tensor([0.0, -0.0, -1.0, 1e-20])
    got = relu2(x.to(gpu)).cpu()
    assert torch.equal(got, x.float().relu().square().to(torch.bfloat16))


def make_ve_case(rows, d, hq, hkv, vocab, seed, row_pad=0, x_pad=0, gate_scale=0.05):
    g = torch.Generator().manual_seed(seed)
    cols = (hq + 2 * hkv) * 128
    qkv = torch.randn((rows, cols + row_pad), generator=g).to(torch.bfloat16)
    x = (torch.randn((rows, d + x_pad), generator=g) * 2).to(torch.bfloat16)
    ve = torch.randn((vocab, hkv * 128), generator=g).to(torch.bfloat16)
    gate = torch.randn((hkv, d), generator=g) * gate_scale
    tok = torch.randint(0, vocab, (rows,), generator=g, dtype=torch.int32)
    return qkv, x, ve, gate, tok


def ve_reference(qkv, n, ve, gate, tok, hq, hkv):
    """fp64: v_h + 2 sigmoid(gate[h] . n) ve[tok]_h on the v heads, rounded to bf16 once."""
    rows = qkv.shape[0]
    want = qkv.clone()
    ok = (tok >= 0) & (tok < ve.shape[0])
    g = 2 * torch.sigmoid(n.double() @ gate.double().t())  # [rows][hkv]
    e = ve[tok.clamp(0, ve.shape[0] - 1).long()].double().view(rows, hkv, 128)
    v0 = (hq + hkv) * 128
    v = qkv[:, v0:v0 + hkv * 128].double().view(rows, hkv, 128)
    mixed = (v + g[..., None] * e).to(torch.bfloat16).view(rows, -1)
    want[ok, v0:v0 + hkv * 128] = mixed[ok]
    return want


@pytest.mark.parametrize("rows, d, hq, hkv, vocab, row_pad, x_pad", [
    (1, 256, 2, 2, 1000, 0, 0),
    (37, 1280, 10, 10, 65536, 0, 0),      # d20's width
    (64, 2048, 16, 4, 5000, 64, 8),       # GQA; padded qkv and x rows
    (5, 8192, 64, 64, 300, 0, 0),         # the widest row and the most kv heads
])
def test_value_embed_matches_torch(gpu, rows, d, hq, hkv, vocab, row_pad, x_pad):
    print(f"value_embed case rows {rows} d {d} hq {hq} hkv {hkv}", flush=True)
    qkv, x, ve, gate, tok = make_ve_case(rows, d, hq, hkv, vocab, seed=rows + d, row_pad=row_pad, x_pad=x_pad)
    tok[0] = vocab - 1
    if rows > 2:
        tok[1] = vocab    # out of range: the row is left as it is
        tok[2] = -1
    xs = x.to(gpu)[:, :d]
    n = add_rms_norm(xs.contiguous(), None)  # the norm the kernel restates
    out = qkv.to(gpu)
    value_embed(out[:, :(hq + 2 * hkv) * 128] if row_pad else out, xs, tok.to(gpu), ve.to(gpu), gate.to(gpu),
                hq, hkv)
    torch.cuda.synchronize()
    got = out.cpu()
    want = ve_reference(qkv[:, :(hq + 2 * hkv) * 128], n.cpu(), ve, gate, tok, hq, hkv)
    v0 = (hq + hkv) * 128
    assert torch.equal(got[:, :v0], qkv[:, :v0])                  # q and k heads untouched
    assert torch.equal(got[:, (hq + 2 * hkv) * 128:], qkv[:, (hq + 2 * hkv) * 128:])  # the row padding too
    if rows > 2:
        assert torch.equal(got[1:3], qkv[1:3])
    assert ulps(got[:, v0:v0 + hkv * 128], want[:, v0:]) <= 1


def test_value_embed_zero_gate_adds_the_embedding_exactly(gpu):
    """gate = 0: g = 2 sigmoid(0) = 1 exactly, so v = bf16(v + ve[tok]) bit for bit (the sum of two bf16 values
    is exact in fp32 at these magnitudes): pins the head and row layout of qkv and ve."""
    rows, d, hq, hkv, vocab = 16, 512, 4, 2, 777
    qkv, x, ve, gate, tok = make_ve_case(rows, d, hq, hkv, vocab, seed=9)
    gate.zero_()
    out = qkv.to(gpu)
    value_embed(out, x.to(gpu), tok.to(gpu), ve.to(gpu), gate.to(gpu), hq, hkv)
    torch.cuda.synchronize()
    v0 = (hq + hkv) * 128
    want = (qkv[:, v0:].float() + ve[tok.long()].float()).to(torch.bfloat16)
    assert torch.equal(out.cpu()[:, v0:], want)
    assert torch.equal(out.cpu()[:, :v0], qkv[:, :v0])


def test_value_embed_gate_saturates(gpu):
    """A large gate . n drives g to 2 (or 0): v = bf16(v + 2 ve) (or v) exactly."""
    rows, d, hq, hkv, vocab = 8, 256, 2, 2, 50
    qkv, x, ve, gate, tok = make_ve_case(rows, d, hq, hkv, vocab, seed=10)
    x = torch.ones((rows, d), dtype=torch.bfloat16)  # norm(x) = 1 everywhere (up to bf16 rounding of rstd)
    gate[0].fill_(1.0)     # dot ~ d: sigmoid = 1 in fp32
    gate[1].fill_(-1.0)    # sigmoid = 0
    out = qkv.to(gpu)
    value_embed(out, x.to(gpu), tok.to(gpu), ve.to(gpu), gate.to(gpu), hq, hkv)
    torch.cuda.synchronize()
    v0 = (hq + hkv) * 128
    e = ve[tok.long()].float().view(rows, hkv, 128)
    v = qkv[:, v0:].float().view(rows, hkv, 128)
    got = out.cpu()[:, v0:].view(rows, hkv, 128)
    assert torch.equal(got[:, 0], (v[:, 0] + 2 * e[:, 0]).to(torch.bfloat16))
    assert torch.equal(got[:, 1], v[:, 1].to(torch.bfloat16))


def test_embed_norm_matches_the_row_norm_and_torch(gpu):
    """nc_embed_rms_norm: a bf16 table gives add_rms_norm(table[tok]) bit for bit; an fp32 table is within one bf16
    step of torch's fp64 norm; a token outside the vocabulary gives a zero row."""
    from nanochat_amd.decoder import embed_norm

    g = torch.Generator().manual_seed(12)
    vocab, d = 500, 1664
    table32 = torch.randn((vocab, d), generator=g) * 0.7
    table16 = table32.to(torch.bfloat16)
    tok = torch.tensor([0, 499, 17, 17, 500, -3, 250], dtype=torch.int32)
    ok = (tok >= 0) & (tok < vocab)
    got16 = embed_norm(table16.to(gpu), tok.to(gpu)).cpu()
    want16 = add_rms_norm(table16.to(gpu)[tok.clamp(0, vocab - 1).long().to(gpu)].contiguous(), None).cpu()
    assert torch.equal(got16[ok], want16[ok])
    assert (got16[~ok].float() == 0).all()
    got32 = embed_norm(table32.to(gpu), tok.to(gpu)).cpu()
    want32 = F.rms_norm(table32[tok[ok].long()].double(), (d,), eps=EPS).to(torch.bfloat16)
    assert ulps(got32[ok], want32) <= 1
    assert (got32[~ok].float() == 0).all()


def test_mix_matches_torch_bit_for_bit(gpu):
    """nc_mix_bf16: bf16(lr x + l0 x0) with fp32 products and sum, exactly torch's three fp32 operations."""
    from nanochat_amd.decoder import mix

    g = torch.Generator().manual_seed(13)
    x = (torch.randn(4096 + 8, generator=g) * 3).to(torch.bfloat16)
    x0 = torch.randn(4096 + 8, generator=g).to(torch.bfloat16)
    for lr, l0 in [(0.93, 0.11), (1.0, 0.0), (1.2, -0.2)]:
        got = mix(x.to(gpu), x0.to(gpu), lr, l0).cpu()
        a, b = torch.tensor(lr, dtype=torch.float32), torch.tensor(l0, dtype=torch.float32)
        assert torch.equal(got, (a * x.float() + b * x0.float()).to(torch.bfloat16)), (lr, l0)
