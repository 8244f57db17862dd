"""The GPU decoder against the reference's own model: the tiny MHA model of tests/golden/make_reference_vectors.py
(sliding windows, a value-embedding layer, a non-identity residual / x0 mix, non-unit QK-norm gains), written in the
export's format and read back by checkpoint.load_hf, prefilled and then stepped through the fixture's own tokens on
the HIP path; its capped logits against the logits inference/modeling_nanochat.py's NanochatForCausalLM gave for
the same tokens through its own DynamicCache (bf16 K/V, eager attention), held to the bound the CPU model meets
(the fp8 cache's own effect)."""

import numpy as np
import pytest
import torch

from test_reference_vectors import CPU_MAX, CPU_MEAN, MODEL, T_PROMPT, _capped, _maker, _rel, cached_reference

pytestmark = pytest.mark.gpu


def test_gpu_decoder_matches_the_reference_model(gpu, tmp_path):
    from nanochat_amd.checkpoint import load_hf, save_hf
    from nanochat_amd.decoder import Fp8Decoder

    save_hf(_maker().fixture_model(), tmp_path, max_positions=64)
    model = load_hf(tmp_path, gpu)
    ids = MODEL["ids"]
    B, T = ids.shape
    dec = Fp8Decoder(model, B, T, gpu)
    dec.prefill(torch.from_numpy(ids[:, :T_PROMPT].astype(np.int32)).to(gpu))
    out = torch.empty(B, dtype=torch.int32, device=gpu)
    got = []
    for p in range(T_PROMPT - 1, T):  # teacher-forced: every step reads the fixture's own token at p
        tok = torch.from_numpy(ids[:, p].astype(np.int32)).to(gpu)
        got.append(dec._step(tok, torch.full((B,), p, dtype=torch.int32, device=gpu), out).cpu().numpy())
    got = _capped(np.stack(got, 1), model.cfg.softcap)
    want = cached_reference()
    mx, mean = _rel(got, want)
    print(f"GPU decoder vs reference: max {mx:.4f}, mean {mean:.4f} of the logits' spread", flush=True)
    assert mx <= CPU_MAX and mean <= CPU_MEAN, (mx, mean)
    top2 = np.sort(want, axis=-1)[..., -2:]
    sure = top2[..., 1] - top2[..., 0] > 2 * CPU_MAX * MODEL["logits"].std()
    np.testing.assert_array_equal(got.argmax(-1)[sure], want.argmax(-1)[sure])


@pytest.mark.parametrize("name", ["decode_mha", "decode_gqa", "prefill"])
def test_gpu_attention_matches_the_reference(gpu, name):
    """The reference's eager attention vectors (tests/golden/reference_attention.npz) on the HIP path: K / V stored
    by nc_kv_store_fp8 into a contiguous fp8 cache (exact here: the rows are e4m3 codes x 2^e), then
    nc_decode_attn_fp8 (decode cases) or nc_prefill_attn_fp8 (the causal chunk). The output is held to the north
    star's bar against the exact result (fp64 over the same cache, beyond one bf16 rounding of the output) and to
    that bar plus the reference's own rounding against the reference."""
    from nanochat_amd.attention import decode_attention, prefill_attention
    from nanochat_amd.kv_cache import Fp8KVCache
    from oracle import golden as G
    from test_reference_vectors import (REF_ATTN_BOUND, attention_case, attention_inputs, oracle_attention,
                                        reference_attention)

    case = attention_case(name)
    _, B, hq, hkv, cached, rows, _, _ = case
    kv, q, pos, seq = attention_inputs(case)
    cache = Fp8KVCache.contiguous(B, max(c + r for c, r in zip(cached, rows)) + 1, hkv, gpu)
    for b in range(B):
        k = np.concatenate([kv[(b, h)][0] for h in range(hkv)], 1)
        v = np.concatenate([kv[(b, h)][1] for h in range(hkv)], 1)
        n = len(k)
        cache.store(torch.from_numpy(k).to(gpu, torch.bfloat16), torch.from_numpy(v).to(gpu, torch.bfloat16),
                    torch.arange(n, dtype=torch.int32, device=gpu), torch.full((n,), b, dtype=torch.int32,
                                                                                 device=gpu))
    qt = torch.from_numpy(q.view(np.int16)).to(gpu).view(torch.bfloat16)
    pt = torch.from_numpy(pos).to(gpu)
    if name.startswith("decode"):
        out = decode_attention(qt, cache, pt + 1, max_ctx=cache.capacity)
    else:
        out = prefill_attention(qt, cache, pt, torch.from_numpy(seq).to(gpu))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().astype(np.float64)
    exact = oracle_attention(case)
    half_ulp = np.abs(G.bf16_to_f32(G.bf16_bits(exact.astype(np.float32))) - exact)  # the output's own rounding
    e = np.maximum(np.abs(got - exact) - half_ulp, 0.0)
    d = np.abs(got - reference_attention(name))
    print(f"{name}: GPU vs exact (beyond the output's rounding) max {e.max():.4f} mean {e.mean():.5f}; "
          f"GPU vs reference max {d.max():.4f} mean {d.mean():.5f}", flush=True)
    assert e.max() <= 2e-2 and e.mean() <= 2e-3, (e.max(), e.mean())
    mx, mean = REF_ATTN_BOUND[name]
    assert d.max() <= mx + 2e-2 and d.mean() <= mean + 2e-3, (d.max(), d.mean())
