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
