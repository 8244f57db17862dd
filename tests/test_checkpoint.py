"""The export format (inference/export_hf.py:40-77) round trip, CPU only: names, dtypes and config fields as the
reference writes them, every tensor back bit for bit, and the rejections of what the decoder cannot run."""

import json

import pytest
import torch
from safetensors.torch import load_file

from nanochat_amd.checkpoint import config_from_hf, load_hf, save_hf
from nanochat_amd.decoder import EPS, ModelConfig, RandomModel

CFG = ModelConfig(layers=4, d_model=256, heads=2, vocab=300, theta=1e6, windows=(16, 16, 16, -1), ve_layers=(1, 3),
                  softcap=15.0)


def trained_like(cfg=CFG):
    m = RandomModel(cfg, "cpu", seed=3)
    g = torch.Generator().manual_seed(4)
    m.resid_lambdas = 0.8 + 0.4 * torch.rand(cfg.layers, generator=g)
    m.x0_lambdas = 0.2 * torch.rand(cfg.layers, generator=g) - 0.1
    for lw in m.layers:
        lw["q_gain"] = 0.5 + torch.rand(128, generator=g)
        lw["k_gain"] = 0.5 + torch.rand(128, generator=g)
        if "ve_gate" in lw:
            lw["ve_gate"] = torch.randn(lw["ve_gate"].shape, generator=g) * 0.05
    return m


def test_round_trip_names_dtypes_and_values(tmp_path):
    m = trained_like()
    save_hf(m, tmp_path, max_positions=512)
    t = load_file(str(tmp_path / "model.safetensors"))
    fp32 = {k for k, v in t.items() if v.dtype == torch.float32}
    # fp32 exactly what the export keeps in fp32: lambdas, QK-norm weights, VE gates
    assert fp32 == {"model.resid_lambdas", "model.x0_lambdas"} | {
        f"model.layers.{i}.self_attn.{n}" for i in range(4) for n in ("q_norm_weight", "k_norm_weight")} | {
        f"model.layers.{i}.self_attn.ve_gate.weight" for i in (1, 3)}
    assert "model.value_embeds.1.weight" in t and "model.value_embeds.0.weight" not in t
    assert t["model.layers.0.self_attn.q_proj.weight"].shape == (256, 256)
    cfg = json.loads((tmp_path / "config.json").read_text())
    assert cfg["sliding_window"] == 17 and cfg["layer_types"][3] == "full_attention"
    assert cfg["num_key_value_heads"] == 2 and cfg["head_dim"] == 128 and cfg["rms_norm_eps"] == EPS
    back = load_hf(tmp_path, "cpu")
    assert back.cfg == CFG
    assert torch.equal(back.wte, m.wte) and torch.equal(back.lm_head, m.lm_head)
    assert torch.equal(back.resid_lambdas, m.resid_lambdas) and torch.equal(back.x0_lambdas, m.x0_lambdas)
    for a, b in zip(back.layers, m.layers):
        assert a.keys() == b.keys()
        for k in a:
            assert torch.equal(a[k], b[k]), k
    assert back.mixes


def test_config_rejections():
    good = {"vocab_size": 300, "hidden_size": 256, "intermediate_size": 1024, "num_hidden_layers": 2,
            "num_attention_heads": 2, "num_key_value_heads": 2, "head_dim": 128}
    assert config_from_hf(good).windows == ()
    for bad, msg in ((dict(head_dim=64), "head_dim"), (dict(tie_word_embeddings=True), "tied"),
                     (dict(rms_norm_eps=1e-6), "rms_norm_eps"), (dict(num_attention_heads=3), "heads"),
                     (dict(intermediate_size=1000), "intermediate_size")):
        with pytest.raises(ValueError, match=msg):
            config_from_hf(good | bad)


def test_one_sliding_window_per_export(tmp_path):
    m = RandomModel(ModelConfig(layers=2, d_model=128, heads=1, vocab=64, windows=(8, 16)), "cpu")
    with pytest.raises(ValueError, match="one sliding window"):
        save_hf(m, tmp_path / "out")
