"""Trained weights for the decoder: the Hugging Face directory inference/export_hf.py writes (config.json and
model.safetensors), read into the decoder's layout (decoder.Weights), and the same format written back.

The format (export_hf.py:40-77; names from inference/modeling_nanochat.py's modules):

    model.embed_tokens.weight                       bf16 [vocab][C]
    model.layers.{i}.self_attn.{q,k,v,o}_proj.weight bf16
    model.layers.{i}.self_attn.{q,k}_norm_weight    fp32 [128]
    model.layers.{i}.self_attn.ve_gate.weight       fp32 [H][C]      value-embedding layers only
    model.layers.{i}.mlp.{up,down}_proj.weight      bf16
    model.value_embeds.{i}.weight                   bf16 [vocab][C]  value-embedding layers only
    model.resid_lambdas, model.x0_lambdas           fp32 [layers]
    lm_head.weight                                  bf16 [vocab][C]

config.json carries vocab_size, hidden_size, intermediate_size, num_hidden_layers, num_attention_heads,
num_key_value_heads, head_dim (128), rope_parameters.rope_theta, sliding_window (keys before a query + 1, the
transformers convention), layer_types ("sliding_attention" / "full_attention"), value_embedding_layers,
final_logit_softcapping and rms_norm_eps (FLT_EPSILON). Tensors are read with safetensors (no pickle).
"""

from __future__ import annotations

import json
from pathlib import Path

import torch
from safetensors.torch import load_file, save_file

from nanochat_amd.decoder import EPS, ModelConfig, Weights
from nanochat_amd.kv_cache import HEAD_DIM


def config_from_hf(cfg: dict) -> ModelConfig:
    """ModelConfig of an export's config.json; rejects what the decoder cannot run."""
    if cfg.get("head_dim", HEAD_DIM) != HEAD_DIM:
        raise ValueError(f"head_dim {cfg.get('head_dim')} != {HEAD_DIM}")
    if cfg.get("tie_word_embeddings", False):
        raise ValueError("tied embeddings: the decoder reads an untied lm_head")
    eps = cfg.get("rms_norm_eps", EPS)
    if abs(eps - EPS) > 1e-12:
        raise ValueError(f"rms_norm_eps {eps}: the decoder's norms use FLT_EPSILON")
    C, n = cfg["hidden_size"], cfg["num_hidden_layers"]
    H, Hkv = cfg["num_attention_heads"], cfg.get("num_key_value_heads", cfg["num_attention_heads"])
    if H * HEAD_DIM != C:
        raise ValueError(f"{H} heads of {HEAD_DIM} != hidden size {C}")
    if cfg["intermediate_size"] % C:
        raise ValueError(f"intermediate_size {cfg['intermediate_size']} is not a multiple of {C}")
    types = cfg.get("layer_types", ["full_attention"] * n)
    short = cfg.get("sliding_window")
    windows = tuple((short - 1) if t == "sliding_attention" else -1 for t in types)
    theta = cfg.get("rope_parameters", {}).get("rope_theta", cfg.get("rope_theta", 10000.0))
    return ModelConfig(layers=n, d_model=C, heads=H, vocab=cfg["vocab_size"], mlp_mult=cfg["intermediate_size"] // C,
                       theta=float(theta), windows=windows if any(w >= 0 for w in windows) else (),
                       ve_layers=tuple(cfg.get("value_embedding_layers", [])), n_kv_heads=0 if Hkv == H else Hkv,
                       softcap=float(cfg.get("final_logit_softcapping", 15.0)))


class LoadedModel(Weights):
    """A model read from an export directory onto `device`."""

    def __init__(self, path, device):
        path = Path(path)
        cfg = config_from_hf(json.loads((path / "config.json").read_text()))
        t = load_file(str(path / "model.safetensors"))
        self.cfg = cfg

        def get(name: str, dtype: torch.dtype) -> torch.Tensor:
            if name not in t:
                raise KeyError(f"{path}: missing tensor {name}")
            return t[name].to(device=device, dtype=dtype).contiguous()

        self.wte = get("model.embed_tokens.weight", torch.bfloat16)
        self.lm_head = get("lm_head.weight", torch.bfloat16)
        self.resid_lambdas = get("model.resid_lambdas", torch.float32)
        self.x0_lambdas = get("model.x0_lambdas", torch.float32)
        self.layers = []
        for i in range(cfg.layers):
            a, m = f"model.layers.{i}.self_attn.", f"model.layers.{i}.mlp."
            lw = dict(wqkv=torch.cat([get(a + f"{p}_proj.weight", torch.bfloat16) for p in "qkv"]).contiguous(),
                      wo=get(a + "o_proj.weight", torch.bfloat16), wup=get(m + "up_proj.weight", torch.bfloat16),
                      wdown=get(m + "down_proj.weight", torch.bfloat16),
                      q_gain=get(a + "q_norm_weight", torch.float32), k_gain=get(a + "k_norm_weight", torch.float32))
            if i in cfg.ve_layers:
                lw["ve"] = get(f"model.value_embeds.{i}.weight", torch.bfloat16)
                lw["ve_gate"] = get(a + "ve_gate.weight", torch.float32)
            self.layers.append(lw)


def load_hf(path, device) -> LoadedModel:
    return LoadedModel(path, device)


def save_hf(model: Weights, path, max_positions: int = 2048) -> None:
    """Write `model` in the export's format (model.safetensors with its names and dtypes, config.json)."""
    cfg = model.cfg
    H, Hkv = cfg.heads, cfg.kv_heads
    cpu = lambda x, dt: x.detach().to("cpu", dt).contiguous()
    windows = [cfg.window(i) for i in range(cfg.layers)]
    short = {w for w in windows if w >= 0}
    if len(short) > 1:
        raise ValueError(f"the format holds one sliding window, the model has {sorted(short)}")
    path = Path(path)
    path.mkdir(parents=True, exist_ok=True)
    t = {"model.embed_tokens.weight": cpu(model.wte, torch.bfloat16),
         "lm_head.weight": cpu(model.lm_head, torch.bfloat16),
         "model.resid_lambdas": cpu(model.resid_lambdas, torch.float32),
         "model.x0_lambdas": cpu(model.x0_lambdas, torch.float32)}
    for i, lw in enumerate(model.layers):
        a, m = f"model.layers.{i}.self_attn.", f"model.layers.{i}.mlp."
        q, k, v = torch.split(lw["wqkv"], [H * HEAD_DIM, Hkv * HEAD_DIM, Hkv * HEAD_DIM])
        t |= {a + "q_proj.weight": cpu(q, torch.bfloat16), a + "k_proj.weight": cpu(k, torch.bfloat16),
              a + "v_proj.weight": cpu(v, torch.bfloat16), a + "o_proj.weight": cpu(lw["wo"], torch.bfloat16),
              a + "q_norm_weight": cpu(lw["q_gain"], torch.float32),
              a + "k_norm_weight": cpu(lw["k_gain"], torch.float32),
              m + "up_proj.weight": cpu(lw["wup"], torch.bfloat16),
              m + "down_proj.weight": cpu(lw["wdown"], torch.bfloat16)}
        if "ve" in lw:
            t[f"model.value_embeds.{i}.weight"] = cpu(lw["ve"], torch.bfloat16)
            t[a + "ve_gate.weight"] = cpu(lw["ve_gate"], torch.float32)
    save_file(t, str(path / "model.safetensors"), metadata={"format": "pt"})
    (path / "config.json").write_text(json.dumps({
        "architectures": ["NanochatForCausalLM"], "model_type": "nanochat",
        "vocab_size": cfg.vocab, "hidden_size": cfg.d_model, "intermediate_size": cfg.mlp_mult * cfg.d_model,
        "num_hidden_layers": cfg.layers, "num_attention_heads": H, "num_key_value_heads": Hkv, "head_dim": HEAD_DIM,
        "max_position_embeddings": max_positions, "rope_parameters": {"rope_type": "default", "rope_theta": cfg.theta},
        "sliding_window": (min(short) + 1) if short else max_positions,
        "layer_types": ["sliding_attention" if w >= 0 else "full_attention" for w in windows],
        "value_embedding_layers": list(cfg.ve_layers), "final_logit_softcapping": cfg.softcap, "rms_norm_eps": EPS,
        "tie_word_embeddings": False, "dtype": "bfloat16"}, indent=2) + "\n")
