"""Writes golden vectors of the reference's own torch path, run on the CPU of the build container, for the parts of
the oracle that the mathematics alone leaves open:

    python tests/golden/make_reference_vectors.py

reference_qk_norm_rope.npz   inference/modeling_nanochat.py:37-45 `qk_norm_rope` (torch.rsqrt of torch's mean, then
                             gain and the -theta rotation, one bf16 rounding) and :29-34 `rotary` on seeded bf16 rows
                             (N(0, 1), 1 % outliers at 8 sigma, rows scaled from 2^-20 to 2^20, a zero row, one-hot
                             rows) at seeded positions, theta 1e4 and 1e6: the inputs, the gains, the reference's cos /
                             sin tables and its output bits.
reference_model_small.npz    inference/modeling_nanochat.py:136-195 `NanochatForCausalLM` (eager attention, bf16
                             weights and activations as export_hf.py writes them) on a tiny MHA model whose weights
                             fixture_model() below derives from a counter hash (no library RNG): 3 layers, d 256,
                             2 heads, vocab 256, a sliding-window layer pair, a value-embedding layer, a non-identity
                             residual / x0 mix and non-unit QK-norm gains; the capped logits of every position of two
                             16-token sequences, from one full forward and from the decode protocol over the
                             reference's own DynamicCache (5 positions prefilled, then one token per call).

reference_attention.npz      inference/modeling_nanochat.py:48-56 `eager_attention_forward` (bf16 scores and
                             products, probabilities cast to bf16) on three cases: decode with MHA (3 sequences,
                             4 heads, contexts 37, 300, 1000), decode with GQA (2 sequences, 16 query / 4 kv heads,
                             contexts 513 and 1500, 1 % of the elements at 8 sigma) and a causal prefill chunk (2
                             sequences, 8 / 2 heads, 40 and 25 rows onto 100 and 250 cached keys); kv heads are
                             repeated for the reference's MHA layout. K and V rows come from fp8_exact_rows(), values
                             both bf16 and e4m3 code x 2^e whose absmax is 448 x 2^e: the reference's bf16 cache and
                             this build's fp8 cache (absmax / 448 = 2^e, exact codes) hold the same numbers. The
                             fixture keeps the q rows and the reference's outputs; the tests rebuild K and V.

The reference module is imported from /root/reference in this container only, by this script; the tests read the
fixtures and never import or read the reference.
"""

from __future__ import annotations

import importlib.util
import json
import os
import sys
import tempfile

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
REFERENCE = "/root/reference/inference/modeling_nanochat.py"

# the tiny model: MHA (the reference's NanochatAttention projects k and v to all H heads)
MODEL = dict(layers=3, d_model=256, heads=2, vocab=256, theta=1e4, windows=(4, -1, 4), ve_layers=(1,), softcap=15.0)
SEQS, SEQ_LEN, IDS_SEED = 2, 16, 11
PREFILL = 5  # the cached run: positions 0..4 prefilled, then one call per position 5..15


def hashed_uniform(n: int, seed: int) -> np.ndarray:
    """n values in [-sqrt(3), sqrt(3)) (unit variance) from a splitmix64 hash of (index, seed): the same values on
    every machine and numpy version."""
    with np.errstate(over="ignore"):
        x = np.arange(n, dtype=np.uint64) * np.uint64(0x9E3779B97F4A7C15) + np.uint64(seed) * np.uint64(
            0xD1B54A32D192ED03)
        x ^= x >> np.uint64(30)
        x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27)
        x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
    u = (x >> np.uint64(11)).astype(np.float64) / float(1 << 53)
    return ((2.0 * u - 1.0) * np.sqrt(3.0)).astype(np.float32)


def fixture_model():
    """The tiny model's weights as a nanochat_amd.decoder.Weights on the CPU (bf16 matrices, fp32 gains, gates and
    mix), every tensor from hashed_uniform with its own seed."""
    sys.path.insert(0, REPO)
    from nanochat_amd.decoder import ModelConfig, Weights

    cfg = ModelConfig(layers=MODEL["layers"], d_model=MODEL["d_model"], heads=MODEL["heads"], vocab=MODEL["vocab"],
                      theta=MODEL["theta"], windows=MODEL["windows"], ve_layers=MODEL["ve_layers"],
                      softcap=MODEL["softcap"])
    seed = iter(range(1000, 2000))
    d, C = cfg.d_model, cfg.heads * 128

    def t(shape, scale, offset=0.0, dtype=torch.bfloat16):
        v = hashed_uniform(int(np.prod(shape)), next(seed)).reshape(shape) * np.float32(scale) + np.float32(offset)
        return torch.from_numpy(v).to(dtype)

    w = Weights()
    w.cfg = cfg
    std = 0.06  # ~ 1/sqrt(d): every sublayer moves the residual stream visibly
    w.wte = t((cfg.vocab, d), 1.0)
    w.layers = []
    for i in range(cfg.layers):
        lw = dict(wqkv=t((3 * C, d), std), wo=t((d, C), std), wup=t((cfg.mlp_mult * d, d), std),
                  wdown=t((d, cfg.mlp_mult * d), std / 2),
                  q_gain=t((128,), 0.25, 1.0, torch.float32), k_gain=t((128,), 0.25, 1.0, torch.float32))
        if i in cfg.ve_layers:
            lw["ve"] = t((cfg.vocab, C), 0.8)
            lw["ve_gate"] = t((cfg.heads, d), 0.2, 0.0, torch.float32)
        w.layers.append(lw)
    w.lm_head = t((cfg.vocab, d), std)
    w.resid_lambdas = t((cfg.layers,), 0.2, 1.0, torch.float32)
    w.x0_lambdas = t((cfg.layers,), 0.1, 0.3, torch.float32)
    return w


def fp8_exact_rows(n: int, seed: int, outliers: float = 0.0) -> np.ndarray:
    """n rows of 128 fp32 values, each exactly a bf16 and an e4m3 code times 2^e (e in [-7, -5] per row: a standard
    deviation of 0.44 to 1.75), with the row's absmax exactly 448 x 2^e: codes of a unit-variance draw times 56 (so
    448 is 8 sigma), one element per row (and, with `outliers`, that fraction of the others) at +-448."""
    sys.path.insert(0, REPO)
    from oracle import golden as G

    v = hashed_uniform(n * 128, seed).reshape(n, 128) * np.float32(56.0)
    v = G.e4m3_decode(G.e4m3_encode(v))
    sign = np.where(hashed_uniform(n * 128, seed + 1).reshape(n, 128) < 0, -1.0, 1.0).astype(np.float32)
    at = ((hashed_uniform(n, seed + 2) / np.sqrt(3.0) + 1.0) * 64.0).astype(np.int64).clip(0, 127)
    v[np.arange(n), at] = 448.0 * sign[np.arange(n), at]
    if outliers > 0:
        hit = (hashed_uniform(n * 128, seed + 3).reshape(n, 128) / np.sqrt(3.0) + 1.0) / 2.0 < outliers
        v = np.where(hit, 448.0 * sign, v)
    e = -5 - ((hashed_uniform(n, seed + 4) / np.sqrt(3.0) + 1.0) * 1.5).astype(np.int64).clip(0, 2)
    return (v * np.exp2(e.astype(np.float32))[:, None]).astype(np.float32)


def hashed_bf16(shape, seed: int) -> np.ndarray:
    """Unit-variance values rounded to bf16, as fp32."""
    x = torch.from_numpy(hashed_uniform(int(np.prod(shape)), seed).reshape(shape))
    return x.to(torch.bfloat16).float().numpy()


# (name, batch, query heads, kv heads, cached keys per sequence, query rows per sequence, outlier fraction, seed);
# decode: one query row at the last position; prefill: the chunk's rows after the cached keys, causal
ATTENTION_CASES = [("decode_mha", 3, 4, 4, (36, 299, 999), (1, 1, 1), 0.0, 3000),
                   ("decode_gqa", 2, 16, 4, (512, 1499), (1, 1), 0.01, 4000),
                   ("prefill", 2, 8, 2, (100, 250), (40, 25), 0.0, 5000)]


def attention_kv(case: tuple, b: int, h: int) -> tuple[np.ndarray, np.ndarray]:
    """K and V rows [keys][128] of sequence b, kv head h: its cached keys and its query rows' own keys."""
    name, B, hq, hkv, cached, rows, outl, seed = case
    n = cached[b] + rows[b]
    base = seed + 100 * b + 10 * h
    return fp8_exact_rows(n, base, outl), fp8_exact_rows(n, base + 5, outl)


def attention_q(case: tuple, b: int) -> np.ndarray:
    """Query rows [rows][hq][128] of sequence b."""
    name, B, hq, hkv, cached, rows, outl, seed = case
    return hashed_bf16((rows[b], hq, 128), seed + 100 * b + 99)


def fixture_ids() -> np.ndarray:
    return np.random.default_rng(IDS_SEED).integers(0, MODEL["vocab"], (SEQS, SEQ_LEN)).astype(np.int64)


def _reference():
    spec = importlib.util.spec_from_file_location("reference_modeling_nanochat", REFERENCE)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def qk_vectors(ref) -> dict:
    rng = np.random.default_rng(3)
    n = 128
    x = rng.standard_normal((n, 128)).astype(np.float32)
    x[rng.random((n, 128)) < 0.01] = 8.0
    x[32:64] *= np.float32(2.0) ** rng.integers(-20, 21, (32, 1)).astype(np.float32)  # scales 2^-20 .. 2^20
    x[64] = 0.0
    x[65:70] = 0.0
    x[65:70, rng.integers(0, 128, 5)] = [1.0, -3.0, 0.5, 2.0 ** -30, 1e30]  # one-hot rows
    xb = torch.from_numpy(x).to(torch.bfloat16)
    gain = torch.from_numpy((0.5 + rng.random(128)).astype(np.float32))
    pos = torch.from_numpy(rng.integers(0, 8192, n).astype(np.int64))
    pos[:8] = torch.tensor([0, 1, 8191, 4096, 16383, 65535, 100000, 131071])  # and long contexts' positions
    out = {"x_bits": xb.view(torch.int16).numpy().view(np.uint16), "gain": gain.numpy(), "pos": pos.numpy()}
    eps = float(torch.finfo(torch.float32).eps)
    for theta in (1e4, 1e6):
        cos, sin = ref.rotary(pos, 128, theta)  # [n][64] fp32
        # qk_norm_rope's x is (..., H, D) with cos (..., D/2): one head per row
        y = ref.qk_norm_rope(xb[:, None, :], gain, cos, sin, eps)[:, 0, :]
        tag = f"{int(theta):d}"
        out[f"cos_{tag}"], out[f"sin_{tag}"] = cos.numpy(), sin.numpy()
        out[f"y_bits_{tag}"] = y.view(torch.int16).numpy().view(np.uint16)
    return out


def model_vectors(ref) -> dict:
    from safetensors.torch import load_file

    sys.path.insert(0, REPO)
    from nanochat_amd.checkpoint import save_hf

    w = fixture_model()
    with tempfile.TemporaryDirectory() as d:
        save_hf(w, d, max_positions=64)
        cfg_json = json.loads(open(os.path.join(d, "config.json")).read())
        state = load_file(os.path.join(d, "model.safetensors"))
    config = ref.NanochatConfig(**cfg_json)
    config._attn_implementation = "eager"  # the reference's own eager_attention_forward (bf16 probabilities)
    model = ref.NanochatForCausalLM(config)
    keep_fp32 = set(ref.NanochatPreTrainedModel._keep_in_fp32_modules_strict)
    for name, p in model.named_parameters():  # the export's dtypes: fp32 where the training forward reads fp32
        p.data = p.data.to(torch.float32 if keep_fp32 & set(name.split(".")) else torch.bfloat16)
    missing, unexpected = model.load_state_dict(state, strict=True)
    assert not missing and not unexpected
    for name, p in model.named_parameters():
        assert p.dtype == state[name].dtype, name
    model.eval()
    ids = fixture_ids()
    t = torch.from_numpy(ids)
    with torch.no_grad():
        logits = model(input_ids=t).logits.float().numpy()
        # the decode protocol through the reference's own cache (DynamicCache.update appends each step's keys and
        # values, modeling_nanochat.py:94-96): positions 0..PREFILL-1 at once, then one token per call
        out = model(input_ids=t[:, :PREFILL], use_cache=True)
        cached = [out.logits[:, -1].float()]
        for p in range(PREFILL, SEQ_LEN):
            out = model(input_ids=t[:, p:p + 1], past_key_values=out.past_key_values, use_cache=True)
            cached.append(out.logits[:, -1].float())
    return {"ids": ids, "logits": logits, "logits_cached": torch.stack(cached, 1).numpy(),
            "cached_from": np.array(PREFILL - 1), "config_json": np.array(json.dumps(cfg_json))}


def attention_vectors(ref) -> dict:
    out = {}
    for case in ATTENTION_CASES:
        name, B, hq, hkv, cached, rows, outl, seed = case
        G = hq // hkv
        res = []
        for b in range(B):
            kv = [attention_kv(case, b, h) for h in range(hkv)]
            k = torch.tensor(np.stack([kv[hh // G][0] for hh in range(hq)]), dtype=torch.bfloat16)[None]
            v = torch.tensor(np.stack([kv[hh // G][1] for hh in range(hq)]), dtype=torch.bfloat16)[None]
            q = torch.tensor(attention_q(case, b), dtype=torch.bfloat16).transpose(0, 1)[None]  # [1][hq][rows][128]
            n = cached[b] + rows[b]
            pos = cached[b] + torch.arange(rows[b])
            allowed = torch.arange(n)[None, :] <= pos[:, None]
            mask = torch.zeros((rows[b], n), dtype=torch.bfloat16).masked_fill(~allowed,
                                                                               torch.finfo(torch.bfloat16).min)
            o, _ = ref.eager_attention_forward(None, q, k, v, mask[None, None], scaling=128 ** -0.5)
            res.append(o[0].view(torch.int16).numpy().view(np.uint16))  # [rows][hq][128]
        out[f"{name}_out_bits"] = np.concatenate(res)
    return out


def main() -> None:
    import transformers

    ref = _reference()
    meta = {"torch": torch.__version__, "transformers": transformers.__version__,
            "reference": "inference/modeling_nanochat.py"}
    qk = qk_vectors(ref)
    np.savez_compressed(os.path.join(HERE, "reference_qk_norm_rope.npz"), meta=np.array(json.dumps(meta)), **qk)
    mv = model_vectors(ref)
    np.savez_compressed(os.path.join(HERE, "reference_model_small.npz"), meta=np.array(json.dumps(meta)), **mv)
    av = attention_vectors(ref)
    np.savez_compressed(os.path.join(HERE, "reference_attention.npz"), meta=np.array(json.dumps(meta)), **av)
    print("wrote reference_qk_norm_rope.npz, reference_model_small.npz and reference_attention.npz", meta)


if __name__ == "__main__":
    main()
