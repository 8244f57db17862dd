"""The oracle against vectors of the reference's own torch path (tests/golden/make_reference_vectors.py ran
inference/modeling_nanochat.py on the build container's CPU and froze its outputs; nothing here imports the
reference):

* rotary tables (modeling_nanochat.py:29-34): oracle.golden.rotary_tables equals the reference's cos / sin bits;
* QK-norm + RoPE (modeling_nanochat.py:37-45): the oracle's fixed-tree rule against torch's mean and rsqrt, bit for
  bit except where the two sums of squares round apart (then one bf16 ulp of the output);
* the whole model (NanochatForCausalLM, eager attention with bf16 probabilities, bf16 K/V): the independent dense
  forward of tests/test_oracle_model.py (fp32 probabilities) against the reference's full forward, and the CpuModel
  (fp8 cache, fp64 attention; prefill, then one step per position) against the reference's own decode protocol over
  its DynamicCache (positions 0..4 prefilled, then one token per call); every structural slip planted in the
  CpuModel must fall outside the CpuModel's bound.
"""

import importlib.util
import json
import os

import numpy as np
import pytest

from oracle import golden as G
from oracle.model import CpuModel
from test_oracle_model import (MixIgnoresX0, MlpNormOfLayerInput, NoFinalNorm, SwappedMix, VeGateWithoutFactor2,
                               WindowOffByOne, cpu_logits, dense_logits)

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _maker():
    spec = importlib.util.spec_from_file_location("make_reference_vectors", os.path.join(HERE,
                                                                                         "make_reference_vectors.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)  # defines the fixture model; the reference is imported only by its main()
    return mod


QK = np.load(os.path.join(HERE, "reference_qk_norm_rope.npz"))
MODEL = np.load(os.path.join(HERE, "reference_model_small.npz"))


@pytest.mark.parametrize("theta", ["10000", "1000000"])
def test_rotary_tables_equal_the_reference(theta):
    cos, sin = G.rotary_tables(131072, float(theta))
    pos = QK["pos"]
    np.testing.assert_array_equal(cos[pos], QK[f"cos_{theta}"])
    np.testing.assert_array_equal(sin[pos], QK[f"sin_{theta}"])


@pytest.mark.parametrize("theta", ["10000", "1000000"])
def test_qk_norm_rope_within_one_ulp_of_the_reference(theta):
    """Measured: 1 element of 16 384 differs (by 1 ulp) at theta 1e4, none at 1e6. The bound allows 1 ulp on at most
    0.1 % of the elements; a wrong order of norm, gain and rotation, a rotation by +theta or a dropped epsilon moves
    most elements by far more."""
    x, gain = QK["x_bits"], QK["gain"]
    y = G.qk_norm_rope(x, gain, QK[f"cos_{theta}"], QK[f"sin_{theta}"])
    want = QK[f"y_bits_{theta}"]
    ulps = np.abs(y.view(np.int16).astype(np.int64) - want.view(np.int16).astype(np.int64))
    same_sign = (y >> 15) == (want >> 15)
    print(f"theta {theta}: {int((y != want).sum())} of {y.size} elements differ")
    assert np.all(same_sign | (y == want) | ((y & 0x7FFF) == 0) & ((want & 0x7FFF) == 0))
    assert ulps.max() <= 1
    assert (y != want).mean() <= 1e-3


def _capped(logits: np.ndarray, cap: float) -> np.ndarray:
    """inference/modeling_nanochat.py:194: c tanh(logits / c) in fp32."""
    return (cap * np.tanh(logits.astype(np.float32) / np.float32(cap))).astype(np.float32)


T_PROMPT = 5  # positions 0..3 prefilled, then steps at 4..15: the reference's cached logits


def _rel(got: np.ndarray, want: np.ndarray) -> tuple[float, float]:
    spread = MODEL["logits"].std()
    err = np.abs(got - want)
    return float(err.max() / spread), float(err.mean() / spread)


def cached_reference() -> np.ndarray:
    """The reference's logits at positions T_PROMPT - 1 .. 15 through its DynamicCache."""
    at = int(MODEL["cached_from"])
    return MODEL["logits_cached"][:, T_PROMPT - 1 - at:]


def _cpu_vs_reference(cls) -> tuple[float, float]:
    w = _maker().fixture_model()
    ids = MODEL["ids"]
    B, T = ids.shape
    got = np.stack(cpu_logits(cls(w, B, T + 1), ids, T_PROMPT, T - T_PROMPT), 1)
    return _rel(_capped(got, w.cfg.softcap), cached_reference())


# Measured against the reference's logits (relative to their spread, 0.93): the dense forward max 0.042, mean 0.006
# (fp32 against bf16 probabilities, summation orders); the CpuModel max 0.077, mean 0.016 (the fp8 cache's own
# effect: the dense forward with fp8 K/V measures max 0.083, mean 0.016). Bounds about twice those.
DENSE_MAX, DENSE_MEAN = 0.08, 0.012
CPU_MAX, CPU_MEAN = 0.15, 0.03


def test_reference_cached_run_equals_its_full_forward():
    """The fixture's two reference runs agree (fp32 noise): its cache path appends and masks as its full forward."""
    at = int(MODEL["cached_from"])
    np.testing.assert_allclose(MODEL["logits_cached"], MODEL["logits"][:, at:], atol=1e-5, rtol=0)


def test_fixture_model_is_the_one_the_vectors_were_made_from():
    w = _maker().fixture_model()
    cfg = json.loads(str(MODEL["config_json"]))
    assert cfg["num_hidden_layers"] == w.cfg.layers and cfg["hidden_size"] == w.cfg.d_model
    assert cfg["value_embedding_layers"] == list(w.cfg.ve_layers)
    assert cfg["sliding_window"] == 5 and cfg["layer_types"][1] == "full_attention"
    assert MODEL["logits"].shape == (*MODEL["ids"].shape, w.cfg.vocab)


def test_dense_forward_matches_the_reference_model():
    w = _maker().fixture_model()
    got = _capped(dense_logits(w, MODEL["ids"], fp8_kv=False).numpy(), w.cfg.softcap)
    mx, mean = _rel(got, MODEL["logits"])
    print(f"dense vs reference: max {mx:.4f}, mean {mean:.4f} of the logits' spread")
    assert mx <= DENSE_MAX and mean <= DENSE_MEAN, (mx, mean)


def test_cpu_model_matches_the_reference_model():
    mx, mean = _cpu_vs_reference(CpuModel)
    print(f"CpuModel vs reference: max {mx:.4f}, mean {mean:.4f} of the logits' spread")
    assert mx <= CPU_MAX and mean <= CPU_MEAN, (mx, mean)


@pytest.mark.parametrize("slip", [MlpNormOfLayerInput, SwappedMix, MixIgnoresX0, NoFinalNorm, VeGateWithoutFactor2,
                                  WindowOffByOne], ids=lambda c: c.__name__)
def test_reference_vectors_catch_structural_slips(slip):
    mx, mean = _cpu_vs_reference(slip)
    print(f"{slip.__name__} vs reference: max {mx:.4f}, mean {mean:.4f} of the logits' spread")
    assert mx > CPU_MAX or mean > CPU_MEAN, f"{slip.__name__} passed the comparison: not pinned"


# ---------------------------------------------------------------------------------------------------------------
# attention: the reference's eager_attention_forward (bf16 scores, probabilities cast to bf16) over K / V rows that
# are exactly the same numbers in its bf16 cache and in the fp8 cache (e4m3 code x 2^e, absmax 448 x 2^e)
# ---------------------------------------------------------------------------------------------------------------

ATTN = np.load(os.path.join(HERE, "reference_attention.npz"))
# The reference's own distance from the exact (fp64) result on these vectors, which its bf16 scores, bf16
# probabilities and bf16 output rounding set: decode MHA max 0.021 / mean 0.0019, decode GQA with 1 % outliers
# (outputs up to 12) max 0.113 / mean 0.0039, the causal prefill chunk (outputs up to 11) max 0.094 / mean 0.0024.
# The oracle (fp64) is held to about 1.5x those; a planted slip moves it by far more.
REF_ATTN_BOUND = {"decode_mha": (0.035, 0.003), "decode_gqa": (0.17, 0.006), "prefill": (0.15, 0.004)}


def attention_case(name: str) -> tuple:
    return next(c for c in _maker().ATTENTION_CASES if c[0] == name)


def attention_inputs(case: tuple):
    """The case's K / V rows per (sequence, kv head), its q rows (bf16 bits [n][hq][128]), positions and sequences
    (int32 [n])."""
    mk = _maker()
    name, B, hq, hkv, cached, rows, outl, seed = case
    kv = {(b, h): mk.attention_kv(case, b, h) for b in range(B) for h in range(hkv)}
    q = np.concatenate([G.bf16_bits(mk.attention_q(case, b)) for b in range(B)])
    pos = np.concatenate([c + np.arange(r) for c, r in zip(cached, rows)]).astype(np.int32)
    seq = np.concatenate([np.full(r, b) for b, r in enumerate(rows)]).astype(np.int32)
    return kv, q, pos, seq


def oracle_attention(case: tuple, pos_shift: int = 0, head_of=None, scale: float = 128 ** -0.5) -> np.ndarray:
    """oracle.golden.rows_attention over the case's cache (K / V through the oracle's quantiser, exact here), fp64
    [n][hq][128]; pos_shift, head_of and scale plant slips (keys up to p + pos_shift, kv head head_of(h))."""
    name, B, hq, hkv, cached, rows, outl, seed = case
    kv, q, pos, seq = attention_inputs(case)
    maxb = max(-(-(c + r + 1) // G.PAGE) for c, r in zip(cached, rows))
    cache = G.PagedCache(B * maxb, hkv)
    for (b, h), (k, v) in kv.items():
        kc, ks = G.quantize_rows(G.bf16_bits(k))
        vc, vs = G.quantize_rows(G.bf16_bits(v))
        assert np.array_equal(G.dequantize(kc, ks), k) and np.array_equal(G.dequantize(vc, vs), v)
        t = np.arange(len(k))
        cache.write(G.PagedCache.block_of(np.full(len(t), b), t, None, maxb), h, t % G.PAGE, kc, ks, vc, vs)
    if head_of is None:
        return G.rows_attention(q, pos + pos_shift, seq, cache, None, maxb, B, -1, hq, hkv, scale)
    out = np.zeros((len(pos), hq, 128))
    for h in range(hq):  # each query head alone against kv head head_of(h), copied into a one-head cache
        one = G.PagedCache(cache.num_blocks, 1)
        one.pages[:, 0] = cache.pages[:, head_of(h)]
        out[:, h:h + 1] = G.rows_attention(q[:, h:h + 1], pos + pos_shift, seq, one, None, maxb, B, -1, 1, 1, scale)
    return out


def reference_attention(name: str) -> np.ndarray:
    return G.bf16_to_f32(ATTN[f"{name}_out_bits"]).astype(np.float64)


@pytest.mark.parametrize("name", ["decode_mha", "decode_gqa", "prefill"])
def test_oracle_attention_matches_the_reference(name):
    d = np.abs(oracle_attention(attention_case(name)) - reference_attention(name))
    print(f"{name}: oracle vs reference max {d.max():.4f} mean {d.mean():.5f}")
    mx, mean = REF_ATTN_BOUND[name]
    assert d.max() <= mx and d.mean() <= mean, (d.max(), d.mean())


@pytest.mark.parametrize("slip", ["own key dropped", "one key too many", "kv head h % hkv", "no 1/sqrt(128)"])
def test_reference_attention_catches_slips(slip):
    case = attention_case("decode_gqa" if "kv head" in slip else "prefill")
    G_ = case[2] // case[3]
    kw = {"own key dropped": dict(pos_shift=-1), "one key too many": dict(pos_shift=1),
          "kv head h % hkv": dict(head_of=lambda h: h % case[3]), "no 1/sqrt(128)": dict(scale=1.0)}[slip]
    if "kv head" in slip:
        assert G_ > 1
    d = np.abs(oracle_attention(case, **kw) - reference_attention(case[0]))
    mx, mean = REF_ATTN_BOUND[case[0]]
    print(f"{slip}: max {d.max():.4f} mean {d.mean():.5f}")
    assert d.max() > mx or d.mean() > mean, f"{slip} passed the comparison: not pinned"


@pytest.mark.parametrize("theta", ["10000", "1000000"])
def test_reference_rows_quantise_as_torch_does(theta):
    """The fp8 scheme (per-row absmax scale, e4m3) on the reference's own QK-norm + RoPE output rows:
    the oracle's quantize_rows against the same scheme written in torch (absmax / 448 in fp32, x / scale cast by
    torch to float8_e4m3fn), codes and scales bit for bit (the GPU append equals the oracle's bytes)."""
    import torch

    y_bits = QK[f"y_bits_{theta}"]
    codes, scale = G.quantize_rows(y_bits)
    x = torch.from_numpy(y_bits.view(np.int16)).view(torch.bfloat16).float()
    s = x.abs().amax(-1) / 448.0
    safe = torch.where(s == 0, torch.ones_like(s), s)
    c = (x / safe[:, None]).to(torch.float8_e4m3fn).view(torch.uint8)
    c = torch.where((s == 0)[:, None], torch.zeros_like(c), c)
    np.testing.assert_array_equal(scale, s.numpy())
    np.testing.assert_array_equal(codes, c.numpy())
