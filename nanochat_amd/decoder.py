"""End-to-end greedy decoding of a random-init nanochat-style transformer over the fp8 KV cache.

The decoder the reference drives through `dec_create` / `dec_prefill` / `dec_launch_body` / `dec_tokens`
(model/kernels/decode.cu:950-1124; host protocol inference/decoder.py:129-222): the prompt minus its last token is
prefilled, then every step feeds one token per sequence and appends the chosen one. Per layer
(decode.cu:848-877, model/modeling.py:104-115):

    h  = x + o_proj(attention(qk_norm_rope(qkv_proj(norm(x)))))     append + attention: this package's kernels
    x' = h + down_proj(relu(up_proj(norm(h)))^2)

with x0 = norm(embed(token)), a final norm, the untied lm_head and the token choice (nc_choose_tokens: greedy, the
largest fp32 logit with the lowest id on ties, unless set_sampling asks for temperature / nucleus sampling). The
weight GEMMs are this package's slot GEMM (nc_slot_gemm_bf16) with the reference's fused epilogues
(decode.cu:169-184,848-877): the norms fold into the qkv, up and lm_head GEMMs as a per-row rstd, ReLU^2 into the
up GEMM, and both residual adds into the o and down GEMMs, in place. Prefill rows use the same calls, which take the
many-rows tile from 512 rows on: every sum in a fixed order, bit-identical to the decode tiles, so a prompt's cache
bytes depend neither on the run nor on the other prompts prefilled with it. The cache append, prefill and decode
attention and the token choice are HIP kernels throughout (a decode step's append and attention are one
nc_decode_step_fp8 call per layer); the decode step is captured once in a hipGraph and replayed.

The architecture is BASELINE config 5's: RoPE, QK-norm, ReLU^2 MLP at 4x, untied embeddings, bf16 weights
N(0, 0.02), full causal attention in every layer. A trained checkpoint (checkpoint.load_hf, the export of
inference/export_hf.py) also brings what config 5 does not name, and the decoder runs it: per-layer sliding windows,
value embeddings (v += 2 sigmoid(ve_gate n) ve[token], inference/modeling_nanochat.py:85-88) and the per-layer
residual / x0 mix (inference/modeling_nanochat.py:170-171), identity at the reference's initialisation.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch
import torch.nn.functional as F
from torch import Tensor

from nanochat_amd.attention import decode_step, decode_workspace, prefill_attention
from nanochat_amd.kv_cache import HEAD_DIM, Fp8KVCache, _require
from nanochat_amd.native import check, hip_library, pointer, stream
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.sampling import choose_tokens, choose_workspace
from nanochat_amd.slot_gemm import NORM_F32, NORM_STORE, RELU2_NORM, RESID, slot_gemm

EPS = torch.finfo(torch.float32).eps  # the RMS norms' epsilon (model/ops/linear.py:20)
# the decode attention's sequence-local pieces (nc_decode_step_fp8_pieces, as the dec_* handle): a request's tokens
# depend on neither the batch nor the other requests (inference/decoder.py:124-125)
PIECE_PAGES = 16


@dataclass(frozen=True)
class ModelConfig:
    """The decoder's architecture. Beyond BASELINE config 5 (full attention everywhere, no value embeddings), the
    fields a trained nanochat checkpoint carries (inference/export_hf.py:63-75): per-layer windows (keys before a
    query; -1 all), the value-embedding layers, the kv head count and the logit cap."""
    layers: int
    d_model: int
    heads: int
    vocab: int
    mlp_mult: int = 4
    theta: float = 10000.0
    windows: tuple[int, ...] = ()     # () : every layer full
    ve_layers: tuple[int, ...] = ()
    n_kv_heads: int = 0               # 0: heads (MHA)
    softcap: float = 15.0

    @property
    def kv_heads(self) -> int:
        return self.n_kv_heads or self.heads

    def window(self, layer: int) -> int:
        return self.windows[layer] if self.windows else -1


@dataclass(frozen=True)
class E2EConfig:
    """the model, the batch, the random prompts' length and the decode steps."""
    name: str
    model: ModelConfig
    batch: int
    prompt: int
    steps: int
    seed: int = 5


CONFIG5 = E2EConfig("cfg5-e2e-l26-d1664-h13-v65536-b128-prompt2048-steps512",
                    ModelConfig(layers=26, d_model=1664, heads=13, vocab=65536), batch=128, prompt=2048, steps=512)


def argmax_rows(logits: Tensor, out: Tensor | None = None) -> Tensor:
    """Greedy choice per row of fp32 logits [rows][cols] (rows contiguous, any row stride): the largest value's
    column, the lowest on ties."""
    if logits.dtype != torch.float32 or not logits.is_cuda or logits.dim() != 2:
        raise ValueError("logits must be a 2-d fp32 tensor on the GPU")
    if logits.stride(1) != 1 or logits.stride(0) < logits.shape[1]:
        raise ValueError("logits rows must be contiguous")
    rows, cols = logits.shape
    if out is None:
        out = torch.empty(rows, dtype=torch.int32, device=logits.device)
    check(hip_library().nc_argmax_f32(pointer(logits), rows, cols, logits.stride(0), pointer(out), stream()))
    return out


class Weights:
    """A model's tensors on the device, as the decoder reads them: wte, lm_head (bf16 [vocab][d]); per layer wqkv
    (q heads, then k heads, then v heads: the fused projection's column blocks, decode.cu:476), wo, wup, wdown (bf16),
    q_gain, k_gain (fp32 [128], the QK-norm weights), and in value-embedding layers ve (bf16 [vocab][H 128]) and
    ve_gate (fp32 [H][d]); resid_lambdas, x0_lambdas (fp32 [layers]) mix each layer's input as
    bf16(resid x + x0 x0) (inference/modeling_nanochat.py:170-171)."""

    cfg: ModelConfig
    wte: Tensor
    lm_head: Tensor
    layers: list
    resid_lambdas: Tensor
    x0_lambdas: Tensor

    @property
    def mixes(self) -> bool:
        """False when every layer's mix is the identity (resid 1, x0 0: the reference's initialisation)."""
        return bool((self.resid_lambdas != 1).any() or (self.x0_lambdas != 0).any())

    def weight_bytes(self, rows: int | None = None) -> int:
        """bf16 weight bytes a decode step reads: every matrix whole, except the embedding table, of which only
        the `rows` rows looked up (one per sequence) are read; rows None counts the whole table."""
        wte = self.wte.numel() if rows is None else min(rows, self.wte.shape[0]) * self.wte.shape[1]
        n = wte + self.lm_head.numel()
        for lw in self.layers:
            n += sum(lw[k].numel() for k in ("wqkv", "wo", "wup", "wdown"))
        return 2 * n


class RandomModel(Weights):
    """bf16 weights N(0, std) from a seeded generator (random init: no checkpoint is loaded); QK-norm gains 1, the
    identity mix, value-embedding tables and gates (if cfg names such layers) N(0, std) and zero."""

    def __init__(self, cfg: ModelConfig, device, seed: int = 5, std: float = 0.02):
        self.cfg = cfg
        g = torch.Generator(device=device).manual_seed(seed)
        d, C = cfg.d_model, cfg.heads * HEAD_DIM
        ckv = cfg.kv_heads * HEAD_DIM

        def w(*shape):
            return (torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std).to(torch.bfloat16)

        self.wte = w(cfg.vocab, d)
        self.layers = []
        for i in range(cfg.layers):
            lw = dict(wqkv=w(C + 2 * ckv, d), wo=w(d, C), wup=w(cfg.mlp_mult * d, d), wdown=w(d, cfg.mlp_mult * d),
                      q_gain=torch.ones(HEAD_DIM, device=device), k_gain=torch.ones(HEAD_DIM, device=device))
            if i in cfg.ve_layers:
                lw["ve"] = w(cfg.vocab, ckv)
                lw["ve_gate"] = torch.zeros((cfg.kv_heads, d), device=device)
            self.layers.append(lw)
        self.lm_head = w(cfg.vocab, d)
        self.resid_lambdas = torch.ones(cfg.layers, device=device)
        self.x0_lambdas = torch.zeros(cfg.layers, device=device)



def rms_norm(x: Tensor) -> Tensor:
    """RMS norm with fp32 statistics, bf16 out (model/modeling.py:47-49), in torch (the CPU-side restatement)."""
    return F.rms_norm(x.float(), (x.shape[-1],), eps=EPS).to(torch.bfloat16)


def add_rms_norm(x: Tensor, delta: Tensor | None, x_out: Tensor | None = None, y: Tensor | None = None) -> Tensor:
    """nc_add_rms_norm_bf16 over rows of x (bf16 [n][d], contiguous): x_out = bf16(x + delta) (in place when x_out
    is x), returns norm(x_out) (written into y if given)."""
    _require(x, "x", torch.bfloat16, 2)
    n, d = x.shape
    for t in (delta, x_out, y):
        if t is not None and (t.shape != x.shape or t.dtype != torch.bfloat16 or not t.is_contiguous()):
            raise ValueError("delta / x_out / y must be contiguous bf16 of x's shape")
    if y is None:
        y = torch.empty_like(x)
    check(hip_library().nc_add_rms_norm_bf16(pointer(x), pointer(delta), pointer(x_out), pointer(y), n, d,
                                             stream()))
    return y


def embed_norm(table: Tensor, tok: Tensor) -> Tensor:
    """nc_embed_rms_norm: bf16 norm(table[tok]) per token (table bf16 or fp32 [vocab][d]; tok int32 [n])."""
    if table.dtype not in (torch.bfloat16, torch.float32) or table.dim() != 2 or not table.is_contiguous():
        raise ValueError("table must be a contiguous bf16 or fp32 [vocab][d] tensor")
    tok = tok.to(torch.int32).contiguous()
    x = torch.empty((tok.shape[0], table.shape[1]), dtype=torch.bfloat16, device=table.device)
    check(hip_library().nc_embed_rms_norm(pointer(table), int(table.dtype == torch.float32), table.shape[0],
                                          pointer(tok), tok.shape[0], table.shape[1], pointer(x), stream()))
    return x


def mix(x: Tensor, x0: Tensor, lr: float, l0: float) -> Tensor:
    """nc_mix_bf16: x = bf16(lr x + l0 x0) in place (contiguous bf16 of one shape)."""
    if x.dtype != torch.bfloat16 or x0.dtype != torch.bfloat16 or x.shape != x0.shape or not (
            x.is_contiguous() and x0.is_contiguous()):
        raise ValueError("mix needs contiguous bf16 x and x0 of one shape")
    check(hip_library().nc_mix_bf16(pointer(x), pointer(x0), x.numel(), float(lr), float(l0), stream()))
    return x


def relu2(x: Tensor) -> Tensor:
    """bf16(relu(x)^2) in place (nc_relu2_bf16)."""
    if x.dtype != torch.bfloat16 or not x.is_contiguous():
        raise ValueError("relu2 needs a contiguous bf16 tensor")
    check(hip_library().nc_relu2_bf16(pointer(x), pointer(x), x.numel(), stream()))
    return x


def value_embed(qkv: Tensor, x: Tensor, tok: Tensor, ve: Tensor, gate: Tensor, hq: int, hkv: int) -> Tensor:
    """nc_value_embed_bf16: in the v heads of the projection rows qkv (bf16 [rows][>= (hq + 2 hkv) 128]),
    v_h = bf16(v_h + 2 sigmoid(gate[h] . norm(x)) ve[tok]_h) (inference/modeling_nanochat.py:85-88). x: the layer
    input rows (bf16 [rows][d]); ve bf16 [vocab][hkv 128]; gate fp32 [hkv][d]. Rows whose token is outside the
    vocabulary are left as they are."""
    rows, d = x.shape
    if qkv.dtype != torch.bfloat16 or qkv.dim() != 2 or qkv.shape[0] != rows or qkv.stride(1) != 1:
        raise ValueError("qkv must be bf16 [rows][cols] with unit column stride")
    if x.dtype != torch.bfloat16 or x.stride(1) != 1:
        raise ValueError("x must be bf16 with unit column stride")
    _require(ve, "ve", torch.bfloat16, 2)
    _require(gate, "gate", torch.float32, 2)
    if ve.shape[1] != hkv * HEAD_DIM or tuple(gate.shape) != (hkv, d):
        raise ValueError(f"ve {tuple(ve.shape)} / gate {tuple(gate.shape)} do not fit {hkv} kv heads, d {d}")
    tok = tok.to(torch.int32).contiguous()
    if tok.numel() != rows:
        raise ValueError(f"{tok.numel()} tokens for {rows} rows")
    check(hip_library().nc_value_embed_bf16(pointer(qkv), qkv.stride(0), pointer(x), x.stride(0), pointer(tok),
                                            pointer(ve), ve.shape[0], pointer(gate), rows, d, hq, hkv, stream()))
    return qkv


class Fp8Decoder:
    """Batch `batch` sequences of at most max_len tokens, one contiguous fp8 cache per layer."""

    def __init__(self, model: Weights, batch: int, max_len: int, device, row_chunk: int = 16384):
        cfg = model.cfg
        self.model, self.cfg, self.batch, self.max_len, self.device = model, cfg, batch, max_len, device
        self.caches = [Fp8KVCache.contiguous(batch, max_len, cfg.kv_heads, device) for _ in range(cfg.layers)]
        self.cos, self.sin = rotary_tables(max_len, cfg.theta, device)
        self.ws = decode_workspace(batch, cfg.heads, cfg.kv_heads, max_len, device)
        self.seq = torch.arange(batch, dtype=torch.int32, device=device)
        self.row_chunk = row_chunk
        self.graph: torch.cuda.CUDAGraph | None = None
        # the slot GEMM takes weight rows in multiples of 32: the lm_head gets zero rows past the vocabulary, whose
        # logits the choice skips
        vp = -(-cfg.vocab // 32) * 32
        self.lm_head = model.lm_head
        if vp != cfg.vocab:
            self.lm_head = torch.zeros((vp, cfg.d_model), dtype=torch.bfloat16, device=device)
            self.lm_head[:cfg.vocab] = model.lm_head
        # the token choice (nc_choose_tokens): greedy until set_sampling; alternatives exclude `lazy`
        self.choose_ws = choose_workspace(batch, cfg.vocab, device)
        self.alt = torch.empty(batch, dtype=torch.int32, device=device)
        self.temperature = self.top_p = self.seeds = self.first = None
        self.slots = self.allow = None  # the choice's slot masks and allowed-token rows (serving.Server sets them)
        self.softcap, self.lazy = cfg.softcap, -1
        self.mixes = model.mixes
        self.lambdas = list(zip(model.resid_lambdas.tolist(), model.x0_lambdas.tolist()))

    def set_sampling(self, temperature, top_p=1.0, seed=0, first=0, softcap: float | None = None) -> None:
        """Per-slot sampling (scalars broadcast; inference/decoder.py:28-40): temperature 0 is greedy, > 0 a
        Gumbel-max sample of softmax(capped logits / temperature) drawn from (seed, position - first) alone, top_p < 1
        nucleus sampling. first: the position of each slot's first generated token. Takes effect for steps launched
        (or graphs captured) afterwards."""
        B, dev = self.batch, self.device
        full = lambda v, dt: torch.as_tensor(np.broadcast_to(np.asarray(v), (B,)).copy()).to(dev, dt).contiguous()
        self.temperature = full(temperature, torch.float32)
        self.top_p = full(top_p, torch.float32)
        self.seeds = full(np.asarray(seed, dtype=np.uint64).view(np.int64), torch.int64)
        self.first = full(first, torch.int32)
        if softcap is not None:
            self.softcap = float(softcap)

    # ---------------------------------------------------------------------------------------------- layers
    def _qkv_append(self, l: int, x: Tensor, pos: Tensor, seq: Tensor, tok: Tensor, q_out: Tensor) -> None:
        """The projection of norm(x) (the norm folded into the GEMM, as in the decode step), the value-embedding mix,
        then QK-norm + RoPE + fp8 append of k, v; q into q_out."""
        lw = self.model.layers[l]
        qkv = slot_gemm(x, lw["wqkv"], NORM_STORE)
        self._value_embed(l, qkv, x, tok)
        self.caches[l].append(qkv, pos, seq, lw["q_gain"], lw["k_gain"], self.cos, self.sin, self.cfg.heads,
                              q_out=q_out)

    def _mix(self, l: int, x: Tensor, x0: Tensor) -> None:
        """x = bf16(resid_lambdas[l] x + x0_lambdas[l] x0) in place (nc_mix_bf16; inference/modeling_nanochat.py:
        170-171); skipped where the mix is the identity (it would return x unchanged)."""
        lr, l0 = self.lambdas[l]
        if self.mixes and (lr != 1.0 or l0 != 0.0):
            mix(x, x0, lr, l0)

    def _value_embed(self, l: int, qkv: Tensor, x: Tensor, tok: Tensor) -> None:
        """In a value-embedding layer, v += 2 sigmoid(ve_gate norm(x)) ve[tok] per head in fp32, rounded to bf16 once,
        in the projection rows qkv (nc_value_embed_bf16; inference/modeling_nanochat.py:85-88, decode.cu:478-493).
        x: the layer input rows."""
        lw = self.model.layers[l]
        if "ve" not in lw:
            return
        value_embed(qkv, x, tok, lw["ve"], lw["ve_gate"], self.cfg.heads, self.cfg.kv_heads)

    def _finish_layer(self, l: int, x: Tensor, o: Tensor) -> None:
        """x += o_proj(o); x += down(relu(up(norm(x)))^2), x updated in place: the decode step's three GEMMs and
        epilogues (decode.cu:848-877)."""
        lw = self.model.layers[l]
        slot_gemm(o.reshape(o.shape[0], -1), lw["wo"], RESID, res=x, out=x)
        u = slot_gemm(x, lw["wup"], RELU2_NORM)
        slot_gemm(u, lw["wdown"], RESID, res=x, out=x)

    # ---------------------------------------------------------------------------------------------- prefill
    @torch.no_grad()
    def prefill(self, prompts: Tensor) -> None:
        """Positions 0..T-2 of every prompt (int32 [batch][T]) into the caches (the last prompt token is the first
        decode step's input, inference/decoder.py:211-222). Per layer every row is appended before any attends
        (decode.cu:859-863); GEMMs and the MLP run in chunks of row_chunk rows (any chunking gives the same bits)."""
        B, T = prompts.shape
        if B != self.batch or T - 1 + 1 > self.max_len:
            raise ValueError(f"prompts {tuple(prompts.shape)} do not fit batch {self.batch}, max_len {self.max_len}")
        if T <= 1:
            return
        tok = prompts[:, :-1].reshape(-1)
        pos = torch.arange(T - 1, dtype=torch.int32, device=self.device).repeat(B)
        seq = torch.arange(B, dtype=torch.int32, device=self.device).repeat_interleave(T - 1)
        self._prefill_rows(tok, pos, seq)

    def _prefill_rows(self, tok: Tensor, pos: Tensor, seq: Tensor) -> None:
        """Rows (token, position, sequence) into the caches, each row attending its sequence's keys up to its
        position; every row of a layer is appended before any attends."""
        n = tok.shape[0]
        x = embed_norm(self.model.wte, tok)  # the residual stream x0 = norm(embed(tok))
        x0 = x.clone() if self.mixes else None
        q = torch.empty((n, self.cfg.heads, HEAD_DIM), dtype=torch.bfloat16, device=self.device)
        o = torch.empty_like(q)
        chunks = [(r, min(r + self.row_chunk, n)) for r in range(0, n, self.row_chunk)]
        for l in range(self.cfg.layers):
            for r0, r1 in chunks:
                if self.mixes:
                    self._mix(l, x[r0:r1], x0[r0:r1])
                self._qkv_append(l, x[r0:r1], pos[r0:r1], seq[r0:r1], tok[r0:r1], q[r0:r1])
            prefill_attention(q, self.caches[l], pos, seq, window=self.cfg.window(l), out=o)
            for r0, r1 in chunks:
                self._finish_layer(l, x[r0:r1], o[r0:r1])

    # ---------------------------------------------------------------------------------------------- decode
    def _step(self, tok: Tensor, pos: Tensor, out_tok: Tensor, slots: Tensor | None = None) -> Tensor:
        """One decode step: token tok[b] at position pos[b] of sequences b < len(tok) (all, or the first ones: the
        narrow step, whose slot masks `slots` replace self.slots); the choice (greedy, or by set_sampling) into
        out_tok, its alternative into self.alt, then pos += 1 (the commit). Returns the fp32 logits. Per layer four
        slot GEMMs (decode.cu:848-877): qkv of norm(x), then append and attention; x += o_proj(o);
        u = relu(up(norm(x)))^2; x += down(u)."""
        n = tok.shape[0]
        part = lambda t: None if t is None else t[:n]
        x = embed_norm(self.model.wte, tok)  # the residual stream x0 = norm(embed(tok))
        x0 = x.clone() if self.mixes else None
        for l in range(self.cfg.layers):
            lw = self.model.layers[l]
            nxt = self.model.layers[l + 1]["wqkv"] if l + 1 < self.cfg.layers else None
            self._mix(l, x, x0)
            # each GEMM's idle compute units pull the next GEMM's weights into the memory-side cache (the o GEMM
            # is too short to hide the up weights' read)
            qkv = slot_gemm(x, lw["wqkv"], NORM_STORE, prefetch=lw["wo"])
            self._value_embed(l, qkv, x, tok)
            # the append (decode.cu:550-565) and attention in one call: sequence b is cache row b
            o = decode_step(qkv, self.caches[l], pos, lw["q_gain"], lw["k_gain"], self.cos, self.sin, self.cfg.heads,
                            max_ctx=self.max_len, window=self.cfg.window(l), workspace=self.ws,
                            piece_pages=PIECE_PAGES)
            slot_gemm(o.reshape(o.shape[0], -1), lw["wo"], RESID, res=x, out=x)
            u = slot_gemm(x, lw["wup"], RELU2_NORM, prefetch=lw["wdown"])
            slot_gemm(u, lw["wdown"], RESID, res=x, out=x, prefetch=nxt)
        logits = slot_gemm(x, self.lm_head, NORM_F32)
        choose_tokens(logits, self.cfg.vocab, pos, temperature=part(self.temperature), top_p=part(self.top_p),
                      seed=part(self.seeds), first=part(self.first), slots=self.slots if slots is None else slots,
                      allow=part(self.allow), softcap=self.softcap, lazy=self.lazy, tokens=out_tok,
                      alt_tokens=self.alt[:n], workspace=self.choose_ws)
        return logits[:, :self.cfg.vocab]

    @torch.no_grad()
    def start(self, last_tokens: Tensor, position: int) -> None:
        """Decode state: every sequence's next input token (int32 [batch]) at `position`; captures the step graph
        (positions and the token history advance on the device: the choice commits pos + 1)."""
        B = self.batch
        self.tok = last_tokens.to(torch.int32).clone()
        self.pos = torch.full((B,), position, dtype=torch.int32, device=self.device)
        self.next = torch.empty(B, dtype=torch.int32, device=self.device)
        self.history = torch.empty((self.max_len, B), dtype=torch.int32, device=self.device)
        self.step_idx = torch.zeros(1, dtype=torch.int64, device=self.device)
        s = torch.cuda.Stream(self.device)
        s.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(s):
            # warm every launch path, then restore the state the warm-up advanced
            self._step(self.tok, self.pos, self.next)
            self.pos.fill_(position)
            s.synchronize()
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=s):
                self._step(self.tok, self.pos, self.next)
                self.history.index_copy_(0, self.step_idx, self.next.unsqueeze(0))
                self.tok.copy_(self.next)
                self.step_idx.add_(1)
        torch.cuda.current_stream(self.device).wait_stream(s)
        self.stream = s

    def run(self, steps: int) -> None:
        """Replay the decode step `steps` times (asynchronous on the decoder's stream)."""
        if self.graph is None:
            raise RuntimeError("start() first")
        with torch.cuda.stream(self.stream):
            for _ in range(steps):
                self.graph.replay()

    def tokens(self, steps: int) -> Tensor:
        """The first `steps` chosen tokens, int32 [batch][steps] (synchronises)."""
        torch.cuda.current_stream(self.device).wait_stream(self.stream)
        return self.history[:steps].t().contiguous()


def generate(cfg: E2EConfig, device, steps: int | None = None, timing: bool = False):
    """Random prompts (seeded), prefill, greedy decode. Returns (tokens [batch][steps], timings dict)."""
    steps = cfg.steps if steps is None else steps
    model = RandomModel(cfg.model, device, seed=cfg.seed)
    g = torch.Generator(device=device).manual_seed(cfg.seed + 1)
    prompts = torch.randint(0, cfg.model.vocab, (cfg.batch, cfg.prompt), generator=g, device=device,
                            dtype=torch.int64).to(torch.int32)
    dec = Fp8Decoder(model, cfg.batch, cfg.prompt - 1 + steps, device)
    torch.cuda.synchronize(device)
    e = [torch.cuda.Event(enable_timing=True) for _ in range(4)]
    e[0].record()
    dec.prefill(prompts)
    e[1].record()
    torch.cuda.synchronize(device)
    dec.start(prompts[:, -1], cfg.prompt - 1)
    torch.cuda.synchronize(device)
    with torch.cuda.stream(dec.stream):
        e[2].record(dec.stream)
        dec.run(steps)
        e[3].record(dec.stream)
    e[3].synchronize()
    toks = dec.tokens(steps)
    prefill_ms, decode_ms = e[0].elapsed_time(e[1]), e[2].elapsed_time(e[3])
    info = {"prefill_ms": prefill_ms, "decode_ms": decode_ms, "decode_ms_per_step": decode_ms / max(steps, 1),
            "weight_bytes": model.weight_bytes(rows=cfg.batch)}
    return toks, info, (model, dec, prompts)
