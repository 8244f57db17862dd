"""CPU restatement of the decoder (TEST INFRASTRUCTURE ONLY; see oracle/__init__.py): the model of
nanochat_amd.decoder on the CPU, torch bf16 tensors and GEMMs, with golden.py's append (QK-norm + RoPE + fp8
quantisation into the page layout) and fp64 attention over the dequantised cache.

Per layer (inference/modeling_nanochat.py:84-100,120-175; model/kernels/decode.cu:848-877): the residual / x0 mix,
qkv = norm(x) W_qkv, the value-embedding term in value-embedding layers, the append of every row before any row
attends (decode.cu:859-863), attention, x += o W_o, x += relu(norm(x) W_up)^2 W_down; the head is
norm(x) W_lm in fp32. It reads the same weights the GPU decoder reads (a nanochat_amd.decoder.Weights) and keeps
its own host copy of the cache layout, so the GPU's cache bytes can be compared with it.
"""

from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from oracle import golden as G

EPS = float(np.finfo(np.float32).eps)  # model/ops/linear.py:20


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def cpu_norm(x: torch.Tensor) -> torch.Tensor:
    """RMS norm with fp32 statistics, bf16 out (model/modeling.py:47-49)."""
    return F.rms_norm(x.float(), (x.shape[-1],), eps=EPS).to(torch.bfloat16)


class CpuModel:
    """`batch` sequences of at most max_len positions of `model` (a Weights) on the CPU."""

    def __init__(self, model, batch: int, max_len: int):
        cfg = model.cfg
        self.cfg, self.batch = cfg, batch
        self.w = [{k: v.cpu() for k, v in lw.items()} for lw in model.layers]
        self.wte, self.lm_head = model.wte.cpu(), model.lm_head.cpu()
        self.lr, self.l0 = model.resid_lambdas.cpu(), model.x0_lambdas.cpu()
        self.max_blocks = -(-max_len // G.PAGE)
        self.caches = [G.PagedCache(batch * self.max_blocks, cfg.kv_heads) for _ in range(cfg.layers)]
        self.cos, self.sin = G.rotary_tables(max_len, cfg.theta)

    def _mix(self, l, x, x0):
        """inference/modeling_nanochat.py:170-171: bf16(resid h + x0 x0) in fp32."""
        return (self.lr[l] * x.float() + self.l0[l] * x0.float()).to(torch.bfloat16)

    def _layer(self, l, x, pos, seq, tok, attend):
        lw, cfg = self.w[l], self.cfg
        n = cpu_norm(x)
        qkv = n @ lw["wqkv"].t()
        if "ve" in lw:  # inference/modeling_nanochat.py:85-88
            H = cfg.kv_heads
            gate = 2 * torch.sigmoid(F.linear(n.float(), lw["ve_gate"]))
            v = qkv[:, (cfg.heads + H) * 128:].reshape(-1, H, 128)
            ve = lw["ve"][torch.from_numpy(np.asarray(tok, np.int64))].reshape(-1, H, 128)
            qkv[:, (cfg.heads + H) * 128:] = (v.float() + gate[..., None] * ve.float()).to(torch.bfloat16).flatten(1)
        q = G.append(self.caches[l], bits(qkv), pos, seq, lw["q_gain"].numpy(), lw["k_gain"].numpy(), self.cos,
                     self.sin, cfg.heads, cfg.kv_heads, None, self.max_blocks)
        o = torch.from_numpy(attend(q, self.caches[l]).astype(np.float32)).to(torch.bfloat16)
        x = x + o.reshape(o.shape[0], -1) @ lw["wo"].t()
        u = (cpu_norm(x) @ lw["wup"].t()).float().relu().square().to(torch.bfloat16)
        return x + u @ lw["wdown"].t()

    def prefill(self, prompts: np.ndarray, seqs: np.ndarray | None = None) -> None:
        """Positions 0..T-2 of every prompt (int [n][T]) into sequences seqs (default 0..n-1)."""
        B, T = prompts.shape
        seqs = np.arange(B) if seqs is None else np.asarray(seqs)
        self.prefill_rows(prompts[:, :-1].reshape(-1), np.tile(np.arange(T - 1), B), np.repeat(seqs, T - 1))

    def prefill_rows(self, tok: np.ndarray, pos: np.ndarray, seq: np.ndarray) -> None:
        """Rows (token, position, sequence): every row's key and value appended in each layer before any row
        attends its sequence's cached keys up to its position (a chunk of a prompt after its earlier chunks)."""
        tok, pos, seq = np.asarray(tok), np.asarray(pos), np.asarray(seq)
        x, x0 = self._embed(tok)
        scale = 128 ** -0.5
        for l in range(self.cfg.layers):
            w = self.cfg.window(l)
            x = self._block(l, x, x0, pos, seq, tok, lambda q, c: G.rows_attention(
                q, pos, seq, c, None, self.max_blocks, self.batch, w, self.cfg.heads, self.cfg.kv_heads, scale))

    def step(self, tok: np.ndarray, position) -> np.ndarray:
        """One decode step of every sequence: token tok[b] at position (an int, or one per sequence); returns the
        fp32 logits [batch][vocab]."""
        B = self.batch
        pos, seq = np.broadcast_to(np.asarray(position), (B,)).copy(), np.arange(B)
        x, x0 = self._embed(tok)
        scale = 128 ** -0.5
        for l in range(self.cfg.layers):
            w = self.cfg.window(l)
            x = self._block(l, x, x0, pos, seq, tok, lambda q, c: G.decode_attention(
                q, c, None, self.max_blocks, pos + 1, w, self.cfg.heads, self.cfg.kv_heads, scale))
        return (cpu_norm(x).float() @ self.lm_head.float().t()).numpy()

    def _embed(self, tok):
        """The residual stream and x0 of tokens tok: both the normed embedding, bf16 (modeling_nanochat.py:150-151)."""
        x0 = cpu_norm(self.wte[torch.from_numpy(np.asarray(tok).astype(np.int64))])
        return x0, x0

    def _block(self, l, x, x0, pos, seq, tok, attend):
        return self._layer(l, self._mix(l, x, x0), pos, seq, tok, attend)


def _rstd(v: torch.Tensor) -> torch.Tensor:
    """rsqrt(mean(v^2) + FLT_EPSILON) per row of an fp32 tensor, in fp32 (the sum in fp64, then rounded)."""
    return torch.rsqrt((v.double().square().mean(-1) + EPS).float())


class EngineCpuModel(CpuModel):
    """CpuModel with the reference CUDA engine's roundings (model/kernels/decode.cu) instead of its torch path's:
    x0 stays fp32 (k_norm EMBED, decode.cu:413-440: v r unrounded); each layer's mix is fma(l1, h, x0 l2) in fp32
    with h = x0 at layer 0, rounded to bf16 for the residual, while the qkv input is bf16(v r) of the unrounded v
    (RESID_NORM); the GEMMs sum in fp32 and round once in their epilogues (decode.cu:169-186); the o-projection's
    fp32 sum (residual included, before rounding) gives the MLP's rstd (k_rstd, decode.cu:443-455) and RELU2 is
    bf16(max(p, 0) p) with p = rstd s (decode.cu:173-176). The attention, the append and the head are CpuModel's.
    Test infrastructure: it measures how often greedy tokens differ between the two roundings; no test pins it to
    the CUDA engine's bits (parity unpinned: the engine needs CUDA)."""

    def __init__(self, model, batch: int, max_len: int):
        super().__init__(model, batch, max_len)
        self.wf = [{k: lw[k].float() for k in ("wqkv", "wo", "wup", "wdown")} for lw in self.w]

    def _embed(self, tok):
        v = self.wte[torch.from_numpy(np.asarray(tok).astype(np.int64))].float()
        return None, v * _rstd(v)[:, None]

    def _block(self, l, x, x0, pos, seq, tok, attend):
        lw, wf, cfg = self.w[l], self.wf[l], self.cfg
        h = x0 if x is None else x.float()
        a = (x0 * self.l0[l].float()).double()
        v = (self.lr[l].double() * h.double() + a).float()  # one rounding: the fma
        mixed = v.to(torch.bfloat16)
        n = (v * _rstd(v)[:, None]).to(torch.bfloat16)
        qkv = (n.float() @ wf["wqkv"].t()).to(torch.bfloat16)
        if "ve" in lw:
            H = cfg.kv_heads
            gate = 2 * torch.sigmoid(F.linear(n.float(), lw["ve_gate"]))
            vv = qkv[:, (cfg.heads + H) * 128:].reshape(-1, H, 128)
            ve = lw["ve"][torch.from_numpy(np.asarray(tok, np.int64))].reshape(-1, H, 128)
            qkv[:, (cfg.heads + H) * 128:] = (vv.float() + gate[..., None] * ve.float()).to(torch.bfloat16).flatten(1)
        q = G.append(self.caches[l], bits(qkv), pos, seq, lw["q_gain"].numpy(), lw["k_gain"].numpy(), self.cos,
                     self.sin, cfg.heads, cfg.kv_heads, None, self.max_blocks)
        o = torch.from_numpy(attend(q, self.caches[l]).astype(np.float32)).to(torch.bfloat16)
        xf = o.reshape(o.shape[0], -1).float() @ wf["wo"].t() + mixed.float()
        xo = xf.to(torch.bfloat16)
        p = (xo.float() @ wf["wup"].t()) * _rstd(xf)[:, None]
        u = (p.clamp_min(0.0) * p).to(torch.bfloat16)
        return (xo.float() + u.float() @ wf["wdown"].t()).to(torch.bfloat16)
