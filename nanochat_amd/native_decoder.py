"""The decoder handle from Python: inference/decoder.py's NativeDecoder (:123-324) over this library's dec_* entry
points (nanochat_amd/csrc/decoder.hip), with the same protocol: start a request in a slot (its prompt loaded from
the prompt store or queued for prefill), prefill the queued prompts in chunks of dec_prefill_rows rows, then per
step set the active and masked slots, launch the body and the head, read the tokens, and give a rejected lazy BOS
its alternative (dec_take_alt).

The native handle runs the whole step (embedding, every layer, lm_head, the choice and its commit) from captured
graphs, so the host only reads tokens; serving.Server is the same protocol driven from torch (Fp8Decoder). A
request is serving.Request. The prompt store keeps whole 16-position pages: a prompt of n positions takes
ceil(n / 16) pages of it.
"""

from __future__ import annotations

import ctypes
import weakref
from typing import Iterable, Iterator

import numpy as np
import torch

from nanochat_amd.decoder import Weights
from nanochat_amd.kv_cache import PAGE
from nanochat_amd.native import hip_library
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.sampling import allow_rows
from nanochat_amd.serving import Request


def _destroy(lib, handle, stream, weights) -> None:
    """dec_destroy; stream and weights are arguments only so that they stay referenced until the handle is gone."""
    lib.dec_destroy(handle)


class NativeDecoder:
    """Up to `batch` slots (0: as many as the free device memory holds, at most 1024) of max_length positions over
    `model`'s weights (kept referenced: the handle reads them through pointers); bos ends a continuation;
    prompt_store: positions of pinned host memory for prefilled prompts."""

    @torch.no_grad()
    def __init__(self, model: Weights, *, bos: int, max_length: int, prompt_store: int = 0, batch: int = 0):
        lib = hip_library()
        cfg = model.cfg
        device = model.wte.device
        self.lib, self.cfg, self.bos, self.max_length = lib, cfg, bos, max_length
        cos, sin = rotary_tables(max_length, cfg.theta, device)
        bf = lambda t: t.to(torch.bfloat16).contiguous()
        f32 = lambda t: t.to(torch.float32).contiguous()
        weights = [bf(model.wte), cos, sin, bf(model.lm_head)]
        for lw in model.layers:
            ve = "ve" in lw
            weights += [bf(lw["wqkv"]), bf(lw["wo"]), bf(lw["wup"]), bf(lw["wdown"]), bf(lw["ve"]) if ve else None,
                        f32(lw["ve_gate"]) if ve else None, f32(lw["q_gain"]), f32(lw["k_gain"])]
        self.weights = weights  # referenced while the handle reads them
        lambdas = torch.stack([model.resid_lambdas.float().cpu(), model.x0_lambdas.float().cpu()], 1).flatten()
        scal = np.append(lambdas.numpy(), np.float32(cfg.softcap)).astype(np.float32)
        window = np.array([cfg.window(l) for l in range(cfg.layers)], dtype=np.int32)
        # dec_create_v2's fields: L, C, F, vocab, max_len, store, lazy, then Hkv, slots, bf16 embedding
        config = np.array([cfg.layers, cfg.d_model, cfg.mlp_mult * cfg.d_model, cfg.vocab, max_length, prompt_store,
                           bos, cfg.kv_heads, batch, 1], dtype=np.int32)
        ptrs = np.array([0 if t is None else t.data_ptr() for t in weights], dtype=np.uint64)
        self.stream = torch.cuda.Stream(device)
        torch.cuda.synchronize(device)  # the weight copies above are on the current stream; the handle uses its own
        handle = lib.dec_create_v2(config.ctypes.data, len(config), ptrs.ctypes.data, scal.ctypes.data,
                                   window.ctypes.data, ctypes.c_void_p(self.stream.cuda_stream))
        if not handle:
            raise ValueError(lib.nc_last_error().decode())
        self.handle = ctypes.c_void_p(handle)
        # the finalizer holds the stream and the weights, so both outlive the handle it destroys
        weakref.finalize(self, _destroy, lib, self.handle, self.stream, weights)
        self.batch = B = lib.dec_batch(self.handle)
        self.tokens = np.zeros(2 * B, dtype=np.int32)  # dec_tokens: the choices, then their alternatives
        words = -(-cfg.vocab // 32)
        self.masks = np.ctypeslib.as_array(ctypes.cast(lib.dec_masks(self.handle), ctypes.POINTER(ctypes.c_uint32)),
                                           shape=(B, words))
        self.prefill_rows = lib.dec_prefill_rows(self.handle)
        self.pending: list[tuple[int, list[int]]] = []  # started slots whose prompts await prefill
        self.store_pages = -(-prompt_store // PAGE)
        self.stored: dict[tuple[int, ...], int] = {}  # prompt -> its first store position
        self.used = 0  # store positions taken (whole pages)
        self.loads = self.alts_taken = 0

    def start(self, b: int, index: int, request: Request) -> None:
        """Start request `index` in slot b at its prompt's last token; earlier positions loaded or queued to
        prefill (inference/decoder.py:196-211)."""
        n = len(request.input_ids) - 1
        if n < 1 or request.max_new_tokens < 1 or n + request.max_new_tokens > self.max_length:
            raise ValueError(f"request {index}: {n + 1} prompt tokens and {request.max_new_tokens} new tokens do not "
                             f"fit max_length {self.max_length}")
        at = self.stored.get(tuple(request.input_ids))
        if at is None:
            self.pending.append((b, list(request.input_ids)))
        else:
            self._check(self.lib.dec_load_prompt(self.handle, b, 0, at, n))
            self.loads += 1
        self.lib.dec_set_prompt(self.handle, b, int(request.input_ids[-1]), n, float(request.temperature),
                                float(request.top_p), int(np.uint64(request.seed)))

    def prefill(self) -> None:
        """Prefill the pending prompts but their last tokens, prefill_rows rows a launch, then store each."""
        if not self.pending:
            return
        rows = np.concatenate([np.array([ids[:-1], range(len(ids) - 1), [b] * (len(ids) - 1)], dtype=np.int32)
                               for b, ids in self.pending], axis=1)
        for i in range(0, rows.shape[1], self.prefill_rows):
            chunk = np.ascontiguousarray(rows[:, i:i + self.prefill_rows])
            self.lib.dec_prefill(self.handle, chunk.shape[1], chunk.ctypes.data)
        for b, ids in self.pending:
            self.save(b, ids)
        self.pending = []

    def save(self, b: int, input_ids: list[int]) -> None:
        """Keep slot b's prompt pages in the store's next free pages, unless stored already or out of room."""
        key, n = tuple(input_ids), len(input_ids) - 1
        pages = -(-n // PAGE)
        if key in self.stored or self.used // PAGE + pages > self.store_pages:
            return
        self._check(self.lib.dec_save_prompt(self.handle, b, 0, self.used, n))
        self.stored[key] = self.used
        self.used += pages * PAGE

    def _check(self, status: int) -> None:
        if status < 0:
            raise ValueError(self.lib.nc_last_error().decode())

    @torch.no_grad()
    def generate(self, requests: Iterable[Request]) -> Iterator[tuple[int, list[int]]]:
        """Continuations of requests, consumed lazily; yields (request index, generated ids) in completion order
        (inference/decoder.py:250-324). Raises ValueError when a request's mask allows no token."""
        lib, handle, B, bos = self.lib, self.handle, self.batch, self.bos
        queue = enumerate(requests)
        slots: list[tuple[int, Request, list[int]] | None] = [None] * B
        flags = np.zeros((2, -(-B // 64) * 64), dtype=bool)  # active slots, masked slots

        def set_active() -> None:
            words = np.packbits(flags, axis=1, bitorder="little").view("<u8")
            lib.dec_set_active(handle, np.ascontiguousarray(words).ctypes.data)

        def fill(b: int) -> None:
            for i, r in queue:
                self.start(b, i, r)
                slots[b] = (i, r, [])
                flags[0, b] = True
                return
            slots[b] = None
            flags[0, b] = False

        for b in range(B):
            fill(b)
        set_active()
        while flags[0].any():
            self.prefill()
            lib.dec_launch_body(handle)
            for b, s in enumerate(slots):  # the masked slots' allowed rows (the previous dec_tokens has waited)
                if s is None or s[1].mask is None:
                    continue
                allowed = s[1].mask(s[2])
                if allowed is not None:
                    self.masks[b] = allow_rows(np.asarray(allowed, bool)[None])[0].view(np.uint32)
                    flags[1, b] = True
            set_active()
            flags[1] = False
            lib.dec_launch_head(handle)
            lib.dec_tokens(handle, self.tokens.ctypes.data)
            finished = []
            for b, s in enumerate(slots):
                if s is None:
                    continue
                index, r, out = s
                token = int(self.tokens[b])
                if token == bos and r.accept_bos and not r.accept_bos(out):
                    token = int(self.tokens[B + b])  # the lazy BOS rejected: the alternative (dec_take_alt)
                    if token < 0:
                        raise ValueError(f"request {index}: nothing but BOS allowed at position {len(out)}")
                    lib.dec_take_alt(handle, b)
                    self.alts_taken += 1
                if token == bos:
                    finished.append(b)
                    continue
                if token < 0:
                    raise ValueError(f"request {index}: its mask allows no token at position {len(out)}")
                out.append(token)
                if len(out) == r.max_new_tokens or (r.stopping_criteria and r.stopping_criteria(out)):
                    finished.append(b)
            if finished:
                for b in finished:
                    index, _, out = slots[b]
                    fill(b)
                    yield index, out
                set_active()
