"""The C++ decoder handle (csrc/decoder.hip, the dec_* entry points) as a backend of serving.serve.

The handle owns the whole decode step: the embedding, every layer, the lm_head, the token choice and its commit run
from graphs it captured, over fp8 caches it allocated, so the host only moves slot state and reads tokens. This
module binds it with ctypes and maps serve's five calls onto the dec_* protocol (the calling order the reference's
handle defines, model/kernels/decode.cu:1026-1131):

  admit   -> dec_load_prompt (a stored prompt) or a prefill queue entry, then dec_set_prompt
  step    -> dec_prefill over the queue, dec_save_prompt of each newly prefilled prompt, dec_set_active (when the
             active slots changed), dec_launch_body, the masked slots' rows into dec_masks while the body runs,
             dec_set_active with the masked slots, dec_launch_head, dec_tokens
  take_alt-> dec_take_alt
  retire  -> nothing on the device: the next dec_set_active idles the slot

The prompt store is position-granular: serving.PromptStore hands out store positions back to back (a prompt of n
cached positions takes n, at whatever position the previous one ended), exactly the offsets dec_save_prompt and
dec_load_prompt receive.
"""

from __future__ import annotations

import ctypes
import weakref
from typing import Callable, Iterable, Iterator

import numpy as np
import torch

from nanochat_amd.decoder import Weights
from nanochat_amd.native import hip_library
from nanochat_amd.rotary import rotary_tables
from nanochat_amd.sampling import allow_rows, slot_masks
from nanochat_amd.serving import PromptStore, Request, prompt_positions, prompt_rows, serve


def _release(lib, handle, keep) -> None:
    """Destroys the handle; `keep` (its stream and the weights it reads) is an argument only so that it stays
    referenced until the handle is gone."""
    lib.dec_destroy(handle)


def handle_config(model: Weights, max_length: int, prompt_store: int, bos: int, batch: int) -> np.ndarray:
    """dec_create_v2's configuration fields: the reference's seven (L, C, F, vocab, max_len, store, lazy), then
    this build's kv head count, slot count (0: as many as fit) and embedding dtype (1: bf16)."""
    c = model.cfg
    return np.array([c.layers, c.d_model, c.mlp_mult * c.d_model, c.vocab, max_length, prompt_store, bos,
                     c.kv_heads, batch, 1], dtype=np.int32)


def handle_pointers(model: Weights, cos: torch.Tensor, sin: torch.Tensor) -> list[torch.Tensor | None]:
    """The tensors dec_create reads, in its pointer order: wte, cos, sin, lm_head, then per layer qkv, o, up, down,
    the value-embedding table and gate (None outside value-embedding layers), the q and k norm gains."""
    bf16 = lambda t: t.to(torch.bfloat16).contiguous()
    fp32 = lambda t: t.to(torch.float32).contiguous()
    out: list[torch.Tensor | None] = [bf16(model.wte), cos, sin, bf16(model.lm_head)]
    for lw in model.layers:
        has_ve = "ve" in lw
        out += [bf16(lw["wqkv"]), bf16(lw["wo"]), bf16(lw["wup"]), bf16(lw["wdown"]),
                bf16(lw["ve"]) if has_ve else None, fp32(lw["ve_gate"]) if has_ve else None,
                fp32(lw["q_gain"]), fp32(lw["k_gain"])]
    return out


class NativeDecoder:
    """`batch` slots (0: as many as the free device memory holds, at most 1024) of max_length positions of the
    handle over `model`'s weights; bos ends a continuation; prompt_store: store positions in pinned host memory."""

    @torch.no_grad()
    def __init__(self, model: Weights, *, bos: int, max_length: int, prompt_store: int = 0, batch: int = 0):
        lib = hip_library()
        cfg = model.cfg
        device = model.wte.device
        cos, sin = rotary_tables(max_length, cfg.theta, device)
        tensors = handle_pointers(model, cos, sin)
        scal = np.concatenate([np.stack([model.resid_lambdas.float().cpu().numpy(),
                                         model.x0_lambdas.float().cpu().numpy()], 1).reshape(-1),
                               [cfg.softcap]]).astype(np.float32)
        windows = np.array([cfg.window(l) for l in range(cfg.layers)], dtype=np.int32)
        config = handle_config(model, max_length, prompt_store, bos, batch)
        addresses = np.array([t.data_ptr() if t is not None else 0 for t in tensors], dtype=np.uint64)
        self.stream = torch.cuda.Stream(device)
        torch.cuda.synchronize(device)  # the copies above ran on torch's stream; the handle runs on its own
        raw = lib.dec_create_v2(config.ctypes.data, len(config), addresses.ctypes.data, scal.ctypes.data,
                                windows.ctypes.data, ctypes.c_void_p(self.stream.cuda_stream))
        if not raw:
            raise ValueError(lib.nc_last_error().decode())
        self.lib, self.bos, self.max_length = lib, bos, max_length
        self.handle = ctypes.c_void_p(raw)
        weakref.finalize(self, _release, lib, self.handle, (self.stream, tensors))
        self.batch = lib.dec_batch(self.handle)
        self.rows_per_call = lib.dec_prefill_rows(self.handle)
        words = -(-cfg.vocab // 32)
        self.mask_rows = np.ctypeslib.as_array(
            ctypes.cast(lib.dec_masks(self.handle), ctypes.POINTER(ctypes.c_uint32)), shape=(self.batch, words))
        self.out = np.empty(2 * self.batch, dtype=np.int32)  # dec_tokens fills [choices | alternatives]
        self.store = PromptStore(prompt_store)
        self.queued: list[tuple[int, list[int]]] = []  # (slot, input_ids) admitted for prefill
        self.sent: np.ndarray | None = None  # the slot words of the last dec_set_active
        self.loads = self.alts_taken = 0

    @property
    def stored(self) -> dict[tuple[int, ...], int]:
        return self.store.where

    def generate(self, requests: Iterable[Request]) -> Iterator[tuple[int, list[int]]]:
        """Continuations of requests, consumed lazily; yields (request index, generated ids) in completion order."""
        return serve(self, requests, self.bos)

    # ------------------------------------------------------------------------------------------ SlotBackend
    def admit(self, b: int, index: int, request: Request) -> None:
        n = prompt_positions(request, index, self.max_length)
        ids = [int(t) for t in request.input_ids]
        at = self.store.find(ids)
        if at is None:
            self.queued.append((b, ids))
        else:
            self.lib.dec_load_prompt(self.handle, b, 0, at, n)
            self.loads += 1
        self.lib.dec_set_prompt(self.handle, b, ids[-1], n, float(request.temperature), float(request.top_p),
                                int(np.uint64(request.seed)))

    def step(self, active: list[bool], masks: Callable[[], dict[int, np.ndarray]]) -> tuple[np.ndarray, np.ndarray]:
        lib, h = self.lib, self.handle
        self._prefill_queued()
        words = slot_masks(active)
        if self.sent is None or not np.array_equal(words, self.sent):
            self._set_active(words)
        lib.dec_launch_body(h)
        rows = masks()  # computed while the body runs; the previous dec_tokens has waited for the last head
        if rows:
            for b, allowed in rows.items():
                self.mask_rows[b] = allow_rows(allowed[None])[0].view(np.uint32)
            self._set_active(slot_masks(active, [b in rows for b in range(self.batch)]))
        lib.dec_launch_head(h)
        lib.dec_tokens(h, self.out.ctypes.data)
        return self.out[:self.batch], self.out[self.batch:]

    def take_alt(self, b: int, token: int) -> None:
        self.lib.dec_take_alt(self.handle, b)
        self.alts_taken += 1

    def retire(self, slots: list[int]) -> None:
        pass  # the slot's bit clears in the next step's dec_set_active, which idles it

    # ------------------------------------------------------------------------------------------ helpers
    def _set_active(self, words: np.ndarray) -> None:
        words = np.ascontiguousarray(words)
        self.lib.dec_set_active(self.handle, words.ctypes.data)
        self.sent = words if not words[1].any() else None  # a masked call is resent unmasked next step

    def _prefill_queued(self) -> None:
        """The queued prompts' rows through dec_prefill, rows_per_call at a time, then each prompt into the store
        if it has room (positions handed out back to back)."""
        if not self.queued:
            return
        rows = prompt_rows(self.queued)
        for lo in range(0, rows.shape[1], self.rows_per_call):
            part = np.ascontiguousarray(rows[:, lo:lo + self.rows_per_call])
            self.lib.dec_prefill(self.handle, part.shape[1], part.ctypes.data)
        for b, ids in self.queued:
            at = self.store.claim(ids, len(ids) - 1)
            if at is not None:
                self.lib.dec_save_prompt(self.handle, b, 0, at, len(ids) - 1)
        self.queued = []
