"""Continuous batching over a decoder's slots: the host protocol of the reference's NativeDecoder.generate
(inference/decoder.py:28-40,194-324) on this package's kernels.

One loop (`serve`) drives either backend: `Server`, whose step is a captured hipGraph of torch-launched kernels over
an Fp8Decoder, and `native_decoder.NativeDecoder`, whose step is the C++ decoder handle's (dec_*). The loop owns the
requests and the slots; a backend owns the device state. Per step:

  1. every free slot takes the next queued request (`admit`: the backend loads the prompt from its store or queues
     it for prefill, and sets the slot's token, position, first generated position and sampling parameters);
  2. the backend runs one decode step over every slot (`step`): it prefills the queued prompts, asks the loop for
     the masked slots' allowed tokens (`masks`, the requests' mask callables: the reference's constraints and
     dec_masks rows, decode.cu:1077-1094) and returns every slot's choice and alternative (the best token but BOS);
  3. the loop finishes a slot on BOS (dropped; unless the request's accept_bos rejects it, when the alternative is
     taken instead through the backend's `take_alt`, the reference's lazy BOS), at max_new_tokens, or when the
     request's stopping criteria hold, and the backend idles it (`retire`) before the slot is refilled.

Idle slots carry position -1: the fused decode step does no work for them and the token choice leaves them
untouched. As the reference's narrow graphs (decode.cu:32-33,995-1005,1090-1093), a second graph over the first
`narrow` slots runs the steps in which no higher slot is active.

The prompt store (decode.cu:1053-1075; inference/decoder.py:196-232): pinned host memory for `prompt_store`
positions holding prefilled prompts as position rows (nc_kv_export_fp8's layout: a position's fp8 K and V codes and
scales per kv head and layer). `PromptStore` hands out positions back to back, one run per prompt, never evicted;
a later request with the same input_ids loads its rows into the slot instead of prefilling.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Iterable, Iterator, Protocol, Sequence

import numpy as np
import torch

from nanochat_amd.decoder import Fp8Decoder, Weights
from nanochat_amd.kv_cache import ROW_BYTES
from nanochat_amd.sampling import allow_rows, slot_masks


@dataclass(frozen=True, kw_only=True)
class Request:
    """A continuation of input_ids (at least two tokens) by at most max_new_tokens (>= 1) tokens (inference/decoder.py
    :28-40): temperature 0 argmax, > 0 a sample drawn from (seed, generated position) alone, top_p < 1 nucleus."""
    input_ids: Sequence[int]
    max_new_tokens: int
    stopping_criteria: Callable[[list[int]], bool] | None = None
    mask: Callable[[list[int]], np.ndarray | None] | None = None  # generated so far -> bool [vocab] or None
    accept_bos: Callable[[list[int]], bool] | None = None  # False: a chosen BOS gives way to the alternative
    temperature: float = 0.0
    top_p: float = 1.0
    seed: int = 0


def prompt_positions(request: Request, index: int, max_len: int) -> int:
    """The cache positions of a request's prompt before its last token (that token is the first step's input);
    raises ValueError when the prompt and its new tokens do not fit max_len positions."""
    n = len(request.input_ids) - 1
    if n < 1 or request.max_new_tokens < 1 or n + request.max_new_tokens > max_len:
        raise ValueError(f"request {index}: {n + 1} prompt tokens and {request.max_new_tokens} new tokens do not "
                         f"fit {max_len} positions")
    return n


def prompt_rows(prompts: Sequence[tuple[int, Sequence[int]]]) -> np.ndarray:
    """The prefill rows of (slot, input_ids) prompts: int32 [3][n] (token, position, slot) over every prompt's
    positions but its last, prompt after prompt."""
    cols = [(np.asarray(ids[:-1], np.int32), np.arange(len(ids) - 1, dtype=np.int32),
             np.full(len(ids) - 1, slot, np.int32)) for slot, ids in prompts]
    return np.stack([np.concatenate(part) for part in zip(*cols)]) if cols else np.zeros((3, 0), np.int32)


class PromptStore:
    """Where each stored prompt's rows sit in a store of `positions` positions: prompts take consecutive runs in the
    order they are stored (a prompt of n cached positions takes n), once each, never evicted."""

    def __init__(self, positions: int):
        self.positions, self.used = positions, 0
        self.where: dict[tuple[int, ...], int] = {}

    def find(self, ids: Sequence[int]) -> int | None:
        return self.where.get(tuple(int(t) for t in ids))

    def claim(self, ids: Sequence[int], n: int) -> int | None:
        """The first position of a new run of n positions for prompt ids, or None when it is stored already or the
        store has no room left."""
        key = tuple(int(t) for t in ids)
        if key in self.where or self.used + n > self.positions:
            return None
        self.where[key] = at = self.used
        self.used += n
        return at


class SlotBackend(Protocol):
    """What `serve` needs of a decoder: `batch` slots, and the five calls of the module docstring."""
    batch: int

    def admit(self, b: int, index: int, request: Request) -> None: ...

    def step(self, active: list[bool], masks: Callable[[], dict[int, np.ndarray]]) -> tuple[np.ndarray, np.ndarray]:
        ...

    def take_alt(self, b: int, token: int) -> None: ...

    def retire(self, slots: list[int]) -> None: ...


@dataclass
class _Slot:
    index: int
    request: Request
    out: list


def serve(backend: SlotBackend, requests: Iterable[Request], bos: int) -> Iterator[tuple[int, list[int]]]:
    """Continuations of requests over the backend's slots, consumed lazily; yields (request index, generated ids) in
    completion order. Raises ValueError when a request's mask allows no token."""
    queue = enumerate(requests)
    slots: list[_Slot | None] = [None] * backend.batch

    def refill(b: int) -> None:
        slots[b] = None
        for index, request in queue:
            backend.admit(b, index, request)
            slots[b] = _Slot(index, request, [])
            return

    def masks() -> dict[int, np.ndarray]:
        """The masked slots' allowed tokens for their next position."""
        rows = {}
        for b, s in enumerate(slots):
            if s is not None and s.request.mask is not None:
                allowed = s.request.mask(s.out)
                if allowed is not None:
                    rows[b] = np.asarray(allowed, bool)
        return rows

    for b in range(backend.batch):
        refill(b)
    while any(s is not None for s in slots):
        chosen, alts = backend.step([s is not None for s in slots], masks)
        done = []
        for b, s in enumerate(slots):
            if s is None:
                continue
            token = int(chosen[b])
            if token == bos and s.request.accept_bos is not None and not s.request.accept_bos(s.out):
                token = int(alts[b])  # the lazy BOS rejected: the step's alternative is the slot's next input
                if token < 0:
                    raise ValueError(f"request {s.index}: nothing but BOS allowed at position {len(s.out)}")
                backend.take_alt(b, token)
            if token == bos:
                done.append(b)
                continue
            if token < 0:
                raise ValueError(f"request {s.index}: its mask allows no token at position {len(s.out)}")
            s.out.append(token)
            r = s.request
            if len(s.out) == r.max_new_tokens or (r.stopping_criteria is not None and r.stopping_criteria(s.out)):
                done.append(b)
        if done:
            backend.retire(done)
            for b in done:
                finished = slots[b]
                refill(b)
                yield finished.index, finished.out


class Server:
    """`batch` slots over one Fp8Decoder (torch-launched kernels, captured step graphs); bos ends a continuation
    (inference/decoder.py:310-312). A `SlotBackend` of `serve`."""

    def __init__(self, model: Weights, batch: int, max_len: int, device, bos: int, prompt_store: int = 0,
                 narrow: int = 256):
        if narrow < 0 or narrow % 64:
            raise ValueError(f"narrow = {narrow}: a multiple of 64 slots (whole slot-mask words)")
        self.dec = d = Fp8Decoder(model, batch, max_len, device)
        self.narrow = narrow if narrow < batch else 0  # 0: one graph
        self.batch, self.max_len, self.bos, self.device = batch, max_len, bos, device
        self.store = PromptStore(prompt_store)
        hkv = model.cfg.kv_heads
        self.store_rows = torch.empty((len(d.caches), prompt_store, hkv, ROW_BYTES), dtype=torch.uint8,
                                      pin_memory=True) if prompt_store else None
        self.staging = torch.empty((max_len, hkv, ROW_BYTES), dtype=torch.uint8, device=device) if prompt_store \
            else None
        self.loads = self.alts_taken = 0
        d.lazy = bos  # every choice also reports its best row but BOS (the alternative)
        B, dev = batch, device
        self.tok = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.full((B,), -1, dtype=torch.int32, device=dev)
        self.next = torch.zeros(B, dtype=torch.int32, device=dev)
        d.temperature = torch.zeros(B, dtype=torch.float32, device=dev)
        d.top_p = torch.ones(B, dtype=torch.float32, device=dev)
        d.seeds = torch.zeros(B, dtype=torch.int64, device=dev)
        d.first = torch.zeros(B, dtype=torch.int32, device=dev)
        d.slots = torch.zeros((2, (B + 63) // 64), dtype=torch.int64, device=dev)
        d.allow = torch.zeros((B, (model.cfg.vocab + 31) // 32), dtype=torch.int32, device=dev)
        self.narrow_slots = torch.zeros((2, self.narrow // 64), dtype=torch.int64, device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.narrow_graph: torch.cuda.CUDAGraph | None = None
        self.narrow_steps = self.steps = 0
        self.stream = torch.cuda.Stream(dev)
        self.admitted: list[tuple[int, Request]] = []

    def generate(self, requests: Iterable[Request]) -> Iterator[tuple[int, list[int]]]:
        """Continuations of requests, consumed lazily; yields (request index, generated ids) in completion order."""
        if self.graph is None:
            self._capture()
        return serve(self, requests, self.bos)

    @property
    def stored(self) -> dict[tuple[int, ...], int]:
        return self.store.where

    def _capture(self) -> None:
        """The step graphs: the decode step over every slot (and over the first `narrow`), then each slot's next
        input is its choice."""
        s = self.stream
        s.wait_stream(torch.cuda.current_stream(self.device))

        def body(n: int) -> None:
            self.dec._step(self.tok[:n], self.pos[:n], self.next[:n], None if n == self.batch else self.narrow_slots)
            self.tok[:n].copy_(self.next[:n])

        with torch.cuda.stream(s):
            saved = self.pos.clone(), self.tok.clone()
            for n in (self.batch, self.narrow):  # warm every launch path (no slot is active yet)
                if n:
                    body(n)
            self.pos.copy_(saved[0])
            self.tok.copy_(saved[1])
            s.synchronize()
            self.graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(self.graph, stream=s):
                body(self.batch)
            if self.narrow:
                self.narrow_graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(self.narrow_graph, stream=s):
                    body(self.narrow)
        torch.cuda.current_stream(self.device).wait_stream(s)

    # ------------------------------------------------------------------------------------------ SlotBackend
    def admit(self, b: int, index: int, request: Request) -> None:
        prompt_positions(request, index, self.max_len)
        self.admitted.append((b, request))

    @torch.no_grad()
    def step(self, active, masks):
        d, dev = self.dec, self.device
        with torch.cuda.stream(self.stream):
            if self.admitted:
                self._start(self.admitted)
                self.admitted = []
            rows = masks()
            for b, allowed in rows.items():
                d.allow[b].copy_(torch.from_numpy(allow_rows(allowed[None])[0]).to(dev))
            words = slot_masks(active, [b in rows for b in range(self.batch)])
            high = max(b for b, a in enumerate(active) if a)
            self.steps += 1
            if high < self.narrow:  # dec_set_active's choice (decode.cu:1090-1093)
                self.narrow_slots.copy_(torch.from_numpy(words[:, :self.narrow // 64].copy()).to(dev))
                self.narrow_graph.replay()
                self.narrow_steps += 1
            else:
                d.slots.copy_(torch.from_numpy(words).to(dev))
                self.graph.replay()
            return self.next.cpu().numpy(), d.alt.cpu().numpy()

    def take_alt(self, b: int, token: int) -> None:
        with torch.cuda.stream(self.stream):
            self.tok[b] = token  # the next input: the alternative (dec_take_alt)
        self.alts_taken += 1

    def retire(self, slots: list[int]) -> None:
        with torch.cuda.stream(self.stream):
            self.pos.index_fill_(0, torch.tensor(slots, dtype=torch.int64, device=self.device), -1)

    # ------------------------------------------------------------------------------------------ prompts
    def _start(self, admitted: list[tuple[int, Request]]) -> None:
        """Load stored prompts, prefill the others but their last tokens in one pass (then store them), and set the
        admitted slots' decode state."""
        d, dev = self.dec, self.device
        fresh = []
        for b, r in admitted:
            at = self.store.find(r.input_ids)
            if at is None:
                fresh.append((b, r.input_ids))
            else:
                self._load(b, at, len(r.input_ids) - 1)
        if fresh:
            rows = torch.from_numpy(prompt_rows(fresh)).to(dev)
            d._prefill_rows(rows[0].contiguous(), rows[1].contiguous(), rows[2].contiguous())
            for b, ids in fresh:
                at = self.store.claim(ids, len(ids) - 1) if self.store_rows is not None else None
                if at is not None:
                    self._save(b, at, len(ids) - 1)
        for b, r in admitted:
            n = len(r.input_ids) - 1
            self.tok[b] = int(r.input_ids[-1])
            self.pos[b] = n
            d.first[b] = n
            d.temperature[b] = float(r.temperature)
            d.top_p[b] = float(r.top_p)
            d.seeds[b] = int(np.uint64(r.seed).view(np.int64))

    def _save(self, b: int, at: int, n: int) -> None:
        """Slot b's positions [0, n), every layer, to store positions [at, at + n) (through the staging rows)."""
        for l, cache in enumerate(self.dec.caches):
            rows = cache.export_rows(b, 0, n, out=self.staging[:n])
            self.store_rows[l, at:at + n].copy_(rows, non_blocking=True)

    def _load(self, b: int, at: int, n: int) -> None:
        for l, cache in enumerate(self.dec.caches):
            self.staging[:n].copy_(self.store_rows[l, at:at + n], non_blocking=True)
            cache.import_rows(self.staging[:n], b, 0)
        self.loads += 1
