"""Continuous batching over the decoder's slots: the host protocol of the reference's NativeDecoder.generate
(inference/decoder.py:28-40,194-324) on this package's kernels.

Requests queue for `batch` slots. A free slot takes the next request: its prompt but the last token is prefilled
into the slot's cache rows (all newly admitted prompts in one prefill), the slot's token, position, first generated
position and sampling parameters are set, and it joins the next decode step. Each step is one replay of a captured
hipGraph over every slot: idle slots carry position -1, so the fused decode step does no work for them and the
token choice (nc_choose_tokens' slot mask) leaves them untouched. As the reference's narrow graphs
(decode.cu:32-33,995-1005,1090-1093), a second graph over the first `narrow` slots runs the steps in which no
higher slot is active: its GEMMs, its lm_head and its choice cover those rows only. After a step the host reads
the choices and finishes a slot on BOS (dropped; unless the request's accept_bos rejects it, when the step's
alternative, the best token but BOS, is taken instead, as the reference's lazy BOS), at max_new_tokens, or when the
request's stopping criteria hold for its tokens, then refills it. A request's mask callable, if any, gives the next
position's allowed tokens (the reference's constraints, decode.cu:1077-1094's dec_masks rows); a masked slot
chooses among them, -1 when none is allowed.

The prompt store (decode.cu:1053-1075; inference/decoder.py:196-232): pinned host memory for `prompt_store`
positions. A prefilled prompt's cache pages (every layer's fp8 codes and scales of the slot's first ceil(n / 16)
pages) are copied there once, in order, never evicted; a later request with the same input_ids loads them into its
slot instead of prefilling. Positions of a loaded last page past the prompt hold whatever the stored slot held:
they are appended before any step attends them.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable, Iterable, Iterator, Sequence

import numpy as np
import torch

from nanochat_amd.decoder import Fp8Decoder, Weights
from nanochat_amd.kv_cache import PAGE
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


@dataclass
class _Slot:
    index: int
    request: Request
    out: list


class Server:
    """`batch` slots over one Fp8Decoder; bos ends a continuation (inference/decoder.py:310-312)."""

    def __init__(self, model: Weights, batch: int, max_len: int, device, bos: int, prompt_store: int = 0,
                 narrow: int = 256):
        if narrow < 0 or narrow % 64:
            raise ValueError(f"narrow = {narrow}: a multiple of 64 slots (whole slot-mask words)")
        self.dec = Fp8Decoder(model, batch, max_len, device)
        self.narrow = narrow if narrow < batch else 0  # 0: one graph
        self.batch, self.max_len, self.bos, self.device = batch, max_len, bos, device
        caches = self.dec.caches
        self.store_pages = prompt_store // PAGE
        self.store = torch.empty((len(caches), self.store_pages) + tuple(caches[0].pages.shape[1:]), dtype=torch.uint8,
                                 pin_memory=True) if self.store_pages else None
        self.stored: dict[tuple[int, ...], int] = {}  # prompt -> its first store page
        self.used = 0
        self.loads = 0
        self.dec.lazy = bos  # every choice also reports its best row but BOS (the alternative)
        self.alts_taken = 0
        vocab = model.cfg.vocab
        B = batch
        dev = device
        self.tok = torch.zeros(B, dtype=torch.int32, device=dev)
        self.pos = torch.full((B,), -1, dtype=torch.int32, device=dev)
        self.next = torch.zeros(B, dtype=torch.int32, device=dev)
        d = self.dec
        d.temperature = torch.zeros(B, dtype=torch.float32, device=dev)
        d.top_p = torch.ones(B, dtype=torch.float32, device=dev)
        d.seeds = torch.zeros(B, dtype=torch.int64, device=dev)
        d.first = torch.zeros(B, dtype=torch.int32, device=dev)
        d.slots = torch.zeros((2, (B + 63) // 64), dtype=torch.int64, device=dev)
        d.allow = torch.zeros((B, (vocab + 31) // 32), dtype=torch.int32, device=dev)
        self.narrow_slots = torch.zeros((2, self.narrow // 64), dtype=torch.int64, device=dev)
        self.graph: torch.cuda.CUDAGraph | None = None
        self.narrow_graph: torch.cuda.CUDAGraph | None = None
        self.narrow_steps = self.steps = 0
        self.stream = torch.cuda.Stream(dev)

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

    @torch.no_grad()
    def generate(self, requests: Iterable[Request]) -> Iterator[tuple[int, list[int]]]:
        """Continuations of requests, consumed lazily; yields (request index, generated ids) in completion order."""
        B, dev = self.batch, self.device
        d = self.dec
        if self.graph is None:
            self._capture()
        queue = enumerate(requests)
        slots: list[_Slot | None] = [None] * B
        admitted: list[int] = []

        def fill(b: int) -> None:
            for i, r in queue:
                n = len(r.input_ids) - 1
                if n < 1 or r.max_new_tokens < 1 or n + r.max_new_tokens > self.max_len:
                    raise ValueError(f"request {i}: {n + 1} prompt tokens and {r.max_new_tokens} new tokens do not "
                                     f"fit max_len {self.max_len}")
                slots[b] = _Slot(i, r, [])
                admitted.append(b)
                return
            slots[b] = None

        for b in range(B):
            fill(b)
        while any(s is not None for s in slots):
            with torch.cuda.stream(self.stream):
                if admitted:
                    self._admit(slots, admitted)
                    admitted.clear()
                masked = self._masks(slots)
                words = slot_masks([s is not None for s in slots], masked)
                high = max(b for b, s in enumerate(slots) if s is not None)
                self.steps += 1
                if high < self.narrow:  # dec_set_active's choice (decode.cu:1090-1093)
                    self.narrow_slots.copy_(torch.from_numpy(words[:, :self.narrow // 64].copy()).to(dev))
                    self.narrow_graph.replay()
                    self.narrow_steps += 1
                else:
                    d.slots.copy_(torch.from_numpy(words).to(dev))
                    self.graph.replay()
                chosen = self.next.cpu().numpy()
                alts = d.alt.cpu().numpy()
            finished = []
            for b, s in enumerate(slots):
                if s is None:
                    continue
                token = int(chosen[b])
                if token == self.bos and s.request.accept_bos and not s.request.accept_bos(s.out):
                    token = int(alts[b])  # the host rejects the lazy BOS (inference/decoder.py:233-248)
                    if token < 0:
                        raise ValueError(f"request {s.index}: nothing but BOS allowed at position {len(s.out)}")
                    with torch.cuda.stream(self.stream):
                        self.tok[b] = token  # the next input: the alternative (dec_take_alt)
                    self.alts_taken += 1
                if token == self.bos:
                    finished.append(b)
                    continue
                if token < 0:
                    raise ValueError(f"request {s.index}: its mask allows no token at position {len(s.out)}")
                s.out.append(token)
                r = s.request
                if len(s.out) == r.max_new_tokens or (r.stopping_criteria and r.stopping_criteria(s.out)):
                    finished.append(b)
            if finished:
                with torch.cuda.stream(self.stream):
                    idle = torch.tensor(finished, dtype=torch.int64, device=dev)
                    self.pos.index_fill_(0, idle, -1)
                for b in finished:
                    done = slots[b]
                    fill(b)
                    yield done.index, done.out

    def _pages(self, l: int, b: int, n: int) -> torch.Tensor:
        """Slot b's first ceil(n / 16) pages of layer l (a contiguous cache: the slot's blocks are consecutive)."""
        mb = self.dec.caches[l].max_blocks
        return self.dec.caches[l].pages[b * mb:b * mb + -(-n // PAGE)]

    def _admit(self, slots, admitted) -> None:
        """Load stored prompts, prefill the others but their last tokens in one pass (then store them), and set the
        admitted slots' decode state."""
        d, dev = self.dec, self.device
        fresh = []
        for b in admitted:
            ids = tuple(int(t) for t in slots[b].request.input_ids)
            at = self.stored.get(ids)
            if at is None:
                fresh.append(b)
                continue
            n = len(ids) - 1
            for l in range(len(d.caches)):
                self._pages(l, b, n).copy_(self.store[l, at:at + -(-n // PAGE)], non_blocking=True)
            self.loads += 1
        if fresh:
            rows = [np.array([s.request.input_ids[:-1], range(len(s.request.input_ids) - 1),
                              [b] * (len(s.request.input_ids) - 1)], dtype=np.int32)
                    for b in fresh for s in (slots[b],)]
            rows = torch.from_numpy(np.concatenate(rows, axis=1)).to(dev)
            d._prefill_rows(rows[0].contiguous(), rows[1].contiguous(), rows[2].contiguous())
            for b in fresh:
                self._save(b, tuple(int(t) for t in slots[b].request.input_ids))
        for b in admitted:
            r = slots[b].request
            n = len(r.input_ids) - 1
            self.tok[b] = int(r.input_ids[-1])
            self.pos[b] = n
            d.first[b] = n
            d.temperature[b] = float(r.temperature)
            d.top_p[b] = float(r.top_p)
            d.seeds[b] = int(np.uint64(r.seed).view(np.int64))

    def _save(self, b: int, ids: tuple[int, ...]) -> None:
        """Keep slot b's prompt pages in the store's next free pages, unless stored already or out of room."""
        n = len(ids) - 1
        pages = -(-n // PAGE)
        if self.store is None or ids in self.stored or self.used + pages > self.store_pages:
            return
        for l in range(len(self.dec.caches)):
            self.store[l, self.used:self.used + pages].copy_(self._pages(l, b, n), non_blocking=True)
        self.stored[ids] = self.used
        self.used += pages

    def _masks(self, slots) -> list[bool]:
        """Each masked slot's allowed-token row for its next position; returns which slots are masked."""
        d = self.dec
        masked = [False] * self.batch
        for b, s in enumerate(slots):
            if s is None or s.request.mask is None:
                continue
            allowed = s.request.mask(s.out)
            if allowed is None:
                continue
            masked[b] = True
            d.allow[b].copy_(torch.from_numpy(allow_rows(np.asarray(allowed, bool)[None])[0]).to(self.device))
        return masked
