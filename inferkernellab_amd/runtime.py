"""Model-independent runtime: request lifecycle, KV block reservation and
the ``prefill_fn`` / ``prefill_batch_fn`` / ``decode_fn`` hooks.

The hooks are the drop-in surface of the reference's runtime
(runtime.py:10-12): runners plug the HIP append and attention operators into
them. What callers observe, and the reference's tests pin
(tests/test_runtime.py:8-81), is kept:

* ``submit`` reserves blocks for ``max(1, prompt_tokens)`` tokens;
* a prefill step grows every scheduled table to its cached tokens, then
  calls ``prefill_batch_fn(requests, starts, ends)`` once with the requests
  whose range is non-empty (or ``prefill_fn`` per request);
* a decode step first reserves room for the token each request writes, then
  calls ``decode_fn(requests)`` — before the scheduler counts that token —
  and finally returns the blocks of finished requests to the allocator.

A step is dispatched on its phase to one handler; block reservation is one
helper that tops a table up to the blocks a token count needs.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Callable

from .cache import PagedKVCache
from .scheduler import InferenceRequest, ScheduleBatch, TokenBudgetScheduler

PrefillFn = Callable[[InferenceRequest, int, int], None]
PrefillBatchFn = Callable[[tuple[InferenceRequest, ...], tuple[int, ...], tuple[int, ...]], None]
DecodeFn = Callable[[tuple[InferenceRequest, ...]], None]


@dataclass(frozen=True)
class RuntimeStats:
    waiting: int
    running: int
    finished: int
    free_blocks: int
    used_blocks: int


@dataclass(frozen=True)
class _Hooks:
    prefill: PrefillFn | None
    prefill_batch: PrefillBatchFn | None
    decode: DecodeFn | None

    def __post_init__(self):
        if self.prefill is not None and self.prefill_batch is not None:
            raise ValueError("prefill_fn and prefill_batch_fn are mutually exclusive")


class InferenceRuntime:
    """Drives a :class:`TokenBudgetScheduler` over a :class:`PagedKVCache`,
    calling the model hooks at each step (no logits of its own)."""

    def __init__(
        self,
        cache: PagedKVCache,
        scheduler: TokenBudgetScheduler,
        *,
        prefill_fn: PrefillFn | None = None,
        prefill_batch_fn: PrefillBatchFn | None = None,
        decode_fn: DecodeFn | None = None,
    ):
        self._hooks = _Hooks(prefill_fn, prefill_batch_fn, decode_fn)
        self.cache = cache
        self.scheduler = scheduler
        self._by_id: dict[int, InferenceRequest] = {}
        self._handlers = {"prefill": self._prefill_step, "decode": self._decode_step}

    @property
    def prefill_fn(self) -> PrefillFn | None:
        return self._hooks.prefill

    @property
    def prefill_batch_fn(self) -> PrefillBatchFn | None:
        return self._hooks.prefill_batch

    @property
    def decode_fn(self) -> DecodeFn | None:
        return self._hooks.decode

    def submit(self, request_id: int, prompt_tokens: int, max_new_tokens: int) -> InferenceRequest:
        if request_id in self._by_id:
            raise ValueError(f"duplicate request_id: {request_id}")
        request = InferenceRequest(request_id, prompt_tokens, max_new_tokens)
        request.block_table = self.cache.allocate_request(request_id, max(1, prompt_tokens))
        self._by_id[request_id] = request
        self.scheduler.add(request)
        return request

    def _reserve(self, request: InferenceRequest, tokens: int) -> None:
        """Tops the request's table up to the blocks `tokens` positions need."""
        short = -(-tokens // self.cache.layout.block_size) - len(request.block_table)
        if short > 0:
            request.block_table += self.cache.allocator.allocate(short, owner=request.request_id)

    def step(self) -> ScheduleBatch:
        # prompt progress of every queued request before the scheduler grants
        # tokens: each prefill range starts there
        progress = {request.request_id: request.cached_tokens for request in self.scheduler.waiting}
        batch = self.scheduler.schedule()
        handler = self._handlers.get(batch.phase)
        if handler is not None:
            handler(batch, progress)
        return batch

    def _prefill_step(self, batch: ScheduleBatch, progress: dict[int, int]) -> None:
        ranges = []
        for request in batch.requests:
            self._reserve(request, max(1, request.cached_tokens))
            lo = progress.get(request.request_id, request.cached_tokens)
            if lo < request.cached_tokens:
                ranges.append((request, lo, request.cached_tokens))
        hooks = self._hooks
        if ranges and hooks.prefill_batch is not None:
            requests, starts, ends = zip(*ranges)
            hooks.prefill_batch(tuple(requests), tuple(starts), tuple(ends))
        elif hooks.prefill is not None:
            for request, lo, hi in ranges:
                hooks.prefill(request, lo, hi)

    def _decode_step(self, batch: ScheduleBatch, progress: dict[int, int]) -> None:
        del progress  # decode ranges are one token at prompt + generated
        for request in batch.requests:
            self._reserve(request, request.prompt_tokens + request.generated_tokens + 1)
        if self._hooks.decode is not None:
            self._hooks.decode(batch.requests)
        self.scheduler.mark_decode_step(batch.requests)
        for request in (r for r in batch.requests if r.finished):
            self.cache.release_request(request.block_table, request_id=request.request_id)
            request.block_table = []

    def stats(self) -> RuntimeStats:
        allocator = self.cache.allocator
        s = self.scheduler
        return RuntimeStats(len(s.waiting), len(s.running), len(s.finished), allocator.num_free_blocks,
                            allocator.num_used_blocks)
