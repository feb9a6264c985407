"""Model-independent runtime: request lifecycle, KV block reservation and
the ``prefill_fn`` / ``prefill_batch_fn`` / ``decode_fn`` hooks.

Same contract as the reference's runtime.py:10-113, which is part of the
drop-in surface: runners plug the HIP append and attention operators into
these hooks.

* ``submit`` reserves blocks for ``max(1, prompt_tokens)`` tokens.
* A prefill step calls ``prefill_batch_fn(requests, starts, ends)`` once
  with every request that received prompt tokens (or ``prefill_fn`` per
  request), after growing each table to ``cached_tokens``.
* A decode step reserves room for one more token per request, calls
  ``decode_fn(requests)`` BEFORE the scheduler counts the generated token,
  then frees the blocks of finished requests.
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


class InferenceRuntime:
    def __init__(
        self,
        cache: PagedKVCache,
        scheduler: TokenBudgetScheduler,
        *,
        prefill_fn: PrefillFn | None = None,
        prefill_batch_fn: PrefillBatchFn | None = None,
        decode_fn: DecodeFn | None = None,
    ):
        if prefill_fn is not None and prefill_batch_fn is not None:
            raise ValueError("prefill_fn and prefill_batch_fn are mutually exclusive")
        self.cache = cache
        self.scheduler = scheduler
        self.prefill_fn = prefill_fn
        self.prefill_batch_fn = prefill_batch_fn
        self.decode_fn = decode_fn
        self._requests: dict[int, InferenceRequest] = {}

    def submit(self, request_id: int, prompt_tokens: int, max_new_tokens: int) -> InferenceRequest:
        if request_id in self._requests:
            raise ValueError(f"duplicate request_id: {request_id}")
        request = InferenceRequest(request_id, prompt_tokens, max_new_tokens)
        request.block_table = self.cache.allocate_request(request_id, max(1, prompt_tokens))
        self._requests[request_id] = request
        self.scheduler.add(request)
        return request

    def _ensure_capacity(self, request: InferenceRequest, num_tokens: int) -> None:
        needed = -(-num_tokens // self.cache.layout.block_size) - len(request.block_table)
        if needed > 0:
            request.block_table.extend(
                self.cache.allocator.allocate(needed, owner=request.request_id)
            )

    def step(self) -> ScheduleBatch:
        before = {id(r): r.cached_tokens for r in self._requests.values()}
        batch = self.scheduler.schedule()
        if batch.phase == "prefill":
            chosen, starts, ends = [], [], []
            for request in batch.requests:
                self._ensure_capacity(request, max(1, request.cached_tokens))
                start, end = before[id(request)], request.cached_tokens
                if start < end:
                    chosen.append(request)
                    starts.append(start)
                    ends.append(end)
            if chosen and self.prefill_batch_fn is not None:
                self.prefill_batch_fn(tuple(chosen), tuple(starts), tuple(ends))
            elif self.prefill_fn is not None:
                for request, start, end in zip(chosen, starts, ends):
                    self.prefill_fn(request, start, end)
        elif batch.phase == "decode":
            for request in batch.requests:
                # room for the token this step writes
                self._ensure_capacity(request, request.prompt_tokens + request.generated_tokens + 1)
            if self.decode_fn is not None:
                self.decode_fn(batch.requests)
            self.scheduler.mark_decode_step(batch.requests)
            for request in batch.requests:
                if request.finished:
                    self.cache.release_request(request.block_table, request_id=request.request_id)
                    request.block_table = []
        return batch

    def stats(self) -> RuntimeStats:
        return RuntimeStats(
            waiting=len(self.scheduler.waiting),
            running=len(self.scheduler.running),
            finished=len(self.scheduler.finished),
            free_blocks=self.cache.allocator.num_free_blocks,
            used_blocks=self.cache.allocator.num_used_blocks,
        )
