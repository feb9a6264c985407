"""FCFS token-budget scheduler behind the runtime hooks.

Observable contract (the reference's scheduler.py:7-95 and the sequences
its tests pin, tests/test_scheduler.py:4-29, tests/test_runtime.py:8-81):

* a step prefills while any request waits: requests are taken in arrival
  order under ``max_num_batched_tokens`` and ``max_num_seqs``; only the first
  request of a step may be cut short (a long prompt is chunked over several
  steps and keeps its place at the head of the queue), a later one is taken
  only if its whole remaining prompt fits;
* a request with nothing left to prefill moves to the running set without
  using budget;
* when nothing is prefilled, up to ``max_num_seqs`` running requests decode
  one token each; ``mark_decode_step`` counts it and retires finished ones.

The step is computed as a plan first — a list of token grants over a prefix
of the queue, nothing mutated — and then committed in queue order, so the
budget rules live in one pure function (:func:`plan_prefill`).
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field
from typing import Iterable, Sequence


@dataclass
class InferenceRequest:
    """A request's lifecycle state; the fields are the reference's
    (scheduler.py:7-25), read by runners and hooks."""

    request_id: int
    prompt_tokens: int
    max_new_tokens: int
    generated_tokens: int = 0
    cached_tokens: int = 0
    status: str = "waiting"
    block_table: list[int] = field(default_factory=list)

    @property
    def prompt_remaining(self) -> int:
        return max(0, self.prompt_tokens - self.cached_tokens)

    @property
    def finished(self) -> bool:
        return self.generated_tokens >= self.max_new_tokens


@dataclass(frozen=True)
class ScheduleBatch:
    requests: tuple[InferenceRequest, ...]
    phase: str  # "prefill" | "decode" | "idle"
    scheduled_tokens: int


@dataclass(frozen=True)
class PrefillPlan:
    """What one prefill step does to the head of the queue.

    ``examined`` requests form a prefix of the queue; ``grants[i]`` is the
    number of prompt tokens request ``examined[i]`` receives (0 for one that
    only moves to the running set). ``chunked`` is true when the last grant
    leaves part of that prompt for a later step."""

    examined: tuple[InferenceRequest, ...]
    grants: tuple[int, ...]
    chunked: bool

    @property
    def tokens(self) -> int:
        return sum(self.grants)


def plan_prefill(queue: Iterable[InferenceRequest], max_seqs: int, max_tokens: int) -> PrefillPlan:
    """Token grants for one step over the queue head (pure: reads only)."""
    examined: list[InferenceRequest] = []
    grants: list[int] = []
    taken = 0  # requests that received tokens
    left = max_tokens
    chunked = False
    for request in queue:
        if taken >= max_seqs or left <= 0:
            break
        need = request.prompt_remaining
        if need and taken and need > left:
            break  # only the step's first prompt may be cut short
        give = min(need, left)
        examined.append(request)
        grants.append(give)
        if give:
            taken += 1
            left -= give
        if give < need:
            chunked = True  # the budget is spent; this prompt resumes next step
            break
    return PrefillPlan(tuple(examined), tuple(grants), chunked)


class TokenBudgetScheduler:
    """FCFS scheduler with a per-step token budget (prefill first)."""

    def __init__(self, max_num_seqs: int = 32, max_num_batched_tokens: int = 2048):
        if max_num_seqs <= 0 or max_num_batched_tokens <= 0:
            raise ValueError("scheduler limits must be positive")
        self.max_num_seqs = max_num_seqs
        self.max_num_batched_tokens = max_num_batched_tokens
        self.waiting: deque[InferenceRequest] = deque()
        self.running: list[InferenceRequest] = []
        self.finished: list[InferenceRequest] = []

    def add(self, request: InferenceRequest) -> None:
        if request.status != "waiting":
            raise ValueError("only waiting requests can be added")
        self.waiting.append(request)

    def schedule(self) -> ScheduleBatch:
        plan = plan_prefill(self.waiting, self.max_num_seqs, self.max_num_batched_tokens)
        prefilled = self._commit(plan)
        if prefilled:
            return ScheduleBatch(prefilled, "prefill", plan.tokens)
        decoding = tuple(self.running[: self.max_num_seqs])
        if decoding:
            return ScheduleBatch(decoding, "decode", len(decoding))
        return ScheduleBatch((), "idle", 0)

    def _commit(self, plan: PrefillPlan) -> tuple[InferenceRequest, ...]:
        """Applies a plan: grants become cached tokens, completed prompts join
        the running set in queue order, a chunked prompt stays at the head."""
        settled = len(plan.examined) - (1 if plan.chunked else 0)
        for _ in range(settled):
            self.waiting.popleft()
        prefilled = []
        for request, give in zip(plan.examined, plan.grants):
            request.cached_tokens += give
            if give:
                prefilled.append(request)
            if request.prompt_remaining:
                request.status = "waiting"
            else:
                request.status = "running"
                self.running.append(request)
        return tuple(prefilled)

    def mark_decode_step(self, requests: Sequence[InferenceRequest]) -> None:
        """Counts one generated token for each running request of the step and
        retires the ones that reached ``max_new_tokens``, in running order."""
        stepped = {id(request) for request in requests}
        still_running = []
        for request in self.running:
            if id(request) in stepped:
                request.generated_tokens += 1
                if request.finished:
                    request.status = "finished"
                    self.finished.append(request)
                    continue
            still_running.append(request)
        self.running[:] = still_running
