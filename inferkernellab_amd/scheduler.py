"""FCFS token-budget scheduler driving the runtime hooks.

Same accounting as the reference's scheduler.py:7-95: waiting requests are
prefilled in FCFS order under ``max_num_batched_tokens`` (a long prompt is
chunked across steps and keeps its place at the head of the queue), and
once nothing is left to prefill the running requests decode one token per
step.
"""

from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field


@dataclass
class InferenceRequest:
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


class TokenBudgetScheduler:
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

    def _admit(self, request: InferenceRequest) -> None:
        request.status = "running"
        self.running.append(request)

    def schedule(self) -> ScheduleBatch:
        batch: list[InferenceRequest] = []
        budget_used = 0
        while self.waiting and len(batch) < self.max_num_seqs:
            head = self.waiting[0]
            budget_left = self.max_num_batched_tokens - budget_used
            if budget_left <= 0:
                break
            need = head.prompt_remaining
            if need == 0:
                self.waiting.popleft()
                self._admit(head)
                continue
            if batch and need > budget_left:
                break
            self.waiting.popleft()
            take = min(need, budget_left)
            head.cached_tokens += take
            budget_used += take
            batch.append(head)
            if head.prompt_remaining == 0:
                self._admit(head)
            else:
                head.status = "waiting"
                self.waiting.appendleft(head)
        if batch:
            return ScheduleBatch(tuple(batch), "prefill", budget_used)
        decode = tuple(self.running[: self.max_num_seqs])
        if not decode:
            return ScheduleBatch((), "idle", 0)
        return ScheduleBatch(decode, "decode", len(decode))

    def mark_decode_step(self, requests) -> None:
        stepped = {id(r) for r in requests}
        for request in list(self.running):
            if id(request) not in stepped:
                continue
            request.generated_tokens += 1
            if request.finished:
                request.status = "finished"
                self.running.remove(request)
                self.finished.append(request)
