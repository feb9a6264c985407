"""Decode runners over the paged runtime: the callers of the HIP operators.

The runners own a paged cache, a token-budget scheduler and an
:class:`InferenceRuntime`, plug their prefill and decode steps into the
runtime hooks, and keep the device-side decode metadata (a block-table
buffer and a context-length buffer) the way the reference's runners do
(decode.py:315-493): the table buffer is allocated once at full width and
only newly appended table entries are copied in; context lengths are
refreshed per step. The KV of the token being decoded is in the cache
before attention runs (decode.py:481-487).

Backends are named like the reference's so configurations carry over:
attention ``hip_paged`` / ``hip_paged_grouped`` (``triton_paged`` /
``triton_paged_grouped`` name the same HIP functions) and append ``hip``
(``triton`` is the same) or ``torch`` (the cache's own ``index_put`` write,
the reference's bit-exact append path). There is no CPU attention backend:
the paged decode attention always runs the HIP kernels.
"""

from __future__ import annotations

import math
import time
from dataclasses import dataclass
from typing import Sequence

import torch
import torch.nn.functional as F

from . import ops
from .cache import PagedKVCache
from .runtime import InferenceRuntime
from .scheduler import InferenceRequest, TokenBudgetScheduler

ATTENTION_BACKENDS = {
    "hip_paged": ops.paged_decode_attention_hip,
    "hip_paged_grouped": ops.paged_decode_attention_hip_grouped,
    "triton_paged": ops.paged_decode_attention_triton,
    "triton_paged_grouped": ops.paged_decode_attention_triton_grouped,
}
APPEND_BACKENDS = ("hip", "triton", "torch")


def percentile(values: Sequence[float], q: float) -> float:
    """Linear-interpolation percentile (numpy's default method)."""
    if not values:
        return 0.0
    xs = sorted(values)
    pos = (len(xs) - 1) * q
    lo, hi = math.floor(pos), math.ceil(pos)
    return xs[lo] + (xs[hi] - xs[lo]) * (pos - lo)


class DecodeMetadata:
    """Device block-table and context-length buffers of a runner's batch.

    ``tables`` is ``[num_requests, width]`` int32, zero-filled once; a
    request's row grows by copying only entries it has not copied before.
    """

    def __init__(self, num_requests: int, width: int, device: torch.device):
        self.width = max(1, width)
        self.tables = torch.zeros((num_requests, self.width), dtype=torch.int32, device=device)
        self.lens = torch.zeros(num_requests, dtype=torch.int32, device=device)
        self._copied = [0] * num_requests
        self.device = device

    def sync_tables(self, requests: Sequence[InferenceRequest]) -> None:
        for r in requests:
            n = len(r.block_table)
            if n > self.width:
                raise RuntimeError("request block table exceeds preallocated metadata capacity")
            done = self._copied[r.request_id]
            if n > done:
                self.tables[r.request_id, done:n].copy_(
                    torch.tensor(r.block_table[done:n], dtype=torch.int32), non_blocking=False)
                self._copied[r.request_id] = n

    def for_batch(self, requests: Sequence[InferenceRequest], context_lengths: Sequence[int]):
        """(tables, lens) rows of `requests` with lens set to `context_lengths`."""
        if len(requests) != len(context_lengths):
            raise ValueError("requests and context_lengths must have the same length")
        self.sync_tables(requests)
        ids = [r.request_id for r in requests]
        lens = torch.tensor(list(context_lengths), dtype=torch.int32)
        if ids == list(range(len(ids))):
            tables = self.tables[: len(ids)]
            out = self.lens[: len(ids)]
            out.copy_(lens)
            return tables, out
        index = torch.tensor(ids, dtype=torch.long, device=self.device)
        return self.tables.index_select(0, index), lens.to(self.device)

    def slots(self, requests: Sequence[InferenceRequest], positions: Sequence[int], block_size: int):
        """int32 physical slots of one position per request, computed on the
        device from the table buffer (tables must be synced)."""
        ids = torch.tensor([r.request_id for r in requests], dtype=torch.long, device=self.device)
        pos = torch.tensor(list(positions), dtype=torch.long, device=self.device)
        blocks = self.tables[ids, pos // block_size].to(torch.long)
        return (blocks * block_size + pos % block_size).to(torch.int32)


def interleaved_tables(cache: PagedKVCache, requests: Sequence[InferenceRequest],
                       token_counts: Sequence[int]) -> list[int]:
    """Re-allocate the requests' initial tables one logical block per request
    per round, with one spacer block between rounds, so every table of more
    than one block is non-contiguous (as a long-running server's are).
    Returns the spacer blocks (owner -1) for the caller to free."""
    for r in requests:
        cache.release_request(r.block_table, request_id=r.request_id)
        r.block_table = []
    bs = cache.layout.block_size
    need = [-(-n // bs) for n in token_counts]
    spacers: list[int] = []
    rounds = max(need, default=0)
    for j in range(rounds):
        for r, n in zip(requests, need):
            if j < n:
                r.block_table += cache.allocator.allocate(1, owner=r.request_id)
        if j + 1 < rounds:
            spacers += cache.allocator.allocate(1, owner=-1)
    return spacers


# ------------------------------------------------------------------ synthetic
@dataclass(frozen=True)
class SyntheticDecoderConfig:
    """Configuration of the one-layer synthetic decoder (decode.py:32-73)."""

    vocab_size: int = 256
    num_heads: int = 32
    num_kv_heads: int = 8
    head_dim: int = 64
    block_size: int = 16
    dtype: torch.dtype = torch.float16
    device: torch.device | str = "cuda"
    seed: int = 0
    backend: str = "hip_paged"
    append_backend: str = "hip"
    max_num_seqs: int = 32
    max_num_batched_tokens: int = 2048
    num_blocks: int | None = None
    prefill_mode: str = "batched"

    def __post_init__(self) -> None:
        object.__setattr__(self, "device", torch.device(self.device))
        if self.vocab_size <= 1:
            raise ValueError("vocab_size must be greater than one")
        if min(self.num_heads, self.num_kv_heads, self.head_dim, self.block_size) <= 0:
            raise ValueError("model and cache dimensions must be positive")
        if self.num_heads % self.num_kv_heads != 0:
            raise ValueError("num_heads must be divisible by num_kv_heads")
        if self.backend not in ATTENTION_BACKENDS:
            raise ValueError(f"unsupported attention backend: {self.backend}")
        if self.append_backend not in APPEND_BACKENDS:
            raise ValueError(f"unsupported append backend: {self.append_backend}")
        if self.max_num_seqs <= 0 or self.max_num_batched_tokens <= 0:
            raise ValueError("scheduler limits must be positive")
        if self.prefill_mode not in ("batched", "token"):
            raise ValueError("prefill_mode must be batched or token")
        if self.num_blocks is not None and self.num_blocks <= 0:
            raise ValueError("num_blocks must be positive when provided")
        if self.device.type != "cuda":
            raise ValueError(f"{self.backend} requires a GPU (torch 'cuda') device")


@dataclass(frozen=True)
class DecodeRunResult:
    """Outcome and timing of a synthetic run (fields of decode.py:76-126)."""

    backend: str
    append_backend: str
    prompt_lengths: tuple[int, ...]
    max_new_tokens: int
    generated_tokens: tuple[tuple[int, ...], ...]
    logits: tuple[torch.Tensor, ...]
    prefill_wall_ms: float
    decode_step_wall_ms: tuple[float, ...]
    ttft_wall_ms: float
    tpot_wall_ms: float
    tokens_per_sec: float
    end_to_end_tokens_per_sec: float
    prefill_device_ms: float
    decode_step_device_ms: tuple[float, ...]
    ttft_device_ms: float
    tpot_device_ms: float
    device_tokens_per_sec: float
    end_to_end_device_tokens_per_sec: float
    peak_memory_allocated_bytes: int
    used_blocks_peak: int
    prefill_step_wall_ms: tuple[float, ...] = ()
    prefill_mode: str = "token"
    prefill_batch_count: int = 0
    prefill_tokens: int = 0
    prefill_padding_tokens: int = 0

    @property
    def decode_step_p50_ms(self) -> float:
        return percentile(self.decode_step_wall_ms, 0.50)

    @property
    def decode_step_p95_ms(self) -> float:
        return percentile(self.decode_step_wall_ms, 0.95)

    @property
    def decode_step_device_p50_ms(self) -> float:
        return percentile(self.decode_step_device_ms, 0.50)

    @property
    def decode_step_device_p95_ms(self) -> float:
        return percentile(self.decode_step_device_ms, 0.95)

    @property
    def prefill_p50_ms(self) -> float:
        return percentile(self.prefill_step_wall_ms, 0.50)

    @property
    def prefill_p95_ms(self) -> float:
        return percentile(self.prefill_step_wall_ms, 0.95)


class SyntheticDecodeRunner:
    """A seeded one-layer decoder (embedding -> q/k/v -> paged attention ->
    out projection -> lm_head -> argmax) run through the paged runtime with
    the HIP append and attention operators (decode.py:151-592)."""

    def __init__(self, config: SyntheticDecoderConfig, prompts: Sequence[Sequence[int]],
                 max_new_tokens: int = 16):
        if not prompts:
            raise ValueError("at least one prompt is required")
        if max_new_tokens <= 0:
            raise ValueError("max_new_tokens must be positive")
        if len(prompts) > config.max_num_seqs:
            raise ValueError("the scheduler max_num_seqs is smaller than the batch")
        self.config = config
        self.device = config.device
        self.max_new_tokens = max_new_tokens
        self.prompts = tuple(tuple(int(t) for t in p) for p in prompts)
        if any(len(p) == 0 for p in self.prompts):
            raise ValueError("prompts must be non-empty")
        if any(not 0 <= t < config.vocab_size for p in self.prompts for t in p):
            raise ValueError("prompt token is outside the configured vocabulary")
        self.prompt_lengths = tuple(len(p) for p in self.prompts)
        self._attend = ATTENTION_BACKENDS[config.backend]
        self._hip_append = config.append_backend in ("hip", "triton")
        if self._hip_append:
            ops._require_backend()

        bs = config.block_size
        final_blocks = sum(-(-(n + max_new_tokens) // bs) for n in self.prompt_lengths)
        first_blocks = [-(-n // bs) for n in self.prompt_lengths]
        minimum = final_blocks + max(0, max(first_blocks) - 1)  # + spacers
        num_blocks = config.num_blocks if config.num_blocks is not None else minimum
        if num_blocks < minimum:
            raise ValueError(f"num_blocks is insufficient: requested={num_blocks}, minimum={minimum}")

        self.weights = self._init_weights()
        self.cache = PagedKVCache(num_blocks, bs, config.num_kv_heads, config.head_dim,
                                  dtype=config.dtype, device=self.device)
        scheduler = TokenBudgetScheduler(max_num_seqs=config.max_num_seqs,
                                         max_num_batched_tokens=config.max_num_batched_tokens)
        batched = config.prefill_mode == "batched"
        self.runtime = InferenceRuntime(
            self.cache, scheduler,
            prefill_fn=None if batched else self._prefill,
            prefill_batch_fn=self._prefill_batch if batched else None,
            decode_fn=self._decode,
        )
        self.requests = [self.runtime.submit(i, len(p), max_new_tokens) for i, p in enumerate(self.prompts)]
        self._spacers = interleaved_tables(self.cache, self.requests, self.prompt_lengths)
        width = max(-(-(n + max_new_tokens) // bs) for n in self.prompt_lengths)
        self.metadata = DecodeMetadata(len(self.requests), width, self.device)
        self._last_token: dict[int, torch.Tensor] = {}
        self._tokens: dict[int, list[torch.Tensor]] = {r.request_id: [] for r in self.requests}
        self._step_logits: list[torch.Tensor] = []
        self._has_run = False

    # ---------------------------------------------------------------- model
    def _init_weights(self) -> dict[str, torch.Tensor]:
        c = self.config
        gen = torch.Generator().manual_seed(c.seed)
        hidden, kv = c.num_heads * c.head_dim, c.num_kv_heads * c.head_dim

        def draw(rows: int, cols: int, std: float) -> torch.Tensor:
            w = torch.randn(rows, cols, generator=gen) * std
            return w.to(device=self.device, dtype=c.dtype)

        std = hidden ** -0.5
        return {
            "embedding": draw(c.vocab_size, hidden, 0.02),
            "q": draw(hidden, hidden, std),
            "k": draw(kv, hidden, std),
            "v": draw(kv, hidden, std),
            "out": draw(hidden, hidden, std),
            "lm_head": draw(c.vocab_size, hidden, std),
        }

    def _hidden(self, ids: torch.Tensor) -> torch.Tensor:
        return F.embedding(ids.to(device=self.device, dtype=torch.long), self.weights["embedding"])

    def _kv(self, hidden: torch.Tensor):
        c = self.config
        k = F.linear(hidden, self.weights["k"]).view(-1, c.num_kv_heads, c.head_dim)
        v = F.linear(hidden, self.weights["v"]).view(-1, c.num_kv_heads, c.head_dim)
        return k, v

    # --------------------------------------------------------------- append
    def _append_slots(self, slots: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> None:
        if self._hip_append:
            ops.append_kv_hip(key.contiguous(), value.contiguous(), self.cache, slots)
        else:
            self.cache.write_slots(0, slots, key, value, validate_slots=False)

    def _prefill_ranges(self, requests, starts, ends) -> None:
        spans = [e - s for s, e in zip(starts, ends)]
        if len(requests) != len(starts) or len(requests) != len(ends):
            raise ValueError("requests and prefill ranges must have matching lengths")
        if any(n <= 0 for n in spans):
            raise ValueError("prefill ranges must be non-empty")
        ids = [t for r, s, e in zip(requests, starts, ends) for t in self.prompts[r.request_id][s:e]]
        key, value = self._kv(self._hidden(torch.tensor(ids)))
        slots = torch.cat([self.cache.slot_mapping(r.block_table, s, n)
                           for r, s, n in zip(requests, starts, spans)]).to(torch.int32)
        self._append_slots(slots, key, value)

    def _prefill(self, request: InferenceRequest, start: int, end: int) -> None:
        self._prefill_ranges((request,), (start,), (end,))

    def _prefill_batch(self, requests, starts, ends) -> None:
        self._prefill_ranges(requests, starts, ends)

    # --------------------------------------------------------------- decode
    def _decode(self, requests: tuple[InferenceRequest, ...]) -> None:
        c = self.config
        current = [self._last_token[r.request_id] if r.generated_tokens
                   else torch.tensor(self.prompts[r.request_id][-1], device=self.device)
                   for r in requests]
        hidden = self._hidden(torch.stack(current))
        query = F.linear(hidden, self.weights["q"]).view(-1, c.num_heads, c.head_dim)
        positions = [r.prompt_tokens + r.generated_tokens for r in requests]
        tables, lens = self.metadata.for_batch(requests, positions)
        attended = self._attention(query, tables, lens, requests, positions)
        logits = F.linear(F.linear(attended.reshape(len(requests), -1), self.weights["out"]),
                          self.weights["lm_head"])
        next_tokens = logits.argmax(dim=-1)
        key, value = self._kv(self._hidden(next_tokens))
        self.metadata.sync_tables(requests)
        slots = self.metadata.slots(requests, positions, c.block_size)
        self._append_slots(slots, key, value)
        self._step_logits.append(logits.detach().float().cpu())
        for row, r in enumerate(requests):
            self._last_token[r.request_id] = next_tokens[row]
            self._tokens[r.request_id].append(next_tokens[row])

    def _attention(self, query, tables, lens, requests, context_lengths) -> torch.Tensor:
        return self._attend(query.contiguous(), self.cache, tables, lens, validate_inputs=True)

    # ------------------------------------------------------------------ run
    def _timed_step(self):
        start_ev, end_ev = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        start_ev.record()
        batch = self.runtime.step()
        end_ev.record()
        end_ev.synchronize()
        return batch, (time.perf_counter() - t0) * 1e3, float(start_ev.elapsed_time(end_ev))

    def run(self) -> DecodeRunResult:
        if self._has_run:
            raise RuntimeError("a SyntheticDecodeRunner instance can only be run once")
        self._has_run = True
        torch.cuda.reset_peak_memory_stats(self.device)
        prefill_steps, prefill_dev, decode_wall, decode_dev = [], 0.0, [], []
        peak_blocks = self.cache.allocator.num_used_blocks
        try:
            with torch.no_grad():  # no inference tensors: callers may capture graphs later
                while self.runtime.scheduler.waiting or self.runtime.scheduler.running:
                    batch, wall_ms, dev_ms = self._timed_step()
                    peak_blocks = max(peak_blocks, self.cache.allocator.num_used_blocks)
                    if batch.phase == "prefill":
                        prefill_steps.append(wall_ms)
                        prefill_dev += dev_ms
                    elif batch.phase == "decode":
                        decode_wall.append(wall_ms)
                        decode_dev.append(dev_ms)
                    else:
                        raise RuntimeError("scheduler became idle before all requests finished")
        finally:
            if self._spacers:
                self.cache.allocator.free(self._spacers, owner=-1)
                self._spacers = []
        generated = tuple(tuple(int(t) for t in torch.stack(self._tokens[r.request_id]).tolist())
                          for r in self.requests)
        total = len(self.requests) * self.max_new_tokens
        if sum(len(g) for g in generated) != total:
            raise RuntimeError("decoder finished with an unexpected number of generated tokens")
        if not decode_wall:
            raise RuntimeError("decoder produced no decode steps")
        prefill_wall = sum(prefill_steps)
        return DecodeRunResult(
            backend=self.config.backend,
            append_backend=self.config.append_backend,
            prompt_lengths=self.prompt_lengths,
            max_new_tokens=self.max_new_tokens,
            generated_tokens=generated,
            logits=tuple(self._step_logits),
            prefill_wall_ms=prefill_wall,
            decode_step_wall_ms=tuple(decode_wall),
            ttft_wall_ms=prefill_wall + decode_wall[0],
            tpot_wall_ms=sum(decode_wall) / len(decode_wall),
            tokens_per_sec=total / (sum(decode_wall) / 1e3),
            end_to_end_tokens_per_sec=total / ((prefill_wall + sum(decode_wall)) / 1e3),
            prefill_device_ms=prefill_dev,
            decode_step_device_ms=tuple(decode_dev),
            ttft_device_ms=prefill_dev + decode_dev[0],
            tpot_device_ms=sum(decode_dev) / len(decode_dev),
            device_tokens_per_sec=total / (sum(decode_dev) / 1e3),
            end_to_end_device_tokens_per_sec=total / ((prefill_dev + sum(decode_dev)) / 1e3),
            peak_memory_allocated_bytes=int(torch.cuda.max_memory_allocated(self.device)),
            used_blocks_peak=peak_blocks,
            prefill_step_wall_ms=tuple(prefill_steps),
            prefill_mode=self.config.prefill_mode,
            prefill_batch_count=len(prefill_steps),
            prefill_tokens=sum(self.prompt_lengths),
            prefill_padding_tokens=0,
        )
