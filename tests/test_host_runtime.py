"""Host-side rows of the path on the CPU: the paged cache's layout,
addressing and torch scatter/gather (cache.py:8-200), the block allocator
(cache.py:17-64), the token-budget scheduler (scheduler.py:7-95) and the
runtime hooks (runtime.py:65-104), checked against the known answers of the
reference's own tests (tests/golden/known_answers.json) and against the
oracle's restatement on random inputs."""

import numpy as np
import pytest
import torch

from inferkernellab_amd.cache import BlockAllocator, PagedKVCache
from inferkernellab_amd.runtime import InferenceRuntime
from inferkernellab_amd.scheduler import InferenceRequest, TokenBudgetScheduler
from tests.helpers import known_answers


def _cache(spec, **kw):
    c = spec["cache"]
    return PagedKVCache(c["num_blocks"], c["block_size"], c["num_kv_heads"], c["head_dim"],
                        dtype=torch.float32, **kw)


# ------------------------------------------------------------------ cache
def test_slot_mapping_known_answer():
    for spec in known_answers()["slot_mapping"]:
        slots = _cache(spec).slot_mapping(spec["block_table"], spec["start"], spec["length"])
        assert slots.dtype == torch.int64
        assert slots.tolist() == spec["expected"]


def test_slot_mapping_rejections():
    for spec in known_answers()["slot_mapping_rejects"]:
        with pytest.raises(ValueError, match=spec["match"]):
            _cache(spec).slot_mapping(spec["block_table"], spec["start"], spec["length"])


def test_slot_mapping_matches_oracle_on_random_tables():
    from oracle import paged_oracle as po

    gen = np.random.default_rng(5)
    for bs in (1, 4, 16):
        cache = PagedKVCache(64, bs, 1, 2, dtype=torch.float32)
        oc = po.OracleCache(64, bs, 1, 2, dtype="float32")
        table = [int(x) for x in gen.permutation(64)[:10]]
        start = int(gen.integers(0, bs * 5))
        length = int(gen.integers(0, bs * 10 - start + 1))
        assert cache.slot_mapping(table, start, length).tolist() == list(oc.slot_mapping(table, start, length))
        assert cache.slot_mapping(torch.tensor(table), start, length).tolist() == \
            list(oc.slot_mapping(table, start, length))


def test_write_and_read_preserve_logical_order():
    spec = known_answers()["write_read_order"]
    cache = _cache(spec)
    key = torch.arange(12, dtype=torch.float32).view(2, 2, 3)
    value = key + 100
    cache.write(0, spec["block_table"], spec["start"], key, value)
    read_key, read_value = cache.read(0, spec["block_table"], spec["read_length"])
    assert torch.equal(read_key[2:], key)
    assert torch.equal(read_value[2:], value)


def test_write_slots_flattened_ranges():
    spec = known_answers()["write_slots_flattened"]
    cache = _cache(spec)
    table = spec["block_table"]
    slots = torch.cat([cache.slot_mapping(table, s, n) for s, n in spec["ranges"]])
    assert slots.tolist() == spec["expected_slots"]
    key = torch.arange(24, dtype=torch.float32).view(4, 2, 3)
    value = key + 100
    cache.write_slots(0, slots, key, value)
    read_key, read_value = cache.read(0, table, spec["read_length"])
    rows = spec["expected_rows_equal_key"]
    assert torch.equal(read_key[rows], key)
    assert torch.equal(read_value[rows], value)


def test_write_slots_is_index_put_bit_for_bit():
    """The torch append path equals torch index_put on the [L,NB,bs,Hkv,D] view."""
    gen = torch.Generator().manual_seed(6)
    cache = PagedKVCache(16, 4, 2, 8, num_layers=2, dtype=torch.bfloat16)
    cache.k.zero_()
    cache.v.zero_()
    slots = torch.randperm(64, generator=gen)[:20]
    key = torch.randn(20, 2, 8, generator=gen).to(torch.bfloat16)
    value = torch.randn(20, 2, 8, generator=gen).to(torch.bfloat16)
    expected_k = cache.k.clone()
    expected_k[1, slots // 4, slots % 4] = key
    cache.write_slots(1, slots, key, value)
    assert torch.equal(cache.k.view(torch.int16), expected_k.view(torch.int16))
    with pytest.raises(ValueError, match="invalid physical cache position"):
        cache.write_slots(0, torch.tensor([64]), key[:1], value[:1])
    with pytest.raises(IndexError, match="layer"):
        cache.write_slots(2, slots, key, value)


def test_layers_are_independent():
    cache = PagedKVCache(4, 4, 1, 2, num_layers=2, dtype=torch.float32)
    key0, key1 = torch.ones(2, 1, 2), torch.full((2, 1, 2), 3.0)
    cache.write(0, [0], 0, key0, key0)
    cache.write(1, [0], 0, key1, key1)
    assert torch.equal(cache.read(0, [0], 2)[0], key0)
    assert torch.equal(cache.read(1, [0], 2)[0], key1)


def test_cache_layout_and_storage():
    cache = PagedKVCache(20, 16, 8, 128, num_layers=3, dtype=torch.bfloat16)
    assert tuple(cache.k.shape) == (3, 20, 16, 8, 128) and cache.v.shape == cache.k.shape
    assert cache.k.is_contiguous() and cache.dtype == torch.bfloat16
    assert cache.numel_bytes == 2 * 3 * 20 * 16 * 8 * 128 * 2
    with pytest.raises(ValueError, match="positive"):
        PagedKVCache(0, 16, 8, 128)


# -------------------------------------------------------------- allocator
def test_allocator_known_answers():
    spec = known_answers()["allocator"]
    a = spec["allocate_request"]
    cache = PagedKVCache(a["num_blocks"], a["block_size"], 1, 2, dtype=torch.float32)
    table = cache.allocate_request(a["request_id"], a["num_tokens"])
    assert cache.allocator.num_free_blocks == a["free_after"]
    cache.release_request(table)
    assert cache.allocator.num_free_blocks == a["free_after_release"]
    asc = spec["ascending_ids"]
    assert BlockAllocator(asc["num_blocks"]).allocate(asc["allocate"]) == asc["expected"]


def test_allocator_rejects_invalid_free_atomically():
    allocator = BlockAllocator(4)
    blocks = allocator.allocate(2, owner=7)
    with pytest.raises(ValueError, match="not allocated"):
        allocator.free([blocks[0], 3])
    with pytest.raises(ValueError, match="invalid block id"):
        allocator.free([9])
    assert (allocator.num_used_blocks, allocator.num_free_blocks) == (2, 2)
    with pytest.raises(ValueError, match="duplicates"):
        allocator.free([blocks[0], blocks[0]])
    with pytest.raises(ValueError, match="not owned"):
        allocator.free(blocks, owner=8)
    assert allocator.num_used_blocks == 2
    allocator.free(blocks, owner=7)
    assert (allocator.num_used_blocks, allocator.num_free_blocks) == (0, 4)
    with pytest.raises(RuntimeError, match="out of KV blocks"):
        allocator.allocate(5)


# -------------------------------------------------------------- scheduler
def test_scheduler_chunks_prefill_then_decodes():
    spec = known_answers()["scheduler_chunks"]
    scheduler = TokenBudgetScheduler(max_num_seqs=spec["max_num_seqs"],
                                     max_num_batched_tokens=spec["max_num_batched_tokens"])
    request = InferenceRequest(*spec["request"])
    scheduler.add(request)
    for phase, scheduled, cached in spec["steps"]:
        batch = scheduler.schedule()
        assert batch.phase == phase
        if scheduled is not None:
            assert batch.scheduled_tokens == scheduled
        assert request.cached_tokens == cached
    scheduler.mark_decode_step(batch.requests)
    assert request.generated_tokens == spec["generated_after_mark"]


def test_scheduler_marks_finished_requests():
    scheduler = TokenBudgetScheduler()
    request = InferenceRequest(1, prompt_tokens=1, max_new_tokens=1)
    scheduler.add(request)
    scheduler.schedule()
    batch = scheduler.schedule()
    scheduler.mark_decode_step(batch.requests)
    assert request.status == "finished" and scheduler.finished == [request]
    assert scheduler.schedule().phase == "idle"


def test_scheduler_fcfs_keeps_a_chunked_prompt_at_the_head():
    scheduler = TokenBudgetScheduler(max_num_seqs=4, max_num_batched_tokens=6)
    a, b = InferenceRequest(1, 10, 1), InferenceRequest(2, 3, 1)
    scheduler.add(a)
    scheduler.add(b)
    first = scheduler.schedule()
    assert [r.request_id for r in first.requests] == [1] and a.cached_tokens == 6
    second = scheduler.schedule()  # a's remaining 4 first, then b does not fit (3 > 2)
    assert [r.request_id for r in second.requests] == [1] and a.cached_tokens == 10
    third = scheduler.schedule()
    assert [r.request_id for r in third.requests] == [2] and third.scheduled_tokens == 3
    assert scheduler.schedule().phase == "decode"


# ---------------------------------------------------------------- runtime
def test_runtime_grows_and_releases_kv_blocks():
    spec = known_answers()["runtime_blocks"]
    runtime = InferenceRuntime(_cache(spec),
                               TokenBudgetScheduler(max_num_batched_tokens=spec["max_num_batched_tokens"]))
    r = spec["request"]
    request = runtime.submit(r["request_id"], prompt_tokens=r["prompt_tokens"],
                             max_new_tokens=r["max_new_tokens"])
    assert runtime.stats().used_blocks == spec["used_blocks_after_submit"]
    phases = [runtime.step().phase for _ in spec["phases"]]
    assert phases == spec["phases"]
    assert request.status == "finished"
    assert runtime.stats().used_blocks == spec["used_blocks_at_end"]


def test_runtime_hook_events_known_answer():
    spec = known_answers()["runtime_events"]
    events = []

    def prefill(request, start, end):
        events.append(["prefill", request.request_id, start, end, request.cached_tokens])

    def decode(requests):
        events.append(["decode", [r.generated_tokens for r in requests]])

    runtime = InferenceRuntime(_cache(spec),
                               TokenBudgetScheduler(max_num_batched_tokens=spec["max_num_batched_tokens"]),
                               prefill_fn=prefill, decode_fn=decode)
    r = spec["request"]
    runtime.submit(r["request_id"], prompt_tokens=r["prompt_tokens"], max_new_tokens=r["max_new_tokens"])
    assert [runtime.step().phase for _ in spec["phases"]] == spec["phases"]
    assert events == spec["events"]


def test_runtime_batch_prefill_one_event_per_batch():
    spec = known_answers()["runtime_batch_prefill"]
    events = []

    def prefill_batch(requests, starts, ends):
        events.append([[r.request_id for r in requests], list(starts), list(ends)])

    runtime = InferenceRuntime(_cache(spec),
                               TokenBudgetScheduler(max_num_seqs=spec["max_num_seqs"],
                                                    max_num_batched_tokens=spec["max_num_batched_tokens"]),
                               prefill_batch_fn=prefill_batch)
    for rid, prompt, new in spec["requests"]:
        runtime.submit(rid, prompt_tokens=prompt, max_new_tokens=new)
    assert [runtime.step().phase for _ in spec["phases"]] == spec["phases"]
    assert events == spec["events"]


def test_runtime_decode_reserves_the_written_slot_before_the_hook():
    """decode_fn sees a block table with room for position prompt+generated."""
    seen = []
    cache = PagedKVCache(8, 4, 1, 2, dtype=torch.float32)

    def decode(requests):
        for r in requests:
            pos = r.prompt_tokens + r.generated_tokens
            seen.append((pos, len(r.block_table) * 4 > pos))

    runtime = InferenceRuntime(cache, TokenBudgetScheduler(), decode_fn=decode)
    runtime.submit(1, prompt_tokens=4, max_new_tokens=3)
    while runtime.step().phase != "idle":
        pass
    assert seen == [(4, True), (5, True), (6, True)]
    assert runtime.stats().used_blocks == 0


def test_runtime_rejects_two_prefill_hooks_and_duplicate_ids():
    cache = PagedKVCache(4, 4, 1, 2, dtype=torch.float32)
    with pytest.raises(ValueError, match="mutually exclusive"):
        InferenceRuntime(cache, TokenBudgetScheduler(), prefill_fn=lambda r, s, e: None,
                         prefill_batch_fn=lambda rs, ss, es: None)
    runtime = InferenceRuntime(cache, TokenBudgetScheduler())
    runtime.submit(1, 2, 1)
    with pytest.raises(ValueError, match="duplicate"):
        runtime.submit(1, 2, 1)


def test_scheduler_admits_empty_prompts_without_budget_and_caps_sequences():
    """A request with nothing to prefill joins the running set in queue order
    without using budget; at most max_num_seqs requests receive tokens per
    step, and a later prompt that does not fit whole ends the step."""
    scheduler = TokenBudgetScheduler(max_num_seqs=2, max_num_batched_tokens=8)
    empty = InferenceRequest(0, 0, 1)
    a, b, c = InferenceRequest(1, 3, 1), InferenceRequest(2, 3, 1), InferenceRequest(3, 1, 1)
    for r in (empty, a, b, c):
        scheduler.add(r)
    first = scheduler.schedule()
    assert first.phase == "prefill" and [r.request_id for r in first.requests] == [1, 2]
    assert first.scheduled_tokens == 6 and [r.request_id for r in scheduler.running] == [0, 1, 2]
    assert list(scheduler.waiting) == [c] and c.cached_tokens == 0
    second = scheduler.schedule()
    assert [r.request_id for r in second.requests] == [3] and second.scheduled_tokens == 1
    decode = scheduler.schedule()
    assert decode.phase == "decode" and [r.request_id for r in decode.requests] == [0, 1]
    scheduler.mark_decode_step(decode.requests)
    assert [r.request_id for r in scheduler.finished] == [0, 1]
    assert [r.request_id for r in scheduler.running] == [2, 3]


def test_scheduler_second_prompt_must_fit_whole():
    scheduler = TokenBudgetScheduler(max_num_seqs=4, max_num_batched_tokens=5)
    a, b = InferenceRequest(1, 3, 1), InferenceRequest(2, 4, 1)
    scheduler.add(a)
    scheduler.add(b)
    first = scheduler.schedule()
    assert [r.request_id for r in first.requests] == [1] and b.cached_tokens == 0
    second = scheduler.schedule()  # b alone is first now: chunked at the budget
    assert [r.request_id for r in second.requests] == [2] and b.cached_tokens == 4
    assert b.status == "running"
