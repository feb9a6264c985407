"""ikl_paged_decode_step: attention then append in one library call, with the
append carried by the split reduce kernel when it runs. The result must be
the attention output of ikl_paged_attention and the cache of a following
ikl_append_kv, bit for bit (append.py:19-66 / cache.py:156-189 for the
append; attention within tolerance of the oracle, attention.py:134-175)."""

import pytest
import torch

from tests.helpers import ATOL, assert_close_up_to_output_rounding, make_case, max_abs_err

pytestmark = pytest.mark.gpu


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


def _step_case(*, batch, heads, kv, head_dim, lengths, dtype, tokens=None, seed, slot_dtype=torch.int32,
               bad_slots=0):
    """A case with room for `tokens` new rows (default: one per request at
    its next position) and the rows to append."""
    case = make_case(batch=batch, num_heads=heads, num_kv_heads=kv, head_dim=head_dim, block_size=16,
                     lengths=[n + 16 for n in lengths], dtype=dtype, seed=seed)
    case.lengths = list(lengths)
    gen = torch.Generator(device="cuda").manual_seed(seed + 100)
    tdtype = getattr(torch, dtype)
    if tokens is None:
        slots = [t[n // 16] * 16 + n % 16 for t, n in zip(case.tables, lengths)]
    else:  # distinct slots in the pool's blocks that no table maps
        mapped = {blk for table in case.tables for blk in table}
        spare = [blk for blk in range(case.oracle_cache.num_blocks) if blk not in mapped]
        assert len(spare) * 16 >= tokens
        slots = [spare[i // 16] * 16 + i % 16 for i in range(tokens)]
    for i in range(bad_slots):  # outside the cache: skipped
        slots[i] = -1 if i % 2 == 0 else case.oracle_cache.num_blocks * 16 + i
    t = len(slots)
    key = torch.randn(t, kv, head_dim, generator=gen, device="cuda").to(tdtype)
    value = torch.randn(t, kv, head_dim, generator=gen, device="cuda").to(tdtype)
    return case, key, value, torch.tensor(slots, dtype=slot_dtype, device="cuda")


def _run_both(case, key, value, slots, **kw):
    from inferkernellab_amd import ops

    fused_cache, ref_cache = case.device_cache(), case.device_cache()
    q, tables, lens = case.device_query(), case.device_tables(), case.device_lengths()
    attn = ops.PreparedPagedAttention(q, fused_cache, tables, lens, **kw)
    step = ops.PreparedDecodeStep(attn, ops.PreparedAppend(key, value, fused_cache, slots))
    out = step().clone()
    ref = ops.paged_decode_attention_hip(q, ref_cache, tables, lens, **kw)
    ops.append_kv_hip(key, value, ref_cache, slots)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(ref))
    assert torch.equal(_bits(fused_cache.k), _bits(ref_cache.k))
    assert torch.equal(_bits(fused_cache.v), _bits(ref_cache.v))
    assert max_abs_err(out, case.expected()) <= ATOL[case.dtype]
    return step


@pytest.mark.parametrize(
    "shape",
    [
        # (batch, heads, kv, head_dim, lengths, dtype, kwargs, fused)
        (8, 32, 8, 128, [4096, 17, 8192, 5000, 1, 6000, 333, 7777], "bfloat16", {"partition_size": -2}, True),
        (4, 32, 8, 128, [2048, 1500, 700, 3000], "bfloat16", {"partition_size": 512}, True),
        (4, 32, 1, 128, [2000, 4000, 1024, 3000], "bfloat16", {}, True),
        (4, 16, 16, 128, [1024, 900, 700, 1200], "float16", {"partition_size": 256}, True),
        (3, 8, 2, 64, [700, 1300, 90], "float32", {"partition_size": 256}, True),
        (2, 8, 2, 64, [100, 40], "float16", {"partition_size": -1}, False),
    ],
)
def test_step_equals_attention_then_append(shape):
    batch, heads, kv, d, lengths, dtype, kw, fused = shape
    print(f"decode step B={batch} H={heads} Hkv={kv} D={d} {dtype} {kw}", flush=True)
    case, key, value, slots = _step_case(batch=batch, heads=heads, kv=kv, head_dim=d, lengths=lengths,
                                         dtype=dtype, seed=60 + batch)
    step = _run_both(case, key, value, slots, **kw)
    assert step.fused == fused
    assert step.kernel_names()[-1] == ("paged_decode_reduce_kernel" if fused else "append_kv_kernel")


def test_step_over_a_folded_plan_appends_with_its_own_launch():
    """fp32 GQA 32/8 hd64, B4 x <= 512: the attention runs each request's
    four 128-token partitions as one 4-wave workgroup (no split, no
    workspace); the step runs that kernel and then the append kernel. Its
    output equals the attention alone bit for bit, and the cache equals
    the separate append's."""
    from inferkernellab_amd import ops

    print("decode step over a folded VALU plan: B=4 H=32 Hkv=8 D=64 float32", flush=True)
    case, key, value, slots = _step_case(batch=4, heads=32, kv=8, head_dim=64, lengths=[512, 1, 300, 129],
                                         dtype="float32", seed=90)
    step_cache, ref_cache = case.device_cache(), case.device_cache()
    q, tables, lens = case.device_query(), case.device_tables(), case.device_lengths()
    attn = ops.PreparedPagedAttention(q, step_cache, tables, lens, max_context_len=512)
    assert (attn.launch["split"], attn.launch["num_warps"]) == ("none", 4)
    assert attn.workspace.numel() == 1  # the attention alone needs none
    step = ops.PreparedDecodeStep(attn, ops.PreparedAppend(key, value, step_cache, slots))
    assert not step.fused
    assert step.kernel_names() == ("paged_decode_scalar_kernel", "append_kv_kernel")
    out = step().clone()
    ref = ops.paged_decode_attention_hip(q, ref_cache, tables, lens, max_context_len=512)
    ops.append_kv_hip(key, value, ref_cache, slots)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out), _bits(ref))
    assert torch.equal(_bits(step_cache.k), _bits(ref_cache.k))
    assert torch.equal(_bits(step_cache.v), _bits(ref_cache.v))
    assert max_abs_err(out, case.expected()) <= ATOL["float32"]


def test_step_appends_more_rows_than_one_pass_covers():
    """One request x 8 heads: 8 reduce workgroups, 2 rows each per pass, 200
    rows to append (100 tokens x 2 heads); int64 slots, some outside the
    cache (skipped)."""
    print("decode step multi-pass append", flush=True)
    case, key, value, slots = _step_case(batch=1, heads=8, kv=2, head_dim=128, lengths=[3000], dtype="bfloat16",
                                         tokens=100, seed=71, slot_dtype=torch.int64, bad_slots=6)
    step = _run_both(case, key, value, slots, partition_size=512)
    assert step.fused


@pytest.mark.parametrize("partition,slot_dtype", [(128, torch.int32), (-2, torch.int64)])
def test_step_over_the_fp8_cache_fuses_the_quantising_append(partition, slot_dtype):
    """Over the FP8 cache the reduce kernel also carries the append, one
    wave per (token, head, K or V) row quantised as ikl_append_kv does: the
    cache codes and scales equal the separate append's and the oracle's
    quantiser (quantize_rows_e4m3) bit for bit, the attention equals the
    attention alone. 37 tokens x 4 heads = 296 rows over 2 x 8 reduce
    workgroups (several passes); one slot outside the cache is skipped."""
    from inferkernellab_amd import ops
    from inferkernellab_amd.cache import PagedKVCache, quantize_rows_e4m3

    print(f"decode step fp8 fused append partition={partition}", flush=True)

    def fresh():
        c = PagedKVCache(64, 16, 4, 128, dtype=torch.float8_e4m3fn, act_dtype=torch.bfloat16, device="cuda")
        c.k.view(torch.uint8).fill_(0x11)
        c.v.view(torch.uint8).fill_(0x22)
        c.k_scale.fill_(0.5)
        c.v_scale.fill_(0.25)
        return c

    cache, ref_cache = fresh(), fresh()
    gen = torch.Generator(device="cuda").manual_seed(7)
    q = torch.randn(2, 8, 128, device="cuda", generator=gen).to(torch.bfloat16)
    tables = torch.arange(64, dtype=torch.int32, device="cuda").view(2, 32)
    lens = torch.tensor([300, 200], dtype=torch.int32, device="cuda")
    key = (torch.randn(37, 4, 128, device="cuda", generator=gen) * 3).to(torch.bfloat16)
    value = torch.randn(37, 4, 128, device="cuda", generator=gen).to(torch.bfloat16)
    key[5].zero_()  # a zero row: scale 1
    slot_list = [400 + i for i in range(36)] + [64 * 16 + 3]  # the last one is outside the cache
    slots = torch.tensor(slot_list, dtype=slot_dtype, device="cuda")
    attn = ops.PreparedPagedAttention(q, cache, tables, lens, partition_size=partition)
    step = ops.PreparedDecodeStep(attn, ops.PreparedAppend(key, value, cache, slots))
    assert step.fused and step.kernel_names()[-1] == "paged_decode_reduce_kernel"
    step()
    ref = ops.paged_decode_attention_hip(q, ref_cache, tables, lens, partition_size=partition)
    ops.append_kv_hip(key, value, ref_cache, slots)
    torch.cuda.synchronize()
    assert torch.equal(step.out.view(torch.int16), ref.view(torch.int16))
    for a, b in ((cache.k, ref_cache.k), (cache.v, ref_cache.v)):
        assert torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    assert torch.equal(cache.k_scale, ref_cache.k_scale) and torch.equal(cache.v_scale, ref_cache.v_scale)
    # against the quantiser directly, row by row
    s = torch.tensor(slot_list[:36], device="cuda")
    blk, off = s // 16, s % 16
    for new, codes, scales in ((key[:36], cache.k, cache.k_scale), (value[:36], cache.v, cache.v_scale)):
        c, sc = quantize_rows_e4m3(new)
        assert torch.equal(codes[0][blk, off].view(torch.uint8), c.view(torch.uint8))
        assert torch.equal(scales[0][blk, :, off], sc)
    assert float(cache.k_scale[0][25, :, 5].min()) == 1.0  # slot 405: the zero row
    # nothing else of the cache changed
    untouched = torch.ones(64 * 16, dtype=torch.bool, device="cuda")
    untouched[s] = False
    assert (cache.k[0].reshape(64 * 16, 4, 128)[untouched].view(torch.uint8) == 0x11).all()


def test_step_function_and_graph_replays():
    """paged_decode_step_hip equals the prepared step; a captured step
    replays to the same output and cache."""
    from inferkernellab_amd import ops

    print("decode step graph", flush=True)
    case, key, value, slots = _step_case(batch=4, heads=32, kv=8, head_dim=128, lengths=[5000, 6000, 7000, 4500],
                                         dtype="bfloat16", seed=80)
    cache = case.device_cache()
    q, tables, lens = case.device_query(), case.device_tables(), case.device_lengths()
    out = ops.paged_decode_step_hip(q, cache, tables, lens, key, value, slots, partition_size=-2)
    torch.cuda.synchronize()
    step = ops.PreparedDecodeStep(ops.PreparedPagedAttention(q, cache, tables, lens, partition_size=-2),
                                  ops.PreparedAppend(key, value, cache, slots))
    assert step.fused
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    for _ in range(3):
        step.out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(step.out.view(torch.int16), out.view(torch.int16))
    blk, off = (slots // 16).long(), (slots % 16).long()
    assert torch.equal(cache.k[0][blk, off].view(torch.int16), key.view(torch.int16))
    assert torch.equal(cache.v[0][blk, off].view(torch.int16), value.view(torch.int16))


def test_step_on_random_shapes():
    """30 seeded random decode steps (dtype, heads, head_dim, batch, lengths,
    split choice): the step's output equals the oracle, and its cache equals
    a following ikl_append_kv bit for bit, whether the append rides on the
    reduce or runs on its own (folded attention plans included)."""
    import random

    from inferkernellab_amd import ops

    rng = random.Random(41)
    for i in range(30):
        kv = rng.choice([1, 4, 8, 32])
        heads = rng.choice([h for h in (8, 32) if h % kv == 0])
        d = rng.choice([64, 128])
        dtype = rng.choice(["float16", "bfloat16", "float32"])
        batch = rng.choice([1, 4, 16])
        maxlen = rng.choice([16, 300, 512, 2000])
        lengths = [rng.randint(1, maxlen) for _ in range(batch)]
        kw = rng.choice([{}, {}, {"partition_size": -1}, {"partition_size": 256}, {"max_context_len": maxlen + 16}])
        if dtype == "float32" and kw.get("partition_size") == -2:
            kw = {}
        print(f"random step {i}: B={batch} H={heads} Hkv={kv} D={d} {dtype} max={maxlen} {kw}", flush=True)
        case, key, value, slots = _step_case(batch=batch, heads=heads, kv=kv, head_dim=d, lengths=lengths,
                                             dtype=dtype, seed=300 + i)
        fused_cache, ref_cache = case.device_cache(), case.device_cache()
        q, tables, lens = case.device_query(), case.device_tables(), case.device_lengths()
        attn = ops.PreparedPagedAttention(q, fused_cache, tables, lens, **kw)
        step = ops.PreparedDecodeStep(attn, ops.PreparedAppend(key, value, fused_cache, slots))
        out = step().clone()
        ops.append_kv_hip(key, value, ref_cache, slots)
        torch.cuda.synchronize()
        assert torch.equal(_bits(fused_cache.k), _bits(ref_cache.k))
        assert torch.equal(_bits(fused_cache.v), _bits(ref_cache.v))
        assert_close_up_to_output_rounding(out, case.expected(), dtype)
