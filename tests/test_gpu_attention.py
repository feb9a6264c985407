"""Paged decode attention through the C ABI vs the fp32 oracle
(paged_reference, attention.py:134-175). Tolerance: max-abs 2e-3 fp16,
1e-2 bf16, 1e-4 fp32 against the fp32 result."""

import numpy as np
import pytest
import torch

from tests.helpers import ATOL, known_answers, make_case, max_abs_err

pytestmark = pytest.mark.gpu


def _check(case, fn, *, label, scale=None, layer=0, **kw):
    from inferkernellab_amd import ops

    print(f"attention case {label} dtype={case.dtype} H={case.num_heads} "
          f"Hkv={case.oracle_cache.num_kv_heads} D={case.oracle_cache.head_dim} "
          f"bs={case.oracle_cache.block_size} lens={case.lengths[:8]} kw={kw}", flush=True)
    cache = case.device_cache()
    out = getattr(ops, fn)(case.device_query(), cache, case.device_tables(), case.device_lengths(),
                           scale=scale, layer=layer, **kw)
    torch.cuda.synchronize()
    expected = case.expected(scale=scale, layer=layer)
    err = max_abs_err(out, expected)
    assert out.dtype == cache.dtype and out.shape == tuple(case.query.shape)
    assert err <= ATOL[case.dtype], f"{label}: max abs err {err}"
    return out


@pytest.mark.parametrize("num_kv_heads", [4, 2, 1])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_reference_shape_matches_oracle(num_kv_heads, dtype):
    """The shape of tests/test_attention.py:119-137 (tables [[13,2,9],[5,14,1]], lens 19/23)."""
    spec = known_answers()["attention_shapes"]["triton_vs_reference"]
    case = make_case(batch=2, num_heads=4, num_kv_heads=num_kv_heads, head_dim=16, block_size=8,
                     lengths=spec["lengths"], dtype=dtype, seed=1, num_blocks=16)
    _check(case, "paged_decode_attention_hip", label="ref-shape")


@pytest.mark.parametrize("num_kv_heads", [8, 4, 1])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_grouped_reference_shape(num_kv_heads, dtype):
    """tests/test_attention.py:140-173: 32 heads, layer 1 of 2, query_group_size 8."""
    case = make_case(batch=2, num_heads=32, num_kv_heads=num_kv_heads, head_dim=16, block_size=8,
                     lengths=[19, 23], dtype=dtype, seed=7, num_blocks=32, num_layers=2, layer=1)
    _check(case, "paged_decode_attention_hip_grouped", label="grouped-ref", layer=1, query_group_size=8)


@pytest.mark.parametrize("query_group_size", [1, 2, 4, 8])
def test_grouped_query_group_sizes(query_group_size):
    """The grouped wrapper (whose matrix-core path shares each tile among all
    6 heads of a KV head), then the C ABI with units of exactly
    min(query_group_size, 6) heads on the matrix cores."""
    from inferkernellab_amd import ops

    case = make_case(batch=3, num_heads=12, num_kv_heads=2, head_dim=64, block_size=16,
                     lengths=[100, 7, 333], dtype="bfloat16", seed=20)
    _check(case, "paged_decode_attention_hip_grouped", label="qgs", query_group_size=query_group_size)
    attn = ops.PreparedPagedAttention(case.device_query(), case.device_cache(), case.device_tables(),
                                      case.device_lengths(), query_group_size=query_group_size)
    out = attn()
    torch.cuda.synchronize()
    assert attn.path == "mfma_grouped"
    assert max_abs_err(out, case.expected()) <= ATOL["bfloat16"]


@pytest.mark.parametrize("head_dim", [16, 32, 64, 96, 128])
@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_head_dims(head_dim, dtype):
    case = make_case(batch=3, num_heads=8, num_kv_heads=2, head_dim=head_dim, block_size=16,
                     lengths=[1, 77, 301], dtype=dtype, seed=head_dim)
    _check(case, "paged_decode_attention_hip", label="head-dim")


@pytest.mark.parametrize("block_size", [1, 4, 8, 16, 32, 5])
def test_block_sizes(block_size):
    case = make_case(batch=2, num_heads=8, num_kv_heads=8, head_dim=128, block_size=block_size,
                     lengths=[250, 1029], dtype="bfloat16", seed=block_size)
    _check(case, "paged_decode_attention_hip", label="block-size")


@pytest.mark.parametrize("partition_size", [-1, 64, 128, 512])
def test_split_partitions_match(partition_size):
    case = make_case(batch=4, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                     lengths=[1, 511, 512, 2049], dtype="bfloat16", seed=30)
    _check(case, "paged_decode_attention_hip", label="split", partition_size=partition_size)


def test_mqa_group_32_bf16():
    case = make_case(batch=4, num_heads=32, num_kv_heads=1, head_dim=128, block_size=16,
                     lengths=[1024, 4096, 1500, 3333], dtype="bfloat16", seed=31, kv_scale=0.5)
    _check(case, "paged_decode_attention_hip", label="mqa")


def test_mha_fp16_with_split():
    # 64 MiB of K/V: above the size the library sends to the MFMA family, so
    # this runs the per-head kernel's split (8 partitions: rotated)
    case = make_case(batch=8, num_heads=32, num_kv_heads=32, head_dim=128, block_size=16,
                     lengths=[512] * 8, dtype="float16", seed=32)
    _check(case, "paged_decode_attention_hip", label="mha", partition_size=64)


def test_custom_scale_and_int64_metadata():
    from inferkernellab_amd import ops

    case = make_case(batch=2, num_heads=8, num_kv_heads=2, head_dim=64, block_size=16,
                     lengths=[40, 90], dtype="float16", seed=33)
    cache = case.device_cache()
    out = ops.paged_decode_attention_hip(case.device_query(), cache, case.device_tables(dtype=torch.int64),
                                         case.device_lengths(dtype=torch.int64), scale=0.05)
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected(scale=0.05)) <= ATOL["float16"]


def test_list_metadata_is_accepted():
    from inferkernellab_amd import ops

    case = make_case(batch=2, num_heads=4, num_kv_heads=2, head_dim=32, block_size=4,
                     lengths=[5, 7], dtype="float32", seed=3)
    cache = case.device_cache()
    width = max(len(t) for t in case.tables)
    tables = [t + [0] * (width - len(t)) for t in case.tables]
    out = ops.paged_decode_attention_hip(case.device_query(), cache, tables, case.lengths)
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected()) <= ATOL["float32"]


def test_nan_poisoned_unread_slots_do_not_leak():
    """Like tests/test_hf_benchmark.py:116-117: unread slots full of NaN."""
    case = make_case(batch=3, num_heads=16, num_kv_heads=4, head_dim=128, block_size=16,
                     lengths=[3, 17, 45], dtype="bfloat16", seed=34, poison=np.nan)
    assert (case.oracle_cache.k == 0x7FC0).any()  # bf16 NaN bits in the unread tails
    out = _check(case, "paged_decode_attention_hip", label="nan-poison")
    assert torch.isfinite(out).all()


def test_invalid_block_ids_are_masked_without_validation():
    """validate_inputs=False: ids outside the cache are masked (triton_ops.py:138)."""
    from inferkernellab_amd import ops
    from oracle import paged_oracle as po

    case = make_case(batch=1, num_heads=4, num_kv_heads=1, head_dim=64, block_size=16,
                     lengths=[48], dtype="float32", seed=35)
    cache = case.device_cache()
    table = list(case.tables[0])
    table[1] = 10_000  # the middle block is invalid -> its 16 tokens are masked
    out = ops.paged_decode_attention_hip(case.device_query(), cache,
                                         torch.tensor([table], dtype=torch.int32, device="cuda"),
                                         case.device_lengths(), validate_inputs=False)
    torch.cuda.synchronize()
    oc = case.oracle_cache
    k_all, v_all = oc.read(0, case.tables[0], 48)
    keep = np.r_[0:16, 32:48]
    ref = po.dense_decode_attention(case.query_f32, k_all[keep], v_all[keep])
    assert max_abs_err(out, ref) <= ATOL["float32"]


def test_validation_messages_match_reference():
    """tests/test_attention.py:176-193."""
    from inferkernellab_amd import PagedKVCache, ops

    cache = PagedKVCache(8, 8, 2, 16, dtype=torch.float16, device="cuda")
    query = torch.randn(1, 4, 16, device="cuda", dtype=torch.float16)
    with pytest.raises(ValueError, match="positive"):
        ops.paged_decode_attention_hip(query, cache, torch.tensor([[0]], dtype=torch.int32, device="cuda"),
                                       torch.tensor([0], dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError, match="physical block"):
        ops.paged_decode_attention_hip(query, cache, torch.tensor([[8]], dtype=torch.int32, device="cuda"),
                                       torch.tensor([1], dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError, match="capacity"):
        ops.paged_decode_attention_hip(query, cache, torch.tensor([[0]], dtype=torch.int32, device="cuda"),
                                       torch.tensor([9], dtype=torch.int32, device="cuda"))
    with pytest.raises(ValueError, match="query_group_size"):
        ops.paged_decode_attention_hip_grouped(query, cache, [[0]], [1], query_group_size=3)
    with pytest.raises(IndexError, match="layer"):
        ops.paged_decode_attention_hip(query, cache, [[0]], [1], layer=1)


def test_repeat_runs_are_bit_identical():
    from inferkernellab_amd import ops

    case = make_case(batch=4, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                     lengths=[700, 1500, 64, 3000], dtype="bfloat16", seed=36)
    cache = case.device_cache()
    args = (case.device_query(), cache, case.device_tables(), case.device_lengths())
    a = ops.paged_decode_attention_hip(*args)
    b = ops.paged_decode_attention_hip(*args)
    torch.cuda.synchronize()
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


# ---------------------------------------------------------------- balanced split
# partition_size=-2 runs the MFMA family's balanced split (None picks it for
# batches above 32768 tiles): the batch's tiles are cut into one equal run
# per workgroup (for units of up to 16 heads, groups of 2, 4 or 8 units of a
# request as the waves of one workgroup walking the same request tiles, or
# one-wave runs when the units per request are odd; 4 waves for 32-head
# units, which share each piece of the run and merge it in LDS), and the
# pieces are merged per unit by the reduce.

@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_balanced_split_more_than_64_requests(dtype):
    """70 requests: the in-kernel request scan walks two 64-request chunks."""
    gen = np.random.default_rng(40)
    lengths = [int(x) for x in gen.integers(1, 700, size=70)]
    lengths[0], lengths[63], lengths[64], lengths[69] = 1, 16, 17, 1000
    case = make_case(batch=70, num_heads=16, num_kv_heads=4, head_dim=128, block_size=16,
                     lengths=lengths, dtype=dtype, seed=41)
    _check(case, "paged_decode_attention_hip", label="sk-70", partition_size=-2)


@pytest.mark.parametrize("batch", [15, 16, 17, 31, 33, 48, 63, 65])
def test_balanced_split_request_scan_boundaries(batch):
    """Batches around the in-kernel scan's 16-lane rows and its 64-request
    chunk (one scan for up to 64 requests, the chunked walk beyond). Two
    requests are emptied on the device (validate_inputs=False), so some
    requests own no tiles: their rows are NaN, the others match the oracle."""
    from inferkernellab_amd import ops

    gen = np.random.default_rng(400 + batch)
    lengths = [int(x) for x in gen.integers(1, 600, size=batch)]
    case = make_case(batch=batch, num_heads=8, num_kv_heads=2, head_dim=64, block_size=16,
                     lengths=lengths, dtype="bfloat16", seed=401 + batch)
    empty = [batch // 2, batch - 1]
    print(f"scan boundary case batch={batch} empty={empty} lens={lengths[:8]}", flush=True)
    lens = case.device_lengths()
    for b in empty:
        lens[b] = 0
    out = ops.paged_decode_attention_hip(case.device_query(), case.device_cache(), case.device_tables(), lens,
                                         validate_inputs=False, partition_size=-2)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    expected = case.expected()
    full = [b for b in range(batch) if b not in empty]
    assert np.isnan(got[empty]).all(), "an empty context gives NaN rows (softmax over nothing)"
    assert np.abs(got[full] - expected[full]).max() <= ATOL["bfloat16"]


def test_balanced_split_one_unit_across_many_waves():
    """One MQA request of 20000 tokens: 1250 tiles, one unit split over ~1250 waves."""
    case = make_case(batch=1, num_heads=8, num_kv_heads=1, head_dim=128, block_size=32,
                     lengths=[20000], dtype="bfloat16", seed=42)
    _check(case, "paged_decode_attention_hip", label="sk-long", partition_size=-2)


@pytest.mark.parametrize("heads,kv,dim,dtype", [(32, 1, 128, "float16"), (32, 1, 128, "bfloat16"),
                                                (48, 2, 64, "bfloat16"), (40, 2, 96, "float16")])
def test_balanced_split_32_head_units(heads, kv, dim, dtype):
    """Units of 17-32 heads (MQA 32/1, and 24- and 20-head units) run 4-wave
    workgroups; ragged lengths (one token, one tile, a tile and one token,
    long) give pieces shorter than a workgroup's waves and pieces spanning
    several runs."""
    from inferkernellab_amd import ops

    gen = np.random.default_rng(44 + heads)
    lengths = [int(x) for x in gen.integers(1, 3000, size=9)]
    lengths[:4] = [1, 16, 17, 4096]
    case = make_case(batch=len(lengths), num_heads=heads, num_kv_heads=kv, head_dim=dim, block_size=16,
                     lengths=lengths, dtype=dtype, seed=45, kv_scale=0.5)
    _check(case, "paged_decode_attention_hip", label="sk-32head", partition_size=-2)
    cfg = ops.paged_decode_grouped_dot_autotune_config()
    assert cfg["num_warps"] == 4


@pytest.mark.parametrize("batch,lo,hi", [(1, 20000, 20000), (300, 1, 50)])
def test_balanced_split_32_head_units_extremes(batch, lo, hi):
    """4-wave runs of 32-head units: one MQA request of 20000 tokens split
    over every run, and 300 short requests (the in-kernel request scan walks
    five 64-request chunks; many runs hold several whole requests)."""
    lengths = [int(x) for x in np.random.default_rng(46).integers(lo, hi + 1, size=batch)]
    case = make_case(batch=batch, num_heads=32, num_kv_heads=1, head_dim=128, block_size=16,
                     lengths=lengths, dtype="bfloat16", seed=47, kv_scale=0.5)
    _check(case, "paged_decode_attention_hip", label="sk-32head-extreme", partition_size=-2)


@pytest.mark.parametrize("lengths", [[1], [1, 1, 1], [15, 16, 17, 33]])
def test_balanced_split_fewer_tiles_than_waves(lengths):
    case = make_case(batch=len(lengths), num_heads=8, num_kv_heads=2, head_dim=64, block_size=16,
                     lengths=lengths, dtype="float16", seed=43)
    _check(case, "paged_decode_attention_hip", label="sk-tiny", partition_size=-2)


@pytest.mark.parametrize("dtype,head_dim", [("float16", 128), ("bfloat16", 64)])
def test_mha_balanced_split_runs_on_the_mfma_family(dtype, head_dim):
    """partition_size=-2 on MHA (one query head per KV head): the launch
    moves from the per-head kernel to the MFMA family's balanced split; the
    plain, grouped and prepared entry points all match the oracle."""
    from inferkernellab_amd import ops

    gen = np.random.default_rng(50 + head_dim)
    lengths = [int(x) for x in gen.integers(1, 1500, size=12)]
    lengths[3] = 1
    case = make_case(batch=12, num_heads=16, num_kv_heads=16, head_dim=head_dim, block_size=16,
                     lengths=lengths, dtype=dtype, seed=51)
    _check(case, "paged_decode_attention_hip", label="mha-sk", partition_size=-2)
    _check(case, "paged_decode_attention_hip_grouped", label="mha-sk-grouped", partition_size=-2,
           query_group_size=8)
    attn = ops.PreparedPagedAttention(case.device_query(), case.device_cache(), case.device_tables(),
                                      case.device_lengths(), max_context_len=max(lengths), partition_size=-2)
    assert attn.path == "mfma_grouped" and attn.balanced_split
    out = attn()
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected()) <= ATOL[dtype]


@pytest.mark.parametrize("partition_size", [None, -2, 256])
def test_empty_contexts_give_nan_rows_and_leave_others_exact(partition_size):
    """validate_inputs=False with zero-length requests: their rows are NaN
    (0/0, as the reference's softmax over nothing) in both split modes; the
    other requests match the oracle."""
    from inferkernellab_amd import ops

    case = make_case(batch=4, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                     lengths=[300, 1, 900, 64], dtype="bfloat16", seed=44)
    lens = case.device_lengths()
    lens[1] = 0
    lens[3] = 0
    out = ops.paged_decode_attention_hip(case.device_query(), case.device_cache(), case.device_tables(),
                                         lens, validate_inputs=False, partition_size=partition_size)
    torch.cuda.synchronize()
    assert torch.isnan(out[1].float()).all() and torch.isnan(out[3].float()).all()
    expected = case.expected()
    for b in (0, 2):
        assert max_abs_err(out[b:b + 1], expected[b:b + 1]) <= ATOL["bfloat16"]


@pytest.mark.parametrize("partition_size", [None, -2, 128])
def test_context_past_table_capacity_is_masked(partition_size):
    """validate_inputs=False, context_lens beyond the table: positions with no
    table entry are masked, so the result is attention over the mapped part."""
    from inferkernellab_amd import ops
    from oracle import paged_oracle as po

    case = make_case(batch=2, num_heads=8, num_kv_heads=2, head_dim=128, block_size=16,
                     lengths=[64, 100], dtype="bfloat16", seed=45)
    # request 0: 4 own blocks, then 3 written blocks of request 1 -> the
    # table maps 7 * 16 = 112 positions, all holding data
    row0 = list(case.tables[0]) + list(case.tables[1][:3])
    tables = torch.tensor([row0, list(case.tables[1])], dtype=torch.int32, device="cuda")
    lens = torch.tensor([5000, 100], dtype=torch.int32, device="cuda")
    out = ops.paged_decode_attention_hip(case.device_query(), case.device_cache(), tables, lens,
                                         validate_inputs=False, partition_size=partition_size)
    torch.cuda.synchronize()
    k0, v0 = case.oracle_cache.read(0, row0, 112)
    ref0 = po.dense_decode_attention(case.query_f32[0:1], po.to_f32(k0, case.dtype), po.to_f32(v0, case.dtype))
    assert max_abs_err(out[0:1], ref0) <= ATOL["bfloat16"]
    assert max_abs_err(out[1:2], case.expected()[1:2]) <= ATOL["bfloat16"]


def test_balanced_and_fixed_partitions_agree():
    from inferkernellab_amd import ops

    case = make_case(batch=8, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                     lengths=[4096, 17, 8192, 5000, 1, 6000, 333, 7777], dtype="bfloat16", seed=46)
    cache = case.device_cache()
    args = (case.device_query(), cache, case.device_tables(), case.device_lengths())
    a = ops.paged_decode_attention_hip(*args, partition_size=-2)
    b = ops.paged_decode_attention_hip(*args, partition_size=512)
    torch.cuda.synchronize()
    expected = case.expected()
    assert max_abs_err(a, expected) <= ATOL["bfloat16"]
    assert max_abs_err(b, expected) <= ATOL["bfloat16"]
    assert (a.float() - b.float()).abs().max().item() <= ATOL["bfloat16"]


# ------------------------------------------------- the benchmark configurations
def _fill_by_append(case, ops):
    """Builds the device cache by appending every context token through the
    HIP append (slot_mapping slots), then checks it bit for bit against the
    oracle cache, which holds the same tokens written by index_put."""
    from inferkernellab_amd.cache import PagedKVCache

    oc = case.oracle_cache
    cache = PagedKVCache(oc.num_blocks, oc.block_size, oc.num_kv_heads, oc.head_dim,
                         dtype=getattr(torch, case.dtype), device="cuda")
    cache.k.zero_()
    cache.v.zero_()
    ref = case.device_cache()
    for b, (table, n) in enumerate(zip(case.tables, case.lengths)):
        slots = cache.slot_mapping(table, 0, n).to(torch.int32)
        blocks, offs = (slots // oc.block_size).long(), (slots % oc.block_size).long()
        ops.append_kv_hip(ref.k[0][blocks, offs].contiguous(), ref.v[0][blocks, offs].contiguous(), cache, slots)
    torch.cuda.synchronize()
    for b, (table, n) in enumerate(zip(case.tables, case.lengths)):
        slots = cache.slot_mapping(table, 0, n)
        blocks, offs = slots // oc.block_size, slots % oc.block_size
        got = cache.k[0][blocks, offs]
        want = ref.k[0][blocks, offs]
        assert torch.equal(got.view(torch.int16) if got.element_size() == 2 else got.view(torch.int32),
                           want.view(torch.int16) if want.element_size() == 2 else want.view(torch.int32))
    return cache


@pytest.mark.parametrize(
    ("heads", "kv", "dim", "dtype", "lengths", "waves"),
    [
        # MHA fp16, 512 (request, head) units: two 256-token partitions -> 2 waves
        (32, 32, 128, "float16", [512, 1, 255, 256, 257, 3] + [int(x) for x in
                                  np.random.default_rng(11).integers(1, 513, size=10)], 2),
        # fp32 GQA 32/8, 32 units at the 128-token floor: four partitions -> 4 waves
        (32, 8, 64, "float32", [512, 1, 3, 300], 4),
        # three 128-token partitions -> 4 waves of 96 tokens
        (32, 8, 128, "float32", [384, 1, 129, 200], 4),
        # MHA fp32 head_dim 32 (the per-head kernel), 64 units: three partitions -> 4 waves
        (16, 16, 32, "float32", [384, 1, 100, 250], 4),
        # MHA bf16 head_dim 16 (no MFMA kernel), two partitions -> 2 waves
        (16, 16, 16, "bfloat16", [256, 255, 1, 17] * 8, 2),
    ],
)
def test_valu_workgroups_fold_up_to_four_partitions(heads, kv, dim, dtype, lengths, waves):
    """When a request needs at most 4 partitions on the VALU family, they run
    as the waves of one workgroup that merges them in LDS (no split, no
    reduce); ragged and one-token contexts leave some waves without tiles."""
    from inferkernellab_amd import ops

    case = make_case(batch=len(lengths), num_heads=heads, num_kv_heads=kv, head_dim=dim, block_size=16,
                     lengths=lengths, dtype=dtype, seed=70 + waves, kv_scale=0.5)
    fn = "paged_decode_attention_hip" if heads == kv else "paged_decode_attention_hip_grouped"
    _check(case, fn, label=f"valu-{waves}-waves")
    cfg = ops.paged_decode_autotune_config() if heads == kv else ops.paged_decode_grouped_autotune_config()
    assert cfg["num_warps"] == waves


def test_config_gqa_fp32_hd64_b4_ctx512():
    """GQA 32/8, head_dim 64, fp32, batch 4 x 512, block 16, 159-block pool,
    scale 1/8; the cache filled by appending every context token."""
    from inferkernellab_amd import ops

    case = make_case(batch=4, num_heads=32, num_kv_heads=8, head_dim=64, block_size=16,
                     lengths=[512] * 4, dtype="float32", seed=0, num_blocks=159)
    cache = _fill_by_append(case, ops)
    out = ops.paged_decode_attention_hip(case.device_query(), cache, case.device_tables(), case.device_lengths(),
                                         scale=0.125)
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected(scale=0.125)) <= ATOL["float32"]


def test_config_mha_fp16_hd128_b16_ctx512_with_append_step():
    """MHA 32/32, head_dim 128, fp16, batch 16: 511 cached tokens, one
    appended per request through slot_mapping, then attention over 512;
    pool batch * ceil(512/16) + 8 = 520 blocks."""
    from inferkernellab_amd import ops

    case = make_case(batch=16, num_heads=32, num_kv_heads=32, head_dim=128, block_size=16,
                     lengths=[512] * 16, dtype="float16", seed=2, num_blocks=520)
    cache = case.device_cache()
    # rewrite token 511 of every request through the HIP append (the step's append)
    slots = torch.cat([cache.slot_mapping(t, 511, 1) for t in case.tables]).to(torch.int32)
    blocks, offs = (slots // 16).long(), (slots % 16).long()
    new_k, new_v = cache.k[0][blocks, offs].clone(), cache.v[0][blocks, offs].clone()
    cache.k[0][blocks, offs] = 0
    cache.v[0][blocks, offs] = 0
    ops.append_kv_hip(new_k, new_v, cache, slots)
    out = ops.paged_decode_attention_hip(case.device_query(), cache, case.device_tables(), case.device_lengths())
    torch.cuda.synchronize()
    assert torch.equal(cache.k[0][blocks, offs].view(torch.int16), new_k.view(torch.int16))
    assert max_abs_err(out, case.expected()) <= ATOL["float16"]


def test_config_mqa_bf16_hd128_b64_ctx1k_4k():
    """MQA 32/1, head_dim 128, bf16, batch 64, contexts U[1024, 4096], K/V
    0.5 * N(0, 1), scattered tables: one 32-head group per K/V tile."""
    gen = np.random.default_rng(3)
    lengths = [int(x) for x in gen.integers(1024, 4097, size=64)]
    case = make_case(batch=64, num_heads=32, num_kv_heads=1, head_dim=128, block_size=16,
                     lengths=lengths, dtype="bfloat16", seed=3, kv_scale=0.5)
    _check(case, "paged_decode_attention_hip", label="mqa-b64")
    _check(case, "paged_decode_attention_hip_grouped", label="mqa-b64-grouped", query_group_size=8)


def test_autotune_reporters_describe_the_last_launch():
    from inferkernellab_amd import ops

    case = make_case(batch=2, num_heads=8, num_kv_heads=2, head_dim=128, block_size=16,
                     lengths=[300, 40], dtype="bfloat16", seed=50)
    ops.paged_decode_attention_hip(case.device_query(), case.device_cache(), case.device_tables(),
                                   case.device_lengths())
    cfg = ops.paged_decode_grouped_dot_autotune_config()
    assert cfg == {"block_n": 16, "num_warps": 4, "num_stages": 2}  # a small batch: fixed partitions
    ops.paged_decode_attention_hip(case.device_query(), case.device_cache(), case.device_tables(),
                                   case.device_lengths(), partition_size=-2)
    cfg = ops.paged_decode_grouped_dot_autotune_config()
    # the balanced split, unit-parallel: the request's 2 units are the 2 waves of a workgroup
    assert cfg == {"block_n": 16, "num_warps": 2, "num_stages": 2}
    case32 = make_case(batch=2, num_heads=8, num_kv_heads=8, head_dim=64, block_size=16,
                       lengths=[30, 40], dtype="float32", seed=51)
    ops.paged_decode_attention_hip(case32.device_query(), case32.device_cache(), case32.device_tables(),
                                   case32.device_lengths())
    mha = ops.paged_decode_autotune_config()
    assert set(mha) == {"block_n", "num_warps", "num_stages"} and mha["num_warps"] == 1


@pytest.mark.parametrize("lengths,heads,kv", [([4096, 17, 8192, 5000, 1, 6000, 333, 7777], 32, 8),
                                             ([20000], 8, 1)])
def test_prepared_balanced_split_repeats_bit_identically(lengths, heads, kv):
    """One prepared workspace serves repeated balanced-split launches (a unit
    over ~1250 waves included) with bit-identical results."""
    from inferkernellab_amd import ops

    case = make_case(batch=len(lengths), num_heads=heads, num_kv_heads=kv, head_dim=128, block_size=16,
                     lengths=lengths, dtype="bfloat16", seed=47)
    attn = ops.PreparedPagedAttention(case.device_query(), case.device_cache(), case.device_tables(),
                                      case.device_lengths(), max_context_len=max(lengths), partition_size=-2)
    assert attn.balanced_split
    first = attn().clone()
    for _ in range(4):
        again = attn()
        torch.cuda.synchronize()
        assert torch.equal(again.view(torch.int16), first.view(torch.int16))
    assert max_abs_err(first, case.expected()) <= ATOL["bfloat16"]


def test_max_context_len_below_a_context_is_rejected():
    """max_context_len sizes the fixed-partition grid; with validate_inputs a
    context longer than it raises instead of being cut short."""
    from inferkernellab_amd import ops

    case = make_case(batch=2, num_heads=8, num_kv_heads=2, head_dim=128, block_size=16,
                     lengths=[1500, 700], dtype="bfloat16", seed=52)
    args = (case.device_query(), case.device_cache(), case.device_tables(), case.device_lengths())
    with pytest.raises(ValueError, match="max_context_len"):
        ops.paged_decode_attention_hip(*args, partition_size=512, max_context_len=1024)
    with pytest.raises(ValueError, match="max_context_len"):
        ops.PreparedPagedAttention(*args, partition_size=512, max_context_len=1024)
    out = ops.paged_decode_attention_hip(*args, partition_size=512, max_context_len=1500)
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected()) <= ATOL["bfloat16"]


@pytest.mark.parametrize("dtype,heads,kv", [("bfloat16", 32, 8), ("float16", 16, 16), ("float32", 8, 2),
                                            ("bfloat16", 32, 1)])
@pytest.mark.parametrize("partition_size", [None, -1, 64, -2])
def test_nan_key_inside_the_context_propagates_like_the_reference(dtype, heads, kv, partition_size):
    """A NaN in one attended key row makes every query head of that KV head
    NaN for that request, as paged_reference's softmax does
    (attention.py:18-36); other heads and requests stay finite and within
    tolerance. Keys past a context (NaN poison, never attended) are covered
    by the other tests."""
    from inferkernellab_amd import ops

    if partition_size == -2 and dtype == "float32":
        pytest.skip("the balanced split runs on the MFMA family (fp16 / bf16)")
    lengths = [300, 45, 700]
    case = make_case(batch=3, num_heads=heads, num_kv_heads=kv, head_dim=64, block_size=16,
                     lengths=lengths, dtype=dtype, seed=90 + heads)
    oc = case.oracle_cache
    bad_head = kv - 1
    slot = oc.slot_mapping(case.tables[2], 123, 1)[0]  # request 2, position 123
    nan = np.uint16(0x7FC0) if dtype == "bfloat16" else np.nan
    oc.k[0, slot // 16, slot % 16, bad_head, 5] = nan
    print(f"nan-key case dtype={dtype} H={heads} Hkv={kv} partition={partition_size}", flush=True)
    out = ops.paged_decode_attention_hip(case.device_query(), case.device_cache(), case.device_tables(),
                                         case.device_lengths(), partition_size=partition_size)
    torch.cuda.synchronize()
    expected = case.expected()
    got = out.float().cpu().numpy()
    assert np.array_equal(np.isnan(got), np.isnan(expected))
    per_kv = heads // kv
    assert np.isnan(expected[2, bad_head * per_kv:(bad_head + 1) * per_kv]).all()
    finite = ~np.isnan(expected)
    assert finite.sum() == expected.size - per_kv * 64
    assert np.abs(got[finite] - expected[finite]).max() <= ATOL[dtype]


@pytest.mark.parametrize(("heads", "kv", "qgs", "dim", "waves"), [
    (32, 8, 0, 128, 8),   # 8 units per request: one 8-wave group
    (16, 16, 0, 64, 8),   # MHA on the matrix cores: 16 one-head units, two 8-unit groups
    (32, 4, 2, 128, 8),   # query groups of 2: 16 units, two groups
    (12, 6, 0, 64, 2),    # 6 units: three 2-unit groups
    (8, 2, 0, 32, 2),     # 2 units
    (24, 3, 0, 128, 1),   # 3 units: one-unit runs
])
def test_balanced_split_unit_parallel_workgroups(heads, kv, qgs, dim, waves):
    """The balanced split's unit-parallel form: each workgroup's waves are
    consecutive units of a request walking the same request tiles, so the
    sequence is (request, unit group, tile) and the reduce finds a unit's
    pieces at stride UW. Ragged lengths (1, block edges, long) over 9
    requests, against the oracle; the launch reports UW waves per group."""
    from inferkernellab_amd import ops

    lengths = [1, 16, 17, 700, 2047, 33, 300, 1024, 5]
    case = make_case(batch=9, num_heads=heads, num_kv_heads=kv, head_dim=dim, block_size=16,
                     lengths=lengths, dtype="bfloat16", seed=heads + kv + dim)
    fn = "paged_decode_attention_hip_grouped" if qgs else "paged_decode_attention_hip"
    kw = {"query_group_size": qgs} if qgs else {}
    _check(case, fn, label=f"unit-parallel-{waves}", partition_size=-2, **kw)
    attn = ops.PreparedPagedAttention(case.device_query(), case.device_cache(), case.device_tables(),
                                      case.device_lengths(), max_context_len=max(lengths), partition_size=-2,
                                      query_group_size=qgs)
    assert attn.balanced_split and attn.launch["num_warps"] == waves
    out = attn()
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected()) <= ATOL["bfloat16"]
