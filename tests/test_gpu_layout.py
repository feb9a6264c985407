"""The head-major block layout ([kv_heads, block_size, head_dim] per block,
`PagedKVCache(head_major=True)`; the default of the FP8 cache) through every
kernel: the same results as the reference's token-major layout, against the
oracle."""

import numpy as np
import pytest
import torch

from oracle import paged_oracle as po
from tests.helpers import ATOL, make_case, make_prefill_case, max_abs_err, storage_to_torch

pytestmark = pytest.mark.gpu


def _head_major_copy(case):
    from inferkernellab_amd import PagedKVCache

    oc = case.oracle_cache
    cache = PagedKVCache(oc.num_blocks, oc.block_size, oc.num_kv_heads, oc.head_dim, dtype=getattr(torch, case.dtype),
                         device="cuda", head_major=True)
    assert cache.k.stride(3) == oc.block_size * oc.head_dim and cache.k.stride(2) == oc.head_dim
    cache.k.copy_(storage_to_torch(oc.k, case.dtype))
    cache.v.copy_(storage_to_torch(oc.v, case.dtype))
    return cache


# the balanced split (-2) is the matrix-core family's; MHA runs the VALU family
@pytest.mark.parametrize("partition,heads,kv", [(p, h, k) for p in (None, -2, 256)
                                                for h, k in ((32, 8), (32, 1), (8, 8)) if not (p == -2 and h == k)])
def test_decode_attention_on_head_major_cache(partition, heads, kv):
    from inferkernellab_amd import ops

    case = make_case(batch=4, num_heads=heads, num_kv_heads=kv, head_dim=128, block_size=16,
                     lengths=[1000, 17, 4097, 300], dtype="bfloat16", seed=heads + kv)
    cache = _head_major_copy(case)
    out = ops.paged_decode_attention_hip_grouped(case.device_query(), cache, case.device_tables(),
                                                 case.device_lengths(), partition_size=partition)
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected()) < ATOL["bfloat16"]


def test_folded_valu_workgroups_on_head_major_cache():
    """fp32 GQA 32/8: each request's four 128-token partitions run as one
    4-wave VALU workgroup, reading head-major blocks."""
    from inferkernellab_amd import ops

    case = make_case(batch=4, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                     lengths=[512, 1, 300, 129], dtype="float32", seed=77)
    cache = _head_major_copy(case)
    out = ops.paged_decode_attention_hip_grouped(case.device_query(), cache, case.device_tables(),
                                                 case.device_lengths())
    torch.cuda.synchronize()
    assert ops.paged_decode_grouped_autotune_config()["num_warps"] == 4
    assert max_abs_err(out, case.expected()) < ATOL["float32"]


def test_prefill_attention_on_head_major_cache():
    from inferkernellab_amd import PreparedPagedPrefill

    case = make_prefill_case(starts=[0, 30], ends=[200, 150], width=200, num_heads=16, num_kv_heads=4,
                             head_dim=128, block_size=16, dtype="bfloat16", seed=3)
    cache = _head_major_copy(case.base)
    prep = PreparedPagedPrefill(cache, case.base.device_tables(), case.starts, case.ends, num_heads=16,
                                query_width=200)
    got = prep(case.device_query(), 0)
    torch.cuda.synchronize()
    assert max_abs_err(got, case.expected()) < ATOL["bfloat16"]


def test_append_and_rope_append_into_head_major_cache():
    from inferkernellab_amd import PagedKVCache, append_kv_hip, rope_append_kv_hip

    gen = torch.Generator().manual_seed(9)
    nb, bs, kv, d, t = 6, 16, 4, 64, 21
    key = torch.randn(t, kv, d, generator=gen).to(torch.bfloat16).cuda()
    value = torch.randn(t, kv, d, generator=gen).to(torch.bfloat16).cuda()
    slots = torch.randperm(nb * bs, generator=gen)[:t].to(torch.int32).cuda()
    caches = [PagedKVCache(nb, bs, kv, d, dtype=torch.bfloat16, device="cuda", head_major=h) for h in (False, True)]
    for c in caches:
        c.k.zero_()
        c.v.zero_()
        append_kv_hip(key, value, c, slots)
    assert torch.equal(caches[0].k, caches[1].k) and torch.equal(caches[0].v, caches[1].v)
    cos = torch.randn(t, d, generator=gen).to(torch.bfloat16).cuda()
    sin = torch.randn(t, d, generator=gen).to(torch.bfloat16).cuda()
    for c in caches:
        rope_append_kv_hip(None, key, value, cos, sin, c, slots)
    torch.cuda.synchronize()
    assert torch.equal(caches[0].k, caches[1].k) and torch.equal(caches[0].v, caches[1].v)
