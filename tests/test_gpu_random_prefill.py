"""Paged prefill attention over seeded random shapes against the fp32
oracle (attention.py:230-321): 1-8 KV heads under up to 32 query heads,
head_dim 16-256 (the MFMA family for fp16/bf16 at 32/64/96/128 with block
sizes that are multiples of 16, the VALU family otherwise), fp16/bf16/fp32,
block sizes 8-48, 1-6 requests with chunks starting anywhere in their
context and shorter chunks padded to the batch's widest. Bound: max-abs
2e-3 fp16, 1e-2 bf16, 1e-4 fp32, plus half an output ulp."""

import random

import pytest
import torch

from tests.helpers import assert_close_up_to_output_rounding, make_prefill_case

pytestmark = pytest.mark.gpu


def _shapes(seed: int, n: int):
    rng = random.Random(seed)
    for i in range(n):
        kv = rng.choice([1, 2, 4, 8])
        heads = kv * rng.choice([1, 2, 3, 4])
        dim = rng.choice([32, 64, 96, 128, 128, 16, 80, 256])
        dtype = rng.choice(["float16", "bfloat16", "float32"])
        bs = rng.choice([16, 16, 32, 48, 8])
        batch = rng.choice([1, 2, 3, 6])
        ends = [rng.randint(1, 600) for _ in range(batch)]
        starts = [rng.choice([0, rng.randint(0, e - 1)]) for e in ends]
        yield i, heads, kv, dim, dtype, bs, starts, ends


@pytest.mark.parametrize("seed", [21, 22])
def test_random_prefill_shapes_match_oracle(seed):
    from inferkernellab_amd import PreparedPagedPrefill

    for i, heads, kv, dim, dtype, bs, starts, ends in _shapes(seed, 30):
        print(f"random prefill {seed}/{i}: H={heads} Hkv={kv} D={dim} {dtype} bs={bs} starts={starts} ends={ends}",
              flush=True)
        case = make_prefill_case(starts=starts, ends=ends, num_heads=heads, num_kv_heads=kv, head_dim=dim,
                                 block_size=bs, dtype=dtype, seed=7000 + 100 * seed + i)
        q = case.device_query()
        prep = PreparedPagedPrefill(case.base.device_cache(), case.base.device_tables(), starts, ends,
                                    num_heads=heads, query_width=q.shape[2])
        out = prep(q, 0)
        torch.cuda.synchronize()
        assert_close_up_to_output_rounding(out, case.expected(), dtype)
