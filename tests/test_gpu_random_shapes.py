"""Decode attention over seeded random shapes against the fp32 oracle:
head counts 8-64 with 1-32 KV heads (MHA, GQA, MQA, 20- and 24-head
groups), head_dim 16-128, fp16/bf16/fp32, block sizes 8/16/32, ragged
batches of 1-70 requests up to 3000 tokens, and every split choice (the
automatic one, unsplit, the balanced split and fixed partitions of
64-512 tokens) through both entry points. This crosses the kernel families'
planning rules (folded VALU workgroups, one-round MQA partitions, 4-wave
balanced runs, the small-MHA routing) with shapes no dedicated test picks;
40 more go over the FP8 cache. Bound: max-abs 2e-3 fp16, 1e-2 bf16, 1e-4 fp32, plus half an output ulp."""

import random

import pytest
import torch

from tests.helpers import assert_close_up_to_output_rounding, make_case

pytestmark = pytest.mark.gpu


def _shapes(seed: int, n: int):
    rng = random.Random(seed)
    for i in range(n):
        kv = rng.choice([1, 2, 4, 8, 16, 32])
        heads = rng.choice([h for h in (8, 16, 24, 32, 40, 48, 64) if h % kv == 0] or [kv])
        dim = rng.choice([16, 32, 64, 96, 128])
        dtype = rng.choice(["float16", "bfloat16", "float32"])
        bs = rng.choice([16, 16, 32, 8])
        batch = rng.choice([1, 2, 3, 5, 8, 16, 33, 70])
        maxlen = rng.choice([1, 17, 128, 300, 512, 700, 1500, 3000])
        lengths = [rng.randint(1, maxlen) for _ in range(batch)]
        if rng.random() < 0.5:
            lengths[0] = maxlen
        part = rng.choice([None, None, None, -1, -2, 64, 128, 256, 512])
        fn = rng.choice(["paged_decode_attention_hip", "paged_decode_attention_hip_grouped"])
        if part == -2 and (dtype == "float32" or dim == 16 or bs % 16):
            part = None  # the balanced split is the MFMA family's
        yield i, heads, kv, dim, dtype, bs, lengths, part, fn


@pytest.mark.parametrize("seed", [11, 12, 13])
def test_random_shapes_match_oracle(seed):
    from inferkernellab_amd import ops

    for i, heads, kv, dim, dtype, bs, lengths, part, fn in _shapes(seed, 40):
        print(f"random shape {seed}/{i}: H={heads} Hkv={kv} D={dim} {dtype} bs={bs} B={len(lengths)} "
              f"max={max(lengths)} P={part} {fn}", flush=True)
        case = make_case(batch=len(lengths), num_heads=heads, num_kv_heads=kv, head_dim=dim, block_size=bs,
                         lengths=lengths, dtype=dtype, seed=5000 + 100 * seed + i, kv_scale=0.5)
        out = getattr(ops, fn)(case.device_query(), case.device_cache(), case.device_tables(),
                               case.device_lengths(), partition_size=part)
        torch.cuda.synchronize()
        assert_close_up_to_output_rounding(out, case.expected(), dtype)


def _fp8_shapes(seed: int, n: int):
    rng = random.Random(seed)
    for i in range(n):
        kv = rng.choice([1, 2, 4, 8])
        heads = kv * rng.choice([1, 2, 4, 8, 16, 32])
        dim = rng.choice([32, 64, 96, 128])
        act = rng.choice(["float16", "bfloat16"])
        bs = rng.choice([16, 32])
        batch = rng.choice([1, 3, 8, 20])
        maxlen = rng.choice([1, 40, 300, 1200, 2500])
        lengths = [rng.randint(1, maxlen) for _ in range(batch)]
        part = rng.choice([None, None, -1, -2, 128, 512])
        yield i, heads, kv, dim, act, bs, lengths, part


def test_random_shapes_over_the_fp8_cache():
    """Decode over the FP8 cache (E4M3 codes + row scales) on 40 seeded
    random shapes and split choices, against the oracle on the dequantised
    cache."""
    from inferkernellab_amd import ops
    from tests.test_gpu_fp8 import _device_fp8_cache, _expected, _fp8_case

    for i, heads, kv, dim, act, bs, lengths, part in _fp8_shapes(31, 40):
        print(f"random fp8 shape {i}: H={heads} Hkv={kv} D={dim} {act} bs={bs} B={len(lengths)} "
              f"max={max(lengths)} P={part}", flush=True)
        base, packed = _fp8_case(batch=len(lengths), heads=heads, kv=kv, dim=dim, bs=bs, lengths=lengths, act=act,
                                 seed=9000 + i)
        cache = _device_fp8_cache(base, packed, act)
        out = ops.paged_decode_attention_hip(base.device_query(), cache, base.device_tables(), base.device_lengths(),
                                             partition_size=part)
        torch.cuda.synchronize()
        assert_close_up_to_output_rounding(out, _expected(base), act)
