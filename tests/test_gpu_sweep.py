"""A seeded random sweep of the decode and prefill launch space against the
oracle. Each case draws a dtype, head_dim, block size, KV heads and heads
per KV head, a query group size, ragged lengths (with 1 and the block edges
over-represented), the split mode, the block layout and, where the MFMA
family runs, the FP8 cache, then checks the kernels through the C ABI.
Even decode cases call the reference's grouped signature, odd ones the C
ABI with the drawn query group size as the exact unit size.
Tolerance: max-abs 2e-3 fp16 / 1e-2 bf16 / 1e-4 fp32 against the fp32
oracle, plus half an ulp of the output at its magnitude (the rounding of
the output itself). Every case prints its configuration before it runs."""

import random

import numpy as np
import pytest
import torch

from oracle import paged_oracle as po
from tests.helpers import assert_close_up_to_output_rounding, make_case, make_prefill_case, storage_to_torch

pytestmark = pytest.mark.gpu

DECODE_CASES = 40
PREFILL_CASES = 24
TORCH = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _decode_config(i: int) -> dict:
    rng = random.Random(7000 + i)
    dtype = rng.choice(["float16", "bfloat16", "float32"])
    fp8 = dtype != "float32" and rng.random() < 0.3
    head_dim = rng.choice([32, 64, 96, 128] if fp8 else [16, 32, 64, 96, 128])
    block_size = rng.choice([16, 32, 48, 64] if fp8 else [1, 4, 8, 16, 24, 32, 48, 64])
    kv = rng.choice([1, 2, 4, 8])
    group = rng.choice([1, 2, 3, 4, 8, 16, 32] if kv <= 2 else [1, 2, 4, 8])
    batch = rng.randint(1, 6)
    lengths = [rng.choice([1, block_size, block_size + 1, rng.randint(1, 700), rng.randint(700, 4000)])
               for _ in range(batch)]
    partition = rng.choice([None, -2, 256, -1, 64 * rng.randint(1, 8)])
    mfma = fp8 or (dtype != "float32" and block_size % 16 == 0 and head_dim in (32, 64, 96, 128) and group > 1)
    if partition == -2 and not mfma:  # the balanced split is the matrix-core family's
        partition = None
    return dict(dtype=dtype, fp8=fp8, head_dim=head_dim, block_size=block_size, kv=kv, heads=kv * group,
                lengths=lengths, partition=partition,
                query_group_size=rng.choice([1, 2, 4, 8]),  # the reference signature's values
                head_major=(not fp8 and dtype != "float32" and rng.random() < 0.3) or (fp8 and rng.random() < 0.7),
                seed=i)


def _fp8_device_cache(case, head_major, act):
    """Quantises the oracle cache's K/V rows in place (the oracle then
    attends the dequantised values) and returns the device FP8 cache."""
    from inferkernellab_amd import PagedKVCache

    oc = case.oracle_cache
    rows_k, rows_v = po.to_f32(oc.k[0], case.dtype), po.to_f32(oc.v[0], case.dtype)
    written = ~np.isnan(rows_k).any(-1)  # [NB, bs, Hkv]: slots holding a token
    kc, ks = po.quantize_rows_e4m3(np.where(written[..., None], rows_k, 0.0).astype(np.float32))
    vc, vs = po.quantize_rows_e4m3(np.where(written[..., None], rows_v, 0.0).astype(np.float32))
    deq_k, deq_v = po.dequantize_rows_e4m3(kc, ks), po.dequantize_rows_e4m3(vc, vs)
    cache = PagedKVCache(oc.num_blocks, oc.block_size, oc.num_kv_heads, oc.head_dim, dtype=torch.float8_e4m3fn,
                         act_dtype=TORCH[act], device="cuda", head_major=head_major)
    cache.k[0].view(torch.uint8).copy_(torch.from_numpy(kc))
    cache.v[0].view(torch.uint8).copy_(torch.from_numpy(vc))
    cache.k_scale[0].copy_(torch.from_numpy(np.ascontiguousarray(ks.transpose(0, 2, 1))))
    cache.v_scale[0].copy_(torch.from_numpy(np.ascontiguousarray(vs.transpose(0, 2, 1))))
    # the oracle now holds the dequantised rows (fp32 storage)
    oc.dtype = "float32"
    oc.k = deq_k[None].astype(np.float32)
    oc.v = deq_v[None].astype(np.float32)
    return cache


def _device_cache(case, head_major):
    from inferkernellab_amd import PagedKVCache

    oc = case.oracle_cache
    cache = PagedKVCache(oc.num_blocks, oc.block_size, oc.num_kv_heads, oc.head_dim, dtype=TORCH[case.dtype],
                         device="cuda", head_major=head_major)
    cache.k.copy_(storage_to_torch(oc.k, case.dtype))
    cache.v.copy_(storage_to_torch(oc.v, case.dtype))
    return cache


@pytest.mark.parametrize("i", range(DECODE_CASES))
def test_decode_sweep(i):
    from inferkernellab_amd import ops

    cfg = _decode_config(i)
    print(f"decode sweep case {i}: {cfg}", flush=True)
    case = make_case(batch=len(cfg["lengths"]), num_heads=cfg["heads"], num_kv_heads=cfg["kv"],
                     head_dim=cfg["head_dim"], block_size=cfg["block_size"], lengths=cfg["lengths"],
                     dtype=cfg["dtype"], seed=cfg["seed"])
    query = case.device_query()
    expected_q = case.query_f32
    if cfg["fp8"]:
        cache = _fp8_device_cache(case, cfg["head_major"], cfg["dtype"])
    else:
        cache = _device_cache(case, cfg["head_major"])
    if i % 2 == 0:  # the reference's grouped signature
        out = ops.paged_decode_attention_hip_grouped(query, cache, case.device_tables(), case.device_lengths(),
                                                     query_group_size=cfg["query_group_size"],
                                                     partition_size=cfg["partition"])
    else:  # the C ABI's explicit group size (units of exactly that many heads)
        out = ops.PreparedPagedAttention(query, cache, case.device_tables(), case.device_lengths(),
                                         query_group_size=cfg["query_group_size"],
                                         partition_size=cfg["partition"])()
    torch.cuda.synchronize()
    expected = po.paged_decode_attention(expected_q, case.oracle_cache, case.tables, case.lengths)
    assert_close_up_to_output_rounding(out, expected, cfg["dtype"])


def _prefill_config(i: int) -> dict:
    rng = random.Random(9000 + i)
    dtype = rng.choice(["float16", "bfloat16", "float32"])
    mfma = dtype != "float32" and rng.random() < 0.75
    fp8 = mfma and rng.random() < 0.3
    head_dim = rng.choice([32, 64, 96, 128]) if mfma else rng.choice([16, 32, 64, 80, 128, 256])
    block_size = rng.choice([16, 32, 48, 64]) if mfma else rng.choice([1, 4, 8, 16, 24, 32])
    kv = rng.choice([1, 2, 4, 8])
    group = rng.choice([1, 2, 3, 4, 8] if kv > 1 else [1, 4, 8, 16, 32])
    batch = rng.randint(1, 4)
    ends = [rng.randint(1, 900) for _ in range(batch)]
    starts = [rng.choice([0, 0, rng.randint(0, e - 1)]) for e in ends]
    width = max(e - s for s, e in zip(starts, ends)) + rng.choice([0, 0, 5])
    return dict(dtype=dtype, fp8=fp8, head_dim=head_dim, block_size=block_size, kv=kv, heads=kv * group,
                starts=starts, ends=ends, width=width, head_major=rng.random() < 0.3 and dtype != "float32",
                seed=100 + i)


@pytest.mark.parametrize("i", range(PREFILL_CASES))
def test_prefill_sweep(i):
    from inferkernellab_amd import PreparedPagedPrefill

    cfg = _prefill_config(i)
    print(f"prefill sweep case {i}: {cfg}", flush=True)
    case = make_prefill_case(starts=cfg["starts"], ends=cfg["ends"], width=cfg["width"], num_heads=cfg["heads"],
                             num_kv_heads=cfg["kv"], head_dim=cfg["head_dim"], block_size=cfg["block_size"],
                             dtype=cfg["dtype"], seed=cfg["seed"])
    query = case.device_query()
    if cfg["fp8"]:
        cache = _fp8_device_cache(case.base, True, cfg["dtype"])
    else:
        cache = _device_cache(case.base, cfg["head_major"])
    prep = PreparedPagedPrefill(cache, case.base.device_tables(), cfg["starts"], cfg["ends"],
                                num_heads=cfg["heads"], query_width=cfg["width"])
    got = prep(query, 0)
    torch.cuda.synchronize()
    expected = po.paged_prefill_attention(case.query_f32, case.base.oracle_cache, case.base.tables,
                                          cfg["starts"], cfg["ends"])
    assert_close_up_to_output_rounding(got, expected, cfg["dtype"])


@pytest.mark.parametrize("dtype_name", ["fp16", "bf16"])
def test_reference_attention_matrix_matches_oracle(dtype_name):
    """The reference's 54-shape attention matrix (docs/benchmark_report.md:
    28-34: batch {1, 4, 16} x context {128, 512, 2048} x KV heads {32, 8, 1},
    32 heads, head_dim 64, block 16), built by the benchmark's own case
    builder with the reference's interleaved tables (benchmark.py:85-95):
    every request and head of the automatic launch against the oracle, at
    max-abs 2e-3 (fp16) / 1e-2 (bf16) plus half an output ulp (the bench's
    parity gate, which `bench.py --sweep` applies before timing each shape)."""
    import bench
    from inferkernellab_amd import ops

    dtype = dict(bench.SWEEP_DTYPES)[dtype_name]
    dev = torch.device("cuda", 0)
    for batch in bench.SWEEP_BATCHES:
        for ctx in bench.SWEEP_CONTEXTS:
            for kv in bench.SWEEP_KV_HEADS:
                print(f"reference matrix {dtype_name} B{batch} ctx{ctx} kv{kv}", flush=True)
                w = bench.build_sweep_case(batch, ctx, kv, dtype, dev)
                out = ops.paged_decode_attention_hip(w["query"], w["cache"], w["tables"], w["lens"])
                torch.cuda.synchronize()
                check = bench.parity(out, bench.oracle_step(bench.oracle_view(w), w), dtype)
                assert check["passed"], (batch, ctx, kv, check)
