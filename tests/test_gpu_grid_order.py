"""GPU parity of the fixed-partition MFMA kernel on its request-fastest grid.

When the units per partition (kv heads x query groups) are not a multiple of
8 but units x partitions is, and the grid has more than 256 workgroups, the
kernel reads its (request, unit, partition) from a request-fastest grid with
the request rotated by partition % 8 (paged_attn.h, spread_grid). These cases
are sized to take that order, including batches below 8 (the rotation then
wraps more than once), a batch that is not a multiple of 8, ragged and
one-token contexts, 4-unit GQA and the FP8 cache; each is checked against the
fp32 oracle (max-abs 2e-3 fp16, 1e-2 bf16)."""

import numpy as np
import pytest
import torch

from tests.helpers import ATOL, make_case, max_abs_err

pytestmark = pytest.mark.gpu


def _takes_request_fastest_grid(units, parts, batch):
    """The library's rule (paged_attn.h spread_grid), restated so that each
    case below documents that it exercises the request-fastest order."""
    return units % 8 != 0 and (units * parts) % 8 == 0 and units * parts * batch > 256


def _parts(lengths, block_size, partition):
    width = max(-(-n // block_size) for n in lengths)
    return -(-(width * block_size) // partition)


CASES = [
    # heads, kv, dim, dtype, lengths, partition
    (32, 1, 128, "bfloat16", [9200, 300, 5000, 1], 128),
    (32, 4, 128, "bfloat16", [int(x) for x in np.random.default_rng(7).integers(200, 1025, size=40)], 512),
    (32, 1, 64, "float16", [int(x) for x in np.random.default_rng(8).integers(1, 2049, size=33)], 256),
]


@pytest.mark.parametrize("heads,kv,dim,dtype,lengths,partition", CASES)
def test_request_fastest_grid_matches_oracle(heads, kv, dim, dtype, lengths, partition):
    from inferkernellab_amd import ops

    lengths = list(lengths)
    if partition == 512:
        lengths[0] = 1024  # the table spans two partitions
    units = kv  # one query group per kv head (heads_per_kv <= 32)
    parts = _parts(lengths, 16, partition)
    assert _takes_request_fastest_grid(units, parts, len(lengths))
    case = make_case(batch=len(lengths), num_heads=heads, num_kv_heads=kv, head_dim=dim, block_size=16,
                     lengths=lengths, dtype=dtype, seed=60 + len(lengths), kv_scale=0.5)
    print(f"grid-order case H={heads} Hkv={kv} D={dim} {dtype} B={len(lengths)} P={partition} parts={parts} "
          f"lens={lengths[:6]}", flush=True)
    out = ops.paged_decode_attention_hip(case.device_query(), case.device_cache(), case.device_tables(),
                                         case.device_lengths(), partition_size=partition)
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected()) <= ATOL[dtype]


def test_request_fastest_grid_over_fp8_cache():
    from inferkernellab_amd import ops
    from tests.test_gpu_fp8 import _device_fp8_cache, _expected, _fp8_case

    lengths = [int(x) for x in np.random.default_rng(9).integers(64, 4097, size=40)]
    lengths[0] = 4096
    parts = _parts(lengths, 16, 512)
    assert _takes_request_fastest_grid(1, parts, len(lengths))
    base, packed = _fp8_case(batch=len(lengths), heads=32, kv=1, dim=128, bs=16, lengths=lengths, act="bfloat16",
                             seed=61)
    cache = _device_fp8_cache(base, packed, "bfloat16")
    print(f"grid-order fp8 case B={len(lengths)} parts={parts}", flush=True)
    attn = ops.PreparedPagedAttention(base.device_query(), cache, base.device_tables(), base.device_lengths(),
                                      partition_size=512, max_context_len=max(lengths))
    assert attn.path == "mfma_grouped"
    got = attn()
    torch.cuda.synchronize()
    out = got.float().cpu().numpy()
    assert not np.isnan(out).any()
    assert max_abs_err(out, _expected(base), "bfloat16") < ATOL["bfloat16"]
