"""The online softmax's lazy rescale with non-zero accumulators. Keys whose
magnitude grows along the context (x1 at position 0 to x12 at the end) make
the running maximum pass its 2^8 bound several times mid-sequence, so every
MFMA kernel rescales accumulators that already hold many keys: decode with
16-head and 32-head units, both split modes, the FP8 cache, and prefill.
Checked against the oracle (max-abs 1e-2 bf16, 2e-3 fp16). The peaked
prefill rows come close to single V values of magnitude >= 4, where half a
bf16 ulp (2^-6) already exceeds 1e-2: there the bound also allows the
rounding of the output itself, which every bf16-output kernel (the
reference's `.to(q.dtype)` included) incurs."""

import numpy as np
import pytest
import torch

from oracle import paged_oracle as po
from tests.helpers import ATOL, assert_close_up_to_output_rounding, make_case, make_prefill_case, max_abs_err

pytestmark = pytest.mark.gpu


def _to_storage(x: np.ndarray, dtype: str) -> np.ndarray:
    if dtype == "bfloat16":
        return po.f32_to_bf16_bits(x.astype(np.float32))
    return x.astype(po.storage_dtype(dtype))


def _grow_keys(case, lengths, dtype):
    """Scales key row p of every request by 1 + 11 p / (n - 1), in place."""
    oc = case.oracle_cache
    for table, n in zip(case.tables, lengths):
        slots = oc.slot_mapping(table, 0, n)
        blk, off = slots // oc.block_size, slots % oc.block_size
        f = (1.0 + 11.0 * np.arange(n) / max(n - 1, 1)).astype(np.float32)
        k = po.to_f32(oc.k[0, blk, off], dtype) * f[:, None, None]
        oc.k[0, blk, off] = _to_storage(k, dtype)


@pytest.mark.parametrize("partition", [None, -2, 256])
@pytest.mark.parametrize("heads,kv,dtype", [(32, 8, "bfloat16"), (32, 1, "bfloat16"), (16, 4, "float16")])
def test_decode_rescale_with_growing_keys(heads, kv, dtype, partition):
    from inferkernellab_amd import ops

    lengths = [3000, 700, 1500]
    case = make_case(batch=3, num_heads=heads, num_kv_heads=kv, head_dim=128, block_size=16, lengths=lengths,
                     dtype=dtype, seed=heads + kv)
    _grow_keys(case, lengths, dtype)
    out = ops.paged_decode_attention_hip_grouped(case.device_query(), case.device_cache(), case.device_tables(),
                                                 case.device_lengths(), partition_size=partition)
    torch.cuda.synchronize()
    assert max_abs_err(out, case.expected()) <= ATOL[dtype]


def test_decode_rescale_with_growing_keys_fp8_cache():
    from inferkernellab_amd import PagedKVCache, ops

    lengths = [2500, 900]
    base = make_case(batch=2, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16, lengths=lengths,
                     dtype="float32", seed=5)
    _grow_keys(base, lengths, "float32")
    oc = base.oracle_cache
    kc, ks = po.quantize_rows_e4m3(oc.k[0])
    vc, vs = po.quantize_rows_e4m3(oc.v[0])
    oc.k[0] = po.dequantize_rows_e4m3(kc, ks)
    oc.v[0] = po.dequantize_rows_e4m3(vc, vs)
    gen = torch.Generator().manual_seed(9)
    q = torch.randn(2, 32, 128, generator=gen).to(torch.bfloat16)
    cache = PagedKVCache(oc.num_blocks, 16, 8, 128, dtype=torch.float8_e4m3fn, device="cuda")
    cache.k[0].view(torch.uint8).copy_(torch.from_numpy(kc))
    cache.v[0].view(torch.uint8).copy_(torch.from_numpy(vc))
    cache.k_scale[0].copy_(torch.from_numpy(np.ascontiguousarray(ks.transpose(0, 2, 1))))
    cache.v_scale[0].copy_(torch.from_numpy(np.ascontiguousarray(vs.transpose(0, 2, 1))))
    out = ops.paged_decode_attention_hip_grouped(q.cuda(), cache, base.device_tables(), base.device_lengths())
    torch.cuda.synchronize()
    expected = po.paged_decode_attention(q.float().numpy(), oc, base.tables, lengths)
    assert max_abs_err(out, expected) <= ATOL["bfloat16"]


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
def test_prefill_rescale_with_growing_keys(dtype):
    from inferkernellab_amd import PreparedPagedPrefill

    starts, ends = [0, 300], [1100, 900]
    case = make_prefill_case(starts=starts, ends=ends, num_heads=16, num_kv_heads=4, head_dim=128, block_size=16,
                             dtype=dtype, seed=12)
    _grow_keys(case.base, ends, dtype)
    q = case.device_query()
    prep = PreparedPagedPrefill(case.base.device_cache(), case.base.device_tables(), starts, ends, num_heads=16,
                                query_width=q.shape[2])
    got = prep(q, 0)
    torch.cuda.synchronize()
    assert prep.path == "mfma_grouped"
    assert_close_up_to_output_rounding(got, case.expected(), dtype)
