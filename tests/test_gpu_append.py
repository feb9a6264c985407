"""KV append through the C ABI: bit-exact against the oracle's write_slots
(torch index_put semantics of cache.py:156-189)."""

import numpy as np
import pytest
import torch

from oracle import paged_oracle as po
from tests.helpers import TORCH_DTYPES, randn_storage, storage_to_torch, torch_to_storage

pytestmark = pytest.mark.gpu


def _run(dtype, num_blocks, block_size, hkv, d, tokens, *, layers=1, layer=0, slot_dtype=torch.int32,
         seed=0, strided=False):
    from inferkernellab_amd import PagedKVCache, append_kv_hip

    print(f"append case dtype={dtype} nb={num_blocks} bs={block_size} hkv={hkv} d={d} T={tokens} "
          f"layer={layer}/{layers} slots={slot_dtype} strided={strided}", flush=True)
    gen = torch.Generator().manual_seed(seed)
    oc = po.OracleCache(num_blocks, block_size, hkv, d, num_layers=layers, dtype=dtype, fill=np.nan)
    slots = torch.randperm(num_blocks * block_size, generator=gen)[:tokens]
    key = randn_storage(gen, (tokens, hkv, d), dtype)
    value = randn_storage(gen, (tokens, hkv, d), dtype)
    cache = PagedKVCache(num_blocks, block_size, hkv, d, num_layers=layers, dtype=TORCH_DTYPES[dtype],
                         device="cuda")
    cache.k.copy_(storage_to_torch(oc.k, dtype))
    cache.v.copy_(storage_to_torch(oc.v, dtype))
    oc.write_slots(layer, slots.numpy(), key, value)
    k_dev = storage_to_torch(key, dtype).cuda()
    v_dev = storage_to_torch(value, dtype).cuda()
    if strided:  # [T, Hkv, D] views into wider rows, e.g. slices of a fused qkv tensor
        wide = torch.zeros(tokens, hkv * 3, d, dtype=k_dev.dtype, device="cuda")
        wide[:, hkv : 2 * hkv] = k_dev
        k_dev = wide[:, hkv : 2 * hkv]
        wide_v = torch.zeros(tokens, hkv * 3, d, dtype=k_dev.dtype, device="cuda")
        wide_v[:, 2 * hkv :] = v_dev
        v_dev = wide_v[:, 2 * hkv :]
    append_kv_hip(k_dev, v_dev, cache, slots.to(slot_dtype).cuda(), layer=layer)
    torch.cuda.synchronize()
    assert np.array_equal(torch_to_storage(cache.k).view(np.uint8), oc.k.view(np.uint8))
    assert np.array_equal(torch_to_storage(cache.v).view(np.uint8), oc.v.view(np.uint8))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_append_bit_exact(dtype):
    _run(dtype, 64, 16, 8, 128, 300)


@pytest.mark.parametrize("slot_dtype", [torch.int32, torch.int64])
def test_append_slot_index_types(slot_dtype):
    _run("bfloat16", 40, 16, 8, 128, 32, slot_dtype=slot_dtype, seed=3)


def test_append_reference_test_shape():
    """tests/test_attention.py:196-207: 8 blocks of 8, 2 kv heads, D 16, 4 tokens."""
    _run("float16", 8, 8, 2, 16, 4, seed=2)


def test_append_layer_and_strided_inputs():
    _run("bfloat16", 32, 16, 4, 64, 40, layers=3, layer=2, strided=True, seed=4)


def test_append_odd_head_dim_and_block_size():
    _run("float16", 13, 3, 3, 20, 30, seed=5)  # 40-byte rows: 4-byte chunk path


def test_append_decode_step_shape():
    """One new token per request, 32 requests, 8x128 bf16 (the GQA decode append)."""
    _run("bfloat16", 20000, 16, 8, 128, 32, seed=6)


def test_append_skips_out_of_range_slots():
    from inferkernellab_amd import PagedKVCache, append_kv_hip

    cache = PagedKVCache(4, 4, 1, 8, dtype=torch.float16, device="cuda")
    cache.k.fill_(7)
    cache.v.fill_(7)
    key = torch.ones(3, 1, 8, dtype=torch.float16, device="cuda")
    slots = torch.tensor([-1, 16, 5], dtype=torch.int64, device="cuda")
    append_kv_hip(key, key * 2, cache, slots)
    torch.cuda.synchronize()
    expect = torch.full_like(cache.k, 7)
    expect[0, 1, 1] = 1
    assert torch.equal(cache.k, expect)


def test_append_validation_messages():
    from inferkernellab_amd import PagedKVCache, append_kv_hip

    cache = PagedKVCache(4, 4, 2, 8, dtype=torch.float16, device="cuda")
    key = torch.ones(2, 2, 8, dtype=torch.float16, device="cuda")
    slots = torch.tensor([0, 1], dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="does not match cache layout"):
        append_kv_hip(key[:, :1], key[:, :1], cache, slots)
    with pytest.raises(ValueError, match="token counts"):
        append_kv_hip(key, key, cache, slots[:1])
    with pytest.raises(IndexError, match="layer"):
        append_kv_hip(key, key, cache, slots, layer=1)
