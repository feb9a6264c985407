"""Fused rotary embedding + KV append (ikl_rope_append_kv) on the GPU
against the oracle's rope_rows and write_slots: rotated queries and the
cache rows bit for bit (the reference's torch RoPE then append,
hf_benchmark.py:419-436)."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _storage(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu()
    return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()


def _run(dtype, *, tokens=19, heads=32, kv=8, head_dim=128, block_size=16, num_blocks=40, in_place=True,
         bad_slot=False, slot_dtype=torch.int32):
    from inferkernellab_amd import ops
    from inferkernellab_amd.cache import PagedKVCache
    from inferkernellab_amd.llama import RotaryEmbedding
    from oracle import paged_oracle as po

    print(f"rope append {dtype} T={tokens} H={heads} Hkv={kv} D={head_dim} bs={block_size}", flush=True)
    gen = torch.Generator().manual_seed(tokens * 7 + head_dim)
    tdt = getattr(torch, dtype)
    q = torch.randn(tokens, heads, head_dim, generator=gen).to(tdt).cuda()
    k = torch.randn(tokens, kv, head_dim, generator=gen).to(tdt).cuda()
    v = torch.randn(tokens, kv, head_dim, generator=gen).to(tdt).cuda()
    pos = torch.randint(0, 5000, (tokens,), generator=gen).cuda()
    cos, sin = RotaryEmbedding(head_dim, 10000.0).cuda()(q, pos.view(-1, 1))
    cos, sin = cos[:, 0].contiguous(), sin[:, 0].contiguous()
    cache = PagedKVCache(num_blocks, block_size, kv, head_dim, num_layers=2, dtype=tdt, device="cuda")
    cache.k.zero_()
    cache.v.zero_()
    slots = torch.randperm(num_blocks * block_size, generator=gen)[:tokens]
    if bad_slot:
        slots[3] = num_blocks * block_size + 5
        slots[5] = -1
    slots = slots.to(slot_dtype).cuda()
    q_in = q.clone()
    out = ops.rope_append_kv_hip(q, k, v, cos, sin, cache, slots, layer=1,
                                 query_out=None if in_place else torch.empty_like(q))
    torch.cuda.synchronize()
    if in_place:
        assert out.data_ptr() == q.data_ptr()
    cs, ss = _storage(cos)[:, None, :], _storage(sin)[:, None, :]
    want_q = po.rope_rows(_storage(q_in), cs, ss, dtype)
    want_k = po.rope_rows(_storage(k), cs, ss, dtype)
    assert np.array_equal(_storage(out).view(np.uint8), want_q.view(np.uint8))
    oc = po.OracleCache(num_blocks, block_size, kv, head_dim, num_layers=2, dtype=dtype, fill=0.0)
    keep = [i for i, s in enumerate(slots.tolist()) if 0 <= s < num_blocks * block_size]
    oc.write_slots(1, slots.cpu().numpy()[keep], want_k[keep], _storage(v)[keep])
    assert np.array_equal(_storage(cache.k).view(np.uint8), oc.k.view(np.uint8))
    assert np.array_equal(_storage(cache.v).view(np.uint8), oc.v.view(np.uint8))


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_append_matches_oracle_bit_for_bit(dtype, head_dim):
    _run(dtype, head_dim=head_dim)


def test_rope_append_out_of_place_int64_slots_and_mqa():
    _run("bfloat16", kv=1, heads=32, in_place=False, slot_dtype=torch.int64)


def test_rope_append_skips_slots_outside_the_cache():
    _run("bfloat16", bad_slot=True, tokens=8)


def test_rope_append_prefill_sized_batch():
    _run("bfloat16", tokens=2048, heads=16, kv=4, num_blocks=200)
