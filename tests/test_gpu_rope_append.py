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


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_rope_append_into_fp8_cache_equals_rope_then_fp8_append(dtype, head_dim):
    """Into the FP8 cache the fused kernel equals ikl_rope_append_kv's own
    rotation followed by ikl_append_kv's quantisation: rotated q, codes and
    scales bit for bit, slots outside the cache skipped."""
    from inferkernellab_amd import ops
    from inferkernellab_amd.cache import PagedKVCache
    from inferkernellab_amd.llama import RotaryEmbedding

    print(f"rope append fp8 {dtype} D={head_dim}", flush=True)
    tokens, heads, kv, bs, nb = 23, 16, 4, 16, 12
    gen = torch.Generator().manual_seed(head_dim)
    tdt = getattr(torch, dtype)
    q = torch.randn(tokens, heads, head_dim, generator=gen).to(tdt).cuda()
    k = (torch.randn(tokens, kv, head_dim, generator=gen) * 4).to(tdt).cuda()
    v = torch.randn(tokens, kv, head_dim, generator=gen).to(tdt).cuda()
    pos = torch.randint(0, 3000, (tokens,), generator=gen).cuda()
    cos, sin = RotaryEmbedding(head_dim, 10000.0).cuda()(q, pos.view(-1, 1))
    cos, sin = cos[:, 0].contiguous().to(tdt), sin[:, 0].contiguous().to(tdt)
    slots = torch.randperm(nb * bs, generator=gen)[:tokens].to(torch.int32)
    slots[4] = -1
    slots[9] = nb * bs
    slots = slots.cuda()

    fused = PagedKVCache(nb, bs, kv, head_dim, dtype=torch.float8_e4m3fn, act_dtype=tdt, device="cuda")
    for t in (fused.k.view(torch.uint8), fused.v.view(torch.uint8)):
        t.fill_(0x11)
    q_fused = ops.rope_append_kv_hip(q.clone(), k, v, cos, sin, fused, slots)

    # reference: the same rotation into a 16-bit cache, then the FP8 append of its rows
    plain = PagedKVCache(nb, bs, kv, head_dim, dtype=tdt, device="cuda")
    plain.k.zero_()
    q_plain = ops.rope_append_kv_hip(q.clone(), k, v, cos, sin, plain, slots)
    k_rot = plain.k[0].reshape(nb * bs, kv, head_dim)
    ok = (slots >= 0) & (slots < nb * bs)
    good = slots[ok].long()
    sep = PagedKVCache(nb, bs, kv, head_dim, dtype=torch.float8_e4m3fn, act_dtype=tdt, device="cuda")
    for t in (sep.k.view(torch.uint8), sep.v.view(torch.uint8)):
        t.fill_(0x11)
    ops.append_kv_hip(k_rot[good].contiguous(), v[ok].contiguous(), sep, slots[ok].contiguous())
    torch.cuda.synchronize()
    assert torch.equal(q_fused.view(torch.uint8) if tdt != torch.float32 else q_fused,
                       q_plain.view(torch.uint8) if tdt != torch.float32 else q_plain)
    assert torch.equal(fused.k.view(torch.uint8), sep.k.view(torch.uint8))
    assert torch.equal(fused.v.view(torch.uint8), sep.v.view(torch.uint8))
    flat_ok = torch.zeros(nb * bs, dtype=torch.bool, device="cuda")
    flat_ok[good] = True
    written = flat_ok.view(nb, bs)
    for a, b in ((fused.k_scale[0], sep.k_scale[0]), (fused.v_scale[0], sep.v_scale[0])):
        assert torch.equal(a.transpose(1, 2)[written], b.transpose(1, 2)[written])
