"""GPU parity of the FP8 KV format: the HIP append's E4M3 codes and per-row
scales bit for bit against the oracle's quantiser, and the MFMA decode
attention over an FP8 cache against the fp32 oracle run on the dequantised
cache (tolerances: max-abs 1e-2 with bf16 queries, 2e-3 with fp16)."""

import numpy as np
import pytest
import torch

from oracle import paged_oracle as po
from tests.helpers import ATOL, make_case, max_abs_err, randn_storage, storage_to_torch

pytestmark = pytest.mark.gpu

TORCH = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _fp8_case(*, batch, heads, kv, dim, bs, lengths, act="bfloat16", seed=0, num_blocks=None):
    """Random K/V quantised row by row into E4M3 codes + scales; the oracle
    attends the dequantised fp32 values (unwritten slots stay NaN)."""
    base = make_case(batch=batch, num_heads=heads, num_kv_heads=kv, head_dim=dim, block_size=bs,
                     lengths=lengths, dtype="float32", seed=seed, num_blocks=num_blocks)
    oc = base.oracle_cache
    kc, ks = po.quantize_rows_e4m3(oc.k[0])  # [NB, bs, Hkv, D] codes, [NB, bs, Hkv] scales
    vc, vs = po.quantize_rows_e4m3(oc.v[0])
    oc.k[0] = po.dequantize_rows_e4m3(kc, ks)
    oc.v[0] = po.dequantize_rows_e4m3(vc, vs)
    gen = torch.Generator().manual_seed(seed + 17)
    q = randn_storage(gen, (batch, heads, dim), act)
    base.query = q.astype(np.float32) if act == "float32" else q
    base.dtype = act
    return base, (kc, ks, vc, vs)


def _device_fp8_cache(base, packed, act):
    from inferkernellab_amd import PagedKVCache

    kc, ks, vc, vs = packed
    oc = base.oracle_cache
    cache = PagedKVCache(oc.num_blocks, oc.block_size, oc.num_kv_heads, oc.head_dim, dtype=torch.float8_e4m3fn,
                         act_dtype=TORCH[act], device="cuda")
    cache.k[0].view(torch.uint8).copy_(torch.from_numpy(kc))
    cache.v[0].view(torch.uint8).copy_(torch.from_numpy(vc))
    cache.k_scale[0].copy_(torch.from_numpy(np.ascontiguousarray(ks.transpose(0, 2, 1))))
    cache.v_scale[0].copy_(torch.from_numpy(np.ascontiguousarray(vs.transpose(0, 2, 1))))
    return cache


def _expected(base):
    q = po.to_f32(base.query, base.dtype) if base.dtype != "float32" else base.query
    return po.paged_decode_attention(q, base.oracle_cache, base.tables, base.lengths)


@pytest.mark.parametrize("act", ["bfloat16", "float16", "float32"])
@pytest.mark.parametrize("dim", [32, 64, 96, 128, 256])
def test_fp8_append_codes_and_scales_are_bit_exact(act, dim):
    from inferkernellab_amd import PagedKVCache, append_kv_hip

    gen = torch.Generator().manual_seed(dim)
    tokens, kv, bs, nb = 37, 4, 16, 8
    key = storage_to_torch(randn_storage(gen, (tokens, kv, dim), act, 3.0), act)
    value = storage_to_torch(randn_storage(gen, (tokens, kv, dim), act, 0.5), act)
    key[5, 2] = 0  # a zero row keeps scale 1
    slots = torch.randperm(nb * bs, generator=gen)[:tokens].to(torch.int32)
    slots[7] = -1  # skipped
    slots[11] = nb * bs + 3  # outside the cache: skipped
    cache = PagedKVCache(nb, bs, kv, dim, dtype=torch.float8_e4m3fn, act_dtype=TORCH[act], device="cuda")
    cache.k.view(torch.uint8).fill_(0x55)
    cache.v.view(torch.uint8).fill_(0x55)
    cache.k_scale.fill_(-2.0)
    cache.v_scale.fill_(-2.0)
    append_kv_hip(key.cuda(), value.cuda(), cache, slots.cuda())
    torch.cuda.synchronize()
    kcodes = cache.k[0].view(torch.uint8).cpu().numpy()
    vcodes = cache.v[0].view(torch.uint8).cpu().numpy()
    kscale = cache.k_scale[0].cpu().numpy()
    vscale = cache.v_scale[0].cpu().numpy()
    written = np.zeros((nb, bs), dtype=bool)
    for t, slot in enumerate(slots.tolist()):
        if not 0 <= slot < nb * bs:
            continue
        b, o = divmod(slot, bs)
        written[b, o] = True
        for rows, codes, scales in ((key, kcodes, kscale), (value, vcodes, vscale)):
            oc_, os_ = po.quantize_rows_e4m3(rows[t].float().numpy())
            assert np.array_equal(codes[b, o], oc_), (t, slot)
            assert np.array_equal(scales[b, :, o], os_), (t, slot)
    assert (kcodes[~written] == 0x55).all() and (kscale.transpose(0, 2, 1)[~written] == -2.0).all()
    assert kscale[divmod(int(slots[5]), bs)[0], 2, divmod(int(slots[5]), bs)[1]] == 1.0


CASES = [
    # heads, kv, dim, bs, lengths
    (32, 8, 128, 16, [4099, 777, 1, 2048, 16, 33]),
    (32, 1, 128, 16, [1024, 515, 2000]),
    (8, 8, 64, 32, [300, 129, 64]),
    (12, 4, 96, 16, [250, 77]),
    (16, 4, 32, 48, [500, 91, 3]),
]


@pytest.mark.parametrize("act", ["bfloat16", "float16"])
@pytest.mark.parametrize("heads,kv,dim,bs,lengths", CASES)
@pytest.mark.parametrize("partition", [None, -2, 256, -1])
def test_fp8_decode_attention_matches_oracle(act, heads, kv, dim, bs, lengths, partition):
    from inferkernellab_amd import ops

    base, packed = _fp8_case(batch=len(lengths), heads=heads, kv=kv, dim=dim, bs=bs, lengths=lengths, act=act,
                             seed=heads + dim)
    cache = _device_fp8_cache(base, packed, act)
    attn = ops.PreparedPagedAttention(base.device_query(), cache, base.device_tables(), base.device_lengths(),
                                      partition_size=partition, max_context_len=max(lengths))
    assert attn.path == "mfma_grouped"
    got = attn()
    torch.cuda.synchronize()
    out = got.float().cpu().numpy()
    assert not np.isnan(out).any()
    assert max_abs_err(out, _expected(base), act) < ATOL[act]


@pytest.mark.parametrize("act,dim", [("bfloat16", 128), ("float16", 128), ("bfloat16", 96), ("float16", 64)])
def test_fp8_cache_8_wave_fixed_partitions(act, dim):
    """MQA 32/1 over the FP8 cache, 64 requests, longest context 4096:
    1024-token partitions on 8-wave workgroups (in place of 512-token ones
    at two 4-wave workgroups per CU). The other lengths are short and ragged
    (one token, a tile and one token, a partition and one token), which
    leaves waves without tiles and partitions part-filled, and keeps the
    oracle cheap."""
    from inferkernellab_amd import ops

    gen = np.random.default_rng(93 + dim)
    lengths = [int(x) for x in gen.integers(1, 600, size=64)]
    lengths[:5] = [4096, 1, 17, 1025, 2049]
    base, packed = _fp8_case(batch=64, heads=32, kv=1, dim=dim, bs=16, lengths=lengths, act=act, seed=94)
    cache = _device_fp8_cache(base, packed, act)
    print(f"fp8 8-wave case act={act} D={dim} lens={lengths[:8]}", flush=True)
    attn = ops.PreparedPagedAttention(base.device_query(), cache, base.device_tables(), base.device_lengths(),
                                      max_context_len=max(lengths))
    launch = attn.launch
    assert (launch["path"], launch["split"], launch["partition_size"], launch["num_warps"]) == \
        ("mfma_grouped", "fixed_partitions", 1024, 8)
    got = attn()
    torch.cuda.synchronize()
    out = got.float().cpu().numpy()
    assert not np.isnan(out).any()
    assert max_abs_err(out, _expected(base), act) < ATOL[act]


def test_fp8_append_then_attention_and_quantisation_error():
    """New tokens quantised by the HIP append, then attended: equal to the
    oracle on the dequantised cache; the FP8 error against the same
    attention on the unquantised bf16 rows stays small."""
    from inferkernellab_amd import PagedKVCache, append_kv_hip, ops

    heads, kv, dim, bs = 32, 8, 128, 16
    lengths = [300, 1025, 64]
    gen = torch.Generator().manual_seed(5)
    need = [-(-n // bs) for n in lengths]
    perm = torch.randperm(sum(need) + 4, generator=gen).tolist()
    tables, used = [], 0
    for n in need:
        tables.append(perm[used : used + n])
        used += n
    nb = sum(need) + 4
    cache = PagedKVCache(nb, bs, kv, dim, dtype=torch.float8_e4m3fn, device="cuda")
    ref16 = po.OracleCache(nb, bs, kv, dim, dtype="float32", fill=np.nan)
    for table, n in zip(tables, lengths):
        k = torch.randn(n, kv, dim, generator=gen).to(torch.bfloat16)
        v = torch.randn(n, kv, dim, generator=gen).to(torch.bfloat16)
        slots = cache.slot_mapping(table, 0, n).to(torch.int32)
        append_kv_hip(k.cuda(), v.cuda(), cache, slots.cuda())
        ref16.write_slots(0, slots.cpu().numpy().astype(np.int64), k.float().numpy(), v.float().numpy())
    q = torch.randn(len(lengths), heads, dim, generator=gen).to(torch.bfloat16)
    width = max(need)
    table_t = torch.tensor([t + [0] * (width - len(t)) for t in tables], dtype=torch.int32, device="cuda")
    out = ops.paged_decode_attention_hip_grouped(q.cuda(), cache, table_t,
                                                 torch.tensor(lengths, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    deq = po.OracleCache(nb, bs, kv, dim, dtype="float32", fill=np.nan)
    kcodes = cache.k[0].view(torch.uint8).cpu().numpy()
    vcodes = cache.v[0].view(torch.uint8).cpu().numpy()
    ks = cache.k_scale[0].cpu().numpy().transpose(0, 2, 1)
    vs = cache.v_scale[0].cpu().numpy().transpose(0, 2, 1)
    deq.k[0] = po.dequantize_rows_e4m3(kcodes, ks)
    deq.v[0] = po.dequantize_rows_e4m3(vcodes, vs)
    exp = po.paged_decode_attention(q.float().numpy(), deq, tables, lengths)
    got = out.float().cpu().numpy()
    assert max_abs_err(got, exp, "bfloat16") < ATOL["bfloat16"]
    exact = po.paged_decode_attention(q.float().numpy(), ref16, tables, lengths)
    quant_err = float(np.max(np.abs(got - exact)))
    print(f"fp8 KV quantisation error vs bf16 rows: max abs {quant_err:.4f}")
    assert quant_err < 0.05


def test_fp8_cache_is_rejected_where_not_supported():
    from inferkernellab_amd import PagedKVCache, ops

    cache = PagedKVCache(8, 16, 2, 64, dtype=torch.float8_e4m3fn, device="cuda")
    q = torch.zeros(1, 4, 64, dtype=torch.bfloat16, device="cuda")
    tables = torch.zeros(1, 2, dtype=torch.int32, device="cuda")
    lens = torch.ones(1, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="FP8"):  # the VALU family does not read E4M3 codes
        ops._launch_attention(q, cache, tables, lens, None, 0, query_group_size=0, partition_size=None,
                              max_context_len=None, path=ops._PATH_IDS["scalar_grouped"])
    with pytest.raises(ValueError, match="query and cache"):
        ops.paged_decode_attention_hip_grouped(q.half(), cache, tables, lens)


@pytest.mark.parametrize("act", ["bfloat16", "float16"])
@pytest.mark.parametrize("heads,kv,dim,bs,starts,ends,width", [
    (32, 8, 128, 16, [0, 40, 300], [77, 200, 420], 160),
    (16, 4, 96, 32, [0, 5], [130, 70], 130),
    (8, 8, 64, 16, [3, 0], [40, 19], 40),
    (32, 1, 32, 48, [0, 60], [100, 100], 100),
])
def test_fp8_prefill_attention_matches_oracle(act, heads, kv, dim, bs, starts, ends, width):
    """The MFMA prefill kernel over an FP8 cache against the oracle's prefill
    attention on the dequantised cache (padding rows: the value at position
    0, rounded to the query dtype)."""
    from inferkernellab_amd import PreparedPagedPrefill

    base, packed = _fp8_case(batch=len(ends), heads=heads, kv=kv, dim=dim, bs=bs, lengths=ends, act=act,
                             seed=dim + bs)
    cache = _device_fp8_cache(base, packed, act)
    gen = torch.Generator().manual_seed(dim)
    q = randn_storage(gen, (len(ends), heads, width, dim), act)
    prep = PreparedPagedPrefill(cache, base.device_tables(), starts, ends, num_heads=heads, query_width=width)
    assert prep.path == "mfma_grouped"
    got = prep(storage_to_torch(q, act).cuda(), 0)
    torch.cuda.synchronize()
    exp = po.paged_prefill_attention(po.to_f32(q, act), base.oracle_cache, base.tables, starts, ends)
    out = got.float().cpu().numpy()
    assert not np.isnan(out).any()
    assert max_abs_err(out, exp, act) < ATOL[act]
