"""Pins the CPU oracle before it is trusted as the parity reference.

Known answers come from the reference's own tests (tests/golden); the
attention restatement is checked against an independent float64 brute
force, closed forms, structural invariants and torch's softmax/einsum, and
planted mistakes in the oracle must be caught by these checks."""

import math

import numpy as np
import pytest
import torch

from oracle import paged_oracle as po
from tests.helpers import known_answers, make_case, randn_storage

KA = known_answers()


def _cache(spec, **kw):
    return po.OracleCache(spec["num_blocks"], spec["block_size"], spec["num_kv_heads"], spec["head_dim"], **kw)


def test_slot_mapping_known_answer():
    for case in KA["slot_mapping"]:
        cache = _cache(case["cache"])
        got = cache.slot_mapping(case["block_table"], case["start"], case["length"])
        assert got.tolist() == case["expected"]


def test_slot_mapping_rejections():
    for case in KA["slot_mapping_rejects"]:
        cache = _cache(case["cache"])
        with pytest.raises(ValueError, match=case["match"]):
            cache.slot_mapping(case["block_table"], case["start"], case["length"])


def test_slot_mapping_closed_form_all_positions():
    cache = po.OracleCache(37, 5, 1, 8)
    rng = np.random.default_rng(4)
    table = rng.permutation(37)[:9].tolist()
    got = cache.slot_mapping(table, 0, 45)
    for p, s in enumerate(got):
        assert s == table[p // 5] * 5 + p % 5
    # bijective onto the table's slots
    assert len(set(got.tolist())) == 45


def test_write_read_known_answers():
    case = KA["write_read_order"]
    cache = _cache(case["cache"], dtype="float32")
    key = np.arange(12, dtype=np.float32).reshape(2, 2, 3)
    cache.write(0, case["block_table"], case["start"], key, key + 100)
    k, v = cache.read(0, case["block_table"], case["read_length"])
    assert np.array_equal(k[2:], key) and np.array_equal(v[2:], key + 100)

    case = KA["write_slots_flattened"]
    cache = _cache(case["cache"], dtype="float32")
    slots = np.concatenate([cache.slot_mapping(case["block_table"], s, n) for s, n in case["ranges"]])
    assert slots.tolist() == case["expected_slots"]
    key = np.arange(24, dtype=np.float32).reshape(4, 2, 3)
    cache.write_slots(0, slots, key, key + 100)
    k, v = cache.read(0, case["block_table"], case["read_length"])
    assert np.array_equal(k[case["expected_rows_equal_key"]], key)
    assert np.array_equal(v[case["expected_rows_equal_key"]], key + 100)


def test_layers_are_independent():
    cache = po.OracleCache(4, 4, 1, 2, num_layers=2)
    cache.write(0, [0], 0, np.ones((2, 1, 2), np.float32), np.ones((2, 1, 2), np.float32))
    cache.write(1, [0], 0, np.full((2, 1, 2), 3, np.float32), np.full((2, 1, 2), 3, np.float32))
    assert np.array_equal(cache.read(0, [0], 2)[0], np.ones((2, 1, 2)))
    assert np.array_equal(cache.read(1, [0], 2)[0], np.full((2, 1, 2), 3))


def test_write_slots_matches_torch_index_put_bits():
    """Append semantics = torch index_put (the reference's torch backend)."""
    gen = torch.Generator().manual_seed(5)
    for dtype in ("float16", "bfloat16", "float32"):
        cache = po.OracleCache(16, 4, 3, 16, dtype=dtype, fill=0.0)
        slots = torch.randperm(64, generator=gen)[:23]
        key = randn_storage(gen, (23, 3, 16), dtype)
        value = randn_storage(gen, (23, 3, 16), dtype)
        cache.write_slots(0, slots.numpy(), key, value)
        tk = torch.zeros(16, 4, 3, 16, dtype=torch.int32 if dtype == "float32" else torch.int16)
        src = torch.from_numpy(key.view(np.int32 if dtype == "float32" else np.int16))
        tk[slots // 4, slots % 4] = src
        assert np.array_equal(cache.k[0].view(np.int32 if dtype == "float32" else np.int16), tk.numpy())


def test_write_slots_rejects_invalid_positions():
    cache = po.OracleCache(4, 4, 1, 2)
    with pytest.raises(ValueError, match="invalid physical cache position"):
        cache.write_slots(0, [16], np.zeros((1, 1, 2), np.float32), np.zeros((1, 1, 2), np.float32))


def test_bf16_conversion_matches_torch():
    x = torch.randn(4096, generator=torch.Generator().manual_seed(0)) * 100
    x = torch.cat([x, torch.tensor([1.00390625, 1.01171875, -0.0, 3.0e38, float("inf")])])
    bits = po.f32_to_bf16_bits(x.numpy())
    ref = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(bits, ref)
    assert np.array_equal(po.bf16_bits_to_f32(bits), x.to(torch.bfloat16).float().numpy())


# ------------------------------------------------------------ attention pins
def _tiny_case(num_heads, num_kv, dtype="float32", seed=0, lengths=(7, 8), head_dim=8, block_size=4):
    return make_case(batch=len(lengths), num_heads=num_heads, num_kv_heads=num_kv, head_dim=head_dim,
                     block_size=block_size, lengths=lengths, dtype=dtype, seed=seed)


@pytest.mark.parametrize("num_heads,num_kv", [(4, 4), (4, 2), (4, 1), (6, 3)])
def test_attention_matches_float64_brute_force(num_heads, num_kv):
    case = _tiny_case(num_heads, num_kv, seed=num_heads * 10 + num_kv)
    got = case.expected()
    for b, (table, n) in enumerate(zip(case.tables, case.lengths)):
        k, v = case.oracle_cache.read(0, table, n)
        ref = po.brute_force_attention_f64(case.query_f32[b].tolist(), k.tolist(), v.tolist())
        assert np.max(np.abs(got[b] - np.array(ref))) < 2e-6


def test_attention_context_one_returns_value():
    case = _tiny_case(4, 2, lengths=(1, 1))
    got = case.expected()
    for b, table in enumerate(case.tables):
        _, v = case.oracle_cache.read(0, table, 1)
        assert np.allclose(got[b], np.repeat(v[0], 2, axis=0), atol=0, rtol=0)


def test_attention_equal_keys_give_mean_value():
    cache = po.OracleCache(8, 4, 2, 8)
    gen = np.random.default_rng(1)
    key = np.repeat(gen.standard_normal((1, 2, 8)).astype(np.float32), 11, axis=0)
    value = gen.standard_normal((11, 2, 8)).astype(np.float32)
    cache.write(0, [3, 6, 1], 0, key, value)
    q = gen.standard_normal((1, 4, 8)).astype(np.float32)
    got = po.paged_decode_attention(q, cache, [[3, 6, 1]], [11])
    mean = value.mean(axis=0)
    assert np.allclose(got[0], np.repeat(mean, 2, axis=0), atol=1e-6)


def test_attention_one_dominant_key_selects_its_value():
    cache = po.OracleCache(8, 4, 1, 8)
    gen = np.random.default_rng(2)
    key = gen.standard_normal((9, 1, 8)).astype(np.float32) * 0.01
    key[5] = 40.0
    value = gen.standard_normal((9, 1, 8)).astype(np.float32)
    cache.write(0, [7, 0, 2], 0, key, value)
    q = np.ones((1, 2, 8), np.float32)
    got = po.paged_decode_attention(q, cache, [[7, 0, 2]], [9])
    assert np.allclose(got[0], np.repeat(value[5], 2, axis=0), atol=1e-6)


def test_gqa_equals_mha_on_expanded_cache():
    case = _tiny_case(8, 2, seed=3)
    gqa = case.expected()
    oc = case.oracle_cache
    mha = po.OracleCache(oc.num_blocks, oc.block_size, 8, oc.head_dim)
    mha.k[:] = np.repeat(oc.k, 4, axis=3)
    mha.v[:] = np.repeat(oc.v, 4, axis=3)
    got = po.paged_decode_attention(case.query_f32, mha, case.tables, case.lengths)
    assert np.allclose(gqa, got, atol=1e-6)


def test_block_table_permutation_invariance():
    case = _tiny_case(4, 2, seed=6, lengths=(13,))
    base = case.expected()
    oc = case.oracle_cache
    # move every block of the request to a different physical id
    remap = {old: new for old, new in zip(case.tables[0], reversed(range(oc.num_blocks)))}
    moved = po.OracleCache(oc.num_blocks, oc.block_size, oc.num_kv_heads, oc.head_dim)
    for old, new in remap.items():
        moved.k[0, new] = oc.k[0, old]
        moved.v[0, new] = oc.v[0, old]
    got = po.paged_decode_attention(case.query_f32, moved, [[remap[b] for b in case.tables[0]]], case.lengths)
    assert np.array_equal(base, got)


def test_attention_matches_torch_softmax_einsum():
    """The reference's own formula through torch (attention.py:30-36)."""
    case = _tiny_case(8, 2, seed=9, lengths=(29, 5, 17), head_dim=16)
    got = case.expected(scale=0.3)
    for b, (table, n) in enumerate(zip(case.tables, case.lengths)):
        k, v = case.oracle_cache.read(0, table, n)
        q = torch.from_numpy(case.query_f32[b : b + 1])
        kt = torch.from_numpy(k).repeat_interleave(4, dim=1).transpose(0, 1)
        vt = torch.from_numpy(v).repeat_interleave(4, dim=1).transpose(0, 1)
        probs = torch.softmax(torch.einsum("bhd,htd->bht", q, kt) * 0.3, dim=-1)
        ref = torch.einsum("bht,htd->bhd", probs, vt)[0].numpy()
        assert np.max(np.abs(got[b] - ref)) < 1e-6


def test_unwritten_nan_slots_never_leak():
    case = _tiny_case(4, 2, seed=11, lengths=(5, 6))  # tails of the last blocks are NaN
    assert np.isnan(case.oracle_cache.k).any()
    assert np.isfinite(case.expected()).all()


def test_planted_head_map_mistake_is_caught(monkeypatch):
    """A wrong query->kv head map (h % Hkv instead of h // group) fails the
    GQA-vs-expanded-MHA pin."""
    case = _tiny_case(8, 2, seed=3)

    def wrong_expand(x, num_heads):
        return np.tile(x, (1, num_heads // x.shape[1], 1))

    monkeypatch.setattr(po, "expand_kv", wrong_expand)
    gqa_wrong = case.expected()
    oc = case.oracle_cache
    mha = po.OracleCache(oc.num_blocks, oc.block_size, 8, oc.head_dim)
    mha.k[:] = np.repeat(oc.k, 4, axis=3)
    mha.v[:] = np.repeat(oc.v, 4, axis=3)
    monkeypatch.undo()
    ref = po.paged_decode_attention(case.query_f32, mha, case.tables, case.lengths)
    assert not np.allclose(gqa_wrong, ref, atol=1e-3)


def test_planted_scale_mistake_is_caught(monkeypatch):
    """Dropping the 1/sqrt(D) scale fails the float64 brute force."""
    case = _tiny_case(4, 4, seed=12)
    real = po.dense_decode_attention
    monkeypatch.setattr(po, "dense_decode_attention", lambda q, k, v, scale=None: real(q, k, v, scale=1.0))
    got = case.expected()
    monkeypatch.undo()
    k, v = case.oracle_cache.read(0, case.tables[0], case.lengths[0])
    ref = np.array(po.brute_force_attention_f64(case.query_f32[0].tolist(), k.tolist(), v.tolist()))
    assert np.max(np.abs(got[0] - ref)) > 1e-3


def test_bench_bytes_formula_matches_reference_kv_term():
    """Uniform lengths reduce bench.py's formula to benchmark.py:271-278's K+V estimate."""
    import bench

    b, ctx, hkv, d, eb = 4, 512, 8, 64, 4
    kv = 2 * b * ctx * hkv * d * eb
    total = bench.attention_bytes([ctx] * b, 32, hkv, d, eb, 16)
    assert kv == 8388608  # the 8.4 MB of the CPU fp32 batch-4 workload
    assert total == kv + 2 * b * 32 * d * eb + b * (ctx // 16) * 4 + b * 4
    assert math.isclose(total / kv, 1.0, rel_tol=0.01)


@pytest.mark.parametrize("batch,ctx", [(1, 128), (4, 512), (16, 2048), (3, 100)])
def test_bench_sweep_tables_follow_the_reference_allocation_order(batch, ctx):
    """The sweep's closed-form tables equal what the block allocator hands
    out in the reference's case construction (benchmark.py:85-95): one block
    per request per logical block, then one reserved block between rounds;
    the pool is exactly the blocks that allocation touches (e.g. 15 for
    batch 1 x 128 and 2175 for batch 16 x 2048, as the reference's A100
    records state)."""
    import bench
    from inferkernellab_amd.cache import BlockAllocator

    w = bench.build_sweep_case(batch, ctx, 8, torch.float16, torch.device("cpu"))
    need = -(-ctx // 16)
    alloc = BlockAllocator(w["pool"])
    tables = [[] for _ in range(batch)]
    for j in range(need):
        for r in range(batch):
            tables[r].extend(alloc.allocate(1, owner=r))
        if j + 1 < need:
            alloc.allocate(1, owner=-1)
    assert w["tables_list"] == tables
    assert alloc.num_free_blocks == 0
    assert {(1, 128): 15, (16, 2048): 2175}.get((batch, ctx), w["pool"]) == w["pool"]


def test_bench_fp8_prefill_reference_paths_agree(monkeypatch):
    """An FP8-cache prefill workload of the bench (E4M3 codes + row scales):
    its torch gather + masked SDPA over the dequantized cache and the oracle
    over the same dequantized cache agree within the bf16 bound, so either
    can check the kernel."""
    import bench

    monkeypatch.setitem(bench.PREFILL_WORKLOADS, "tiny_fp8", (2, 8, 2, 64, torch.bfloat16, 0, 64, "fp8"))
    w = bench.build_prefill_workload("tiny_fp8", torch.device("cpu"))
    assert w["fp8"] and w["cache"].k.dtype == torch.float8_e4m3fn
    sdpa = bench.torch_gather_sdpa(w).to(torch.bfloat16)
    check = bench.prefill_parity(w, sdpa, rows=16)
    assert check["passed"], check


def test_bench_sweep_covers_the_published_matrix():
    """Every one of the 54 sweep shapes has its published A100 timings."""
    import bench

    shapes = {(n, b, c, kv) for n, _ in bench.SWEEP_DTYPES for b in bench.SWEEP_BATCHES
              for c in bench.SWEEP_CONTEXTS for kv in bench.SWEEP_KV_HEADS}
    assert len(shapes) == 54 and shapes == set(bench.A100_SWEEP_US)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16", "float32"])
def test_rope_rows_match_torch_ops_bit_for_bit(dtype):
    """rope_rows against torch's elementwise sequence of hf_benchmark.py:69-85
    (x * cos + rotate_half(x) * sin in the tensor dtype)."""
    gen = torch.Generator().manual_seed(11)
    tdt = getattr(torch, dtype)
    x = torch.randn(7, 4, 64, generator=gen).to(tdt)
    ang = torch.rand(7, 32, generator=gen) * 50
    emb = torch.cat([ang, ang], dim=-1)
    cos, sin = emb.cos().to(tdt), emb.sin().to(tdt)

    def rot(v):
        return torch.cat((-v[..., 32:], v[..., :32]), dim=-1)

    want = x * cos[:, None, :] + rot(x) * sin[:, None, :]

    def storage(t):
        return t.view(torch.int16).numpy().view(np.uint16) if t.dtype == torch.bfloat16 else t.numpy()

    got = po.rope_rows(storage(x), storage(cos)[:, None, :], storage(sin)[:, None, :], dtype)
    assert np.array_equal(got.view(np.uint8), storage(want).view(np.uint8))
    ones, zeros = torch.ones(7, 64).to(tdt), torch.zeros(7, 64).to(tdt)
    ident = po.rope_rows(storage(x), storage(ones)[:, None, :], storage(zeros)[:, None, :], dtype)
    assert np.array_equal(ident.view(np.uint8), storage(x).view(np.uint8))


def test_planted_rope_sign_mistake_is_caught(monkeypatch):
    gen = torch.Generator().manual_seed(12)
    x = torch.randn(3, 2, 16, generator=gen)
    emb = torch.rand(3, 16, generator=gen)
    cos, sin = emb.cos(), emb.sin()
    want = x * cos[:, None] + torch.cat((-x[..., 8:], x[..., :8]), -1) * sin[:, None]
    real = po.rope_rows

    def wrong(xs, c, s, dtype):  # the sin term's sign flipped
        return real(xs, c, -s, dtype)

    monkeypatch.setattr(po, "rope_rows", wrong)
    got = po.rope_rows(x.numpy(), cos.numpy()[:, None], sin.numpy()[:, None], "float32")
    assert np.abs(got - want.numpy()).max() > 1e-3
