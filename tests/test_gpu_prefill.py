"""GPU parity of the paged prefill attention kernels against the oracle's
restatement of attention.py:230-321 (tolerances: max-abs 2e-3 fp16, 1e-2
bf16, 1e-4 fp32 against the fp32 oracle).

Covered: the reference test's own geometry (fp32), the MFMA family over
head_dim {32, 64, 96, 128}, MHA / GQA / MQA and a non-power-of-two group,
block sizes 16 / 32 / 48, chunked prefill (chunks starting past 0), padding
rows, positions past the chunk end poisoned with NaN, strided query/output
views, the VALU family forced on the same inputs, a long GQA chunk, and
table entries outside the cache (their keys are dropped, as in the decode
kernels)."""

import numpy as np
import pytest
import torch

from tests.helpers import ATOL, make_prefill_case, max_abs_err

pytestmark = pytest.mark.gpu


def _run(case, *, path=None, scale=None, query=None, out=None, layer=0, table_dtype=torch.int32):
    from inferkernellab_amd import PreparedPagedPrefill

    cache = case.base.device_cache()
    tables = case.base.device_tables(dtype=table_dtype)
    q = case.device_query() if query is None else query
    prep = PreparedPagedPrefill(cache, tables, case.starts, case.ends, num_heads=q.shape[1],
                                query_width=q.shape[2], scale=scale, path=path)
    res = prep(q, layer, out=out)
    torch.cuda.synchronize()
    return res, prep


def _err(actual, expected):
    a = actual.detach().float().cpu().numpy()
    assert not np.isnan(a).any(), "NaN in the kernel output"
    return max_abs_err(actual, expected)


def test_reference_case_fp32():
    """tests/test_attention.py:90-116: tables [[17, 3, 12], [5, 21, 8]],
    chunks [0, 5) and [2, 7), width 5, 4 heads over 2 KV heads of dim 8."""
    from inferkernellab_amd import PagedKVCache, paged_prefill_attention_hip
    from oracle import paged_oracle as po

    rng = np.random.default_rng(11)
    oc = po.OracleCache(24, 4, 2, 8, dtype="float32", fill=np.nan)
    tables, starts, ends = [[17, 3, 12], [5, 21, 8]], [0, 2], [5, 7]
    for table, end in zip(tables, ends):
        k = rng.standard_normal((end, 2, 8)).astype(np.float32)
        v = rng.standard_normal((end, 2, 8)).astype(np.float32)
        oc.write(0, table, 0, k, v)
    q = rng.standard_normal((2, 4, 5, 8)).astype(np.float32)
    cache = PagedKVCache(24, 4, 2, 8, dtype=torch.float32, device="cuda")
    cache.k.copy_(torch.from_numpy(oc.k))
    cache.v.copy_(torch.from_numpy(oc.v))
    got = paged_prefill_attention_hip(torch.from_numpy(q).cuda(), cache, tables, starts, ends)
    expected = po.paged_prefill_attention(q, oc, tables, starts, ends)
    assert _err(got, expected) < 1e-5


MFMA_CASES = [
    # (heads, kv_heads, head_dim, block_size, starts, ends, width)
    (32, 8, 128, 16, [0, 40, 300], [77, 200, 420], 160),
    (16, 4, 128, 16, [0, 0, 0, 0], [512, 300, 129, 1], 512),
    (8, 8, 64, 32, [5, 0], [70, 33], 80),
    (32, 1, 64, 16, [0, 17], [40, 90], 73),
    (12, 4, 96, 48, [0, 100], [150, 260], 160),
    (8, 2, 32, 16, [3, 0, 60], [20, 1, 64], 24),
]


@pytest.mark.parametrize("dtype", ["bfloat16", "float16"])
@pytest.mark.parametrize("heads,kv,dim,bs,starts,ends,width", MFMA_CASES)
def test_mfma_prefill_matches_oracle(dtype, heads, kv, dim, bs, starts, ends, width):
    case = make_prefill_case(starts=starts, ends=ends, width=width, num_heads=heads, num_kv_heads=kv,
                             head_dim=dim, block_size=bs, dtype=dtype, seed=heads + dim + bs, table_slack=1)
    got, prep = _run(case)
    assert prep.path == "mfma_grouped"
    assert _err(got, case.expected()) < ATOL[dtype]


@pytest.mark.parametrize("dtype", ["bfloat16", "float16", "float32"])
def test_scalar_prefill_matches_oracle(dtype):
    case = make_prefill_case(starts=[0, 9, 2], ends=[33, 30, 70], width=68, num_heads=8, num_kv_heads=2,
                             head_dim=64, block_size=16, dtype=dtype, seed=21, table_slack=1)
    got, prep = _run(case, path="scalar_grouped")
    assert prep.path == "scalar_grouped"
    assert _err(got, case.expected()) < ATOL[dtype]


@pytest.mark.parametrize("dim,bs,dtype", [(256, 8, "float32"), (80, 4, "bfloat16"), (128, 24, "float16"),
                                          (16, 16, "float16")])
def test_scalar_family_covers_other_shapes(dim, bs, dtype):
    case = make_prefill_case(starts=[0, 4], ends=[21, 30], width=26, num_heads=4, num_kv_heads=2,
                             head_dim=dim, block_size=bs, dtype=dtype, seed=dim + bs)
    got, prep = _run(case)
    assert prep.path == "scalar_grouped"
    assert _err(got, case.expected()) < ATOL[dtype]


def test_mfma_and_scalar_agree_on_the_same_inputs():
    case = make_prefill_case(starts=[0, 31], ends=[97, 160], width=129, num_heads=16, num_kv_heads=4,
                             head_dim=128, block_size=16, dtype="bfloat16", seed=8)
    mfma, _ = _run(case)
    scalar, _ = _run(case, path="scalar_grouped")
    expected = case.expected()
    assert _err(mfma, expected) < ATOL["bfloat16"]
    assert _err(scalar, expected) < ATOL["bfloat16"]


def test_scale_argument():
    case = make_prefill_case(starts=[0, 3], ends=[50, 45], width=50, num_heads=8, num_kv_heads=2,
                             head_dim=64, block_size=16, dtype="float16", seed=30)
    got, _ = _run(case, scale=0.05)
    assert _err(got, case.expected(scale=0.05)) < ATOL["float16"]


def test_strided_query_and_output_views():
    """query / out as [B, T, H, D] buffers viewed as [B, H, T, D] (the layout
    the projections produce), int64 tables, second layer."""
    case = make_prefill_case(starts=[0, 8], ends=[40, 50], width=42, num_heads=16, num_kv_heads=4,
                             head_dim=128, block_size=16, dtype="bfloat16", seed=12, num_layers=2, layer=1)
    q_bhtd = case.device_query()
    q_bthd = q_bhtd.transpose(1, 2).contiguous()
    out_bthd = torch.full_like(q_bthd, float("nan"))
    got, _ = _run(case, query=q_bthd.transpose(1, 2), out=out_bthd.transpose(1, 2), layer=1,
                  table_dtype=torch.int64)
    assert got.data_ptr() == out_bthd.data_ptr()
    assert _err(out_bthd.transpose(1, 2), case.expected(layer=1)) < ATOL["bfloat16"]


def test_padding_rows_equal_position_zero_value_exactly():
    case = make_prefill_case(starts=[5, 0], ends=[9, 3], width=40, num_heads=8, num_kv_heads=2, head_dim=128,
                             block_size=16, dtype="bfloat16", seed=4)
    got, _ = _run(case)
    exp = case.expected()
    for b, (s, e) in enumerate(zip(case.starts, case.ends)):
        pad = got[b, :, e - s :].float().cpu().numpy()
        assert np.array_equal(pad, exp[b, :, e - s :])


def test_long_chunked_prefill_gqa():
    """A 1024-token chunk appended after a 1024-token prefix, next to a
    1024-token prompt (GQA 32/8, head_dim 128, bf16)."""
    case = make_prefill_case(starts=[1024, 0], ends=[2048, 1024], width=1024, num_heads=32, num_kv_heads=8,
                             head_dim=128, block_size=16, dtype="bfloat16", seed=77)
    got, _ = _run(case)
    assert _err(got, case.expected()) < ATOL["bfloat16"]


def test_reference_validation_messages_on_gpu():
    from inferkernellab_amd import PagedKVCache, paged_prefill_attention_hip

    cache = PagedKVCache(8, 16, 2, 64, dtype=torch.bfloat16, device="cuda")
    q = torch.zeros(1, 4, 8, 64, dtype=torch.bfloat16, device="cuda")
    wide = torch.zeros(1, 4, 32, 64, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(ValueError, match="context length exceeds block table capacity"):
        paged_prefill_attention_hip(wide, cache, [[0]], [0], [17])
    with pytest.raises(ValueError, match="query width is smaller than a prefill range"):
        paged_prefill_attention_hip(q, cache, [[0, 1]], [0], [9])
    with pytest.raises(ValueError, match="query and cache must have the same dtype"):
        paged_prefill_attention_hip(q.float(), cache, [[0]], [0], [8])


def _expected_dropping_blocks(case, dropped, scale=None):
    """The oracle's prefill attention with the keys of the logical blocks in
    dropped[b] removed from every row of request b (no row loses all of its
    keys here: block 0 stays)."""
    from oracle import paged_oracle as po

    oc = case.base.oracle_cache
    q = case.query_f32
    _, heads, _, dim = q.shape
    sc = np.float32(scale if scale is not None else dim ** -0.5)
    out = np.empty_like(q)
    for b, (s, e) in enumerate(zip(case.starts, case.ends)):
        k_raw, v_raw = oc.read(0, case.base.tables[b], e)
        k = po.expand_kv(po.to_f32(k_raw, oc.dtype), heads).transpose(1, 0, 2)
        v = po.expand_kv(po.to_f32(v_raw, oc.dtype), heads).transpose(1, 0, 2)
        keep = np.array([pos // oc.block_size not in dropped[b] for pos in range(e)])
        n = e - s
        allow = po.causal_allow(s + np.arange(n), e) & keep[None]
        scores = np.where(allow[None], np.matmul(q[b, :, :n], k.transpose(0, 2, 1)) * sc, -np.inf)
        scores = (scores - scores.max(axis=-1, keepdims=True)).astype(np.float32)
        probs = np.exp(scores)
        probs /= probs.sum(axis=-1, keepdims=True)
        out[b, :, :n] = np.matmul(probs, v)
        out[b, :, n:] = v[:, :1, :]
    return out


@pytest.mark.parametrize("heads,kv,dim,bs,starts,ends,dropped,dtype,path", [
    # a hole past the first 1024 keys (the kernel's table window moves there)
    (16, 4, 128, 16, [0, 40], [300, 1500], [{1, 5}, {3, 70}], "bfloat16", None),
    (8, 2, 64, 48, [0, 10], [200, 130], [{1}, {2}], "float16", None),
    (8, 2, 64, 16, [0, 10], [200, 130], [{1, 2}, {4}], "float16", "scalar_grouped"),
])
def test_table_entries_outside_the_cache_are_dropped(heads, kv, dim, bs, starts, ends, dropped, dtype, path):
    from inferkernellab_amd import PreparedPagedPrefill

    case = make_prefill_case(starts=starts, ends=ends, num_heads=heads, num_kv_heads=kv, head_dim=dim,
                             block_size=bs, dtype=dtype, seed=dim + bs + 3)
    nb = case.base.oracle_cache.num_blocks
    width = max(len(t) for t in case.base.tables)
    rows = []
    for b, table in enumerate(case.base.tables):
        row = list(table) + [0] * (width - len(table))
        for i, lb in enumerate(sorted(dropped[b])):
            row[lb] = -1 if i % 2 == 0 else nb + 5  # negative and past-the-end ids
        rows.append(row)
    tables = torch.tensor(rows, dtype=torch.int32, device="cuda")
    q = case.device_query()
    prep = PreparedPagedPrefill(case.base.device_cache(), tables, starts, ends, num_heads=heads,
                                query_width=q.shape[2], path=path)
    got = prep(q, 0)
    torch.cuda.synchronize()
    assert prep.path == (path or "mfma_grouped")
    assert _err(got, _expected_dropping_blocks(case, dropped)) < ATOL[dtype]


@pytest.mark.parametrize("dtype,path", [("bfloat16", None), ("float16", None), ("float32", None),
                                        ("bfloat16", "scalar_grouped")])
def test_nan_key_inside_the_context_propagates_like_the_reference(dtype, path):
    """A NaN in one key row inside the prefix makes the query rows that
    attend it NaN (rows at or past its position, for the query heads of its
    KV head), and only those, as the reference's causal SDPA does
    (attention.py:230-321: a NaN score under a boolean mask is kept for
    allowed positions and masked out for the others). The MFMA prefill is
    built without NaN semantics for its own arithmetic (it produces no NaN
    of its own); a NaN from the cache still reaches the row sum and the PV
    product, so the output row is NaN."""
    heads, kv, dim, bs = 16, 4, 64, 16
    starts, ends = [0, 40, 10], [77, 200, 90]
    case = make_prefill_case(starts=starts, ends=ends, width=160, num_heads=heads, num_kv_heads=kv,
                             head_dim=dim, block_size=bs, dtype=dtype, seed=33)
    oc = case.base.oracle_cache
    nan = np.uint16(0x7FC0) if dtype == "bfloat16" else np.nan
    # request 1: a key inside its chunk (position 50) and request 2: one in
    # the prefix before its chunk (position 4)
    for b, pos, h in ((1, 50, 1), (2, 4, 3)):
        slot = oc.slot_mapping(case.base.tables[b], pos, 1)[0]
        oc.k[0, slot // bs, slot % bs, h, 7] = nan
    print(f"prefill nan-key case dtype={dtype} path={path}", flush=True)
    got, prep = _run(case, path=path)
    out = got.float().cpu().numpy()
    expected = case.expected()
    nan_rows = np.isnan(expected)
    assert np.array_equal(np.isnan(out), nan_rows)
    per_kv = heads // kv
    # request 1, heads of kv head 1: rows of positions >= 50 (t >= 10) are NaN, earlier rows finite
    assert nan_rows[1, per_kv:2 * per_kv, 10:ends[1] - starts[1]].all()
    assert not nan_rows[1, per_kv:2 * per_kv, :10].any()
    # request 2, heads of kv head 3: every row of the chunk attends position 4
    assert nan_rows[2, 3 * per_kv:4 * per_kv, :ends[2] - starts[2]].all()
    finite = ~nan_rows
    assert np.abs(out[finite] - expected[finite]).max() <= ATOL[dtype]
