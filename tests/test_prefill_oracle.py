"""Pins of the oracle's paged prefill attention (attention.py:230-321).

The decode attention of the oracle is pinned independently (test_oracle.py);
here every attending prefill row must equal it over the row's own prefix —
the check of the reference's own prefill test (tests/test_attention.py:90-116,
same tables and ranges) — and the whole result, padding rows included, must
match a float64 brute force and torch SDPA under the reference's mask
construction. A planted off-by-one in the causal mask must be caught."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import paged_oracle as po
from tests.helpers import make_prefill_case


def _reference_case(dtype="float32", seed=11):
    """The reference test's geometry: 24 blocks of 4 tokens, 2 KV heads of
    dim 8, 4 query heads, tables [[17, 3, 12], [5, 21, 8]], chunks [0, 5) and
    [2, 7), query width 5."""
    rng = np.random.default_rng(seed)
    oc = po.OracleCache(24, 4, 2, 8, dtype=dtype, fill=np.nan)
    tables = [[17, 3, 12], [5, 21, 8]]
    starts, ends = [0, 2], [5, 7]
    for table, end in zip(tables, ends):
        k = rng.standard_normal((end, 2, 8)).astype(np.float32)
        v = rng.standard_normal((end, 2, 8)).astype(np.float32)
        oc.write(0, table, 0, k.astype(po.storage_dtype(dtype)), v.astype(po.storage_dtype(dtype)))
    query = rng.standard_normal((2, 4, 5, 8)).astype(np.float32)
    return oc, tables, starts, ends, query


def _rows_equal_decode_over_prefix(out, q, oc, tables, starts, ends, atol):
    for b, (table, s, e) in enumerate(zip(tables, starts, ends)):
        for t in range(e - s):
            dec = po.paged_decode_attention(q[b, :, t][None], oc, [table], [s + t + 1])[0]
            if not np.allclose(out[b, :, t], dec, atol=atol, rtol=atol):
                return False
    return True


def test_prefill_rows_equal_decode_over_their_prefix_reference_case():
    oc, tables, starts, ends, q = _reference_case()
    out = po.paged_prefill_attention(q, oc, tables, starts, ends)
    assert _rows_equal_decode_over_prefix(out, q, oc, tables, starts, ends, atol=1e-5)


@pytest.mark.parametrize("num_heads,num_kv,dtype", [(4, 4, "float32"), (4, 2, "bfloat16"), (8, 1, "float16")])
def test_prefill_rows_equal_decode_random_ragged(num_heads, num_kv, dtype):
    case = make_prefill_case(starts=[0, 5, 17], ends=[9, 12, 40], width=24, num_heads=num_heads,
                             num_kv_heads=num_kv, head_dim=16, block_size=8, dtype=dtype, seed=3,
                             table_slack=1)
    out = case.expected()
    assert not np.isnan(out).any()
    assert _rows_equal_decode_over_prefix(out, case.query_f32, case.base.oracle_cache, case.base.tables,
                                          case.starts, case.ends, atol=1e-5)


def test_prefill_matches_float64_brute_force():
    case = make_prefill_case(starts=[3, 0], ends=[9, 4], width=6, num_heads=4, num_kv_heads=2, head_dim=8,
                             block_size=4, dtype="bfloat16", seed=5)
    out = case.expected()
    oc = case.base.oracle_cache
    for b, (table, s, e) in enumerate(zip(case.base.tables, case.starts, case.ends)):
        k, v = oc.read(0, table, e)
        k, v = po.to_f32(k, "bfloat16").tolist(), po.to_f32(v, "bfloat16").tolist()
        ref = np.array(po.brute_force_prefill_f64(case.query_f32[b, :, : e - s].tolist(), k, v, s))
        assert np.max(np.abs(out[b, :, : e - s] - ref)) < 2e-6


def test_prefill_matches_torch_sdpa_with_the_reference_mask():
    """Gather + mask construction of attention.py:289-321 restated in torch
    (fp32 SDPA on the CPU); padding rows included."""
    case = make_prefill_case(starts=[0, 6, 2], ends=[7, 10, 10], width=8, num_heads=6, num_kv_heads=3,
                             head_dim=16, block_size=4, dtype="float32", seed=9)
    oc = case.base.oracle_cache
    batch, heads, width, dim = case.query.shape
    bs = oc.block_size
    span = max(case.ends)
    kpos = torch.arange(span)
    table = torch.tensor([t + [0] * (-(-span // bs) - len(t)) for t in case.base.tables])
    phys = table[:, kpos // bs]
    key = torch.from_numpy(oc.k[0])[phys, (kpos % bs).unsqueeze(0)]  # [B, L, Hkv, D]
    value = torch.from_numpy(oc.v[0])[phys, (kpos % bs).unsqueeze(0)]
    lengths = torch.tensor(case.ends).view(-1, 1, 1)
    starts = torch.tensor(case.starts).view(-1, 1, 1)
    key_ok = kpos.view(1, 1, -1) < lengths
    valid = key_ok.squeeze(1).unsqueeze(-1).unsqueeze(-1)
    key = key.masked_fill(~valid, 0)
    value = value.masked_fill(~valid, 0)
    qpos = torch.arange(width)
    valid_query = qpos.view(1, -1, 1) < (lengths - starts).view(-1, 1, 1)
    causal = kpos.view(1, 1, -1) <= starts + qpos.view(1, -1, 1)
    allow = (valid_query & key_ok & causal) | ((~valid_query) & (kpos.view(1, 1, -1) == 0))
    rep = heads // oc.num_kv_heads
    k = key.permute(0, 2, 1, 3).repeat_interleave(rep, dim=1)
    v = value.permute(0, 2, 1, 3).repeat_interleave(rep, dim=1)
    ref = F.scaled_dot_product_attention(torch.from_numpy(case.query_f32), k, v, attn_mask=allow.unsqueeze(1))
    assert np.max(np.abs(case.expected() - ref.numpy())) < 2e-6


def test_prefill_padding_rows_take_the_value_at_position_zero():
    case = make_prefill_case(starts=[4, 1], ends=[6, 9], width=8, num_heads=2, num_kv_heads=1, head_dim=8,
                             block_size=4, dtype="float16", seed=2)
    out = case.expected()
    oc = case.base.oracle_cache
    for b, (table, s, e) in enumerate(zip(case.base.tables, case.starts, case.ends)):
        _, v = oc.read(0, table, 1)
        v0 = po.to_f32(v, "float16")[0, 0]
        assert np.array_equal(out[b, :, e - s :], np.broadcast_to(v0, out[b, :, e - s :].shape))


def test_prefill_scale_argument_is_the_softmax_scale():
    case = make_prefill_case(starts=[0], ends=[5], num_heads=2, num_kv_heads=2, head_dim=8, block_size=4,
                             dtype="float32", seed=4)
    oc = case.base.oracle_cache
    k, v = oc.read(0, case.base.tables[0], 5)
    ref = np.array(po.brute_force_prefill_f64(case.query_f32[0].tolist(), k.tolist(), v.tolist(), 0, scale=0.3))
    assert np.max(np.abs(case.expected(scale=0.3)[0] - ref)) < 2e-6


def test_planted_causal_off_by_one_is_caught(monkeypatch):
    """A strict causal mask (keys < position) fails the row == decode pin."""
    oc, tables, starts, ends, q = _reference_case(seed=3)
    monkeypatch.setattr(po, "causal_allow", lambda pos, n: np.arange(n)[None, :] < np.asarray(pos)[:, None])
    with np.errstate(invalid="ignore"):
        wrong = po.paged_prefill_attention(q, oc, tables, starts, ends)
    monkeypatch.undo()
    assert not _rows_equal_decode_over_prefix(wrong, q, oc, tables, starts, ends, atol=1e-5)


@pytest.mark.parametrize(
    "starts,ends,width,message",
    [
        ([0], [5, 7], 5, "one entry per query batch"),
        ([0, -1], [5, 7], 8, "non-empty and non-negative"),
        ([0, 7], [5, 7], 8, "non-empty and non-negative"),
        ([0, 0], [5, 7], 5, "query width is smaller"),
    ],
)
def test_prefill_oracle_rejects_like_the_reference(starts, ends, width, message):
    oc, tables, _, _, _ = _reference_case()
    q = np.zeros((2, 4, width, 8), dtype=np.float32)
    with pytest.raises(ValueError, match=message):
        po.paged_prefill_attention(q, oc, tables, starts, ends)
