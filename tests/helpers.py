"""Shared builders for the parity tests: seeded inputs written into the
oracle cache, then copied bit for bit into the product's device cache."""

from __future__ import annotations

import json
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np
import torch

from oracle import paged_oracle as po

GOLDEN = Path(__file__).resolve().parent / "golden"

TORCH_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float32": torch.float32}
# Tolerances stated for this path: max-abs vs the fp32 oracle.
ATOL = {"float16": 2e-3, "bfloat16": 1e-2, "float32": 1e-4}


def known_answers() -> dict:
    return json.loads((GOLDEN / "known_answers.json").read_text())


def storage_to_torch(arr: np.ndarray, dtype: str) -> torch.Tensor:
    """numpy storage (bf16 as uint16 bits) -> torch tensor of `dtype`, same bits."""
    arr = np.ascontiguousarray(arr)
    if dtype == "bfloat16":
        return torch.from_numpy(arr.view(np.int16)).view(torch.bfloat16)
    return torch.from_numpy(arr)


def torch_to_storage(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def randn_storage(gen: torch.Generator, shape, dtype: str, scale: float = 1.0) -> np.ndarray:
    x = torch.randn(shape, generator=gen, dtype=torch.float32) * scale
    return torch_to_storage(x.to(TORCH_DTYPES[dtype]))


@dataclass
class Case:
    dtype: str
    oracle_cache: po.OracleCache
    query: np.ndarray  # storage
    tables: list[list[int]]
    lengths: list[int]
    num_heads: int

    @property
    def query_f32(self) -> np.ndarray:
        return po.to_f32(self.query, self.dtype)

    def expected(self, scale=None, layer=0) -> np.ndarray:
        return po.paged_decode_attention(
            self.query_f32, self.oracle_cache, self.tables, self.lengths, scale=scale, layer=layer
        )

    def device_cache(self, device="cuda"):
        from inferkernellab_amd.cache import PagedKVCache

        oc = self.oracle_cache
        cache = PagedKVCache(
            oc.num_blocks,
            oc.block_size,
            oc.num_kv_heads,
            oc.head_dim,
            num_layers=oc.num_layers,
            dtype=TORCH_DTYPES[self.dtype],
            device=device,
        )
        cache.k.copy_(storage_to_torch(oc.k, self.dtype))
        cache.v.copy_(storage_to_torch(oc.v, self.dtype))
        return cache

    def device_query(self, device="cuda") -> torch.Tensor:
        return storage_to_torch(self.query, self.dtype).to(device)

    def device_tables(self, device="cuda", dtype=torch.int32) -> torch.Tensor:
        width = max(len(t) for t in self.tables)
        padded = [list(t) + [0] * (width - len(t)) for t in self.tables]
        return torch.tensor(padded, dtype=dtype, device=device)

    def device_lengths(self, device="cuda", dtype=torch.int32) -> torch.Tensor:
        return torch.tensor(self.lengths, dtype=dtype, device=device)


def make_case(
    *,
    batch: int,
    num_heads: int,
    num_kv_heads: int,
    head_dim: int,
    block_size: int,
    lengths,
    dtype: str,
    seed: int = 0,
    num_blocks: int | None = None,
    num_layers: int = 1,
    layer: int = 0,
    kv_scale: float = 1.0,
    poison=np.nan,
) -> Case:
    """Random permutation block tables drawn from a pool; K/V ~ N(0,1)*kv_scale
    written through slot_mapping; unwritten slots hold `poison`."""
    lengths = [int(x) for x in lengths]
    assert len(lengths) == batch
    need = [-(-n // block_size) for n in lengths]
    pool = num_blocks if num_blocks is not None else sum(need) + 8
    gen = torch.Generator().manual_seed(seed)
    perm = torch.randperm(pool, generator=gen).tolist()
    tables, used = [], 0
    for n in need:
        tables.append(perm[used : used + n])
        used += n
    cache = po.OracleCache(pool, block_size, num_kv_heads, head_dim, num_layers=num_layers,
                           dtype=dtype, fill=poison)
    for table, n in zip(tables, lengths):
        key = randn_storage(gen, (n, num_kv_heads, head_dim), dtype, kv_scale)
        value = randn_storage(gen, (n, num_kv_heads, head_dim), dtype, kv_scale)
        slots = cache.slot_mapping(table, 0, n)
        cache.write_slots(layer, slots, key, value)
    query = randn_storage(gen, (batch, num_heads, head_dim), dtype)
    return Case(dtype, cache, query, tables, lengths, num_heads)


# Every parity check of the session, for the summary tests/conftest.py prints
# at the end of the run: (test id, dtype, strict max-abs error, tolerance,
# elements that took the output-rounding allowance, largest error among them).
PARITY_LOG: list[tuple[str, str, float, float, int, float]] = []

_DTYPE_NAMES = {torch.float16: "float16", torch.bfloat16: "bfloat16", torch.float32: "float32"}


def _current_test() -> str:
    return os.environ.get("PYTEST_CURRENT_TEST", "?").rsplit(" (", 1)[0]


def record_parity(dtype: str, err: float, tol: float, allowed: int = 0, allowed_err: float = 0.0) -> None:
    PARITY_LOG.append((_current_test(), dtype, float(err), float(tol), int(allowed), float(allowed_err)))


def max_abs_err(actual, expected: np.ndarray, dtype: str | None = None) -> float:
    """Strict max-abs error of a kernel output (a tensor, or its fp32 numpy
    copy with the output's `dtype` name) against the oracle, recorded for
    the end-of-run parity summary."""
    if isinstance(actual, torch.Tensor):
        dtype = dtype or _DTYPE_NAMES.get(actual.dtype, str(actual.dtype))
        actual = actual.detach().float().cpu().numpy()
    assert dtype is not None, "a numpy output needs its dtype name"
    err = float(np.max(np.abs(actual - expected))) if actual.size else 0.0
    record_parity(dtype, err, ATOL.get(dtype, float("nan")))
    return err


def assert_close_up_to_output_rounding(out: torch.Tensor, expected: np.ndarray, dtype: str) -> None:
    """|out - expected| <= ATOL everywhere, except where half an ulp of the
    output dtype at |expected| exceeds half of ATOL (bf16 |x| >= 2, fp16
    |x| >= 4): there the bound is ATOL + that half ulp.

    Half a bf16 ulp at |x| in [4, 8) is 2^-7 ~ 7.8e-3, most of the 1e-2
    budget: the rounding of the output itself, which every bf16-output
    kernel (the reference's `.to(q.dtype)` included) incurs, so elements of
    that size get it on top. Everywhere else the stated max-abs is strict.
    The strict max-abs over all elements is recorded for the summary."""
    got = out.detach().float().cpu().numpy()
    assert not np.isnan(got).any(), "NaN in the kernel output"
    bits = {"bfloat16": 8, "float16": 11, "float32": 24}[dtype]  # significand bits
    _, e = np.frexp(np.abs(expected).astype(np.float64))
    half_ulp = np.ldexp(1.0, e - bits - 1)
    allowance = np.where(half_ulp > ATOL[dtype] / 2, half_ulp, 0.0)
    err = np.abs(got - expected)
    excess = err - (ATOL[dtype] + allowance)
    took = allowance > 0
    record_parity(dtype, float(err.max()) if err.size else 0.0, ATOL[dtype], int(took.sum()),
                  float(err[took].max()) if took.any() else 0.0)
    strict = err[~took]
    assert excess.max() <= 0, (f"max excess {excess.max()} (max abs err {err.max()}, "
                               f"{strict.max() if strict.size else 0.0} where the bound is strict)")


@dataclass
class PrefillCase:
    """A ragged prompt-chunk batch: request b's chunk covers positions
    [starts[b], ends[b]) of a context already written up to ends[b]."""

    base: Case
    query: np.ndarray  # storage [B, H, T, D]
    starts: list[int]
    ends: list[int]

    @property
    def dtype(self) -> str:
        return self.base.dtype

    @property
    def query_f32(self) -> np.ndarray:
        return po.to_f32(self.query, self.dtype)

    def expected(self, scale=None, layer=0) -> np.ndarray:
        return po.paged_prefill_attention(self.query_f32, self.base.oracle_cache, self.base.tables,
                                          self.starts, self.ends, scale=scale, layer=layer)

    def device_query(self, device="cuda") -> torch.Tensor:
        return storage_to_torch(self.query, self.dtype).to(device)


def make_prefill_case(*, starts, ends, width: int | None = None, num_heads: int, num_kv_heads: int,
                      head_dim: int, block_size: int, dtype: str, seed: int = 0, num_layers: int = 1,
                      layer: int = 0, table_slack: int = 0) -> PrefillCase:
    """make_case() with context lengths `ends`, plus a seeded [B, H, T, D]
    query whose width T defaults to the longest chunk. `table_slack` extra
    blocks of context room are allocated per request (unwritten, NaN)."""
    ends = [int(e) for e in ends]
    starts = [int(s) for s in starts]
    base = make_case(batch=len(ends), num_heads=num_heads, num_kv_heads=num_kv_heads, head_dim=head_dim,
                     block_size=block_size, lengths=[e + table_slack * block_size for e in ends],
                     dtype=dtype, seed=seed, num_layers=num_layers, layer=layer)
    # positions past ends[b] stay mapped by the table but must never be
    # attended: poison them with NaN
    oc = base.oracle_cache
    nan = np.uint16(0x7FC0) if dtype == "bfloat16" else np.nan
    for table, e in zip(base.tables, ends):
        total = len(table) * block_size
        if total > e:
            slots = oc.slot_mapping(table, e, total - e)
            oc.k[layer, slots // block_size, slots % block_size] = nan
            oc.v[layer, slots // block_size, slots % block_size] = nan
    base.lengths = ends
    width = width or max(e - s for s, e in zip(starts, ends))
    gen = torch.Generator().manual_seed(seed + 7919)
    query = randn_storage(gen, (len(ends), num_heads, width, head_dim), dtype)
    return PrefillCase(base, query, starts, ends)
