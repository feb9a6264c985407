"""Paged KV storage with the reference's layout and addressing.

Mirrors ``cache.py`` of the reference (CacheLayout 8-14, BlockAllocator
17-64, PagedKVCache 67-200): storage is ``[layer, block, token-in-block,
kv-head, head-dim]`` per K and V, a request owns a list of physical block
ids (its block table), and token position ``p`` of a request lives at slot
``table[p // block_size] * block_size + p % block_size``. Validation rules
and error messages follow the reference so callers see the same failures.

The torch scatter/gather methods (``write``, ``write_slots``, ``read``) are
the reference's ``append_backend="torch"`` path and its gather; the HIP
append lives in :mod:`inferkernellab_amd.ops`.

``dtype=torch.float8_e4m3fn`` selects the FP8 KV format (no counterpart in
the reference): ``k`` / ``v`` hold OCP E4M3 codes and ``k_scale`` /
``v_scale`` ``[layers, blocks, kv_heads, block_size]`` one power-of-two
fp32 scale per (token, KV head) row; ``act_dtype`` (default bfloat16) is the type of the
rows written into it and of the queries that attend it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

FP8_E4M3 = torch.float8_e4m3fn
E4M3_MAX = 448.0


@dataclass(frozen=True)
class CacheLayout:
    num_layers: int
    num_blocks: int
    block_size: int
    num_kv_heads: int
    head_dim: int


class BlockAllocator:
    """Deterministic physical-block allocator (cache.py:17-64).

    Free ids are kept in a stack initialised high-to-low, so fresh allocations
    come out in ascending order. ``free`` validates the whole request before
    mutating anything.
    """

    def __init__(self, num_blocks: int):
        if num_blocks <= 0:
            raise ValueError("num_blocks must be positive")
        self._capacity = num_blocks
        self._free_stack: list[int] = list(reversed(range(num_blocks)))
        self._in_use: set[int] = set()
        self._owner_of: dict[int, int] = {}

    @property
    def num_free_blocks(self) -> int:
        return len(self._free_stack)

    @property
    def num_used_blocks(self) -> int:
        return len(self._in_use)

    def allocate(self, count: int, owner: int | None = None) -> list[int]:
        if count < 0:
            raise ValueError("count must be non-negative")
        if count > len(self._free_stack):
            raise RuntimeError(
                f"out of KV blocks: requested={count}, free={len(self._free_stack)}"
            )
        taken = [self._free_stack.pop() for _ in range(count)]
        self._in_use.update(taken)
        if owner is not None:
            self._owner_of.update((block, owner) for block in taken)
        return taken

    def free(self, block_ids, owner: int | None = None) -> None:
        ids = tuple(block_ids)
        if len(set(ids)) != len(ids):
            raise ValueError("block_ids must not contain duplicates")
        for block in ids:
            if not isinstance(block, int) or not 0 <= block < self._capacity:
                raise ValueError(f"invalid block id: {block}")
            if block not in self._in_use:
                raise ValueError(f"block {block} is not allocated")
            if owner is not None and self._owner_of.get(block) != owner:
                raise ValueError(f"block {block} is not owned by request {owner}")
        for block in ids:
            self._in_use.discard(block)
            self._owner_of.pop(block, None)
            self._free_stack.append(block)

    def owner(self, block_id: int) -> int | None:
        return self._owner_of.get(block_id)


class PagedKVCache:
    """K/V storage ``[layers, blocks, block_size, kv_heads, head_dim]``.

    Tensors are allocated uninitialised (``torch.empty``) like the reference
    (cache.py:90-92); unread slots may hold anything, including NaN.
    """

    def __init__(
        self,
        num_blocks: int,
        block_size: int,
        num_kv_heads: int,
        head_dim: int,
        *,
        num_layers: int = 1,
        dtype: torch.dtype = torch.float16,
        device: torch.device | str = "cpu",
        act_dtype: torch.dtype | None = None,
        head_major: bool | None = None,
    ):
        if min(num_layers, num_blocks, block_size, num_kv_heads, head_dim) <= 0:
            raise ValueError("cache dimensions must be positive")
        self.layout = CacheLayout(num_layers, num_blocks, block_size, num_kv_heads, head_dim)
        # head_major stores each block as [kv_heads, block_size, head_dim], so the
        # rows of one head are contiguous; k / v stay [layers, blocks,
        # block_size, kv_heads, head_dim] views either way (the kernels take
        # strides). The reference's layout (token-major) is the default; the
        # FP8 format, which no caller shares with the reference, is head-major.
        self.head_major = (dtype == FP8_E4M3) if head_major is None else bool(head_major)
        dev = torch.device(device)
        if self.head_major:
            store = (num_layers, num_blocks, num_kv_heads, block_size, head_dim)
            self.k = torch.empty(store, dtype=dtype, device=dev).transpose(2, 3)
            self.v = torch.empty(store, dtype=dtype, device=dev).transpose(2, 3)
        else:
            shape = (num_layers, num_blocks, block_size, num_kv_heads, head_dim)
            self.k = torch.empty(shape, dtype=dtype, device=dev)
            self.v = torch.empty_like(self.k)
        self.device = self.k.device
        self.allocator = BlockAllocator(num_blocks)
        self.fp8 = dtype == FP8_E4M3
        if self.fp8:
            self.act_dtype = act_dtype or torch.bfloat16
            if self.act_dtype not in (torch.float16, torch.bfloat16, torch.float32):
                raise ValueError("act_dtype of an FP8 cache must be float16, bfloat16 or float32")
            scale_shape = (num_layers, num_blocks, num_kv_heads, block_size)
            self.k_scale = torch.ones(scale_shape, dtype=torch.float32, device=self.device)
            self.v_scale = torch.ones_like(self.k_scale)
        else:
            if act_dtype is not None and act_dtype != dtype:
                raise ValueError("act_dtype differs from dtype only for the FP8 cache")
            self.act_dtype = dtype
            self.k_scale = self.v_scale = None

    @property
    def dtype(self) -> torch.dtype:
        """Storage type of ``k`` / ``v`` (``float8_e4m3fn`` for the FP8 cache)."""
        return self.k.dtype

    @property
    def numel_bytes(self) -> int:
        scales = 2 * self.k_scale.numel() * 4 if self.fp8 else 0
        return 2 * self.k.numel() * self.k.element_size() + scales

    def allocate_request(self, request_id: int, num_tokens: int) -> list[int]:
        if num_tokens <= 0:
            raise ValueError("num_tokens must be positive")
        blocks = -(-num_tokens // self.layout.block_size)
        return self.allocator.allocate(blocks, owner=request_id)

    def release_request(self, block_table, request_id: int | None = None) -> None:
        self.allocator.free(block_table, owner=request_id)

    def slot_mapping(self, block_table, start: int, length: int) -> torch.Tensor:
        """Physical slots of logical positions ``[start, start + length)``
        (cache.py:113-129), int64 on the cache device."""
        bs = self.layout.block_size
        if start < 0 or length < 0:
            raise ValueError("start and length must be non-negative")
        if isinstance(block_table, torch.Tensor):
            if block_table.ndim != 1:
                raise ValueError("block_table must be one-dimensional")
        elif any(
            not isinstance(block, int) or not 0 <= block < self.layout.num_blocks
            for block in block_table
        ):
            raise ValueError("block_table contains an invalid physical block id")
        if length and (start + length - 1) // bs >= len(block_table):
            raise ValueError("block_table is shorter than the requested range")
        positions = torch.arange(start, start + length, dtype=torch.long, device=self.device)
        table = torch.as_tensor(block_table, dtype=torch.long, device=self.device)
        return table[positions // bs] * bs + positions % bs

    def _check_kv(self, key: torch.Tensor, value: torch.Tensor) -> None:
        if key.shape != value.shape or key.ndim != 3:
            raise ValueError("key/value must have the same [T, H, D] shape")
        if tuple(key.shape[1:]) != (self.layout.num_kv_heads, self.layout.head_dim):
            raise ValueError("key/value shape does not match cache layout")

    def write(self, layer: int, block_table, start: int, key: torch.Tensor, value: torch.Tensor) -> None:
        """Write ``[T, Hkv, D]`` rows at logical positions ``start..start+T``."""
        self._check_kv(key, value)
        slots = self.slot_mapping(block_table, start, key.shape[0])
        if not 0 <= layer < self.layout.num_layers:
            raise IndexError("layer is out of range")
        self._scatter(layer, slots, key.to(self.device), value.to(self.device))

    def write_slots(
        self,
        layer: int,
        slots: torch.Tensor,
        key: torch.Tensor,
        value: torch.Tensor,
        *,
        validate_slots: bool = True,
    ) -> None:
        """Write flattened rows at physical slots (cache.py:156-189)."""
        self._check_kv(key, value)
        if slots.ndim != 1 or slots.numel() != key.shape[0]:
            raise ValueError("slots must have one entry per key/value token")
        if not 0 <= layer < self.layout.num_layers:
            raise IndexError("layer is out of range")
        slots = slots.to(device=self.device, dtype=torch.long)
        if validate_slots and slots.numel():
            limit = self.layout.num_blocks * self.layout.block_size
            if bool((slots < 0).any()) or bool((slots >= limit).any()):
                raise ValueError("slots contain an invalid physical cache position")
        self._scatter(layer, slots, key.to(self.device), value.to(self.device))

    def _scatter(self, layer: int, slots: torch.Tensor, key: torch.Tensor, value: torch.Tensor) -> None:
        bs = self.layout.block_size
        blocks = torch.div(slots, bs, rounding_mode="floor")
        offsets = slots.remainder(bs)
        if self.fp8:
            for store, scales, rows in ((self.k, self.k_scale, key), (self.v, self.v_scale, value)):
                codes, scale = quantize_rows_e4m3(rows)
                store[layer, blocks, offsets, :, :] = codes
                scales[layer, blocks, :, offsets] = scale
            return
        self.k[layer, blocks, offsets, :, :] = key
        self.v[layer, blocks, offsets, :, :] = value

    def read(self, layer: int, block_table, length: int) -> tuple[torch.Tensor, torch.Tensor]:
        """Gather the first ``length`` logical tokens in order (cache.py:191-200)."""
        if length < 0:
            raise ValueError("length must be non-negative")
        slots = self.slot_mapping(block_table, 0, length)
        if not 0 <= layer < self.layout.num_layers:
            raise IndexError("layer is out of range")
        bs = self.layout.block_size
        blocks = torch.div(slots, bs, rounding_mode="floor")
        offsets = slots.remainder(bs)
        if self.fp8:  # dequantised, float32
            k = self.k[layer, blocks, offsets].float() * self.k_scale[layer, blocks, :, offsets].unsqueeze(-1)
            v = self.v[layer, blocks, offsets].float() * self.v_scale[layer, blocks, :, offsets].unsqueeze(-1)
            return k, v
        return self.k[layer, blocks, offsets], self.v[layer, blocks, offsets]


def pow2_scale(amax: torch.Tensor) -> torch.Tensor:
    """2^ceil(log2(amax / 448)) (at least 2^-126) read off the fp32 bits of
    amax / 448; 1 where amax is 0 or not finite."""
    ok = (amax > 0) & torch.isfinite(amax)
    t = torch.where(ok, amax, torch.full_like(amax, E4M3_MAX)) / torch.full_like(amax, E4M3_MAX)
    bits = t.view(torch.int32)
    e = ((bits >> 23) & 0xFF) - 127 + ((bits & 0x7FFFFF) != 0).to(torch.int32)
    e = e.clamp(-126, 127)
    scale = ((e + 127) << 23).view(torch.float32)
    return torch.where(ok, scale, torch.ones_like(scale))


def quantize_rows_e4m3(rows: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """[..., D] rows -> (E4M3 codes [..., D], fp32 scales [...]): a
    power-of-two scale per row, 2^ceil(log2(amax / 448)), and codes
    e4m3(x / scale) saturated to +-448. Dividing by a power of two is exact,
    so the HIP append produces the same codes."""
    x = rows.float()
    scale = pow2_scale(x.abs().amax(dim=-1))
    codes = (x / scale.unsqueeze(-1)).clamp(-E4M3_MAX, E4M3_MAX).to(FP8_E4M3)
    return codes, scale
