"""Operator surface of the paged-KV decode path, backed by libikl_paged.so.

Same call signatures, argument meaning and error behaviour as the
reference's Triton operators:

* :func:`paged_decode_attention_hip` — ``paged_decode_attention_triton``
  (triton_ops.py:404-478);
* :func:`paged_decode_attention_hip_grouped` —
  ``paged_decode_attention_triton_grouped`` (triton_ops.py:481-610);
* :func:`append_kv_hip` — ``append_kv_triton`` (append.py:69-106);
* :func:`paged_prefill_attention_hip` — ``paged_prefill_attention_sdpa``
  (attention.py:230-321), one kernel over the paged cache instead of the
  gather + masked SDPA;
* :func:`paged_decode_grouped_path` — ``paged_decode_grouped_path``
  (triton_ops.py:56-75), answering with this library's kernel families;
* :func:`hip_available` / :func:`hip_append_available` —
  ``triton_available`` / ``triton_append_available``.

The ``*_triton`` names are kept as aliases of the same functions so callers
written against the reference bind unchanged. Every operator launches the
HIP kernels on the current torch stream and never computes on another path:
without the built library or a GPU it raises ``RuntimeError``.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib

_DTYPES = {
    torch.float16: _lib.IKL_F16,
    torch.bfloat16: _lib.IKL_BF16,
    torch.float32: _lib.IKL_F32,
}
_INDEX_TYPES = {torch.int32: _lib.IKL_I32, torch.int64: _lib.IKL_I64}

_PATH_NAMES = {
    _lib.IKL_PATH_MHA_FALLBACK: "mha_fallback",
    _lib.IKL_PATH_SCALAR_GROUPED: "scalar_grouped",
    _lib.IKL_PATH_MFMA_GROUPED: "mfma_grouped",
}
_PATH_IDS = {name: ident for ident, name in _PATH_NAMES.items()}


def hip_available() -> bool:
    """True when libikl_paged.so loads and a GPU is visible."""
    return torch.cuda.is_available() and _lib.library_loaded()


def hip_append_available() -> bool:
    return hip_available()


def _require_backend() -> ctypes.CDLL:
    if not torch.cuda.is_available():
        raise RuntimeError("HIP paged-decode backend is unavailable: no GPU is visible")
    try:
        return _lib.load()
    except RuntimeError as exc:
        raise RuntimeError(f"HIP paged-decode backend is unavailable: {exc}") from exc


# Kernel family names of paged_decode_grouped_path -> the reference's names
# for the corresponding kernel (triton_ops.py:56-75).
REFERENCE_PATH_NAMES = {
    "mha_fallback": "mha_fallback",
    "mfma_grouped": "tensorcore_short_context",
    "scalar_grouped": "scalar_grouped",
}


def paged_decode_grouped_path(
    *,
    dtype: torch.dtype,
    head_dim: int,
    table_width: int,
    heads_per_kv: int,
    query_group_size: int,
    block_size: int = 16,
) -> str:
    """Kernel family a grouped launch of this static shape runs.

    ``"mha_fallback"`` when every KV head serves one query head;
    ``"mfma_grouped"`` (matrix cores) for fp16/bf16 caches with head_dim in
    {32, 64, 96, 128} and a block size that is a multiple of 16; otherwise
    ``"scalar_grouped"`` (the query group shares each K/V tile on the VALU).
    Pure function of its arguments, like triton_ops.py:56-75; ``block_size``
    (keyword, default 16 like the reference's caches) is an addition the
    MFMA tiles need. The library's ``ikl_paged_attention_path`` applies the
    same rule.

    ``"mfma_grouped"`` is this library's counterpart of the reference's
    ``"tensorcore_short_context"`` (``REFERENCE_PATH_NAMES`` maps each
    name); the reference picks it only for table_width <= 16 and groups of
    at least 4 heads, and answers ``"scalar_grouped"`` elsewhere, where the
    matrix cores here still run.
    """
    if heads_per_kv == 1:
        return "mha_fallback"
    if (
        dtype in (torch.float16, torch.bfloat16)
        and head_dim in (32, 64, 96, 128)
        and block_size > 0
        and block_size % 16 == 0
    ):
        return "mfma_grouped"
    return "scalar_grouped"


def _as_index_tensor(value, device: torch.device) -> torch.Tensor:
    if isinstance(value, list):
        return torch.tensor(value, dtype=torch.int32, device=device)
    return value


def _validate_attention(query, cache, block_tables, context_lens, layer, validate_inputs,
                        max_context_len=None):
    """Checks of triton_ops.py:415-457, in the same order with the same
    messages, plus this library's ``max_context_len`` hint (a bound of
    ``context_lens`` that sizes the fixed-partition grid); returns the table
    and length tensors."""
    if query.ndim != 3 or query.device.type != "cuda":
        raise ValueError("query must be a GPU (torch 'cuda' device) tensor with shape [B,H,D]")
    if query.shape[0] <= 0 or query.shape[1] <= 0 or query.shape[2] <= 0:
        raise ValueError("query dimensions must be positive")
    if query.shape[-1] > 128:
        raise ValueError("the current HIP kernel supports head_dim <= 128")
    if query.stride(-1) != 1:
        raise ValueError("query must be contiguous in the head_dim dimension")
    block_tables = _as_index_tensor(block_tables, query.device)
    context_lens = _as_index_tensor(context_lens, query.device)
    layout = cache.layout
    if not 0 <= layer < layout.num_layers:
        raise IndexError("layer is out of range")
    if query.shape[-1] != layout.head_dim:
        raise ValueError("query head_dim does not match cache layout")
    if query.shape[1] % layout.num_kv_heads != 0:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    if query.dtype != cache.act_dtype or query.device != cache.device:
        raise ValueError("query and cache must have the same dtype and device")
    if block_tables.ndim != 2 or block_tables.shape[0] != query.shape[0]:
        raise ValueError("block_tables must have shape [B, max_blocks]")
    if context_lens.ndim != 1 or context_lens.shape[0] != query.shape[0]:
        raise ValueError("context_lens must have shape [B]")
    if block_tables.device != query.device or context_lens.device != query.device:
        raise ValueError("block_tables and context_lens must be on the query device")
    if block_tables.dtype not in _INDEX_TYPES:
        raise ValueError("block_tables must use int32 or int64")
    if context_lens.dtype not in _INDEX_TYPES:
        raise ValueError("context_lens must use int32 or int64")
    if block_tables.shape[1] <= 0:
        raise ValueError("block_tables must contain at least one logical block")
    if validate_inputs:
        if bool(torch.any(context_lens <= 0).item()):
            raise ValueError("context lengths must be positive")
        max_context = block_tables.shape[1] * layout.block_size
        if bool(torch.any(context_lens > max_context).item()):
            raise ValueError("context length exceeds block table capacity")
        if bool(torch.any(block_tables < 0).item()) or bool(
            torch.any(block_tables >= layout.num_blocks).item()
        ):
            raise ValueError("block table contains an invalid physical block id")
        if max_context_len and bool(torch.any(context_lens > max_context_len).item()):
            raise ValueError("context length exceeds max_context_len")
    if query.dtype not in _DTYPES:
        raise ValueError("query dtype must be float16, bfloat16 or float32")
    return block_tables, context_lens


def _aligned_rows(t: torch.Tensor) -> bool:
    vec = 16 // t.element_size()
    return t.data_ptr() % 16 == 0 and all(s % vec == 0 for s in t.stride()[:-1])


def _attention_args(
    query,
    cache,
    block_tables,
    context_lens,
    out,
    scale,
    layer,
    query_group_size,
    partition_size,
    max_context_len,
    path,
):
    layout = cache.layout
    k_cache = cache.k[layer]
    v_cache = cache.v[layer]
    if block_tables.stride(-1) != 1:
        block_tables = block_tables.contiguous()
    if context_lens.stride(0) != 1:
        context_lens = context_lens.contiguous()
    args = _lib.PagedAttentionArgs()
    args.query = query.data_ptr()
    args.q_stride_b, args.q_stride_h = query.stride(0), query.stride(1)
    args.k_cache = k_cache.data_ptr()
    args.v_cache = v_cache.data_ptr()
    args.k_stride_block, args.k_stride_token, args.k_stride_head = k_cache.stride()[:3]
    args.v_stride_block, args.v_stride_token, args.v_stride_head = v_cache.stride()[:3]
    args.block_tables = block_tables.data_ptr()
    args.table_type = _INDEX_TYPES[block_tables.dtype]
    args.table_stride_b = block_tables.stride(0)
    args.table_width = block_tables.shape[1]
    args.context_lens = context_lens.data_ptr()
    args.lens_type = _INDEX_TYPES[context_lens.dtype]
    args.out = out.data_ptr()
    args.out_stride_b, args.out_stride_h = out.stride(0), out.stride(1)
    args.batch = query.shape[0]
    args.num_blocks = layout.num_blocks
    args.num_heads = query.shape[1]
    args.num_kv_heads = layout.num_kv_heads
    args.head_dim = layout.head_dim
    args.block_size = layout.block_size
    args.dtype = _DTYPES[query.dtype]
    args.scale = float(scale if scale is not None else layout.head_dim**-0.5)
    args.query_group_size = int(query_group_size)
    args.partition_size = int(partition_size)
    args.max_context_len = int(max_context_len)
    args.path = int(path)
    keep = (block_tables, context_lens, k_cache, v_cache)
    if cache.fp8:
        ks, vs = cache.k_scale[layer], cache.v_scale[layer]
        args.cache_dtype = _lib.IKL_FP8_E4M3
        args.k_scale, args.v_scale = ks.data_ptr(), vs.data_ptr()
        args.scale_stride_block, args.scale_stride_head = ks.stride(0), ks.stride(1)
        keep = keep + (ks, vs)
    # keep the tensors whose pointers the struct holds alive with it
    return args, keep


def _launch_attention(
    query,
    cache,
    block_tables,
    context_lens,
    scale,
    layer,
    *,
    query_group_size: int,
    partition_size: int | None,
    max_context_len: int | None,
    path: int = -1,
    events=None,
) -> torch.Tensor:
    lib = _require_backend()
    if not _aligned_rows(query):
        query = query.contiguous()
    for tensor in (cache.k, cache.v):
        if not _aligned_rows(tensor):
            raise ValueError("cache tensors must have 16-byte aligned head_dim rows")
    output = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    args, keep = _attention_args(
        query,
        cache,
        block_tables,
        context_lens,
        output,
        scale,
        layer,
        query_group_size,
        partition_size or 0,
        max_context_len or 0,
        path,
    )
    ws_bytes = lib.ikl_paged_attention_workspace_size(ctypes.byref(args))
    _lib.check(ws_bytes if ws_bytes < 0 else 0, "paged attention")
    workspace = None
    if ws_bytes > 0:
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=query.device)
        args.workspace = workspace.data_ptr()
        args.workspace_bytes = ws_bytes
    if events is not None:
        for i, ev in enumerate(events):
            args.events[i] = ev
    with torch.cuda.device(query.device):
        stream = torch.cuda.current_stream(query.device).cuda_stream
        status = lib.ikl_paged_attention(ctypes.byref(args), ctypes.c_void_p(stream))
    _lib.check(status, "paged attention")
    _record_launch(args)
    del keep, workspace  # the caching allocator keeps stream order
    return output


# ------------------------------------------------------- launch reporting
_SPLIT_NAMES = {0: "none", 1: "fixed_partitions", 2: "balanced"}
_last_launch: dict[str, dict] = {}


def launch_config(args) -> dict:
    """The launch an ikl_paged_attention_args struct resolves to (planning
    only: needs the library, not a GPU)."""
    lib = _lib.load()
    out = _lib.LaunchConfig()
    out.struct_size = ctypes.sizeof(out)
    _lib.check(lib.ikl_paged_attention_launch_config(ctypes.byref(args), ctypes.byref(out)), "launch config")
    return {
        "path": _PATH_NAMES[out.path],
        "block_n": out.tile_tokens,
        "num_warps": out.waves_per_workgroup,
        "num_stages": out.stages,
        "split": _SPLIT_NAMES[out.split],
        "partition_size": out.partition_size,
        "workgroups": out.workgroups,
        "group_size": out.group_size,
    }


def _record_launch(args) -> None:
    cfg = launch_config(args)
    _last_launch[cfg["path"]] = cfg
    if args.num_heads == args.num_kv_heads:
        _last_launch["one_head_per_kv"] = cfg  # whichever family ran it
    else:
        _last_launch["grouped"] = cfg  # the last launch of either grouped family


def _reported(path: str) -> dict | None:
    cfg = _last_launch.get(path)
    return None if cfg is None else {k: cfg[k] for k in ("block_n", "num_warps", "num_stages")}


def paged_decode_autotune_config() -> dict | None:
    """Tile configuration of the most recent one-head-per-KV-head launch
    (triton_ops.py:17-27 reports the Triton autotuner's pick the same way);
    ``block_n`` = positions per wave loop step, ``num_warps`` = waves per
    workgroup, ``num_stages`` = tiles in flight per wave. None before any
    such launch. The library runs small one-head-per-KV-head launches (and
    any with ``partition_size=-2``) on the matrix-core family; this reports
    whichever family ran the most recent one."""
    return _reported("one_head_per_kv")


def paged_decode_grouped_autotune_config() -> dict | None:
    """As :func:`paged_decode_autotune_config` for the most recent grouped
    launch of either family, VALU or matrix-core (triton_ops.py:30-40).

    The reference's callers pick the reporter by path name
    (hf_benchmark.py:942-945, scripts/run_decode_sweep.py:249): the tl.dot
    reporter for ``"tensorcore_short_context"``, this one otherwise. This
    library's matrix-core path is named ``"mfma_grouped"``, so those callers
    land here, and get the matrix-core launch they ran."""
    return _reported("grouped")


def paged_decode_grouped_dot_autotune_config() -> dict | None:
    """As :func:`paged_decode_autotune_config` for the MFMA kernel, the
    counterpart of the reference's tl.dot grouped kernel (triton_ops.py:43-53)."""
    return _reported("mfma_grouped")


def paged_decode_attention_hip(
    query,
    cache,
    block_tables,
    context_lens,
    scale=None,
    layer=0,
    *,
    validate_inputs=True,
    partition_size: int | None = None,
    max_context_len: int | None = None,
    events=None,
):
    """Paged decode attention; disable value checks only for prevalidated inputs.

    Signature of ``paged_decode_attention_triton`` (triton_ops.py:404-413).
    All query heads of a KV head share each K/V tile in one workgroup (the
    kernel family is picked by :func:`paged_decode_grouped_path`). Extra
    keyword-only knobs: ``partition_size`` (tokens per split-context
    partition; ``-1`` never splits, ``-2`` asks for the matrix-core
    family's balanced split, ``None`` picks automatically),
    ``max_context_len`` (a host-known bound of ``context_lens`` used to size
    the split grid: positions past it are not attended on the fixed
    partitions, so with ``validate_inputs`` a longer context raises
    ``ValueError``) and ``events`` (up to three raw hipEvent_t handles
    recorded before the attention kernel, after it and after the split
    reduce, for timing).
    """
    block_tables, context_lens = _validate_attention(
        query, cache, block_tables, context_lens, layer, validate_inputs, max_context_len
    )
    return _launch_attention(
        query,
        cache,
        block_tables,
        context_lens,
        scale,
        layer,
        query_group_size=0,
        partition_size=partition_size,
        max_context_len=max_context_len,
        events=events,
    )


def paged_decode_attention_hip_grouped(
    query,
    cache,
    block_tables,
    context_lens,
    scale=None,
    layer=0,
    *,
    query_group_size=8,
    validate_inputs=True,
    partition_size: int | None = None,
    max_context_len: int | None = None,
):
    """Grouped-query paged attention with one K/V tile per query group.

    Signature of ``paged_decode_attention_triton_grouped``
    (triton_ops.py:481-491): on the VALU path ``min(query_group_size,
    H/Hkv)`` query heads share each K/V tile; MHA shapes take the one-head
    path (541-551). ``query_group_size`` is a tiling choice there (the
    Triton kernel's ``block_h``), not part of the result. On the matrix-core
    path every query head of a KV head shares the tile (up to 32 per wave),
    whatever the group size: a smaller group would only read K/V once more
    per group (MQA 32/1, batch 64: 66.7 µs with groups of 8 against 35.5 µs).
    """
    block_tables, context_lens = _validate_attention(
        query, cache, block_tables, context_lens, layer, validate_inputs, max_context_len
    )
    if query_group_size not in (1, 2, 4, 8):
        raise ValueError("query_group_size must be one of 1, 2, 4, or 8")
    heads_per_kv = query.shape[1] // cache.layout.num_kv_heads
    path_name = paged_decode_grouped_path(
        dtype=query.dtype,
        head_dim=cache.layout.head_dim,
        table_width=block_tables.shape[1],
        heads_per_kv=heads_per_kv,
        query_group_size=query_group_size,
        block_size=cache.layout.block_size,
    )
    return _launch_attention(
        query,
        cache,
        block_tables,
        context_lens,
        scale,
        layer,
        query_group_size=1 if heads_per_kv == 1 else (0 if path_name == "mfma_grouped" else query_group_size),
        partition_size=partition_size,
        max_context_len=max_context_len,
        # the FP8 cache is read by the MFMA family only, and partition_size -2
        # (the balanced split) leaves the family to the library, which runs
        # it on the MFMA family (MHA included) where that supports the shape
        path=-1 if cache.fp8 or partition_size == -2 else _PATH_IDS[path_name],
    )


def append_kv_hip(key: torch.Tensor, value: torch.Tensor, cache, slots: torch.Tensor, layer: int = 0) -> None:
    """Append ``[tokens, kv_heads, head_dim]`` rows into paged cache slots.

    Signature and checks of ``append_kv_triton`` (append.py:69-106); writes
    ``cache.k[layer]`` / ``cache.v[layer]`` in place on the current stream.
    Slots outside ``[0, num_blocks * block_size)`` are skipped.
    """
    lib = _require_backend()
    if key.shape != value.shape or key.ndim != 3:
        raise ValueError("key/value must have shape [T, Hkv, D]")
    if key.device.type != "cuda" or slots.device != key.device or value.device != key.device:
        raise ValueError("key/value/slots must be on the same GPU device")
    layout = cache.layout
    if tuple(key.shape[1:]) != (layout.num_kv_heads, layout.head_dim):
        raise ValueError("key/value shape does not match cache layout")
    if slots.numel() != key.shape[0]:
        raise ValueError("slots and key/value token counts must match")
    if not 0 <= layer < layout.num_layers:
        raise IndexError("layer is out of range")
    if key.dtype != cache.act_dtype or value.dtype != cache.act_dtype:
        raise ValueError("key/value dtype must match the cache dtype")
    if slots.dtype not in _INDEX_TYPES:
        raise ValueError("slots must use int32 or int64")
    if key.stride(-1) != 1:
        key = key.contiguous()
    if value.stride(-1) != 1:
        value = value.contiguous()
    slots = slots.reshape(-1)
    if slots.numel() and slots.stride(0) != 1:
        slots = slots.contiguous()
    if key.shape[0] == 0:
        return
    args, keep = _append_args(key, value, cache, slots, layer)
    with torch.cuda.device(key.device):
        stream = torch.cuda.current_stream(key.device).cuda_stream
        status = lib.ikl_append_kv(ctypes.byref(args), ctypes.c_void_p(stream))
    del keep
    _lib.check(status, "append_kv")


def rope_append_kv_hip(query: torch.Tensor | None, key: torch.Tensor, value: torch.Tensor,
                       cos: torch.Tensor, sin: torch.Tensor, cache, slots: torch.Tensor, layer: int = 0,
                       *, query_out: torch.Tensor | None = None) -> torch.Tensor | None:
    """Rotary embedding of q and k fused with the KV append (one launch).

    ``query`` ``[T, H, D]`` (or None), ``key`` / ``value`` ``[T, Hkv, D]``,
    ``cos`` / ``sin`` ``[T, D]`` rows of each token's position in the tensors'
    dtype, ``slots`` ``[T]``. Writes ``rope(key)`` and ``value`` into
    ``cache.k[layer]`` / ``cache.v[layer]`` at the slots and returns
    ``rope(query)`` (into ``query_out``, default: ``query`` in place).
    ``rope(x) = x * cos + rotate_half(x) * sin`` as hf_benchmark.py:69-85,
    bit-exact with the torch elementwise ops on the same rows. Slots outside
    the cache are skipped.
    """
    lib = _require_backend()
    layout = cache.layout
    if key.shape != value.shape or key.ndim != 3 or tuple(key.shape[1:]) != (layout.num_kv_heads, layout.head_dim):
        raise ValueError("key/value must have shape [T, Hkv, D] matching the cache layout")
    t = key.shape[0]
    if cos.shape != (t, layout.head_dim) or sin.shape != cos.shape:
        raise ValueError("cos/sin must have shape [T, head_dim]")
    if query is not None and (query.ndim != 3 or query.shape[0] != t or query.shape[2] != layout.head_dim
                              or query.shape[1] % layout.num_kv_heads != 0):
        raise ValueError("query must have shape [T, H, head_dim] with H a multiple of num_kv_heads")
    tensors = [key, value, cos, sin] + ([query] if query is not None else [])
    if any(x.dtype != cache.act_dtype for x in tensors):
        raise ValueError("query/key/value/cos/sin must share the cache dtype")
    if any(x.device != cache.device for x in tensors) or slots.device != cache.device:
        raise ValueError("tensors must be on the cache device")
    if slots.dtype not in _INDEX_TYPES or slots.numel() != t:
        raise ValueError("slots must be int32/int64 with one entry per token")
    if not 0 <= layer < layout.num_layers:
        raise IndexError("layer is out of range")
    key, value, cos, sin = (x if _aligned_rows(x) else x.contiguous() for x in (key, value, cos, sin))
    if query is not None:
        if not _aligned_rows(query):
            query = query.contiguous()
        if query_out is None:
            query_out = query
        elif query_out.shape != query.shape or query_out.dtype != query.dtype or not _aligned_rows(query_out):
            raise ValueError("query_out must match query and have 16-byte aligned rows")
    slots = slots.reshape(-1).contiguous()
    if t == 0:
        return query_out
    a = _lib.RopeAppendArgs()
    if query is not None:
        a.query, a.q_stride_t, a.q_stride_h = query.data_ptr(), query.stride(0), query.stride(1)
        a.query_out, a.q_out_stride_t, a.q_out_stride_h = query_out.data_ptr(), query_out.stride(0), query_out.stride(1)
        a.num_heads = query.shape[1]
    a.key, a.key_stride_t, a.key_stride_h = key.data_ptr(), key.stride(0), key.stride(1)
    a.value, a.value_stride_t, a.value_stride_h = value.data_ptr(), value.stride(0), value.stride(1)
    a.cos, a.cos_stride_t = cos.data_ptr(), cos.stride(0)
    a.sin, a.sin_stride_t = sin.data_ptr(), sin.stride(0)
    a.slots = slots.data_ptr()
    a.slot_type = _INDEX_TYPES[slots.dtype]
    kc, vc = cache.k[layer], cache.v[layer]
    a.k_cache, a.v_cache = kc.data_ptr(), vc.data_ptr()
    a.k_stride_block, a.k_stride_token, a.k_stride_head = kc.stride(0), kc.stride(1), kc.stride(2)
    a.v_stride_block, a.v_stride_token, a.v_stride_head = vc.stride(0), vc.stride(1), vc.stride(2)
    a.num_tokens, a.num_blocks, a.block_size = t, layout.num_blocks, layout.block_size
    a.num_kv_heads, a.head_dim, a.dtype = layout.num_kv_heads, layout.head_dim, _DTYPES[cache.act_dtype]
    if cache.fp8:
        ks, vs = cache.k_scale[layer], cache.v_scale[layer]
        a.cache_dtype = _lib.IKL_FP8_E4M3
        a.k_scale, a.v_scale = ks.data_ptr(), vs.data_ptr()
        a.scale_stride_block, a.scale_stride_head = ks.stride(0), ks.stride(1)
    with torch.cuda.device(key.device):
        stream = torch.cuda.current_stream(key.device).cuda_stream
        status = lib.ikl_rope_append_kv(ctypes.byref(a), ctypes.c_void_p(stream))
    _lib.check(status, "rope_append_kv")
    return query_out


def _append_args(key, value, cache, slots, layer):
    layout = cache.layout
    k_cache = cache.k[layer]
    v_cache = cache.v[layer]
    args = _lib.AppendArgs()
    args.key, args.value = key.data_ptr(), value.data_ptr()
    args.key_stride_t, args.key_stride_h = key.stride(0), key.stride(1)
    args.value_stride_t, args.value_stride_h = value.stride(0), value.stride(1)
    args.slots = slots.data_ptr()
    args.slot_type = _INDEX_TYPES[slots.dtype]
    args.k_cache, args.v_cache = k_cache.data_ptr(), v_cache.data_ptr()
    args.k_stride_block, args.k_stride_token, args.k_stride_head = k_cache.stride()[:3]
    args.v_stride_block, args.v_stride_token, args.v_stride_head = v_cache.stride()[:3]
    args.num_tokens = key.shape[0]
    args.num_blocks = layout.num_blocks
    args.block_size = layout.block_size
    args.num_kv_heads = layout.num_kv_heads
    args.head_dim = layout.head_dim
    args.dtype = _DTYPES[key.dtype]
    keep = (key, value, slots, k_cache, v_cache)
    if cache.fp8:
        ks, vs = cache.k_scale[layer], cache.v_scale[layer]
        args.cache_dtype = _lib.IKL_FP8_E4M3
        args.k_scale, args.v_scale = ks.data_ptr(), vs.data_ptr()
        args.scale_stride_block, args.scale_stride_head = ks.stride(0), ks.stride(1)
        keep = keep + (ks, vs)
    return args, keep


class PreparedPagedAttention:
    """Paged decode attention validated once on fixed buffers.

    Binds the query, one cache layer, block tables, context lengths, an
    output buffer and the split workspace; each call only enqueues the
    kernels on the current stream (no validation, allocation or host sync).
    Callers may update the bound tensors in place between calls (new query
    rows, longer contexts up to ``max_context_len``, appended table
    entries) — the same metadata reuse as the reference's decode loop
    (decode.py:361-391). Results equal :func:`paged_decode_attention_hip`.
    """

    def __init__(self, query, cache, block_tables, context_lens, scale=None, layer=0, *,
                 query_group_size: int = 0, partition_size: int | None = None,
                 max_context_len: int | None = None, validate_inputs: bool = True):
        self._lib = _require_backend()
        block_tables, context_lens = _validate_attention(
            query, cache, block_tables, context_lens, layer, validate_inputs, max_context_len
        )
        if not _aligned_rows(query):
            raise ValueError("query rows must be 16-byte aligned for a prepared launch")
        for tensor in (cache.k, cache.v):
            if not _aligned_rows(tensor):
                raise ValueError("cache tensors must have 16-byte aligned head_dim rows")
        self.query = query
        self.block_tables = block_tables
        self.context_lens = context_lens
        self.out = torch.empty(query.shape, dtype=query.dtype, device=query.device)
        self._args, self._keep = _attention_args(
            query, cache, block_tables, context_lens, self.out, scale, layer, query_group_size,
            partition_size or 0, max_context_len or 0, -1,
        )
        ws = self._lib.ikl_paged_attention_workspace_size(ctypes.byref(self._args))
        _lib.check(ws if ws < 0 else 0, "paged attention")
        self.workspace = torch.empty(max(ws, 1), dtype=torch.uint8, device=query.device)
        self._args.workspace = self.workspace.data_ptr()
        self._args.workspace_bytes = ws
        self.partition_size = self._lib.ikl_paged_attention_partition_size(ctypes.byref(self._args))
        a = self._args
        self.launch = launch_config(a)
        self.path = self.launch["path"]
        self.balanced_split = self.launch["split"] == "balanced"
        _record_launch(a)
        self.device = query.device

    def kernel_names(self) -> tuple[str, str | None]:
        """(attention kernel, reduce kernel or None) this launch enqueues."""
        if self.path == "mfma_grouped":
            if not self.balanced_split:
                main = "paged_decode_mfma_kernel"
            elif self.launch["group_size"] <= 16 and self.launch["num_warps"] > 1:
                main = "paged_decode_mfma_unitk_kernel"  # unit-parallel: one unit per wave
            else:
                main = "paged_decode_mfma_streamk_kernel"
        else:
            main = "paged_decode_scalar_kernel"
        return main, ("paged_decode_reduce_kernel" if self.launch["split"] != "none" else None)

    def __call__(self, events=None) -> torch.Tensor:
        for i in range(3):
            self._args.events[i] = events[i] if events is not None else None
        stream = torch.cuda.current_stream(self.device).cuda_stream
        status = self._lib.ikl_paged_attention(ctypes.byref(self._args), ctypes.c_void_p(stream))
        _lib.check(status, "paged attention")
        return self.out


class PreparedAppend:
    """KV append validated once on fixed key/value/slot buffers; each call
    only enqueues the scatter (see :func:`append_kv_hip`)."""

    def __init__(self, key, value, cache, slots, layer: int = 0):
        self._lib = _require_backend()
        if key.shape != value.shape or key.ndim != 3 or key.stride(-1) != 1 or value.stride(-1) != 1:
            raise ValueError("key/value must be [T, Hkv, D] with a contiguous last dimension")
        if tuple(key.shape[1:]) != (cache.layout.num_kv_heads, cache.layout.head_dim):
            raise ValueError("key/value shape does not match cache layout")
        if slots.ndim != 1 or slots.numel() != key.shape[0] or slots.stride(0) != 1:
            raise ValueError("slots and key/value token counts must match")
        if slots.dtype not in _INDEX_TYPES:
            raise ValueError("slots must use int32 or int64")
        if key.dtype != cache.act_dtype or value.dtype != cache.act_dtype:
            raise ValueError("key/value dtype must match the cache dtype")
        if not 0 <= layer < cache.layout.num_layers:
            raise IndexError("layer is out of range")
        self._args, self._keep = _append_args(key, value, cache, slots, layer)
        self.device = key.device

    def __call__(self) -> None:
        stream = torch.cuda.current_stream(self.device).cuda_stream
        status = self._lib.ikl_append_kv(ctypes.byref(self._args), ctypes.c_void_p(stream))
        _lib.check(status, "append_kv")


class PreparedDecodeStep:
    """One decode step on bound buffers: paged decode attention of
    ``attention`` (a :class:`PreparedPagedAttention`), then the KV append of
    ``append`` (a :class:`PreparedAppend`), in the synthetic runner's order
    (decode.py:480-487), enqueued by one library call
    (``ikl_paged_decode_step``). When the attention splits, the reduce
    kernel also carries the append — one launch less per step — with the
    same result as calling the two separately (``fused`` tells which); an
    unsplit attention is followed by the append's own launch. The step
    runs on the attention's own arguments and workspace
    (``ikl_paged_decode_step_workspace_size`` equals the attention's)."""

    def __init__(self, attention: PreparedPagedAttention, append: PreparedAppend):
        if attention.device != append.device:
            raise ValueError("attention and append must be on the same device")
        self._lib = _require_backend()
        self.attention, self.append = attention, append
        self._args = attention._args
        app = ctypes.byref(append._args)
        need = self._lib.ikl_paged_decode_step_workspace_size(ctypes.byref(self._args), app)
        _lib.check(need if need < 0 else 0, "decode step")
        if need > attention._args.workspace_bytes:
            raise RuntimeError(f"decode step: needs {need} bytes of workspace, the attention holds "
                               f"{attention._args.workspace_bytes}")
        mode = self._lib.ikl_paged_decode_step_fused(ctypes.byref(self._args), app)
        _lib.check(mode if mode < 0 else 0, "decode step")
        self.fused = mode == 1
        self.device = attention.device

    @property
    def out(self) -> torch.Tensor:
        return self.attention.out

    def kernel_names(self) -> tuple[str, ...]:
        """Kernels one step enqueues, in order."""
        main, reduce = self.attention.kernel_names()
        if self.fused:
            return main, "paged_decode_reduce_kernel"
        return tuple(n for n in (main, reduce) if n) + ("append_kv_kernel",)

    def __call__(self, events=None) -> torch.Tensor:
        a = self._args
        for i in range(3):
            a.events[i] = events[i] if events is not None else None
        stream = torch.cuda.current_stream(self.device).cuda_stream
        status = self._lib.ikl_paged_decode_step(ctypes.byref(a), ctypes.byref(self.append._args),
                                                 ctypes.c_void_p(stream))
        _lib.check(status, "decode step")
        return self.attention.out


def paged_decode_step_hip(query, cache, block_tables, context_lens, key, value, slots, scale=None, layer=0, *,
                          validate_inputs=True, partition_size: int | None = None,
                          max_context_len: int | None = None) -> torch.Tensor:
    """Attention of ``query`` over the paged contexts, then the append of
    ``key`` / ``value`` rows ``[T, Hkv, D]`` at ``slots`` (same checks as
    :func:`paged_decode_attention_hip` and :func:`append_kv_hip`); returns the
    attention output. One library call; see :class:`PreparedDecodeStep`."""
    if key.stride(-1) != 1:
        key = key.contiguous()
    if value.stride(-1) != 1:
        value = value.contiguous()
    slots = slots.reshape(-1)
    if slots.numel() and slots.stride(0) != 1:
        slots = slots.contiguous()
    if not _aligned_rows(query):
        query = query.contiguous()
    attention = PreparedPagedAttention(query, cache, block_tables, context_lens, scale, layer,
                                       partition_size=partition_size, max_context_len=max_context_len,
                                       validate_inputs=validate_inputs)
    append = PreparedAppend(key, value, cache, slots, layer)
    return PreparedDecodeStep(attention, append)()


# ------------------------------------------------------------ prefill
def paged_prefill_path(*, dtype: torch.dtype, head_dim: int, block_size: int = 16) -> str:
    """Kernel family of a prefill launch: ``"mfma_grouped"`` for fp16/bf16
    with head_dim in {32, 64, 96, 128} and a block size that is a multiple
    of 16, else ``"scalar_grouped"``. Same rule as the library's
    ``ikl_paged_prefill_path``."""
    if (
        dtype in (torch.float16, torch.bfloat16)
        and head_dim in (32, 64, 96, 128)
        and block_size > 0
        and block_size % 16 == 0
    ):
        return "mfma_grouped"
    return "scalar_grouped"


def _prefill_ranges(query_starts, context_lens, batch: int, query_width: int) -> tuple[list[int], list[int]]:
    """Host copies of the chunk ranges with the checks of attention.py:257-273."""
    starts = (
        query_starts.detach().cpu().tolist() if isinstance(query_starts, torch.Tensor) else list(query_starts)
    )
    ends = context_lens.detach().cpu().tolist() if isinstance(context_lens, torch.Tensor) else list(context_lens)
    if len(starts) != batch or len(ends) != batch:
        raise ValueError("query_starts and context_lens must have one entry per query batch")
    spans = [int(e) - int(s) for s, e in zip(starts, ends)]
    if any(int(s) < 0 or n <= 0 for s, n in zip(starts, spans)):
        raise ValueError("prefill ranges must be non-empty and non-negative")
    if max(spans) > query_width:
        raise ValueError("query width is smaller than a prefill range")
    return [int(s) for s in starts], [int(e) for e in ends]


def _prefill_table(block_tables, cache, batch: int, ends: list[int]) -> torch.Tensor:
    """Block table on the cache device with the checks of attention.py:275-288."""
    if isinstance(block_tables, torch.Tensor):
        dtype = block_tables.dtype if block_tables.dtype in _INDEX_TYPES else torch.int64
        table = block_tables.to(device=cache.device, dtype=dtype)
    else:
        table = torch.as_tensor(block_tables, dtype=torch.int32, device=cache.device)
    if table.ndim != 2 or table.shape[0] != batch:
        raise ValueError("block_tables must have one row per query batch")
    max_context = max(ends)
    if max_context <= 0:
        raise ValueError("context lengths must be positive")
    bs = cache.layout.block_size
    if (max_context + bs - 1) // bs > table.shape[1]:
        raise ValueError("context length exceeds block table capacity")
    return table if table.stride(-1) == 1 else table.contiguous()


def _aligned_prefill_rows(t: torch.Tensor, width: int) -> bool:
    vec = max(1, width // t.element_size())
    return t.data_ptr() % width == 0 and all(s % vec == 0 for s in t.stride()[:-1]) and t.stride(-1) == 1


class PreparedPagedPrefill:
    """Paged prefill attention for one batch of prompt chunks, checked once.

    Binds the cache, the block tables and the chunk ranges (row ``t`` of
    request ``b`` sits at position ``query_starts[b] + t``; the chunk ends at
    ``context_lens[b]``); each call takes one layer's query ``[B, H, T, D]``
    and enqueues one kernel on the current stream, so a layer loop pays the
    range checks and the host-to-device copy of the ranges once. Results
    equal :func:`paged_prefill_attention_hip`.
    """

    def __init__(self, cache, block_tables, query_starts, context_lens, *, num_heads: int,
                 query_width: int, scale: float | None = None, path: str | None = None):
        layout = cache.layout
        if num_heads <= 0 or num_heads % layout.num_kv_heads != 0:
            raise ValueError("num_heads must be divisible by num_kv_heads")
        batch = len(query_starts)
        self.starts, self.ends = _prefill_ranges(query_starts, context_lens, batch, query_width)
        self.block_tables = _prefill_table(block_tables, cache, batch, self.ends)
        if cache.act_dtype not in _DTYPES:
            raise ValueError("cache dtype must be float16, bfloat16 or float32")
        self.path = path or paged_prefill_path(dtype=cache.act_dtype, head_dim=layout.head_dim,
                                               block_size=layout.block_size)
        if cache.fp8 and self.path != "mfma_grouped":
            raise ValueError("the FP8 cache is read by the MFMA prefill kernel only (fp16/bf16, head_dim "
                             "32/64/96/128, block size a multiple of 16)")
        if self.path not in ("mfma_grouped", "scalar_grouped"):
            raise ValueError("path must be 'mfma_grouped' or 'scalar_grouped'")
        self._row_align = 16 if self.path == "mfma_grouped" else 4
        for tensor in (cache.k, cache.v):
            if not _aligned_prefill_rows(tensor, self._row_align):
                raise ValueError("cache tensors must have aligned head_dim rows")
        self._lib = _require_backend()
        self.cache = cache
        self.shape = (batch, num_heads, query_width, layout.head_dim)
        ranges = torch.tensor([self.starts, self.ends], dtype=torch.int32)
        self.ranges = ranges.to(cache.device, non_blocking=False)
        a = _lib.PagedPrefillArgs()
        a.block_tables = self.block_tables.data_ptr()
        a.table_type = _INDEX_TYPES[self.block_tables.dtype]
        a.table_stride_b = self.block_tables.stride(0)
        a.table_width = self.block_tables.shape[1]
        a.query_starts = self.ranges[0].data_ptr()
        a.context_lens = self.ranges[1].data_ptr()
        a.lens_type = _lib.IKL_I32
        a.batch, a.query_width = batch, query_width
        a.num_blocks = layout.num_blocks
        a.num_heads, a.num_kv_heads = num_heads, layout.num_kv_heads
        a.head_dim, a.block_size = layout.head_dim, layout.block_size
        a.dtype = _DTYPES[cache.act_dtype]
        a.cache_dtype = _lib.IKL_FP8_E4M3 if cache.fp8 else 0
        a.scale = float(scale if scale is not None else layout.head_dim**-0.5)
        a.path = _PATH_IDS[self.path]
        self._args = a

    def kernel_name(self) -> str:
        return "paged_prefill_mfma_kernel" if self.path == "mfma_grouped" else "paged_prefill_scalar_kernel"

    def __call__(self, query: torch.Tensor, layer: int = 0, *, out: torch.Tensor | None = None,
                 events=None) -> torch.Tensor:
        layout = self.cache.layout
        if tuple(query.shape) != self.shape:
            raise ValueError(f"query must have shape {list(self.shape)}")
        if query.dtype != self.cache.act_dtype or query.device != self.cache.device:
            raise ValueError("query and cache must have the same dtype and device")
        if not 0 <= layer < layout.num_layers:
            raise IndexError("layer is out of range")
        if not _aligned_prefill_rows(query, self._row_align):
            query = query.contiguous()
        if out is None:
            out = torch.empty(self.shape, dtype=query.dtype, device=query.device)
        elif (tuple(out.shape) != self.shape or out.dtype != query.dtype or out.device != query.device
              or not _aligned_prefill_rows(out, 8 if self.path == "mfma_grouped" else 4)):
            raise ValueError("out must match the query shape, dtype and device with aligned rows")
        kc, vc = self.cache.k[layer], self.cache.v[layer]
        a = self._args
        a.query = query.data_ptr()
        a.q_stride_b, a.q_stride_h, a.q_stride_t = query.stride(0), query.stride(1), query.stride(2)
        a.k_cache, a.v_cache = kc.data_ptr(), vc.data_ptr()
        a.k_stride_block, a.k_stride_token, a.k_stride_head = kc.stride()[:3]
        a.v_stride_block, a.v_stride_token, a.v_stride_head = vc.stride()[:3]
        a.out = out.data_ptr()
        a.out_stride_b, a.out_stride_h, a.out_stride_t = out.stride(0), out.stride(1), out.stride(2)
        if self.cache.fp8:
            ks, vs = self.cache.k_scale[layer], self.cache.v_scale[layer]
            a.k_scale, a.v_scale = ks.data_ptr(), vs.data_ptr()
            a.scale_stride_block, a.scale_stride_head = ks.stride(0), ks.stride(1)
        for i in range(2):
            a.events[i] = events[i] if events is not None else None
        with torch.cuda.device(query.device):
            stream = torch.cuda.current_stream(query.device).cuda_stream
            status = self._lib.ikl_paged_prefill_attention(ctypes.byref(a), ctypes.c_void_p(stream))
        _lib.check(status, "paged prefill attention")
        return out


def paged_prefill_attention_hip(
    query: torch.Tensor,
    cache,
    block_tables,
    query_starts,
    context_lens,
    *,
    scale: float | None = None,
    layer: int = 0,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """Causal attention of a ragged prefill batch over the paged cache.

    Arguments, checks (same order and messages) and result of
    ``paged_prefill_attention_sdpa`` (attention.py:230-321): ``query`` is
    ``[B, H, T, D]``; row ``t`` of request ``b`` sits at position
    ``query_starts[b] + t`` and attends positions up to its own inside
    ``[0, context_lens[b])``; rows past ``context_lens[b] - query_starts[b]``
    are padding and receive the value at position 0, as the reference's mask
    leaves them. The cache must already hold the chunk's keys and values.
    One HIP kernel reads K/V straight from the paged cache — no gathered
    copy of the prefix is made.
    """
    if query.ndim != 4:
        raise ValueError("query must be [B,H,T,D]")
    batch, num_heads, query_width, head_dim = query.shape
    layout = cache.layout
    if head_dim != layout.head_dim:
        raise ValueError("query head_dim does not match cache")
    if num_heads % layout.num_kv_heads != 0:
        raise ValueError("num_heads must be divisible by num_kv_heads")
    if query.device != cache.device:
        raise ValueError("query and cache must be on the same device")
    starts, ends = _prefill_ranges(query_starts, context_lens, batch, query_width)
    if not 0 <= layer < layout.num_layers:
        raise IndexError("layer is out of range")
    prepared = PreparedPagedPrefill(cache, block_tables, starts, ends, num_heads=num_heads,
                                    query_width=query_width, scale=scale)
    return prepared(query, layer, out=out)


# Names of the reference's operators, bound to the same HIP functions.
paged_decode_attention_triton = paged_decode_attention_hip
paged_decode_attention_triton_grouped = paged_decode_attention_hip_grouped
append_kv_triton = append_kv_hip
triton_available = hip_available
triton_append_available = hip_append_available
