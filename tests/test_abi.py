"""The C-ABI library loads on the CPU host and exports every symbol that
include/ikl_paged.h declares; its pure host functions (path selection,
workspace and partition planning) behave as documented. No kernels run."""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from inferkernellab_amd import _lib, ops

HEADER = Path(__file__).resolve().parents[1] / "include" / "ikl_paged.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(ikl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_what_python_binds():
    assert _declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.ikl_version().decode().startswith("ikl_paged")


def test_struct_layouts_match_header_field_order():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    for struct_name, cls in (("ikl_append_args", _lib.AppendArgs),
                             ("ikl_paged_attention_args", _lib.PagedAttentionArgs),
                             ("ikl_rope_append_args", _lib.RopeAppendArgs),
                             ("ikl_paged_prefill_args", _lib.PagedPrefillArgs),
                             ("ikl_launch_config", _lib.LaunchConfig)):
        body = re.search(r"typedef struct %s \{(.*?)\}" % struct_name, text, flags=re.S).group(1)
        fields = []
        for decl in body.split(";"):
            decl = decl.strip()
            if not decl:
                continue
            names = decl.split(None, 1)[1] if not decl.startswith("const") else decl.split(None, 2)[2]
            for name in names.split(","):
                fields.append(re.sub(r"[\s*]|\[\d+\]", "", name))
        assert fields == [f[0] for f in cls._fields_], struct_name


def _args(**kw):
    a = _lib.PagedAttentionArgs()
    a.batch, a.num_heads, a.num_kv_heads, a.head_dim = 32, 32, 8, 128
    a.block_size, a.num_blocks, a.table_width = 16, 20000, 513
    a.table_type = a.lens_type = _lib.IKL_I32
    a.dtype = _lib.IKL_BF16
    a.path = -1
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_partition_planning_for_the_gqa_decode_shape():
    lib = _lib.load()
    a = _args(partition_size=512, max_context_len=8192)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 512
    ws = lib.ikl_paged_attention_workspace_size(ctypes.byref(a))
    rows = 32 * 32 * 16
    assert ws >= rows * 128 * 4 + rows * 4
    # never split
    a = _args(partition_size=-1, max_context_len=8192)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 0
    assert lib.ikl_paged_attention_workspace_size(ctypes.byref(a)) == 0
    # automatic on the scalar family: 512 tokens, halved (down to 128) while
    # there are fewer than 1024 waves (one per SIMD of 256 CUs); when a
    # request then needs at most 4 partitions they become the waves of one
    # workgroup and nothing is split
    a = _args(partition_size=0, max_context_len=512, batch=16, num_kv_heads=32, dtype=_lib.IKL_F32)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 0  # 512 units x 2 waves, no split
    assert ops.launch_config(a)["num_warps"] == 2
    a = _args(partition_size=0, max_context_len=512, batch=4, num_kv_heads=32, dtype=_lib.IKL_F32)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 0  # 128 x 4 covers 512
    assert ops.launch_config(a)["num_warps"] == 4
    a = _args(partition_size=0, max_context_len=8192, batch=16, num_kv_heads=32, dtype=_lib.IKL_F32)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 512  # 16 partitions stay split
    assert ops.launch_config(a)["num_warps"] == 1
    # an explicit partition size keeps one-wave workgroups
    a = _args(partition_size=256, max_context_len=8192, batch=16, num_kv_heads=32, dtype=_lib.IKL_F32)
    assert ops.launch_config(a)["num_warps"] == 1


def test_balanced_split_planning_on_the_mfma_family():
    """partition_size=0 on bf16 GQA: the balanced split, unit-parallel (the
    8 units of a request are the 8 waves of each workgroup, walking the same
    request tiles), over W resident workgroups (runs); the workspace holds
    (requests x unit groups + W) slots of 8 units x group_size rows."""
    lib = _lib.load()
    a = _args(partition_size=0, max_context_len=8192)
    part = lib.ikl_paged_attention_partition_size(ctypes.byref(a))
    ws = lib.ikl_paged_attention_workspace_size(ctypes.byref(a))
    units, group, tiles, uw = 32 * 8, 4, 32 * 8 * 512, 8
    seq = tiles // uw  # (request, unit group, tile) entries
    assert part > 0 and part % 16 == 0
    runs = -(-seq // (part // 16))  # lower bound on W from the longest run
    assert ws >= (units // uw + runs) * uw * group * (128 * 4 + 4)
    cfg = ops.launch_config(a)
    assert (cfg["split"], cfg["num_warps"]) == ("balanced", uw)
    if not torch.cuda.is_available():  # planning without a device assumes 256 CUs x 8 waves
        assert cfg["workgroups"] == 256
        assert part == 16 * (seq // 256)
        rows = (units // uw + 256) * uw * group
        assert ws == -(-(rows * 128 * 4) // 256) * 256 + rows * 4


def test_split_choice_by_batch_size_on_the_mfma_family():
    """Automatic on the MFMA family: the balanced split above 32768 tiles at
    the longest context, fixed partitions below it (512 tokens, halved down
    to 128 while fewer than 160 workgroups); -2 asks for the balanced split
    at any size and only on the MFMA family."""
    lib = _lib.load()
    # B32 x 8 kv heads x 8192 tokens: 131072 tiles -> balanced (partition = a wave's run)
    a = _args(partition_size=0, max_context_len=8192)
    assert ops.launch_config(a)["split"] == "balanced"
    # B32 x 8 x 1024: 16384 tiles, 256 units (a workgroup per CU of 256) -> unsplit
    a = _args(partition_size=0, max_context_len=1024)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 0
    assert ops.launch_config(a)["split"] == "none"
    # B16 x 8 x 1024: 128 units -> fixed 512-token partitions (256 workgroups)
    a = _args(partition_size=0, max_context_len=1024, batch=16)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 512
    # B2 x 8 x 1024: 16 units -> 32, 64, then 128 workgroups -> 128-token partitions
    a = _args(partition_size=0, max_context_len=1024, batch=2)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 128
    # B16 x 4 x 544 (the Llama decode shape): 128 workgroups at 512, 192 at 256 -> 256
    a = _args(partition_size=0, max_context_len=544, batch=16, num_heads=16, num_kv_heads=4)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 256
    # B32 x 512: one 512-token partition covers the context -> no split
    a = _args(partition_size=0, max_context_len=512)
    assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == 0
    # 32-head units: balanced once 512-token partitions exceed one round of
    # resident workgroups (512 without a device: 256 CUs x 2 four-wave groups)
    if not torch.cuda.is_available():
        a = _args(partition_size=0, max_context_len=4096, batch=64, num_kv_heads=1)  # 512 workgroups
        assert ops.launch_config(a)["split"] == "fixed_partitions"
        a = _args(partition_size=0, max_context_len=4096, batch=80, num_kv_heads=1)  # 640
        assert ops.launch_config(a)["split"] == "balanced"
        a = _args(partition_size=0, max_context_len=2048, batch=96, num_kv_heads=1)  # 384
        assert ops.launch_config(a)["split"] == "fixed_partitions"
        # their fixed partitions: the longest of 128-1024 tokens that still
        # launches a workgroup per CU (two over the FP8 cache), on 4-wave
        # workgroups; over the FP8 cache, 1024-token partitions with a
        # workgroup per CU, all resident (256 without a device: one 8-wave
        # group per CU), run on 8 waves instead
        fp8 = {"cache_dtype": _lib.IKL_FP8_E4M3, "k_scale": 0x60000, "v_scale": 0x70000}
        for batch, ctx, kw, want, waves in ((64, 4096, {}, 1024, 4), (16, 4096, {}, 256, 4),
                                            (64, 2048, {}, 512, 4), (8, 512, {}, 128, 4),
                                            (64, 4096, fp8, 1024, 8), (32, 8192, fp8, 1024, 8),
                                            (16, 4096, fp8, 128, 4), (64, 2048, fp8, 256, 4)):
            a = _args(partition_size=0, max_context_len=ctx, batch=batch, num_kv_heads=1, **kw)
            assert lib.ikl_paged_attention_partition_size(ctypes.byref(a)) == want, (batch, ctx, kw)
            cfg = ops.launch_config(a)
            assert (cfg["split"], cfg["num_warps"]) == ("fixed_partitions", waves), (batch, ctx, kw)
        # an explicit partition size keeps 4-wave workgroups
        a = _args(partition_size=1024, max_context_len=4096, batch=64, num_kv_heads=1, **fp8)
        assert ops.launch_config(a)["num_warps"] == 4
    # -2: the balanced split on a small batch too
    a = _args(partition_size=-2, max_context_len=1024, batch=2)
    part = lib.ikl_paged_attention_partition_size(ctypes.byref(a))
    assert part > 0 and part % 16 == 0 and ops.launch_config(a)["split"] == "balanced"
    # 1024 tiles at the longest context, the 8 units of a request in one
    # workgroup: 128 (request, tile) entries, at least 4 per run: 32 runs of 4
    assert part == 64 and ops.launch_config(a)["workgroups"] == 32
    # 32-head units run 4-wave workgroups, at least 4 tiles per wave
    a = _args(partition_size=-2, max_context_len=4096, batch=64, num_kv_heads=1)
    cfg = ops.launch_config(a)
    assert (cfg["split"], cfg["num_warps"]) == ("balanced", 4)
    if not torch.cuda.is_available():  # 256 CUs x 1 workgroup of 4 waves
        assert cfg["workgroups"] == 256
    # -2 where the MFMA family does not run (fp32) is refused
    a = _args(partition_size=-2, max_context_len=1024, dtype=_lib.IKL_F32)
    assert lib.ikl_paged_attention_workspace_size(ctypes.byref(a)) == _lib.IKL_EUNSUPPORTED
    assert "balanced split" in _lib.last_error()


def test_invalid_arguments_report_errors():
    lib = _lib.load()
    a = _args(num_heads=30)
    assert lib.ikl_paged_attention_workspace_size(ctypes.byref(a)) == _lib.IKL_EINVAL
    assert "divisible" in _lib.last_error()
    a = _args(head_dim=200)
    assert lib.ikl_paged_attention_workspace_size(ctypes.byref(a)) == _lib.IKL_EUNSUPPORTED
    a = _args(partition_size=100)
    assert lib.ikl_paged_attention_workspace_size(ctypes.byref(a)) == _lib.IKL_EINVAL
    assert "multiple of 64" in _lib.last_error()


@pytest.mark.parametrize(
    ("dtype", "head_dim", "block_size", "table_width", "heads_per_kv", "expected"),
    [
        # the cases of tests/test_attention.py:22-42 (head_dim 64, block 16)
        (torch.float16, 64, 16, 8, 4, "mfma_grouped"),
        (torch.bfloat16, 64, 16, 16, 32, "mfma_grouped"),
        (torch.float16, 64, 16, 17, 32, "mfma_grouped"),
        (torch.float32, 64, 16, 8, 32, "scalar_grouped"),
        (torch.float16, 64, 16, 8, 1, "mha_fallback"),
        # shapes the MFMA tiles cannot take
        (torch.bfloat16, 16, 16, 8, 4, "scalar_grouped"),
        (torch.bfloat16, 128, 8, 8, 4, "scalar_grouped"),
        (torch.bfloat16, 128, 32, 8, 4, "mfma_grouped"),
        (torch.float16, 80, 16, 8, 4, "scalar_grouped"),
    ],
)
def test_grouped_path_truth_table_matches_library(dtype, head_dim, block_size, table_width,
                                                  heads_per_kv, expected):
    """Same role as tests/test_attention.py:22-42, answered with this
    library's families; the Python selector and the C one agree."""
    got = ops.paged_decode_grouped_path(dtype=dtype, head_dim=head_dim, table_width=table_width,
                                        heads_per_kv=heads_per_kv, query_group_size=8,
                                        block_size=block_size)
    assert got == expected
    code = _lib.load().ikl_paged_attention_path(ops._DTYPES[dtype], head_dim, block_size, table_width,
                                                heads_per_kv, 8)
    assert ops._PATH_NAMES[code] == expected


def test_operators_fail_loudly_without_a_gpu():
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from inferkernellab_amd import PagedKVCache

    cache = PagedKVCache(4, 4, 1, 16, dtype=torch.float16)
    key = torch.zeros(1, 1, 16, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="unavailable"):
        ops.append_kv_hip(key, key, cache, torch.zeros(1, dtype=torch.int32))
    assert not ops.hip_available()
    assert ops.triton_available is ops.hip_available


def test_small_mha_launches_take_the_mfma_family():
    """One query head per KV head, path left to the library: at most 32 MiB
    of K/V at the longest context runs on the MFMA family (latency-bound
    launches), more stays on the per-head kernel; fp32 always does."""
    lib = _lib.load()
    small = _args(dtype=_lib.IKL_F16, num_heads=32, num_kv_heads=32, head_dim=64, batch=4, max_context_len=128)
    assert ops.launch_config(small)["path"] == "mfma_grouped"  # 4 x 32 x 128 x 64 x 2 x 2 B = 4 MiB
    edge = _args(dtype=_lib.IKL_BF16, num_heads=32, num_kv_heads=32, head_dim=128, batch=4, max_context_len=512)
    assert ops.launch_config(edge)["path"] == "mfma_grouped"  # exactly 32 MiB
    big = _args(dtype=_lib.IKL_F16, num_heads=32, num_kv_heads=32, head_dim=64, batch=16, max_context_len=2048)
    assert ops.launch_config(big)["path"] == "mha_fallback"  # 256 MiB
    f32 = _args(dtype=_lib.IKL_F32, num_heads=32, num_kv_heads=32, head_dim=64, batch=1, max_context_len=128)
    assert ops.launch_config(f32)["path"] == "mha_fallback"
    # an explicit per-head path is kept
    small.path = _lib.IKL_PATH_MHA_FALLBACK
    assert ops.launch_config(small)["path"] == "mha_fallback"
    assert lib.ikl_paged_attention_path(_lib.IKL_F16, 64, 16, 8, 1, 0) == _lib.IKL_PATH_MHA_FALLBACK


@pytest.mark.parametrize(
    ("dtype", "heads_per_kv", "partition", "expect"),
    [
        # the balanced split runs unit-parallel: 8 units per request -> 8-wave workgroups
        (_lib.IKL_BF16, 4, 0, ("mfma_grouped", 16, 8, "balanced")),
        (_lib.IKL_BF16, 4, 512, ("mfma_grouped", 16, 4, "fixed_partitions")),
        (_lib.IKL_BF16, 4, -1, ("mfma_grouped", 16, 4, "none")),
        (_lib.IKL_F32, 4, 0, ("scalar_grouped", None, 1, "fixed_partitions")),
        (_lib.IKL_F16, 1, 0, ("mha_fallback", None, 1, "fixed_partitions")),
        # -2 asks for the balanced split, which moves MHA to the MFMA family
        (_lib.IKL_F16, 1, -2, ("mfma_grouped", 16, 8, "balanced")),
        (_lib.IKL_BF16, 1, -2, ("mfma_grouped", 16, 8, "balanced")),
    ],
)
def test_launch_config_reports_the_resolved_launch(dtype, heads_per_kv, partition, expect):
    """ikl_paged_attention_launch_config: the counterpart of the autotune
    reporters (triton_ops.py:17-53), computed without a launch."""
    lib = _lib.load()
    a = _args(dtype=dtype, num_heads=8 * heads_per_kv, num_kv_heads=8, partition_size=partition,
              max_context_len=8192)
    out = _lib.LaunchConfig()
    out.struct_size = ctypes.sizeof(out)
    assert lib.ikl_paged_attention_launch_config(ctypes.byref(a), ctypes.byref(out)) == 0
    cfg = ops.launch_config(a)
    path, tile, waves, split = expect
    assert (cfg["path"], cfg["num_warps"], cfg["split"]) == (path, waves, split)
    if tile is not None:
        assert cfg["block_n"] == tile
    assert 0 < cfg["block_n"] <= 64 and cfg["num_stages"] >= 2 and cfg["workgroups"] > 0
    if split == "fixed_partitions" and partition > 0:
        assert cfg["workgroups"] == (8192 // partition) * 8 * a.batch
    assert lib.ikl_paged_attention_launch_config(ctypes.byref(a), None) == _lib.IKL_EINVAL


def test_launch_config_honours_the_callers_struct_size():
    """ikl_launch_config carries its size: the library rejects a struct
    shorter than the first version and never writes past the size a caller
    declares (a caller built against an older, shorter header)."""
    lib = _lib.load()
    assert lib.ikl_abi_version() == _lib.IKL_ABI_VERSION
    a = _args(partition_size=512, max_context_len=8192)
    out = _lib.LaunchConfig()
    out.struct_size = 0
    assert lib.ikl_paged_attention_launch_config(ctypes.byref(a), ctypes.byref(out)) == _lib.IKL_EINVAL
    assert "struct_size" in lib.ikl_last_error().decode()
    min_bytes = _lib.LaunchConfig.group_size.offset
    out.struct_size = min_bytes - 1
    assert lib.ikl_paged_attention_launch_config(ctypes.byref(a), ctypes.byref(out)) == _lib.IKL_EINVAL
    # the first version's size: filled up to workgroups, group_size untouched
    out.struct_size = min_bytes
    out.group_size = -7
    assert lib.ikl_paged_attention_launch_config(ctypes.byref(a), ctypes.byref(out)) == 0
    assert out.struct_size == min_bytes and out.workgroups > 0 and out.group_size == -7
    out.struct_size = ctypes.sizeof(out)
    assert lib.ikl_paged_attention_launch_config(ctypes.byref(a), ctypes.byref(out)) == 0
    assert out.group_size == 4
    header = Path(__file__).resolve().parents[1] / "include" / "ikl_paged.h"
    text = header.read_text()
    assert f"#define IKL_LAUNCH_CONFIG_MIN_BYTES {min_bytes}" in text
    assert f"#define IKL_ABI_VERSION {_lib.IKL_ABI_VERSION}" in text


def test_autotune_reporters_are_none_before_a_launch():
    import importlib

    fresh = importlib.reload(ops)
    assert fresh.paged_decode_autotune_config() is None
    assert fresh.paged_decode_grouped_autotune_config() is None
    assert fresh.paged_decode_grouped_dot_autotune_config() is None


def test_grouped_reporter_covers_the_matrix_core_path():
    """The reference's callers ask paged_decode_grouped_autotune_config() for
    every grouped path not named "tensorcore_short_context" (hf_benchmark.py:
    942-945): it reports the last grouped launch of either family."""
    import importlib

    fresh = importlib.reload(ops)
    fresh._record_launch(_args())  # bf16 GQA 32/8: matrix cores
    dot = fresh.paged_decode_grouped_dot_autotune_config()
    assert dot is not None and fresh.paged_decode_grouped_autotune_config() == dot
    fresh._record_launch(_args(dtype=_lib.IKL_F32))  # fp32: the VALU grouped kernel
    scalar = fresh.paged_decode_grouped_autotune_config()
    assert scalar is not None and scalar != dot and scalar["num_warps"] == 1
    assert fresh.paged_decode_grouped_dot_autotune_config() == dot
    assert fresh.paged_decode_autotune_config() is None


def _doc_structures(path: Path) -> dict:
    """ctypes.Structure classes of the ```python blocks of a markdown file:
    name -> [(field, ctypes type), ...] (parsed, not executed)."""
    import ast

    text = path.read_text()
    found = {}
    for block in re.findall(r"```python\n(.*?)```", text, flags=re.S):
        for node in ast.walk(ast.parse(block)):
            if not isinstance(node, ast.ClassDef):
                continue
            for stmt in node.body:
                if isinstance(stmt, ast.Assign) and getattr(stmt.targets[0], "id", "") == "_fields_":
                    fields = []
                    for elt in stmt.value.elts:
                        name, typ = elt.elts
                        assert isinstance(typ, ast.Attribute) and typ.value.id == "ctypes"
                        fields.append((name.value, getattr(ctypes, typ.attr)))
                    found[node.name] = fields
    return found


def test_integration_stub_declares_every_struct_field():
    """The binding INTEGRATION.md gives maintainers matches _lib.py (and so
    the header) field for field, type for type."""
    doc = _doc_structures(Path(__file__).resolve().parents[1] / "INTEGRATION.md")
    assert "AppendArgs" in doc
    for name, fields in doc.items():
        cls = getattr(_lib, name)
        assert fields == [(f, t) for f, t in cls._fields_], name

        class Doc(ctypes.Structure):
            _fields_ = fields

        assert ctypes.sizeof(Doc) == ctypes.sizeof(cls), name


def test_rope_append_rejects_bad_arguments_without_a_gpu():
    """ikl_rope_append_kv validates before launching: errors, not launches."""
    lib = _lib.load()
    a = _lib.RopeAppendArgs()
    assert lib.ikl_rope_append_kv(None, None) == _lib.IKL_EINVAL
    a.num_tokens = 4
    assert lib.ikl_rope_append_kv(ctypes.byref(a), None) == _lib.IKL_EINVAL  # zero dims
    a.num_blocks, a.block_size, a.num_kv_heads, a.head_dim, a.dtype = 8, 16, 2, 128, _lib.IKL_BF16
    assert lib.ikl_rope_append_kv(ctypes.byref(a), None) == _lib.IKL_EINVAL
    assert "null tensor" in _lib.last_error()
    a.num_tokens = 0
    assert lib.ikl_rope_append_kv(ctypes.byref(a), None) == _lib.IKL_OK  # nothing to do


@pytest.mark.parametrize(
    ("dtype", "head_dim", "block_size", "expected"),
    [
        (torch.bfloat16, 128, 16, "mfma_grouped"),
        (torch.float16, 96, 48, "mfma_grouped"),
        (torch.bfloat16, 32, 32, "mfma_grouped"),
        (torch.float32, 128, 16, "scalar_grouped"),
        (torch.bfloat16, 128, 8, "scalar_grouped"),
        (torch.float16, 256, 16, "scalar_grouped"),
        (torch.bfloat16, 80, 16, "scalar_grouped"),
    ],
)
def test_prefill_path_truth_table_matches_library(dtype, head_dim, block_size, expected):
    assert ops.paged_prefill_path(dtype=dtype, head_dim=head_dim, block_size=block_size) == expected
    code = _lib.load().ikl_paged_prefill_path(ops._DTYPES[dtype], head_dim, block_size)
    assert ops._PATH_NAMES[code] == expected


def _prefill_args(**kw):
    a = _lib.PagedPrefillArgs()
    a.batch, a.query_width, a.num_heads, a.num_kv_heads, a.head_dim = 2, 64, 32, 8, 128
    a.block_size, a.num_blocks, a.table_width = 16, 100, 8
    a.table_type = a.lens_type = _lib.IKL_I32
    a.dtype = _lib.IKL_BF16
    a.path = -1
    a.k_stride_block = a.v_stride_block = 16 * 8 * 128
    a.k_stride_token = a.v_stride_token = 8 * 128
    a.k_stride_head = a.v_stride_head = 128
    for k, v in kw.items():
        setattr(a, k, v)
    return a


def test_prefill_entry_rejects_bad_arguments_before_any_launch():
    """Every check below returns before the library touches a device."""
    lib = _lib.load()
    assert lib.ikl_paged_prefill_attention(None, None) == _lib.IKL_EINVAL
    a = _prefill_args(num_heads=30)
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EINVAL
    assert "sizes must be positive" in _lib.last_error() or "divisible" in _lib.last_error()
    a = _prefill_args(query_width=0)
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EINVAL
    assert "positive" in _lib.last_error()
    a = _prefill_args()  # NULL tensors
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EINVAL
    assert "NULL" in _lib.last_error()
    fake = 1 << 20  # never dereferenced: the checks below fail first
    ptrs = dict(query=fake, k_cache=fake, v_cache=fake, block_tables=fake, query_starts=fake,
                context_lens=fake, out=fake)
    a = _prefill_args(dtype=_lib.IKL_F32, head_dim=512, **ptrs)
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EUNSUPPORTED
    a = _prefill_args(dtype=_lib.IKL_F32, path=_lib.IKL_PATH_MFMA_GROUPED, **ptrs)
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EUNSUPPORTED
    assert "no MFMA kernel" in _lib.last_error()
    a = _prefill_args(path=7, **ptrs)
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EINVAL
    a = _prefill_args(q_stride_t=100, **ptrs)  # 200-byte rows: not 16-byte aligned
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EINVAL
    assert "misaligned" in _lib.last_error()
    a = _prefill_args(k_stride_token=64, **ptrs)  # token rows overlap
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EINVAL
    assert "token strides" in _lib.last_error()
    a = _prefill_args(table_width=1 << 27, **ptrs)  # positions past 2^31
    assert lib.ikl_paged_prefill_attention(ctypes.byref(a), None) == _lib.IKL_EINVAL
    assert "2^31" in _lib.last_error()


@pytest.mark.parametrize(
    ("shape", "tables", "starts", "ends", "layer", "error", "message"),
    [
        ((2, 4, 8), [[0], [1]], [0, 0], [4, 4], 0, ValueError, r"query must be \[B,H,T,D\]"),
        ((2, 4, 8, 32), [[0], [1]], [0, 0], [4, 4], 0, ValueError, "head_dim does not match"),
        ((2, 3, 8, 16), [[0], [1]], [0, 0], [4, 4], 0, ValueError, "divisible by num_kv_heads"),
        ((2, 4, 8, 16), [[0], [1]], [0], [4, 4], 0, ValueError, "one entry per query batch"),
        ((2, 4, 8, 16), [[0], [1]], [0, 4], [4, 4], 0, ValueError, "non-empty and non-negative"),
        ((2, 4, 8, 16), [[0], [1]], [-1, 0], [4, 4], 0, ValueError, "non-empty and non-negative"),
        ((2, 4, 8, 16), [[0, 1], [2, 3]], [0, 0], [9, 4], 0, ValueError, "query width is smaller"),
        ((2, 4, 8, 16), [[0], [1]], [0, 0], [4, 4], 2, IndexError, "layer is out of range"),
        ((2, 4, 8, 16), [[0]], [0, 0], [4, 4], 0, ValueError, "one row per query batch"),
        ((2, 4, 8, 16), [[0], [1]], [0, 0], [5, 4], 0, ValueError, "exceeds block table capacity"),
        ((2, 4, 8, 16), [[0], [1]], [0, 0], [4, 4], 0, RuntimeError, "unavailable"),
    ],
)
def test_prefill_operator_checks_in_the_reference_order(shape, tables, starts, ends, layer, error, message):
    """attention.py:252-288's checks (same order, same messages); a valid
    call on a host without a GPU fails loudly instead of computing."""
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    from inferkernellab_amd import PagedKVCache

    cache = PagedKVCache(8, 4, 2, 16, dtype=torch.bfloat16)
    q = torch.zeros(shape, dtype=torch.bfloat16)
    with pytest.raises(error, match=message):
        ops.paged_prefill_attention_hip(q, cache, tables, starts, ends, layer=layer)


def _append_args(**kw):
    a = _lib.AppendArgs()
    a.key, a.value, a.slots, a.k_cache, a.v_cache = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000
    a.key_stride_t, a.key_stride_h = 8 * 128, 128
    a.value_stride_t, a.value_stride_h = 8 * 128, 128
    a.k_stride_block, a.k_stride_token, a.k_stride_head = 16 * 8 * 128, 8 * 128, 128
    a.v_stride_block, a.v_stride_token, a.v_stride_head = 16 * 8 * 128, 8 * 128, 128
    a.num_tokens, a.num_blocks, a.block_size, a.num_kv_heads, a.head_dim = 32, 20000, 16, 8, 128
    a.slot_type, a.dtype = _lib.IKL_I32, _lib.IKL_BF16
    for k, v in kw.items():
        setattr(a, k, v)
    return a


@pytest.mark.parametrize(
    "attn_kw,append_kw,expect",
    [
        ({}, {}, 1),                                   # balanced split + 16-byte rows: fused
        ({"partition_size": 512}, {}, 1),              # fixed partitions split too
        ({"partition_size": -1}, {}, 0),               # no reduce kernel: separate append
        # FP8 append: quantised on the reduce as well, when its rows are in the query dtype
        ({}, {"cache_dtype": _lib.IKL_FP8_E4M3, "k_scale": 0x60000, "v_scale": 0x70000}, 1),
        ({}, {"cache_dtype": _lib.IKL_FP8_E4M3, "k_scale": 0x60000, "v_scale": 0x70000,
              "dtype": _lib.IKL_F16}, 0),
        ({}, {"cache_dtype": _lib.IKL_FP8_E4M3}, _lib.IKL_EINVAL),  # no scale tensors
        ({}, {"key": 0x10008}, 0),                     # rows only 8-byte aligned: separate
        ({}, {"num_tokens": 0}, 0),                    # nothing to append
        ({}, {"key": 0}, _lib.IKL_EINVAL),             # invalid append
        ({"num_heads": 7}, {}, _lib.IKL_EINVAL),       # invalid attention
    ],
)
def test_decode_step_fuses_the_append_into_the_reduce(attn_kw, append_kw, expect):
    """ikl_paged_decode_step_fused: planning only, no GPU."""
    lib = _lib.load()
    a = _args(max_context_len=8192, **attn_kw)
    assert lib.ikl_paged_decode_step_fused(ctypes.byref(a), ctypes.byref(_append_args(**append_kw))) == expect


def test_decode_step_on_a_folded_plan_appends_with_its_own_launch():
    """MHA fp16 B16 x 512 on the VALU family: the attention folds each
    request's two partitions into one 2-wave workgroup and needs no
    workspace; the step runs it and then the append kernel, whatever
    workspace it is given (keeping the split for the reduce to carry the
    append measured slower)."""
    lib = _lib.load()
    a = _args(dtype=_lib.IKL_F16, batch=16, num_heads=32, num_kv_heads=32, max_context_len=512)
    cfg = ops.launch_config(a)
    assert (cfg["path"], cfg["num_warps"], cfg["split"]) == ("mha_fallback", 2, "none")
    assert lib.ikl_paged_attention_workspace_size(ctypes.byref(a)) == 0
    app = _append_args(dtype=_lib.IKL_F16, num_kv_heads=32, num_tokens=16, key_stride_t=32 * 128,
                       value_stride_t=32 * 128)
    assert lib.ikl_paged_decode_step_workspace_size(ctypes.byref(a), ctypes.byref(app)) == 0
    assert lib.ikl_paged_decode_step_fused(ctypes.byref(a), ctypes.byref(app)) == 0
    a.workspace, a.workspace_bytes = 0x100000, 1 << 20
    assert lib.ikl_paged_decode_step_fused(ctypes.byref(a), ctypes.byref(app)) == 0
    # a split attention: the step's workspace is the attention's, and the reduce carries the append
    b = _args(max_context_len=8192)
    need = lib.ikl_paged_attention_workspace_size(ctypes.byref(b))
    assert need > 0 and lib.ikl_paged_decode_step_workspace_size(ctypes.byref(b), ctypes.byref(_append_args())) == need
    b.workspace, b.workspace_bytes = 0x100000, need
    assert lib.ikl_paged_decode_step_fused(ctypes.byref(b), ctypes.byref(_append_args())) == 1
    a.workspace, a.workspace_bytes = 0, 0
    assert lib.ikl_paged_decode_step_workspace_size(ctypes.byref(a), ctypes.byref(_append_args(num_tokens=0))) == 0
    assert lib.ikl_paged_decode_step_workspace_size(ctypes.byref(a), ctypes.byref(_append_args(key=0))) == \
        _lib.IKL_EINVAL


def test_noalloc_rejects_a_split_beyond_its_scratch_without_a_gpu():
    """A launch whose split workspace exceeds the 16 MiB scratch is refused
    before anything is touched or enqueued."""
    lib = _lib.load()
    a = _args(batch=64, partition_size=64, max_context_len=8192, table_width=512)
    assert lib.ikl_paged_attention_workspace_size(ctypes.byref(a)) > (16 << 20)
    assert lib.ikl_paged_attention_noalloc(ctypes.byref(a), None) == _lib.IKL_EWORKSPACE
    assert "scratch" in _lib.last_error()


@pytest.mark.parametrize(
    ("dtype", "table_width", "heads_per_kv", "reference_answer"),
    [  # tests/test_attention.py:22-42 verbatim (head_dim 64, query_group_size 8)
        (torch.float16, 8, 4, "tensorcore_short_context"),
        (torch.bfloat16, 16, 32, "tensorcore_short_context"),
        (torch.float16, 17, 32, "scalar_grouped"),
        (torch.float32, 8, 32, "scalar_grouped"),
        (torch.float16, 8, 1, "mha_fallback"),
    ],
)
def test_reference_truth_table_under_the_name_mapping(dtype, table_width, heads_per_kv, reference_answer):
    """The reference's truth table read through REFERENCE_PATH_NAMES: every
    row agrees except table_width 17, where the reference's tensor-core
    kernel stops (W <= 16) and this library's matrix-core kernel does not."""
    got = ops.paged_decode_grouped_path(dtype=dtype, head_dim=64, table_width=table_width,
                                        heads_per_kv=heads_per_kv, query_group_size=8)
    mapped = ops.REFERENCE_PATH_NAMES[got]
    if table_width > 16 and dtype in (torch.float16, torch.bfloat16) and heads_per_kv > 1:
        assert (reference_answer, mapped) == ("scalar_grouped", "tensorcore_short_context")
    else:
        assert mapped == reference_answer
