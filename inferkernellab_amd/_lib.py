"""ctypes binding of libikl_paged.so (declared in include/ikl_paged.h).

The library is loaded from this package directory only; when it is missing
or cannot be loaded every operator raises instead of computing anything on
another path. ``torch`` is imported first so the HIP runtime the library
links against (soname libamdhip64.so.7) resolves to the copy torch already
loaded.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (loads the HIP runtime before the library)

LIB_PATH = Path(__file__).resolve().parent / "libikl_paged.so"

# enum ikl_dtype / ikl_index_type / ikl_status / ikl_attention_path
IKL_F16, IKL_BF16, IKL_F32, IKL_FP8_E4M3 = 0, 1, 2, 3
IKL_I32, IKL_I64 = 0, 1
IKL_OK, IKL_EINVAL, IKL_EUNSUPPORTED, IKL_ELAUNCH, IKL_EWORKSPACE = 0, -1, -2, -3, -4
IKL_PATH_MHA_FALLBACK, IKL_PATH_SCALAR_GROUPED, IKL_PATH_MFMA_GROUPED = 0, 1, 2
# IKL_ABI_VERSION of the header these mirrors follow; load() refuses a
# library that reports another
IKL_ABI_VERSION = 3

EXPORTED_SYMBOLS = (
    "ikl_last_error",
    "ikl_version",
    "ikl_abi_version",
    "ikl_append_kv",
    "ikl_paged_attention_workspace_size",
    "ikl_paged_attention_partition_size",
    "ikl_paged_attention",
    "ikl_paged_attention_path",
    "ikl_paged_attention_launch_config",
    "ikl_rope_append_kv",
    "ikl_paged_prefill_attention",
    "ikl_paged_prefill_path",
    "ikl_paged_decode_step",
    "ikl_paged_decode_step_fused",
    "ikl_paged_decode_step_workspace_size",
    "ikl_paged_attention_noalloc",
    "ikl_hbm_read_probe",
)

_c_i64 = ctypes.c_int64
_c_i32 = ctypes.c_int32
_c_ptr = ctypes.c_void_p


class AppendArgs(ctypes.Structure):
    """Mirror of ikl_append_args."""

    _fields_ = [
        ("key", _c_ptr),
        ("value", _c_ptr),
        ("key_stride_t", _c_i64),
        ("key_stride_h", _c_i64),
        ("value_stride_t", _c_i64),
        ("value_stride_h", _c_i64),
        ("slots", _c_ptr),
        ("slot_type", _c_i32),
        ("k_cache", _c_ptr),
        ("v_cache", _c_ptr),
        ("k_stride_block", _c_i64),
        ("k_stride_token", _c_i64),
        ("k_stride_head", _c_i64),
        ("v_stride_block", _c_i64),
        ("v_stride_token", _c_i64),
        ("v_stride_head", _c_i64),
        ("num_tokens", _c_i64),
        ("num_blocks", _c_i64),
        ("block_size", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("dtype", _c_i32),
        ("cache_dtype", _c_i32),
        ("k_scale", _c_ptr),
        ("v_scale", _c_ptr),
        ("scale_stride_block", _c_i64),
        ("scale_stride_head", _c_i64),
    ]


class PagedAttentionArgs(ctypes.Structure):
    """Mirror of ikl_paged_attention_args."""

    _fields_ = [
        ("query", _c_ptr),
        ("q_stride_b", _c_i64),
        ("q_stride_h", _c_i64),
        ("k_cache", _c_ptr),
        ("v_cache", _c_ptr),
        ("k_stride_block", _c_i64),
        ("k_stride_token", _c_i64),
        ("k_stride_head", _c_i64),
        ("v_stride_block", _c_i64),
        ("v_stride_token", _c_i64),
        ("v_stride_head", _c_i64),
        ("block_tables", _c_ptr),
        ("table_type", _c_i32),
        ("table_stride_b", _c_i64),
        ("table_width", _c_i64),
        ("context_lens", _c_ptr),
        ("lens_type", _c_i32),
        ("out", _c_ptr),
        ("out_stride_b", _c_i64),
        ("out_stride_h", _c_i64),
        ("batch", _c_i64),
        ("num_blocks", _c_i64),
        ("num_heads", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("block_size", _c_i32),
        ("dtype", _c_i32),
        ("scale", ctypes.c_float),
        ("query_group_size", _c_i32),
        ("partition_size", _c_i32),
        ("max_context_len", _c_i64),
        ("path", _c_i32),
        ("workspace", _c_ptr),
        ("workspace_bytes", _c_i64),
        ("events", _c_ptr * 3),
        ("cache_dtype", _c_i32),
        ("k_scale", _c_ptr),
        ("v_scale", _c_ptr),
        ("scale_stride_block", _c_i64),
        ("scale_stride_head", _c_i64),
    ]


class RopeAppendArgs(ctypes.Structure):
    """Mirror of ikl_rope_append_args."""

    _fields_ = [
        ("query", _c_ptr),
        ("q_stride_t", _c_i64),
        ("q_stride_h", _c_i64),
        ("query_out", _c_ptr),
        ("q_out_stride_t", _c_i64),
        ("q_out_stride_h", _c_i64),
        ("key", _c_ptr),
        ("key_stride_t", _c_i64),
        ("key_stride_h", _c_i64),
        ("value", _c_ptr),
        ("value_stride_t", _c_i64),
        ("value_stride_h", _c_i64),
        ("cos", _c_ptr),
        ("cos_stride_t", _c_i64),
        ("sin", _c_ptr),
        ("sin_stride_t", _c_i64),
        ("slots", _c_ptr),
        ("slot_type", _c_i32),
        ("k_cache", _c_ptr),
        ("v_cache", _c_ptr),
        ("k_stride_block", _c_i64),
        ("k_stride_token", _c_i64),
        ("k_stride_head", _c_i64),
        ("v_stride_block", _c_i64),
        ("v_stride_token", _c_i64),
        ("v_stride_head", _c_i64),
        ("num_tokens", _c_i64),
        ("num_blocks", _c_i64),
        ("block_size", _c_i32),
        ("num_heads", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("dtype", _c_i32),
        ("cache_dtype", _c_i32),
        ("k_scale", _c_ptr),
        ("v_scale", _c_ptr),
        ("scale_stride_block", _c_i64),
        ("scale_stride_head", _c_i64),
    ]


class PagedPrefillArgs(ctypes.Structure):
    """Mirror of ikl_paged_prefill_args."""

    _fields_ = [
        ("query", _c_ptr),
        ("q_stride_b", _c_i64),
        ("q_stride_h", _c_i64),
        ("q_stride_t", _c_i64),
        ("k_cache", _c_ptr),
        ("v_cache", _c_ptr),
        ("k_stride_block", _c_i64),
        ("k_stride_token", _c_i64),
        ("k_stride_head", _c_i64),
        ("v_stride_block", _c_i64),
        ("v_stride_token", _c_i64),
        ("v_stride_head", _c_i64),
        ("block_tables", _c_ptr),
        ("table_type", _c_i32),
        ("table_stride_b", _c_i64),
        ("table_width", _c_i64),
        ("query_starts", _c_ptr),
        ("context_lens", _c_ptr),
        ("lens_type", _c_i32),
        ("out", _c_ptr),
        ("out_stride_b", _c_i64),
        ("out_stride_h", _c_i64),
        ("out_stride_t", _c_i64),
        ("batch", _c_i64),
        ("query_width", _c_i64),
        ("num_blocks", _c_i64),
        ("num_heads", _c_i32),
        ("num_kv_heads", _c_i32),
        ("head_dim", _c_i32),
        ("block_size", _c_i32),
        ("dtype", _c_i32),
        ("scale", ctypes.c_float),
        ("path", _c_i32),
        ("events", _c_ptr * 2),
        ("cache_dtype", _c_i32),
        ("k_scale", _c_ptr),
        ("v_scale", _c_ptr),
        ("scale_stride_block", _c_i64),
        ("scale_stride_head", _c_i64),
    ]


class LaunchConfig(ctypes.Structure):
    """Mirror of ikl_launch_config."""

    _fields_ = [
        ("struct_size", _c_i32),
        ("path", _c_i32),
        ("tile_tokens", _c_i32),
        ("waves_per_workgroup", _c_i32),
        ("stages", _c_i32),
        ("split", _c_i32),
        ("partition_size", _c_i32),
        ("workgroups", _c_i64),
        ("group_size", _c_i32),
    ]


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_load_error: str | None = None


def _declare(lib: ctypes.CDLL) -> None:
    lib.ikl_last_error.restype = ctypes.c_char_p
    lib.ikl_last_error.argtypes = []
    lib.ikl_version.restype = ctypes.c_char_p
    lib.ikl_version.argtypes = []
    lib.ikl_abi_version.restype = _c_i32
    lib.ikl_abi_version.argtypes = []
    lib.ikl_append_kv.restype = ctypes.c_int
    lib.ikl_append_kv.argtypes = [ctypes.POINTER(AppendArgs), _c_ptr]
    lib.ikl_paged_attention_workspace_size.restype = _c_i64
    lib.ikl_paged_attention_workspace_size.argtypes = [ctypes.POINTER(PagedAttentionArgs)]
    lib.ikl_paged_attention_partition_size.restype = _c_i32
    lib.ikl_paged_attention_partition_size.argtypes = [ctypes.POINTER(PagedAttentionArgs)]
    lib.ikl_paged_attention.restype = ctypes.c_int
    lib.ikl_paged_attention.argtypes = [ctypes.POINTER(PagedAttentionArgs), _c_ptr]
    lib.ikl_paged_attention_path.restype = _c_i32
    lib.ikl_paged_attention_path.argtypes = [_c_i32, _c_i32, _c_i32, _c_i64, _c_i32, _c_i32]
    lib.ikl_rope_append_kv.restype = ctypes.c_int
    lib.ikl_rope_append_kv.argtypes = [ctypes.POINTER(RopeAppendArgs), _c_ptr]
    lib.ikl_paged_prefill_attention.restype = ctypes.c_int
    lib.ikl_paged_prefill_attention.argtypes = [ctypes.POINTER(PagedPrefillArgs), _c_ptr]
    lib.ikl_paged_prefill_path.restype = _c_i32
    lib.ikl_paged_prefill_path.argtypes = [_c_i32, _c_i32, _c_i32]
    lib.ikl_paged_attention_noalloc.restype = ctypes.c_int
    lib.ikl_paged_attention_noalloc.argtypes = [ctypes.POINTER(PagedAttentionArgs), _c_ptr]
    lib.ikl_paged_decode_step.restype = ctypes.c_int
    lib.ikl_paged_decode_step.argtypes = [ctypes.POINTER(PagedAttentionArgs), ctypes.POINTER(AppendArgs), _c_ptr]
    lib.ikl_paged_decode_step_fused.restype = _c_i32
    lib.ikl_paged_decode_step_fused.argtypes = [ctypes.POINTER(PagedAttentionArgs), ctypes.POINTER(AppendArgs)]
    lib.ikl_paged_decode_step_workspace_size.restype = _c_i64
    lib.ikl_paged_decode_step_workspace_size.argtypes = [ctypes.POINTER(PagedAttentionArgs),
                                                         ctypes.POINTER(AppendArgs)]
    lib.ikl_hbm_read_probe.restype = ctypes.c_int
    lib.ikl_hbm_read_probe.argtypes = [_c_ptr, _c_i64, _c_ptr, _c_i64, _c_ptr]
    lib.ikl_paged_attention_launch_config.restype = ctypes.c_int
    lib.ikl_paged_attention_launch_config.argtypes = [ctypes.POINTER(PagedAttentionArgs),
                                                      ctypes.POINTER(LaunchConfig)]


def load() -> ctypes.CDLL:
    """Return the loaded library or raise RuntimeError naming why it is absent."""
    global _lib, _load_error
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            _load_error = (
                f"{LIB_PATH.name} is not built; run `python -m inferkernellab_amd.build`"
            )
            raise RuntimeError(_load_error)
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:  # pragma: no cover - depends on the host
            _load_error = f"cannot load {LIB_PATH}: {exc}"
            raise RuntimeError(_load_error) from exc
        _declare(lib)
        version = lib.ikl_abi_version()
        if version != IKL_ABI_VERSION:
            _load_error = (f"{LIB_PATH.name} implements C ABI version {version}, these bindings "
                           f"version {IKL_ABI_VERSION}; rebuild with `python -m inferkernellab_amd.build`")
            raise RuntimeError(_load_error)
        _lib = lib
        return lib


def library_loaded() -> bool:
    try:
        load()
    except RuntimeError:
        return False
    return True


def last_error() -> str:
    return load().ikl_last_error().decode()


def check(status: int, what: str) -> None:
    """Raise the Python exception matching a non-zero ikl status."""
    if status == IKL_OK:
        return
    message = last_error()
    if status in (IKL_EINVAL, IKL_EUNSUPPORTED):
        raise ValueError(message or f"{what}: invalid argument")
    raise RuntimeError(f"{what} failed ({status}): {message}")
