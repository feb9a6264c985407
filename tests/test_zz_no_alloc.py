"""ikl_paged_attention_noalloc: the split workspace comes from the
library's per-device scratch array instead of the caller. Called through
the C ABI and compared, bit for bit, with ikl_paged_attention on a caller
workspace (and with the oracle, attention.py:134-175, within tolerance), on
two calls in a row, the second with a smaller input."""

import ctypes

import pytest
import torch

from tests.helpers import ATOL, make_case, max_abs_err

pytestmark = pytest.mark.gpu


def _noalloc(case, cache, partition_size):
    from inferkernellab_amd import _lib, ops

    q, tables, lens = case.device_query(), case.device_tables(), case.device_lengths()
    out = torch.empty_like(q)
    args, keep = ops._attention_args(q, cache, tables, lens, out, None, 0, 0, partition_size,
                                     max(case.lengths), -1)
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    status = lib.ikl_paged_attention_noalloc(ctypes.byref(args), ctypes.c_void_p(stream))
    _lib.check(status, "paged attention (no-alloc)")
    ws = lib.ikl_paged_attention_workspace_size(ctypes.byref(args))
    del keep
    return out, ws


def _reference(case, cache, partition_size):
    from inferkernellab_amd import ops

    return ops.paged_decode_attention_hip(case.device_query(), cache, case.device_tables(), case.device_lengths(),
                                          partition_size=partition_size, max_context_len=max(case.lengths))


@pytest.mark.parametrize("order", ["large_then_small", "small_path_then_unsplit"])
def test_noalloc_matches_the_workspace_entry_point(order):
    first = make_case(batch=16, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                      lengths=[8192, 4100, 7000, 5000, 6100, 4096, 8000, 7777, 4500, 5500, 6500, 7500,
                               4321, 5678, 6789, 7890], dtype="bfloat16", seed=90)
    second = make_case(batch=4, num_heads=16, num_kv_heads=2, head_dim=64, block_size=16,
                       lengths=[2000, 1500, 700, 33], dtype="float16", seed=91)
    plan = [(first, 0), (second, 512)] if order == "large_then_small" else [(second, 256), (second, -1)]
    for i, (case, partition) in enumerate(plan):
        print(f"no-alloc call {i}: B={len(case.lengths)} H={case.num_heads} dtype={case.dtype} "
              f"partition={partition}", flush=True)
        cache = case.device_cache()
        got, ws = _noalloc(case, cache, partition)
        want = _reference(case, cache, partition)
        torch.cuda.synchronize()
        assert (ws > 0) == (partition != -1)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"call {i}"
        assert max_abs_err(got, case.expected()) <= ATOL[case.dtype]


@pytest.mark.parametrize("partition", [0, 512])
def test_noalloc_under_graph_capture_replays_the_eager_result(partition):
    """The caller the entry point exists for: code under HIP graph capture.
    One eager call first (it resolves the device's scratch address, which
    must happen outside capture), then the call captured into a graph and
    replayed three times with eager work between the replays; every replay
    equals the eager output bit for bit."""
    from inferkernellab_amd import _lib, ops

    case = make_case(batch=6, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                     lengths=[3000, 17, 1200, 4096, 2500, 640], dtype="bfloat16", seed=92)
    print(f"no-alloc graph capture: partition={partition}", flush=True)
    cache = case.device_cache()
    eager, ws = _noalloc(case, cache, partition)
    torch.cuda.synchronize()
    assert ws > 0  # the launch splits: its partials live in the scratch array
    q, tables, lens = case.device_query(), case.device_tables(), case.device_lengths()
    out = torch.empty_like(q)
    args, keep = ops._attention_args(q, cache, tables, lens, out, None, 0, 0, partition, max(case.lengths), -1)
    lib = _lib.load()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        status = lib.ikl_paged_attention_noalloc(ctypes.byref(args),
                                                 ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(status, "paged attention (no-alloc, captured)")
    for i in range(3):
        out.fill_(float("nan"))
        scratch_user = _reference(case, cache, partition)  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), eager.view(torch.int16)), f"replay {i}"
        assert torch.equal(scratch_user.view(torch.int16), eager.view(torch.int16))
    del keep
