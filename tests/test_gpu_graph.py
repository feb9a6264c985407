"""A decode step (prepared paged attention with its split reduce, then the
prepared append) captured as a HIP graph: every replay equals the eager
launches on the current buffer contents, with eager work and host
synchronisation between replays (the bound buffers are updated in place,
the way a decode loop feeds a captured step)."""

import pytest
import torch

from tests.helpers import ATOL, make_case, max_abs_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("partition_size", [None, -2, 256])
def test_captured_step_replays_match_eager(partition_size):
    from inferkernellab_amd import ops

    case = make_case(batch=6, num_heads=32, num_kv_heads=8, head_dim=128, block_size=16,
                     lengths=[700, 33, 1500, 64, 2000, 257], dtype="bfloat16", seed=60)
    cache = case.device_cache()
    query = case.device_query().clone()
    tables, lens = case.device_tables(), case.device_lengths()
    attn = ops.PreparedPagedAttention(query, cache, tables, lens, partition_size=partition_size,
                                      max_context_len=max(case.lengths))
    new_k = torch.randn(6, 8, 128, device="cuda").to(torch.bfloat16)
    new_v = torch.randn(6, 8, 128, device="cuda").to(torch.bfloat16)
    # the appended rows go to a block no table uses, so the contexts stay the oracle's
    used = {blk for t in case.tables for blk in t}
    free = next(blk for blk in range(cache.layout.num_blocks) if blk not in used)
    spare = torch.arange(6, dtype=torch.int32, device="cuda") + free * 16
    app = ops.PreparedAppend(new_k, new_v, cache, spare)

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        attn()
        app()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        attn()
        app()

    for rep in range(3):
        query.copy_(torch.randn_like(query, dtype=torch.float32).to(torch.bfloat16))  # eager work
        new_k.mul_(-1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        replayed = attn.out.clone()
        eager = ops.paged_decode_attention_hip(query, cache, tables, lens, partition_size=partition_size)
        torch.cuda.synchronize()
        assert torch.equal(replayed.view(torch.int16), eager.view(torch.int16)), f"replay {rep}"
        slots = spare.long()
        assert torch.equal(cache.k[0][slots // 16, slots % 16].view(torch.int16), new_k.view(torch.int16))
    from oracle import paged_oracle as po

    q32 = po.to_f32(query.cpu().view(torch.int16).numpy().view("uint16"), "bfloat16")
    expected = po.paged_decode_attention(q32, case.oracle_cache, case.tables, case.lengths)
    assert max_abs_err(replayed, expected) <= ATOL["bfloat16"]
