"""The attention entry points under HIP graph capture (a serving loop's captured decode step).

Each captured call is replayed three times, with the program's own eager work and a
synchronisation between replays, and every replay must give the eager call's bits: the
kernels take no host-side allocation or memset, and a mixed batch's second stream (the tile
pass beside the row pass) joins the capture through its fork and join events.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from paged_kv_serving_amd import ops
from paged_kv_serving_amd.workloads import decode_batch, mixed_batch

pytestmark = pytest.mark.gpu


def _replays_equal_eager(device, call) -> None:
    eager = call().clone()
    torch.cuda.synchronize()
    stream = torch.cuda.Stream(device=device)
    stream.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(stream):
        call()  # warm torch's allocator outside the capture (pkv_init ran at the first call)
    torch.cuda.current_stream(device).wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for replay in range(3):
        scratch = torch.randn(1 << 20, device=device)  # eager work between the replays
        scratch.mul_(2.0)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), replay


def test_fused_decode_step_replays_in_a_graph(device) -> None:
    print("graph: fused decode step", flush=True)
    batch = decode_batch(num_seqs=16, context_low=100, context_high=900, heads=8, num_blocks=2000,
                         device=device)  # fmt: skip
    heads, dim = batch.key_cache.shape[2], batch.key_cache.shape[3]
    need = ops.attention_workspace_bytes(batch.num_queries, heads, dim, batch.max_context_len,
                                         batch.plan.partition_size if batch.plan else 0)  # fmt: skip
    workspace = torch.empty(max(need // 4, 1), dtype=torch.float32, device=device)
    out = torch.empty_like(batch.queries)

    def call():
        return ops.paged_attention_ragged(
            batch.queries, batch.query_positions, batch.query_seq, batch.key_cache,
            batch.value_cache, batch.block_tables, batch.context_lens, batch.scale,
            max_context_len=batch.max_context_len, out=out, workspace=workspace, plan=batch.plan,
            append=(batch.new_keys, batch.new_values, batch.slot_mapping),
        )  # fmt: skip

    assert batch.decode_rows_only()
    _replays_equal_eager(device, call)


def test_mixed_batch_with_tiles_beside_rows_replays_in_a_graph(device) -> None:
    print("graph: mixed batch", flush=True)
    batch = mixed_batch(num_prefill=2, chunk=128, offset_high=600, num_decode=24, decode_high=1500,
                        heads=4, num_blocks=3000, device=device)  # fmt: skip
    assert batch.plan is not None and batch.plan.num_tiles > 0 and batch.plan.num_rows > 0
    heads, dim = batch.key_cache.shape[2], batch.key_cache.shape[3]
    need = ops.attention_workspace_bytes(batch.num_queries, heads, dim, batch.max_context_len,
                                         batch.plan.partition_size)  # fmt: skip
    workspace = torch.empty(max(need // 4, 1), dtype=torch.float32, device=device)
    out = torch.empty_like(batch.queries)

    def call():
        return ops.paged_attention_ragged(
            batch.queries, batch.query_positions, batch.query_seq, batch.key_cache,
            batch.value_cache, batch.block_tables, batch.context_lens, batch.scale,
            max_context_len=batch.max_context_len, out=out, workspace=workspace, plan=batch.plan,
        )  # fmt: skip

    _replays_equal_eager(device, call)
    assert np.isfinite(out.cpu().numpy()).all()
