"""pkv_paged_attention_noalloc: the attention entry point that allocates nothing, through the C ABI.

It takes pkv_paged_attention's arguments without the workspace and uses the library's static
per-device scratch instead. Two calls in a row (a mixed batch with MFMA tiles, decode rows and a
split-context reduce, then a smaller decode batch) must give exactly what pkv_paged_attention
gives with a caller workspace for the same plan, and match the oracle. Which call finds the
device's copy of the scratch (hipGetSymbolAddress) depends on the process: run alone in a fresh
process, this file's first no-alloc call is the library's first attention call on the device and
finds it itself (nothing before it calls pkv_init: the append is the only library call); after
other tests, pkv_init has found it already and the call reuses that address. A batch whose
workspace exceeds the scratch is refused before anything is enqueued.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.attention import paged_attention
from paged_kv_serving_amd import _native, ops
from paged_kv_serving_amd.workloads import decode_batch, mixed_batch

pytestmark = pytest.mark.gpu


def _args(batch, plan, out):
    """pkv_paged_attention's arguments up to (and including) flags, for ``batch`` and ``plan``."""
    merge = plan.merge
    flags = (_native.PKV_ATTN_SHARED_KV if plan.shared_kv else 0) | (
        _native.PKV_ATTN_SHORT_ROWS if plan.short_rows else 0
    )
    heads, dim = batch.key_cache.shape[2], batch.key_cache.shape[3]
    return (
        out.data_ptr(), batch.queries.data_ptr(), heads * dim,
        batch.query_positions.data_ptr(), batch.query_seq.data_ptr(), batch.num_queries, None,
        plan.rows.data_ptr() if plan.num_rows else None, plan.num_rows,
        plan.tiles.data_ptr() if plan.num_tiles else None, plan.num_tiles,
        merge.data_ptr() if merge is not None and merge.numel() else None,
        -1 if merge is None else int(merge.numel()),
        batch.key_cache.data_ptr(), batch.value_cache.data_ptr(), ops.kv_dtype_code(batch.key_cache.dtype),
        batch.key_cache.shape[0], batch.key_cache.shape[1],
        batch.block_tables.data_ptr(), batch.block_tables.shape[1], batch.context_lens.data_ptr(),
        batch.num_seqs, heads, dim, float(batch.scale), batch.max_context_len, plan.partition_size, flags,
    )  # fmt: skip


def _both(batch, device):
    """(no-alloc output, workspace output) of one batch under the planner's plan; the no-alloc
    call goes first."""
    lib = _native.library()
    ops.append_kv(batch.key_cache, batch.value_cache, batch.new_keys, batch.new_values, batch.slot_mapping)
    plan = batch.plan
    heads, dim = batch.key_cache.shape[2], batch.key_cache.shape[3]
    stream = torch.cuda.current_stream(device).cuda_stream
    static_out = torch.full((batch.num_queries, heads, dim), float("nan"), device=device)
    rc = lib.pkv_paged_attention_noalloc(*_args(batch, plan, static_out), device.index, stream)
    assert rc == 0, _native.library().pkv_error_string(rc)
    need = ops.attention_workspace_bytes(batch.num_queries, heads, dim, batch.max_context_len, plan.partition_size)
    assert 0 < need <= _native.STATIC_SCRATCH_BYTES, "the case must use the scratch"
    workspace = torch.empty(need // 4, dtype=torch.float32, device=device)
    caller_out = torch.full_like(static_out, float("nan"))
    rc = lib.pkv_paged_attention(*_args(batch, plan, caller_out), workspace.data_ptr(), need, device.index, stream)
    assert rc == 0, _native.library().pkv_error_string(rc)
    torch.cuda.synchronize(device)
    return static_out.cpu().numpy(), caller_out.cpu().numpy()


def _oracle_gap(batch, got, seqs) -> float:
    worst = 0.0
    for s in seqs:
        keys, values, q, positions = batch.host_rows(s)
        rows = np.nonzero(batch.host_seq == s)[0]
        # host_rows gives keys in logical order: a pool of one-token blocks, table 0, 1, 2, ...
        want = paged_attention(q, positions, keys.reshape(-1, 1, *keys.shape[1:]),
                               values.reshape(-1, 1, *values.shape[1:]), np.arange(keys.shape[0]),
                               int(batch.host_context[s]), batch.scale, tile_blocks=128)  # fmt: skip
        worst = max(worst, float(np.max(np.abs(got[rows] - want))))
    return worst


def test_two_calls_in_a_row_match_the_workspace_entry_point(device) -> None:
    fresh = device.index not in _native._READY  # nothing has called pkv_init on this device yet
    print("no-alloc: first attention call of the process" if fresh else "no-alloc: pkv_init ran before", flush=True)
    first = mixed_batch(seed=3, num_prefill=2, chunk=96, offset_high=1500, num_decode=40, decode_low=300,
                        decode_high=3000, heads=8, head_dim=128, num_blocks=8000, device=device)  # fmt: skip
    first.replan(0)
    assert first.plan.num_tiles > 0 and first.plan.num_rows > 0, "tiles beside rows"
    static_out, caller_out = _both(first, device)
    print("no-alloc call 1:", first.num_queries, "rows", flush=True)
    assert np.array_equal(static_out, caller_out)
    assert _oracle_gap(first, static_out, [0, 2, 17, 41]) < 1e-5

    second = decode_batch(seed=4, num_seqs=6, context_low=600, context_high=1400, heads=8, head_dim=128,
                          num_blocks=800, device=device)  # fmt: skip
    second.replan(256)
    static_out, caller_out = _both(second, device)
    print("no-alloc call 2:", second.num_queries, "rows", flush=True)
    assert np.array_equal(static_out, caller_out)
    assert _oracle_gap(second, static_out, range(6)) < 1e-5


def test_a_batch_beyond_the_scratch_is_refused(device) -> None:
    lib = _native.library()
    small = decode_batch(seed=5, num_seqs=2, context_low=100, context_high=200, heads=8, head_dim=128,
                         num_blocks=64, device=device)  # fmt: skip
    small.replan(0)
    args = list(_args(small, small.plan, small.queries.clone()))
    # positions of num_queries, max_context_len and partition_size in the argument list
    assert (args[5], args[25], args[26]) == (small.num_queries, small.max_context_len, small.plan.partition_size)
    args[5] = 4096  # num_queries: 4096 x 8 heads x 64 partitions x 130 floats > 64 MiB
    args[25] = 32768  # max_context_len
    args[26] = 512  # partition_size
    need = ops.attention_workspace_bytes(4096, 8, 128, 32768, 512)
    assert need > _native.STATIC_SCRATCH_BYTES
    assert lib.pkv_paged_attention_noalloc(*args, device.index, None) == _native.PKV_ETOOBIG
