"""Seeded random ragged batches through the whole host plan (``ops.plan_batch``) and the kernels.

Each case draws the head count, head_dim, block size, pool dtype, context lengths, which
sequences bring a prefill run (tile pass) and which a decode row (row pass), and the partition
size; one case in four is a batch of decode rows that share a leading run of blocks, so the
planner builds shared-prefix tiles. Every output row is compared with the oracle's paged
attention (reference attention.py:42-121) at the float32 bar of 1e-5; bfloat16 pools are
compared with the oracle run on the bf16-rounded K/V. The plan decides tiles, whole tiles,
partition size, merge list and launch hints, so this covers their combinations, not only the
hand-built plans of the other kernel tests.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle.attention import paged_attention
from oracle.bf16 import bf16_round
from paged_kv_serving_amd import ops

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
CASES = int(os.environ.get("PKV_RANDOM_CASES", "48"))  # seeds 0 .. CASES - 1


def _random_batch(rng):
    heads = int(rng.choice([1, 2, 3, 4, 8]))
    dim = int(rng.choice([8, 16, 32, 64, 128, 256]))
    block = int(rng.choice([1, 2, 5, 8, 16, 32]))
    shared = rng.random() < 0.25
    tables, contexts, positions, seq_of = [], [], [], []
    next_block = 0
    if shared:
        # Decode rows of 18-24 sequences over one common prefix of >= 512 tokens.
        seqs = int(rng.integers(18, 25))
        prefix_tokens = int(rng.integers(512, 1200))
        prefix_blocks = prefix_tokens // block
        prefix = list(range(prefix_blocks))
        next_block = prefix_blocks
        for s in range(seqs):
            ctx = prefix_blocks * block + int(rng.integers(-40, 300))
            ctx = max(ctx, 1)
            own = max(0, -(-ctx // block) - prefix_blocks)
            tables.append(prefix[: -(-ctx // block)] + list(range(next_block, next_block + own)))
            next_block += own
            contexts.append(ctx)
            positions.append(ctx - 1)
            seq_of.append(s)
    else:
        seqs = int(rng.integers(1, 9))
        max_ctx = int(rng.integers(1, 1400 if block > 1 else 600))
        for s in range(seqs):
            ctx = int(rng.integers(1, max_ctx + 1))
            need = -(-ctx // block)
            tables.append(list(range(next_block, next_block + need)))
            next_block += need
            contexts.append(ctx)
            prefill = rng.random() < 0.5
            nq = int(rng.integers(1, min(ctx, 150) + 1)) if prefill else 1
            positions += list(range(ctx - nq, ctx))
            seq_of += [s] * nq
    pool = next_block + 3
    perm = rng.permutation(pool)  # scatter the blocks over the pool
    tables = [perm[np.asarray(t, dtype=np.int64)].astype(np.int32) for t in tables]
    kc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    q = rng.standard_normal((len(seq_of), heads, dim)).astype(np.float32)
    kv = torch.bfloat16 if rng.random() < 0.3 else torch.float32
    partition = int(rng.choice([0, 0, 16, 64, 256, 1024]))
    return (heads, dim, block, kv, partition, tables, np.asarray(contexts), np.asarray(positions),
            np.asarray(seq_of), kc, vc, q)  # fmt: skip


@pytest.mark.parametrize("seed", range(CASES))
def test_random_batch_through_the_planner_matches_the_oracle(device, seed) -> None:
    rng = np.random.default_rng(7000 + seed)
    heads, dim, block, kv, partition, tables, contexts, positions, seq_of, kc, vc, q = _random_batch(rng)
    print("random batch", seed, heads, dim, block, kv, partition, len(tables), q.shape[0], flush=True)
    if kv == torch.bfloat16:
        kc, vc = bf16_round(kc), bf16_round(vc)
    scale = dim**-0.5
    want = np.zeros_like(q)
    for s, (table, ctx) in enumerate(zip(tables, contexts)):
        rows = np.nonzero(seq_of == s)[0]
        want[rows] = paged_attention(q[rows], positions[rows], kc, vc, table, int(ctx), scale)
    host = ops.plan_batch(seq_of, dim, heads, tables, contexts, block, partition_size=partition,
                          query_positions=positions, kv_dtype=kv)  # fmt: skip
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -3, dtype=np.int32)  # padding is never read
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    got = ops.paged_attention_ragged(
        torch.from_numpy(q).to(device), torch.from_numpy(positions.astype(np.int32)).to(device),
        torch.from_numpy(seq_of.astype(np.int32)).to(device),
        torch.from_numpy(kc).to(device).to(kv), torch.from_numpy(vc).to(device).to(kv),
        torch.from_numpy(padded).to(device), torch.from_numpy(contexts.astype(np.int32)).to(device),
        scale, max_context_len=int(contexts.max()), plan=ops.upload_batch_plan(host, device),
    ).cpu().numpy()  # fmt: skip
    err = float(np.max(np.abs(got - want)))
    assert err < FP32_TOL, (seed, err, host.tiles.shape[0], host.partition_size, host.dominant_tiles)


FUSED_CASES = int(os.environ.get("PKV_RANDOM_FUSED_CASES", "32"))  # seeds 0 .. FUSED_CASES - 1


def _random_decode_batch(rng):
    """One decode row per sequence at its last position, each writing a block of its own; half
    of the cases share a leading run of whole blocks (shared-prefix tiles beside the rows)."""
    heads = int(rng.choice([1, 2, 4, 8, 32]))
    dim = int(rng.choice([32, 64, 128]))
    if heads * dim > 2048:
        heads = 2048 // dim
    block = int(rng.choice([1, 4, 5, 16, 32]))
    shared = rng.random() < 0.5
    seqs = int(rng.integers(18, 41)) if shared else int(rng.integers(1, 25))
    prefix_blocks = int(rng.integers(512, 1100)) // block if shared else 0
    tables, contexts, next_block = [], [], prefix_blocks
    for _ in range(seqs):
        ctx = prefix_blocks * block + int(rng.integers(1, 300)) if shared else int(rng.integers(1, 900))
        own = -(-ctx // block) - prefix_blocks  # the last visible block is always a private one
        tables.append(list(range(prefix_blocks)) + list(range(next_block, next_block + own)))
        next_block += own
        contexts.append(ctx)
    pool = next_block + 2
    perm = rng.permutation(pool)
    tables = [perm[np.asarray(t, dtype=np.int64)].astype(np.int32) for t in tables]
    kv = torch.bfloat16 if rng.random() < 0.4 else torch.float32
    partition = int(rng.choice([0, 0, 64, 256]))
    return heads, dim, block, kv, partition, tables, np.asarray(contexts), pool


@pytest.mark.parametrize("seed", range(FUSED_CASES))
def test_random_decode_batch_with_the_fused_append_and_caller_rows(device, seed) -> None:
    """pkv_paged_attention_append over a planned random decode batch whose rows reach the caller's
    rows through a random caller_rows permutation: the pools equal pkv_append's bit for bit, and
    every output row is within 1e-5 of the oracle over the appended pools (bfloat16 pools: the
    new rows rounded to nearest even, as the append stores them)."""
    rng = np.random.default_rng(9000 + seed)
    heads, dim, block, kv, partition, tables, contexts, pool = _random_decode_batch(rng)
    seqs = len(tables)
    print("random fused decode", seed, heads, dim, block, kv, partition, seqs, flush=True)
    positions = contexts - 1
    seq_of = np.arange(seqs)
    slots = np.asarray([int(t[p // block]) * block + p % block for t, p in zip(tables, positions)], np.int64)
    kc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    q, new_k, new_v = (rng.standard_normal((seqs, heads, dim)).astype(np.float32) for _ in range(3))
    if kv == torch.bfloat16:
        kc, vc = bf16_round(kc), bf16_round(vc)
    kh, vh = kc.copy(), vc.copy()  # the pools after the append, as the oracle sees them
    kh.reshape(-1, heads, dim)[slots] = bf16_round(new_k) if kv == torch.bfloat16 else new_k
    vh.reshape(-1, heads, dim)[slots] = bf16_round(new_v) if kv == torch.bfloat16 else new_v
    scale = dim**-0.5
    want = np.zeros_like(q)
    for s in range(seqs):
        want[s] = paged_attention(q[s : s + 1], positions[s : s + 1], kh, vh, tables[s], int(contexts[s]), scale)[0]
    host = ops.plan_batch(seq_of, dim, heads, tables, contexts, block, partition_size=partition,
                          query_positions=positions, kv_dtype=kv)  # fmt: skip
    width = max(len(t) for t in tables)
    padded = np.full((seqs, width), -3, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    order = rng.permutation(seqs)  # planner row t reads and writes caller row order[t]

    def caller(a: np.ndarray) -> np.ndarray:
        out = np.empty_like(a)
        out[order] = a
        return out

    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    k_ref, v_ref = to(kc).to(kv), to(vc).to(kv)
    ops.append_kv(k_ref, v_ref, to(new_k), to(new_v), to(slots))
    k_fus, v_fus = to(kc).to(kv), to(vc).to(kv)
    got = ops.paged_attention_ragged(
        to(caller(q)), to(positions.astype(np.int32)), to(seq_of.astype(np.int32)), k_fus, v_fus, to(padded),
        to(contexts.astype(np.int32)), scale, max_context_len=int(contexts.max()),
        plan=ops.upload_batch_plan(host, device), append=(to(caller(new_k)), to(caller(new_v)), to(caller(slots))),
        caller_rows=to(order.astype(np.int32)),
    )  # fmt: skip
    assert torch.equal(k_fus, k_ref) and torch.equal(v_fus, v_ref), seed
    err = float(np.max(np.abs(got.cpu().numpy()[order] - want)))
    assert err < FP32_TOL, (seed, err, host.tiles.shape[0], host.partition_size)
