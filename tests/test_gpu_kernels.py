"""GPU parity of the three kernels against the CPU oracle, through the C ABI.

Integer and byte work is bit-exact: the append (float32 and bfloat16 pools, strided sources),
the copy-on-write block copy, and the bfloat16 rounding of the append. Attention is compared
with the oracle's paged attention (reference attention.py:42-121) and with the float64 closed
form; the tolerance is the north star's 1e-5 max abs for float32 KV, and for bfloat16 KV the
same 1e-5 against the oracle run on the bf16-rounded keys and values (both sides then see
identical inputs and differ only by float32 accumulation order).
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from oracle.attention import dense_attention, gather_context, paged_attention
from oracle.bf16 import bf16_bits, bf16_round
from paged_kv_serving_amd import ops

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5


def say(*parts) -> None:
    print(*parts, flush=True)


# --- append ------------------------------------------------------------------------------------


@pytest.mark.parametrize(
    ("blocks", "block", "heads", "dim", "tokens"),
    [(7, 4, 2, 8, 11), (64, 16, 4, 32, 100), (300, 16, 32, 128, 64), (5, 3, 3, 6, 9)],
)
def test_append_float32_is_bit_exact(device, blocks, block, heads, dim, tokens) -> None:
    say("append f32", blocks, block, heads, dim, tokens)
    rng = np.random.default_rng(blocks + tokens)
    pool_k = rng.standard_normal((blocks, block, heads, dim)).astype(np.float32)
    pool_v = rng.standard_normal((blocks, block, heads, dim)).astype(np.float32)
    slots = rng.permutation(blocks * block)[:tokens].astype(np.int64)
    keys = rng.standard_normal((tokens, heads, dim)).astype(np.float32)
    values = rng.standard_normal((tokens, heads, dim)).astype(np.float32)
    dk, dv = torch.from_numpy(pool_k).to(device), torch.from_numpy(pool_v).to(device)
    ops.append_kv(dk, dv, torch.from_numpy(keys).to(device), torch.from_numpy(values).to(device),
                  torch.from_numpy(slots).to(device))  # fmt: skip
    pool_k.reshape(-1, heads, dim)[slots] = keys
    pool_v.reshape(-1, heads, dim)[slots] = values
    assert np.array_equal(dk.cpu().numpy().view(np.uint32), pool_k.view(np.uint32))
    assert np.array_equal(dv.cpu().numpy().view(np.uint32), pool_v.view(np.uint32))


def test_append_from_a_fused_qkv_view(device) -> None:
    """Keys and values as token-strided views of a (T, 3, H, D) projection, no copy."""
    say("append strided")
    rng = np.random.default_rng(5)
    tokens, heads, dim, blocks, block = 13, 4, 16, 9, 8
    fused = rng.standard_normal((tokens, 3, heads, dim)).astype(np.float32)
    slots = rng.permutation(blocks * block)[:tokens].astype(np.int64)
    dfused = torch.from_numpy(fused).to(device)
    want_k = np.zeros((blocks * block, heads, dim), dtype=np.float32)
    want_v = np.zeros_like(want_k)
    want_k[slots] = fused[:, 1]
    want_v[slots] = fused[:, 2]
    # both strided; then contiguous keys (as after RoPE) with strided values
    for keys in (dfused[:, 1], dfused[:, 1].contiguous()):
        dk = torch.zeros((blocks, block, heads, dim), device=device)
        dv = torch.zeros_like(dk)
        ops.append_kv(dk, dv, keys, dfused[:, 2], torch.from_numpy(slots).to(device))
        assert np.array_equal(dk.cpu().numpy().reshape(-1, heads, dim), want_k)
        assert np.array_equal(dv.cpu().numpy().reshape(-1, heads, dim), want_v)


@pytest.mark.parametrize("dim", [8, 128, 6])
def test_append_float32_into_bfloat16_rounds_to_nearest_even(device, dim) -> None:
    say("append f32->bf16", dim)
    rng = np.random.default_rng(dim)
    tokens, heads, blocks, block = 21, 2, 6, 4
    keys = (rng.standard_normal((tokens, heads, dim)) * 3).astype(np.float32)
    values = (rng.standard_normal((tokens, heads, dim)) * 3).astype(np.float32)
    keys[0, 0, :2] = [1.0 + 2.0**-8, 1.0 + 3 * 2.0**-8]  # ties: to even (down, up)
    slots = rng.permutation(blocks * block)[:tokens].astype(np.int64)
    dk = torch.zeros((blocks, block, heads, dim), dtype=torch.bfloat16, device=device)
    dv = torch.zeros_like(dk)
    ops.append_kv(dk, dv, torch.from_numpy(keys).to(device), torch.from_numpy(values).to(device),
                  torch.from_numpy(slots).to(device))  # fmt: skip
    got_k = dk.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1, heads, dim)
    got_v = dv.view(torch.int16).cpu().numpy().view(np.uint16).reshape(-1, heads, dim)
    assert np.array_equal(got_k[slots], bf16_bits(keys))
    assert np.array_equal(got_v[slots], bf16_bits(values))
    unused = np.setdiff1d(np.arange(blocks * block), slots)
    assert not got_k[unused].any() and not got_v[unused].any()


def test_append_bfloat16_into_bfloat16_copies_bits(device) -> None:
    say("append bf16->bf16")
    g = torch.Generator(device=device).manual_seed(3)
    keys = torch.randn((10, 2, 64), generator=g, device=device).to(torch.bfloat16)
    values = torch.randn((10, 2, 64), generator=g, device=device).to(torch.bfloat16)
    slots = torch.tensor([3, 9, 0, 31, 17, 8, 22, 5, 14, 28], dtype=torch.int64, device=device)
    dk = torch.zeros((8, 4, 2, 64), dtype=torch.bfloat16, device=device)
    dv = torch.zeros_like(dk)
    ops.append_kv(dk, dv, keys, values, slots)
    assert torch.equal(dk.view(-1, 2, 64)[slots].view(torch.int16), keys.view(torch.int16))
    assert torch.equal(dv.view(-1, 2, 64)[slots].view(torch.int16), values.view(torch.int16))


def test_append_skips_slots_outside_the_pool(device) -> None:
    say("append bad slots")
    dk = torch.zeros((2, 4, 1, 8), device=device)
    dv = torch.zeros_like(dk)
    rows = torch.ones((3, 1, 8), device=device)
    slots = torch.tensor([-1, 8, 5], dtype=torch.int64, device=device)
    ops.append_kv(dk, dv, rows, rows, slots)
    flat = dk.view(-1, 8).cpu().numpy()
    assert flat[5].tolist() == [1.0] * 8
    assert flat.sum() == 8.0


# --- copy-on-write ----------------------------------------------------------------------------


@pytest.mark.parametrize(
    ("layers", "blocks", "block", "heads", "dim", "dtype"),
    [(2, 16, 4, 2, 8, torch.float32), (1, 600, 16, 32, 128, torch.float32),
     (3, 40, 16, 4, 32, torch.bfloat16), (2, 9, 3, 1, 6, torch.float32)],
)  # fmt: skip
def test_copy_blocks_is_bit_exact(device, layers, blocks, block, heads, dim, dtype) -> None:
    say("copy", layers, blocks, block, heads, dim, dtype)
    g = torch.Generator(device=device).manual_seed(blocks)
    keys = torch.randn((layers, blocks, block, heads, dim), generator=g, device=device).to(dtype)
    values = torch.randn((layers, blocks, block, heads, dim), generator=g, device=device).to(dtype)
    rng = np.random.default_rng(blocks)
    ids = rng.permutation(blocks)
    n = blocks // 3
    pairs = np.stack([ids[:n], ids[n : 2 * n]], axis=1).astype(np.int64)
    want_k, want_v = keys.clone(), values.clone()
    for src, dst in pairs:
        want_k[:, dst] = want_k[:, src]
        want_v[:, dst] = want_v[:, src]
    ops.copy_blocks(keys, values, torch.from_numpy(pairs).to(device))
    assert torch.equal(keys.view(torch.uint8), want_k.view(torch.uint8))
    assert torch.equal(values.view(torch.uint8), want_v.view(torch.uint8))


def test_dependent_copies_apply_in_order(device) -> None:
    """A -> B then B -> C: C must receive A's bytes (two groups, launched in order)."""
    say("copy chain")
    keys = torch.arange(1 * 4 * 2 * 1 * 4, dtype=torch.float32, device=device).view(1, 4, 2, 1, 4)
    values = -keys
    pairs = [(0, 1), (1, 2), (3, 0)]
    groups = ops.independent_groups(pairs)
    assert groups == [[(0, 1)], [(1, 2), (3, 0)]]
    before = keys.clone()
    for group in groups:
        ops.copy_blocks(keys, values, torch.tensor(group, dtype=torch.int64, device=device))
    assert torch.equal(keys[0, 1], before[0, 0])
    assert torch.equal(keys[0, 2], before[0, 0])
    assert torch.equal(keys[0, 0], before[0, 3])


# --- attention --------------------------------------------------------------------------------


def _ragged_case(rng, *, heads, dim, block, pool, seqs, max_ctx, prefill, max_rows=9):
    """Random ragged batch: each sequence gets 1 (decode) or several (prefill chunk) queries."""
    kc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    contexts = rng.integers(1, max_ctx + 1, seqs)
    need = [-(-int(c) // block) for c in contexts]
    assert sum(need) <= pool
    perm = rng.permutation(pool)
    tables, offset = [], 0
    for n in need:
        tables.append(perm[offset : offset + n])
        offset += n
    positions, seq_of = [], []
    for s, c in enumerate(contexts):
        nq = int(rng.integers(1, min(int(c), max_rows) + 1)) if prefill else 1
        positions += list(range(int(c) - nq, int(c)))
        seq_of += [s] * nq
    q = rng.standard_normal((len(positions), heads, dim)).astype(np.float32)
    return kc, vc, tables, contexts, np.asarray(positions), np.asarray(seq_of), q


def _run_kernel(device, kc, vc, tables, contexts, positions, seq_of, q, scale, *, partition=0,
                dtype=torch.float32, tiles=False):  # fmt: skip
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -7, dtype=np.int32)  # padding is never read
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    dk = torch.from_numpy(kc).to(device).to(dtype)
    dv = torch.from_numpy(vc).to(device).to(dtype)
    plan = None
    if tiles:  # runs of >= 2 rows of one sequence go to the MFMA tile pass
        rows, tile_list = ops.plan_rows(seq_of, q.shape[2], min_tile_rows=2)
        visible = np.minimum(np.asarray(contexts)[seq_of], positions + 1)
        plan = ops.upload_plan(ops.expand_rows(rows, visible, partition), tile_list, device)
    out = ops.paged_attention_ragged(
        torch.from_numpy(q).to(device),
        torch.from_numpy(positions.astype(np.int32)).to(device),
        torch.from_numpy(seq_of.astype(np.int32)).to(device),
        dk, dv, torch.from_numpy(padded).to(device),
        torch.from_numpy(contexts.astype(np.int32)).to(device),
        scale, max_context_len=int(contexts.max()), partition_size=partition, plan=plan,
    )  # fmt: skip
    return out.cpu().numpy()


def _oracle(kc, vc, tables, contexts, positions, seq_of, q, scale):
    out = np.zeros_like(q)
    dense = np.zeros(q.shape, dtype=np.float64)
    for s, (table, ctx) in enumerate(zip(tables, contexts)):
        rows = np.nonzero(seq_of == s)[0]
        out[rows] = paged_attention(q[rows], positions[rows], kc, vc, table, int(ctx), scale)
        dense[rows] = dense_attention(q[rows], gather_context(kc, table, int(ctx)),
                                      gather_context(vc, table, int(ctx)), scale, positions[rows])  # fmt: skip
    return out, dense


@pytest.mark.parametrize("tiles", [False, True], ids=["rows", "tiles"])
@pytest.mark.parametrize("dim", [8, 16, 32, 64, 128, 256])
@pytest.mark.parametrize("block", [1, 3, 4, 16, 32])
def test_ragged_attention_matches_the_oracle(device, dim, block, tiles) -> None:
    say("ragged attention", dim, block, tiles)
    rng = np.random.default_rng(dim * 100 + block)
    heads = 2 if dim >= 128 else 3
    max_ctx = 700 if block > 1 else 300
    case = _ragged_case(rng, heads=heads, dim=dim, block=block, pool=5 * max_ctx // block + 8,
                        seqs=5, max_ctx=max_ctx, prefill=True)  # fmt: skip
    scale = dim**-0.5
    want, dense = _oracle(*case, scale)
    for partition in (0, 16, 48, 1024):
        got = _run_kernel(device, *case, scale, partition=partition, tiles=tiles)
        assert np.max(np.abs(got - want)) < FP32_TOL, partition
        assert np.max(np.abs(got - dense)) < FP32_TOL, partition


@pytest.mark.parametrize("dim", [32, 64, 128, 256])
@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_long_prefill_runs_through_the_mfma_tiles(device, dim, kv) -> None:
    """Runs of up to 150 rows: several full and partial 64-row tiles, causal inside the chunk,
    mixed with decode rows, across partition sizes."""
    say("mfma tiles", dim, kv)
    rng = np.random.default_rng(dim + 7)
    case = _ragged_case(rng, heads=2, dim=dim, block=16, pool=300, seqs=6, max_ctx=700,
                        prefill=True, max_rows=150)  # fmt: skip
    kc, vc, tables, contexts, positions, seq_of, q = case
    scale = dim**-0.5
    if kv == torch.bfloat16:
        kc, vc = bf16_round(kc), bf16_round(vc)
    want, dense = _oracle(kc, vc, tables, contexts, positions, seq_of, q, scale)
    rows, tile_list = ops.plan_rows(seq_of, dim, min_tile_rows=2)
    assert len(tile_list) >= 3 and any(n < 64 for _, n, _, _ in tile_list)
    for partition in (0, 128, 1024):
        got = _run_kernel(device, kc, vc, tables, contexts, positions, seq_of, q, scale,
                          partition=partition, dtype=kv, tiles=True)  # fmt: skip
        assert np.max(np.abs(got - want)) < FP32_TOL, partition
        assert np.max(np.abs(got - dense)) < FP32_TOL, partition


@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_shared_prefix_tiles_match_the_oracle(device, kv) -> None:
    """Decode rows of 40 sequences: 24 share 70 leading blocks (one of them ends inside the
    prefix), 16 share 33 others; the planner turns each prefix into tiles over whole partitions
    and starts those rows' row pass after it. Same results as the plain plan and the oracle."""
    say("shared prefix", kv)
    rng = np.random.default_rng(21)
    heads, dim, block = 4, 128, 16
    pool = 1200
    kc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    if kv == torch.bfloat16:
        kc, vc = bf16_round(kc), bf16_round(vc)
    ids = iter(rng.permutation(pool).tolist())
    prefix_a = [next(ids) for _ in range(70)]
    prefix_b = [next(ids) for _ in range(33)]
    tables, contexts = [], []
    for i in range(40):
        prefix = prefix_a if i < 24 else prefix_b
        ctx = len(prefix) * block + int(rng.integers(1, 300))
        if i == 5:
            ctx = 600  # ends inside prefix a
        need = -(-ctx // block)
        table = prefix[:need] + [next(ids) for _ in range(max(0, need - len(prefix)))]
        tables.append(np.asarray(table))
        contexts.append(ctx)
    contexts = np.asarray(contexts)
    positions = contexts - 1
    seq_of = np.arange(40)
    q = rng.standard_normal((40, heads, dim)).astype(np.float32)
    plan = ops.plan_batch(seq_of, dim, heads, tables, contexts, block)
    # every row-pass item lies after the prefix partitions the tiles cover (a row whose context
    # ends inside the prefix has no row-pass item at all)
    assert plan.tiles.shape[0] >= 2 and np.all(plan.rows[:, 1] > 0)
    assert len(set(plan.rows[:, 0].tolist())) >= 36
    want, dense = _oracle(kc, vc, tables, contexts, positions, seq_of, q, 0.09)
    width = max(len(t) for t in tables)
    padded = np.full((40, width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    args = [
        torch.from_numpy(q).to(device), torch.from_numpy(positions.astype(np.int32)).to(device),
        torch.from_numpy(seq_of.astype(np.int32)).to(device),
        torch.from_numpy(kc).to(device).to(kv), torch.from_numpy(vc).to(device).to(kv),
        torch.from_numpy(padded).to(device), torch.from_numpy(contexts.astype(np.int32)).to(device), 0.09,
    ]  # fmt: skip
    got = ops.paged_attention_ragged(
        *args, max_context_len=int(contexts.max()), plan=ops.upload_batch_plan(plan, device)
    ).cpu().numpy()
    plain = ops.paged_attention_ragged(
        *args, max_context_len=int(contexts.max()), partition_size=plan.partition_size
    ).cpu().numpy()
    assert np.max(np.abs(got - want)) < FP32_TOL
    assert np.max(np.abs(got - dense)) < FP32_TOL
    assert np.max(np.abs(got - plain)) < FP32_TOL


def test_tile_rows_with_arbitrary_positions_and_no_visible_keys(device) -> None:
    """A tile's rows need not be consecutive positions; a row with position < 0 sees nothing."""
    say("tile positions")
    rng = np.random.default_rng(5)
    heads, dim, block = 2, 64, 16
    kc = rng.standard_normal((20, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((20, block, heads, dim)).astype(np.float32)
    table = rng.permutation(20)[:12]
    positions = np.asarray([150, -1, 3, 190, 0, 77, 77, 12, 160, 5, 100, 130], dtype=np.int64)
    seq_of = np.zeros(positions.size, dtype=np.int64)
    q = rng.standard_normal((positions.size, heads, dim)).astype(np.float32)
    case = (kc, vc, [table], np.asarray([191]), positions, seq_of, q)
    want, dense = _oracle(*case, 0.125)
    for partition in (0, 64):
        got = _run_kernel(device, *case, 0.125, partition=partition, tiles=True)
        assert np.array_equal(got[1], np.zeros_like(got[1]))
        assert np.max(np.abs(got - dense)) < FP32_TOL


@pytest.mark.parametrize("dim", [8, 64, 128])
def test_bfloat16_kv_matches_the_oracle_on_rounded_inputs(device, dim) -> None:
    say("bf16 attention", dim)
    rng = np.random.default_rng(dim + 1)
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=2, dim=dim, block=16, pool=200, seqs=4, max_ctx=700, prefill=True
    )
    scale = dim**-0.5
    got = _run_kernel(device, kc, vc, tables, contexts, positions, seq_of, q, scale, dtype=torch.bfloat16)
    want, dense = _oracle(bf16_round(kc), bf16_round(vc), tables, contexts, positions, seq_of, q, scale)
    assert np.max(np.abs(got - want)) < FP32_TOL
    assert np.max(np.abs(got - dense)) < FP32_TOL


@pytest.mark.parametrize("heads", [1, 3, 4, 6])
@pytest.mark.parametrize("dim", [8, 32, 64, 128, 256])
@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
def test_row_pass_head_pairs_match_the_oracle(device, kv, dim, heads) -> None:
    """The row pass reads two adjacent heads per workgroup when a head row is at most 256 bytes
    and the head count is even, one otherwise: both layouts, every head of the batch."""
    say("row pass heads", kv, dim, heads)
    rng = np.random.default_rng(1000 * heads + dim)
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=heads, dim=dim, block=16, pool=160, seqs=5, max_ctx=600, prefill=True, max_rows=4
    )
    scale = dim**-0.5
    if kv == torch.bfloat16:
        kc, vc = bf16_round(kc), bf16_round(vc)
    want, dense = _oracle(kc, vc, tables, contexts, positions, seq_of, q, scale)
    for partition in (0, 64):
        got = _run_kernel(device, kc, vc, tables, contexts, positions, seq_of, q, scale,
                          partition=partition, dtype=kv)  # fmt: skip
        assert np.max(np.abs(got - want)) < FP32_TOL, partition
        assert np.max(np.abs(got - dense)) < FP32_TOL, partition


@pytest.mark.parametrize("dim", [64, 128, 256])
@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("block", [16, 5])
def test_short_row_workgroups_match_the_oracle(device, dim, kv, block) -> None:
    """PKV_ATTN_SHORT_ROWS launches the lighter row-pass workgroup (half the keys in flight per
    wavefront); it must give the same rows as the default one (block 5: the hint is ignored)."""
    say("short rows", dim, kv, block)
    rng = np.random.default_rng(dim + block)
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=4, dim=dim, block=block, pool=700, seqs=7, max_ctx=500, prefill=True, max_rows=3
    )
    scale = dim**-0.5
    if kv == torch.bfloat16:
        kc, vc = bf16_round(kc), bf16_round(vc)
    want, dense = _oracle(kc, vc, tables, contexts, positions, seq_of, q, scale)
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    visible = np.minimum(contexts[seq_of], positions + 1)
    rows = np.stack([np.arange(seq_of.size), np.zeros(seq_of.size, np.int64)], axis=1)
    for partition in (64, 0):
        items = ops.expand_rows(rows, visible, partition)
        for short in (False, True):
            plan = ops.upload_plan(items, np.zeros((0, 4), np.int32), device, partition_size=partition,
                                   short_rows=short)  # fmt: skip
            got = ops.paged_attention_ragged(
                torch.from_numpy(q).to(device), torch.from_numpy(positions.astype(np.int32)).to(device),
                torch.from_numpy(seq_of.astype(np.int32)).to(device),
                torch.from_numpy(kc).to(device).to(kv), torch.from_numpy(vc).to(device).to(kv),
                torch.from_numpy(padded).to(device), torch.from_numpy(contexts.astype(np.int32)).to(device),
                scale, max_context_len=int(contexts.max()), plan=plan,
            ).cpu().numpy()  # fmt: skip
            assert np.max(np.abs(got - want)) < FP32_TOL, (partition, short)
            assert np.max(np.abs(got - dense)) < FP32_TOL, (partition, short)


@pytest.mark.parametrize("heads", [3, 4])
@pytest.mark.parametrize("block", [16, 5])
@pytest.mark.parametrize("kinds", ["f32<-f32", "bf16<-f32", "bf16<-bf16"])
def test_fused_decode_append_equals_append_then_attention(device, kinds, block, heads) -> None:
    """pkv_paged_attention_append: the row pass writes each decode row's new key and value to its
    slot and uses them as that position's key; the pools end bit for bit as after pkv_append and
    the rows match the oracle on the appended pools (block 5 has no fused instantiation: the call
    runs the append kernel first)."""
    say("fused append", kinds, block, heads)
    pool_dtype = torch.float32 if kinds.startswith("f32") else torch.bfloat16
    src_dtype = torch.float32 if kinds.endswith("f32") else torch.bfloat16
    rng = np.random.default_rng(block * 10 + heads)
    dim, seqs = 128, 9
    pool = seqs * -(-700 // block) + 8
    contexts = rng.integers(1, 700, seqs)
    perm = rng.permutation(pool)
    tables, offset = [], 0
    for c in contexts:
        n = -(-int(c) // block)
        tables.append(perm[offset : offset + n])
        offset += n
    width = max(len(t) for t in tables)
    padded = np.full((seqs, width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    positions = contexts - 1
    slots = np.asarray([int(t[p // block]) * block + p % block for t, p in zip(tables, positions)])
    g = torch.Generator(device=device)
    g.manual_seed(block * 10 + heads)
    kc = torch.randn((pool, block, heads, dim), generator=g, device=device).to(pool_dtype)
    vc = torch.randn((pool, block, heads, dim), generator=g, device=device).to(pool_dtype)
    q = torch.randn((seqs, heads, dim), generator=g, device=device)
    new_k = torch.randn((seqs, heads, dim), generator=g, device=device).to(src_dtype)
    new_v = torch.randn((seqs, heads, dim), generator=g, device=device).to(src_dtype)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    args = (q, to(positions.astype(np.int32)), to(np.arange(seqs, dtype=np.int32)))
    meta = (to(padded), to(contexts.astype(np.int32)), dim**-0.5)
    slot_d = to(slots.astype(np.int64))
    for partition in (0, 64):
        k_sep, v_sep = kc.clone(), vc.clone()
        ops.append_kv(k_sep, v_sep, new_k, new_v, slot_d)
        want = ops.paged_attention_ragged(*args, k_sep, v_sep, *meta, max_context_len=int(contexts.max()),
                                          partition_size=partition)  # fmt: skip
        k_fus, v_fus = kc.clone(), vc.clone()
        got = ops.paged_attention_ragged(*args, k_fus, v_fus, *meta, max_context_len=int(contexts.max()),
                                         partition_size=partition, append=(new_k, new_v, slot_d))  # fmt: skip
        assert torch.equal(k_fus.view(torch.int16) if pool_dtype == torch.bfloat16 else k_fus,
                           k_sep.view(torch.int16) if pool_dtype == torch.bfloat16 else k_sep)  # fmt: skip
        assert torch.equal(v_fus.view(torch.int16) if pool_dtype == torch.bfloat16 else v_fus,
                           v_sep.view(torch.int16) if pool_dtype == torch.bfloat16 else v_sep)  # fmt: skip
        assert float((got - want).abs().max()) < 1e-6, partition
        kh, vh = k_sep.float().cpu().numpy(), v_sep.float().cpu().numpy()
        qh = q.cpu().numpy()
        oracle, dense = _oracle(kh, vh, tables, contexts, positions, np.arange(seqs), qh, dim**-0.5)
        assert np.max(np.abs(got.cpu().numpy() - oracle)) < FP32_TOL, partition
        assert np.max(np.abs(got.cpu().numpy() - dense)) < FP32_TOL, partition


@pytest.mark.parametrize("kv", ["f32", "bf16"])
@pytest.mark.parametrize("heads", [4, 32], ids=["alone", "overlapped"])
def test_fused_append_beside_shared_prefix_tiles(device, heads, kv) -> None:
    """A decode batch whose sequences share a prefix: the plan reads the prefix as MFMA tiles and
    the fused append writes each row's new key and value (into its private last block) from the
    row pass, beside the tile pass (at 32 heads on the second stream). float32 new rows into
    float32 or bfloat16 pools (rounded to nearest even). Pools bit for bit as after pkv_append;
    outputs within 1e-6 of append-then-attention and 1e-5 of the oracle over the pools' values."""
    say("fused append beside prefix tiles", heads, kv)
    rng = np.random.default_rng(heads)
    dim, block, seqs = 128, 16, 64
    prefix = 40  # blocks: 640 shared tokens
    suffix = rng.integers(20, 300, seqs)
    contexts = prefix * block + suffix
    need = [-(-int(c) // block) - prefix for c in contexts]
    pool = prefix + sum(need)
    ids = rng.permutation(pool)
    shared = ids[:prefix].tolist()
    tables, offset = [], prefix
    for n in need:
        tables.append(np.asarray(shared + ids[offset : offset + n].tolist()))
        offset += n
    padded = np.zeros((seqs, max(len(t) for t in tables)), dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    positions = contexts - 1
    slots = np.asarray([int(t[p // block]) * block + p % block for t, p in zip(tables, positions)], np.int64)
    kc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    q, new_k, new_v = (rng.standard_normal((seqs, heads, dim)).astype(np.float32) for _ in range(3))
    seq_of = np.arange(seqs)
    kv_dtype = torch.float32 if kv == "f32" else torch.bfloat16
    plan = ops.plan_batch(seq_of, dim, heads, tables, contexts, block, query_positions=positions, kv_dtype=kv_dtype)
    assert plan.tiles.shape[0] >= 1, "prefix tiles"
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    args = (to(q), to(positions.astype(np.int32)), to(seq_of.astype(np.int32)))
    meta = (to(padded), to(contexts.astype(np.int32)), dim**-0.5)
    dplan = ops.upload_batch_plan(plan, device)
    k_sep, v_sep = to(kc).to(kv_dtype), to(vc).to(kv_dtype)
    ops.append_kv(k_sep, v_sep, to(new_k), to(new_v), to(slots))
    want = ops.paged_attention_ragged(*args, k_sep, v_sep, *meta, max_context_len=int(contexts.max()), plan=dplan)
    k_fus, v_fus = to(kc).to(kv_dtype), to(vc).to(kv_dtype)
    got = ops.paged_attention_ragged(*args, k_fus, v_fus, *meta, max_context_len=int(contexts.max()), plan=dplan,
                                     append=(to(new_k), to(new_v), to(slots)))  # fmt: skip
    assert torch.equal(k_fus, k_sep) and torch.equal(v_fus, v_sep)
    assert float((got - want).abs().max()) < 1e-6
    kh, vh = k_sep.float().cpu().numpy(), v_sep.float().cpu().numpy()
    oracle, dense = _oracle(kh, vh, tables, contexts, positions, seq_of, q, dim**-0.5)
    assert np.max(np.abs(got.cpu().numpy() - oracle)) < FP32_TOL
    assert np.max(np.abs(got.cpu().numpy() - dense)) < FP32_TOL
    if heads == 32:
        assert plan.rows.shape[0] * heads >= 2048, "the overlapped grid"


def _whole_tile_plan(seq_of, positions, contexts, dim, partition, device, *, explicit_merge):
    """Every run of >= 2 rows of one sequence as whole tiles; the rest in the row pass."""
    rows, tiles = ops.plan_rows(seq_of, dim, min_tile_rows=2)
    tiles[:, 3] = ops.TILE_WHOLE
    visible = np.minimum(contexts[seq_of], positions + 1)
    merge = None
    if explicit_merge:
        merge = ops.merge_rows_for(seq_of.size, tiles, visible, partition or 512)
    items = ops.expand_rows(rows, visible, partition)
    return ops.upload_plan(items, tiles, device, partition_size=partition, merge=merge)


@pytest.mark.parametrize("dim", [32, 64, 128, 256])
@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("block", [1, 16])
def test_whole_tiles_match_the_oracle(device, dim, kv, block) -> None:
    """Whole tiles: one workgroup per (tile, head) over every visible key, final rows written
    directly, beside row-pass rows that the reduce merges. At block_size 1 the contexts exceed
    the 1028 table entries a workgroup stages at once, so the staged window moves."""
    say("whole tiles", dim, kv, block)
    rng = np.random.default_rng(dim + block + (7 if kv == torch.bfloat16 else 0))
    max_ctx = 1500 if block == 1 else 900
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=2, dim=dim, block=block, pool=5 * max_ctx // block + 8, seqs=6, max_ctx=max_ctx,
        prefill=True, max_rows=150,
    )  # fmt: skip
    scale = dim**-0.5
    if kv == torch.bfloat16:
        kc, vc = bf16_round(kc), bf16_round(vc)
    want, dense = _oracle(kc, vc, tables, contexts, positions, seq_of, q, scale)
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    args = (
        torch.from_numpy(q).to(device), torch.from_numpy(positions.astype(np.int32)).to(device),
        torch.from_numpy(seq_of.astype(np.int32)).to(device),
        torch.from_numpy(kc).to(device).to(kv), torch.from_numpy(vc).to(device).to(kv),
        torch.from_numpy(padded).to(device), torch.from_numpy(contexts.astype(np.int32)).to(device),
        scale,
    )  # fmt: skip
    for partition in (0, 64):
        for explicit in (False, True):
            plan = _whole_tile_plan(seq_of, positions, contexts, dim, partition, device,
                                    explicit_merge=explicit)  # fmt: skip
            got = ops.paged_attention_ragged(
                *args, max_context_len=int(contexts.max()), plan=plan
            ).cpu().numpy()  # fmt: skip
            assert np.max(np.abs(got - want)) < FP32_TOL, (partition, explicit)
            assert np.max(np.abs(got - dense)) < FP32_TOL, (partition, explicit)


@pytest.mark.parametrize("dim", [32, 64, 128, 256])
@pytest.mark.parametrize("block", [1, 5, 16])
@pytest.mark.parametrize("whole", [False, True], ids=["partitions", "whole"])
def test_tiles_beside_rows_equal_tiles_alone(device, dim, block, whole) -> None:
    """Beside row-pass rows the float32 tile pass is a persistent grid that loads key and value
    tiles straight into LDS (or, with the dominant-tiles hint, three register-staged workgroups
    per CU); on its own it runs one workgroup per item through registers. All form the same sums
    in the same order, so the tile rows come out bit-identical; and they match the oracle. At
    block_size 1 whole tiles move their staged table window."""
    say("tile paths", dim, block, whole)
    rng = np.random.default_rng(dim * 7 + block + whole)
    max_ctx = 1400 if block == 1 else 800
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=2, dim=dim, block=block, pool=5 * max_ctx // block + 8, seqs=6, max_ctx=max_ctx,
        prefill=True, max_rows=150,
    )  # fmt: skip
    # Two more decode sequences, so the batch surely has row-pass rows next to the tiles.
    extra = [rng.permutation(kc.shape[0])[: -(-c // block)] for c in (max_ctx - 3, 37)]
    tables = list(tables) + extra
    contexts = np.concatenate([contexts, [max_ctx - 3, 37]])
    positions = np.concatenate([positions, [max_ctx - 4, 36]])
    seq_of = np.concatenate([seq_of, [len(tables) - 2, len(tables) - 1]])
    q = np.concatenate([q, rng.standard_normal((2,) + q.shape[1:]).astype(np.float32)])
    scale = dim**-0.5
    want, _ = _oracle(kc, vc, tables, contexts, positions, seq_of, q, scale)
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    args = (
        torch.from_numpy(q).to(device), torch.from_numpy(positions.astype(np.int32)).to(device),
        torch.from_numpy(seq_of.astype(np.int32)).to(device),
        torch.from_numpy(kc).to(device), torch.from_numpy(vc).to(device),
        torch.from_numpy(padded).to(device), torch.from_numpy(contexts.astype(np.int32)).to(device),
        scale,
    )  # fmt: skip
    rows, tiles = ops.plan_rows(seq_of, dim, min_tile_rows=2)
    assert rows.shape[0] >= 2 and tiles.shape[0] >= 2
    if whole:
        tiles[:, 3] = ops.TILE_WHOLE
    tile_rows = np.concatenate([np.arange(t0, t0 + n) for t0, n, _, _ in tiles])
    visible = np.minimum(contexts[seq_of], positions + 1)
    for partition in (0, 64):
        beside = ops.upload_plan(ops.expand_rows(rows, visible, partition), tiles, device,
                                 partition_size=partition)  # fmt: skip
        alone = ops.upload_plan(np.zeros((0, 2), np.int32), tiles, device, partition_size=partition,
                                merge=ops.merge_rows_for(seq_of.size, tiles, visible, partition or 512)
                                if whole else None)  # fmt: skip
        mc = int(contexts.max())
        got = ops.paged_attention_ragged(*args, max_context_len=mc, plan=beside).cpu().numpy()
        solo = ops.paged_attention_ragged(*args, max_context_len=mc, plan=alone).cpu().numpy()
        dominant = dataclasses.replace(beside, dominant_tiles=True)
        hinted = ops.paged_attention_ragged(*args, max_context_len=mc, plan=dominant).cpu().numpy()
        assert np.max(np.abs(got - want)) < FP32_TOL, partition
        assert np.array_equal(got[tile_rows], solo[tile_rows]), partition
        assert np.array_equal(hinted, got), partition


@pytest.mark.parametrize("dim", [64, 128])
@pytest.mark.parametrize("block", [5, 16])
@pytest.mark.parametrize("whole", [False, True], ids=["partitions", "whole"])
def test_caller_rows_reach_the_rows_the_plan_orders(device, dim, block, whole) -> None:
    """caller_rows[t] is the row of queries and out that planner row t reads and writes. With
    the queries permuted and the permutation passed, the row pass, the tile pass (alone, and at
    block 16 beside a row pass large enough for the second stream and the direct-to-LDS grid)
    and the reduce write bit for bit what the unpermuted call writes, into the permuted rows. A
    caller row outside the batch skips its query: its output row keeps what it held."""
    say("caller rows", dim, block, whole)
    rng = np.random.default_rng(dim + block + 3 * whole)
    heads, max_ctx = 4, 700
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=heads, dim=dim, block=block, pool=5 * max_ctx // block + 8, seqs=5, max_ctx=max_ctx,
        prefill=True, max_rows=120,
    )  # fmt: skip
    # decode rows of 60 more sequences: at partition 64 the row pass then has more than 2,048
    # workgroups (items x heads), so the tile pass runs beside it on the second stream
    decode_ctx = rng.integers(600, max_ctx, 60)
    need = [-(-int(c) // block) for c in decode_ctx]
    first, extra = kc.shape[0], sum(need)
    kc = np.concatenate([kc, rng.standard_normal((extra,) + kc.shape[1:]).astype(np.float32)])
    vc = np.concatenate([vc, rng.standard_normal((extra,) + vc.shape[1:]).astype(np.float32)])
    free = iter(range(first, first + extra))  # fresh blocks for the decode sequences
    tables = list(tables) + [np.asarray([next(free) for _ in range(n)]) for n in need]
    seq_of = np.concatenate([seq_of, np.arange(len(contexts), len(contexts) + decode_ctx.size)])
    contexts = np.concatenate([contexts, decode_ctx])
    positions = np.concatenate([positions, decode_ctx - 1])
    q = np.concatenate([q, rng.standard_normal((decode_ctx.size, heads, dim)).astype(np.float32)])
    total, scale = seq_of.size, dim**-0.5
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    meta = (to(positions.astype(np.int32)), to(seq_of.astype(np.int32)), to(kc), to(vc), to(padded),
            to(contexts.astype(np.int32)), scale)  # fmt: skip
    rows, tiles = ops.plan_rows(seq_of, dim, min_tile_rows=2)
    assert tiles.shape[0] >= 2
    if whole:
        tiles[:, 3] = ops.TILE_WHOLE
    visible = np.minimum(contexts[seq_of], positions + 1)
    perm = rng.permutation(total)  # planner row t lives at caller row perm[t]
    q_caller = np.empty_like(q)
    q_caller[perm] = q
    bad = perm.copy()
    skipped = int(rng.integers(total))
    bad[skipped] = total  # outside the batch
    for partition in (0, 64):
        plan = ops.upload_plan(ops.expand_rows(rows, visible, partition), tiles, device, partition_size=partition)
        mc = int(contexts.max())
        want = ops.paged_attention_ragged(to(q), *meta, max_context_len=mc, plan=plan)
        got = ops.paged_attention_ragged(to(q_caller), *meta, max_context_len=mc, plan=plan,
                                         caller_rows=to(perm.astype(np.int32)))  # fmt: skip
        assert torch.equal(got[to(perm)], want), partition
        held = torch.full_like(want, float("nan"))
        ops.paged_attention_ragged(to(q_caller), *meta, max_context_len=mc, plan=plan, out=held,
                                   caller_rows=to(bad.astype(np.int32)))  # fmt: skip
        kept = np.delete(np.arange(total), skipped)
        assert torch.equal(held[to(perm[kept])], want[to(kept)]), partition
        assert bool(torch.isnan(held[int(perm[skipped])]).all()), partition
        if partition == 64 and block == 16:
            assert plan.num_rows * heads >= 2048, "the overlapped grid"


@pytest.mark.parametrize("block", [16, 5])
def test_caller_rows_with_the_fused_append(device, block) -> None:
    """The fused decode append takes query t's new key and value from row caller_rows[t] of the
    new rows and writes it to slot_mapping[caller_rows[t]]: permuted inputs give the same pools
    bit for bit and the same outputs in the permuted rows (block 5 appends before the call)."""
    say("caller rows, fused append", block)
    rng = np.random.default_rng(40 + block)
    heads, dim, seqs = 4, 128, 11
    pool = seqs * -(-700 // block) + 8
    contexts = rng.integers(1, 700, seqs)
    ids = rng.permutation(pool)
    tables, offset = [], 0
    for c in contexts:
        n = -(-int(c) // block)
        tables.append(ids[offset : offset + n])
        offset += n
    padded = np.full((seqs, max(len(t) for t in tables)), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    positions = contexts - 1
    slots = np.asarray([int(t[p // block]) * block + p % block for t, p in zip(tables, positions)], np.int64)
    to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
    kc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    q, new_k, new_v = (rng.standard_normal((seqs, heads, dim)).astype(np.float32) for _ in range(3))
    perm = rng.permutation(seqs)  # query t at caller row perm[t]

    def caller(a: np.ndarray) -> np.ndarray:
        out = np.empty_like(a)
        out[perm] = a
        return out

    meta = (to(padded), to(contexts.astype(np.int32)), dim**-0.5)
    args = (to(positions.astype(np.int32)), to(np.arange(seqs, dtype=np.int32)))
    k_plain, v_plain = to(kc), to(vc)
    want = ops.paged_attention_ragged(to(q), *args, k_plain, v_plain, *meta, max_context_len=int(contexts.max()),
                                      partition_size=64, append=(to(new_k), to(new_v), to(slots)))  # fmt: skip
    k_perm, v_perm = to(kc), to(vc)
    got = ops.paged_attention_ragged(
        to(caller(q)), *args, k_perm, v_perm, *meta, max_context_len=int(contexts.max()), partition_size=64,
        append=(to(caller(new_k)), to(caller(new_v)), to(caller(slots))), caller_rows=to(perm.astype(np.int32)),
    )  # fmt: skip
    assert torch.equal(k_perm, k_plain) and torch.equal(v_perm, v_plain)
    assert torch.equal(got[to(perm)], want)


@pytest.mark.parametrize("kv", [torch.float32, torch.bfloat16], ids=["f32", "bf16"])
@pytest.mark.parametrize("whole", [False, True], ids=["partitions", "whole"])
def test_nan_in_a_block_no_table_holds_reaches_no_output(device, kv, whole) -> None:
    """The tile pass loads the keys past a tile's end (its last 32-key step is partial) as zeros,
    on both staging paths: beside row-pass rows (float32: straight into LDS) and alone (through
    registers). So a pool block that no table holds may contain NaN or inf, as the reference
    never reads it, and no output changes."""
    say("unreferenced NaN block", kv, whole)
    rng = np.random.default_rng(77 + whole)
    dim, block, max_ctx = 128, 16, 700
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=2, dim=dim, block=block, pool=5 * max_ctx // block + 8, seqs=6, max_ctx=max_ctx,
        prefill=True, max_rows=150,
    )  # fmt: skip
    extra = [rng.permutation(kc.shape[0])[: -(-c // block)] for c in (max_ctx - 3, 37)]
    tables = list(tables) + extra
    contexts = np.concatenate([contexts, [max_ctx - 3, 37]])
    positions = np.concatenate([positions, [max_ctx - 4, 36]])
    seq_of = np.concatenate([seq_of, [len(tables) - 2, len(tables) - 1]])
    q = np.concatenate([q, rng.standard_normal((2,) + q.shape[1:]).astype(np.float32)])
    spare = sorted(set(range(1, kc.shape[0])) - {int(b) for t in tables for b in t})[0]
    tables = [np.where(np.asarray(t) == 0, spare, t) for t in tables]  # no table holds block 0
    kc[0], vc[0] = np.nan, np.inf
    scale = dim**-0.5
    if kv == torch.bfloat16:
        kc, vc = bf16_round(kc), bf16_round(vc)
    want, _ = _oracle(kc, vc, tables, contexts, positions, seq_of, q, scale)
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    args = (
        torch.from_numpy(q).to(device), torch.from_numpy(positions.astype(np.int32)).to(device),
        torch.from_numpy(seq_of.astype(np.int32)).to(device),
        torch.from_numpy(kc).to(device).to(kv), torch.from_numpy(vc).to(device).to(kv),
        torch.from_numpy(padded).to(device), torch.from_numpy(contexts.astype(np.int32)).to(device),
        scale,
    )  # fmt: skip
    rows, tiles = ops.plan_rows(seq_of, dim, min_tile_rows=2)
    visible = np.minimum(contexts[seq_of], positions + 1)
    assert rows.shape[0] >= 2 and tiles.shape[0] >= 2
    assert any(visible[t0 : t0 + n].max() % 32 for t0, n, _, _ in tiles)  # a partial last key step
    if whole:
        tiles[:, 3] = ops.TILE_WHOLE
    tile_rows = np.concatenate([np.arange(t0, t0 + n) for t0, n, _, _ in tiles])
    merge = ops.merge_rows_for(seq_of.size, tiles, visible, 512) if whole else None
    mc = int(contexts.max())
    beside = ops.upload_plan(ops.expand_rows(rows, visible, 0), tiles, device, merge=merge)
    alone = ops.upload_plan(np.zeros((0, 2), np.int32), tiles, device, merge=merge)
    for name, plan, done in (("beside", beside, np.arange(seq_of.size)), ("alone", alone, tile_rows)):
        got = ops.paged_attention_ragged(*args, max_context_len=mc, plan=plan).cpu().numpy()[done]
        assert np.all(np.isfinite(got)), name
        assert np.max(np.abs(got - want[done])) < FP32_TOL, name


@pytest.mark.parametrize("block", [16, 5])
@pytest.mark.parametrize("whole", [False, True], ids=["partitions", "whole"])
@pytest.mark.parametrize("short", [False, True], ids=["rows", "lean-rows"])
def test_bf16_tiles_beside_rows_in_every_grid_shape(device, block, whole, short) -> None:
    """A bfloat16 pool's tile pass beside row-pass rows (two register-staged workgroups per CU,
    three with the dominant-tiles hint, beside full or lean row workgroups) and alone (one per
    item) give bit-identical tile rows, and match the oracle on the bf16-rounded pools."""
    say("bf16 tile grids", block, whole, short)
    rng = np.random.default_rng(90 + block + 2 * whole + 4 * short)
    dim, max_ctx = 128, 800
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=2, dim=dim, block=block, pool=5 * max_ctx // block + 8, seqs=6, max_ctx=max_ctx,
        prefill=True, max_rows=150,
    )  # fmt: skip
    extra = [rng.permutation(kc.shape[0])[: -(-c // block)] for c in (max_ctx - 3, 37)]
    tables = list(tables) + extra
    contexts = np.concatenate([contexts, [max_ctx - 3, 37]])
    positions = np.concatenate([positions, [max_ctx - 4, 36]])
    seq_of = np.concatenate([seq_of, [len(tables) - 2, len(tables) - 1]])
    q = np.concatenate([q, rng.standard_normal((2,) + q.shape[1:]).astype(np.float32)])
    kc, vc = bf16_round(kc), bf16_round(vc)
    scale = dim**-0.5
    want, _ = _oracle(kc, vc, tables, contexts, positions, seq_of, q, scale)
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    args = (
        torch.from_numpy(q).to(device), torch.from_numpy(positions.astype(np.int32)).to(device),
        torch.from_numpy(seq_of.astype(np.int32)).to(device),
        torch.from_numpy(kc).to(device).to(torch.bfloat16), torch.from_numpy(vc).to(device).to(torch.bfloat16),
        torch.from_numpy(padded).to(device), torch.from_numpy(contexts.astype(np.int32)).to(device),
        scale,
    )  # fmt: skip
    rows, tiles = ops.plan_rows(seq_of, dim, min_tile_rows=2)
    assert rows.shape[0] >= 2 and tiles.shape[0] >= 2
    if whole:
        tiles[:, 3] = ops.TILE_WHOLE
    tile_rows = np.concatenate([np.arange(t0, t0 + n) for t0, n, _, _ in tiles])
    visible = np.minimum(contexts[seq_of], positions + 1)
    merge = ops.merge_rows_for(seq_of.size, tiles, visible, 512) if whole else None
    mc = int(contexts.max())
    beside = ops.upload_plan(ops.expand_rows(rows, visible, 0), tiles, device, merge=merge, short_rows=short)
    outs = [
        ops.paged_attention_ragged(*args, max_context_len=mc, plan=plan).cpu().numpy()
        for plan in (beside, dataclasses.replace(beside, dominant_tiles=True))
    ]
    alone = ops.upload_plan(np.zeros((0, 2), np.int32), tiles, device, merge=merge)
    solo = ops.paged_attention_ragged(*args, max_context_len=mc, plan=alone).cpu().numpy()
    assert np.max(np.abs(outs[0] - want)) < FP32_TOL
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(outs[0][tile_rows], solo[tile_rows])


def _attention_skipping_bad_blocks(q, positions, seq_of, kc, vc, tables, contexts, scale):
    """float64 attention in which keys whose block id lies outside the pool take no part (the
    library's rule for such table entries; the reference would raise on them)."""
    pool, block = kc.shape[0], kc.shape[1]
    out = np.zeros(q.shape, dtype=np.float64)
    for t in range(q.shape[0]):
        s = int(seq_of[t])
        visible = min(int(contexts[s]), int(positions[t]) + 1)
        keep = [p for p in range(visible) if 0 <= tables[s][p // block] < pool]
        if not keep:
            continue
        k = np.stack([kc[tables[s][p // block], p % block] for p in keep]).astype(np.float64)
        v = np.stack([vc[tables[s][p // block], p % block] for p in keep]).astype(np.float64)
        scores = np.einsum("hd,nhd->hn", q[t].astype(np.float64), k) * scale
        w = np.exp(scores - scores.max(axis=1, keepdims=True))
        w /= w.sum(axis=1, keepdims=True)
        out[t] = np.einsum("hn,nhd->hd", w, v)
    return out


@pytest.mark.parametrize("block", [16, 5])
@pytest.mark.parametrize("bad", [-1, 10**6], ids=["negative", "past-pool"])
def test_blocks_outside_the_pool_are_skipped_by_every_pass(device, block, bad) -> None:
    """A table entry outside [0, num_blocks) inside a visible context is never read: the row
    pass, the tile pass beside it (direct-to-LDS stages) and the tile pass alone (registers)
    all leave its keys out of the softmax."""
    say("bad blocks", block, bad)
    rng = np.random.default_rng(block + (bad > 0))
    dim, heads = 128, 2
    kc, vc, tables, contexts, positions, seq_of, q = _ragged_case(
        rng, heads=heads, dim=dim, block=block, pool=2000, seqs=6, max_ctx=900, prefill=True,
        max_rows=150,
    )  # fmt: skip
    extra = rng.permutation(kc.shape[0])[: -(-700 // block)]
    tables = [np.asarray(t).copy() for t in tables] + [extra]
    contexts = np.concatenate([contexts, [700]])
    positions = np.concatenate([positions, [699]])
    seq_of = np.concatenate([seq_of, [len(tables) - 1]])
    q = np.concatenate([q, rng.standard_normal((1,) + q.shape[1:]).astype(np.float32)])
    for t in tables:  # spoil about one in eight of each table's used entries
        t[rng.random(t.size) < 0.125] = bad
    scale = dim**-0.5
    want = _attention_skipping_bad_blocks(q, positions, seq_of, kc, vc, tables, contexts, scale)
    width = max(len(t) for t in tables)
    padded = np.full((len(tables), width), -7, dtype=np.int32)
    for i, t in enumerate(tables):
        padded[i, : len(t)] = t
    args = (
        torch.from_numpy(q).to(device), torch.from_numpy(positions.astype(np.int32)).to(device),
        torch.from_numpy(seq_of.astype(np.int32)).to(device),
        torch.from_numpy(kc).to(device), torch.from_numpy(vc).to(device),
        torch.from_numpy(padded).to(device), torch.from_numpy(contexts.astype(np.int32)).to(device),
        scale,
    )  # fmt: skip
    mc = int(contexts.max())
    rows, tiles = ops.plan_rows(seq_of, dim, min_tile_rows=2)
    assert rows.shape[0] >= 1 and tiles.shape[0] >= 2
    visible = np.minimum(contexts[seq_of], positions + 1)
    tile_rows = np.concatenate([np.arange(t0, t0 + n) for t0, n, _, _ in tiles])
    row_only = ops.paged_attention_ragged(*args, max_context_len=mc).cpu().numpy()
    beside = ops.paged_attention_ragged(
        *args, max_context_len=mc,
        plan=ops.upload_plan(ops.expand_rows(rows, visible, 0), tiles, device),
    ).cpu().numpy()  # fmt: skip
    alone = ops.paged_attention_ragged(
        *args, max_context_len=mc, plan=ops.upload_plan(np.zeros((0, 2), np.int32), tiles, device),
    ).cpu().numpy()  # fmt: skip
    assert np.max(np.abs(row_only - want)) < FP32_TOL
    assert np.max(np.abs(beside - want)) < FP32_TOL
    assert np.max(np.abs(alone[tile_rows] - want[tile_rows])) < FP32_TOL


def test_poisoned_slots_and_padding_are_never_read(device) -> None:
    say("poison")
    rng = np.random.default_rng(9)
    heads, dim, block = 2, 8, 4
    kc = np.full((6, block, heads, dim), np.inf, dtype=np.float32)
    vc = np.full_like(kc, np.nan)
    flat_k = rng.standard_normal((5, heads, dim)).astype(np.float32)
    flat_v = rng.standard_normal((5, heads, dim)).astype(np.float32)
    table = np.asarray([4, 1])
    kc[4], vc[4] = flat_k[:4], flat_v[:4]
    kc[1, 0], vc[1, 0] = flat_k[4], flat_v[4]
    q = rng.standard_normal((2, heads, dim)).astype(np.float32)
    got = _run_kernel(device, kc, vc, [table], np.asarray([5]), np.asarray([2, 4]), np.asarray([0, 0]),
                      q, 0.35)  # fmt: skip
    want = dense_attention(q, flat_k, flat_v, 0.35, np.asarray([2, 4]))
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) < FP32_TOL


def test_a_fully_masked_query_is_zero(device) -> None:
    say("masked")
    rng = np.random.default_rng(2)
    kc = rng.standard_normal((3, 4, 1, 16)).astype(np.float32)
    got = _run_kernel(device, kc, kc.copy(), [np.asarray([2, 0])], np.asarray([6]),
                      np.asarray([-1, 0]), np.asarray([0, 0]), np.ones((2, 1, 16), np.float32), 0.25)  # fmt: skip
    assert np.array_equal(got[0], np.zeros((1, 16), np.float32))
    assert np.allclose(got[1], kc[2, 0])


# --- the benchmark configurations at full size ---------------------------------------------------


def _torch_dense(batch, rows):
    """float64 dense attention of selected query rows, on the device (torch reference)."""
    out = {}
    for t in rows:
        s = int(batch.host_seq[t])
        ctx = int(batch.host_context[s])
        visible = min(ctx, int(batch.host_positions[t]) + 1)
        table = torch.from_numpy(batch.host_tables[s].astype(np.int64)).to(batch.queries.device)
        k = batch.key_cache[table].reshape(-1, *batch.key_cache.shape[2:])[:visible].double()
        v = batch.value_cache[table].reshape(-1, *batch.value_cache.shape[2:])[:visible].double()
        q = batch.queries[t].double()
        scores = torch.einsum("hd,jhd->hj", q, k) * batch.scale
        out[t] = torch.einsum("hj,jhd->hd", torch.softmax(scores, dim=1), v).float()
    return out


def _run_batch(batch, partition=0, plan=True):
    ops.append_kv(batch.key_cache, batch.value_cache, batch.new_keys, batch.new_values, batch.slot_mapping)
    return ops.paged_attention_ragged(
        batch.queries, batch.query_positions, batch.query_seq, batch.key_cache, batch.value_cache,
        batch.block_tables, batch.context_lens, batch.scale, max_context_len=batch.max_context_len,
        partition_size=partition, plan=batch.plan if plan else None,
    )  # fmt: skip


def _run_fused(batch):
    """The decode step as one pkv_paged_attention_append call (append done by the row pass)."""
    return ops.paged_attention_ragged(
        batch.queries, batch.query_positions, batch.query_seq, batch.key_cache, batch.value_cache,
        batch.block_tables, batch.context_lens, batch.scale, max_context_len=batch.max_context_len,
        plan=batch.plan, append=(batch.new_keys, batch.new_values, batch.slot_mapping),
    )  # fmt: skip


def _oracle_rows(batch, out, seqs, tol):
    """CPU oracle (reference algorithm, 128-key tiles) on every row of the chosen sequences."""
    got = out.cpu().numpy()
    heads, dim = batch.key_cache.shape[2], batch.key_cache.shape[3]
    for s in seqs:
        keys, values, q, pos = batch.host_rows(s)
        pool_k = keys.reshape(-1, 1, heads, dim)
        pool_v = values.reshape(-1, 1, heads, dim)
        want = paged_attention(q, pos, pool_k, pool_v, np.arange(keys.shape[0]),
                               int(batch.host_context[s]), batch.scale, tile_blocks=128)  # fmt: skip
        rows = np.nonzero(batch.host_seq == s)[0]
        assert np.max(np.abs(got[rows] - want)) < tol, s


def test_config2_decode_64x4k_matches_the_oracle(device) -> None:
    from paged_kv_serving_amd.workloads import decode_batch

    say("config 2: build")
    batch = decode_batch(seed=0, device=device)
    say("config 2: fused append + attention (the bench's step)")
    fused = _run_fused(batch)
    torch.cuda.synchronize()
    # appended rows landed, bit-exact
    slots = batch.slot_mapping
    assert torch.equal(batch.key_cache.view(-1, 32, 128)[slots], batch.new_keys)
    assert torch.equal(batch.value_cache.view(-1, 32, 128)[slots], batch.new_values)
    say("config 2: run")
    out = _run_batch(batch)  # appends the same rows again, then attends
    assert float((fused - out).abs().max()) < 1e-6
    # every sequence against the float64 torch reference
    ref = _torch_dense(batch, range(batch.num_queries))
    worst = max(float((out[t] - ref[t]).abs().max()) for t in ref)
    say("config 2: worst vs float64 torch", worst)
    assert worst < FP32_TOL
    # a sample of sequences against the CPU oracle (reference algorithm, tile_blocks 8)
    got = out.cpu().numpy()
    for s in (0, 17, 63):
        keys, values, q, pos = batch.host_rows(s)
        pool_k = keys.reshape(1, -1, 32, 128)
        pool_v = values.reshape(1, -1, 32, 128)
        want = paged_attention(q, pos, pool_k.transpose(1, 0, 2, 3), pool_v.transpose(1, 0, 2, 3),
                               np.arange(keys.shape[0]), int(batch.host_context[s]), batch.scale,
                               tile_blocks=128)  # fmt: skip
        assert np.max(np.abs(got[s] - want[0])) < FP32_TOL, s
    # partition size changes nothing beyond rounding
    for partition in (64, 256, 1024):
        other = ops.paged_attention_ragged(
            batch.queries, batch.query_positions, batch.query_seq, batch.key_cache,
            batch.value_cache, batch.block_tables, batch.context_lens, batch.scale,
            max_context_len=batch.max_context_len, partition_size=partition,
        )  # fmt: skip
        assert float((other - out).abs().max()) < FP32_TOL, partition
    # cached loads (the shared-prefix hint) give the same bits as the streaming loads
    assert not batch.plan.shared_kv and batch.plan.partition_size == 512
    cached = ops.paged_attention_ragged(
        batch.queries, batch.query_positions, batch.query_seq, batch.key_cache, batch.value_cache,
        batch.block_tables, batch.context_lens, batch.scale, max_context_len=batch.max_context_len,
        plan=batch.plan, shared_kv=True,
    )  # fmt: skip
    assert torch.equal(cached, out)


def test_config3_mixed_prefill_and_decode_matches_the_oracle(device) -> None:
    """8 chunked-prefill rows of 512 tokens at offsets U[0, 2048] (MFMA tiles) plus 120 decode
    rows with contexts U[256, 4096] (row pass), 32 heads x 128, fp32, one ragged call."""
    from paged_kv_serving_amd.workloads import mixed_batch

    say("config 3: build")
    batch = mixed_batch(seed=0, device=device)
    assert batch.plan.num_tiles == 64
    assert set(batch.plan.rows[:, 0].tolist()) == set(range(4096, 4216)), "decode rows: row pass"
    say("config 3: run")
    out = _run_batch(batch)
    torch.cuda.synchronize()
    # every 8th prefill row and every decode row against float64 torch
    rows = list(range(0, 4096, 8)) + list(range(4096, batch.num_queries))
    ref = _torch_dense(batch, rows)
    worst = max(float((out[t] - ref[t]).abs().max()) for t in ref)
    say("config 3: worst vs float64 torch", worst)
    assert worst < FP32_TOL
    _oracle_rows(batch, out, (0, 5, 8, 100), FP32_TOL)
    # the row pass alone computes the same thing
    rows_only = _run_batch(batch, plan=False)
    assert float((rows_only - out).abs().max()) < FP32_TOL


def test_config5_long_context_bf16_matches_the_oracle(device) -> None:
    """16 sequences at 32,768 context, bf16 K/V, 40k-block shuffled pool, split-context."""
    from paged_kv_serving_amd.workloads import long_context_batch

    say("config 5: build")
    batch = long_context_batch(seed=0, device=device)
    fused = _run_fused(batch)
    torch.cuda.synchronize()
    slots = batch.slot_mapping
    want_bits = batch.new_keys.to(torch.bfloat16).view(torch.int16)
    assert torch.equal(batch.key_cache.view(-1, 32, 128)[slots].view(torch.int16), want_bits)
    want_bits = batch.new_values.to(torch.bfloat16).view(torch.int16)
    assert torch.equal(batch.value_cache.view(-1, 32, 128)[slots].view(torch.int16), want_bits)
    out = _run_batch(batch)
    assert float((fused - out).abs().max()) < 1e-6
    ref = _torch_dense(batch, range(batch.num_queries))  # on the stored (bf16) K/V, in float64
    worst = max(float((out[t] - ref[t]).abs().max()) for t in ref)
    say("config 5: worst vs float64 torch on bf16 K/V", worst)
    assert worst < FP32_TOL
    _oracle_rows(batch, out, (0, 15), FP32_TOL)


def test_config4_prefix_sharing_cow_then_decode(device) -> None:
    """256 children fork a 1016-token prefix; reserve() COWs the partial shared block once per
    child (pairs from the host BlockManager); one batched copy launch, then one decode step."""
    from paged_kv_serving_amd.workloads import prefix_sharing_step

    say("config 4: build")
    step = prefix_sharing_step(seed=0, device=device)
    assert len(step.host_pairs) == 256 and step.shared_blocks == 64
    assert len({src for src, _ in step.host_pairs}) == 1  # every child copies the partial block
    assert len({dst for _, dst in step.host_pairs}) == 256
    src = step.host_pairs[0][0]
    before_k = step.key_cache[0, src].clone()
    ops.copy_blocks(step.key_cache, step.value_cache, step.cow_pairs)
    dsts = torch.tensor([d for _, d in step.host_pairs], device=device)
    assert torch.equal(step.key_cache[0, dsts], before_k.expand(256, *before_k.shape))
    assert torch.equal(step.value_cache[0, dsts], step.value_cache[0, src].expand(256, *before_k.shape))
    assert torch.equal(step.key_cache[0, src], before_k)
    say("config 4: decode")
    out = _run_batch(step.decode)
    torch.cuda.synchronize()
    ref = _torch_dense(step.decode, range(0, 256, 5))
    worst = max(float((out[t] - ref[t]).abs().max()) for t in ref)
    say("config 4: worst vs float64 torch", worst)
    assert worst < FP32_TOL
    _oracle_rows(step.decode, out, (0, 255), FP32_TOL)
    # the planner computed the shared 1008-token prefix as tiles over three 336-key partitions
    plan = step.decode.plan
    assert plan.partition_size == 336 and not plan.shared_kv
    assert plan.tiles.cpu().tolist() == [[64 * i, 64, 0, 3] for i in range(4)]
    d = step.decode
    common = (d.queries, d.query_positions, d.query_seq, d.key_cache, d.value_cache, d.block_tables,
              d.context_lens, d.scale)  # fmt: skip
    # the plain plan (every row streams its whole context) agrees within rounding
    plain = ops.paged_attention_ragged(*common, max_context_len=d.max_context_len, partition_size=336)
    assert float((plain - out).abs().max()) < FP32_TOL
    # the load hint only changes how K/V rows are loaded: same bits either way
    runs = [
        ops.paged_attention_ragged(*common, max_context_len=d.max_context_len, plan=plan, shared_kv=flag)
        for flag in (False, True)
    ]
    assert torch.equal(runs[0], runs[1]) and torch.equal(runs[0], out)
    # a plan's partition indices belong to its partition size
    with pytest.raises(ValueError, match="partition"):
        ops.paged_attention_ragged(*common, max_context_len=d.max_context_len, plan=plan, partition_size=512)
    # every child writes its own copied block and the prefix tiles cover no new position, so the
    # bench and the runner fuse the append into the call; the fused step agrees with append-then-
    # attention (the batch's rows were appended above, so this rewrites the same values)
    assert d.fusable_append()
    fused = _run_fused(d)
    assert float((fused - out).abs().max()) < 1e-6


def test_empty_inputs_leave_the_pools_alone(device) -> None:
    """Zero tokens, zero copy pairs, zero query rows and zero logits rows are no-ops: every entry
    point returns before launching, and the pools keep their bits."""
    say("empty inputs")
    heads, dim, block = 2, 32, 4
    keys = torch.randn((1, 6, block, heads, dim), device=device)
    values = torch.randn_like(keys)
    before = (keys.clone(), values.clone())
    none = torch.zeros((0, heads, dim), device=device)
    no_slots = torch.zeros(0, dtype=torch.int64, device=device)
    ops.append_kv(keys[0], values[0], none, none, no_slots)
    ops.copy_blocks(keys, values, torch.zeros((0, 2), dtype=torch.int64, device=device))
    cos = torch.ones((8, dim // 2), device=device)
    rotated = ops.rope_append(keys[0], values[0], none, none, none, no_slots, cos, torch.zeros_like(cos), no_slots)
    assert rotated.shape == (0, heads, dim)
    out = ops.paged_attention_ragged(
        none, torch.zeros(0, dtype=torch.int32, device=device), torch.zeros(0, dtype=torch.int32, device=device),
        keys[0], values[0], torch.zeros((1, 2), dtype=torch.int32, device=device),
        torch.ones(1, dtype=torch.int32, device=device), dim**-0.5, max_context_len=1,
    )  # fmt: skip
    assert out.shape == (0, heads, dim)
    assert ops.greedy_tokens(torch.zeros((0, 16), device=device)).shape == (0,)
    torch.cuda.synchronize()
    assert torch.equal(keys, before[0]) and torch.equal(values, before[1])
