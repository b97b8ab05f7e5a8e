"""Pin the CPU oracle's paged attention before trusting it as the GPU checker.

The reference commits no golden vectors for this path, so the oracle (a restatement of
attention.py:42-121) is pinned by what the mathematics fixes:

* the float64 closed form (one softmax over each query's whole visible score row);
* the reference test suite's own known answers (tests/unit/test_attention.py, shapes
  HEADS 2, DIM 8, BLOCK 4): tile-size independence, the single-query einsum form, block-table
  order sensitivity, prefix-only visibility, poisoned unused slots, argument errors;
* brute force on tiny inputs (a per-key Python loop).

Planted mistakes (an off-by-one causal mask, a transposed block table, a wrong scale, a missing
online rescale) must each fail the closed-form check, so the check is shown to bite.
"""

from __future__ import annotations

import math

import numpy as np
import pytest

from oracle.attention import dense_attention, gather_context, paged_attention

HEADS, DIM, BLOCK = 2, 8, 4


def build_cache(length: int, blocks: int, seed: int = 0):
    rng = np.random.default_rng(seed)
    keys = np.zeros((blocks, BLOCK, HEADS, DIM), dtype=np.float32)
    values = np.zeros_like(keys)
    flat_k = rng.standard_normal((length, HEADS, DIM)).astype(np.float32)
    flat_v = rng.standard_normal((length, HEADS, DIM)).astype(np.float32)
    keys.reshape(-1, HEADS, DIM)[:length] = flat_k
    values.reshape(-1, HEADS, DIM)[:length] = flat_v
    return keys, values, flat_k, flat_v


def scattered_case(seed: int, length: int, nq: int, pool: int, block: int, heads=3, dim=16):
    """Random pool, a shuffled table, and queries at random positions below the context."""
    rng = np.random.default_rng(seed)
    used = -(-length // block)
    kc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    table = rng.permutation(pool)[:used].astype(np.int64)
    q = rng.standard_normal((nq, heads, dim)).astype(np.float32)
    pos = np.sort(rng.integers(0, length, nq))
    pos[-1] = length - 1
    return q, pos, kc, vc, table


def closed_form_error(fn, seed: int) -> float:
    """Max |fn - float64 closed form| on a scattered multi-query case."""
    q, pos, kc, vc, table = scattered_case(seed, length=37, nq=5, pool=23, block=4)
    scale = 16**-0.5
    got = fn(q, pos, kc, vc, table, 37, scale)
    keys = gather_context(kc, table, 37)
    values = gather_context(vc, table, 37)
    want = dense_attention(q, keys, values, scale, pos)
    return float(np.max(np.abs(got - want)))


@pytest.mark.parametrize("tile_blocks", [1, 2, 3, 8])
def test_matches_the_dense_reference_for_every_tile_size(tile_blocks: int) -> None:
    length = 11
    blocks = -(-length // BLOCK)
    keys, values, flat_k, flat_v = build_cache(length, blocks)
    queries = np.random.default_rng(1).standard_normal((length, HEADS, DIM)).astype(np.float32)
    scale = DIM**-0.5
    got = paged_attention(
        queries, np.arange(length), keys, values, np.arange(blocks), length, scale,
        tile_blocks=tile_blocks,
    )  # fmt: skip
    want = dense_attention(queries, flat_k, flat_v, scale, np.arange(length))
    assert np.max(np.abs(got - want)) < 1e-5


def test_single_decode_query_matches_the_einsum_form() -> None:
    length = 9
    blocks = -(-length // BLOCK)
    keys, values, flat_k, flat_v = build_cache(length, blocks, seed=2)
    query = np.random.default_rng(3).standard_normal((1, HEADS, DIM)).astype(np.float32)
    scale = DIM**-0.5
    scores = np.einsum("qhd,khd->hqk", query, flat_k) * scale
    weights = np.exp(scores - scores.max(-1, keepdims=True))
    weights /= weights.sum(-1, keepdims=True)
    want = np.einsum("hqk,khd->qhd", weights, flat_v)
    got = paged_attention(
        query, np.asarray([length - 1]), keys, values, np.arange(blocks), length, scale, tile_blocks=1
    )
    assert np.max(np.abs(got - want)) < 1e-5


def test_the_block_table_order_selects_the_keys() -> None:
    keys, values, _, _ = build_cache(8, 2, seed=4)
    query = np.ones((1, HEADS, DIM), dtype=np.float32)
    pos = np.asarray([3])
    forward = paged_attention(query, pos, keys, values, np.asarray([0, 1]), 8, 0.5)
    swapped = paged_attention(query, pos, keys, values, np.asarray([1, 0]), 8, 0.5)
    assert not np.allclose(forward, swapped)


def test_a_query_below_the_context_sees_only_its_own_prefix() -> None:
    length = 12
    keys, values, flat_k, flat_v = build_cache(length, 3, seed=5)
    query = np.random.default_rng(6).standard_normal((1, HEADS, DIM)).astype(np.float32)
    scale = DIM**-0.5
    got = paged_attention(query, np.asarray([3]), keys, values, np.arange(3), length, scale, tile_blocks=1)
    want = dense_attention(query, flat_k[:4], flat_v[:4], scale, np.asarray([3]))
    assert np.max(np.abs(got - want)) < 1e-5


def test_poisoned_unused_slots_are_never_read() -> None:
    keys, values, _, _ = build_cache(5, 2, seed=7)
    keys.reshape(-1, HEADS, DIM)[5:] = 1e6
    values.reshape(-1, HEADS, DIM)[5:] = 1e6
    query = np.random.default_rng(8).standard_normal((1, HEADS, DIM)).astype(np.float32)
    got = paged_attention(query, np.asarray([4]), keys, values, np.asarray([0, 1]), 5, DIM**-0.5)
    assert np.all(np.isfinite(got)) and np.max(np.abs(got)) < 100.0


def test_a_fully_masked_query_returns_zeros() -> None:
    """Empty-sum guard (attention.py:120-121): no visible key -> accumulator / 1 = 0."""
    keys, values, _, _ = build_cache(8, 2, seed=9)
    query = np.ones((1, HEADS, DIM), dtype=np.float32)
    got = paged_attention(query, np.asarray([-1]), keys, values, np.asarray([0, 1]), 8, 0.5)
    assert np.array_equal(got, np.zeros_like(got))


@pytest.mark.parametrize(
    ("kwargs", "message"),
    [
        ({"context_len": 0}, "context_len must be >= 1"),
        ({"context_len": 99}, "exceeds the blocks"),
        ({"tile_blocks": 0}, "tile_blocks must be >= 1"),
    ],
)
def test_invalid_arguments_are_refused(kwargs, message: str) -> None:
    keys, values, _, _ = build_cache(4, 1)
    call = dict(
        queries=np.zeros((1, HEADS, DIM), dtype=np.float32), query_positions=np.asarray([0]),
        key_cache=keys, value_cache=values, block_table=np.asarray([0]), context_len=4, scale=0.5,
    )  # fmt: skip
    call.update(kwargs)
    with pytest.raises(ValueError, match=message):
        paged_attention(**call)


@pytest.mark.parametrize("seed", range(6))
@pytest.mark.parametrize("tile_blocks", [1, 3, 8])
def test_scattered_multi_query_matches_the_closed_form(seed: int, tile_blocks: int) -> None:
    def run(q, pos, kc, vc, table, ctx, scale):
        return paged_attention(q, pos, kc, vc, table, ctx, scale, tile_blocks=tile_blocks)

    assert closed_form_error(run, seed) < 1e-5

    def run64(q, pos, kc, vc, table, ctx, scale):
        return paged_attention(q, pos, kc, vc, table, ctx, scale, tile_blocks=tile_blocks, dtype=np.float64)

    assert closed_form_error(run64, seed) < 1e-12


def test_brute_force_per_key_loop_on_a_tiny_case() -> None:
    """Softmax written one key at a time, in pure Python, against the oracle."""
    q, pos, kc, vc, table = scattered_case(11, length=7, nq=3, pool=5, block=2, heads=2, dim=4)
    scale = 0.5
    got = paged_attention(q, pos, kc, vc, table, 7, scale, dtype=np.float64)
    for i, p in enumerate(pos):
        for h in range(2):
            weights, rows = [], []
            for key_pos in range(int(p) + 1):
                blk, off = int(table[key_pos // 2]), key_pos % 2
                s = sum(float(q[i, h, d]) * float(kc[blk, off, h, d]) for d in range(4)) * scale
                weights.append(math.exp(s))
                rows.append(vc[blk, off, h].astype(np.float64))
            total = sum(weights)
            want = sum(w * r for w, r in zip(weights, rows)) / total
            assert np.max(np.abs(got[i, h] - want)) < 1e-12


# --- planted mistakes: each must fail the closed-form check -------------------------------------


def _off_by_one_mask(q, pos, kc, vc, table, ctx, scale):
    return paged_attention(q, pos + 1, kc, vc, table, ctx, scale)  # sees one key too many


def _transposed_table(q, pos, kc, vc, table, ctx, scale):
    return paged_attention(q, pos, kc, vc, table[::-1].copy(), ctx, scale)


def _wrong_scale(q, pos, kc, vc, table, ctx, scale):
    return paged_attention(q, pos, kc, vc, table, ctx, scale * 1.01)


def _no_rescale(q, pos, kc, vc, table, ctx, scale):
    """Per-tile softmaxes summed without the running-max rescale."""
    out = np.zeros(q.shape, dtype=np.float64)
    block = kc.shape[1]
    used = -(-ctx // block)
    for first in range(used):
        tile_ctx = min((first + 1) * block, ctx)
        part = paged_attention(q, pos, kc, vc, table, tile_ctx, scale, dtype=np.float64)
        out = part if first == 0 else 0.5 * (out + part)
    return out


@pytest.mark.parametrize("mutant", [_off_by_one_mask, _transposed_table, _wrong_scale, _no_rescale])
def test_planted_mistakes_fail_the_closed_form(mutant) -> None:
    assert closed_form_error(mutant, 3) > 1e-4
