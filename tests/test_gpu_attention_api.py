"""The reference-signature wrapper ``paged_kv_serving_amd.attention.paged_attention`` (the drop-in
for attention.py:42-121) on the GPU, held to the reference's own unit assertions
(tests/unit/test_attention.py, shapes HEADS 2, DIM 8, BLOCK 4) in both of its forms: NumPy arrays
in and a NumPy array out (the reference's call, sent through one pinned transfer), and device
tensors in and out. The bar is the reference's 1e-5 against dense attention and the float64
closed form.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.attention import dense_attention, gather_context
from paged_kv_serving_amd.attention import paged_attention

pytestmark = pytest.mark.gpu

HEADS, DIM, BLOCK = 2, 8, 4
TOL = 1e-5


def build_cache(length: int, blocks: int, seed: int = 0):
    rng = np.random.default_rng(seed)
    keys = np.zeros((blocks, BLOCK, HEADS, DIM), dtype=np.float32)
    values = np.zeros_like(keys)
    flat_k = rng.standard_normal((length, HEADS, DIM)).astype(np.float32)
    flat_v = rng.standard_normal((length, HEADS, DIM)).astype(np.float32)
    keys.reshape(-1, HEADS, DIM)[:length] = flat_k
    values.reshape(-1, HEADS, DIM)[:length] = flat_v
    return keys, values, flat_k, flat_v


@pytest.fixture(params=["numpy", "device"])
def attend(request, device):
    """The wrapper called with NumPy arrays, or with the same data as device tensors."""
    if request.param == "numpy":

        def on_host(*args, **kwargs):
            out = paged_attention(*args, **kwargs)
            assert isinstance(out, np.ndarray) and out.dtype == np.float32
            return out

        return on_host

    def on_device(q, pos, keys, values, table, context, scale, **kwargs):
        to = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
        out = paged_attention(to(q), to(pos), to(keys), to(values), to(table), context, scale, **kwargs)
        assert isinstance(out, torch.Tensor) and out.is_cuda
        return out.cpu().numpy()

    return on_device


@pytest.mark.parametrize("tile_blocks", [1, 2, 3, 8])
def test_matches_dense_attention_for_every_tile_size(attend, tile_blocks) -> None:
    length = 11
    blocks = -(-length // BLOCK)
    keys, values, flat_k, flat_v = build_cache(length, blocks)
    queries = np.random.default_rng(1).standard_normal((length, HEADS, DIM)).astype(np.float32)
    scale = DIM**-0.5
    got = attend(queries, np.arange(length), keys, values, np.arange(blocks), length, scale,
                 tile_blocks=tile_blocks)  # fmt: skip
    assert np.max(np.abs(got - dense_attention(queries, flat_k, flat_v, scale, np.arange(length)))) < TOL


def test_a_single_decode_query_attends_to_the_whole_context(attend) -> None:
    length = 9
    blocks = -(-length // BLOCK)
    keys, values, flat_k, flat_v = build_cache(length, blocks, seed=2)
    query = np.random.default_rng(3).standard_normal((1, HEADS, DIM)).astype(np.float32)
    scale = DIM**-0.5
    scores = np.einsum("qhd,khd->hqk", query, flat_k) * scale
    weights = np.exp(scores - scores.max(-1, keepdims=True))
    weights /= weights.sum(-1, keepdims=True)
    want = np.einsum("hqk,khd->qhd", weights, flat_v)
    got = attend(query, np.asarray([length - 1]), keys, values, np.arange(blocks), length, scale, tile_blocks=1)
    assert np.max(np.abs(got - want)) < TOL


def test_the_block_table_order_selects_the_keys(attend) -> None:
    keys, values, _, _ = build_cache(8, 2, seed=4)
    query = np.ones((1, HEADS, DIM), dtype=np.float32)
    forward = attend(query, np.asarray([3]), keys, values, np.asarray([0, 1]), 8, 0.5)
    swapped = attend(query, np.asarray([3]), keys, values, np.asarray([1, 0]), 8, 0.5)
    assert not np.allclose(forward, swapped)


def test_a_query_below_the_context_sees_only_its_prefix(attend) -> None:
    keys, values, flat_k, flat_v = build_cache(12, 3, seed=5)
    query = np.random.default_rng(6).standard_normal((1, HEADS, DIM)).astype(np.float32)
    scale = DIM**-0.5
    got = attend(query, np.asarray([3]), keys, values, np.arange(3), 12, scale)
    assert np.max(np.abs(got - dense_attention(query, flat_k[:4], flat_v[:4], scale, np.asarray([3])))) < TOL


def test_poisoned_unused_slots_are_never_read(attend) -> None:
    keys, values, _, _ = build_cache(5, 2, seed=7)
    keys.reshape(-1, HEADS, DIM)[5:] = 1e6
    values.reshape(-1, HEADS, DIM)[5:] = 1e6
    query = np.random.default_rng(8).standard_normal((1, HEADS, DIM)).astype(np.float32)
    got = attend(query, np.asarray([4]), keys, values, np.asarray([0, 1]), 5, DIM**-0.5)
    assert np.all(np.isfinite(got)) and np.max(np.abs(got)) < 100.0


@pytest.mark.parametrize("seed", range(6))
def test_scattered_queries_match_the_float64_closed_form(attend, seed) -> None:
    rng = np.random.default_rng(seed)
    length, pool, block, heads, dim = 37, 23, 4, 3, 16
    kc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    vc = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
    table = rng.permutation(pool)[: -(-length // block)].astype(np.int64)
    q = rng.standard_normal((5, heads, dim)).astype(np.float32)
    pos = np.sort(rng.integers(0, length, 5))
    pos[-1] = length - 1
    scale = dim**-0.5
    want = dense_attention(q, gather_context(kc, table, length), gather_context(vc, table, length), scale, pos)
    assert np.max(np.abs(attend(q, pos, kc, vc, table, length, scale) - want)) < TOL


@pytest.mark.parametrize(
    ("kwargs", "message"),
    [
        ({"context_len": 0}, "context_len must be >= 1"),
        ({"context_len": 99}, "exceeds the blocks"),
        ({"tile_blocks": 0}, "tile_blocks must be >= 1"),
        ({"query_positions": np.asarray([0, 1])}, "one position per query"),
    ],
)
def test_invalid_arguments_are_refused_with_the_reference_messages(device, kwargs, message) -> None:
    keys, values, _, _ = build_cache(4, 1)
    call = dict(
        queries=np.zeros((1, HEADS, DIM), dtype=np.float32), query_positions=np.asarray([0]),
        key_cache=keys, value_cache=values, block_table=np.asarray([0]), context_len=4, scale=0.5,
    )  # fmt: skip
    call.update(kwargs)
    with pytest.raises(ValueError, match=message):
        paged_attention(**call)


def test_host_calls_of_changing_sizes_reuse_the_staging_buffer(device) -> None:
    """Back-to-back NumPy calls, growing past the first staging buffer and shrinking again, each
    give the dense result: the pinned buffer is refilled only after the previous result is back."""
    rng = np.random.default_rng(30)
    for length, heads, dim in ((9, 2, 8), (4000, 8, 64), (300, 4, 32), (9, 2, 8)):
        blocks = -(-length // 16)
        kc = rng.standard_normal((blocks + 2, 16, heads, dim)).astype(np.float32)
        vc = rng.standard_normal((blocks + 2, 16, heads, dim)).astype(np.float32)
        table = rng.permutation(blocks + 2)[:blocks]
        q = rng.standard_normal((3, heads, dim)).astype(np.float32)
        pos = np.asarray([length // 3, length // 2, length - 1])
        scale = dim**-0.5
        want = dense_attention(q, gather_context(kc, table, length), gather_context(vc, table, length), scale, pos)
        got = paged_attention(q, pos, kc, vc, table, length, scale)
        assert np.max(np.abs(got - want)) < TOL, (length, heads, dim)
