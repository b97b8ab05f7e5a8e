"""GPU parity of the fused RoPE + append kernel (pkv_rope_append) against the CPU oracle.

The oracle is the reference's float32 NumPy rotation (model.py:70-81, restated in
oracle/model.py) followed by its fancy-index append (runner.py:195-196, oracle/runner.py); the
kernel rounds every product and sum separately, so rotated queries and pool rows must be equal
bit for bit, and into a bfloat16 pool equal to the oracle's rows rounded to nearest even. Rows of
the pool that no token targets must keep their bits.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.bf16 import bf16_bits, bf16_round
from oracle.model import apply_rope, rope_tables
from oracle.runner import append
from paged_kv_serving_amd import ops

pytestmark = pytest.mark.gpu


def say(*parts) -> None:
    print(*parts, flush=True)


def _case(seed, tokens, heads, dim, slots_total, table_rows=4096):
    rng = np.random.default_rng(seed)
    fused = rng.standard_normal((tokens, 3, heads, dim)).astype(np.float32)
    positions = rng.integers(0, table_rows, tokens).astype(np.int64)
    positions[:1] = 0  # the identity rotation
    positions[-1:] = table_rows - 1
    slots = rng.permutation(slots_total)[:tokens].astype(np.int64)
    cos, sin = rope_tables(table_rows, dim, 10_000.0)
    return fused, positions, slots, cos, sin


def _oracle(fused, positions, slots, cos, sin, pool_k, pool_v):
    q = apply_rope(fused[:, 0], positions, cos, sin)
    k = apply_rope(fused[:, 1], positions, cos, sin)
    append(pool_k, pool_v, slots, k, fused[:, 2])
    return q


def _device(device, *arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).to(device) for a in arrays]


@pytest.mark.parametrize(
    ("tokens", "heads", "dim"),
    [(1, 1, 8), (7, 4, 32), (300, 32, 128), (33, 2, 256), (9, 3, 6), (5, 2, 2)],
)
def test_rope_append_float32_is_bit_exact(device, tokens, heads, dim) -> None:
    say("rope f32", tokens, heads, dim)
    num_slots = 4 * tokens + 3
    fused, positions, slots, cos, sin = _case(tokens * 7 + dim, tokens, heads, dim, num_slots)
    sentinel = np.full((num_slots, heads, dim), 3.5, dtype=np.float32)
    want_k, want_v = sentinel.copy(), sentinel.copy()
    want_q = _oracle(fused, positions, slots, cos, sin, want_k, want_v)

    d_fused, d_pos, d_slots, d_cos, d_sin, pool_k, pool_v = _device(
        device, fused, positions, slots, cos, sin, sentinel, sentinel
    )
    out = ops.rope_append(pool_k, pool_v, d_fused[:, 0], d_fused[:, 1], d_fused[:, 2], d_pos, d_cos, d_sin, d_slots)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want_q.view(np.uint32))
    assert np.array_equal(pool_k.cpu().numpy().view(np.uint32), want_k.view(np.uint32))
    assert np.array_equal(pool_v.cpu().numpy().view(np.uint32), want_v.view(np.uint32))


@pytest.mark.parametrize("dim", [8, 128])
def test_rope_append_into_bfloat16_rounds_to_nearest_even(device, dim) -> None:
    tokens, heads, num_slots = 40, 4, 64
    fused, positions, slots, cos, sin = _case(5, tokens, heads, dim, num_slots)
    fused[3, 1, 0, :4] = [1.00390625, 1.01171875, -2.0078125, np.inf]  # ties and an infinity
    want_k = np.zeros((num_slots, heads, dim), dtype=np.float32)
    want_v = np.zeros_like(want_k)
    want_q = _oracle(fused, positions, slots, cos, sin, want_k, want_v)
    d_fused, d_pos, d_slots, d_cos, d_sin = _device(device, fused, positions, slots, cos, sin)
    pool_k = torch.zeros((num_slots, heads, dim), dtype=torch.bfloat16, device=device)
    pool_v = torch.zeros_like(pool_k)
    out = ops.rope_append(pool_k, pool_v, d_fused[:, 0], d_fused[:, 1], d_fused[:, 2], d_pos, d_cos, d_sin, d_slots)
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint32), want_q.view(np.uint32))
    got_k = pool_k.view(torch.int16).cpu().numpy().view(np.uint16)
    got_v = pool_v.view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(got_k, bf16_bits(want_k))
    assert np.array_equal(got_v, bf16_bits(want_v))
    assert np.array_equal(bf16_round(want_k[slots]), pool_k[torch.from_numpy(slots).to(device)].float().cpu().numpy())


def test_rope_append_in_place_on_a_fused_projection(device) -> None:
    """Queries rotated in place inside the fused [T, 3, H, D] output, as ModelRunner.execute does."""
    tokens, heads, dim, num_slots = 64, 8, 64, 200
    fused, positions, slots, cos, sin = _case(11, tokens, heads, dim, num_slots)
    want_k = np.zeros((num_slots, heads, dim), dtype=np.float32)
    want_v = np.zeros_like(want_k)
    want_q = _oracle(fused, positions, slots, cos, sin, want_k, want_v)
    d_fused, d_pos, d_slots, d_cos, d_sin = _device(device, fused, positions, slots, cos, sin)
    pool_k = torch.zeros((num_slots, heads, dim), device=device)
    pool_v = torch.zeros_like(pool_k)
    q_view = d_fused[:, 0]
    out = ops.rope_append(pool_k, pool_v, q_view, d_fused[:, 1], d_fused[:, 2], d_pos, d_cos, d_sin, d_slots, out=q_view)
    torch.cuda.synchronize()
    assert out.data_ptr() == q_view.data_ptr()
    got = d_fused.cpu().numpy()
    assert np.array_equal(got[:, 0].view(np.uint32), want_q.view(np.uint32))
    assert np.array_equal(got[:, 1:], fused[:, 1:])  # keys and values of the projection untouched
    assert np.array_equal(pool_k.cpu().numpy(), want_k) and np.array_equal(pool_v.cpu().numpy(), want_v)


def test_rope_append_skips_bad_slots_and_positions(device) -> None:
    tokens, heads, dim, num_slots = 6, 2, 16, 10
    fused, positions, slots, cos, sin = _case(2, tokens, heads, dim, num_slots, table_rows=32)
    slots[1], slots[2] = -1, num_slots  # outside the pool: pool writes skipped
    positions[4] = 32  # outside the table: the whole token skipped
    d_fused, d_pos, d_slots, d_cos, d_sin = _device(device, fused, positions, slots, cos, sin)
    pool_k = torch.full((num_slots, heads, dim), 7.0, device=device)
    pool_v = torch.full_like(pool_k, 7.0)
    out = torch.full((tokens, heads, dim), -1.0, device=device)
    ops.rope_append(pool_k, pool_v, d_fused[:, 0], d_fused[:, 1], d_fused[:, 2], d_pos, d_cos, d_sin, d_slots, out=out)
    torch.cuda.synchronize()
    good = [0, 1, 2, 3, 5]
    want_q = apply_rope(fused[good, 0], positions[good], cos, sin)
    assert np.array_equal(out.cpu().numpy()[good], want_q)
    assert torch.all(out[4] == -1.0)
    want_k = np.full((num_slots, heads, dim), 7.0, dtype=np.float32)
    want_v = want_k.copy()
    keep = [0, 3, 5]
    append(want_k, want_v, slots[keep], apply_rope(fused[keep, 1], positions[keep], cos, sin), fused[keep, 2])
    assert np.array_equal(pool_k.cpu().numpy(), want_k) and np.array_equal(pool_v.cpu().numpy(), want_v)


def test_config3_sized_rope_append_matches_torch_elementwise(device) -> None:
    """4,216 tokens x 32 heads x 128 (config 3's append) against the same rotation composed from
    torch's elementwise float32 ops on the device, which round every operation separately."""
    tokens, heads, dim, blocks, block = 4216, 32, 128, 600, 16
    gen = torch.Generator(device=device)
    gen.manual_seed(3)
    fused = torch.randn((tokens, 3, heads, dim), generator=gen, device=device)
    positions = torch.randint(0, 4096, (tokens,), generator=gen, device=device)
    slots = torch.randperm(blocks * block, generator=gen, device=device)[:tokens]
    cos, sin = (torch.from_numpy(t).to(device) for t in rope_tables(4096, dim, 10_000.0))
    pool_k = torch.zeros((blocks, block, heads, dim), device=device)
    pool_v = torch.zeros_like(pool_k)
    out = ops.rope_append(pool_k, pool_v, fused[:, 0], fused[:, 1], fused[:, 2], positions, cos, sin, slots)
    c, s = cos[positions][:, None, :], sin[positions][:, None, :]

    def rotate(x):
        lo, hi = x[..., : dim // 2], x[..., dim // 2 :]
        return torch.cat([lo * c - hi * s, hi * c + lo * s], dim=-1)

    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int32), rotate(fused[:, 0]).view(torch.int32))
    flat_k, flat_v = pool_k.view(-1, heads, dim), pool_v.view(-1, heads, dim)
    assert torch.equal(flat_k[slots].view(torch.int32), rotate(fused[:, 1]).view(torch.int32))
    assert torch.equal(flat_v[slots], fused[:, 2])
    untouched = torch.ones(blocks * block, dtype=torch.bool, device=device)
    untouched[slots] = False
    assert not torch.any(flat_k[untouched]) and not torch.any(flat_v[untouched])
