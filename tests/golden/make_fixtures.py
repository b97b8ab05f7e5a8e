"""Writes tests/golden/attention_cases.npz and rope_cases.npz: small seeded cases with expected
outputs, so the GPU tests can check the kernels on the GPU box without recomputing anything.

Attention expectations come from the float64 dense closed form (softmax over the visible keys,
gathered through the block table), which is independent of the paged online-softmax recurrence
that both the oracle and the kernels implement. RoPE expectations are the reference's float32
NumPy expression (model.py:70-81) evaluated elementwise. The reference itself is not imported;
nothing here reads /root/reference.

    python tests/golden/make_fixtures.py          # rewrite the files
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from oracle.attention import dense_attention, gather_context  # noqa: E402
from oracle.model import rope_tables  # noqa: E402

# (heads, head_dim, block_size, pool blocks, sequences, max context, prefill rows)
ATTENTION_SHAPES = [
    (2, 8, 4, 40, 3, 60, 0),
    (2, 32, 16, 30, 4, 110, 20),
    (1, 64, 16, 24, 3, 120, 70),
    (1, 128, 1, 260, 2, 120, 9),
    (1, 256, 8, 24, 2, 90, 40),
]


def attention_cases() -> dict[str, np.ndarray]:
    out: dict[str, np.ndarray] = {}
    rng = np.random.default_rng(2024)
    for index, (heads, dim, block, pool, seqs, max_ctx, prefill) in enumerate(ATTENTION_SHAPES):
        keys = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
        values = rng.standard_normal((pool, block, heads, dim)).astype(np.float32)
        order = rng.permutation(pool)
        contexts = rng.integers(1, max_ctx + 1, seqs)
        width = int(-(-contexts.max() // block))
        tables = np.full((seqs, width), -1, dtype=np.int32)
        used = 0
        positions, seq_of = [], []
        for s, ctx in enumerate(contexts.tolist()):
            need = -(-ctx // block)
            tables[s, :need] = order[used : used + need]
            used += need
            rows = min(ctx, prefill) if s == 0 and prefill else 1
            positions += list(range(ctx - rows, ctx))
            seq_of += [s] * rows
        positions = np.asarray(positions, dtype=np.int32)
        seq_of = np.asarray(seq_of, dtype=np.int32)
        queries = rng.standard_normal((positions.size, heads, dim)).astype(np.float32)
        scale = float(dim**-0.5)
        expected = np.zeros(queries.shape, dtype=np.float64)
        for s, ctx in enumerate(contexts.tolist()):
            rows = np.flatnonzero(seq_of == s)
            table = tables[s, : -(-ctx // block)]
            expected[rows] = dense_attention(
                queries[rows], gather_context(keys, table, ctx), gather_context(values, table, ctx),
                scale, positions[rows],
            )  # fmt: skip
        prefix = f"c{index}_"
        out.update({
            prefix + "keys": keys, prefix + "values": values, prefix + "tables": tables,
            prefix + "contexts": contexts.astype(np.int32), prefix + "positions": positions,
            prefix + "seq": seq_of, prefix + "queries": queries,
            prefix + "scale": np.float64(scale), prefix + "expected": expected,
        })  # fmt: skip
    out["count"] = np.int64(len(ATTENTION_SHAPES))
    return out


def rotate_elementwise(x: np.ndarray, positions: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """The rotation of model.py:77-81 evaluated one element at a time in float32 scalars, each
    product and sum rounded on its own: out[i] = x[i] cos - x[i + D/2] sin and
    out[i + D/2] = x[i + D/2] cos + x[i] sin, with (cos, sin) = table[position][i]. Written
    independently of the vectorised oracle.apply_rope, so the fixture pins it."""
    tokens, heads, dim = x.shape
    half = dim // 2
    out = np.empty_like(x)
    for t in range(tokens):
        p = int(positions[t])
        for h in range(heads):
            for i in range(half):
                c, s = np.float32(cos[p, i]), np.float32(sin[p, i])
                lo, hi = np.float32(x[t, h, i]), np.float32(x[t, h, i + half])
                out[t, h, i] = np.float32(np.float32(lo * c) - np.float32(hi * s))
                out[t, h, i + half] = np.float32(np.float32(hi * c) + np.float32(lo * s))
    return out


def rope_cases() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(7)
    out: dict[str, np.ndarray] = {}
    for index, (tokens, heads, dim, rows) in enumerate([(5, 2, 8, 64), (33, 4, 64, 700), (7, 3, 128, 512)]):
        cos, sin = rope_tables(rows, dim, 10_000.0)
        fused = rng.standard_normal((tokens, 3, heads, dim)).astype(np.float32)
        positions = rng.integers(0, rows, tokens).astype(np.int64)
        positions[0] = rows - 1
        prefix = f"r{index}_"
        out.update({
            prefix + "fused": fused, prefix + "positions": positions,
            prefix + "cos": cos, prefix + "sin": sin,
            prefix + "q": rotate_elementwise(fused[:, 0], positions, cos, sin),
            prefix + "k": rotate_elementwise(fused[:, 1], positions, cos, sin),
        })  # fmt: skip
    out["count"] = np.int64(3)
    return out


def main() -> int:
    np.savez_compressed(HERE / "attention_cases.npz", **attention_cases())
    np.savez_compressed(HERE / "rope_cases.npz", **rope_cases())
    for name in ("attention_cases.npz", "rope_cases.npz"):
        print(name, (HERE / name).stat().st_size, "bytes")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
