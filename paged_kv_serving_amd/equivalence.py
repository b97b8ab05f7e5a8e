"""The paged path against a cache-free recompute, on the device (reference equivalence.py).

The reference tracks its central correctness claim as a number: logits computed through the
paged cache -- chunked prefill, scattered block tables, continuous batching -- against one dense
causal pass over the same tokens with no cache at all (src/paged_kv_serving/engine/
equivalence.py:49-187; bench_baseline.py:217-284 reports it). This module is that harness for
the GPU path: :func:`dense_logits` is the cache-free pass in float32 torch on the device (one
softmax over the whole causal score matrix, model.py:206-221 and :269-288), and
:func:`paged_chunked_logits` / :func:`max_logit_gap` / :func:`rows_logit_gap` run the paged side
through :class:`~paged_kv_serving_amd.runner.ModelRunner`.
"""

from __future__ import annotations

from collections.abc import Sequence

import numpy as np
import torch

from paged_kv_serving_amd.runner import BatchEntry, ExecutionBatch, ModelRunner

__all__ = ["dense_logits", "max_logit_gap", "paged_chunked_logits", "rows_logit_gap", "split_sizes"]


def split_sizes(total: int, chunk: int) -> list[int]:
    """``total`` tokens in chunks of ``chunk``, the last one possibly shorter (equivalence.py:39-46)."""
    if total < 1 or chunk < 1:
        raise ValueError("total and chunk must be >= 1")
    return [chunk] * (total // chunk) + ([total % chunk] if total % chunk else [])


def _rms(x: torch.Tensor, weight: torch.Tensor, eps: float) -> torch.Tensor:
    return x / torch.sqrt(torch.mean(x * x, dim=-1, keepdim=True) + eps) * weight


def dense_logits(model, token_ids: Sequence[int], device: torch.device | str) -> np.ndarray:
    """Logits at every position of ``token_ids`` from one dense causal pass, float32, no cache:
    embed, then per layer RMSNorm -> fused QKV -> RoPE on q and k (half-split rotation) -> one
    masked softmax over all scores -> output projection, RMSNorm -> SwiGLU; final RMSNorm and
    the tied embedding. Returns host ``float32[T, vocab]``."""
    config = model.config
    tokens = torch.as_tensor(np.asarray(token_ids, dtype=np.int64), device=device)
    count, heads, dim, eps = tokens.numel(), config.n_heads, config.head_dim, config.norm_eps

    def up(array) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).to(device)

    weights = model.weights
    embedding = up(weights.token_embedding)
    cos, sin = (up(table)[:count][:, None, :] for table in model.rope)
    half = dim // 2

    def rope(x: torch.Tensor) -> torch.Tensor:
        lo, hi = x[..., :half], x[..., half:]
        return torch.cat([lo * cos - hi * sin, hi * cos + lo * sin], dim=-1)

    causal = torch.triu(torch.ones(count, count, dtype=torch.bool, device=device), diagonal=1)
    hidden = embedding[tokens]
    for layer in weights.layers:
        fused = (_rms(hidden, up(layer.attn_norm), eps) @ up(layer.qkv_proj)).view(count, 3, heads, dim)
        q = rope(fused[:, 0]).transpose(0, 1).contiguous()  # [H, T, D]
        k = rope(fused[:, 1]).transpose(0, 1).contiguous()
        v = fused[:, 2].transpose(0, 1).contiguous()
        scores = torch.matmul(q, k.transpose(1, 2).contiguous()) * model.attention_scale
        scores = scores.masked_fill(causal, float("-inf"))
        attended = torch.matmul(torch.softmax(scores, dim=-1), v).transpose(0, 1).reshape(count, config.d_model)
        hidden = hidden + attended @ up(layer.out_proj)
        normed = _rms(hidden, up(layer.ffn_norm), eps)
        gate = normed @ up(layer.gate_proj)
        silu = gate * (1.0 / (1.0 + torch.exp(-torch.clamp(gate, -60.0, 60.0))))
        hidden = hidden + (silu * (normed @ up(layer.up_proj))) @ up(layer.down_proj)
    logits = _rms(hidden, up(weights.final_norm), eps) @ embedding.T
    return logits.cpu().numpy()


def paged_chunked_logits(
    model, token_ids: Sequence[int], *, block_size: int = 16, chunks: Sequence[int] | None = None,
    block_order: Sequence[int] | None = None, device: torch.device | str | None = None,
) -> np.ndarray:  # fmt: skip
    """Logits at the last position computed through a fresh paged pool in ``chunks``, with the
    sequence's blocks at ``block_order`` (equivalence.py:49-92)."""
    tokens = list(token_ids)
    if not tokens:
        raise ValueError("token_ids must not be empty")
    sizes = list(chunks) if chunks is not None else [len(tokens)]
    if sum(sizes) != len(tokens) or any(size < 1 for size in sizes):
        raise ValueError("chunks must be positive and sum to the number of tokens")
    needed = -(-len(tokens) // block_size)
    table = tuple(block_order) if block_order is not None else tuple(range(needed))
    if len(table) < needed or len(set(table)) != len(table):
        raise ValueError("block_order must list at least one distinct block per block of tokens")
    runner = ModelRunner(model, num_blocks=max(table) + 1, block_size=block_size, device=device)
    start, logits = 0, None
    for size in sizes:
        stop = start + size
        entry = BatchEntry(
            seq_id="equiv", token_ids=tuple(tokens[start:stop]), positions=tuple(range(start, stop)),
            block_table=table, logits_index=size - 1 if stop == len(tokens) else None,
        )  # fmt: skip
        logits = runner.execute(ExecutionBatch((entry,))).get("equiv", logits)
        start = stop
    return logits


def max_logit_gap(model, token_ids: Sequence[int], *, device, **paged) -> float:
    """Largest |paged - dense| at the last position (equivalence.py:95-108)."""
    paged_row = paged_chunked_logits(model, token_ids, device=device, **paged)
    return float(np.max(np.abs(paged_row - dense_logits(model, token_ids, device)[-1])))


def rows_logit_gap(model, rows, row_seqs, tokens, device) -> tuple[float, int]:
    """Largest |row - dense(full tokens)[context - 1]| over engine rows, and rows checked
    (equivalence.py:162-187): one dense pass per sequence covers every step it took."""
    dense: dict[str, np.ndarray] = {}
    worst, checked = 0.0, 0
    for row, (seq_id, context) in zip(rows, row_seqs):
        if seq_id not in dense:
            dense[seq_id] = dense_logits(model, tokens[seq_id], device)
        worst = max(worst, float(np.max(np.abs(dense[seq_id][context - 1] - row))))
        checked += 1
    return worst, checked
