"""The reference's fp32 decoder and its cache-free recompute, on the CPU -- test infrastructure.

Restates src/paged_kv_serving/engine/model.py:43-288: pre-norm RMSNorm, rotary embeddings on
queries and keys (half-split rotation), multi-head causal attention, SwiGLU, and the output
projection tied to the token embedding. ``reference_forward`` recomputes a whole sequence with
dense attention and no cache; the paged engine must reproduce its logits to within 1e-4
(tests/property/test_equivalence.py:34 of the reference).

``config`` is any object with the fields of the reference's ModelConfig (config.py:35-66);
``weights`` any object with ``token_embedding``, ``layers`` (each with ``attn_norm, qkv_proj,
out_proj, ffn_norm, gate_proj, up_proj, down_proj``) and ``final_norm``.
"""

from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np

__all__ = [
    "OracleModel",
    "apply_rope",
    "dense_causal_attention",
    "random_weights",
    "rms_norm",
    "rope_tables",
    "silu",
    "softmax_last",
]


def rms_norm(x: np.ndarray, weight: np.ndarray, eps: float) -> np.ndarray:
    """x / sqrt(mean(x^2) + eps) * weight, float32 (model.py:43-46)."""
    mean_square = np.mean(np.square(x, dtype=np.float32), axis=-1, keepdims=True)
    return ((x / np.sqrt(mean_square + eps)) * weight).astype(np.float32)


def silu(x: np.ndarray) -> np.ndarray:
    """x * sigmoid(x) with the exponent clipped to [-60, 60] (model.py:49-51)."""
    return (x * (1.0 / (1.0 + np.exp(-np.clip(x, -60.0, 60.0))))).astype(np.float32)


def softmax_last(x: np.ndarray) -> np.ndarray:
    """Max-shifted softmax over the last axis (model.py:54-57)."""
    e = np.exp(x - np.max(x, axis=-1, keepdims=True))
    return (e / np.sum(e, axis=-1, keepdims=True)).astype(np.float32)


def rope_tables(max_seq_len: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos/sin of position * theta^(-2i/head_dim), (max_seq_len, head_dim/2) (model.py:60-67)."""
    if head_dim % 2:
        raise ValueError("head_dim must be even for rotary embeddings")
    half = head_dim // 2
    # 1 / theta^x rather than theta^-x: the two differ in the last float64 bit for some i, which
    # flips float32 table entries at head_dim >= 64.
    frequencies = 1.0 / (theta ** (np.arange(half, dtype=np.float64) * 2.0 / head_dim))
    angles = np.outer(np.arange(max_seq_len, dtype=np.float64), frequencies)
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


def apply_rope(x: np.ndarray, positions: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate the (first half, second half) pairs of each head by the position's angle
    (model.py:70-81)."""
    half = x.shape[-1] // 2
    c = cos[positions][:, None, :]
    s = sin[positions][:, None, :]
    first, second = x[..., :half], x[..., half:]
    return np.concatenate([first * c - second * s, second * c + first * s], axis=-1)


def random_weights(config, seed: int = 0) -> SimpleNamespace:
    """Seeded weights with the reference's draw order (model.py:173-203).

    One ``np.random.default_rng(seed)``; per layer, in order: qkv (d, 3d), out (d, d), gate
    (d, ff), up (d, ff) scaled by d^-0.5, down (ff, d) scaled by ff^-0.5; then the embedding
    (vocab, d) scaled by 0.05. Norm weights are ones. Each draw is standard_normal in float64,
    scaled, then cast to float32.
    """
    rng = np.random.default_rng(seed)

    def draw(rows: int, cols: int, scale: float) -> np.ndarray:
        return (rng.standard_normal((rows, cols)) * scale).astype(np.float32)

    d, ff = config.d_model, config.d_ff
    layers = []
    for _ in range(config.n_layers):
        qkv = draw(d, 3 * d, d**-0.5)
        out = draw(d, d, d**-0.5)
        gate = draw(d, ff, d**-0.5)
        up = draw(d, ff, d**-0.5)
        down = draw(ff, d, ff**-0.5)
        layers.append(
            SimpleNamespace(
                attn_norm=np.ones(d, dtype=np.float32),
                qkv_proj=qkv,
                out_proj=out,
                ffn_norm=np.ones(d, dtype=np.float32),
                gate_proj=gate,
                up_proj=up,
                down_proj=down,
            )
        )
    embedding = draw(config.vocab_size, d, 0.05)
    return SimpleNamespace(
        token_embedding=embedding, layers=tuple(layers), final_norm=np.ones(d, dtype=np.float32)
    )


def dense_causal_attention(
    queries: np.ndarray, keys: np.ndarray, values: np.ndarray, scale: float
) -> np.ndarray:
    """One softmax over the full lower-triangular score matrix, float32 (model.py:206-221)."""
    n = queries.shape[0]
    scores = np.matmul(queries.transpose(1, 0, 2), keys.transpose(1, 2, 0)) * np.float32(scale)
    above = np.triu(np.ones((n, n), dtype=bool), k=1)
    scores = np.where(above[None], np.float32(-np.inf), scores)
    attended = np.matmul(softmax_last(scores), values.transpose(1, 0, 2))
    return attended.transpose(1, 0, 2).astype(np.float32)


class OracleModel:
    """Weights plus the NumPy forward pieces of model.py:224-288."""

    def __init__(self, config, weights) -> None:
        self.config = config
        self.weights = weights
        self.cos, self.sin = rope_tables(config.max_seq_len, config.head_dim, config.rope_theta)

    @property
    def attention_scale(self) -> float:
        return 1.0 / math.sqrt(self.config.head_dim)

    def project_qkv(self, hidden, layer, positions):
        """rms_norm -> fused QKV -> (T, 3, H, D) -> RoPE on q and k (model.py:243-254)."""
        c = self.config
        fused = rms_norm(hidden, layer.attn_norm, c.norm_eps) @ layer.qkv_proj
        shaped = fused.reshape(-1, 3, c.n_heads, c.head_dim)
        q = apply_rope(shaped[:, 0], positions, self.cos, self.sin)
        k = apply_rope(shaped[:, 1], positions, self.cos, self.sin)
        return q, k, np.ascontiguousarray(shaped[:, 2])

    def feed_forward(self, hidden, layer):
        """SwiGLU (model.py:256-259)."""
        normed = rms_norm(hidden, layer.ffn_norm, self.config.norm_eps)
        return ((silu(normed @ layer.gate_proj) * (normed @ layer.up_proj)) @ layer.down_proj).astype(
            np.float32
        )

    def logits_from_hidden(self, hidden):
        """Final norm and the tied projection (model.py:261-264)."""
        normed = rms_norm(hidden, self.weights.final_norm, self.config.norm_eps)
        return (normed @ self.weights.token_embedding.T).astype(np.float32)

    def embed(self, tokens):
        return np.ascontiguousarray(self.weights.token_embedding[tokens])

    def reference_forward(self, token_ids) -> np.ndarray:
        """Logits of every position with no cache at all (model.py:269-288)."""
        tokens = np.asarray(token_ids, dtype=np.int64)
        if tokens.ndim != 1 or tokens.size == 0:
            raise ValueError("token_ids must be a non-empty 1-D sequence")
        if tokens.size > self.config.max_seq_len:
            raise ValueError("sequence longer than max_seq_len")
        if np.any(tokens < 0) or np.any(tokens >= self.config.vocab_size):
            raise ValueError("token id outside the vocabulary")
        positions = np.arange(tokens.size, dtype=np.int64)
        hidden = self.embed(tokens)
        for layer in self.weights.layers:
            q, k, v = self.project_qkv(hidden, layer, positions)
            attended = dense_causal_attention(q, k, v, self.attention_scale)
            hidden = hidden + attended.reshape(tokens.size, self.config.d_model) @ layer.out_proj
            hidden = (hidden + self.feed_forward(hidden, layer)).astype(np.float32)
        return self.logits_from_hidden(hidden)
