"""Host-side model containers with the reference's API (no CPU forward pass).

Mirrors the data half of src/paged_kv_serving/engine/model.py: ``LayerWeights`` and
``TransformerWeights`` (model.py:84-101), ``random_weights`` with the reference's seeded draw
order (model.py:173-203), ``rope_tables`` (model.py:60-67) and a ``LanguageModel`` exposing
``config``, ``weights``, ``rope`` and ``attention_scale`` (model.py:224-241). Those attributes
are all the GPU :class:`~paged_kv_serving_amd.runner.ModelRunner` reads, so the reference's own
LanguageModel can be passed in its place. The forward pass itself runs on the device
(runner.py of this package).
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import numpy as np

from paged_kv_serving_amd.config import ModelConfig

__all__ = ["LanguageModel", "LayerWeights", "TransformerWeights", "random_weights", "rope_tables"]


@dataclass(frozen=True)
class LayerWeights:
    attn_norm: np.ndarray
    qkv_proj: np.ndarray
    out_proj: np.ndarray
    ffn_norm: np.ndarray
    gate_proj: np.ndarray
    up_proj: np.ndarray
    down_proj: np.ndarray


@dataclass(frozen=True)
class TransformerWeights:
    """Every parameter, float32, never mutated after construction."""

    token_embedding: np.ndarray
    layers: tuple[LayerWeights, ...]
    final_norm: np.ndarray

    def validate(self, config: ModelConfig) -> None:
        """Shapes, dtype and finiteness, with the reference's messages (model.py:103-128)."""
        d, ff = config.d_model, config.d_ff
        expected = [
            ("token_embedding", self.token_embedding, (config.vocab_size, d)),
            ("final_norm", self.final_norm, (d,)),
        ]
        if len(self.layers) != config.n_layers:
            raise ValueError(f"expected {config.n_layers} layers, found {len(self.layers)}")
        for i, layer in enumerate(self.layers):
            expected += [
                (f"layers.{i}.attn_norm", layer.attn_norm, (d,)),
                (f"layers.{i}.qkv_proj", layer.qkv_proj, (d, 3 * d)),
                (f"layers.{i}.out_proj", layer.out_proj, (d, d)),
                (f"layers.{i}.ffn_norm", layer.ffn_norm, (d,)),
                (f"layers.{i}.gate_proj", layer.gate_proj, (d, ff)),
                (f"layers.{i}.up_proj", layer.up_proj, (d, ff)),
                (f"layers.{i}.down_proj", layer.down_proj, (ff, d)),
            ]
        for name, array, shape in expected:
            if array.shape != shape:
                raise ValueError(f"{name}: expected shape {shape}, found {array.shape}")
            if array.dtype != np.float32:
                raise ValueError(f"{name}: expected float32, found {array.dtype}")
            if not np.all(np.isfinite(array)):
                raise ValueError(f"{name}: contains NaN or infinite values")


def random_weights(config: ModelConfig, seed: int = 0) -> TransformerWeights:
    """Seeded initialisation in the reference's draw order (model.py:179-201).

    A single ``np.random.default_rng(seed)`` draws, layer by layer, qkv, out, gate and up
    (scaled by d_model^-0.5) and down (scaled by d_ff^-0.5), then the token embedding (scaled by
    0.05); norms are ones. Draws are float64 standard normals, scaled, then cast to float32.
    """
    rng = np.random.default_rng(seed)

    def normal(*shape: int, scale: float) -> np.ndarray:
        return (rng.standard_normal(shape) * scale).astype(np.float32)

    d, ff = config.d_model, config.d_ff
    layers = []
    for _ in range(config.n_layers):
        qkv = normal(d, 3 * d, scale=d**-0.5)
        out = normal(d, d, scale=d**-0.5)
        gate = normal(d, ff, scale=d**-0.5)
        up = normal(d, ff, scale=d**-0.5)
        down = normal(ff, d, scale=ff**-0.5)
        ones = np.ones(d, dtype=np.float32)
        layers.append(LayerWeights(ones, qkv, out, ones.copy(), gate, up, down))
    weights = TransformerWeights(
        token_embedding=normal(config.vocab_size, d, scale=0.05),
        layers=tuple(layers),
        final_norm=np.ones(d, dtype=np.float32),
    )
    weights.validate(config)
    return weights


def rope_tables(max_seq_len: int, head_dim: int, theta: float) -> tuple[np.ndarray, np.ndarray]:
    """cos and sin of position * theta^(-2i/head_dim), float32 (max_seq_len, head_dim/2)."""
    if head_dim % 2:
        raise ValueError("head_dim must be even for rotary embeddings")
    half = head_dim // 2
    inverse = 1.0 / (theta ** (np.arange(half, dtype=np.float64) * 2.0 / head_dim))
    angles = np.outer(np.arange(max_seq_len, dtype=np.float64), inverse)
    return np.cos(angles).astype(np.float32), np.sin(angles).astype(np.float32)


class LanguageModel:
    """Config, weights and rotary tables (model.py:224-241)."""

    def __init__(self, config: ModelConfig, weights: TransformerWeights) -> None:
        weights.validate(config)
        self.config = config
        self.weights = weights
        self._cos, self._sin = rope_tables(config.max_seq_len, config.head_dim, config.rope_theta)

    @property
    def rope(self) -> tuple[np.ndarray, np.ndarray]:
        return self._cos, self._sin

    @property
    def attention_scale(self) -> float:
        return 1.0 / math.sqrt(self.config.head_dim)
