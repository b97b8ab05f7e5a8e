"""The model configuration, with the reference's fields, defaults and validation messages.

Mirrors ModelConfig of src/paged_kv_serving/engine/config.py:35-66. The scheduler's EngineConfig
(config.py:98-160) belongs to the caller and is not restated here. The ModelRunner reads only ``vocab_size, d_model, n_layers, n_heads, head_dim, max_seq_len,
rope_theta, norm_eps``, so the reference's own config objects work in its place unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass

__all__ = ["ModelConfig"]


@dataclass(frozen=True)
class ModelConfig:
    """Shape of the decoder (config.py:35-66): RMSNorm, RoPE, MHA, SwiGLU, tied embedding."""

    vocab_size: int
    d_model: int
    n_layers: int
    n_heads: int
    d_ff: int
    max_seq_len: int
    rope_theta: float = 10_000.0
    norm_eps: float = 1e-5

    def __post_init__(self) -> None:
        for name in ("vocab_size", "d_model", "n_layers", "n_heads", "d_ff", "max_seq_len"):
            if getattr(self, name) < 1:
                raise ValueError(f"{name} must be >= 1")
        if self.d_model % self.n_heads:
            raise ValueError("d_model must be divisible by n_heads")
        if self.rope_theta <= 1.0:
            raise ValueError("rope_theta must be > 1")
        if self.norm_eps <= 0.0:
            raise ValueError("norm_eps must be > 0")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.n_heads
