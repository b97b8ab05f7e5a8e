"""Model and engine configuration, with the reference's fields, defaults and validation messages.

Mirrors src/paged_kv_serving/engine/config.py:35-160 (ModelConfig, EngineConfig). The
ModelRunner reads only ``vocab_size, d_model, n_layers, n_heads, head_dim, max_seq_len,
rope_theta, norm_eps``, so the reference's own config objects work in its place unchanged.
"""

from __future__ import annotations

from dataclasses import dataclass

__all__ = ["EngineConfig", "ModelConfig"]


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


@dataclass(frozen=True)
class EngineConfig:
    """Scheduling and memory limits (config.py:98-160); defaults are the reference's."""

    block_size: int = 16
    num_blocks: int = 512
    max_batched_tokens: int = 256
    max_running_seqs: int = 32
    max_prompt_tokens: int = 512
    max_new_tokens: int = 128
    max_context_tokens: int = 1024
    enable_prefix_cache: bool = True
    watermark: float = 0.02
    lower_class_prefill_share: float = 0.25

    def __post_init__(self) -> None:
        if self.block_size < 1:
            raise ValueError("block_size must be >= 1")
        if self.num_blocks < 1:
            raise ValueError("num_blocks must be >= 1")
        if self.max_batched_tokens < 1:
            raise ValueError("max_batched_tokens must be >= 1")
        if self.max_running_seqs < 1:
            raise ValueError("max_running_seqs must be >= 1")
        if self.max_prompt_tokens < 1 or self.max_new_tokens < 1:
            raise ValueError("max_prompt_tokens and max_new_tokens must be >= 1")
        if self.max_context_tokens < self.max_prompt_tokens + self.max_new_tokens:
            raise ValueError("max_context_tokens must cover max_prompt_tokens + max_new_tokens")
        if not 0.0 <= self.watermark < 1.0:
            raise ValueError("watermark must be in [0, 1)")
        if not 0.0 < self.lower_class_prefill_share <= 1.0:
            raise ValueError("lower_class_prefill_share must be in (0, 1]")
        if self.num_blocks * self.block_size < self.max_context_tokens:
            raise ValueError("the KV cache cannot hold a single max-length sequence")

    @property
    def cache_capacity_tokens(self) -> int:
        return self.num_blocks * self.block_size

    @property
    def lower_class_prefill_tokens(self) -> int:
        """Per-iteration prefill allowance of classes below the highest one with work."""
        return max(1, int(self.max_batched_tokens * self.lower_class_prefill_share))
