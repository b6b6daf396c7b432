"""Model shape configuration, field-for-field the reference's ``GPTConfig``.

Field names, defaults (GPT-2 124M) and validation messages follow
``src/transformer_internals/config.py:23-159`` so a reference config object's
``to_dict()`` round-trips into this one; ``GPT2_SIZES`` / ``gpt2_config`` give
the released shapes (``:138-159``). The training-side ``TrainConfig`` is not
part of the quantized-inference path and is not provided.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass
from typing import Any, Literal

__all__ = ["GPT2_SIZES", "GPTConfig", "gpt2_config"]


@dataclass
class GPTConfig:
    vocab_size: int = 50257
    n_positions: int = 1024
    n_layer: int = 12
    n_head: int = 12
    n_kv_head: int | None = None
    n_embd: int = 768
    dropout: float = 0.0
    layer_norm_epsilon: float = 1e-5
    norm_position: Literal["pre", "post"] = "pre"
    pos_embedding: Literal["learned", "sinusoidal"] = "learned"
    tie_weights: bool = True
    activation: Literal["gelu_tanh", "gelu_exact", "relu"] = "gelu_tanh"
    residual_scaled_init: bool = True
    attn_bias: bool = True
    mlp_bias: bool = True
    use_sdpa: bool = False

    def __post_init__(self) -> None:
        if self.n_embd % self.n_head != 0:
            raise ValueError(f"n_embd={self.n_embd} must be divisible by n_head={self.n_head}")
        if self.n_kv_head is not None and (self.n_kv_head < 1 or self.n_head % self.n_kv_head != 0):
            raise ValueError(f"n_head={self.n_head} must be divisible by n_kv_head={self.n_kv_head}")
        if self.norm_position not in ("pre", "post"):
            raise ValueError(f"norm_position must be 'pre' or 'post', got {self.norm_position!r}")
        if self.pos_embedding not in ("learned", "sinusoidal"):
            raise ValueError(f"unknown pos_embedding {self.pos_embedding!r}")
        if self.activation not in ("gelu_tanh", "gelu_exact", "relu"):
            raise ValueError(f"unknown activation {self.activation!r}")

    @property
    def head_dim(self) -> int:
        return self.n_embd // self.n_head

    @property
    def kv_heads(self) -> int:
        return self.n_head if self.n_kv_head is None else self.n_kv_head

    def kv_cache_bytes_per_token(self, dtype_bytes: int = 4) -> int:
        """``2 * n_layer * kv_heads * head_dim * dtype_bytes`` per token per sequence."""
        return 2 * self.n_layer * self.kv_heads * self.head_dim * dtype_bytes

    def to_dict(self) -> dict[str, Any]:
        return asdict(self)


GPT2_SIZES: dict[str, dict[str, int]] = {
    "gpt2": {"n_layer": 12, "n_head": 12, "n_embd": 768},
    "gpt2-medium": {"n_layer": 24, "n_head": 16, "n_embd": 1024},
    "gpt2-large": {"n_layer": 36, "n_head": 20, "n_embd": 1280},
    "gpt2-xl": {"n_layer": 48, "n_head": 25, "n_embd": 1600},
}


def gpt2_config(size: str = "gpt2", **overrides: Any) -> GPTConfig:
    if size not in GPT2_SIZES:
        raise ValueError(f"unknown GPT-2 size {size!r}; expected one of {sorted(GPT2_SIZES)}")
    return GPTConfig(**{**GPT2_SIZES[size], **overrides})
