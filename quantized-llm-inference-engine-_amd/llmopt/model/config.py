"""Architecture description of the decoder-only model (``src/llmopt/config.py:34-78``).

Same fields, defaults and checks as the reference's ``ModelConfig``, plus the presets this
package measures: :meth:`ModelConfig.llama3_8b` (the end-to-end workload) and
:meth:`ModelConfig.tiny` (tests).
"""

from __future__ import annotations

import dataclasses
from collections.abc import Mapping
from typing import Any

__all__ = ["ModelConfig"]


@dataclasses.dataclass
class ModelConfig:
    vocab_size: int = 32000
    hidden_size: int = 1024
    intermediate_size: int = 2816
    num_hidden_layers: int = 12
    num_attention_heads: int = 16
    num_key_value_heads: int = 4
    max_position_embeddings: int = 4096
    rms_norm_eps: float = 1e-6
    rope_theta: float = 10000.0
    tie_word_embeddings: bool = False
    attn_implementation: str = "auto"
    torch_dtype: str = "bfloat16"

    def __post_init__(self) -> None:
        if self.hidden_size % self.num_attention_heads:
            raise ValueError(
                f"hidden_size ({self.hidden_size}) must be divisible by num_attention_heads "
                f"({self.num_attention_heads})"
            )
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError(
                f"num_attention_heads ({self.num_attention_heads}) must be divisible by "
                f"num_key_value_heads ({self.num_key_value_heads})"
            )
        if self.intermediate_size % 2:
            raise ValueError("intermediate_size must be even for SwiGLU")

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads

    @property
    def num_query_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads

    def to_dict(self) -> dict[str, Any]:
        return dataclasses.asdict(self)

    @classmethod
    def from_dict(cls, data: Mapping[str, Any]) -> ModelConfig:
        names = {f.name for f in dataclasses.fields(cls)}
        return cls(**{k: v for k, v in data.items() if k in names})

    @classmethod
    def llama3_8b(cls) -> ModelConfig:
        """Llama-3-8B: 32 layers, hidden 4096, 32 heads / 8 KV heads of 128, FFN 14336,
        vocab 128256, RoPE base 500000, RMSNorm eps 1e-5."""
        return cls(vocab_size=128256, hidden_size=4096, intermediate_size=14336, num_hidden_layers=32,
                   num_attention_heads=32, num_key_value_heads=8, max_position_embeddings=8192,
                   rms_norm_eps=1e-5, rope_theta=500000.0)

    @classmethod
    def tiny(cls, vocab_size: int = 512) -> ModelConfig:
        """Two layers, hidden 256, 4 heads / 2 KV heads of 64, FFN 512 (a multiple of 128, so
        every projection takes the packed kernels' group-128 paths)."""
        return cls(vocab_size=vocab_size, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
                   num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024)
