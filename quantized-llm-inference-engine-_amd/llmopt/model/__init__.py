"""Decoder-only model whose linears run on the quantized-linear kernels (``src/llmopt/model``)."""

from llmopt.model.config import ModelConfig
from llmopt.model.generate import GreedyGenerator
from llmopt.model.layers import DecoderLayer, PagedAttentionLayer, RMSNorm, SwiGLUMLP
from llmopt.model.modeling import (DecoderOnlyModel, ModelOutput, fuse_projections_, random_quantized_model,
                                   reference_twin)
from llmopt.model.rotary import RotaryEmbedding, apply_rotary_pos_emb, rotate_half

__all__ = [
    "DecoderLayer",
    "DecoderOnlyModel",
    "GreedyGenerator",
    "ModelConfig",
    "ModelOutput",
    "PagedAttentionLayer",
    "RMSNorm",
    "RotaryEmbedding",
    "SwiGLUMLP",
    "apply_rotary_pos_emb",
    "fuse_projections_",
    "random_quantized_model",
    "reference_twin",
    "rotate_half",
]
