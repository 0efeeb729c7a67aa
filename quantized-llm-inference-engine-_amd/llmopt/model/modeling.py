"""Decoder-only model over a paged KV cache (``src/llmopt/model/modeling.py:31-145``).

``DecoderOnlyModel.forward`` has the reference's signature and returns ``[seq, q_len, vocab]``
logits; with ``last_only=True`` it projects only each sequence's last position onto the
vocabulary (what the engine reads, ``engine/model_runner.py:93-114``), which is
:func:`llmopt.logits.last_token_logits`.

:func:`fuse_projections_` turns a model whose linears ``quantize_model_`` has replaced into
the fused form (q/k/v in one packed weight, gate/up in one with the SiLU product in the
kernel); :func:`random_quantized_model` builds the random-init, RTN-quantized model of a config
directly on a device, the way the end-to-end measurement needs it.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from llmopt.logits import last_token_hidden
from llmopt.model.config import ModelConfig
from llmopt.model.layers import DecoderLayer, RMSNorm

__all__ = ["DecoderOnlyModel", "ModelOutput", "fuse_projections_", "random_quantized_model", "reference_twin"]


@dataclass
class ModelOutput:
    """Logits ``[seq, q_len, vocab]`` (``q_len`` is 1 for ``last_only`` forwards)."""

    logits: torch.Tensor
    hidden_states: torch.Tensor | None = None

    def last_logits(self) -> torch.Tensor:
        """``[seq, vocab]``: each sequence's final position."""
        return self.logits[:, -1, :]


class DecoderOnlyModel(nn.Module):
    """Embedding, ``num_hidden_layers`` pre-norm decoder layers, final RMSNorm, ``lm_head``."""

    def __init__(self, config: ModelConfig, backend: str = "auto", dtype: torch.dtype | None = None) -> None:
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList(DecoderLayer(config, i, backend) for i in range(config.num_hidden_layers))
        self.norm = RMSNorm(config.hidden_size, config.rms_norm_eps)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        # False: every down projection finishes its own K-split reduction (the results are the
        # same bits either way).
        self.defer_reductions = True
        if config.tie_word_embeddings:
            self.lm_head.weight = self.embed_tokens.weight
        self.to(dtype or torch.float32)

    def num_parameters(self) -> int:
        return sum(p.numel() for p in self.parameters())

    def forward(self, input_ids: torch.Tensor, positions: torch.Tensor, cache: object | None = None,
                block_ids: torch.Tensor | None = None, context_lens: torch.Tensor | None = None,
                token_offsets: torch.Tensor | None = None, q_len: int = 1, last_only: bool = False) -> ModelOutput:
        """One engine step: ``input_ids``/``positions`` ``[seq * q_len]`` (or ``[seq, q_len]``),
        per-sequence cache metadata as in :class:`PagedAttentionLayer`."""
        input_ids = input_ids.reshape(-1)
        positions = positions.reshape(-1)
        hidden = self.embed_tokens(input_ids)
        if token_offsets is None and context_lens is not None and block_ids is not None:
            # Where this step's tokens go in the cache: computed once here, not in every layer.
            token_offsets = context_lens - q_len
        pending = None  # each layer's MLP output, added inside the next norm's kernel
        last = len(self.layers) - 1
        # The final norm takes the last layer's partial sums too unless it first keeps only each
        # sequence's last row (last_only with several tokens per sequence).
        defer_last = not last_only or q_len == 1
        for i, layer in enumerate(self.layers):
            # A layer may hand its down projection's partial sums to the next norm.
            hidden, pending = layer.forward_chained(hidden, pending, positions, cache=cache, block_ids=block_ids,
                                                    context_lens=context_lens, token_offsets=token_offsets,
                                                    q_len=q_len,
                                                    defer_mlp=self.defer_reductions and (i < last or defer_last))
        seqs = int(hidden.shape[0]) // max(1, q_len)
        if last_only and q_len > 1:
            # The residual add, RMSNorm and lm_head act row by row, so keeping only the last rows
            # first is exact.
            hidden = last_token_hidden(hidden, q_len).contiguous()
            if pending is not None:
                pending = last_token_hidden(pending, q_len).contiguous()
        normed = self.norm(hidden) if pending is None else self.norm.add_forward(pending, hidden)[0]
        logits = self.lm_head(normed)
        return ModelOutput(logits=logits.view(seqs, 1 if last_only else q_len, -1))

    def allocate_cache(self, num_blocks: int, block_size: int, dtype: torch.dtype, device: torch.device | str) -> object:
        """A :class:`PagedKVCache` for this model (``modeling.py:132-145``)."""
        from llmopt.cache.paged_cache import PagedKVCache

        return PagedKVCache(self.config.num_hidden_layers, num_blocks, block_size, self.config.num_key_value_heads,
                            self.config.head_dim, dtype=dtype, device=device)


def fuse_projections_(model: nn.Module) -> int:
    """Fuse every layer's quantized q/k/v and gate/up projections in place; returns the number
    of fused modules created."""
    fused = 0
    for layer in model.modules():
        if isinstance(layer, DecoderLayer):
            fused += int(layer.self_attn.fuse_qkv()) + int(layer.mlp.fuse_gate_up())
    return fused


@torch.no_grad()
def random_quantized_model(config: ModelConfig, *, device: torch.device | str, dtype: torch.dtype = torch.bfloat16,
                           seed: int = 0, std: float = 0.02, bits: int = 4, group_size: int = 128,
                           symmetric: bool = False, fuse: bool = True, backend: str = "auto") -> DecoderOnlyModel:
    """A model with every weight ``std * N(0, 1)`` (norm weights 1), its decoder linears
    round-to-nearest quantized (embedding and ``lm_head`` stay dense, as ``quantize_model_``
    leaves them), built layer by layer on ``device`` so that the dense linears of only one
    layer exist at a time."""
    from llmopt.quantization.quant_linear import QuantLinear
    from llmopt.quantization.quantizers import RoundToNearestQuantizer

    gen = torch.Generator(device=device).manual_seed(seed)
    with torch.device("meta"):
        model = DecoderOnlyModel(config, backend=backend, dtype=dtype)
    quantizer = RoundToNearestQuantizer(bits=bits, group_size=group_size, symmetric=symmetric)

    def dense(shape: tuple[int, ...]) -> torch.Tensor:
        return (torch.randn(shape, generator=gen, device=device, dtype=torch.float32) * std).to(dtype)

    model.embed_tokens = nn.Embedding.from_pretrained(dense((config.vocab_size, config.hidden_size)), freeze=True)
    for layer in model.layers:
        for parent, names in ((layer.self_attn, ("q_proj", "k_proj", "v_proj", "o_proj")),
                              (layer.mlp, ("gate_proj", "up_proj", "down_proj"))):
            for name in names:
                meta = getattr(parent, name)
                weight = dense((meta.out_features, meta.in_features))
                qt = quantizer.quantize(weight.float())
                module = QuantLinear.from_float(nn.Linear(meta.in_features, meta.out_features, bias=False,
                                                          device="meta"), qt, compute_dtype=dtype)
                setattr(parent, name, module)
                del weight
        for norm in (layer.input_layernorm, layer.post_attention_layernorm):
            norm.weight = nn.Parameter(torch.ones(config.hidden_size, device=device, dtype=dtype), requires_grad=False)
        layer.self_attn.rotary = type(layer.self_attn.rotary)(config.head_dim, config.max_position_embeddings,
                                                              config.rope_theta).to(device)
    model.norm.weight = nn.Parameter(torch.ones(config.hidden_size, device=device, dtype=dtype), requires_grad=False)
    if config.tie_word_embeddings:
        model.lm_head.weight = model.embed_tokens.weight
    else:
        model.lm_head.weight = nn.Parameter(dense((config.vocab_size, config.hidden_size)), requires_grad=False)
    if fuse:
        fuse_projections_(model)
    return model.eval()


@torch.no_grad()
def reference_twin(model: DecoderOnlyModel) -> DecoderOnlyModel:
    """A copy of an unfused quantized ``model`` that computes the way the reference does: each
    ``QuantLinear`` becomes a dense ``nn.Linear`` holding its dequantized weight (what the
    reference's ``QuantLinear`` caches and multiplies, ``quant_linear.py:93-113``), norms and
    rotary run the torch sequences, attention the torch sequence over the gathered cache
    (backend ``"sdpa"``). For measuring the reference's approach on the same device."""
    import copy

    from llmopt.attention.paged_attention import PagedAttention, PagedAttentionConfig
    from llmopt.quantization.quant_linear import QuantLinear
    from llmopt.quantization.quantizers import dequantize

    twin = copy.deepcopy(model)
    swaps = []
    for parent in twin.modules():
        for name, child in parent.named_children():
            if isinstance(child, QuantLinear):
                swaps.append((parent, name, child))
            elif name in ("qkv_proj", "gate_up") and child is not None:
                raise ValueError("reference_twin needs the unfused model (build it before fuse_projections_)")
    for parent, name, child in swaps:
        dense = nn.Linear(child.in_features, child.out_features, bias=child.bias is not None,
                          device="meta")
        dense.weight = nn.Parameter(dequantize(child.quantized_tensor(), child.config.compute_dtype),
                                    requires_grad=False)
        if child.bias is not None:
            dense.bias = nn.Parameter(child.bias.detach().clone(), requires_grad=False)
        setattr(parent, name, dense)
    for module in twin.modules():
        if hasattr(module, "fused_ops"):
            module.fused_ops = False
        if isinstance(module, DecoderLayer):
            attn = module.self_attn
            attn.attn = PagedAttention(attn.num_heads, attn.num_kv_heads, attn.head_dim,
                                       config=PagedAttentionConfig(block_size=16), backend="sdpa")
    return twin
